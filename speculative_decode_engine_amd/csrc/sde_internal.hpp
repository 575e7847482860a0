// Internal definitions shared by the HIP translation units of libsde_paged.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "sde/spec_device.hpp"
#include "sde_paged_kv.h"

// The opaque cache handle.  Device memory: pool (owned or borrowed), the
// per-layer block tables, the seq_len word, and a lazily grown attention
// workspace.  Host mirrors keep validation free of device round trips.
struct sde_kv_cache {
  sde_kv_config cfg;  // pool_blocks already resolved (never 0 here)
  int device = 0;
  uint16_t* pool = nullptr;
  size_t pool_bytes = 0;
  bool owns_pool = false;
  int32_t* d_tables = nullptr;          // [n_layers][max_blocks_per_layer]
  std::vector<int32_t> h_tables;        // host mirror of d_tables
  std::vector<int32_t> n_mapped;        // leading mapped logical blocks per layer
  int32_t* d_seq_len = nullptr;
  int seq_len = 0;                      // host mirror of *d_seq_len
  bool seq_len_on_device = false;       // *d_seq_len was set by a device-side rewind
  void* workspace = nullptr;            // internal attention workspace
  size_t workspace_bytes = 0;
  // Workspaces outgrown by a larger call: kept until the cache is
  // destroyed, because work already queued, or a graph captured earlier,
  // may still use them.
  std::vector<void*> retired_workspaces;
  // Arrival counters of the fused partition combine, one per (KV head, row
  // group) of a call; zero at rest (the last arriving workgroup resets its
  // counter), so calls on one cache must be stream-ordered.
  uint32_t* d_counters = nullptr;
  int n_cus = 256;  // compute units of `device` (sizes attention grids)
};

namespace sde {
// Attention arrival counters per cache; after them the stochastic
// acceptance's scratch (kSpecScratchWords, sde/spec_device.hpp: arrival
// counters zero at rest, per-row results and per-slice statistics).
constexpr int kMaxAttnCounters = 4096;
}  // namespace sde

namespace sde {

// Makes the cache's device current for the scope and restores the caller's.
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != dev) ok_ = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev_ >= 0 && ok_) (void)hipSetDevice(prev_);
  }
  bool ok() const { return ok_; }
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int prev_ = -1;
  bool ok_ = true;
};

// Tokens [0, mapped_tokens) of a layer have a physical block.
inline int64_t mapped_tokens(const sde_kv_cache* c, int layer) {
  return (int64_t)c->n_mapped[layer] * c->cfg.block_size;
}

inline const int32_t* layer_table(const sde_kv_cache* c, int layer) {
  return c->d_tables + (size_t)layer * c->cfg.max_blocks_per_layer;
}

// Status of the most recent launch on this thread.
inline int launch_status() {
  return hipGetLastError() == hipSuccess ? SDE_OK : SDE_ERR_HIP;
}

}  // namespace sde
