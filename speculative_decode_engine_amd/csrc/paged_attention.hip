// Paged GQA decode / speculative-verify attention for gfx950 (wave64).
//
// Computes what cublas_attention_kernel (kernels.cu:904-940) computes with
// device_flash_attention_gqa (attention.h:21-127): for query m of a window,
// out[m][h] = softmax(q[m][h] . K[0..pos_base+m]^T * dph^-1/2) V, with query
// head h reading KV head h*nkv/nh, keys gathered through the block table.
//
// The "rows" of a KV head are its (query, head-in-group) pairs; a row group
// (2 to 16 rows) shares every K/V byte it loads.  The context of each (KV
// head, row group) is split into partitions, one 8-wave workgroup each
// (about one per CU); a single-partition context writes the normalised
// output directly, otherwise per-row partials go to the workspace and the
// last workgroup of a (KV head, row group) to finish -- found with one
// arrival counter per pair -- merges all partitions with a log-sum-exp
// combine in partition order, so the result does not depend on arrival
// order and one call is one launch.
//
// Both kernels (attn_mfma_kernel, and attn_rope_kernel for the fused RoPE +
// append + attention step) run the MFMA tile path of
// sde/attention_device.hpp: K and V stream from HBM into VGPRs in the
// coalesced load layout (lane = token slot x 16-byte feature chunk),
// software-pipelined a tile (32 tokens) ahead, and are staged per wave in
// LDS; the logits (K . Q^T) and the output (V^T . P^T, V read transposed
// with ds_read_b64_tr_b16) are 16x16x32 fp16 MFMA products with fp32
// accumulation, q and P entering as fp16 hi + lo parts, and the online
// softmax is lane-local per row.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <mutex>

#include "sde/attention_device.hpp"
#include "attention_generic.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace attn {

// Decode and verify steps on the MFMA tile path.
template <int DPH, int RPW, int CHUNK>
__global__ __launch_bounds__(64 * kStreamWaves) void attn_mfma_kernel(AttnArgs a) {
  __shared__ MfmaLds<DPH, kStreamWaves> lds;
  const int3 w = stream_coords<CHUNK>();
  stream_item<DPH, RPW, CHUNK, kStreamWaves, false, MfmaLds<DPH, kStreamWaves>, false, true>(
      a, w.x, w.y, w.z, lds);
}

// attn_mfma_kernel with RoPE of q and of the window's k, and the window's
// append, fused in (sde_rope_append_attention).
template <int DPH, int RPW, int CHUNK>
__global__ __launch_bounds__(64 * kStreamWaves) void attn_rope_kernel(AttnArgs a, RopeArgs rp) {
  __shared__ MfmaLds<DPH, kStreamWaves> lds;
  const int3 w = stream_coords<CHUNK>();
  stream_item<DPH, RPW, CHUNK, kStreamWaves, true, MfmaLds<DPH, kStreamWaves>, false, true>(
      a, w.x, w.y, w.z, lds, kStreamWaves, &rp);
}

}  // namespace attn
}  // namespace sde

namespace {

using namespace sde::attn;


// Upper bound of the plans' n_parts over every L <= max_total_len: a
// partition holds at least one tile per wave and there are at most
// kStreamMaxParts of them.
int parts_bound(int max_total_len) {
  const int n_tiles = (max_total_len + kTile - 1) / kTile;
  const int by_len = (n_tiles + kStreamWaves - 1) / kStreamWaves;
  return by_len < kStreamMaxParts ? by_len : kStreamMaxParts;
}

// The plan of a call: 8-wave workgroups, one per CU.
StreamPlan plan_for(int L_max, int nkv, int R, int n_cus) {
  return stream_plan8_spread(L_max, nkv, R, n_cus);
}

// Polls of a split combine's wait (sde_debug_set_slice_spin).
std::atomic<uint32_t> g_slice_spin{kSliceSpinLimit};

size_t partial_bytes(int nkv, int R, int n_parts, int dph) {
  return n_parts > 1 ? (size_t)nkv * R * n_parts * (size_t)(dph + 2) * sizeof(float) : 0;
}

template <int DPH>
int launch(const StreamPlan& p, const AttnArgs& a, int nkv, hipStream_t s,
           const RopeArgs* rope) {
  const dim3 grid(p.n_parts, nkv, p.row_groups);
  const dim3 block(64 * kStreamWaves);
#define SDE_MFMA(R, C)                                                \
  if (!rope && p.rpw == R && p.chunk == C) {                          \
    attn_mfma_kernel<DPH, R, C><<<grid, block, 0, s>>>(a);            \
    return sde::launch_status();                                      \
  }
#define SDE_ROPE(R, C)                                                \
  if (rope && p.rpw == R && p.chunk == C) {                           \
    attn_rope_kernel<DPH, R, C><<<grid, block, 0, s>>>(a, *rope);     \
    return sde::launch_status();                                      \
  }
  SDE_MFMA(2, 1)
  SDE_MFMA(2, 2)
  SDE_MFMA(2, 3)
  SDE_MFMA(2, 4)
  SDE_MFMA(4, 1)
  SDE_MFMA(4, 2)
  SDE_MFMA(4, 3)
  SDE_MFMA(4, 4)
  SDE_MFMA(8, 1)
  SDE_MFMA(8, 2)
  SDE_MFMA(8, 3)
  SDE_MFMA(8, 4)
  SDE_MFMA(16, 1)
  SDE_MFMA(16, 2)
  SDE_MFMA(16, 3)
  SDE_MFMA(16, 4)
  SDE_ROPE(2, 1)
  SDE_ROPE(2, 2)
  SDE_ROPE(2, 3)
  SDE_ROPE(2, 4)
  SDE_ROPE(4, 1)
  SDE_ROPE(4, 2)
  SDE_ROPE(4, 3)
  SDE_ROPE(4, 4)
  SDE_ROPE(8, 1)
  SDE_ROPE(8, 2)
  SDE_ROPE(8, 3)
  SDE_ROPE(8, 4)
  SDE_ROPE(16, 1)
  SDE_ROPE(16, 2)
  SDE_ROPE(16, 3)
  SDE_ROPE(16, 4)
#undef SDE_MFMA
#undef SDE_ROPE
  return SDE_ERR_UNSUPPORTED;
}

int check_attention(const sde_kv_cache* c, int layer, const float* d_q,
                    const float* d_out, int nh, int nkv, int dph, int pos_base,
                    int n_queries) {
  if (!c || !d_q || !d_out) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= c->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  if (nh < 1 || nkv < 1 || dph < 1 || nh % nkv != 0) return SDE_ERR_INVALID_ARGUMENT;
  if ((int64_t)nkv * dph != c->cfg.kv_dim) return SDE_ERR_INVALID_ARGUMENT;
  if (pos_base < 0 || n_queries < 1 || n_queries > 4096) return SDE_ERR_INVALID_ARGUMENT;
  if (dph > sde::gen::kMaxDph) return SDE_ERR_UNSUPPORTED;
  if ((((uintptr_t)d_q) & 7u) != 0 || (((uintptr_t)d_out) & 7u) != 0)
    return SDE_ERR_INVALID_ARGUMENT;
  if ((int64_t)pos_base + n_queries > sde::mapped_tokens(c, layer)) return SDE_ERR_CAPACITY;
  return SDE_OK;
}

}  // namespace

extern "C" {

size_t sde_paged_attention_workspace_size(const sde_kv_cache* cache, int nh,
                                          int nkv, int dph, int n_queries,
                                          int max_total_len) {
  if (!cache || nh < 1 || nkv < 1 || nh % nkv != 0 || n_queries < 1 || max_total_len < 1)
    return 0;
  const int R = n_queries * (nh / nkv);
  return partial_bytes(nkv, R, parts_bound(max_total_len), dph);
}

size_t sde_grid_attention_workspace_size(int nh, int nkv, int dph, int n_queries,
                                         int max_total_len) {
  return sde::grid_attention_workspace_size(nh, nkv, dph, n_queries, max_total_len);
}

}  // extern "C"

namespace {

int run_attention(sde_kv_cache* cache, int layer, const float* d_q, float* d_out, int nh,
                  int nkv, int dph, int pos_base, int n_queries, void* d_workspace,
                  size_t workspace_bytes, sde_stream_t stream, const RopeArgs* rope,
                  const sde::gen::GenRope* grope = nullptr) {
  sde::DeviceGuard guard(cache->device);
  if (!guard.ok()) return SDE_ERR_HIP;

  const int G = nh / nkv;
  const int R = n_queries * G;
  const int L_max = pos_base + n_queries;
  const bool generic = sde::gen::needs_generic(dph, cache->cfg.block_size);
  StreamPlan plan{};
  sde::gen::GenPlan gplan{};
  size_t need = 0;
  if (generic) {
    gplan = sde::gen::generic_plan(L_max, nkv, R, dph, cache->n_cus, parts_bound(L_max));
    need = sde::gen::generic_partial_bytes(gplan, nkv, R, dph);
  } else {
    plan = plan_for(L_max, nkv, R, cache->n_cus);
    if ((int64_t)nkv * plan.row_groups > sde::kMaxAttnCounters) return SDE_ERR_UNSUPPORTED;
    need = partial_bytes(nkv, R, plan.n_parts, dph);
  }
  float* partials = nullptr;
  if (need > 0) {
    if (d_workspace) {
      if (workspace_bytes < need) return SDE_ERR_WORKSPACE;
      partials = static_cast<float*>(d_workspace);
    } else {
      if (cache->workspace_bytes < need) {
        // Grow the cache-owned workspace.  Not while the stream is being
        // captured: the allocation cannot be recorded, and a graph would
        // keep its address.  The old buffer stays allocated (queued work
        // or an earlier graph may still use it) until the cache is freed,
        // so the size at least doubles: a context that grows call by call
        // retires O(log) buffers, at most about twice the peak need in all.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess) return SDE_ERR_HIP;
        if (cap != hipStreamCaptureStatusNone) return SDE_ERR_WORKSPACE;
        const size_t grow = need > 2 * cache->workspace_bytes ? need : 2 * cache->workspace_bytes;
        void* grown = nullptr;
        if (hipMalloc(&grown, grow) != hipSuccess) return SDE_ERR_HIP;
        if (cache->workspace) cache->retired_workspaces.push_back(cache->workspace);
        cache->workspace = grown;
        cache->workspace_bytes = grow;
      }
      partials = static_cast<float*>(cache->workspace);
    }
  }

  if (generic)
    return sde::gen::generic_attention(cache->pool, sde::layer_table(cache, layer),
                                       cache->cfg.kv_dim, cache->cfg.block_size, d_q, d_out,
                                       partials, nh, nkv, dph, pos_base, n_queries, gplan, grope,
                                       (hipStream_t)stream);

  AttnArgs a;
  a.src.pool = cache->pool;
  a.src.table = sde::layer_table(cache, layer);
  a.src.kv_dim = cache->cfg.kv_dim;
  a.src.bs = cache->cfg.block_size;
  a.src.L_max = L_max;
  a.q = d_q;
  a.out = d_out;
  a.partials = partials;
  a.counters = cache->d_counters;
  a.nh = nh;
  a.nkv = nkv;
  a.G = G;
  a.R = R;
  a.row_groups = plan.row_groups;
  a.pos_base = pos_base;
  a.n_parts = plan.n_parts;
  a.tiles_per_part = plan.tiles_per_part;
  a.qscale = (float)(kLog2e / std::sqrt((double)dph));
  // Each arrival counter on a 128-byte line of its own where they fit: a
  // split combine's waiting workgroups poll theirs while other groups'
  // arrivals update theirs.
  a.ctr_stride = (int64_t)nkv * plan.row_groups * 32 <= sde::kMaxAttnCounters ? 32 : 1;
  a.slice_spin = g_slice_spin.load(std::memory_order_relaxed);

  const hipStream_t s = (hipStream_t)stream;
  return dph == 128 ? launch<128>(plan, a, nkv, s, rope) : launch<64>(plan, a, nkv, s, rope);
}

}  // namespace

extern "C" {

int sde_paged_attention(sde_kv_cache* cache, int layer, const float* d_q,
                        float* d_out, int nh, int nkv, int dph, int pos_base,
                        int n_queries, void* d_workspace, size_t workspace_bytes,
                        sde_stream_t stream) {
  const int st = check_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries);
  if (st != SDE_OK) return st;
  return run_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries,
                       d_workspace, workspace_bytes, stream, nullptr);
}

int sde_rope_append_attention(sde_kv_cache* cache, int layer, const float* d_q,
                              const float* d_k, const float* d_v, float* d_out, int nh,
                              int nkv, int dph, int pos_base, int n_queries,
                              const sde_rope_config* rope, void* d_workspace,
                              size_t workspace_bytes, sde_stream_t stream) {
  const int st = check_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries);
  if (st != SDE_OK) return st;
  if (!d_k || !d_v || !rope || rope->scaling_type < SDE_ROPE_NONE ||
      rope->scaling_type > SDE_ROPE_YARN || !std::isfinite(rope->theta) ||
      !std::isfinite(rope->scaling_factor))
    return SDE_ERR_INVALID_ARGUMENT;
  if ((((uintptr_t)d_k) & 3u) != 0 || (((uintptr_t)d_v) & 3u) != 0)
    return SDE_ERR_INVALID_ARGUMENT;
  if (n_queries > kRopeMaxQueries) return SDE_ERR_UNSUPPORTED;
  // rope_apply_inplace (model.cu:281-323): theta defaults to 10000; NTK
  // scales theta by factor^(dph/(dph-2)); linear and YaRN divide the
  // position by the factor; each applies only for a factor above 1.
  RopeArgs rp;
  rp.k_new = d_k;
  rp.v_new = d_v;
  rp.pool = cache->pool;
  const double factor = rope->scaling_factor;
  double theta = rope->theta > 1e-6f ? (double)rope->theta : 10000.0;
  if (rope->scaling_type == SDE_ROPE_NTK && factor > 1.0)
    theta *= std::pow(factor, (double)dph / ((double)dph - 2.0));
  const bool div = (rope->scaling_type == SDE_ROPE_LINEAR || rope->scaling_type == SDE_ROPE_YARN) &&
                   factor > 1.0;
  rp.pos_div = div ? rope->scaling_factor : 1.0f;
  const double log_theta = std::log(theta);
  if (sde::gen::needs_generic(dph, cache->cfg.block_size)) {
    // the generic path: RoPE of k and the append, then attention with q
    // rotated in-kernel (same frequency rule, up to dph / 2 = 256 pairs)
    sde::gen::GenRope gr;
    gr.k_new = d_k;
    gr.v_new = d_v;
    gr.pos_div = rp.pos_div;
    for (int j = 0; j < sde::gen::kMaxDph / 2; j++)
      gr.inv_freq[j] = j < dph / 2 ? (float)std::exp(-log_theta * (2.0 * j) / dph) : 0.f;
    return run_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries,
                         d_workspace, workspace_bytes, stream, nullptr, &gr);
  }
  for (int j = 0; j < 64; j++)
    rp.inv_freq[j] = j < dph / 2 ? (float)std::exp(-log_theta * (2.0 * j) / dph) : 0.f;
  return run_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries,
                       d_workspace, workspace_bytes, stream, &rp);
}

int sde_paged_attention_noalloc(sde_kv_cache* cache, int layer, const float* d_q,
                                float* d_out, int nh, int nkv, int dph, int pos_base,
                                int n_queries, sde_stream_t stream);

uint32_t sde_debug_set_slice_spin(uint32_t polls) {
  return g_slice_spin.exchange(polls == 0 ? 0u : polls, std::memory_order_relaxed);
}

int sde_debug_attention_plan(int total_len, int nkv, int rows, int n_cus, int32_t* out) {
  if (total_len < 1 || nkv < 1 || rows < 1 || n_cus < 1 || !out) return SDE_ERR_INVALID_ARGUMENT;
  const StreamPlan p = plan_for(total_len, nkv, rows, n_cus);
  out[0] = p.rpw;
  out[1] = p.row_groups;
  out[2] = p.chunk;
  out[3] = p.tiles_per_part;
  out[4] = p.n_parts;
  out[5] = parts_bound(total_len);
  return SDE_OK;
}

int sde_attention_dispatch(int attn_type, sde_kv_cache* cache, int layer,
                           const float* d_q, float* d_out, int nh, int nkv,
                           int dph, int pos_base, int n_queries,
                           void* d_workspace, size_t workspace_bytes,
                           sde_stream_t stream) {
  if (attn_type != SDE_ATTN_SOFTMAX) return SDE_ERR_UNSUPPORTED;
  return sde_paged_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base,
                             n_queries, d_workspace, workspace_bytes, stream);
}

}  // extern "C"

// ---- sde_paged_attention_noalloc: partials in a static device array -------

namespace {

constexpr int kMaxDevices = 64;

// The split-context partials of sde_paged_attention_noalloc, one copy per
// device (each GPU the library runs on holds it until the process ends).
// In host code this name is a host-side stand-in, not a device address:
// host code uses only the address hipGetSymbolAddress returns for the
// current device (scratch_address).  No part of it must start at zero
// (each call writes every partial it later reads).
static __device__ __align__(256) char scratch[SDE_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mutex;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on `device`, which must be current:
// looked up on the first call on that device, then kept.
int scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return SDE_ERR_UNSUPPORTED;
  void* p = g_scratch_ptr[device].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[device].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SDE_ERR_HIP;
      g_scratch_ptr[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SDE_OK;
}

}  // namespace

extern "C" int sde_paged_attention_noalloc(sde_kv_cache* cache, int layer, const float* d_q,
                                           float* d_out, int nh, int nkv, int dph, int pos_base,
                                           int n_queries, sde_stream_t stream) {
  const int st = check_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries);
  if (st != SDE_OK) return st;
  sde::DeviceGuard guard(cache->device);
  if (!guard.ok()) return SDE_ERR_HIP;
  void* ws = nullptr;
  const int sst = scratch_address(cache->device, &ws);
  if (sst != SDE_OK) return sst;
  // A plan whose partials exceed the array gets SDE_ERR_WORKSPACE from
  // run_attention, before any launch; nothing here allocates.
  return run_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries, ws,
                       SDE_NOALLOC_SCRATCH_BYTES, stream, nullptr);
}
