// Paged KV cache: allocation, block tables, seq_len bookkeeping, and the
// append / fp16-write / gather kernels behind the C-ABI of sde_paged_kv.h.
//
// Reference semantics (arkhamHack/speculative_decode_engine):
//   kv_cache_alloc/free/reset   cuda/src/kv_cache.cu:8-52
//   block_ptr                   cuda/src/kv_cache.cu:58-68
//   kv_cache_append             cuda/src/kv_cache.cu:70-93
//   cublas_kv_append_kernel     cuda/src/kernels.cu:826-844
//   kv_cache_read               cuda/src/kv_cache.cu:95-114
//   rollback / set_seq_len      cuda/src/kv_cache.cu:116-120, kernels.cu:546-548
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>

#include "sde/spec_device.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace kv {

constexpr int kAppendThreads = 256;

// Element offset (in halves) of token `pos`'s K row in the pool; the V row
// is block_size * kv_dim further.  64-bit: an 8 GiB pool exceeds 2^32 halves.
__device__ __forceinline__ size_t k_row_offset(const int32_t* __restrict__ table,
                                               int pos, int bs, int kv_dim) {
  const int lb = pos / bs;
  const int slot = pos - lb * bs;
  const size_t phys = (size_t)table[lb];
  return (phys * 2u * (size_t)bs + (size_t)slot) * (size_t)kv_dim;
}

// fp32 -> fp16 bits with the hardware's round-to-nearest-even conversion.
__device__ __forceinline__ uint16_t f2h_bits(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// One token per blockIdx.y; 4 consecutive features per thread.  Requires
// kv_dim % 4 == 0 and 16-byte aligned source rows (checked on the host).
__global__ __launch_bounds__(kAppendThreads) void append_vec4_kernel(
    uint16_t* __restrict__ pool, const int32_t* __restrict__ table,
    const float* __restrict__ k, const float* __restrict__ v, int kv_dim,
    int bs, int pos_base) {
  const int m = blockIdx.y;
  const int i = (blockIdx.x * kAppendThreads + threadIdx.x) * 4;
  if (i >= kv_dim) return;
  const size_t kofs = k_row_offset(table, pos_base + m, bs, kv_dim);
  const size_t vofs = kofs + (size_t)bs * kv_dim;
  const float4 kk = *reinterpret_cast<const float4*>(k + (size_t)m * kv_dim + i);
  const float4 vv = *reinterpret_cast<const float4*>(v + (size_t)m * kv_dim + i);
  uint2 kh, vh;
  kh.x = (uint32_t)f2h_bits(kk.x) | ((uint32_t)f2h_bits(kk.y) << 16);
  kh.y = (uint32_t)f2h_bits(kk.z) | ((uint32_t)f2h_bits(kk.w) << 16);
  vh.x = (uint32_t)f2h_bits(vv.x) | ((uint32_t)f2h_bits(vv.y) << 16);
  vh.y = (uint32_t)f2h_bits(vv.z) | ((uint32_t)f2h_bits(vv.w) << 16);
  *reinterpret_cast<uint2*>(pool + kofs + i) = kh;
  *reinterpret_cast<uint2*>(pool + vofs + i) = vh;
}

// Any kv_dim / alignment: one feature per thread.
__global__ __launch_bounds__(kAppendThreads) void append_scalar_kernel(
    uint16_t* __restrict__ pool, const int32_t* __restrict__ table,
    const float* __restrict__ k, const float* __restrict__ v, int kv_dim,
    int bs, int pos_base) {
  const int m = blockIdx.y;
  const int i = blockIdx.x * kAppendThreads + threadIdx.x;
  if (i >= kv_dim) return;
  const size_t kofs = k_row_offset(table, pos_base + m, bs, kv_dim);
  const size_t vofs = kofs + (size_t)bs * kv_dim;
  pool[kofs + i] = f2h_bits(k[(size_t)m * kv_dim + i]);
  pool[vofs + i] = f2h_bits(v[(size_t)m * kv_dim + i]);
}

// Raw fp16 rows, one feature per thread (a prefill helper, not hot).
__global__ __launch_bounds__(kAppendThreads) void write_fp16_kernel(
    uint16_t* __restrict__ pool, const int32_t* __restrict__ table,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int kv_dim,
    int bs, int pos_base) {
  const int m = blockIdx.y;
  const int i = blockIdx.x * kAppendThreads + threadIdx.x;
  if (i >= kv_dim) return;
  const size_t kofs = k_row_offset(table, pos_base + m, bs, kv_dim);
  const size_t vofs = kofs + (size_t)bs * kv_dim;
  pool[kofs + i] = k[(size_t)m * kv_dim + i];
  pool[vofs + i] = v[(size_t)m * kv_dim + i];
}

__global__ __launch_bounds__(kAppendThreads) void gather_kernel(
    const uint16_t* __restrict__ pool, const int32_t* __restrict__ table,
    float* __restrict__ k, float* __restrict__ v, int kv_dim, int bs, int pos) {
  const int m = blockIdx.y;
  const int i = blockIdx.x * kAppendThreads + threadIdx.x;
  if (i >= kv_dim) return;
  const size_t kofs = k_row_offset(table, pos + m, bs, kv_dim);
  const size_t vofs = kofs + (size_t)bs * kv_dim;
  k[(size_t)m * kv_dim + i] = h2f(pool[kofs + i]);
  v[(size_t)m * kv_dim + i] = h2f(pool[vofs + i]);
}

// set_seq_len_kernel (kernels.cu:546-548).  A kernel rather than a memset so
// the write stays stream-ordered and safe to record into a HIP graph.
__global__ void set_seq_len_kernel(int32_t* seq_len, int value) {
  if (threadIdx.x == 0) *seq_len = value;
}

// sde_spec_accept_greedy: one thread applies the reference's greedy rule.
__global__ void spec_accept_kernel(const int32_t* draft_tokens, const int32_t* target_tokens,
                                   int k, int target_save, int draft_save, sde_kv_view target,
                                   sde_kv_view draft, int has_draft, int32_t* result) {
  if (threadIdx.x != 0) return;
  const SpecAccept r = spec_accept_greedy(draft_tokens, target_tokens, k, target_save,
                                          draft_save, target, has_draft ? &draft : nullptr,
                                          result + 4);
  result[0] = r.n_accepted;
  result[1] = r.bonus;
  result[2] = r.target_seq;
  result[3] = r.draft_seq;
}

}  // namespace kv
}  // namespace sde

namespace {

using namespace sde::kv;

bool valid_config(const sde_kv_config* cfg) {
  if (!cfg) return false;
  if (cfg->n_layers < 1 || cfg->kv_dim < 1 || cfg->max_blocks_per_layer < 1)
    return false;
  if (cfg->block_size < 1 || cfg->block_size > 1024) return false;
  if (cfg->pool_blocks < 0) return false;
  const int64_t pool = cfg->pool_blocks
                           ? cfg->pool_blocks
                           : (int64_t)cfg->n_layers * cfg->max_blocks_per_layer;
  if (pool > INT32_MAX) return false;
  if (pool < cfg->max_blocks_per_layer) return false;
  // Token positions are int32 everywhere (as in the reference).
  if ((int64_t)cfg->max_blocks_per_layer * cfg->block_size > INT32_MAX) return false;
  // The pool's byte size must be representable: K and V fp16 rows of every
  // block (without this, a large kv_dim wraps the size_t product and the
  // pool would be allocated smaller than its tables address).
  const int64_t block_bytes = (int64_t)4 * cfg->block_size * cfg->kv_dim;
  if (pool > PTRDIFF_MAX / block_bytes) return false;
  return true;
}

sde_kv_config resolved(const sde_kv_config* cfg) {
  sde_kv_config c = *cfg;
  if (c.pool_blocks == 0) c.pool_blocks = c.n_layers * c.max_blocks_per_layer;
  return c;
}

size_t pool_bytes_of(const sde_kv_config& c) {
  return (size_t)c.pool_blocks * 2u * (size_t)c.block_size * (size_t)c.kv_dim *
         sizeof(uint16_t);
}

void release(sde_kv_cache* c) {
  if (!c) return;
  if (c->owns_pool && c->pool) (void)hipFree(c->pool);
  if (c->d_tables) (void)hipFree(c->d_tables);
  if (c->d_seq_len) (void)hipFree(c->d_seq_len);
  if (c->workspace) (void)hipFree(c->workspace);
  for (void* w : c->retired_workspaces) (void)hipFree(w);
  if (c->d_counters) (void)hipFree(c->d_counters);
  delete c;
}

// Shared tail of both create paths: tables (reference static assignment when
// it fits the pool, kv_cache.cu:29-37), seq_len = 0, zeroed combine counters.
int finish_create(sde_kv_cache* c, sde_kv_cache** out) {
  const sde_kv_config& cfg = c->cfg;
  const size_t n_entries = (size_t)cfg.n_layers * cfg.max_blocks_per_layer;
  c->h_tables.assign(n_entries, -1);
  c->n_mapped.assign(cfg.n_layers, 0);
  if ((int64_t)cfg.n_layers * cfg.max_blocks_per_layer <= cfg.pool_blocks) {
    int next_free_block = 0;
    for (int l = 0; l < cfg.n_layers; l++) {
      for (int b = 0; b < cfg.max_blocks_per_layer; b++)
        c->h_tables[(size_t)l * cfg.max_blocks_per_layer + b] = next_free_block++;
      c->n_mapped[l] = cfg.max_blocks_per_layer;
    }
  }
  if (hipMalloc(&c->d_tables, n_entries * sizeof(int32_t)) != hipSuccess ||
      hipMemcpy(c->d_tables, c->h_tables.data(), n_entries * sizeof(int32_t),
                hipMemcpyHostToDevice) != hipSuccess ||
      hipMalloc(&c->d_seq_len, sizeof(int32_t)) != hipSuccess ||
      hipMemset(c->d_seq_len, 0, sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&c->d_counters, (sde::kMaxAttnCounters + sde::kSpecScratchWords) *
                                    sizeof(uint32_t)) != hipSuccess ||
      hipMemset(c->d_counters, 0, (sde::kMaxAttnCounters + sde::kSpecScratchWords) *
                                      sizeof(uint32_t)) != hipSuccess ||
      hipDeviceGetAttribute(&c->n_cus, hipDeviceAttributeMultiprocessorCount, c->device) !=
          hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    release(c);
    return SDE_ERR_HIP;
  }
  *out = c;
  return SDE_OK;
}

int check_rows(const sde_kv_cache* c, int layer, int pos, int n) {
  if (!c) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= c->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  if (pos < 0 || n < 0) return SDE_ERR_INVALID_ARGUMENT;
  if ((int64_t)pos + n > sde::mapped_tokens(c, layer)) return SDE_ERR_CAPACITY;
  return SDE_OK;
}

}  // namespace

extern "C" {

const char* sde_status_string(int status) {
  switch (status) {
    case SDE_OK: return "ok";
    case SDE_ERR_INVALID_ARGUMENT: return "invalid argument";
    case SDE_ERR_CAPACITY: return "position beyond the layer's mapped blocks";
    case SDE_ERR_RANGE: return "value out of range (block table entry or rollback target)";
    case SDE_ERR_UNSUPPORTED: return "unsupported attention type, head_dim or block_size";
    case SDE_ERR_WORKSPACE: return "workspace too small";
    case SDE_ERR_HIP: return "HIP runtime error";
    case SDE_ERR_NO_DEVICE: return "no usable device";
    case SDE_ERR_IO: return "weight file cannot be read";
    case SDE_ERR_FORMAT: return "bad weight file header or tensor size";
    default: return "unknown status";
  }
}

int sde_kv_config_validate(const sde_kv_config* cfg) {
  return valid_config(cfg) ? SDE_OK : SDE_ERR_INVALID_ARGUMENT;
}

size_t sde_kv_pool_bytes(const sde_kv_config* cfg) {
  if (!valid_config(cfg)) return 0;
  return pool_bytes_of(resolved(cfg));
}

int sde_kv_cache_create(const sde_kv_config* cfg, sde_kv_cache** out) {
  if (!out) return SDE_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (!valid_config(cfg)) return SDE_ERR_INVALID_ARGUMENT;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SDE_ERR_NO_DEVICE;
  sde_kv_cache* c = new (std::nothrow) sde_kv_cache();
  if (!c) return SDE_ERR_HIP;
  c->cfg = resolved(cfg);
  c->device = dev;
  c->pool_bytes = pool_bytes_of(c->cfg);
  c->owns_pool = true;
  if (hipMalloc(&c->pool, c->pool_bytes) != hipSuccess ||
      hipMemset(c->pool, 0, c->pool_bytes) != hipSuccess) {
    release(c);
    return SDE_ERR_HIP;
  }
  return finish_create(c, out);
}

int sde_kv_cache_create_external(const sde_kv_config* cfg, void* d_pool,
                                 size_t pool_bytes, sde_kv_cache** out) {
  if (!out) return SDE_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (!valid_config(cfg) || !d_pool) return SDE_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)d_pool & 15u) != 0) return SDE_ERR_INVALID_ARGUMENT;
  const sde_kv_config r = resolved(cfg);
  if (pool_bytes < pool_bytes_of(r)) return SDE_ERR_CAPACITY;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SDE_ERR_NO_DEVICE;
  sde_kv_cache* c = new (std::nothrow) sde_kv_cache();
  if (!c) return SDE_ERR_HIP;
  c->cfg = r;
  c->device = dev;
  c->pool = static_cast<uint16_t*>(d_pool);
  c->pool_bytes = pool_bytes_of(r);
  c->owns_pool = false;
  return finish_create(c, out);
}

int sde_kv_cache_destroy(sde_kv_cache* cache) {
  if (!cache) return SDE_OK;
  sde::DeviceGuard g(cache->device);
  (void)hipDeviceSynchronize();
  release(cache);
  return SDE_OK;
}

int sde_kv_set_seq_len(sde_kv_cache* cache, int len, sde_stream_t stream) {
  if (!cache) return SDE_ERR_INVALID_ARGUMENT;
  if (len < 0 ||
      (int64_t)len > (int64_t)cache->cfg.max_blocks_per_layer * cache->cfg.block_size)
    return SDE_ERR_RANGE;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  hipLaunchKernelGGL(set_seq_len_kernel, dim3(1), dim3(64), 0,
                     (hipStream_t)stream, cache->d_seq_len, len);
  const int st = sde::launch_status();
  if (st == SDE_OK) {
    cache->seq_len = len;
    cache->seq_len_on_device = false;
  }
  return st;
}

int sde_kv_reset(sde_kv_cache* cache, sde_stream_t stream) {
  return sde_kv_set_seq_len(cache, 0, stream);
}

// Refreshes the host mirror after a device-side rewind (synchronizes).
static int refresh_seq_len(sde_kv_cache* cache) {
  if (!cache->seq_len_on_device) return SDE_OK;
  int v = 0;
  const int st = sde_kv_device_seq_len(cache, &v);
  if (st != SDE_OK) return st;
  cache->seq_len = v;
  cache->seq_len_on_device = false;
  return SDE_OK;
}

int sde_kv_rollback(sde_kv_cache* cache, int target_len, sde_stream_t stream) {
  if (!cache) return SDE_ERR_INVALID_ARGUMENT;
  const int st = refresh_seq_len(cache);
  if (st != SDE_OK) return st;
  if (target_len < 0 || target_len > cache->seq_len) return SDE_ERR_RANGE;
  return sde_kv_set_seq_len(cache, target_len, stream);
}

int sde_kv_seq_len(const sde_kv_cache* cache, int* out_len) {
  if (!cache || !out_len) return SDE_ERR_INVALID_ARGUMENT;
  const int st = refresh_seq_len(const_cast<sde_kv_cache*>(cache));
  if (st != SDE_OK) return st;
  *out_len = cache->seq_len;
  return SDE_OK;
}

int sde_spec_accept_greedy(sde_kv_cache* target, sde_kv_cache* draft,
                           const int32_t* d_draft_tokens, const int32_t* d_target_tokens, int k,
                           int target_save, int draft_save, int32_t* d_result,
                           sde_stream_t stream) {
  if (!target || !d_target_tokens || !d_result || (k > 0 && !d_draft_tokens))
    return SDE_ERR_INVALID_ARGUMENT;
  if (k < 0 || k > 64 || target_save < 0 || draft_save < 0) return SDE_ERR_RANGE;
  const bool has_draft = draft != nullptr && draft != target;
  const int64_t t_cap = (int64_t)target->cfg.max_blocks_per_layer * target->cfg.block_size;
  if ((int64_t)target_save + k + 1 > t_cap) return SDE_ERR_RANGE;
  if (has_draft) {
    if (draft->device != target->device) return SDE_ERR_INVALID_ARGUMENT;
    const int64_t d_cap = (int64_t)draft->cfg.max_blocks_per_layer * draft->cfg.block_size;
    if ((int64_t)draft_save + k > d_cap) return SDE_ERR_RANGE;
  }
  sde::DeviceGuard g(target->device);
  if (!g.ok()) return SDE_ERR_HIP;
  sde_kv_view tv, dv{};
  int st = sde_kv_get_view(target, &tv);
  if (st == SDE_OK && has_draft) st = sde_kv_get_view(draft, &dv);
  if (st != SDE_OK) return st;
  hipLaunchKernelGGL(spec_accept_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     d_draft_tokens, d_target_tokens, k, target_save, draft_save, tv, dv,
                     has_draft ? 1 : 0, d_result);
  st = sde::launch_status();
  if (st == SDE_OK) {
    target->seq_len_on_device = true;
    if (has_draft) draft->seq_len_on_device = true;
  }
  return st;
}

int sde_kv_device_seq_len(const sde_kv_cache* cache, int* out_len) {
  if (!cache || !out_len) return SDE_ERR_INVALID_ARGUMENT;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  int32_t v = 0;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&v, cache->d_seq_len, sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess)
    return SDE_ERR_HIP;
  *out_len = v;
  return SDE_OK;
}

int sde_kv_set_block_table(sde_kv_cache* cache, int layer,
                           const int32_t* host_table, int n_blocks) {
  if (!cache || !host_table) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= cache->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  if (n_blocks < 0 || n_blocks > cache->cfg.max_blocks_per_layer)
    return SDE_ERR_CAPACITY;
  for (int b = 0; b < n_blocks; b++)
    if (host_table[b] < 0 || host_table[b] >= cache->cfg.pool_blocks)
      return SDE_ERR_RANGE;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  const size_t row = (size_t)layer * cache->cfg.max_blocks_per_layer;
  if (n_blocks > 0 &&
      (hipMemcpy(cache->d_tables + row, host_table, (size_t)n_blocks * sizeof(int32_t),
                 hipMemcpyHostToDevice) != hipSuccess))
    return SDE_ERR_HIP;
  std::memcpy(cache->h_tables.data() + row, host_table, (size_t)n_blocks * sizeof(int32_t));
  cache->n_mapped[layer] = n_blocks;
  return SDE_OK;
}

int sde_kv_get_block_table(const sde_kv_cache* cache, int layer,
                           int32_t* host_table, int n_blocks) {
  if (!cache || !host_table) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= cache->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  if (n_blocks < 0 || n_blocks > cache->cfg.max_blocks_per_layer)
    return SDE_ERR_CAPACITY;
  std::memcpy(host_table,
              cache->h_tables.data() + (size_t)layer * cache->cfg.max_blocks_per_layer,
              (size_t)n_blocks * sizeof(int32_t));
  return SDE_OK;
}

int sde_kv_append(sde_kv_cache* cache, int layer, const float* d_k,
                  const float* d_v, int pos_base, int n_tokens,
                  sde_stream_t stream) {
  int st = check_rows(cache, layer, pos_base, n_tokens);
  if (st != SDE_OK) return st;
  if (n_tokens == 0) return SDE_OK;  // no-op; the row pointers may be NULL
  if (!d_k || !d_v) return SDE_ERR_INVALID_ARGUMENT;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  const int kv_dim = cache->cfg.kv_dim;
  const bool vec = (kv_dim % 4 == 0) && (((uintptr_t)d_k & 15u) == 0) &&
                   (((uintptr_t)d_v & 15u) == 0);
  const int per_block = vec ? kAppendThreads * 4 : kAppendThreads;
  // grid.y is limited to 65535: split long prefills.
  for (int done = 0; done < n_tokens; done += 65535) {
    const int n = (n_tokens - done) < 65535 ? (n_tokens - done) : 65535;
    dim3 grid((kv_dim + per_block - 1) / per_block, n);
    const float* k = d_k + (size_t)done * kv_dim;
    const float* v = d_v + (size_t)done * kv_dim;
    if (vec)
      hipLaunchKernelGGL(append_vec4_kernel, grid, dim3(kAppendThreads), 0,
                         (hipStream_t)stream, cache->pool, sde::layer_table(cache, layer),
                         k, v, kv_dim, cache->cfg.block_size, pos_base + done);
    else
      hipLaunchKernelGGL(append_scalar_kernel, grid, dim3(kAppendThreads), 0,
                         (hipStream_t)stream, cache->pool, sde::layer_table(cache, layer),
                         k, v, kv_dim, cache->cfg.block_size, pos_base + done);
    st = sde::launch_status();
    if (st != SDE_OK) return st;
  }
  return SDE_OK;
}

int sde_kv_write_fp16(sde_kv_cache* cache, int layer, const uint16_t* d_k,
                      const uint16_t* d_v, int pos_base, int n_tokens,
                      sde_stream_t stream) {
  int st = check_rows(cache, layer, pos_base, n_tokens);
  if (st != SDE_OK) return st;
  if (n_tokens == 0) return SDE_OK;  // no-op; the row pointers may be NULL
  if (!d_k || !d_v) return SDE_ERR_INVALID_ARGUMENT;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  const int kv_dim = cache->cfg.kv_dim;
  // grid.y is limited to 65535: split long prefills.
  for (int done = 0; done < n_tokens; done += 65535) {
    const int n = (n_tokens - done) < 65535 ? (n_tokens - done) : 65535;
    dim3 grid((kv_dim + kAppendThreads - 1) / kAppendThreads, n);
    hipLaunchKernelGGL(write_fp16_kernel, grid, dim3(kAppendThreads), 0,
                       (hipStream_t)stream, cache->pool, sde::layer_table(cache, layer),
                       d_k + (size_t)done * kv_dim, d_v + (size_t)done * kv_dim,
                       kv_dim, cache->cfg.block_size, pos_base + done);
    st = sde::launch_status();
    if (st != SDE_OK) return st;
  }
  return SDE_OK;
}

int sde_kv_gather(const sde_kv_cache* cache, int layer, int pos, int n_tokens,
                  float* d_k, float* d_v, sde_stream_t stream) {
  int st = check_rows(cache, layer, pos, n_tokens);
  if (st != SDE_OK) return st;
  if (n_tokens == 0) return SDE_OK;  // no-op; the row pointers may be NULL
  if (!d_k || !d_v) return SDE_ERR_INVALID_ARGUMENT;
  sde::DeviceGuard g(cache->device);
  if (!g.ok()) return SDE_ERR_HIP;
  const int kv_dim = cache->cfg.kv_dim;
  for (int done = 0; done < n_tokens; done += 65535) {
    const int n = (n_tokens - done) < 65535 ? (n_tokens - done) : 65535;
    dim3 grid((kv_dim + kAppendThreads - 1) / kAppendThreads, n);
    hipLaunchKernelGGL(gather_kernel, grid, dim3(kAppendThreads), 0,
                       (hipStream_t)stream, cache->pool, sde::layer_table(cache, layer),
                       d_k + (size_t)done * kv_dim, d_v + (size_t)done * kv_dim,
                       kv_dim, cache->cfg.block_size, pos + done);
    st = sde::launch_status();
    if (st != SDE_OK) return st;
  }
  return SDE_OK;
}

int sde_kv_get_view(const sde_kv_cache* cache, sde_kv_view* out) {
  if (!cache || !out) return SDE_ERR_INVALID_ARGUMENT;
  out->pool = cache->pool;
  out->block_tables = cache->d_tables;
  out->seq_len = cache->d_seq_len;
  out->n_layers = cache->cfg.n_layers;
  out->kv_dim = cache->cfg.kv_dim;
  out->block_size = cache->cfg.block_size;
  out->max_blocks_per_layer = cache->cfg.max_blocks_per_layer;
  out->pool_blocks = cache->cfg.pool_blocks;
  out->reserved = 0;
  return SDE_OK;
}

}  // extern "C"
