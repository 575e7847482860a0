// Test kernels for the device-side API of include/sde/attention_device.hpp
// and include/sde/matvec_device.hpp
// (test infrastructure, built beside libsde_paged by its build script): each
// wraps one reference-named device function in a kernel the way an
// in-kernel caller (a persistent decode loop) would use it, behind a plain
// C launcher that tests/test_gpu_device_api.py calls through ctypes.
#include <hip/hip_cooperative_groups.h>
#include <hip/hip_runtime.h>

#include "sde/attention_device.hpp"
#include "sde/spec_device.hpp"
#include "sde/kv_cache.hpp"
#include "sde/matvec_device.hpp"

namespace {

// One block per query, like cublas_attention_kernel (kernels.cu:904-940):
// query m sees positions [0, pos_base + m].  The device attention wants up
// to ~240 VGPRs per lane, so its callers are declared with at most 512
// threads per block.
__global__ __launch_bounds__(512) void attention_kernel(sde_kv_view kv, int layer, const float* q,
                                                        float* out, int nh, int nkv, int dph,
                                                        int pos_base, int attn_type,
                                                        int* status) {
  const int m = blockIdx.x;
  const size_t d = (size_t)nh * dph;
  const int st = sde::device_attention_dispatch(attn_type, q + m * d, out + m * d, kv, layer, nh,
                                                nkv, dph, pos_base + m + 1);
  if (threadIdx.x == 0) status[m] = st;
}

// One block per appended token (cublas_kv_append_kernel, kernels.cu:826-844).
__global__ void append_kernel(sde_kv_view kv, int layer, const float* k, const float* v,
                              int pos_base) {
  const int m = blockIdx.x;
  sde::kv_cache_append(kv, layer, k + (size_t)m * kv.kv_dim, v + (size_t)m * kv.kv_dim,
                       pos_base + m);
}

__global__ void read_kernel(sde_kv_view kv, int layer, int pos, float* k, float* v) {
  const int m = blockIdx.x;
  sde::kv_cache_read(kv, layer, pos + m, k + (size_t)m * kv.kv_dim, v + (size_t)m * kv.kv_dim);
}

__global__ void rollback_kernel(sde_kv_view kv, int target) { sde::kv_cache_rollback(kv, target); }

// The reference's layer attention (model.cu:400-432) with its own argument
// list: q_all and attn_out live in the caller's dynamic shared memory
// (smem[d..2d) and smem[0..d)), blk_logits in its scratch, the five
// scalars are __shared__; only the cache's type differs (sde_kv_view for
// KVCache).  One block per query m, total_len = pos_base + m + 1.
__global__ __launch_bounds__(512) void ref_layer_attention_kernel(sde_kv_view kv, int layer,
                                                                  const float* q, float* out,
                                                                  int nh, int nkv, int dph,
                                                                  int pos_base, int attn_type,
                                                                  int* status) {
  extern __shared__ float smem[];
  const int d = nh * dph;
  const int kd = nkv * dph;
  const int tid = threadIdx.x;
  const int m = blockIdx.x;
  float* q_all = smem + d;
  float* attn_out = smem;
  float* scratch = smem + 2 * d + 2 * kd;
  float* blk_logits = scratch;
  __shared__ float s_attn_m;
  __shared__ float s_attn_l;
  __shared__ float s_tile_m_new;
  __shared__ float s_attn_alpha;
  __shared__ float s_attn_inv_den;
  for (int i = tid; i < d; i += blockDim.x) q_all[i] = q[(size_t)m * d + i];
  const int total_len = pos_base + m + 1;
  for (int i = tid; i < d; i += blockDim.x) attn_out[i] = 0.0f;
  __syncthreads();
  const int st = sde::device_attention_dispatch(
      attn_type, q_all, attn_out, kv, layer, nh, nkv, dph, total_len, blk_logits, s_attn_m,
      s_attn_l, s_tile_m_new, s_attn_alpha, s_attn_inv_den);
  for (int i = tid; i < d; i += blockDim.x) out[(size_t)m * d + i] = attn_out[i];
  if (tid == 0) status[m] = st;
}

// The megakernel's RoPE'd-input step on block 0 (kernels.cu:2727-2739):
// kv_cache_append of the token at `seq`, zero g_attn, then
// device_attention_dispatch over seq + 1 positions with __shared__ scalars
// and scratch, the reference's argument lists.
__global__ __launch_bounds__(256) void ref_megakernel_step_kernel(sde_kv_view kv, int l,
                                                                  const float* g_k,
                                                                  const float* g_v,
                                                                  const float* g_q, float* g_attn,
                                                                  int nh, int nkv, int dph,
                                                                  int seq, int attn_type,
                                                                  int* status) {
  const int tid = threadIdx.x;
  const int d = nh * dph;
  __shared__ float s_scratch[64];
  if (blockIdx.x == 0) {
    sde::kv_cache_append(kv, l, g_k, g_v, seq);
    for (int i = tid; i < d; i += blockDim.x) g_attn[i] = 0.f;
    __syncthreads();
    __shared__ float s_m, s_l, s_tm, s_al, s_iv;
    const int st = sde::device_attention_dispatch(attn_type, g_q, g_attn, kv, l, nh, nkv, dph,
                                                  seq + 1, s_scratch, s_m, s_l, s_tm, s_al,
                                                  s_iv);
    if (tid == 0) status[0] = st;
  }
}

// Every block of an arbitrary grid calls the grid-cooperative attention
// (4-wave staging: 64 KiB of LDS, or 8 waves: 128 KiB).
template <int MaxWaves>
__global__ __launch_bounds__(512) void grid_attention_kernel(sde_kv_view kv, int layer,
                                                             const float* q, float* out, int nh,
                                                             int nkv, int dph, int pos_base,
                                                             int n_queries, void* ws,
                                                             size_t ws_bytes, int* status) {
  const int st = sde::device_flash_attention_gqa_grid<MaxWaves>(
      q, out, kv, layer, nh, nkv, dph, pos_base, n_queries, ws, ws_bytes);
  if (threadIdx.x == 0) status[blockIdx.x] = st;
}

// A persistent decode / verify loop in one cooperative launch, the shape of
// the reference's megakernel (kernels.cu:2727-2747, 3043-3093) with the
// attention spread over the whole grid: for step s and layer l, block 0
// appends the window's M tokens at pos[s] (block-cooperative
// kv_cache_append per token), grid barrier, every block runs the grid
// attention of the window, grid barrier; after the last layer block 0 sets
// seq_len to the next step's pos (an O(1) rewind when drafts were
// rejected) or, after the last step, to pos + M.
__global__ __launch_bounds__(512) void persistent_loop_kernel(sde_kv_view kv, const int* pos, int n_steps, int M,
                                       int nh, int nkv, int dph, const float* k, const float* v,
                                       const float* q, float* out, void* ws, size_t ws_bytes,
                                       int* status) {
  namespace cg = cooperative_groups;
  cg::grid_group grid = cg::this_grid();
  const size_t kvd = (size_t)kv.kv_dim;
  const size_t qd = (size_t)nh * dph;
  int st_all = SDE_OK;
  for (int s = 0; s < n_steps; s++) {
    for (int l = 0; l < kv.n_layers; l++) {
      const size_t sl = (size_t)s * kv.n_layers + l;
      if (blockIdx.x == 0)
        for (int m = 0; m < M; m++)
          sde::kv_cache_append(kv, l, k + (sl * M + m) * kvd, v + (sl * M + m) * kvd, pos[s] + m);
      grid.sync();
      const int st = sde::device_flash_attention_gqa_grid(q + sl * M * qd, out + sl * M * qd, kv,
                                                          l, nh, nkv, dph, pos[s], M, ws, ws_bytes);
      if (st != SDE_OK) st_all = st;
      grid.sync();
    }
    sde::kv_cache_rollback(kv, s + 1 < n_steps ? pos[s + 1] : pos[s] + M);
  }
  if (threadIdx.x == 0) status[blockIdx.x] = st_all;
}

// coop_layer_forward's output projection (kernels.cu:2742-2747): blocks
// take GEMV_COL_TILE-column stripes in turns and fold x @ W[:, stripe] into
// out with the block-level device_matvec_partial_accum (or the
// non-accumulating device_matvec_partial).
__global__ void stripe_matvec_kernel(const float* x, const uint16_t* W, float* out, int d_in,
                                     int d_out, int col_tile, int accumulate) {
  for (int ct = blockIdx.x; ct * col_tile < d_out; ct += gridDim.x) {
    const int cs = ct * col_tile;
    const int cc = cs + col_tile <= d_out ? col_tile : d_out - cs;
    if (accumulate)
      sde::device_matvec_partial_accum(x, W, out, d_in, d_out, cs, cc);
    else
      sde::device_matvec_partial(x, W, out, d_in, d_out, cs, cc);
  }
}

// device_matvec_batched (utils.h:248-280) by one block.
__global__ void batched_matvec_kernel(const float* x, const uint16_t* W, float* out, int d_in,
                                      int d_out, int B) {
  sde::device_matvec_batched(x, W, out, d_in, d_out, B);
}

// Every block of an arbitrary grid calls the grid-cooperative projection.
__global__ void grid_matvec_kernel(const float* x, const uint16_t* W, float* out, int d_in,
                                   int d_out, int M, int accumulate, void* ws, size_t ws_bytes,
                                   int* status) {
  const int st = sde::device_matvec_grid(x, W, out, d_in, d_out, M, accumulate, ws, ws_bytes);
  if (threadIdx.x == 0) status[blockIdx.x] = st;
}

// Every block of a cooperative grid calls the grid form of the stochastic
// acceptance, with the cooperative-groups grid barrier between its passes.
__global__ void stochastic_grid_kernel(const float* tl, const float* dl, const int32_t* drafts,
                                       int k, int V, float tt, float td, uint64_t seed,
                                       uint64_t* offset, int ts, int ds, sde_kv_view target,
                                       sde_kv_view draft, int has_draft, int32_t* result, void* ws,
                                       size_t ws_bytes, int* status) {
  namespace cg = cooperative_groups;
  cg::grid_group grid = cg::this_grid();
  const int st = sde::device_spec_accept_stochastic_grid(
      tl, dl, drafts, k, V, tt, td, seed, offset, ts, ds, target, has_draft ? &draft : nullptr,
      result, ws, ws_bytes, [&] { grid.sync(); });
  if (threadIdx.x == 0) status[blockIdx.x] = st;
}

// sde::attn::rope_sincos (the fused RoPE step's sin / cos) over n angles.
__global__ void rope_sincos_kernel(const float* x, float* sn, float* cs, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) sde::attn::rope_sincos(x[i], sn[i], cs[i]);
}

int status_of(hipError_t e) { return e == hipSuccess ? 0 : 6; }

}  // namespace

extern "C" {

int sdet_attention(const sde_kv_view* kv, int layer, const float* q, float* out, int nh, int nkv,
                   int dph, int pos_base, int n_queries, int threads, int attn_type, int* status,
                   void* stream) {
  if (!kv || threads < 64 || threads % 64 != 0 || threads > 512 || n_queries < 1) return 1;
  attention_kernel<<<n_queries, threads, 0, (hipStream_t)stream>>>(*kv, layer, q, out, nh, nkv, dph,
                                                                   pos_base, attn_type, status);
  return status_of(hipGetLastError());
}

// ref_layer_attention_kernel: one block per query; dynamic shared memory
// (2d + 2kd + 16) floats as model.cu sizes it.
int sdet_ref_layer_attention(const sde_kv_view* kv, int layer, const float* q, float* out, int nh,
                             int nkv, int dph, int pos_base, int n_queries, int threads,
                             int attn_type, int* status, void* stream) {
  if (!kv || threads < 64 || threads % 64 != 0 || threads > 512 || n_queries < 1) return 1;
  const size_t smem = (size_t)(2 * nh * dph + 2 * nkv * dph + 16) * sizeof(float);
  if (smem > 64 * 1024) return 1;
  ref_layer_attention_kernel<<<n_queries, threads, smem, (hipStream_t)stream>>>(
      *kv, layer, q, out, nh, nkv, dph, pos_base, attn_type, status);
  return status_of(hipGetLastError());
}

int sdet_ref_megakernel_step(const sde_kv_view* kv, int layer, const float* k, const float* v,
                             const float* q, float* attn, int nh, int nkv, int dph, int seq,
                             int blocks, int attn_type, int* status, void* stream) {
  if (!kv || blocks < 1) return 1;
  ref_megakernel_step_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
      *kv, layer, k, v, q, attn, nh, nkv, dph, seq, attn_type, status);
  return status_of(hipGetLastError());
}

// max_waves 4 or 8: the grid function's staging variant.
int sdet_grid_attention(const sde_kv_view* kv, int layer, const float* q, float* out, int nh,
                        int nkv, int dph, int pos_base, int n_queries, int blocks, int threads,
                        int max_waves, void* ws, size_t ws_bytes, int* status, void* stream) {
  if (!kv || blocks < 1 || threads < 64 || threads % 64 != 0 || threads > 512) return 1;
  if (max_waves == 8)
    grid_attention_kernel<8><<<blocks, threads, 0, (hipStream_t)stream>>>(
        *kv, layer, q, out, nh, nkv, dph, pos_base, n_queries, ws, ws_bytes, status);
  else if (max_waves == 4)
    grid_attention_kernel<4><<<blocks, threads, 0, (hipStream_t)stream>>>(
        *kv, layer, q, out, nh, nkv, dph, pos_base, n_queries, ws, ws_bytes, status);
  else
    return 1;
  return status_of(hipGetLastError());
}

// Cooperative launch of persistent_loop_kernel; blocks must all be resident
// (returns 2 when the device cannot hold that many).
int sdet_persistent_loop(const sde_kv_view* kv, const int* d_pos, int n_steps, int M, int nh,
                         int nkv, int dph, const float* k, const float* v, const float* q,
                         float* out, void* ws, size_t ws_bytes, int* status, int blocks,
                         int threads, void* stream) {
  if (!kv || blocks < 1 || threads < 256 || threads % 64 != 0 || threads > 512) return 1;
  int dev = 0, per_cu = 0, cus = 0, coop = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, persistent_loop_kernel, threads, 0) !=
          hipSuccess)
    return 6;
  if (!coop || blocks > per_cu * cus) return 2;
  sde_kv_view view = *kv;
  void* args[] = {&view, (void*)&d_pos, &n_steps, &M, &nh, &nkv, &dph, (void*)&k, (void*)&v,
                  (void*)&q, &out, &ws, &ws_bytes, &status};
  return status_of(hipLaunchCooperativeKernel((const void*)persistent_loop_kernel, dim3(blocks),
                                              dim3(threads), args, 0, (hipStream_t)stream));
}

// Cooperative launch of stochastic_grid_kernel (blocks all resident).
int sdet_stochastic_grid(const float* tl, const float* dl, const int32_t* drafts, int k, int V,
                         float tt, float td, uint64_t seed, uint64_t* offset, int ts, int ds,
                         const sde_kv_view* target, const sde_kv_view* draft, int32_t* result,
                         void* ws, size_t ws_bytes, int* status, int blocks, int threads,
                         void* stream) {
  if (!target || blocks < 1 || threads < 64 || threads > 1024) return 1;
  int dev = 0, per_cu = 0, cus = 0, coop = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, stochastic_grid_kernel, threads, 0) !=
          hipSuccess)
    return 6;
  if (!coop || blocks > per_cu * cus) return 2;
  sde_kv_view t = *target;
  sde_kv_view d = draft ? *draft : sde_kv_view{};
  int has_draft = draft ? 1 : 0;
  void* args[] = {(void*)&tl, (void*)&dl, (void*)&drafts, &k, &V, &tt, &td, &seed, &offset, &ts,
                  &ds, &t, &d, &has_draft, &result, &ws, &ws_bytes, &status};
  return status_of(hipLaunchCooperativeKernel((const void*)stochastic_grid_kernel, dim3(blocks),
                                              dim3(threads), args, 0, (hipStream_t)stream));
}

int sdet_append(const sde_kv_view* kv, int layer, const float* k, const float* v, int pos_base,
                int n, int threads, void* stream) {
  if (!kv || threads < 64 || threads > 1024 || n < 1) return 1;
  append_kernel<<<n, threads, 0, (hipStream_t)stream>>>(*kv, layer, k, v, pos_base);
  return status_of(hipGetLastError());
}

int sdet_read(const sde_kv_view* kv, int layer, int pos, int n, float* k, float* v, int threads,
              void* stream) {
  if (!kv || threads < 64 || threads > 1024 || n < 1) return 1;
  read_kernel<<<n, threads, 0, (hipStream_t)stream>>>(*kv, layer, pos, k, v);
  return status_of(hipGetLastError());
}

// The C++ host names of sde/kv_cache.hpp end to end on a fresh cache:
// alloc, tables, append M rows at pos_base, set_seq_len, attention of the
// n_q-query window at q_base, rollback to `rollback_to`; copies the pool to
// pool_out and the device seq_len to *seq_len_out, then frees the cache.
int sdet_cpp_pipeline(int n_layers, int kv_dim, int max_blocks, int block_size, int pool_blocks,
                      const int32_t* tables, int layer, const float* k, const float* v,
                      int pos_base, int M, const float* q, float* out, int nh, int nkv, int dph,
                      int q_base, int n_q, int rollback_to, void* pool_out, int* seq_len_out) {
  sde::KVCache kv;
  sde::kv_cache_alloc(kv, n_layers, kv_dim, max_blocks, block_size, pool_blocks);
  for (int l = 0; l < n_layers; l++)
    sde::kv_cache_set_block_table(kv, l, tables + (size_t)l * max_blocks, max_blocks);
  sde::cublas_kv_append_kernel(kv, layer, k, v, kv_dim, pos_base, M);
  sde::set_seq_len_kernel(kv, pos_base + M);
  sde::cublas_attention_kernel(q, out, kv, layer, nh, nkv, dph, kv_dim, q_base, n_q);
  sde::kv_cache_rollback(kv, rollback_to);
  const size_t pool_bytes = (size_t)pool_blocks * 2u * block_size * kv_dim * 2u;
  hipError_t e = hipMemcpy(pool_out, kv.view.pool, pool_bytes, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(seq_len_out, kv.view.seq_len, sizeof(int), hipMemcpyDeviceToHost);
  sde::kv_cache_free(kv);
  return status_of(e);
}

int sdet_rollback(const sde_kv_view* kv, int target, void* stream) {
  if (!kv) return 1;
  rollback_kernel<<<1, 64, 0, (hipStream_t)stream>>>(*kv, target);
  return status_of(hipGetLastError());
}

int sdet_stripe_matvec(const float* x, const uint16_t* W, float* out, int d_in, int d_out,
                       int col_tile, int accumulate, int blocks, int threads, void* stream) {
  if (blocks < 1 || threads < 64 || threads % 64 != 0 || threads > 1024 || col_tile < 1 ||
      col_tile % 8 != 0 || d_out % 8 != 0)
    return 1;
  stripe_matvec_kernel<<<blocks, threads, 0, (hipStream_t)stream>>>(x, W, out, d_in, d_out,
                                                                    col_tile, accumulate);
  return status_of(hipGetLastError());
}

int sdet_batched_matvec(const float* x, const uint16_t* W, float* out, int d_in, int d_out,
                        int B, int threads, void* stream) {
  if (threads < 64 || threads % 64 != 0 || threads > 1024 || d_out % 8 != 0 || B < 1) return 1;
  batched_matvec_kernel<<<1, threads, 0, (hipStream_t)stream>>>(x, W, out, d_in, d_out, B);
  return status_of(hipGetLastError());
}

int sdet_grid_matvec(const float* x, const uint16_t* W, float* out, int d_in, int d_out, int M,
                     int accumulate, int blocks, int threads, void* ws, size_t ws_bytes,
                     int* status, void* stream) {
  if (blocks < 1 || threads < 64 || threads % 64 != 0 || threads > 1024) return 1;
  grid_matvec_kernel<<<blocks, threads, 0, (hipStream_t)stream>>>(
      x, W, out, d_in, d_out, M, accumulate, ws, ws_bytes, status);
  return status_of(hipGetLastError());
}

int sdet_rope_sincos(const float* x, float* sn, float* cs, int n, void* stream) {
  if (n < 1) return 1;
  rope_sincos_kernel<<<(n + 255) / 256, 256, 0, (hipStream_t)stream>>>(x, sn, cs, n);
  return status_of(hipGetLastError());
}

}  // extern "C"
