// Paged GQA attention for any head_dim up to 512 and any block size: the
// shapes libsde_paged's tile kernels (head_dim 64 / 128, block sizes that
// are multiples of 8) do not take.  The work unit's body (plain fp32,
// online softmax, split-context partitions) is
// sde/attention_generic_device.hpp's gen_unit, shared with the device API's
// fallback; this file holds the host path's kernels: the fused path's
// RoPE + append, one workgroup of 256 threads per (partition, KV head, row
// group), and the partition combine as a kernel of its own.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attention_generic.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace gen {
namespace {

constexpr int kThreads = 256;

// kv_cache_append of the window with k rotated (model_layer_kv_phase,
// model.cu:346-384): thread per (window row m, feature e), fp16 RNE.
__global__ __launch_bounds__(kThreads) void gen_rope_append_kernel(GenArgs a, GenRope rp) {
  const int m = blockIdx.y;
  const int e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= a.kv_dim) return;
  const int pos = a.pos_base + m;
  const int h = e / a.dph, d = e - h * a.dph;
  const float* krow = rp.k_new + (size_t)m * a.kv_dim + (size_t)h * a.dph;
  const size_t ko = k_row(a, pos);
  a.pool[ko + e] = f2h(rope_elem(krow, d, a.dph, pos, rp));
  a.pool[ko + (size_t)a.bs * a.kv_dim + e] = f2h(rp.v_new[(size_t)m * a.kv_dim + e]);
}

template <bool ROPE>
__global__ __launch_bounds__(kThreads) void gen_attn_kernel(GenArgs a, GenRope rp) {
  __shared__ GenLds lds;
  gen_unit<ROPE, kThreads>(a, &rp, blockIdx.x, blockIdx.y, blockIdx.z, lds);
}

// Log-sum-exp merge of a row's partitions: workgroup (row rho, KV head).
__global__ __launch_bounds__(kThreads) void gen_combine_kernel(GenArgs a) {
  gen_combine_row(a, blockIdx.y, blockIdx.x, threadIdx.x, kThreads);
}

}  // namespace

GenPlan generic_plan(int L_max, int nkv, int R, int dph, int n_cus, int max_parts) {
  GenPlan p;
  p.row_groups = (R + kGenRows - 1) / kGenRows;
  const int64_t units = (int64_t)nkv * p.row_groups;
  int64_t parts = (2 * (int64_t)n_cus) / units;
  if (parts > max_parts) parts = max_parts;
  const int64_t by_len = ((int64_t)L_max + 63) / 64;
  if (parts > by_len) parts = by_len;
  // Every plan's partials fit the static array of the allocation-free entry
  // point, so both entry points run the same plan (same results, same errors).
  const int64_t by_bytes =
      (int64_t)(SDE_NOALLOC_SCRATCH_BYTES / ((size_t)nkv * R * (size_t)(dph + 2) * sizeof(float)));
  if (parts > by_bytes) parts = by_bytes;
  if (parts < 1) parts = 1;
  const int64_t len = ((L_max + parts - 1) / parts + 63) / 64 * 64;
  p.part_len = (int)len;
  p.n_parts = (int)((L_max + len - 1) / len);
  return p;
}

size_t generic_partial_bytes(const GenPlan& p, int nkv, int R, int dph) {
  return p.n_parts > 1 ? (size_t)nkv * R * p.n_parts * (size_t)(dph + 2) * sizeof(float) : 0;
}

int generic_attention(uint16_t* pool, const int32_t* table, int kv_dim, int block_size,
                      const float* q, float* out, float* partials, int nh, int nkv, int dph,
                      int pos_base, int n_queries, const GenPlan& plan, const GenRope* rope,
                      hipStream_t stream) {
  if (dph > kMaxDph) return SDE_ERR_UNSUPPORTED;
  GenArgs a;
  a.pool = pool;
  a.table = table;
  a.q = q;
  a.out = out;
  a.partials = partials;
  a.kv_dim = kv_dim;
  a.bs = block_size;
  a.nh = nh;
  a.nkv = nkv;
  a.dph = dph;
  a.G = nh / nkv;
  a.R = n_queries * a.G;
  a.pos_base = pos_base;
  a.L_max = pos_base + n_queries;
  a.n_parts = plan.n_parts;
  a.part_len = plan.part_len;
  a.qscale = (float)(1.4426950408889634 / std::sqrt((double)dph));
  GenRope rp{};
  rp.pos_div = 1.f;
  if (rope) {
    rp = *rope;
    const dim3 grid((kv_dim + kThreads - 1) / kThreads, n_queries);
    gen_rope_append_kernel<<<grid, kThreads, 0, stream>>>(a, rp);
    const int st = launch_status();
    if (st != SDE_OK) return st;
  }
  const dim3 grid(plan.n_parts, nkv, plan.row_groups);
  if (rope)
    gen_attn_kernel<true><<<grid, kThreads, 0, stream>>>(a, rp);
  else
    gen_attn_kernel<false><<<grid, kThreads, 0, stream>>>(a, rp);
  int st = launch_status();
  if (st != SDE_OK || plan.n_parts == 1) return st;
  gen_combine_kernel<<<dim3(a.R, nkv), kThreads, 0, stream>>>(a);
  return launch_status();
}

}  // namespace gen
}  // namespace sde
