// Paged GQA attention for any head_dim up to 512 and any block size: the
// shapes libsde_paged's tile kernels (head_dim 64 / 128, block sizes that
// are multiples of 8) do not take.  The reference's
// device_flash_attention_gqa (attention.h:21-126) loops over any dph; this
// path keeps that generality on the GPU with plain fp32 arithmetic: q fp32
// (scaled by log2(e)/sqrt(dph)), K / V widened from fp16, an online softmax
// in exp2, the same causal rule (query m sees positions [0, pos_base + m];
// positions it does not see are never read into its sums) and the same
// split-context partitions and log-sum-exp combine as the tile kernels.
//
// Work: workgroup (partition, KV head, group of up to 8 rows), 256 threads.
// Per chunk of 256 tokens each thread computes the logits of one token for
// every row (its K row against q held in LDS), each wave reduces the max
// and sum of two rows, and each thread accumulates P.V for the features
// tid and tid + 256 of every row.  Bandwidth is not this path's aim: it is
// the correct answer for shapes the tile kernels reject.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attention_generic.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace gen {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 8;     // rows (query, head in group) per workgroup
constexpr int kChunk = 256;  // tokens per chunk: one per thread
constexpr float kNegInf = -__builtin_inff();

struct GenArgs {
  uint16_t* pool;
  const int32_t* table;
  const float* q;
  float* out;
  float* partials;  // [nkv][R][n_parts][dph + 2]: acc, then max, sum
  int kv_dim, bs;
  int nh, nkv, dph, G, R;
  int pos_base, L_max, n_parts, part_len;
  float qscale;
};

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Element offset of token t's K row in the pool (V is bs * kv_dim further).
__device__ __forceinline__ size_t k_row(const GenArgs& a, int t) {
  const int lb = t / a.bs;
  const int slot = t - lb * a.bs;
  return ((size_t)(uint32_t)a.table[lb] * 2u * (size_t)a.bs + (size_t)slot) * (size_t)a.kv_dim;
}

// rotate-half RoPE of element d of a head row x (rope_apply_inplace,
// model.cu:281-323): pair (j, j + dph/2) rotates by (pos / pos_div) *
// inv_freq[j]; an odd head_dim leaves its last element unrotated.
__device__ __forceinline__ float rope_elem(const float* x, int d, int dph, int pos,
                                           const GenRope& rp) {
  const int half = dph / 2;
  if (d >= 2 * half) return x[d];
  const int j = d < half ? d : d - half;
  float sn, cs;
  sincosf(((float)pos / rp.pos_div) * rp.inv_freq[j], &sn, &cs);
  const float x0 = x[j], x1 = x[j + half];
  return d < half ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
}

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
  __shared__ float qs[kRows][kMaxDph];
  __shared__ float sc[kRows][kChunk];
  __shared__ float row_m[kRows], row_l[kRows], row_alpha[kRows];
  const int part = blockIdx.x, h = blockIdx.y;
  const int rho0 = blockIdx.z * kRows;
  const int nr = min(kRows, a.R - rho0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dph = a.dph;

  // q rows (rotated when ROPE), pre-scaled into the log2 domain.
  for (int i = tid; i < nr * dph; i += kThreads) {
    const int r = i / dph, d = i - r * dph;
    const int rho = rho0 + r;
    const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
    const float* qrow = a.q + (size_t)m * a.nh * dph + (size_t)head * dph;
    const float x = ROPE ? rope_elem(qrow, d, dph, a.pos_base + m, rp) : qrow[d];
    qs[r][d] = x * a.qscale;
  }
  if (tid < kRows) {
    row_m[tid] = kNegInf;
    row_l[tid] = 0.f;
  }
  int lim[kRows];  // last position row r sees
#pragma unroll
  for (int r = 0; r < kRows; r++) lim[r] = a.pos_base + (rho0 + min(r, nr - 1)) / a.G;
  float acc[kRows][2];
#pragma unroll
  for (int r = 0; r < kRows; r++) acc[r][0] = acc[r][1] = 0.f;
  __syncthreads();

  const int t0 = part * a.part_len;
  const int t1 = min(a.L_max, t0 + a.part_len);
  const size_t kv_head = (size_t)h * dph;
  const size_t v_off = (size_t)a.bs * a.kv_dim;
  for (int c0 = t0; c0 < t1; c0 += kChunk) {
    // logits of token c0 + tid for every row
    const int t = c0 + tid;
    if (t < t1) {
      const uint16_t* kp = a.pool + k_row(a, t) + kv_head;
      float s[kRows];
#pragma unroll
      for (int r = 0; r < kRows; r++) s[r] = 0.f;
      for (int d = 0; d < dph; d++) {
        const float kd = h2f(kp[d]);
#pragma unroll
        for (int r = 0; r < kRows; r++) s[r] = __builtin_fmaf(qs[r][d], kd, s[r]);
      }
#pragma unroll
      for (int r = 0; r < kRows; r++)
        if (r < nr) sc[r][tid] = t <= lim[r] ? s[r] : kNegInf;
    } else {
#pragma unroll
      for (int r = 0; r < kRows; r++)
        if (r < nr) sc[r][tid] = kNegInf;
    }
    __syncthreads();

    // online softmax: wave w takes rows w and w + 4
    for (int r = wave; r < nr; r += kThreads / 64) {
      float v[kChunk / 64];
      float mx = kNegInf;
#pragma unroll
      for (int i = 0; i < kChunk / 64; i++) {
        v[i] = sc[r][lane + 64 * i];
        mx = fmaxf(mx, v[i]);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_old = row_m[r];
      const float m_new = fmaxf(m_old, mx);
      float alpha = 1.f, sum = 0.f;
      if (m_new != kNegInf) {
        alpha = exp2f(m_old - m_new);  // 0 while m_old is -inf
#pragma unroll
        for (int i = 0; i < kChunk / 64; i++) {
          v[i] = exp2f(v[i] - m_new);
          sum += v[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < kChunk / 64; i++) v[i] = 0.f;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
#pragma unroll
      for (int i = 0; i < kChunk / 64; i++) sc[r][lane + 64 * i] = v[i];
      if (lane == 0) {
        row_m[r] = m_new;
        row_l[r] = row_l[r] * alpha + sum;
        row_alpha[r] = alpha;
      }
    }
    __syncthreads();

    // P.V for features tid and tid + 256; positions a row does not see
    // are selected out (their V may hold anything, NaN included)
    const int n_tok = min(kChunk, t1 - c0);
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
      for (int r = 0; r < kRows; r++) acc[r][k] *= r < nr ? row_alpha[r] : 1.f;
    for (int tt = 0; tt < n_tok; tt++) {
      const int tok = c0 + tt;
      const uint16_t* vp = a.pool + k_row(a, tok) + v_off + kv_head;
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int d = tid + kThreads * k;
        if (d < dph) {
          const float vd = h2f(vp[d]);
#pragma unroll
          for (int r = 0; r < kRows; r++)
            if (r < nr && tok <= lim[r]) acc[r][k] = __builtin_fmaf(sc[r][tt], vd, acc[r][k]);
        }
      }
    }
    __syncthreads();
  }

  // the workgroup's rows: final output, or a partial for the combine
#pragma unroll
  for (int r = 0; r < kRows; r++) {
    if (r >= nr) break;
    const int rho = rho0 + r;
    const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
    if (a.n_parts == 1) {
      const float inv = 1.f / row_l[r];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int d = tid + kThreads * k;
        if (d < dph) a.out[(size_t)m * a.nh * dph + (size_t)head * dph + d] = acc[r][k] * inv;
      }
    } else {
      float* pp = a.partials + (((size_t)h * a.R + rho) * a.n_parts + part) * (size_t)(dph + 2);
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int d = tid + kThreads * k;
        if (d < dph) pp[d] = acc[r][k];
      }
      if (tid == 0) {
        pp[dph] = row_m[r];
        pp[dph + 1] = row_l[r];
      }
    }
  }
}

// Log-sum-exp merge of a row's partitions: workgroup (row rho, KV head).
__global__ __launch_bounds__(kThreads) void gen_combine_kernel(GenArgs a) {
  const int rho = blockIdx.x, h = blockIdx.y;
  const int dph = a.dph;
  const float* base = a.partials + ((size_t)h * a.R + rho) * a.n_parts * (size_t)(dph + 2);
  float M = kNegInf;
  for (int p = 0; p < a.n_parts; p++) M = fmaxf(M, base[(size_t)p * (dph + 2) + dph]);
  // A partition no position of which the row sees has sum 0 and max -inf
  // and is skipped; a NaN sum (a NaN logit) is kept, as in the reference.
  float L = 0.f;
  for (int p = 0; p < a.n_parts; p++) {
    const float* pp = base + (size_t)p * (dph + 2);
    if (pp[dph + 1] != 0.f) L += pp[dph + 1] * exp2f(pp[dph] - M);
  }
  const float inv = 1.f / L;
  const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
  for (int d = threadIdx.x; d < dph; d += kThreads) {
    float o = 0.f;
    for (int p = 0; p < a.n_parts; p++) {
      const float* pp = base + (size_t)p * (dph + 2);
      if (pp[dph + 1] != 0.f) o += pp[d] * exp2f(pp[dph] - M);
    }
    a.out[(size_t)m * a.nh * dph + (size_t)head * dph + d] = o * inv;
  }
}

}  // namespace

GenPlan generic_plan(int L_max, int nkv, int R, int dph, int n_cus, int max_parts) {
  GenPlan p;
  p.row_groups = (R + kRows - 1) / kRows;
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
