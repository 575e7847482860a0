// Paged GQA attention for any head_dim up to 512 and any block size, as
// device code: the body of libsde_paged's generic kernel (the shapes its
// MFMA tile kernels -- head_dim 64 / 128, block sizes that are multiples of
// 8 -- do not take), and the block- and grid-cooperative forms the device
// API (sde/attention_device.hpp) falls back to for those shapes.
//
// Reference: device_flash_attention_gqa (attention.h:21-126) loops over any
// dph.  This path keeps that generality with plain fp32 arithmetic: q fp32
// (scaled by log2(e)/sqrt(dph)), K / V widened from fp16, an online softmax
// in exp2, the causal rule (query m sees positions [0, pos_base + m];
// positions it does not see are never read into its sums), split-context
// partitions and a log-sum-exp combine.
//
// Work unit: (partition, KV head, group of up to 8 rows) on one workgroup,
// NT = 64, 128 or 256 active threads (threads past NT only meet the
// barriers).  Per chunk of NT tokens each thread computes the logits of one
// token for every row (its K row against q held in LDS), each wave reduces
// the max and sum of its rows, and each thread accumulates P.V for the
// features tid, tid + NT, ... of every row.  Bandwidth is not this path's
// aim: it is the correct answer for shapes the tile kernels reject.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "sde_paged_kv.h"

namespace sde {
namespace gen {

constexpr int kMaxDph = 512;  // head_dim limit (LDS for q)
constexpr int kGenRows = 8;   // rows (query, head in group) per work unit
constexpr int kGenChunk = 256;

// The generic path serves every (dph, block size) the tile kernels do not.
__host__ __device__ inline bool needs_generic(int dph, int block_size) {
  return !(dph == 64 || dph == 128) || block_size % 8 != 0;
}

// Rotate-half RoPE of the fused entry point: inv_freq[j] for j < dph / 2
// (theta already NTK-scaled, computed on the host in double precision and
// rounded to fp32) and the linear / YaRN position divisor.
struct GenRope {
  const float* k_new;  // [M][kv_dim] fp32, before RoPE
  const float* v_new;  // [M][kv_dim] fp32
  float pos_div;
  float inv_freq[kMaxDph / 2];
};

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

// The work unit's LDS (24.1 KiB): the rows' scaled q, a chunk's logits /
// probabilities, and the rows' running max, sum and rescale factor.  The
// caller provides it (the device API lends the tile path's staging area).
struct GenLds {
  float qs[kGenRows][kMaxDph];
  float sc[kGenRows][kGenChunk];
  float row_m[kGenRows], row_l[kGenRows], row_alpha[kGenRows];
};

// Work unit (part, KV head h, row group rg) on the calling workgroup
// (blockDim.x >= NT; every thread calls it): writes the normalised rows
// (one partition) or their partial (acc, max, sum).  rp: the RoPE of q when
// ROPE (k was rotated by the append).
template <bool ROPE, int NT>
__device__ __forceinline__ void gen_unit(const GenArgs& a, const GenRope* rp, int part, int h,
                                         int rg, GenLds& lds) {
  static_assert(NT == 64 || NT == 128 || NT == 256, "active threads");
  constexpr int FPT = kMaxDph / NT;  // P.V features per thread
  constexpr float kNegInf = -__builtin_inff();
  auto& qs = lds.qs;
  auto& sc = lds.sc;
  auto& row_m = lds.row_m;
  auto& row_l = lds.row_l;
  auto& row_alpha = lds.row_alpha;
  const int rho0 = rg * kGenRows;
  const int nr = min(kGenRows, a.R - rho0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool active = tid < NT;
  const int dph = a.dph;

  __syncthreads();  // the previous unit's readers of the shared arrays are done
  if (active) {
    // q rows (rotated when ROPE), pre-scaled into the log2 domain.
    for (int i = tid; i < nr * dph; i += NT) {
      const int r = i / dph, d = i - r * dph;
      const int rho = rho0 + r;
      const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
      const float* qrow = a.q + (size_t)m * a.nh * dph + (size_t)head * dph;
      float x;
      if constexpr (ROPE)
        x = rope_elem(qrow, d, dph, a.pos_base + m, *rp);
      else
        x = qrow[d];
      qs[r][d] = x * a.qscale;
    }
    if (tid < kGenRows) {
      row_m[tid] = kNegInf;
      row_l[tid] = 0.f;
    }
  }
  int lim[kGenRows];  // last position row r sees
#pragma unroll
  for (int r = 0; r < kGenRows; r++) lim[r] = a.pos_base + (rho0 + min(r, nr - 1)) / a.G;
  float acc[kGenRows][FPT];
#pragma unroll
  for (int r = 0; r < kGenRows; r++)
#pragma unroll
    for (int k = 0; k < FPT; k++) acc[r][k] = 0.f;
  __syncthreads();

  const int t0 = part * a.part_len;
  const int t1 = min(a.L_max, t0 + a.part_len);
  const size_t kv_head = (size_t)h * dph;
  const size_t v_off = (size_t)a.bs * a.kv_dim;
  for (int c0 = t0; c0 < t1; c0 += NT) {
    // logits of token c0 + tid for every row
    if (active) {
      const int t = c0 + tid;
      if (t < t1) {
        const uint16_t* kp = a.pool + k_row(a, t) + kv_head;
        float s[kGenRows];
#pragma unroll
        for (int r = 0; r < kGenRows; r++) s[r] = 0.f;
        for (int d = 0; d < dph; d++) {
          const float kd = h2f(kp[d]);
#pragma unroll
          for (int r = 0; r < kGenRows; r++) s[r] = __builtin_fmaf(qs[r][d], kd, s[r]);
        }
#pragma unroll
        for (int r = 0; r < kGenRows; r++)
          if (r < nr) sc[r][tid] = t <= lim[r] ? s[r] : kNegInf;
      } else {
#pragma unroll
        for (int r = 0; r < kGenRows; r++)
          if (r < nr) sc[r][tid] = kNegInf;
      }
    }
    __syncthreads();

    // online softmax: wave w takes rows w, w + NT/64, ...
    if (active) {
      for (int r = wave; r < nr; r += NT / 64) {
        float v[NT / 64];
        float mx = kNegInf;
#pragma unroll
        for (int i = 0; i < NT / 64; i++) {
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
          for (int i = 0; i < NT / 64; i++) {
            v[i] = exp2f(v[i] - m_new);
            sum += v[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < NT / 64; i++) v[i] = 0.f;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
#pragma unroll
        for (int i = 0; i < NT / 64; i++) sc[r][lane + 64 * i] = v[i];
        if (lane == 0) {
          row_m[r] = m_new;
          row_l[r] = row_l[r] * alpha + sum;
          row_alpha[r] = alpha;
        }
      }
    }
    __syncthreads();

    // P.V for features tid, tid + NT, ...; positions a row does not see
    // are selected out (their V may hold anything, NaN included)
    if (active) {
      const int n_tok = min(NT, t1 - c0);
#pragma unroll
      for (int k = 0; k < FPT; k++)
#pragma unroll
        for (int r = 0; r < kGenRows; r++) acc[r][k] *= r < nr ? row_alpha[r] : 1.f;
      for (int tt = 0; tt < n_tok; tt++) {
        const int tok = c0 + tt;
        const uint16_t* vp = a.pool + k_row(a, tok) + v_off + kv_head;
#pragma unroll
        for (int k = 0; k < FPT; k++) {
          const int d = tid + NT * k;
          if (d < dph) {
            const float vd = h2f(vp[d]);
#pragma unroll
            for (int r = 0; r < kGenRows; r++)
              if (r < nr && tok <= lim[r]) acc[r][k] = __builtin_fmaf(sc[r][tt], vd, acc[r][k]);
          }
        }
      }
    }
    __syncthreads();
  }

  // the unit's rows: final output, or a partial for the combine
  if (!active) return;
#pragma unroll
  for (int r = 0; r < kGenRows; r++) {
    if (r >= nr) break;
    const int rho = rho0 + r;
    const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
    if (a.n_parts == 1) {
      const float inv = 1.f / row_l[r];
#pragma unroll
      for (int k = 0; k < FPT; k++) {
        const int d = tid + NT * k;
        if (d < dph) a.out[(size_t)m * a.nh * dph + (size_t)head * dph + d] = acc[r][k] * inv;
      }
    } else {
      float* pp = a.partials + (((size_t)h * a.R + rho) * a.n_parts + part) * (size_t)(dph + 2);
#pragma unroll
      for (int k = 0; k < FPT; k++) {
        const int d = tid + NT * k;
        if (d < dph) pp[d] = acc[r][k];
      }
      if (tid == 0) {
        pp[dph] = row_m[r];
        pp[dph + 1] = row_l[r];
      }
    }
  }
}

// The log-sum-exp merge of row rho (KV head h) over its partitions: the
// row's max M and sum L (every thread computes them; a partition no
// position of which the row sees has sum 0 and max -inf and is skipped; a
// NaN sum is kept, as in the reference), then features d = d0, d0 + step, ...
__device__ __forceinline__ void gen_combine_row(const GenArgs& a, int h, int rho, int d0,
                                                int step) {
  const int dph = a.dph;
  const float* base = a.partials + ((size_t)h * a.R + rho) * a.n_parts * (size_t)(dph + 2);
  float M = -__builtin_inff();
  for (int p = 0; p < a.n_parts; p++) M = fmaxf(M, base[(size_t)p * (dph + 2) + dph]);
  float L = 0.f;
  for (int p = 0; p < a.n_parts; p++) {
    const float* pp = base + (size_t)p * (dph + 2);
    if (pp[dph + 1] != 0.f) L += pp[dph + 1] * exp2f(pp[dph] - M);
  }
  const float inv = 1.f / L;
  const int m = rho / a.G, head = h * a.G + (rho - m * a.G);
  for (int d = d0; d < dph; d += step) {
    float o = 0.f;
    for (int p = 0; p < a.n_parts; p++) {
      const float* pp = base + (size_t)p * (dph + 2);
      if (pp[dph + 1] != 0.f) o += pp[d] * exp2f(pp[dph] - M);
    }
    a.out[(size_t)m * a.nh * dph + (size_t)head * dph + d] = o * inv;
  }
}

// Active threads for a workgroup of `threads` (>= 64).
__device__ __forceinline__ int gen_threads(int threads) {
  return threads >= 256 ? 256 : (threads >= 128 ? 128 : 64);
}

// Every unit of a call on the calling block, one partition each (the
// output is written directly).
template <int NT>
__device__ __forceinline__ void gen_block_units(const GenArgs& a, GenLds& lds) {
  const int rgs = (a.R + kGenRows - 1) / kGenRows;
  for (int u = 0; u < a.nkv * rgs; u++)
    gen_unit<false, NT>(a, nullptr, 0, u % a.nkv, u / a.nkv, lds);
  __syncthreads();
}

// The items (partition, KV head, row group) of a call, taken by the grid's
// blocks in turns; the last block to finish a (KV head, row group) merges
// its partitions.  Partials are plain stores made visible device-wide by
// one agent-scope release fence before the arrival; the last arrival
// acquires before reading them.  counters[kvh * row_groups + rg] start at
// zero and are left at zero.
template <int NT>
__device__ __forceinline__ void gen_grid_items(const GenArgs& a, uint32_t* counters, GenLds& lds) {
  __shared__ int s_last;
  const int rgs = (a.R + kGenRows - 1) / kGenRows;
  const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
  const int block = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int items = a.n_parts * a.nkv * rgs;
  for (int it = block; it < items; it += n_blocks) {
    const int part = it % a.n_parts;
    const int rest = it / a.n_parts;
    const int h = rest % a.nkv, rg = rest / a.nkv;
    gen_unit<false, NT>(a, nullptr, part, h, rg, lds);
    if (a.n_parts == 1) continue;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      uint32_t* ctr = counters + (size_t)h * rgs + rg;
      const uint32_t prev =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (uint32_t)(a.n_parts - 1);
      if (last) {
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
      s_last = last;
    }
    __syncthreads();
    if (s_last) {
      const int rho0 = rg * kGenRows;
      const int nr = min(kGenRows, a.R - rho0);
      for (int r = 0; r < nr; r++)
        gen_combine_row(a, h, rho0 + r, (int)threadIdx.x, (int)blockDim.x);
    }
  }
  __syncthreads();
}

}  // namespace gen
}  // namespace sde
