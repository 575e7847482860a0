// Stochastic acceptance of speculative decoding on the device, for gfx950.
//
// Computes what the reference's stochastic round computes after a verify
// pass -- batch_stochastic_accept_kernel (kernels.cu:550-572), the
// correction sample on the first rejection (device_corrected_adjusted_sample,
// kernels.cu:319-380) and the bonus sample when every draft is accepted
// (softmax_sample_temperature_kernel) -- followed by the greedy-style rewind
// of both caches (kernels.cu:2428-2466).  The reference runs these on
// thread 0 of one block, serially over the vocabulary.  Here each window
// row is cut into vocabulary slices of ~4096 tokens, one 1024-thread
// workgroup each: a first kernel reduces each slice's temperature-softmax
// (max, sum), a second merges them per row (in slice order), applies the
// accept test, and sums each slice's sampling weights; the last slice of a
// row to arrive finds the slice and then the token where the cumulative
// weight crosses u * total (the correction token for a draft row, the
// bonus token for row k), and the last row to arrive picks the first
// rejection, writes the results and rewinds.  Every reduction and search
// runs in a fixed order, so a call is a pure function of its inputs, the
// seed and the call index.  The inverse-CDF token order is slice-major,
// then l % 1024, then l / 1024 of the offset l in the slice (coalesced
// passes); the reference walks tokens in index order with its own
// generator, so individual draws differ from it and only their
// distribution is shared.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cmath>

#include "sde/spec_device.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace spec {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

struct StochArgs {
  const float* target_logits;  // [k+1][V]
  const float* draft_logits;   // [k][V]
  const int32_t* draft_tokens;
  int k;
  int V;
  int S;  // vocabulary slices per row (one workgroup each)
  int L;  // tokens per slice
  float inv_tt;  // 1 / target temperature
  float inv_td;  // 1 / draft temperature
  uint64_t seed;
  uint64_t* offset;  // call index, incremented by the call
  int target_save;
  int draft_save;
  sde_kv_view target;
  sde_kv_view draft;
  int has_draft;
  int32_t* result;    // k+5
  uint32_t* scratch;  // layout: Scratch; counters zero at rest
};

constexpr int kUnroll = 16;  // loads in flight per thread and row

// Adds x to a running (max, sum of exp(. - max)); -inf (a masked logit)
// adds nothing.
__device__ __forceinline__ void ms_add(float& m, float& s, float x) {
  if (x > m) {
    s = (m == -INFINITY ? 0.f : s * __expf(m - x)) + 1.f;
    m = x;
  } else if (x != -INFINITY) {
    s += __expf(x - m);
  }
}

// Online (max, sum of exp(x - max)) pair merge.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.f : s * __expf(m - mn);
  const float b = m2 == -INFINITY ? 0.f : s2 * __expf(m2 - mn);
  m = mn;
  s = a + b;
}

// Block-wide (max, sum) pairs: xor butterfly in each wave, then the waves'
// pairs in wave order.  Every thread gets the result.
__device__ void block_ms(float& m, float& s, float2* lds) {
  for (int off = 32; off > 0; off >>= 1)
    ms_merge(m, s, __shfl_xor(m, off), __shfl_xor(s, off));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[w] = make_float2(m, s);
  __syncthreads();
  m = -INFINITY;
  s = 0.f;
  for (int i = 0; i < kWaves; i++) ms_merge(m, s, lds[i].x, lds[i].y);
}

__device__ float block_sum(float x, float* lds) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = x;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kWaves; i++) t += lds[i];
  return t;
}

// Two block sums at once, each in block_sum's order (the same bits).
__device__ float2 block_sum2(float x, float y, float2* lds) {
  for (int off = 32; off > 0; off >>= 1) {
    x += __shfl_xor(x, off);
    y += __shfl_xor(y, off);
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = make_float2(x, y);
  __syncthreads();
  float2 t = make_float2(0.f, 0.f);
  for (int i = 0; i < kWaves; i++) {
    t.x += lds[i].x;
    t.y += lds[i].y;
  }
  return t;
}

// Exclusive prefix of x over the threads in thread order.
__device__ float block_exclusive_scan(float x, float* lds) {
  const int lane = threadIdx.x & 63;
  float incl = x;
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  __syncthreads();
  if (lane == 63) lds[threadIdx.x >> 6] = incl;
  __syncthreads();
  float before = 0.f;
  for (int i = 0; i < (int)(threadIdx.x >> 6); i++) before += lds[i];
  return before + incl - x;
}

// Sampling weight of token i of row b: the residual max(0, p - q) for a
// draft row (or p when the residual is empty), p for the bonus row.
struct RowWeights {
  const float* p;
  const float* q;  // null for the bonus row or when sampling from p
  float mp, inv_sp, mq, inv_sq, inv_tt, inv_td;
  __device__ __forceinline__ float of(float pl, float ql) const {
    const float pi = __expf(pl * inv_tt - mp) * inv_sp;
    if (!q) return pi;
    const float qi = __expf(ql * inv_td - mq) * inv_sq;
    return fmaxf(pi - qi, 0.f);
  }
  __device__ __forceinline__ float operator()(int i) const { return of(p[i], q ? q[i] : 0.f); }
  // This thread's sums of the residual max(0, p - q) and of p over tokens
  // lo + tid, lo + tid + 1024, ... below hi in one pass (q non-null); each
  // sum in thread_sum's order.
  __device__ __forceinline__ float2 thread_sums(int tid, int lo, int hi) const {
    float cr = 0.f, cp = 0.f;
    for (int i0 = lo + tid; i0 < hi; i0 += kThreads * kUnroll) {
      float xp[kUnroll], xq[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; u++) {
        const int i = i0 + u * kThreads;
        xp[u] = i < hi ? p[i] : -INFINITY;
        xq[u] = i < hi ? q[i] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; u++)
        if (i0 + u * kThreads < hi) {
          const float pi = __expf(xp[u] * inv_tt - mp) * inv_sp;
          const float qi = __expf(xq[u] * inv_td - mq) * inv_sq;
          cr += fmaxf(pi - qi, 0.f);
          cp += pi;
        }
    }
    return make_float2(cr, cp);
  }
  // Sum of this thread's weights over tokens lo + tid, lo + tid + 1024, ...
  // below hi, loads batched.
  __device__ __forceinline__ float thread_sum(int tid, int lo, int hi) const {
    float cs = 0.f;
    for (int i0 = lo + tid; i0 < hi; i0 += kThreads * kUnroll) {
      float xp[kUnroll], xq[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; u++) {
        const int i = i0 + u * kThreads;
        xp[u] = i < hi ? p[i] : -INFINITY;
        xq[u] = (q && i < hi) ? q[i] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; u++)
        if (i0 + u * kThreads < hi) cs += of(xp[u], xq[u]);
    }
    return cs;
  }
};

// Scratch words: [0] row-arrival counter; [1 + r] slice-arrival counter of
// row r; [1 + R + 2r] (flag, token) of row r; then per (row, slice) the
// statistics (mp, sp, mq, sq) and the weight totals (residual, p).
struct Scratch {
  uint32_t* base;
  int R;  // rows = k + 1
  int S;
  __device__ uint32_t* rows_arrived() const { return base; }
  __device__ uint32_t* slices_arrived(int r) const { return base + 1 + r; }
  __device__ uint32_t* row_out(int r) const { return base + 1 + R + 2 * r; }
  __device__ float* stats(int r, int s) const {
    return reinterpret_cast<float*>(base + 1 + 3 * R) + 4 * ((size_t)r * S + s);
  }
  __device__ float* totals(int r, int s) const {
    return reinterpret_cast<float*>(base + 1 + 3 * R) + 4 * (size_t)R * S + 2 * ((size_t)r * S + s);
  }
};

__device__ __forceinline__ float ld_dev(const float* p) {
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_dev(float* p, float x) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, x),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Kernel 1: (max, sum) of the temperature-scaled target (and draft) logits
// of one vocabulary slice per workgroup; thread t takes the slice's tokens
// t, t + 1024, ... with kUnroll loads in flight.
__global__ __launch_bounds__(kThreads) void spec_slice_stats_kernel(StochArgs a) {
  __shared__ float2 red2[kWaves];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int V = a.V;
  const float* p = a.target_logits + (size_t)b * V;
  const float* q = b < a.k ? a.draft_logits + (size_t)b * V : nullptr;
  const int lo = s * a.L, hi = min(V, lo + a.L);
  float mp = -INFINITY, sp = 0.f, mq = -INFINITY, sq = 0.f;
  for (int i0 = lo + tid; i0 < hi; i0 += kThreads * kUnroll) {
    float xp[kUnroll], xq[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int i = i0 + u * kThreads;
      xp[u] = i < hi ? p[i] : -INFINITY;
      xq[u] = (q && i < hi) ? q[i] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      ms_add(mp, sp, xp[u] * a.inv_tt);
      if (q) ms_add(mq, sq, xq[u] * a.inv_td);
    }
  }
  block_ms(mp, sp, red2);
  if (q) block_ms(mq, sq, red2);
  if (tid == 0) {
    const Scratch sc{a.scratch, a.k + 1, a.S};
    float* st = sc.stats(b, s);
    st[0] = mp;
    st[1] = sp;
    st[2] = mq;
    st[3] = sq;
  }
}

// Kernel 2 (after kernel 1 on the stream): row statistics from the slices
// (merged in slice order), the accept gate (slice 0), this slice's weight
// totals; the last slice of a row to arrive finds the crossing slice and
// token; the last row to arrive decides and rewinds.
__global__ __launch_bounds__(kThreads) void spec_slice_sample_kernel(StochArgs a) {
  __shared__ float red[kWaves];
  __shared__ float2 red2[kWaves];
  __shared__ int s_pick, s_last_pos, s_token, s_last_slice;
  __shared__ float s_before;
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int V = a.V;
  const Scratch sc{a.scratch, a.k + 1, a.S};
  const uint64_t offset = *a.offset;  // read before any workgroup can arrive last
  float u_accept, u_sample;
  spec_draws(a.seed, offset, b, u_accept, u_sample);
  const float* p = a.target_logits + (size_t)b * V;
  const float* q = b < a.k ? a.draft_logits + (size_t)b * V : nullptr;

  // Row statistics: lane i of each wave loads slice i's (one round trip)
  // and a fixed xor butterfly merges them (S <= 64).
  float mp = -INFINITY, sp = 0.f, mq = -INFINITY, sq = 0.f;
  {
    const int lane = tid & 63;
    if (lane < a.S) {
      const float4 st = *reinterpret_cast<const float4*>(sc.stats(b, lane));
      mp = st.x;
      sp = st.y;
      mq = st.z;
      sq = st.w;
    }
    for (int off = 32; off > 0; off >>= 1) {
      ms_merge(mp, sp, __shfl_xor(mp, off), __shfl_xor(sp, off));
      ms_merge(mq, sq, __shfl_xor(mq, off), __shfl_xor(sq, off));
    }
  }

  if (s == 0 && tid == 0) {  // accept test of draft token b (batch_stochastic_accept_kernel)
    int flag = 1;
    if (q) {
      const int d = a.draft_tokens[b];
      if (d < 0 || d >= V) {
        flag = 0;
      } else {
        const float pd = __expf(p[d] * a.inv_tt - mp) / sp;
        const float qd = __expf(q[d] * a.inv_td - mq) / sq;
        flag = u_accept < fminf(1.f, pd / fmaxf(qd, 1e-36f)) ? 1 : 0;
      }
    }
    __hip_atomic_store(sc.row_out(b), (uint32_t)flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // This slice's totals of the residual max(0, p - q) and of p.
  const int lo = s * a.L, hi = min(V, lo + a.L);
  RowWeights w{p, q, mp, 1.f / sp, mq, q ? 1.f / sq : 0.f, a.inv_tt, a.inv_td};
  float tr, tp;
  if (q) {
    const float2 ts = w.thread_sums(tid, lo, hi);
    const float2 t = block_sum2(ts.x, ts.y, red2);
    tr = t.x;
    tp = t.y;
  } else {
    tr = tp = block_sum(w.thread_sum(tid, lo, hi), red);
  }
  if (tid == 0) {
    st_dev(sc.totals(b, s), tr);
    st_dev(sc.totals(b, s) + 1, tp);
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev = __hip_atomic_fetch_add(sc.slices_arrived(b), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)(a.S - 1);
    if (last)
      __hip_atomic_store(sc.slices_arrived(b), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last_slice = last;
  }
  __syncthreads();
  if (!s_last_slice) return;

  // ---- the row's sample: the first token, in slice-major order, whose
  // cumulative weight reaches u * total (kernels.cu:361-380) ---------------
  // Lane i of each wave holds slice i's totals (one round trip); wave
  // prefix sums in slice order give the totals and the crossing slice.
  const int lane = tid & 63;
  float t_r = 0.f, t_p = 0.f;
  if (lane < a.S) {
    t_r = ld_dev(sc.totals(b, lane));
    t_p = ld_dev(sc.totals(b, lane) + 1);
  }
  float c_r = t_r, c_p = t_p;
  for (int off = 1; off < 64; off <<= 1) {
    const float yr = __shfl_up(c_r, off), yp = __shfl_up(c_p, off);
    if (lane >= off) {
      c_r += yr;
      c_p += yp;
    }
  }
  const float R = __shfl(c_r, 63);
  const bool use_p = !q || R <= 1e-20f;  // empty residual: sample from p
  if (use_p) w.q = nullptr;
  const float total = use_p ? __shfl(c_p, 63) : R;
  const float goal = u_sample * total;
  const float t_s = use_p ? t_p : t_r;
  const float c_s = use_p ? c_p : c_r;
  const uint64_t cross = __ballot(t_s > 0.f && c_s >= goal);
  const uint64_t positive = __ballot(t_s > 0.f);
  const bool slice_crossing = cross != 0;
  int ss = slice_crossing ? (int)__builtin_ctzll(cross)
                          : (positive ? 63 - (int)__builtin_clzll(positive) : -1);
  const float before_slice = slice_crossing ? __shfl(c_s - t_s, ss) : 0.f;
  if (tid == 0) {
    s_pick = INT_MAX;
    s_last_pos = -1;
    s_token = V - 1;  // non-finite weights: the reference's fallback (kernels.cu:312-315)
  }
  __syncthreads();
  if (ss >= 0) {
    const int slo = ss * a.L, shi = min(V, slo + a.L);
    const float cs = w.thread_sum(tid, slo, shi);
    const float before = before_slice + block_exclusive_scan(cs, red);
    if (cs > 0.f && slice_crossing && before + cs >= goal) atomicMin(&s_pick, tid);
    if (cs > 0.f) atomicMax(&s_last_pos, tid);
    __syncthreads();
    // The chunk holding the crossing (else the last chunk with a positive
    // weight); wave 0 scans it in rounds of 64 with a wave prefix sum.
    const bool crossing = s_pick != INT_MAX;
    const int owner = crossing ? s_pick : s_last_pos;
    if (tid == owner) s_before = before;
    __syncthreads();
    if (owner >= 0 && tid < 64) {
      const int lane = tid;
      const float base = s_before;
      float run = 0.f;
      int tok = -1, last_pos = -1;
      for (int r = 0; slo + owner + r * 64 * kThreads < shi && tok < 0; r++) {
        const int i = slo + owner + (r * 64 + lane) * kThreads;
        const float wi = i < shi ? w(i) : 0.f;
        float incl = wi;
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(incl, off);
          if (lane >= off) incl += y;
        }
        const uint64_t hits = __ballot(crossing && wi > 0.f && base + run + incl >= goal);
        if (hits) tok = slo + owner + (r * 64 + (int)__builtin_ctzll(hits)) * kThreads;
        const uint64_t pos = __ballot(wi > 0.f);
        if (pos) last_pos = slo + owner + (r * 64 + 63 - (int)__builtin_clzll(pos)) * kThreads;
        run += __shfl(incl, 63);
      }
      if (lane == 0) s_token = tok >= 0 ? tok : last_pos;
    }
  }
  __syncthreads();

  // ---- publish the row; the last row decides and rewinds -----------------
  if (tid == 0) {
    __hip_atomic_store(sc.row_out(b) + 1, (uint32_t)s_token, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev = __hip_atomic_fetch_add(sc.rows_arrived(), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)a.k) {  // k+1 rows arrived
      __hip_atomic_store(sc.rows_arrived(), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int n = 0;
      while (n < a.k &&
             __hip_atomic_load(sc.row_out(n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
        n++;
      const int tok = (int)__hip_atomic_load(sc.row_out(n) + 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      for (int i = 0; i < n; i++) a.result[4 + i] = a.draft_tokens[i];
      a.result[4 + n] = tok;
      const int t_seq = a.target_save + n + 1;
      const int d_seq = a.has_draft ? a.draft_save + n : t_seq;
      a.result[0] = n;
      a.result[1] = tok;
      a.result[2] = t_seq;
      a.result[3] = d_seq;
      *a.target.seq_len = t_seq;
      if (a.has_draft) *a.draft.seq_len = d_seq;
      *a.offset = offset + 1;
    }
  }
}

}  // namespace spec
}  // namespace sde

extern "C" int sde_spec_accept_stochastic(sde_kv_cache* target, sde_kv_cache* draft,
                                          const float* d_target_logits,
                                          const float* d_draft_logits,
                                          const int32_t* d_draft_tokens, int k, int vocab,
                                          float temp_target, float temp_draft, uint64_t seed,
                                          uint64_t* d_rng_offset, int target_save,
                                          int draft_save, int32_t* d_result,
                                          sde_stream_t stream) {
  using namespace sde::spec;
  if (!target || !d_target_logits || !d_result || !d_rng_offset ||
      (k > 0 && (!d_draft_logits || !d_draft_tokens)))
    return SDE_ERR_INVALID_ARGUMENT;
  if (vocab < 1 || !std::isfinite(temp_target) || !std::isfinite(temp_draft))
    return SDE_ERR_INVALID_ARGUMENT;
  if (k < 0 || k > sde::kSpecMaxK || target_save < 0 || draft_save < 0) return SDE_ERR_RANGE;
  const bool has_draft = draft != nullptr && draft != target;
  const int64_t t_cap = (int64_t)target->cfg.max_blocks_per_layer * target->cfg.block_size;
  if ((int64_t)target_save + k + 1 > t_cap) return SDE_ERR_RANGE;
  if (has_draft) {
    if (draft->device != target->device) return SDE_ERR_INVALID_ARGUMENT;
    const int64_t d_cap = (int64_t)draft->cfg.max_blocks_per_layer * draft->cfg.block_size;
    if ((int64_t)draft_save + k > d_cap) return SDE_ERR_RANGE;
  }
  if ((((uintptr_t)d_rng_offset) & 7u) != 0) return SDE_ERR_INVALID_ARGUMENT;
  sde::DeviceGuard g(target->device);
  if (!g.ok()) return SDE_ERR_HIP;
  StochArgs a;
  a.target_logits = d_target_logits;
  a.draft_logits = d_draft_logits;
  a.draft_tokens = d_draft_tokens;
  a.k = k;
  a.V = vocab;
  // the reference clamps temperatures at 1e-6 (kernels.cu:58-59, 298)
  a.inv_tt = 1.f / fmaxf(temp_target, 1e-6f);
  a.inv_td = 1.f / fmaxf(temp_draft, 1e-6f);
  a.seed = seed;
  a.offset = d_rng_offset;
  a.target_save = target_save;
  a.draft_save = draft_save;
  int st = sde_kv_get_view(target, &a.target);
  a.draft = sde_kv_view{};
  if (st == SDE_OK && has_draft) st = sde_kv_get_view(draft, &a.draft);
  if (st != SDE_OK) return st;
  a.has_draft = has_draft ? 1 : 0;
  a.result = d_result;
  a.scratch = target->d_counters + sde::kMaxAttnCounters;
  // about 4096 tokens per slice workgroup, at most kSpecMaxSlices slices
  a.S = (vocab + 4095) / 4096;
  if (a.S > sde::kSpecMaxSlices) a.S = sde::kSpecMaxSlices;
  a.L = (vocab + a.S - 1) / a.S;
  const dim3 grid(a.S, k + 1);
  hipLaunchKernelGGL(spec_slice_stats_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  st = sde::launch_status();
  if (st != SDE_OK) return st;
  hipLaunchKernelGGL(spec_slice_sample_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  st = sde::launch_status();
  if (st == SDE_OK) {
    target->seq_len_on_device = true;
    if (has_draft) draft->seq_len_on_device = true;
  }
  return st;
}
