/*
 * sde/spec_device.hpp — on-device acceptance and O(1) cache rewind of
 * speculative decoding, for persistent (megakernel) loops and for
 * sde_spec_accept_greedy / sde_spec_accept_stochastic.
 *
 * Reference (arkhamHack/speculative_decode_engine):
 *   cuda/src/kernels.cu:2428-2466   host loop: greedy match, emit accepted
 *                                   drafts + bonus, rewind target / draft
 *   cuda/src/kernels.cu:3050-3072   the same inside the megakernel
 *                                   (thread 0 of block 0)
 *   cuda/src/kernels.cu:285-291,    speculative sampling: accept test,
 *     319-380, 550-572              correction sample, bonus sample
 */
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>

#include "sde_paged_kv.h"

namespace sde {

struct SpecAccept {
  int n_accepted;  // leading drafts equal to the target's tokens
  int bonus;       // the target's token after them
  int target_seq;  // target seq_len after the rewind
  int draft_seq;   // draft seq_len after the rewind
};

// One thread's work (the reference runs it on thread 0 of block 0):
// draft_tokens[0..k) against target_tokens[0..k] (the verify window's
// argmaxes), emitted[0..n_accepted] = accepted drafts then the bonus, and
// the rewinds: target seq_len <- target_save + n_accepted + 1, draft
// seq_len <- draft_save + n_accepted (the reference's rule; the draft
// re-appends from there), or the target's value when `draft` is null or
// shares the target's seq_len word (self-speculation over one cache).
__device__ inline SpecAccept spec_accept_greedy(const int32_t* draft_tokens,
                                                const int32_t* target_tokens, int k,
                                                int target_save, int draft_save,
                                                const sde_kv_view& target,
                                                const sde_kv_view* draft, int32_t* emitted) {
  int n = 0;
  while (n < k && draft_tokens[n] == target_tokens[n]) n++;
  SpecAccept r;
  r.n_accepted = n;
  r.bonus = target_tokens[n];
  r.target_seq = target_save + n + 1;
  const bool shared = draft == nullptr || draft->seq_len == target.seq_len;
  r.draft_seq = shared ? r.target_seq : draft_save + n;
  for (int i = 0; i < n; i++) emitted[i] = draft_tokens[i];
  emitted[n] = r.bonus;
  *target.seq_len = r.target_seq;
  if (!shared) *draft->seq_len = r.draft_seq;
  return r;
}


// ---- stochastic acceptance (kernels.cu:285-291, 319-380, 550-572) ----------

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC'11): a counter-based generator, so any (key,
// counter) pair is a stream position that every thread computes directly.
// The reference draws from a sequential curand state instead; draws are
// therefore not the reference's, only their distribution is.
struct Philox4 {
  uint32_t v[4];
};

__host__ __device__ inline Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2,
                                                 uint32_t c3, uint32_t k0, uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;  // round multipliers
  constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;  // key schedule (Weyl)
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)kM0 * c0;
    const uint64_t p1 = (uint64_t)kM1 * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
    k0 += kW0;
    k1 += kW1;
  }
  return Philox4{{c0, c1, c2, c3}};
}

// Uniform in (0, 1): the top 24 bits, centred in their interval.
__host__ __device__ inline float philox_uniform(uint32_t x) {
  return ((float)(x >> 8) + 0.5f) * (1.0f / 16777216.0f);
}

// The two draws of window row b in one call: [0] the accept test,
// [1] the token sample.  Counter = (b, offset lo, offset hi, 0).
__host__ __device__ inline void spec_draws(uint64_t seed, uint64_t offset, int b, float& u_accept,
                                           float& u_sample) {
  const Philox4 r = philox4x32_10((uint32_t)b, (uint32_t)offset, (uint32_t)(offset >> 32), 0u,
                                  (uint32_t)seed, (uint32_t)(seed >> 32));
  u_accept = philox_uniform(r.v[0]);
  u_sample = philox_uniform(r.v[1]);
}


// ---- speculative sampling over vocabulary slices ---------------------------
//
// Each window row b (k draft rows, then the bonus row k) is cut into S
// vocabulary slices of L tokens (S = min(ceil(V / 4096), 64)).  Pass 1 (one
// item per (row, slice)): the slice's temperature-softmax (max, sum) of the
// target and the draft logits.  Pass 2 (after every pass-1 item): the row's
// statistics from its slices in slice order, the accept gate (slice 0), the
// slice's sampling-weight totals; the last slice of a row to arrive finds the
// slice, then the token, where the cumulative weight crosses u * total; the
// last row to arrive takes the first rejection, writes the result and
// rewinds.  Every sum runs in the order of a 1024-thread workgroup (thread t
// takes the slice's tokens t, t + 1024, ...; per-wave butterflies; the 16
// waves in order): a block of 512 or 256 threads plays 2 or 4 of those
// threads each, so any block size gives the same bits.  The inverse-CDF
// token order is slice-major, then l % 1024, then l / 1024 of the offset l
// in the slice.

constexpr int kSpecMaxK = 64;
constexpr int kSpecMaxSlices = 64;
// Scratch words, at offsets that do not depend on the call's k (calls with
// different k share one scratch, and its counters must stay zero at rest):
// [0] row arrivals; [1 + r] slice arrivals of row r (both zero at rest);
// [1 + kMaxRows + 2r] (flag, token) of row r; then, from
// 1 + 3 kMaxRows, per (row, slice) the statistics (mp, sp, mq, sq) and the
// weight totals (residual, p) of the call.
constexpr int kSpecMaxRows = kSpecMaxK + 1;
constexpr int kSpecScratchWords = 1 + 3 * kSpecMaxRows + 6 * kSpecMaxRows * kSpecMaxSlices;

namespace spec {

constexpr int kVThreads = 1024;  // the virtual workgroup that fixes the orders
constexpr int kVWaves = kVThreads / 64;
constexpr int kUnroll = 16;      // loads in flight per (virtual) thread

struct StochArgs {
  const float* target_logits;  // [k+1][V]
  const float* draft_logits;   // [k][V]
  const int32_t* draft_tokens;
  int k;
  int V;
  int S;  // vocabulary slices per row
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
  uint32_t* scratch;  // kSpecScratchWords; counters zero at rest
};

// Slices and tokens per slice of a vocabulary (about 4096 tokens per slice).
__host__ __device__ inline void slice_plan(int vocab, int& S, int& L) {
  S = (vocab + 4095) / 4096;
  if (S > kSpecMaxSlices) S = kSpecMaxSlices;
  L = (vocab + S - 1) / S;
}

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

// The virtual thread real thread t plays in slot j.
template <int VT>
__device__ __forceinline__ int vthread(int j) {
  return (int)threadIdx.x + j * (kVThreads / VT);
}

// Block-wide (max, sum) pairs: xor butterfly in each virtual wave, then the
// virtual waves' pairs in order.  Every thread gets the result.
template <int VT>
__device__ void block_ms(float (&m)[VT], float (&s)[VT], float2* lds) {
  constexpr int NW = kVWaves / VT;  // real waves
#pragma unroll
  for (int j = 0; j < VT; j++)
    for (int off = 32; off > 0; off >>= 1)
      ms_merge(m[j], s[j], __shfl_xor(m[j], off), __shfl_xor(s[j], off));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int j = 0; j < VT; j++) lds[w + j * NW] = make_float2(m[j], s[j]);
  __syncthreads();
  float M = -INFINITY, Sum = 0.f;
  for (int i = 0; i < kVWaves; i++) ms_merge(M, Sum, lds[i].x, lds[i].y);
#pragma unroll
  for (int j = 0; j < VT; j++) {
    m[j] = M;
    s[j] = Sum;
  }
}

template <int VT>
__device__ float block_sum(const float (&x)[VT], float* lds) {
  constexpr int NW = kVWaves / VT;
  float y[VT];
#pragma unroll
  for (int j = 0; j < VT; j++) {
    y[j] = x[j];
    for (int off = 32; off > 0; off >>= 1) y[j] += __shfl_xor(y[j], off);
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int j = 0; j < VT; j++) lds[(threadIdx.x >> 6) + j * NW] = y[j];
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kVWaves; i++) t += lds[i];
  return t;
}

// Two block sums at once, each in block_sum's order (the same bits).
template <int VT>
__device__ float2 block_sum2(const float (&x)[VT], const float (&y)[VT], float2* lds) {
  constexpr int NW = kVWaves / VT;
  float a[VT], b[VT];
#pragma unroll
  for (int j = 0; j < VT; j++) {
    a[j] = x[j];
    b[j] = y[j];
    for (int off = 32; off > 0; off >>= 1) {
      a[j] += __shfl_xor(a[j], off);
      b[j] += __shfl_xor(b[j], off);
    }
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int j = 0; j < VT; j++) lds[(threadIdx.x >> 6) + j * NW] = make_float2(a[j], b[j]);
  __syncthreads();
  float2 t = make_float2(0.f, 0.f);
  for (int i = 0; i < kVWaves; i++) {
    t.x += lds[i].x;
    t.y += lds[i].y;
  }
  return t;
}

// Exclusive prefix of x over the virtual threads in order.
template <int VT>
__device__ void block_exclusive_scan(const float (&x)[VT], float (&out)[VT], float* lds) {
  constexpr int NW = kVWaves / VT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float incl[VT];
#pragma unroll
  for (int j = 0; j < VT; j++) {
    incl[j] = x[j];
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(incl[j], off);
      if (lane >= off) incl[j] += y;
    }
  }
  __syncthreads();
  if (lane == 63)
#pragma unroll
    for (int j = 0; j < VT; j++) lds[w + j * NW] = incl[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < VT; j++) {
    float before = 0.f;
    for (int i = 0; i < w + j * NW; i++) before += lds[i];
    out[j] = before + incl[j] - x[j];
  }
}

// Sampling weight of token i of a row: the residual max(0, p - q) for a
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
  // A virtual thread's batch of kUnroll tokens i0, i0 + 1024, ...: the
  // logits, -inf / 0 past hi.
  struct Batch {
    float p[kUnroll], q[kUnroll];
  };
  __device__ __forceinline__ void load(int i0, int hi, Batch& x) const {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int i = i0 + u * kVThreads;
      x.p[u] = i < hi ? p[i] : -INFINITY;
      x.q[u] = (q && i < hi) ? q[i] : 0.f;
    }
  }
  // Virtual thread vt's sums of the residual max(0, p - q) and of p over
  // tokens lo + vt, lo + vt + 1024, ... below hi (q non-null); each sum in
  // thread_sum's order.  With PRE the first batch is `first`, loaded
  // earlier (load(lo + vt, hi, first)).
  template <bool PRE = false>
  __device__ __forceinline__ float2 thread_sums(int vt, int lo, int hi,
                                                const Batch* first = nullptr) const {
    float cr = 0.f, cp = 0.f;
    for (int i0 = lo + vt; i0 < hi; i0 += kVThreads * kUnroll) {
      Batch x;
      if (PRE && i0 == lo + vt)
        x = *first;
      else
        load(i0, hi, x);
#pragma unroll
      for (int u = 0; u < kUnroll; u++)
        if (i0 + u * kVThreads < hi) {
          const float pi = __expf(x.p[u] * inv_tt - mp) * inv_sp;
          const float qi = __expf(x.q[u] * inv_td - mq) * inv_sq;
          cr += fmaxf(pi - qi, 0.f);
          cp += pi;
        }
    }
    return make_float2(cr, cp);
  }
  // Sum of virtual thread vt's weights over tokens lo + vt, lo + vt + 1024,
  // ... below hi, loads batched (PRE: as in thread_sums).
  template <bool PRE = false>
  __device__ __forceinline__ float thread_sum(int vt, int lo, int hi,
                                              const Batch* first = nullptr) const {
    float cs = 0.f;
    for (int i0 = lo + vt; i0 < hi; i0 += kVThreads * kUnroll) {
      Batch x;
      if (PRE && i0 == lo + vt)
        x = *first;
      else
        load(i0, hi, x);
#pragma unroll
      for (int u = 0; u < kUnroll; u++)
        if (i0 + u * kVThreads < hi) cs += of(x.p[u], x.q[u]);
    }
    return cs;
  }
};

struct Scratch {
  uint32_t* base;
  int R;  // rows of this call = k + 1
  int S;
  __device__ uint32_t* rows_arrived() const { return base; }
  __device__ uint32_t* slices_arrived(int r) const { return base + 1 + r; }
  __device__ uint32_t* row_out(int r) const { return base + 1 + kSpecMaxRows + 2 * r; }
  __device__ float* stats(int r, int s) const {
    return reinterpret_cast<float*>(base + 1 + 3 * kSpecMaxRows) + 4 * ((size_t)r * S + s);
  }
  __device__ float* totals(int r, int s) const {
    return reinterpret_cast<float*>(base + 1 + 3 * kSpecMaxRows) + 4 * (size_t)R * S +
           2 * ((size_t)r * S + s);
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

// Pass 1 for (slice s, row b) on the calling block: the slice's (max, sum)
// of the temperature-scaled target (and draft) logits, stored device-scope.
template <int VT>
__device__ void slice_stats(const StochArgs& a, int s, int b, float2* red2) {
  const int V = a.V;
  const float* p = a.target_logits + (size_t)b * V;
  const float* q = b < a.k ? a.draft_logits + (size_t)b * V : nullptr;
  const int lo = s * a.L, hi = min(V, lo + a.L);
  float mp[VT], sp[VT], mq[VT], sq[VT];
#pragma unroll
  for (int j = 0; j < VT; j++) {
    mp[j] = -INFINITY;
    sp[j] = 0.f;
    mq[j] = -INFINITY;
    sq[j] = 0.f;
    for (int i0 = lo + vthread<VT>(j); i0 < hi; i0 += kVThreads * kUnroll) {
      float xp[kUnroll], xq[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; u++) {
        const int i = i0 + u * kVThreads;
        xp[u] = i < hi ? p[i] : -INFINITY;
        xq[u] = (q && i < hi) ? q[i] : -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; u++) {
        ms_add(mp[j], sp[j], xp[u] * a.inv_tt);
        if (q) ms_add(mq[j], sq[j], xq[u] * a.inv_td);
      }
    }
  }
  block_ms<VT>(mp, sp, red2);
  if (q) block_ms<VT>(mq, sq, red2);
  if (threadIdx.x == 0) {
    const Scratch sc{a.scratch, a.k + 1, a.S};
    float* st = sc.stats(b, s);
    st_dev(st, mp[0]);
    st_dev(st + 1, sp[0]);
    st_dev(st + 2, mq[0]);
    st_dev(st + 3, sq[0]);
  }
}

// LDS of pass 2 on one block.
struct SampleLds {
  float red[kVWaves];
  float2 red2[kVWaves];
  int pick, last_pos, token, last_slice, last_row;
  float before;
};

// Pass 2 for (slice s, row b), after every pass-1 item of the call: row
// statistics from the slices (merged in slice order), the accept gate
// (slice 0), this slice's weight totals; the last slice of a row to arrive
// finds the crossing slice and token; the last row to arrive decides and
// rewinds.  Every thread of the block calls it.
// (The default of slice_sample's `hook`: nothing.)
struct NoHook {
  __device__ void operator()(int, int, int, int) const {}
};

template <int VT, class Hook = NoHook>
__device__ void slice_sample(const StochArgs& a, int s, int b, SampleLds& sl,
                             const Hook& hook = Hook{}) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const Scratch sc{a.scratch, a.k + 1, a.S};
  const float* p = a.target_logits + (size_t)b * V;
  const float* q = b < a.k ? a.draft_logits + (size_t)b * V : nullptr;
  const int lo = s * a.L, hi = min(V, lo + a.L);
  // The accept test's draft token (slice 0, one thread), the call index,
  // this slice's first batch of logits and the row statistics below are
  // all requested before any of them is used: one round trip for the lot.
  const bool gate = q && s == 0 && tid == 0;
  const int d = gate ? a.draft_tokens[b] : 0;
  // (the call index is read before any block can arrive last: the last
  // row's arrival needs this item's totals, published below)
  const uint64_t offset = *a.offset;
  const RowWeights ahead{p, q, 0.f, 0.f, 0.f, 0.f, a.inv_tt, a.inv_td};
  RowWeights::Batch first;
  ahead.load(lo + vthread<VT>(0), hi, first);

  // Row statistics: lane i of each wave loads slice i's (one round trip)
  // and a fixed xor butterfly merges them (S <= 64).
  float mp = -INFINITY, sp = 0.f, mq = -INFINITY, sq = 0.f;
  {
    const int lane = tid & 63;
    if (lane < a.S) {
      const float* st = sc.stats(b, lane);
      mp = ld_dev(st);
      sp = ld_dev(st + 1);
      mq = ld_dev(st + 2);
      sq = ld_dev(st + 3);
    }
    for (int off = 32; off > 0; off >>= 1) {
      ms_merge(mp, sp, __shfl_xor(mp, off), __shfl_xor(sp, off));
      ms_merge(mq, sq, __shfl_xor(mq, off), __shfl_xor(sq, off));
    }
  }

  float u_accept, u_sample;
  spec_draws(a.seed, offset, b, u_accept, u_sample);

  if (s == 0 && tid == 0) {  // accept test of draft token b (batch_stochastic_accept_kernel)
    int flag = 1;
    if (q) {
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
  RowWeights w{p, q, mp, 1.f / sp, mq, q ? 1.f / sq : 0.f, a.inv_tt, a.inv_td};
  float tr, tp;
  if (q) {
    float xr[VT], xp[VT];
#pragma unroll
    for (int j = 0; j < VT; j++) {
      const float2 ts = j == 0 ? w.thread_sums<true>(vthread<VT>(j), lo, hi, &first)
                               : w.thread_sums(vthread<VT>(j), lo, hi);
      xr[j] = ts.x;
      xp[j] = ts.y;
    }
    const float2 t = block_sum2<VT>(xr, xp, sl.red2);
    tr = t.x;
    tp = t.y;
  } else {
    float x[VT];
#pragma unroll
    for (int j = 0; j < VT; j++)
      x[j] = j == 0 ? w.thread_sum<true>(vthread<VT>(j), lo, hi, &first)
                    : w.thread_sum(vthread<VT>(j), lo, hi);
    tr = tp = block_sum<VT>(x, sl.red);
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
    sl.last_slice = last;
  }
  __syncthreads();
  if (!sl.last_slice) return;

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
  const int ss = slice_crossing ? (int)__builtin_ctzll(cross)
                                : (positive ? 63 - (int)__builtin_clzll(positive) : -1);
  const float before_slice = slice_crossing ? __shfl(c_s - t_s, ss) : 0.f;
  if (tid == 0) {
    sl.pick = INT_MAX;
    sl.last_pos = -1;
    sl.token = V - 1;  // non-finite weights: the reference's fallback (kernels.cu:312-315)
  }
  __syncthreads();
  if (ss >= 0) {
    const int slo = ss * a.L, shi = min(V, slo + a.L);
    float cs[VT], before[VT];
#pragma unroll
    for (int j = 0; j < VT; j++) cs[j] = w.thread_sum(vthread<VT>(j), slo, shi);
    block_exclusive_scan<VT>(cs, before, sl.red);
#pragma unroll
    for (int j = 0; j < VT; j++) {
      before[j] += before_slice;
      if (cs[j] > 0.f && slice_crossing && before[j] + cs[j] >= goal)
        atomicMin(&sl.pick, vthread<VT>(j));
      if (cs[j] > 0.f) atomicMax(&sl.last_pos, vthread<VT>(j));
    }
    __syncthreads();
    // The chunk holding the crossing (else the last chunk with a positive
    // weight); wave 0 scans it in rounds of 64 with a wave prefix sum.
    const bool crossing = sl.pick != INT_MAX;
    const int owner = crossing ? sl.pick : sl.last_pos;
#pragma unroll
    for (int j = 0; j < VT; j++)
      if (vthread<VT>(j) == owner) sl.before = before[j];
    __syncthreads();
    if (owner >= 0 && tid < 64) {
      const float base = sl.before;
      float run = 0.f;
      int tok = -1, last_pos = -1;
      for (int r = 0; slo + owner + r * 64 * kVThreads < shi && tok < 0; r++) {
        const int i = slo + owner + (r * 64 + lane) * kVThreads;
        const float wi = i < shi ? w(i) : 0.f;
        float incl = wi;
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(incl, off);
          if (lane >= off) incl += y;
        }
        const uint64_t hits = __ballot(crossing && wi > 0.f && base + run + incl >= goal);
        if (hits) tok = slo + owner + (r * 64 + (int)__builtin_ctzll(hits)) * kVThreads;
        const uint64_t pos = __ballot(wi > 0.f);
        if (pos) last_pos = slo + owner + (r * 64 + 63 - (int)__builtin_clzll(pos)) * kVThreads;
        run += __shfl(incl, 63);
      }
      if (lane == 0) sl.token = tok >= 0 ? tok : last_pos;
    }
  }
  __syncthreads();

  // ---- publish the row; the last row decides and rewinds -----------------
  if (tid == 0) {
    __hip_atomic_store(sc.row_out(b) + 1, (uint32_t)sl.token, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev = __hip_atomic_fetch_add(sc.rows_arrived(), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)a.k;  // k+1 rows arrived
    if (last) __hip_atomic_store(sc.rows_arrived(), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sl.last_row = last;
  }
  __syncthreads();
  if (!sl.last_row || tid >= 64) return;
  // Wave 0 of the last row: lane i loads draft row i's accept flag, row i's
  // token and draft token i together (one round trip); the first rejected
  // row n (k when every draft is accepted) gives the corrected token, or
  // the bonus row's token.
  const bool draft_lane = lane < a.k;
  const uint32_t flag = draft_lane ? __hip_atomic_load(sc.row_out(lane), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 1u;
  const int row_tok = lane <= a.k ? (int)__hip_atomic_load(sc.row_out(lane) + 1,
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                  : 0;
  const int drafted = draft_lane ? a.draft_tokens[lane] : 0;
  const uint64_t rejected = __ballot(draft_lane && flag == 0u);
  const int n = rejected ? (int)__builtin_ctzll(rejected) : a.k;
  int tok = __shfl(row_tok, n & 63);
  if (n >= 64)  // k = 64 and every draft accepted: the bonus row is past the lanes
    tok = (int)__hip_atomic_load(sc.row_out(n) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane < n) a.result[4 + lane] = drafted;
  if (lane == 0) {
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
    hook(n, tok, t_seq, d_seq);
  }
}

template <int VT, class Sync, class Hook = NoHook>
__device__ void stochastic_grid(const StochArgs& a, Sync& sync, const Hook& hook = Hook{}) {
  __shared__ float2 red2[kVWaves];
  __shared__ SampleLds sl;
  const int items = a.S * (a.k + 1);
  const int blk = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int nblk = gridDim.x * gridDim.y * gridDim.z;
  for (int it = blk; it < items; it += nblk) {
    slice_stats<VT>(a, it % a.S, it / a.S, red2);
    __syncthreads();  // red2 reused by the block's next item
  }
  sync();
  for (int it = blk; it < items; it += nblk) {
    slice_sample<VT>(a, it % a.S, it / a.S, sl, hook);
    __syncthreads();  // sl reused by the block's next item
  }
}

}  // namespace spec

// Bytes of device_spec_accept_stochastic_grid's workspace (its counters must
// be zero before the first call; every call leaves them zero).
__host__ __device__ inline size_t spec_stochastic_workspace_size() {
  return (size_t)kSpecScratchWords * sizeof(uint32_t);
}

// Grid-cooperative form of sde_spec_accept_stochastic (speculative sampling
// and the rewinds, kernels.cu:285-291, 319-380, 550-572, 2428-2466) for
// persistent kernels: every block of the caller's grid calls it with the
// same arguments (blockDim.x 256, 512 or 1024; any grid size: blocks take
// the (row, slice) items in turn), and `sync()` must be a grid-wide barrier
// that orders memory device-wide (e.g. a cooperative_groups grid sync); it
// is called once, between the two passes.  The result (d_result of
// sde_spec_accept_stochastic: n_accepted, token, target seq_len, draft
// seq_len, emitted tokens), the caches' seq_len words and *offset are
// written by the block that finishes last, complete once the grid has
// synchronized after the call.  `draft` null, or sharing the target's
// seq_len word, is self-speculation over one cache.  The same inputs, seed
// and offset give the same bits as sde_spec_accept_stochastic, whatever the
// grid and block sizes.  Returns the same status in every thread, before any
// work: SDE_ERR_UNSUPPORTED (block size), SDE_ERR_RANGE (k outside [0, 64]),
// SDE_ERR_INVALID_ARGUMENT, SDE_ERR_WORKSPACE.  `hook(n_accepted, token,
// target_seq, draft_seq)`, when given, runs once per call on the one thread
// that decides, right after it has written the result, the seq_len words and
// *offset (a persistent loop's follow-up without a grid barrier of its own;
// its stores are visible to the grid after the caller's next grid barrier).
template <class Sync, class Hook = spec::NoHook>
__device__ int device_spec_accept_stochastic_grid(
    const float* target_logits, const float* draft_logits, const int32_t* draft_tokens, int k,
    int vocab, float temp_target, float temp_draft, uint64_t seed, uint64_t* offset,
    int target_save, int draft_save, const sde_kv_view& target, const sde_kv_view* draft,
    int32_t* result, void* workspace, size_t workspace_bytes, Sync sync, Hook hook = Hook{}) {
  using namespace spec;
  if (blockDim.x != 256 && blockDim.x != 512 && blockDim.x != 1024) return SDE_ERR_UNSUPPORTED;
  if (k < 0 || k > kSpecMaxK) return SDE_ERR_RANGE;
  if (!target_logits || (k > 0 && (!draft_logits || !draft_tokens)) || !offset || !result ||
      !workspace || vocab < 1 || !target.seq_len)
    return SDE_ERR_INVALID_ARGUMENT;
  if (workspace_bytes < spec_stochastic_workspace_size()) return SDE_ERR_WORKSPACE;
  StochArgs a;
  a.target_logits = target_logits;
  a.draft_logits = draft_logits;
  a.draft_tokens = draft_tokens;
  a.k = k;
  a.V = vocab;
  slice_plan(vocab, a.S, a.L);
  // the reference clamps temperatures at 1e-6 (kernels.cu:58-59, 298)
  a.inv_tt = 1.f / fmaxf(temp_target, 1e-6f);
  a.inv_td = 1.f / fmaxf(temp_draft, 1e-6f);
  a.seed = seed;
  a.offset = offset;
  a.target_save = target_save;
  a.draft_save = draft_save;
  a.target = target;
  a.has_draft = draft != nullptr && draft->seq_len != target.seq_len ? 1 : 0;
  a.draft = a.has_draft ? *draft : sde_kv_view{};
  a.result = result;
  a.scratch = static_cast<uint32_t*>(workspace);
  if (blockDim.x == 1024)
    stochastic_grid<1>(a, sync, hook);
  else if (blockDim.x == 512)
    stochastic_grid<2>(a, sync, hook);
  else
    stochastic_grid<4>(a, sync, hook);
  return SDE_OK;
}

}  // namespace sde

