// Stochastic acceptance of speculative decoding on the device, for gfx950.
//
// Computes what the reference's stochastic round computes after a verify
// pass -- batch_stochastic_accept_kernel (kernels.cu:550-572), the
// correction sample on the first rejection (device_corrected_adjusted_sample,
// kernels.cu:319-380) and the bonus sample when every draft is accepted
// (softmax_sample_temperature_kernel) -- followed by the greedy-style rewind
// of both caches (kernels.cu:2428-2466).  The reference runs these on
// thread 0 of one block, serially over the vocabulary; here one 1024-thread
// workgroup per window row does its row's temperature softmax with block
// reductions, the accept test, and a speculative sample (the correction
// token for a draft row, the bonus token for row k), and the last workgroup
// to arrive picks the first rejection and writes the results.  Every
// reduction and the CDF search run in a fixed order, so a call is a pure
// function of its inputs, the seed and the call index.
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
  uint32_t* scratch;  // [0] arrival counter, then (flag, token) per row
};

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
  __device__ __forceinline__ float operator()(int i) const {
    const float pi = __expf(p[i] * inv_tt - mp) * inv_sp;
    if (!q) return pi;
    const float qi = __expf(q[i] * inv_td - mq) * inv_sq;
    return fmaxf(pi - qi, 0.f);
  }
};

__global__ __launch_bounds__(kThreads) void spec_stochastic_kernel(StochArgs a) {
  __shared__ float2 red2[kWaves];
  __shared__ float red[kWaves];
  __shared__ int s_pick;
  __shared__ int s_last_pos;
  __shared__ int s_token;
  const int b = blockIdx.x;  // window row: b < k draft rows, b == k the bonus row
  const int tid = threadIdx.x;
  const int V = a.V;
  const uint64_t offset = *a.offset;  // read before any workgroup can arrive last
  float u_accept, u_sample;
  spec_draws(a.seed, offset, b, u_accept, u_sample);

  const float* p = a.target_logits + (size_t)b * V;
  const float* q = b < a.k ? a.draft_logits + (size_t)b * V : nullptr;
  const int per = (V + kThreads - 1) / kThreads;
  const int lo = min(V, tid * per);
  const int hi = min(V, lo + per);

  // ---- temperature softmax statistics of p (and q) ------------------------
  float mp = -INFINITY, sp = 0.f, mq = -INFINITY, sq = 0.f;
  for (int i = lo; i < hi; i++) {
    const float x = p[i] * a.inv_tt;
    if (x > mp) {
      sp = (mp == -INFINITY ? 0.f : sp * __expf(mp - x)) + 1.f;
      mp = x;
    } else {
      sp += __expf(x - mp);
    }
    if (q) {
      const float y = q[i] * a.inv_td;
      if (y > mq) {
        sq = (mq == -INFINITY ? 0.f : sq * __expf(mq - y)) + 1.f;
        mq = y;
      } else {
        sq += __expf(y - mq);
      }
    }
  }
  block_ms(mp, sp, red2);
  if (q) block_ms(mq, sq, red2);

  // ---- accept test of draft token b (batch_stochastic_accept_kernel) -------
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

  // ---- speculative sample: smallest i with cumulative weight >= u * total --
  RowWeights w{p, q, mp, 1.f / sp, mq, q ? 1.f / sq : 0.f, a.inv_tt, a.inv_td};
  float cs = 0.f;
  for (int i = lo; i < hi; i++) cs += w(i);
  float total = block_sum(cs, red);
  if (q && total <= 1e-20f) {  // empty residual: sample from p (kernels.cu:361-369)
    w.q = nullptr;
    cs = 0.f;
    for (int i = lo; i < hi; i++) cs += w(i);
    total = block_sum(cs, red);
  }
  const float goal = u_sample * total;
  const float before = block_exclusive_scan(cs, red);
  if (tid == 0) {
    s_pick = INT_MAX;
    s_last_pos = -1;
    s_token = V - 1;  // non-finite weights: the reference's fallback (kernels.cu:312-315)
  }
  __syncthreads();
  if (cs > 0.f && before + cs >= goal) atomicMin(&s_pick, tid);
  if (cs > 0.f) atomicMax(&s_last_pos, tid);
  __syncthreads();
  // The chunk holding the crossing; if rounding left the goal above every
  // prefix, the last chunk with a positive weight.
  const bool crossing = s_pick != INT_MAX;
  if (tid == (crossing ? s_pick : s_last_pos)) {
    int tok = -1;
    if (crossing) {
      float c = before;
      for (int i = lo; i < hi; i++) {
        const float wi = w(i);
        c += wi;
        if (wi > 0.f && c >= goal) {
          tok = i;
          break;
        }
      }
    }
    for (int i = hi - 1; tok < 0 && i >= lo; i--)
      if (w(i) > 0.f) tok = i;
    s_token = tok;
  }
  __syncthreads();
  const int token = s_token;

  // ---- publish this row; the last workgroup decides and rewinds ----------
  if (tid == 0) {
    __hip_atomic_store(a.scratch + 1 + 2 * b, (uint32_t)flag, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.scratch + 2 + 2 * b, (uint32_t)token, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t prev =
        __hip_atomic_fetch_add(a.scratch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)a.k) {  // k+1 rows arrived
      __hip_atomic_store(a.scratch, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int n = 0;
      while (n < a.k && __hip_atomic_load(a.scratch + 1 + 2 * n, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) != 0u)
        n++;
      const int tok = (int)__hip_atomic_load(a.scratch + 2 + 2 * n, __ATOMIC_RELAXED,
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
  hipLaunchKernelGGL(spec_stochastic_kernel, dim3(k + 1), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  st = sde::launch_status();
  if (st == SDE_OK) {
    target->seq_len_on_device = true;
    if (has_draft) draft->seq_len_on_device = true;
  }
  return st;
}
