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

constexpr int kThreads = kVThreads;  // one 1024-thread workgroup per (slice, row)

// Kernel 1: (max, sum) of the temperature-scaled target (and draft) logits
// of one vocabulary slice per workgroup.
__global__ __launch_bounds__(kThreads) void spec_slice_stats_kernel(StochArgs a) {
  __shared__ float2 red2[kVWaves];
  slice_stats<1>(a, blockIdx.x, blockIdx.y, red2);
}

// Kernel 2 (after kernel 1 on the stream): the rest of the call.
__global__ __launch_bounds__(kThreads) void spec_slice_sample_kernel(StochArgs a) {
  __shared__ SampleLds sl;
  slice_sample<1>(a, blockIdx.x, blockIdx.y, sl);
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
  slice_plan(vocab, a.S, a.L);  // about 4096 tokens per slice, at most 64 slices
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
