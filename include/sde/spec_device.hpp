/*
 * sde/spec_device.hpp — on-device greedy acceptance and O(1) cache rewind of
 * speculative decoding, for persistent (megakernel) loops and for
 * sde_spec_accept_greedy.
 *
 * Reference (arkhamHack/speculative_decode_engine):
 *   cuda/src/kernels.cu:2428-2466   host loop: greedy match, emit accepted
 *                                   drafts + bonus, rewind target / draft
 *   cuda/src/kernels.cu:3050-3072   the same inside the megakernel
 *                                   (thread 0 of block 0)
 */
#pragma once

#include <hip/hip_runtime.h>

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

}  // namespace sde
