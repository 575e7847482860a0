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

}  // namespace sde
