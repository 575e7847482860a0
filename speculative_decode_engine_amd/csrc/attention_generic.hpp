// Attention for the shapes the tile kernels do not cover (head_dim other
// than 64 / 128, block sizes not a multiple of 8): the interface between
// paged_attention.hip's entry points and attention_generic.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "sde/attention_generic_device.hpp"

namespace sde {
namespace gen {

// (kMaxDph, needs_generic and GenRope come from sde/attention_generic_device.hpp.)

struct GenPlan {
  int row_groups;
  int n_parts;
  int part_len;  // tokens per partition (a multiple of 64)
};

// The partition plan of a call: partitions of at least 64 tokens, at most
// as many as parts_bound (the bound the attention workspace is sized for),
// about two workgroups per CU over all (KV head, row group) units, and no
// more partials than SDE_NOALLOC_SCRATCH_BYTES holds.
GenPlan generic_plan(int L_max, int nkv, int R, int dph, int n_cus, int max_parts);

// Bytes of partials the plan needs (0 for one partition).
size_t generic_partial_bytes(const GenPlan& p, int nkv, int R, int dph);

// Launches the generic path on `stream`: (RoPE of k and append of k, v at
// pos_base.. when rope != nullptr), attention with the query rows rotated
// in-kernel when rope != nullptr, and the partition combine when the plan
// has more than one partition.  Returns an sde status.
int generic_attention(uint16_t* pool, const int32_t* table, int kv_dim, int block_size,
                      const float* q, float* out, float* partials, int nh, int nkv, int dph,
                      int pos_base, int n_queries, const GenPlan& plan,
                      const GenRope* rope, hipStream_t stream);

}  // namespace gen
}  // namespace sde
