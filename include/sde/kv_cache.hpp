/*
 * sde/kv_cache.hpp — the reference's host-side C++ names over the C-ABI of
 * sde_paged_kv.h, for in-tree C++ callers that used
 *   cuda/include/kv_cache.h:38-63   KVCache, kv_cache_alloc/free/reset
 *   cuda/src/kernels.cu:546-548     set_seq_len_kernel
 *   cuda/src/kernels.cu:826-844     cublas_kv_append_kernel
 *   cuda/src/kernels.cu:904-940     cublas_attention_kernel
 * The three kernels become host functions with the reference's argument
 * lists plus a trailing stream, so `name<<<grid, block>>>(args)` becomes
 * `name(args)`.  Errors print the status and exit, as the reference's
 * CUDA_CHECK does (utils.h:387-395); use the C-ABI directly to handle them.
 * Device code takes `KVCache::view` (sde_kv_view) by value, like the
 * reference's POD KVCache, and calls sde/attention_device.hpp.
 */
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "sde_paged_kv.h"

namespace sde {

struct KVCache {
  sde_kv_cache* handle = nullptr;  // owns pool, tables, seq_len, workspace
  sde_kv_view view{};              // device pointers + sizes (reference layout)
};

inline void check_status(int status, const char* what) {
  if (status != SDE_OK) {
    std::fprintf(stderr, "sde: %s failed: %s\n", what, sde_status_string(status));
    std::exit(EXIT_FAILURE);
  }
}

// kv_cache.h:56-57 / kv_cache.cu:8-42.  `d_head` is the reference's name for
// kv_dim = n_kv_heads * head_dim.  With pool_blocks 0 the pool holds
// n_layers * max_blocks_per_layer blocks assigned statically (layer l gets
// blocks l*max .. l*max+max-1, kv_cache.cu:32-37); a larger pool takes its
// tables from kv_cache_set_block_table.
inline void kv_cache_alloc(KVCache& kv, int n_layers, int d_head, int max_blocks_per_layer,
                           int block_size = 16, int pool_blocks = 0) {
  const sde_kv_config cfg{n_layers, d_head, max_blocks_per_layer, block_size, pool_blocks};
  check_status(sde_kv_cache_create(&cfg, &kv.handle), "kv_cache_alloc");
  check_status(sde_kv_get_view(kv.handle, &kv.view), "kv_cache_alloc");
}

// kv_cache.h:59 / kv_cache.cu:44-48.
inline void kv_cache_free(KVCache& kv) {
  check_status(sde_kv_cache_destroy(kv.handle), "kv_cache_free");
  kv.handle = nullptr;
  kv.view = sde_kv_view{};
}

// kv_cache.h:61 / kv_cache.cu:50-52: seq_len <- 0, tables and pool kept.
inline void kv_cache_reset(KVCache& kv, hipStream_t stream = nullptr) {
  check_status(sde_kv_reset(kv.handle, stream), "kv_cache_reset");
}

// Installs a layer's block table (the reference assigns blocks statically
// only); `n` entries, each a block of the pool.
inline void kv_cache_set_block_table(KVCache& kv, int layer, const int32_t* table, int n) {
  check_status(sde_kv_set_block_table(kv.handle, layer, table, n), "kv_cache_set_block_table");
}

// kernels.cu:546-548: stream-ordered device seq_len write (and the host
// mirror used for validation).
inline void set_seq_len_kernel(KVCache& kv, int len, hipStream_t stream = nullptr) {
  check_status(sde_kv_set_seq_len(kv.handle, len, stream), "set_seq_len_kernel");
}

// kv_cache.cu:116-120: O(1) rewind to target_len (<= the current length).
inline void kv_cache_rollback(KVCache& kv, int target_len, hipStream_t stream = nullptr) {
  check_status(sde_kv_rollback(kv.handle, target_len, stream), "kv_cache_rollback");
}

// kernels.cu:826-844: rows g_k, g_v fp32 [M][kd] -> fp16 (RNE) at positions
// pos_base .. pos_base+M-1 of `layer`.
inline void cublas_kv_append_kernel(const KVCache& kv, int layer, const float* g_k,
                                    const float* g_v, int kd, int pos_base, int M,
                                    hipStream_t stream = nullptr) {
  if (kd != kv.view.kv_dim) check_status(SDE_ERR_INVALID_ARGUMENT, "cublas_kv_append_kernel");
  check_status(sde_kv_append(kv.handle, layer, g_k, g_v, pos_base, M, stream),
               "cublas_kv_append_kernel");
}

// kernels.cu:904-940: queries g_Q fp32 [M][nh*dph]; query m attends to
// positions [0, pos_base+m] of `layer` (causal verify window), g_out fp32
// [M][nh*dph].  The cache keeps the split-context workspace.
inline void cublas_attention_kernel(const float* g_Q, float* g_out, const KVCache& kv, int layer,
                                    int nh, int nkv, int dph, int kd, int pos_base, int M,
                                    hipStream_t stream = nullptr) {
  if (kd != kv.view.kv_dim || kd != nkv * dph)
    check_status(SDE_ERR_INVALID_ARGUMENT, "cublas_attention_kernel");
  check_status(sde_paged_attention(kv.handle, layer, g_Q, g_out, nh, nkv, dph, pos_base, M,
                                   nullptr, 0, stream),
               "cublas_attention_kernel");
}

}  // namespace sde
