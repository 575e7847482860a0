/*
 * sde_paged_kv.h — C-ABI of the MI355X (gfx950) paged KV cache and paged
 * GQA decode/verify attention.
 *
 * Every entry point is plain C: opaque handles, raw device pointers, sizes,
 * and a hipStream_t passed as `void*` (NULL = the default stream).  No entry
 * point ever exits the process; each returns an `sde_status` code and does
 * no device work when it rejects its arguments.
 *
 * Reference interface replaced (arkhamHack/speculative_decode_engine):
 *   cuda/include/kv_cache.h:5-79       cache layout, host + device API
 *   cuda/src/kv_cache.cu:8-120         alloc/free/reset/append/read/rollback
 *   cuda/include/attention.h:21-164    device_flash_attention_gqa / dispatch
 *   cuda/src/kernels.cu:546-548        set_seq_len_kernel
 *   cuda/src/kernels.cu:826-844        cublas_kv_append_kernel
 *   cuda/src/kernels.cu:904-940        cublas_attention_kernel
 *
 * Physical layout (identical to kv_cache.h:5-18 so cache bytes match the
 * reference bit for bit): the pool is `pool_blocks` blocks; block b holds
 *   K: fp16[block_size][kv_dim]   then   V: fp16[block_size][kv_dim]
 * with all KV heads interleaved in each token row (kv_dim = n_kv_heads *
 * head_dim).  Token `pos` of layer `l` lives in physical block
 * table[l][pos / block_size], slot pos % block_size.
 */
#ifndef SDE_PAGED_KV_H
#define SDE_PAGED_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sde_kv_cache sde_kv_cache; /* opaque; owns tables + seq_len */
typedef void* sde_stream_t;               /* hipStream_t, NULL = default   */

typedef enum sde_status {
  SDE_OK = 0,
  SDE_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative count, bad config  */
  SDE_ERR_CAPACITY = 2,         /* position beyond the layer's mapped blocks */
  SDE_ERR_RANGE = 3,            /* table entry outside pool, bad rollback    */
  SDE_ERR_UNSUPPORTED = 4,      /* attention type / head_dim / block_size    */
  SDE_ERR_WORKSPACE = 5,        /* caller workspace smaller than required    */
  SDE_ERR_HIP = 6,              /* a HIP call or a host allocation failed    */
  SDE_ERR_NO_DEVICE = 7,        /* no usable gfx950 device                   */
  SDE_ERR_IO = 8,               /* weight file cannot be opened / short read */
  SDE_ERR_FORMAT = 9            /* weight file header or tensor count bad    */
} sde_status;

/* AttentionType values of cuda/include/config.h:51-56. */
typedef enum sde_attention_type {
  SDE_ATTN_SOFTMAX = 0,
  SDE_ATTN_SLIDING_WINDOW = 1, /* reserved in the reference: unsupported */
  SDE_ATTN_KDA = 2,            /* reserved in the reference: unsupported */
  SDE_ATTN_LINEAR = 3          /* reserved in the reference: unsupported */
} sde_attention_type;

/* Runtime form of the reference's compile-time bounds (config.h:8-12) and
 * of kv_cache_alloc's arguments (kv_cache.h:56-57).  pool_blocks == 0 means
 * the reference sizing n_layers * max_blocks_per_layer (kv_cache.cu:15). */
typedef struct sde_kv_config {
  int32_t n_layers;
  int32_t kv_dim;               /* reference KVCache::d_head (kv_cache.h:42) */
  int32_t max_blocks_per_layer; /* reference MAX_KV_BLOCKS (config.h:12)     */
  int32_t block_size;           /* reference KV_BLOCK_SIZE (config.h:10)     */
  int32_t pool_blocks;          /* reference KVCache::pool_size              */
} sde_kv_config;

/* Device-side view of a cache, a plain POD like the reference KVCache that
 * loop drivers copy by value into kernels (kernels.cu:3614-3630). */
typedef struct sde_kv_view {
  uint16_t* pool;        /* fp16 bits, pool_blocks * 2*block_size*kv_dim  */
  int32_t* block_tables; /* [n_layers][max_blocks_per_layer]              */
  int32_t* seq_len;      /* one int32 on the device (write-only bookkeeping) */
  int32_t n_layers;
  int32_t kv_dim;
  int32_t block_size;
  int32_t max_blocks_per_layer;
  int32_t pool_blocks;
  int32_t reserved;
} sde_kv_view;

/* Message for a status code; never NULL. */
const char* sde_status_string(int status);

/* Host-only check of a configuration (no device work).  Rules:
 * n_layers, kv_dim, max_blocks_per_layer >= 1; block_size in [1, 1024];
 * pool_blocks >= 0 (0 = reference sizing) and >= max_blocks_per_layer; the
 * resolved pool_blocks and max_blocks_per_layer * block_size fit int32; the
 * pool's byte size (pool_blocks * 2 * block_size * kv_dim * 2) fits
 * ptrdiff_t. */
int sde_kv_config_validate(const sde_kv_config* cfg);

/* Bytes of the pool a configuration needs (0 on an invalid config). */
size_t sde_kv_pool_bytes(const sde_kv_config* cfg);

/* kv_cache_alloc (kv_cache.h:56-57, kv_cache.cu:8-42): allocate and zero
 * the pool, the per-layer tables and seq_len; layer l gets the reference's
 * static assignment table[l][b] = l*max_blocks_per_layer + b when that fits
 * the pool (otherwise tables start as -1 = unmapped).  seq_len = 0. */
int sde_kv_cache_create(const sde_kv_config* cfg, sde_kv_cache** out);

/* As sde_kv_cache_create, but the caller owns the pool memory (a device
 * buffer of at least sde_kv_pool_bytes(cfg) bytes, 16-byte aligned).  The
 * pool is not cleared.  No counterpart in the reference: it lets a host
 * framework (e.g. a caching allocator) own the 8 GiB pools. */
int sde_kv_cache_create_external(const sde_kv_config* cfg, void* d_pool,
                                 size_t pool_bytes, sde_kv_cache** out);

/* kv_cache_free (kv_cache.h:60, kv_cache.cu:44-48).  NULL is accepted. */
int sde_kv_cache_destroy(sde_kv_cache* cache);

/* kv_cache_reset (kv_cache.h:63, kv_cache.cu:50-52): seq_len = 0 on the
 * host mirror and (stream-ordered) on the device.  Tables and pool kept. */
int sde_kv_reset(sde_kv_cache* cache, sde_stream_t stream);

/* Map logical blocks [0, n_blocks) of `layer` to physical blocks (host
 * array).  Replaces the static assignment of kv_cache.cu:29-37; every entry
 * must lie in [0, pool_blocks).  Synchronous. */
int sde_kv_set_block_table(sde_kv_cache* cache, int layer,
                           const int32_t* host_table, int n_blocks);

/* Copy the first n_blocks entries of a layer's table to host memory. */
int sde_kv_get_block_table(const sde_kv_cache* cache, int layer,
                           int32_t* host_table, int n_blocks);

/* Host mirror of KVCache::seq_len. */
int sde_kv_seq_len(const sde_kv_cache* cache, int* out_len);

/* Synchronous read of the device-side seq_len word (what the reference's
 * loop drivers write, kernels.cu:2459, 3068-3069); for checks and tests. */
int sde_kv_device_seq_len(const sde_kv_cache* cache, int* out_len);

/* set_seq_len_kernel (kernels.cu:546-548): seq_len = len, on the host and
 * stream-ordered on the device.  0 <= len <= capacity. */
int sde_kv_set_seq_len(sde_kv_cache* cache, int len, sde_stream_t stream);

/* kv_cache_rollback (kv_cache.h:79, kv_cache.cu:116-120) as used by the
 * loop drivers (kernels.cu:2457-2459, 3068-3069): seq_len = target_len.
 * O(1): moves no pool bytes; stale K/V are overwritten by later appends.
 * Requires 0 <= target_len <= current seq_len. */
int sde_kv_rollback(sde_kv_cache* cache, int target_len, sde_stream_t stream);

/* cublas_kv_append_kernel (kernels.cu:826-844) / kv_cache_append
 * (kv_cache.cu:70-93): write n_tokens fp32 K and V rows ([n_tokens][kv_dim]
 * device arrays) as fp16 (round-to-nearest-even) at positions
 * pos_base .. pos_base+n_tokens-1 of `layer`.  seq_len is not changed (the
 * reference loop drivers advance it separately).  Every position must be
 * mapped: pos_base + n_tokens <= mapped blocks * block_size.  n_tokens == 0
 * is a no-op (the row pointers may then be NULL); so for the two below. */
int sde_kv_append(sde_kv_cache* cache, int layer, const float* d_k,
                  const float* d_v, int pos_base, int n_tokens,
                  sde_stream_t stream);

/* As sde_kv_append with fp16 rows (raw bits, [n_tokens][kv_dim]) copied
 * without conversion.  No counterpart in the reference: a prefill helper
 * that lands pre-quantised context rows. */
int sde_kv_write_fp16(sde_kv_cache* cache, int layer, const uint16_t* d_k,
                      const uint16_t* d_v, int pos_base, int n_tokens,
                      sde_stream_t stream);

/* kv_cache_read (kv_cache.cu:95-114) over a range: K[pos..pos+n) and
 * V[pos..pos+n) of `layer` widened exactly to fp32 into [n][kv_dim]. */
int sde_kv_gather(const sde_kv_cache* cache, int layer, int pos,
                  int n_tokens, float* d_k, float* d_v, sde_stream_t stream);

/* Device-side view (pointers + shape) for in-tree HIP callers. */
int sde_kv_get_view(const sde_kv_cache* cache, sde_kv_view* out);

/* Workspace bytes sde_paged_attention needs for any call with these head
 * shapes, n_queries, and pos_base + n_queries <= max_total_len. */
size_t sde_paged_attention_workspace_size(const sde_kv_cache* cache, int nh,
                                          int nkv, int dph, int n_queries,
                                          int max_total_len);

/* Workspace bytes of the grid-cooperative device function
 * sde::device_flash_attention_gqa_grid (include/sde/attention_device.hpp),
 * which a persistent kernel calls in place of the block-0-only attention of
 * the reference's megakernel (kernels.cu:2727-2739), for windows of up to
 * n_queries queries over up to max_total_len positions.  0 for invalid
 * shapes.  The workspace's leading arrival counters must be zero before its
 * first use (every call leaves them zero). */
size_t sde_grid_attention_workspace_size(int nh, int nkv, int dph, int n_queries,
                                         int max_total_len);

/* cublas_attention_kernel (kernels.cu:904-940) + device_flash_attention_gqa
 * (attention.h:21-127): causal paged GQA attention for n_queries queries.
 * d_q, d_out: fp32 [n_queries][nh*dph] (q with RoPE applied).  Query m sees
 * keys/values at positions [0, pos_base+m+1) of `layer`; query head h reads
 * KV head h*nkv/nh (attention.h:37); scale dph^-1/2.  n_queries = 1 is a
 * decode step, n_queries = k+1 the speculative verify window.
 * d_workspace may be NULL (the cache then keeps its own, grown on demand);
 * otherwise it must hold sde_paged_attention_workspace_size(...) bytes.
 * Any dph up to 512 and any block size, nkv | nh, 1 <= n_queries <= 4096
 * (SDE_ERR_UNSUPPORTED for dph > 512): dph 64 / 128 with block sizes that
 * are multiples of 8 run the matrix-core tile kernels (those also need
 * nkv * ceil(n_queries * nh/nkv / 4) <= 4096), every other shape a plain
 * fp32 kernel with the same semantics and workspace.  The tile kernels
 * feed q * log2(e)/sqrt(dph) to the matrix cores as fp16 hi + lo parts, so
 * its elements must stay below 65504 in magnitude (|q| < 5.1e5 at dph 128,
 * 3.6e5 at dph 64; larger values overflow to Inf); the softmax weights are
 * at most 1.  Calls on one cache must be ordered on one stream (they share
 * the cache's arrival counters). */
int sde_paged_attention(sde_kv_cache* cache, int layer, const float* d_q,
                        float* d_out, int nh, int nkv, int dph, int pos_base,
                        int n_queries, void* d_workspace,
                        size_t workspace_bytes, sde_stream_t stream);

/* Bytes of the static device array sde_paged_attention_noalloc keeps its
 * partials in (one per device).  The tile kernels' partials (head sizes
 * 64 / 128) are at most (CUs x 16 rows) x (dph + 2) x 4 bytes, 2.1 MB on
 * MI355X's 256 CUs; the plain fp32 kernel of the other head sizes caps its
 * partition count so that its partials fit this size.  So on MI355X every
 * plan fits, and both entry points run the same plan. */
#define SDE_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

/* sde_paged_attention without a workspace, allocating nothing: the
 * split-context partials go to a static device array of the library
 * (SDE_NOALLOC_SCRATCH_BYTES per device, held until the process ends) and
 * the arrival counters are the cache's.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory during the call --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation.  Same arguments, results and errors as sde_paged_attention
 * (minus the workspace), plus SDE_ERR_WORKSPACE for a call whose partials
 * would exceed the array.  The first call on a device looks up the array's
 * address there (with the cache's device current).  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (on different
 * streams, or on different caches used concurrently) race on it and must
 * be ordered by the caller. */
int sde_paged_attention_noalloc(sde_kv_cache* cache, int layer, const float* d_q,
                                float* d_out, int nh, int nkv, int dph, int pos_base,
                                int n_queries, sde_stream_t stream);

/* Test hook for failure handling, no counterpart in the reference: sets the
 * number of polls (process-wide, for later calls) that a workgroup waiting
 * to combine a slice of a (KV head, row group)'s rows spends before it
 * gives up and leaves its slice to the group's last arriving workgroup
 * (0: give up at once).  Results are the same either way; only the combine's
 * parallelism changes.  Returns the previous value (the default is 16384). */
uint32_t sde_debug_set_slice_spin(uint32_t polls);

/* Test hook, no counterpart in the reference: the plan the tile path of
 * sde_paged_attention / sde_rope_append_attention takes for total_len keys,
 * nkv KV heads, `rows` = n_queries * (nh / nkv) rows per KV head, on a
 * device of n_cus compute units (host arithmetic only, no device call):
 * out[0] rows per group, out[1] row groups, out[2] tiles per wave in flight,
 * out[3] tiles per partition, out[4] partitions, out[5] the partition count
 * the workspace of sde_paged_attention_workspace_size(.., total_len) is
 * sized for.  SDE_ERR_INVALID_ARGUMENT for a non-positive size or a NULL
 * out. */
int sde_debug_attention_plan(int total_len, int nkv, int rows, int n_cus, int32_t out[6]);

/* Greedy acceptance + O(1) rewind of speculative decoding on the device,
 * with no host round trip (the reference's host loop kernels.cu:2428-2466
 * copies the tokens back and rewinds from the host; its megakernel does it
 * on thread 0, kernels.cu:3050-3072).  d_draft_tokens [k] and
 * d_target_tokens [k+1] (the verify window's argmaxes) are device int32.
 * Writes d_result[0..3] = {n_accepted, bonus token, target seq_len, draft
 * seq_len} and d_result[4 .. 4+n_accepted] = the emitted tokens (accepted
 * drafts, then the bonus): k+5 int32.  The target cache's seq_len becomes
 * target_save + n_accepted + 1; the draft cache's draft_save + n_accepted
 * (the reference's rule), or the target's value when draft is NULL or the
 * target itself (self-speculation over one cache).  The caches' host copy
 * of seq_len is refreshed from the device on the next host call that needs
 * it (sde_kv_seq_len, sde_kv_rollback), which then synchronizes the
 * device.  0 <= k <= 64; target_save + k + 1 and draft_save + k within the
 * caches' capacity (SDE_ERR_RANGE otherwise). */
int sde_spec_accept_greedy(sde_kv_cache* target, sde_kv_cache* draft,
                           const int32_t* d_draft_tokens,
                           const int32_t* d_target_tokens, int k,
                           int target_save, int draft_save, int32_t* d_result,
                           sde_stream_t stream);

/* Stochastic acceptance (Leviathan / Chen speculative sampling) + O(1)
 * rewind on the device: the reference's batch_stochastic_accept_kernel
 * (kernels.cu:550-572: accept draft i iff u < min(1, p_i / q_i), p_i the
 * target's and q_i the draft's probability of draft token i), its
 * correction sample on the first rejection (corrected_sample_adjusted_logits,
 * kernels.cu:319-380: a token from norm(max(0, p - q)), or from p when that
 * is empty), the bonus sample from p at row k when every draft was
 * accepted (softmax_sample_temperature_kernel), and the rewinds of
 * sde_spec_accept_greedy.  d_target_logits fp32 [k+1][vocab] (softmax at
 * temp_target), d_draft_logits fp32 [k][vocab] (at temp_draft; temperatures
 * below 1e-6 act as 1e-6), d_draft_tokens int32 [k].  Random draws:
 * Philox4x32-10 keyed by `seed` at the call index *d_rng_offset (a device
 * uint64 the call increments), two draws per window row, so a call is a
 * pure function of its inputs and the offset.  d_result as for
 * sde_spec_accept_greedy (k+5 int32: n_accepted, emitted token after the
 * accepted drafts, target seq_len, draft seq_len, emitted tokens).
 * 0 <= k <= 64, vocab >= 1.  One workgroup per window row. */
int sde_spec_accept_stochastic(sde_kv_cache* target, sde_kv_cache* draft,
                               const float* d_target_logits,
                               const float* d_draft_logits,
                               const int32_t* d_draft_tokens, int k, int vocab,
                               float temp_target, float temp_draft, uint64_t seed,
                               uint64_t* d_rng_offset, int target_save,
                               int draft_save, int32_t* d_result,
                               sde_stream_t stream);

/* RoPE scaling types: the reference's RopeScalingType (config.h:42-47). */
enum {
  SDE_ROPE_NONE = 0,
  SDE_ROPE_LINEAR = 1,
  SDE_ROPE_NTK = 2,
  SDE_ROPE_YARN = 3
};

typedef struct sde_rope_config {
  float theta;          /* rope_theta; <= 1e-6 selects 10000 (model.cu:290)  */
  int32_t scaling_type; /* SDE_ROPE_*                                          */
  float scaling_factor; /* applies when > 1                                   */
} sde_rope_config;

/* One layer's KV phase and attention fused in one launch: the work of
 * model_layer_kv_phase's RoPE and append (model.cu:346-384, i.e.
 * cublas_rope_kernel kernels.cu:797-817 + cublas_kv_append_kernel
 * kernels.cu:826-844) and cublas_attention_kernel (kernels.cu:904-940).
 * d_q fp32 [n_queries][nh*dph] and d_k, d_v fp32 [n_queries][nkv*dph] are
 * the projections BEFORE RoPE (not modified).  q and k are rotated by
 * rotate-half RoPE at positions pos_base+m (rope_apply_inplace,
 * model.cu:281-323: pair (j, j+dph/2), angle = pos' * theta^(-2j/dph), the
 * frequencies computed in double precision and rounded to fp32; the angle
 * and the rotation in fp32, sin / cos within 4.3e-7 of float64 -- for head
 * sizes 64 / 128 a 2 pi reduction and the hardware's sin / cos, sincosf
 * otherwise), k and v are appended (fp16 RNE) at those positions,
 * and query m attends causally to [0, pos_base+m].  Same shapes, limits,
 * workspace and errors as sde_paged_attention, plus SDE_ERR_INVALID_ARGUMENT
 * for a NULL d_k / d_v / rope, an unknown scaling type, or unaligned
 * d_k / d_v, and SDE_ERR_UNSUPPORTED for n_queries > 32 (a verify window is
 * at most MAX_VERIFY_BATCH = 9 rows, config.h:26; prefill takes the unfused
 * calls). */
int sde_rope_append_attention(sde_kv_cache* cache, int layer, const float* d_q,
                              const float* d_k, const float* d_v, float* d_out,
                              int nh, int nkv, int dph, int pos_base,
                              int n_queries, const sde_rope_config* rope,
                              void* d_workspace, size_t workspace_bytes,
                              sde_stream_t stream);

/* device_attention_dispatch (attention.h:140-164) as a host entry point:
 * SDE_ATTN_SOFTMAX runs sde_paged_attention; the reserved types return
 * SDE_ERR_UNSUPPORTED (where the reference traps) and launch nothing. */
int sde_attention_dispatch(int attn_type, sde_kv_cache* cache, int layer,
                           const float* d_q, float* d_out, int nh, int nkv,
                           int dph, int pos_base, int n_queries,
                           void* d_workspace, size_t workspace_bytes,
                           sde_stream_t stream);

/* Workspace bytes of sde_matvec and of the grid-cooperative device function
 * sde::device_matvec_grid (include/sde/matvec_device.hpp) for any call with
 * these shapes; 0 for invalid shapes.  Zero it once after allocation: its
 * leading arrival counters must start at zero (every call leaves them
 * zero). */
size_t sde_matvec_workspace_size(int d_in, int d_out, int n_rows);

/* The output projection after attention, across all CUs:
 * d_out[m][c] = (accumulate ? d_out[m][c] : 0) + sum_r d_x[m][r] * W[r][c]
 * for m < n_rows, c < d_out_dim, with W fp16 bits [d_in][d_out_dim]
 * (row-major, the SDEC weight layout, model.h:19) and fp32 x, out and
 * accumulation.  Replaces device_matvec_partial_accum striped over the
 * blocks of coop_layer_forward (utils.h:437-452, kernels.cu:2742-2747:
 * g_hidden += Wo(attn), accumulate = 1), device_matvec_batched for the
 * verify window's Wo (utils.h:248-280, model.cu:717: n_rows = B <= 9,
 * accumulate = 0) and the multi-kernel path's Wo GEMM + residual add
 * (kernels.cu:1069-1075, here with fp32 activations).  1 <= n_rows <= 16;
 * d_out_dim a multiple of 8, W 16-byte aligned, and one row range of W
 * (d_in split over the CUs) under 2 GiB (SDE_ERR_UNSUPPORTED otherwise).
 * d_workspace holds sde_matvec_workspace_size(...) bytes
 * (SDE_ERR_WORKSPACE when smaller); calls sharing a workspace must be
 * ordered on one stream.  Deterministic: the sum order does not depend on
 * scheduling.  One or two rows of x multiply in fp32 on the VALU; three or
 * more go to the matrix cores as fp16 hi + lo parts of x scaled, per row
 * and workgroup, by a power of two that keeps it within the fp16 range
 * (1 for |x| < 16384, so every Wo input; the sums are scaled back exactly):
 * any finite x at every row count, as in sde_matvec_packed. */
int sde_matvec(const float* d_x, const uint16_t* d_W, float* d_out, int d_in,
               int d_out_dim, int n_rows, int accumulate, void* d_workspace,
               size_t workspace_bytes, sde_stream_t stream);

/* Bytes of the panel-packed copy of a d_in x d_out fp16 W that
 * sde_matvec_packed streams (include/sde/matvec_packed.hpp gives the
 * layout); 0 when d_in or d_out is not a positive multiple of 8. */
size_t sde_matvec_packed_size(int d_in, int d_out_dim);

/* Writes the panel-packed copy of row-major W [d_in][d_out_dim] (fp16 bits,
 * 16-byte aligned) into d_packed (sde_matvec_packed_size bytes, 16-byte
 * aligned; SDE_ERR_WORKSPACE when smaller), stream-ordered.  A one-time
 * re-layout at weight-load time: the reference loads W as stored
 * (model.cu:89-260) and has no counterpart. */
int sde_matvec_pack(const uint16_t* d_W, int d_in, int d_out_dim, void* d_packed,
                    size_t packed_bytes, sde_stream_t stream);

/* sde_matvec's product over a packed copy: d_out[m][c] = (accumulate ?
 * d_out[m][c] : 0) + sum_r d_x[m][r] * W[r][c], the same replacement of
 * device_matvec_partial_accum / device_matvec_batched (utils.h:248-280,
 * 437-452; kernels.cu:2742-2747; model.cu:717) for callers that packed W
 * once.  One workgroup per panel of output columns, no workspace, no
 * cross-workgroup reduction; deterministic.  1 <= n_rows <= 16, d_in and
 * d_out_dim positive multiples of 8, d_x 16-byte aligned
 * (SDE_ERR_UNSUPPORTED otherwise). */
int sde_matvec_packed(const float* d_x, const void* d_packed, float* d_out, int d_in,
                      int d_out_dim, int n_rows, int accumulate, sde_stream_t stream);

/* ---- SDEC weight files (model_load_weights, model.cu:68-260) ------------ */

/* ModelConfig (config.h:67-83) as read from an SDEC header, plus the file
 * version.  v1/v2 files store expanded Wk/Wv and report n_kv_heads =
 * n_heads; kv_dim = n_kv_heads * (d_model / n_heads). */
typedef struct sde_model_config {
  int32_t n_layers;
  int32_t d_model;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t d_ff;
  int32_t vocab_size;
  float rope_theta;            /* 10000 before v2                         */
  int32_t rope_scaling_type;   /* SDE_ROPE_*, 0 before v3                 */
  float rope_scaling_factor;   /* 1 before v3                             */
  int32_t attention_type;      /* SDE_ATTN_*, 0 before v4                 */
  int32_t has_qkv_bias;        /* 0/1, v5                                 */
  uint32_t version;            /* 1..5                                    */
} sde_model_config;

/* LayerWeights (model.h:32-47): device pointers to fp16 bits, row-major
 * [in][out] as in the file; the biases are NULL without has_qkv_bias. */
typedef struct sde_layer_weights {
  const uint16_t* rms_attn_weight;  /* [d_model]           */
  const uint16_t* Wq;               /* [d_model][d_model]  */
  const uint16_t* Wk;               /* [d_model][kv_dim]   */
  const uint16_t* Wv;               /* [d_model][kv_dim]   */
  const uint16_t* Wo;               /* [d_model][d_model]  */
  const uint16_t* rms_mlp_weight;   /* [d_model]           */
  const uint16_t* W_gate;           /* [d_model][d_ff]     */
  const uint16_t* W_up;             /* [d_model][d_ff]     */
  const uint16_t* W_down;           /* [d_ff][d_model]     */
  const uint16_t* Wq_bias;          /* [d_model] or NULL   */
  const uint16_t* Wk_bias;          /* [kv_dim] or NULL    */
  const uint16_t* Wv_bias;          /* [kv_dim] or NULL    */
} sde_layer_weights;

/* The global tensors of ModelWeights (model.h:49-55). */
typedef struct sde_model_globals {
  const uint16_t* token_embedding;   /* [vocab_size][d_model] */
  const uint16_t* rms_final_weight;  /* [d_model]             */
  const uint16_t* output_proj;       /* [d_model][vocab_size] */
} sde_model_globals;

typedef struct sde_model sde_model;   /* opaque: the weights on one device */

/* Reads and validates an SDEC header (versions 1-5) the way
 * model_load_weights does (model.cu:83-192): magic "SDEC", version, the
 * version's fields, n_layers <= 40 (MAX_LAYERS, config.h:21), n_heads |
 * d_model, n_kv_heads | n_heads (and both >= 1).  Host only.  SDE_ERR_IO
 * for an unreadable file or a truncated header, SDE_ERR_FORMAT for a bad
 * magic, version or shape. */
int sde_model_read_header(const char* path, sde_model_config* cfg);

/* Device bytes sde_model_load allocates for a model of this config (one
 * arena, every tensor 256-byte aligned); 0 for an invalid config. */
size_t sde_model_weights_bytes(const sde_model_config* cfg);

/* model_load_weights (model.cu:83-260) onto the current device: the header
 * as sde_model_read_header, then token_embedding, rms_final_weight,
 * output_proj and per layer rms_attn, Wq, Wk, Wv, Wo, rms_mlp, W_gate,
 * W_up, W_down (+ Wq_bias, Wk_bias, Wv_bias with has_qkv_bias), each a
 * uint32 element count that must equal the shape's, then that many fp16
 * values.  The file is streamed through pinned staging buffers, disk reads
 * overlapping host-to-device copies.  On any error nothing stays allocated
 * and *out is NULL (SDE_ERR_FORMAT for a count mismatch, SDE_ERR_IO for a
 * short read).  cfg_out may be NULL. */
int sde_model_load(const char* path, sde_model** out, sde_model_config* cfg_out);

int sde_model_get_config(const sde_model* model, sde_model_config* cfg);
int sde_model_get_layer(const sde_model* model, int layer, sde_layer_weights* out);
int sde_model_get_globals(const sde_model* model, sde_model_globals* out);

/* model_free (model.cu:54-65). */
int sde_model_free(sde_model* model);

/* ---- persistent speculative decoding loop --------------------------------
 * megakernel_speculative (kernels.cu:2864-3106, host launcher
 * kernels.cu:3593-3755): the whole draft / verify / accept / rewind loop in
 * one cooperative launch, self-speculative over one cache (model.cu:838-890:
 * layers [0, n_draft) draft, layers [n_draft, n_layers) verify the k+1-token
 * window from the prefix layers' outputs).  The reference's loop runs its
 * transformer; this one runs the paged-KV path's model: layer l of token t
 * has q, k, v rows emb_q/emb_k/emb_v[l][t], q adding the previous layer's
 * attention output of the same row, and `head` (fp16, row-major [in][out] as
 * the reference stores weights, model.h:19) maps the last layer's attention
 * output to logits.  Every block of the grid runs the attention
 * (sde::device_flash_attention_gqa_grid) and the head (over a panel-packed
 * copy of it that the launch makes first in the workspace, sde_matvec_pack's
 * layout); each round drafts k tokens by greedy argmax,
 * verifies them, accepts the leading matches plus the target's next token
 * (sde::spec_accept_greedy) and rewinds seq_len to save + n_accepted + 1; the
 * next round starts at the device seq_len.  k = 0 is plain greedy decoding
 * through all layers (one token per round).  Head sizes 64 / 128 with block
 * sizes that are multiples of 8 run the grid attention's MFMA tile path;
 * other head sizes (up to 512) and block sizes run its generic fp32 path
 * (SDE_ERR_UNSUPPORTED above 512, or when n_heads * head_dim is not a
 * multiple of 8). */
typedef struct sde_loop_model {
  const float* emb_q;   /* [n_layers][vocab][n_heads*head_dim]                  */
  const float* emb_k;   /* [n_layers][vocab][kv_dim]                            */
  const float* emb_v;   /* [n_layers][vocab][kv_dim]                            */
  const uint16_t* head; /* fp16 bits [n_heads*head_dim][vocab], 16-byte aligned */
  int32_t vocab;        /* a multiple of 8                                      */
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t head_dim;     /* up to 512; n_kv_heads*head_dim == the cache's kv_dim */
} sde_loop_model;

/* Workspace bytes of sde_spec_loop_greedy and sde_spec_loop_stochastic for
 * this cache, model and k (the packed head copy included:
 * sde_matvec_packed_size(n_heads * head_dim, vocab) of them); 0 for invalid
 * shapes.  No initialisation needed (the loop writes what it uses). */
size_t sde_spec_loop_workspace_size(const sde_kv_cache* cache, const sde_loop_model* model,
                                    int k);

/* Runs rounds until max_new tokens are emitted.  The cache holds the
 * context at positions [0, seq_len) (the device seq_len word at launch);
 * d_state int32[8]: in [0] the last emitted token (not yet in the cache);
 * out [0] the last emitted token, [1] tokens emitted (max_new .. max_new+k-1),
 * [2] rounds, [3] status (SDE_OK, or SDE_ERR_CAPACITY when a window would
 * pass the layers' mapped blocks), [4] drafts proposed, [5] accepted.
 * d_emitted int32[max_new + k], d_accepted int32[max_new] (per round).
 * 0 <= k <= 15; 1 <= n_draft < n_layers when k > 0.  d_workspace: 256-byte
 * aligned, sde_spec_loop_workspace_size bytes.  One block per CU, all
 * resident (a cooperative launch); the cache's seq_len is then on the device
 * (sde_kv_device_seq_len). */
int sde_spec_loop_greedy(sde_kv_cache* cache, const sde_loop_model* model, int k, int n_draft,
                         int max_new, int32_t* d_state, int32_t* d_emitted,
                         int32_t* d_accepted, void* d_workspace, size_t workspace_bytes,
                         sde_stream_t stream);

/* Sampling parameters of the stochastic loop: the megakernel's
 * draft_temp_initial, adaptive_enabled, min/max_draft_temp,
 * adapt_tgt_accept, adapt_gain, adapt_ewma_mix and rng_seed
 * (kernels.cu:3108-3133). */
typedef struct sde_loop_sampling {
  float draft_temp;     /* initial draft temperature (below 1e-6 acts as 1e-6) */
  int32_t adaptive;     /* adapt the draft temperature after every round      */
  float min_temp;       /* clamp of the adapted temperature                   */
  float max_temp;
  float target_accept;  /* acceptance rate the adaptation aims at             */
  float gain;           /* temperature step per unit of rate error            */
  float ewma_mix;       /* weight of a round in the rate average (1e-6..1-1e-6) */
  uint64_t seed;        /* Philox key of every draw                           */
} sde_loop_sampling;

/* megakernel_speculative_stochastic_kernel (kernels.cu:3108-3481) in its
 * self-speculative form, in one cooperative launch like
 * sde_spec_loop_greedy: each draft token is sampled from the prefix layers'
 * logits at the draft temperature T_d, the window is verified by the
 * remaining layers, and speculative sampling (sde_spec_accept_stochastic's
 * rules and draws: target temperature 1, q at T_d) accepts, emits the
 * corrected or bonus sample and rewinds seq_len; T_d then adapts when
 * `adaptive` (an exponential average of the round's acceptance rate, moved
 * toward target_accept by gain, clamped).  Random draws: Philox4x32-10 keyed
 * by seed at the call index *d_rng_offset (device uint64, 8-byte aligned),
 * one call per draft token and one per acceptance, in that order.  d_state
 * as for sde_spec_loop_greedy, plus out [6] the final T_d and [7] the rate
 * average (float bits).  Same limits and errors as sde_spec_loop_greedy,
 * plus SDE_ERR_INVALID_ARGUMENT for a NULL sampling / offset, non-finite
 * parameters or min_temp > max_temp with adaptive set. */
int sde_spec_loop_stochastic(sde_kv_cache* cache, const sde_loop_model* model, int k,
                             int n_draft, int max_new, const sde_loop_sampling* sampling,
                             uint64_t* d_rng_offset, int32_t* d_state, int32_t* d_emitted,
                             int32_t* d_accepted, void* d_workspace, size_t workspace_bytes,
                             sde_stream_t stream);

/* The loop's whole configuration: GenerationParams' spec_k, max_new_tokens,
 * eos_token and self_speculative (config.h:139-160) as megakernel_speculative
 * (kernels.cu:3593-3755) reads them.  With draft_cache and draft_model set
 * (self_speculative false, kernels.cu:2864-2875 shared_kv false) a separate
 * draft model over a cache of its own drafts: per round, k one-token steps
 * through all its layers (window token s at draft position D+s, D its device
 * seq_len at the round's start), then the target verifies the window through
 * all its layers.  After the accept (sde::spec_accept_greedy, or the sampling
 * accept) the target rewinds to P + n + 1 and the draft to D + n
 * (draft_save + n_accepted), then the draft's catch-up forward
 * (kernels.cu:3079-3093) appends, at D + n, the last draft when all k were
 * accepted, else the bonus (the reference's order: the bonus then also sits
 * at D + n + 1 after the next round's first step), leaving the draft's
 * seq_len at D + n + 1.  eos_token >= 0 ends the loop after a round whose
 * bonus (its last emitted token) is that token (kernels.cu:3095, 3471);
 * d_state[1] then counts the tokens out, possibly below max_new. */
typedef struct sde_spec_loop_config {
  int32_t k;                        /* drafts per round, 0..15 (>= 1 with a draft model) */
  int32_t n_draft;                  /* self-speculative prefix layers (no draft model)   */
  int32_t max_new;                  /* tokens to emit (>= 1)                             */
  int32_t eos_token;                /* < 0: none                                        */
  sde_kv_cache* draft_cache;        /* NULL: self-speculative over `cache`              */
  const sde_loop_model* draft_model; /* the draft model over draft_cache (same vocab)   */
} sde_spec_loop_config;

/* Workspace bytes of sde_spec_loop for this configuration (both heads'
 * packed copies and the larger model's buffers included); 0 when invalid. */
size_t sde_spec_loop_config_workspace_size(const sde_kv_cache* cache,
                                           const sde_loop_model* model,
                                           const sde_spec_loop_config* cfg);

/* sde_spec_loop_greedy (sampling NULL) or sde_spec_loop_stochastic under a
 * configuration: the same state words, buffers, limits and errors, plus
 * SDE_ERR_INVALID_ARGUMENT for a draft model without its cache (or the
 * reverse), the target's own cache as the draft's, k = 0 with a draft model,
 * a different vocabulary or device.  Both caches' seq_len are then on the
 * device. */
int sde_spec_loop(sde_kv_cache* cache, const sde_loop_model* model,
                  const sde_spec_loop_config* cfg, const sde_loop_sampling* sampling,
                  uint64_t* d_rng_offset, int32_t* d_state, int32_t* d_emitted,
                  int32_t* d_accepted, void* d_workspace, size_t workspace_bytes,
                  sde_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* SDE_PAGED_KV_H */
