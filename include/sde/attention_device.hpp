/*
 * sde/attention_device.hpp — HIP device side of the MI355X (gfx950) paged KV
 * cache and paged GQA attention, for in-kernel callers (persistent /
 * megakernel decode loops) and for libsde_paged's own kernels.
 *
 * Reference device interface replaced (arkhamHack/speculative_decode_engine):
 *   cuda/include/kv_cache.h:70-79     kv_cache_append / kv_cache_read /
 *                                     kv_cache_rollback (device functions)
 *   cuda/include/attention.h:21-29    device_flash_attention_gqa
 *   cuda/include/attention.h:140-150  device_attention_dispatch
 * with the cache passed as the POD sde_kv_view (sde_kv_get_view), whose pool
 * and table layout is the reference's (kv_cache.h:5-18).  Both attention
 * functions also come with the reference's full argument list (the caller's
 * shared-memory scratch `blk_logits` and the five shared scalars), so a call
 * site of the reference compiles unchanged once its cache type is
 * sde_kv_view.
 *
 * The functions in namespace sde are block-cooperative like the reference's:
 * every thread of the calling block calls them with the same arguments
 * (blockDim.x a multiple of 64).  Their own staging lives in static LDS (see
 * each function).  Building blocks of the streaming attention live in
 * namespace sde::attn.
 *
 * Arithmetic: K and V are the cache's fp16 values.  q and the softmax
 * weights P enter the matrix cores as fp16 hi + lo pairs (x = hi + lo with
 * hi = fp16(x), lo = fp16(x - hi)), so each product carries ~22 bits of the
 * fp32 operand, as in the reference's fp32 q.K and P.V (attention.h:61-62,
 * 103-112); products and sums are fp32.
 */
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "sde_paged_kv.h"
#include "sde/attention_generic_device.hpp"
#include "sde/wave_uniform.hpp"

namespace sde {
namespace attn {

constexpr int kTile = 32;  // tokens per tile
constexpr double kLog2e = 1.4426950408889634;

// Where a (layer, context) of the paged cache lives: the pool, that layer's
// block table, and L_max, the number of positions [0, L_max) the window can
// see (every position below it has been written).
struct TileSource {
  const uint16_t* pool;
  const int32_t* table;
  int kv_dim;
  int bs;
  int L_max;
};

// Cross-lane moves (gfx950 lane semantics):
//  * DPP quad_perm [1,0,3,2] / [2,3,0,1] exchange lanes i^1 / i^2;
//  * v_permlane16_swap(x, x) returns rows {0,0,2,2} and {1,1,3,3} of the
//    four 16-lane rows;
//  * v_permlane32_swap(a, b) returns [a.lo | b.lo] and [a.hi | b.hi], so
//    their sum holds a's half-sum in lanes 0-31 and b's in lanes 32-63.
__device__ __forceinline__ float dpp_f(float x, int ctrl_sel) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  if (ctrl_sel == 0)
    r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);  // i^1
  else
    r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);  // i^2
  return __builtin_bit_cast(float, r);
}

// (even row, odd row) of this lane's pair of 16-lane rows.
__device__ __forceinline__ float2 row_pair(float x) {
  const int v = __builtin_bit_cast(int, x);
  const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return make_float2(__builtin_bit_cast(float, (int)p[0]), __builtin_bit_cast(float, (int)p[1]));
}

// Sums a (partial over lanes 0-31 and 32-63) and b likewise: lanes 0-31
// get a's total, lanes 32-63 b's total.
__device__ __forceinline__ float half_pair_total(float a, float b) {
  const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a),
                                                  __builtin_bit_cast(int, b), false, false);
  return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}

// Max / sum over the four 16-lane rows of a wave, returned to every lane
// (fixed order: rows (0 + 2) and (1 + 3), then the two pairs).
__device__ __forceinline__ float groups_max(float x) {
  const int v = __builtin_bit_cast(int, x);
  const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  x = fmaxf(__builtin_bit_cast(float, (int)h[0]), __builtin_bit_cast(float, (int)h[1]));
  const int w = __builtin_bit_cast(int, x);
  const auto r = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}

__device__ __forceinline__ float groups_sum(float x) {
  x = half_pair_total(x, x);
  const float2 p = row_pair(x);
  return p.x + p.y;
}

typedef const __attribute__((address_space(4))) int32_t* const_table_t;

// The block table is read-only during the kernel: reading it through the
// constant address space turns the entries into scalar loads (lgkmcnt),
// which never wait behind outstanding tile loads (vmcnt).
__device__ __forceinline__ const_table_t const_table(const TileSource& a) {
  return (const_table_t)a.table;
}

__device__ __forceinline__ uint4 ld16(const char* p) { return *reinterpret_cast<const uint4*>(p); }

// threadIdx.x through an opaque (volatile) move, taken once per work item:
// values derived from it (lane roles, LDS and load offsets) are then
// computed per item instead of being hoisted out of a caller's loop over
// items and kept live across the partition combine, which would spill.
__device__ __forceinline__ int item_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Physical block and in-block slot of the first token of each load group of
// tile ts (SL tokens per group, SL divides block_size).  Groups at or past
// L_max are pinned to token L_max-1 so every address stays on written data.
template <int NLD, int SL>
__device__ __forceinline__ void tile_groups(const TileSource& a, const_table_t table, int ts,
                                            int (&blk)[NLD], int (&slot)[NLD]) {
  if (ts + kTile <= a.L_max) {
    int lb = ts / a.bs;
    int s = ts - lb * a.bs;
#pragma unroll
    for (int j = 0; j < NLD; j++) {
      blk[j] = table[lb];
      slot[j] = s;
      s += SL;
      if (s == a.bs) {
        s = 0;
        ++lb;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NLD; j++) {
      const int g = min(ts + j * SL, a.L_max - 1);
      const int lb = g / a.bs;
      blk[j] = table[lb];
      slot[j] = g - lb * a.bs;
    }
  }
}

// Issues the K (is_v false) or V loads of tile ts: load j brings token
// ts + j*SL + sl, 16-byte chunk c (lane_off = sl*row_bytes + 16c from the
// group's first token).  Lanes whose token is at or past L_max read the
// group's first token instead (chunk_off = 16c); their logits are masked.
// Every path issues the same NLD loads, so the compiler's vmcnt bookkeeping
// stays exact across tiles.
template <int DPH>
__device__ __forceinline__ void stream_load(const TileSource& a, const char* head_base, int ts,
                                            int sl, uint32_t lane_off, uint32_t chunk_off,
                                            bool is_v, const int (&blk)[kTile / (512 / DPH)],
                                            const int (&slot)[kTile / (512 / DPH)],
                                            uint4 (&x)[kTile / (512 / DPH)]) {
  constexpr int SL = 512 / DPH;
  constexpr int NLD = kTile / SL;
  const uint32_t row_bytes = 2u * (uint32_t)a.kv_dim;
  const uint32_t v_bytes = (uint32_t)a.bs * row_bytes;
  const bool full = ts + kTile <= a.L_max;
#pragma unroll
  for (int j = 0; j < NLD; j++) {
    const char* ub = head_base + (uint64_t)(uint32_t)blk[j] * (2ull * v_bytes) +
                     (uint32_t)slot[j] * row_bytes + (is_v ? v_bytes : 0u);
    const uint32_t off = (full || ts + j * SL + sl < a.L_max) ? lane_off : chunk_off;
    x[j] = ld16(ub + off);
  }
  // Compiler barriers: keep the loads here instead of letting them sink to
  // their first use a tile later, and keep the scheduler from interleaving
  // neighbouring tiles' work (code-motion fences only; no wait).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Fused RoPE + append (sde_rope_append_attention): the window's k and v
// rows before RoPE, and the rotate-half RoPE of rope_apply_inplace
// (model.cu:281-323): pair (j, j + dph/2) of a head rotates by angle
// (pos / pos_div) * inv_freq[j], with pos_div the linear / YaRN position
// divisor (1 otherwise) and inv_freq[j] = theta^(-2j/dph) (theta already
// NTK-scaled) computed on the host in double precision.
struct RopeArgs {
  const float* k_new;  // [M][kv_dim] fp32, before RoPE
  const float* v_new;  // [M][kv_dim] fp32
  uint16_t* pool;      // the pool (written)
  float pos_div;
  float inv_freq[64];  // dph/2 entries
};

// A persistent loop's window taken straight from its model's tables (the
// gathered form of the grid attention): q row m is q_table row tok[m], plus
// q_add row m when q_add is set (the previous layer's output); the window's
// K / V rows (positions pos_base + m) are k_table / v_table rows tok[m],
// rounded to fp16 and appended by the partitions that read them.
struct GatherArgs {
  const int32_t* tok;     // [M] the window's tokens
  const float* q_table;   // [vocab][nh*dph] (the layer's)
  const float* q_add;     // [M][nh*dph], or null
  const float* k_table;   // [vocab][kv_dim] (the layer's)
  const float* v_table;   // [vocab][kv_dim]
  uint16_t* pool;         // the pool (written)
};

__device__ __forceinline__ float rope_angle(const RopeArgs& rp, int pos, int j) {
  return ((float)pos / rp.pos_div) * rp.inv_freq[j];
}

// sin and cos of an fp32 angle x (radians) for RoPE.  The hardware's
// v_sin_f32 / v_cos_f32 take revolutions and are accurate on a reduced
// argument, so x is reduced by 2 pi first (Cody-Waite): k = rint(x / 2 pi),
// r = x - k (C1 + C2 + C3) with 2 pi = C1 + C2 + C3 to 2e-14 (C1 = 201/32 and
// C2 = 507 * 2^-18 short enough that every partial difference is exact for
// |x| < 2^17, C3 = the fp32 remainder), then r / 2 pi, within [-0.51, 0.51].
// Measured error at most 4.3e-7 against float64 (sincosf: ~6e-8), nearly
// all of it the reduction's and the revolution product's rounding
// (tests/test_gpu_fused_rope.py, test_rope_sincos_against_float64); the
// reference's fast-math sinf / cosf (model.cu:308-309 under
// --use_fast_math) reduce nothing at all.  Angles of 2^17 or more take
// sincosf.
__device__ __forceinline__ void rope_sincos(float x, float& sn, float& cs) {
  if (fabsf(x) < 131072.f) {
    constexpr float kInv2Pi = 0x1.45f306p-3f;
    const float k = rintf(x * kInv2Pi);
    float r = fmaf(-k, 6.28125f, x);
    r = fmaf(-k, 0x1.fbp-10f, r);
    r = fmaf(-k, 0x1.5110b4p-20f, r);
    const float rev = r * kInv2Pi;
    sn = __builtin_amdgcn_sinf(rev);
    cs = __builtin_amdgcn_cosf(rev);
  } else {
    sincosf(x, &sn, &cs);
  }
}

// Window rows the fused entry point takes (a speculative window is k + 1
// rows; each wave's rotation table covers only its own group's queries).
constexpr int kRopeMaxQueries = 32;

// RoPE of a wave's q rows (mfma_pack_q): the window queries its rows
// belong to are p0 .. p0+nm-1 (positions); lane l holds inv_freq[l % (dph/2)]
// in fr (loaded before the lane's q, so the table waits for no q load) and
// reads the table row of its own query, mi (0 for a padding row).  The
// angle is rope_angle's, so q and the appended k rotate alike.
struct QRope {
  float fr;
  float pos_div;
  int p0, nm, mi;
};

// attention.h:120-126: normalise unless the sum is tiny or not finite.
__device__ __forceinline__ float finish_scale(float l) {
  return (l > 1e-20f && isfinite(l)) ? 1.f / l : 0.f;
}

// ---- split-context partitions (libsde_paged's kernel and the grid API) ----

// One split-context attention call: rows of KV head kvh are its
// (query m, head-in-group g) pairs r = m*G + g; row groups of RPW rows; the
// context [0, L_max) is cut into n_parts partitions of tiles_per_part tiles.
struct AttnArgs {
  TileSource src;        // pool, this layer's table, kv_dim, block_size, L_max
  const float* q;        // [M][nh*dph]
  float* out;            // [M][nh*dph]
  float* partials;       // [nkv][R][n_parts][dph] acc, then [nkv][R][n_parts][2] (max, sum)
  uint32_t* counters;    // [nkv][row_groups] arrival counters, zero at rest
  int nh;
  int nkv;
  int G;           // query heads per KV head
  int R;           // rows per KV head = M * G
  int row_groups;  // ceil(R / rows per group)
  int pos_base;    // query m sees positions [0, pos_base+m]
  int n_parts;
  int tiles_per_part;
  float qscale;    // log2(e) / sqrt(dph)
  int ctr_stride = 1;  // words between the arrival counters (32: one 128-byte line each)
  uint32_t slice_spin = 1u << 14;  // polls of a split combine's wait (kSliceSpinLimit)
};

constexpr int kStreamWaves = 8;      // waves per workgroup of libsde_paged's kernel
constexpr int kStreamMaxParts = 64;  // partitions per (KV head, row group)
constexpr int kSliceRows = 4;        // rows per slice of a split combine (stream_item)

// Rows per slice for groups of RPW rows: groups of 8 and 16 rows in 2-row
// slices (at most 8, the most the arrival word's give-up bits track), the
// decodes' 4-row groups whole (measured on MI355X, two boxes: the
// Qwen2.5-7B window 19.3 -> 19.1-19.3 us, fused 18.0-18.5 -> 17.9, a
// 5-query window over 16K keys 27.4-27.7 -> 27.1-27.4, the Qwen2.5-7B
// draft step's 7-row group 14.2 -> 14.1, the 4K windows unchanged; 2-row
// slices of the decodes' 4-row groups measured slower).
template <int RPW>
constexpr int slice_rows() { return RPW >= 8 ? 2 : kSliceRows; }
constexpr uint32_t kSliceSpinLimit = 1u << 14;  // polls of a slice's wait (~10 ms)

// Device-scope (agent) relaxed atomic accesses for the partition partials.
// Memory-ordering argument (gfx950): an agent-scope relaxed store is a
// global store with the sc1 cache policy, which writes through the issuing
// XCD's L2 to the device coherence point (MALL / HBM); an agent-scope
// relaxed load (sc1) misses in the reader's L2 and reads that point.  The
// publisher issues its partial stores, waits for them (s_waitcnt vmcnt(0):
// a store's counter drops once it is acknowledged at the coherence point),
// then increments the arrival counter with an agent-scope atomic, which
// itself executes at that point.  The combiner observes the final count
// from the same atomic, so every publisher's stores were acknowledged
// before it, and its sc1 loads cannot hit a stale L2 line.  No L2
// writeback/invalidate fence is needed (those cost microseconds per
// workgroup here).
__device__ __forceinline__ void store_dev2(float* p, float x, float y) {
  const uint64_t bits = (uint64_t)__builtin_bit_cast(uint32_t, x) |
                        ((uint64_t)__builtin_bit_cast(uint32_t, y) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 load_dev2(const float* p) {
  const uint64_t bits = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__builtin_bit_cast(float, (uint32_t)bits),
                     __builtin_bit_cast(float, (uint32_t)(bits >> 32)));
}

// 16 bytes at base + byte_off with the same device-scope cache policy as
// load_dev2 (buffer_load_dwordx4 ... sc1; raw buffer, range-checked by
// `bytes`).  One 16-byte request instead of two 8-byte ones: the combine's
// partial loads are request-bound.
__device__ __forceinline__ float4 load_dev16(const float* base, uint32_t bytes,
                                             uint32_t byte_off) {
  constexpr int kSc1 = 16;                     // cache policy bit of sc1
  constexpr int kRsrcWord3 = 0x00020000;       // gfx9 raw buffer, 32-bit data format
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(wave_uniform(base)), 0,
                                        (int)wave_uniform(bytes), kRsrcWord3);
  // Bit-cast the whole vector: extracting elements of the builtin's integer
  // vector result makes this compiler shrink the load to one dword.
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v v = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
  return make_float4(v.x, v.y, v.z, v.w);
}

// 8 bytes at base + byte_off, device scope like load_dev2, through a raw
// buffer of `bytes` bytes: an offset past the range reads zeros and sends
// no request to memory.
__device__ __forceinline__ float2 load_dev8(const float* base, uint32_t bytes, uint32_t byte_off) {
  constexpr int kSc1 = 16;
  constexpr int kRsrcWord3 = 0x00020000;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(wave_uniform(base)), 0,
                                        (int)wave_uniform(bytes), kRsrcWord3);
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v v = __builtin_bit_cast(f2v, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kSc1));
  return make_float2(v.x, v.y);
}

// An offset no buffer of this library's partials reaches: the load returns
// zeros without a memory request.
constexpr uint32_t kOutOfRange = 0xFFFFFFF0u;

// Lane i ^ 4 / i ^ 8 (ds_swizzle, bit-mask mode within 32 lanes).
__device__ __forceinline__ float swz_xor4(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x101F));
}
__device__ __forceinline__ float swz_xor8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x201F));
}

// Max / sum over the 64 lanes by xor butterflies (within 16-lane rows, then
// across rows): every lane gets the same bits, in a fixed order.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f(x, 0));
  x = fmaxf(x, dpp_f(x, 1));
  x = fmaxf(x, swz_xor4(x));
  x = fmaxf(x, swz_xor8(x));
  return groups_max(x);
}
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f(x, 0);
  x += dpp_f(x, 1);
  x += swz_xor4(x);
  x += swz_xor8(x);
  return groups_sum(x);
}

// One pass of the partition combine.  An item is one row's 64-feature
// column slice, served by a whole wave: lane (sub = lane/16, c = lane%16)
// takes float4 column c of the slice for partitions sub, sub+4, ..., so the
// 16 lanes of a sub-group read 256 contiguous bytes of one partition's
// record.  The combine is bound by the rate at which one CU issues these
// device-scope loads, so slots past the last partition load from beyond
// the buffer (zeros, no request), and every load of the pass is issued
// before any arithmetic (one round trip; a load under `if (p < P)` would
// get a wait of its own at the join).  Per item, lane p holds partition
// p's (max, sum): the row's max, each partition's weight exp2(m_p - max)
// and the weighted sum of the sums are wave reductions done once, and each
// lane reads its partitions' weights across lanes; the four sub-groups of
// a column then reduce by lane swaps in a fixed order, so the result does
// not depend on arrival order.
template <int DPH, int PMAX, int NIT, int WAVES>
__device__ __forceinline__ void combine_pass(const AttnArgs& a, int tid, int kvh, int r0,
                                             int nrows, int it0) {
  constexpr int SUB = 4;
  constexpr int SLICES = DPH / 64;  // column slices per row
  const int P = a.n_parts;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane >> 4;
  const int c = lane & 15;
  const size_t acc_floats = (size_t)a.nkv * a.R * P * DPH;
  const uint32_t acc_bytes = (uint32_t)(acc_floats * 4);
  const uint32_t all_bytes = (uint32_t)((acc_floats + (size_t)a.nkv * a.R * P * 2) * 4);
  float4 v[NIT][PMAX];
  float2 ml[NIT];
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int item = wave + (it0 + it) * WAVES;  // uniform per wave
    const int r = item / SLICES;
    if (r < nrows) {
      const int col4 = (item - r * SLICES) * 16 + c;
      const size_t row = (size_t)kvh * a.R + r0 + r;
      const uint32_t acc_off = (uint32_t)((row * P * DPH + 4 * col4) * 4);
#pragma unroll
      for (int i = 0; i < PMAX; i++) {
        const int p = sub + i * SUB;
        v[it][i] = load_dev16(a.partials, acc_bytes,
                              p < P ? acc_off + (uint32_t)p * (DPH * 4) : kOutOfRange);
      }
      ml[it] = load_dev8(a.partials, all_bytes,
                         lane < P ? (uint32_t)((acc_floats + row * P * 2 + (size_t)lane * 2) * 4)
                                  : kOutOfRange);
    }
  }
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int item = wave + (it0 + it) * WAVES;
    const int r = item / SLICES;
    if (r >= nrows) break;
    const int col4 = (item - r * SLICES) * 16 + c;
    const float m = lane < P ? ml[it].x : -INFINITY;
    const float mx = wave_max(m);
    const float wgt = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mx);
    const float l = wave_sum(lane < P ? ml[it].y * wgt : 0.f);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < PMAX; i++) {
      const float w = __shfl(wgt, sub + i * SUB);  // 0 past the last partition
      o.x += w * v[it][i].x;
      o.y += w * v[it][i].y;
      o.z += w * v[it][i].z;
      o.w += w * v[it][i].w;
    }
    o.x = groups_sum(o.x);
    o.y = groups_sum(o.y);
    o.z = groups_sum(o.z);
    o.w = groups_sum(o.w);
    if (sub == 0) {
      const float inv = finish_scale(l);
      const int gr = r0 + r;
      const int mq = gr / a.G;
      const int h = kvh * a.G + (gr - mq * a.G);
      float2* dst = reinterpret_cast<float2*>(a.out + (size_t)mq * a.nh * DPH + (size_t)h * DPH +
                                              4 * col4);
      dst[0] = make_float2(o.x * inv, o.y * inv);
      dst[1] = make_float2(o.z * inv, o.w * inv);
    }
  }
}

// Passes of up to 32 in-flight partial loads per thread.
template <int DPH, int RPW, int PMAX, int WAVES>
__device__ __forceinline__ void combine_rows(const AttnArgs& a, int tid, int kvh, int r0,
                                             int nrows) {
  constexpr int ITEMS = RPW * (DPH / 64);
  constexpr int PER_WAVE = (ITEMS + WAVES - 1) / WAVES;
  constexpr int CAP = 32 / PMAX;
  constexpr int NIT = PER_WAVE < CAP ? PER_WAVE : CAP;
#pragma unroll
  for (int it0 = 0; it0 < PER_WAVE; it0 += NIT)
    combine_pass<DPH, PMAX, NIT, WAVES>(a, tid, kvh, r0, nrows, it0);
}

// Partition combine, run by the last workgroup of a (KV head, row group) to
// finish (the rows r0 .. r0+nrows-1 of KV head kvh).
template <int DPH, int RPW, int WAVES>
__device__ __forceinline__ void stream_combine(const AttnArgs& a, int tid, int kvh, int r0,
                                               int nrows) {
  static_assert(kStreamMaxParts == 64, "combine buckets");
  static_assert(DPH % 64 == 0, "a wave serves one 64-feature column slice of a row");
  if (tid >= 64 * WAVES) return;  // waves past WAVES idle
  const int P = a.n_parts;
  if (P <= 16)
    combine_rows<DPH, RPW, 4, WAVES>(a, tid, kvh, r0, nrows);
  else if (P <= 32)
    combine_rows<DPH, RPW, 8, WAVES>(a, tid, kvh, r0, nrows);
  else
    combine_rows<DPH, RPW, 16, WAVES>(a, tid, kvh, r0, nrows);
}

// A split combine's protocol on one 32-bit word per (KV head, row group),
// zero at rest: bits 0-7 count the arrivals (n_parts <= 64), bits 8-15 the
// waiting workgroups' final operations, bits 16-23 the slices given up.
// The workgroup arriving s places before the last (1 <= s < n_slices)
// waits for the arrivals to complete (bounded: `limit` polls), then adds
// its final operation and combines slice s; if its wait runs out first it
// adds its final operation with its give-up bit -- and still combines the
// slice when that add shows every arrival in (the last arrival, having
// come in between, did not see the bit).  The last arrival combines slice
// 0 and every slice its arrival add shows given up.  Whichever operation
// is the word's last (n_parts arrivals + n_slices - 1 finals) resets it.
// So no wait holds up the grid, every slice is combined exactly once, and
// nobody reads the word after its final operation.  Returns this
// workgroup's slice (-1: none); `extra` receives, for the last arrival,
// the slices given up (bit s: slice s).
constexpr uint32_t kSliceFinal = 1u << 8;

__device__ __forceinline__ int slice_arrive(uint32_t* ctr, uint32_t prev, int n_parts,
                                            int n_slices, uint32_t limit, int& extra) {
  const uint32_t want = (uint32_t)n_parts;
  const uint32_t last_op = want | ((uint32_t)(n_slices - 1) << 8);  // the word after every op
  const uint32_t arrived = prev & 0xFFu;
  if (arrived >= want) return -1;  // impossible: the word is zero at rest
  const int rank = n_parts - 1 - (int)arrived;
  if (rank == 0) {  // the last arrival
    const uint32_t now = prev + 1u;
    if ((now & 0xFFFFu) == last_op)  // every wait gave up already
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    extra = (int)((prev >> 16) & 0xFFu);
    return 0;
  }
  if (rank >= n_slices) return -1;
  bool all_in = false;
  for (uint32_t spin = 0; spin < limit; spin++) {
    if ((__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0xFFu) >= want) {
      all_in = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  const uint32_t add = kSliceFinal | (all_in ? 0u : (1u << (16 + rank)));
  const uint32_t old = __hip_atomic_fetch_add(ctr, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t now = old + add;
  if ((now & 0xFFFFu) == last_op)
    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // given up but every arrival already in: the last arrival did not see the bit
  return (all_in || (old & 0xFFu) >= want) ? rank : -1;
}

// The window's rows (positions pos_base .. pos_base+M-1) of KV head kvh:
// k rotated by RoPE, k and v rounded to fp16 (RNE) into the pool
// (kv_cache_append, kv_cache.cu:70-93), by the whole workgroup, one thread
// per (row, rotation pair) -- its k pair, v pair and rope_sincos, all loads
// issued together; returns once the stores are visible to the workgroup's
// loads.
template <int DPH>
__device__ __forceinline__ void rope_append_slice(const AttnArgs& a, const RopeArgs& rp,
                                                  int kvh) {
  constexpr int HALF = DPH / 2;
  const int M = a.R / a.G;
  const int kvd = a.src.kv_dim;
  const int bs = a.src.bs;
  for (int t = threadIdx.x; t < M * HALF; t += blockDim.x) {
    const int m = t / HALF;
    const int j = t - m * HALF;
    const int pos = a.pos_base + m;
    const size_t in = (size_t)m * kvd + (size_t)kvh * DPH + j;
    const float x0 = rp.k_new[in], x1 = rp.k_new[in + HALF];
    const float v0 = rp.v_new[in], v1 = rp.v_new[in + HALF];
    const int lb = pos / bs;
    const int slot = pos - lb * bs;
    uint16_t* kd = rp.pool + ((size_t)(uint32_t)a.src.table[lb] * 2u * bs + slot) * kvd +
                   (size_t)kvh * DPH + j;
    uint16_t* vd = kd + (size_t)bs * kvd;
    float sn, cs;
    rope_sincos(rope_angle(rp, pos, j), sn, cs);
    kd[0] = __builtin_bit_cast(uint16_t, (_Float16)(x0 * cs - x1 * sn));
    kd[HALF] = __builtin_bit_cast(uint16_t, (_Float16)(x0 * sn + x1 * cs));
    vd[0] = __builtin_bit_cast(uint16_t, (_Float16)v0);
    vd[HALF] = __builtin_bit_cast(uint16_t, (_Float16)v1);
  }
  __syncthreads();
}

// ---- MFMA tile path (v_mfma_f32_16x16x32_f16, up to 16 rows per wave) ----
//
// K and V stream in with coalesced loads (a token's slice read by dph/8
// lanes, 16 bytes each) and are staged per wave in LDS, row-major by token
// with the 16-byte units of row t stored at unit u ^ (t % UNITS), which
// keeps both the stores and the operand reads below free of bank
// conflicts.  Per tile of 32 tokens:
//  * logits S^T[token][row] = K . Q^T: A = K read from LDS in the operand
//    layout (lane l: token l%16 of a 16-token block, features
//    32ks + 8(l/16) .. +7), B = Q^T (row l%16, the same features), once
//    with q's hi part and once with its lo part.  The C layout leaves lane
//    l the logits of row l%16 for tokens 4(l/16) + i and 16 + 4(l/16) + i
//    (i < 4), so the online softmax is lane-local per row: one cross-group
//    max per tile (two lane swaps), sums reduced once.
//  * O^T[feature][row] += V^T . P^T: B = P^T straight from the logits'
//    registers as fp16 hi and lo parts (k order: tokens 4(l/16)+i, then
//    16+4(l/16)+i), A = V^T read with ds_read_b64_tr_b16: in each 16-lane
//    group lane 4b+t receives element t of the 8-byte pieces addressed by
//    lanes b, b+4, b+8, b+12, so lane m' addressing token base + m'/4,
//    features 16db + 4(m'%4) gives lane m feature 16db + m of tokens
//    base..base+3 (the A layout).
// The output C layout holds features 16db + 4(l/16) + i of row l%16 in lane
// l, so the rescale by the row's exp2(m_old - m_new) is lane-local too.
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;

template <int DPH>
struct MfmaShape {
  static constexpr int KS = DPH / 32;         // k-steps of the logits product
  static constexpr int DB = DPH / 16;         // 16-feature blocks of the output
  static constexpr int UNITS = DPH / 8;       // 16-byte units per token row
  static constexpr int ROWB = 2 * DPH;        // bytes per staged row
  static constexpr int TILEB = kTile * ROWB;  // bytes of one staged K or V tile
  static constexpr int WAVEB = 2 * TILEB;     // LDS bytes per wave (K and V)
};

// x = hi + lo to ~22 bits: hi = fp16(x), lo = fp16(x - hi) (the difference
// is exact in fp32).  x is pinned as a rounded fp32 register first: when x
// is a product, the compiler would otherwise form the hi it subtracts with
// a fused multiply-convert (v_fma_mixlo_f16: one rounding of the exact
// product) but the hi it stores with v_mul_f32 + v_cvt_pk_f16_f32 (two
// roundings), and where the fp32 product lands on an fp16 tie the two
// differ by one fp16 ulp, which hi + lo would then carry.
__device__ __forceinline__ void split_h8(const float (&x)[8], h8_t& hi, h8_t& lo) {
#pragma unroll
  for (int e = 0; e < 8; e++) {
    float v = x[e];
    asm("" : "+v"(v));
    const _Float16 h = (_Float16)v;
    hi[e] = h;
    lo[e] = (_Float16)(v - (float)h);
  }
}

// Byte offset of 16-byte unit u of token row t in a staged tile.
template <int DPH>
__device__ __forceinline__ int staged(int t, int u) {
  using Sh = MfmaShape<DPH>;
  return t * Sh::ROWB + 16 * (u ^ (t & (Sh::UNITS - 1)));
}

// Stores a tile held in the load layout (load j: token j*SL + sl, unit c).
template <int DPH>
__device__ __forceinline__ void stage_tile(char* st, int sl, int c,
                                           const uint4 (&x)[kTile / (512 / DPH)]) {
  constexpr int SL = 512 / DPH;
#pragma unroll
  for (int j = 0; j < kTile / SL; j++)
    *reinterpret_cast<uint4*>(st + staged<DPH>(j * SL + sl, c)) = x[j];
}

// Logits of a tile, masking (token position > lim), the online softmax
// update and the rescale of o; p receives the tile's probabilities in the
// C layout (p[4tb + i]: token 16tb + 4(l/16) + i of row l%16).  kst: this
// wave's staged K tile.
template <int DPH>
__device__ __forceinline__ void mfma_logits(int ts, int lane, int q, int l16, int lim,
                                            const h8_t* qop, const char* kst, float& m_run,
                                            float& l_run, f4_t (&o)[MfmaShape<DPH>::DB],
                                            float (&p)[8]) {
  using Sh = MfmaShape<DPH>;
  f4_t s[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int ks = 0; ks < Sh::KS; ks++) {
    const h8_t qh = qop[ks * 64 + lane];
    const h8_t ql = qop[(Sh::KS + ks) * 64 + lane];
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
      const h8_t kx = __builtin_bit_cast(
          h8_t, *reinterpret_cast<const uint4*>(kst + staged<DPH>(16 * tb + l16, 4 * ks + q)));
      s[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kx, qh, s[tb], 0, 0, 0);
      s[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kx, ql, s[tb], 0, 0, 0);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int tb = 0; tb < 2; tb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float x = ts + 16 * tb + 4 * q + i <= lim ? s[tb][i] : -INFINITY;
      s[tb][i] = x;
      mx = fmaxf(mx, x);
    }
  const float m_new = fmaxf(m_run, groups_max(mx));
  const float m_use = m_new == -INFINITY ? 0.f : m_new;
  const float al = __builtin_amdgcn_exp2f(m_run - m_use);
  m_run = m_new;
  float ps = 0.f;
#pragma unroll
  for (int tb = 0; tb < 2; tb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p[4 * tb + i] = __builtin_amdgcn_exp2f(s[tb][i] - m_use);
      ps += p[4 * tb + i];
    }
  l_run = l_run * al + ps;
#pragma unroll
  for (int db = 0; db < Sh::DB; db++) o[db] *= al;
}

// o += V^T . P^T for a tile (P as hi + lo parts); vst: this wave's staged
// V tile.
template <int DPH>
__device__ __forceinline__ void mfma_pv(int q, int l16, const h8_t ph, const h8_t pl,
                                        const char* vst, f4_t (&o)[MfmaShape<DPH>::DB]) {
  using Sh = MfmaShape<DPH>;
  const int t0 = 4 * q + (l16 >> 2);   // token of this lane's piece (first half)
  const int sub = 8 * (l16 & 1);       // byte within the 16-byte unit
  const int u0 = (l16 & 3) >> 1;       // unit within the 32 bytes of a feature block
#pragma unroll
  for (int db = 0; db < Sh::DB; db++) {
    const s4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s4_t*)(vst + staged<DPH>(t0, 2 * db + u0) + sub));
    const s4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s4_t*)(vst + staged<DPH>(t0 + 16, 2 * db + u0) + sub));
    const s4_t both[2] = {lo, hi};
    const h8_t a = __builtin_bit_cast(h8_t, both);
    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, o[db], 0, 0, 0);
    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, o[db], 0, 0, 0);
  }
}

// Bits 15 / 31 set where the low / high fp16 of x has an all-ones exponent
// (Inf or NaN): adding 1 to the 5-bit exponent field carries into the bit
// above it only from 31, and the low field's carry stops at bit 15.
__device__ __forceinline__ uint32_t nonfinite_h2(uint32_t x) {
  return ((x & 0x7C007C00u) + 0x04000400u) & 0x80008000u;
}

// Whether any lane holds a non-finite V element in a slot of tile ts that
// some real row of the wave may not see (position > wmin, the smallest
// limit over the real rows; this includes slots past L_max, which hold a
// copy of another token, and the fully masked slots past a wave's last
// tile).  Those slots have zero weight for such rows, and the matrix
// product would turn 0 x Inf into NaN there; the reference never reads
// them (attention.h:98-115).  Wave-uniform.
template <int DPH>
__device__ __forceinline__ bool hidden_nonfinite(int ts, int sl, int wmin,
                                                 const uint4 (&v)[kTile / (512 / DPH)]) {
  constexpr int SL = 512 / DPH;
  uint32_t bad = 0;
#pragma unroll
  for (int j = 0; j < kTile / SL; j++) {
    const uint32_t nf = nonfinite_h2(v[j].x) | nonfinite_h2(v[j].y) | nonfinite_h2(v[j].z) |
                        nonfinite_h2(v[j].w);
    if (ts + j * SL + sl > wmin) bad |= nf;
  }
  return __builtin_amdgcn_ballot_w64(bad != 0) != 0;
}

// o += P . V for a tile over the tokens each row sees, skipping the rest
// (the reference's loop, attention.h:98-115): the exact-semantics path of
// a tile for which hidden_nonfinite holds.  The tile's probabilities go
// over the wave's staged K tile (dead after the logits; a wave's LDS
// operations complete in order), then each lane accumulates its row's
// visible tokens against its features of the staged V rows in fp32.
template <int DPH>
__device__ __forceinline__ void masked_pv(int ts, int q, int l16, int lim, const float (&p)[8],
                                          char* kst, const char* vst,
                                          f4_t (&o)[MfmaShape<DPH>::DB]) {
  using Sh = MfmaShape<DPH>;
  float* pt = reinterpret_cast<float*>(kst);
#pragma unroll
  for (int tb = 0; tb < 2; tb++)
#pragma unroll
    for (int i = 0; i < 4; i++) pt[l16 * kTile + 16 * tb + 4 * q + i] = p[4 * tb + i];
#pragma unroll 1
  for (int t = 0; t < kTile; t++) {
    const float w = pt[l16 * kTile + t];
    const bool vis = ts + t <= lim;
#pragma unroll
    for (int db = 0; db < Sh::DB; db++) {
      // features 16db + 4q .. +3: unit 2db + q/2, byte 8(q%2) of it
      const uint2 v =
          *reinterpret_cast<const uint2*>(vst + staged<DPH>(t, 2 * db + (q >> 1)) + 8 * (q & 1));
      const float x[4] = {(float)__builtin_bit_cast(_Float16, (uint16_t)(v.x & 0xffffu)),
                          (float)__builtin_bit_cast(_Float16, (uint16_t)(v.x >> 16)),
                          (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y & 0xffffu)),
                          (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y >> 16))};
#pragma unroll
      for (int i = 0; i < 4; i++) o[db][i] = vis ? fmaf(w, x[i], o[db][i]) : o[db][i];
    }
  }
}

// This lane's q operand (row l%16, features 32ks + 8(l/16) + e) from its
// raw fp32 values: rotated by RoPE when rq is given -- the wave first
// writes the (cos, sin) table of its rows' queries (one rope_sincos per lane
// and query for dph 128) to tab, its own LDS, free until its first tile is
// staged; the partner of feature f is f +- dph/2, k-step ks +- KS/2 of the
// same lane -- then scaled into the exp2 domain and split into fp16 hi and
// lo parts, stored to the workgroup's q operand area: hi of k-step ks at
// qop[ks*64 + lane], lo at qop[(KS + ks)*64 + lane].  Every wave of a
// workgroup serves the same rows and stores the same bytes, so a wave reads
// back what it wrote (a wave's LDS operations complete in order) whatever
// the other waves do: no barrier.
template <int DPH>
__device__ __forceinline__ void mfma_pack_q(const float2 (&qr)[MfmaShape<DPH>::KS][4], float sc,
                                            const QRope* rq, int lane, char* tab, h8_t* qop) {
  const int grp = lane >> 4;
  constexpr int KS = MfmaShape<DPH>::KS;
  float x[KS][8];
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int w = 0; w < 4; w++) {
      x[ks][2 * w] = qr[ks][w].x;
      x[ks][2 * w + 1] = qr[ks][w].y;
    }
  if (rq) {
    constexpr int HALF = DPH / 2;
    float2* ct = reinterpret_cast<float2*>(tab);
    // entry t = query (t / HALF), pair t % HALF = lane % HALF (64 is a
    // multiple of HALF)
    for (int t = lane; t < rq->nm * HALF; t += 64) {
      float sn, c;
      rope_sincos(((float)(rq->p0 + t / HALF) / rq->pos_div) * rq->fr, sn, c);
      ct[t] = make_float2(c, sn);
    }
    const float2* cs = ct + rq->mi * HALF;
#pragma unroll
    for (int ks = 0; ks < KS / 2; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float2 k = cs[32 * ks + 8 * grp + e];
        const float a = x[ks][e], b = x[ks + KS / 2][e];
        x[ks][e] = a * k.x - b * k.y;
        x[ks + KS / 2][e] = a * k.y + b * k.x;
      }
  }
#pragma unroll
  for (int ks = 0; ks < KS; ks++) {
#pragma unroll
    for (int e = 0; e < 8; e++) x[ks][e] *= sc;
    h8_t hi, lo;
    split_h8(x[ks], hi, lo);
    qop[ks * 64 + lane] = hi;
    qop[(KS + ks) * 64 + lane] = lo;
  }
}

// Per-wave constants of the MFMA tile loop.
struct MfmaWave {
  const char* head_base;  // this KV head's slice in the pool
  const_table_t table;
  uint32_t lane_off, chunk_off;
  int lane;
  int sl, c, l16, q;      // load role (slot, chunk) and operand role (row, group)
  int last, stride, lim;
  int wmin;               // smallest lim over the wave's real rows
  char* kst;              // staged K tile; the V tile follows
  h8_t* qop;              // the workgroup's packed q operand (mfma_pack_q)
};

// One chunk of a wave's tiles, starting at tile c0, pipelined a tile ahead:
// K of tile i+1 is issued before tile i's logits and V of tile i+1 before
// tile i's output product, so a tile of loads stays in flight while the
// wave computes, and no in-flight register is carried across a loop edge
// (the compiler would copy it, which waits for it).  Chunk slots past the
// wave's last tile re-read that tile (an L2 hit) and are fully masked.
// FIRST: the wave's first chunk, which packs q once its first loads are in
// flight (q was loaded before them, so this waits for no tile data); the
// raw q registers are dead after it.
template <int DPH, int CHUNK, bool FIRST>
__device__ __forceinline__ void mfma_chunk(const TileSource& src, const MfmaWave& w, int c0,
                                           const float2 (&qr)[MfmaShape<DPH>::KS][4], float qsc,
                                           const QRope* rq, float& m_run, float& l_run,
                                           f4_t (&o)[MfmaShape<DPH>::DB], bool balance) {
  constexpr int SL = 512 / DPH, NLD = kTile / SL;
  char* vst = w.kst + MfmaShape<DPH>::TILEB;
  uint4 kbuf[2][NLD], vbuf[2][NLD];
  int blk[2][NLD], slot[2][NLD];
  tile_groups<NLD, SL>(src, w.table, min(c0, w.last) * kTile, blk[0], slot[0]);
  stream_load<DPH>(src, w.head_base, min(c0, w.last) * kTile, w.sl, w.lane_off, w.chunk_off,
                   false, blk[0], slot[0], kbuf[0]);
  stream_load<DPH>(src, w.head_base, min(c0, w.last) * kTile, w.sl, w.lane_off, w.chunk_off,
                   true, blk[0], slot[0], vbuf[0]);
  if (CHUNK > 1)
    tile_groups<NLD, SL>(src, w.table, min(c0 + w.stride, w.last) * kTile, blk[1], slot[1]);
#pragma unroll
  for (int i = 0; i < CHUNK; i++) {
    const int t = c0 + i * w.stride;
    const int b = i & 1, nb = b ^ 1;
    const int tn = min(t + w.stride, w.last);
    if (i + 1 < CHUNK)
      stream_load<DPH>(src, w.head_base, tn * kTile, w.sl, w.lane_off, w.chunk_off, false,
                       blk[nb], slot[nb], kbuf[nb]);
    if (FIRST && i == 0) mfma_pack_q<DPH>(qr, qsc, rq, w.lane, w.kst, w.qop);
    if (balance) {
      if (2 * i < CHUNK) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // A slot past the wave's last tile: every token masked (no-op).
    const int ts_mask = t <= w.last ? t * kTile : INT_MAX / 2;
    stage_tile<DPH>(w.kst, w.sl, w.c, kbuf[b]);
    float p[8];
    mfma_logits<DPH>(ts_mask, w.lane, w.q, w.l16, w.lim, w.qop, w.kst, m_run, l_run, o, p);
    if (i + 1 < CHUNK) {
      stream_load<DPH>(src, w.head_base, tn * kTile, w.sl, w.lane_off, w.chunk_off, true,
                       blk[nb], slot[nb], vbuf[nb]);
      if (i + 2 < CHUNK)
        tile_groups<NLD, SL>(src, w.table, min(t + 2 * w.stride, w.last) * kTile, blk[b],
                             slot[b]);
    }
    // Tiles reaching a position some real row cannot see get the non-finite
    // check (wave-uniform condition: the window's tail and the context end).
    const bool exact = ts_mask + kTile - 1 > w.wmin &&
                       hidden_nonfinite<DPH>(ts_mask, w.sl, w.wmin, vbuf[b]);
    stage_tile<DPH>(vst, w.sl, w.c, vbuf[b]);
    if (exact) {
      masked_pv<DPH>(ts_mask, w.q, w.l16, w.lim, p, w.kst, vst, o);
    } else {
      h8_t ph, pl;
      split_h8(p, ph, pl);
      mfma_pv<DPH>(w.q, w.l16, ph, pl, vst, o);
    }
  }
}

// A wave's tiles first, first+stride, ... < te of KV head kvh on the MFMA
// path.  lim: last visible position of this lane's row (-1: a padding
// row); wmin: the smallest lim over the wave's real rows.  qr, qsc, rq: the
// lane's raw q values, their scale and RoPE (mfma_pack_q); qop: the
// workgroup's q operand area.  st: this wave's LDS (K tile, then V tile).
template <int DPH, int CHUNK>
__device__ __forceinline__ void mfma_attend(const TileSource& src, int lane, int kvh, int first,
                                            int te, int stride, int lim, int wmin,
                                            const float2 (&qr)[MfmaShape<DPH>::KS][4], float qsc,
                                            const QRope* rq, char* st, h8_t* qop, float& m_run,
                                            float& l_run, f4_t (&o)[MfmaShape<DPH>::DB],
                                            bool balance) {
  constexpr int CH = DPH / 8;
  if (first >= te) return;
  MfmaWave w;
  w.lane = lane;
  w.sl = lane / CH;
  w.c = lane % CH;
  w.l16 = lane & 15;
  w.q = lane >> 4;
  w.table = const_table(src);
  w.head_base = reinterpret_cast<const char*>(src.pool) + (size_t)kvh * DPH * 2u;
  w.lane_off = (uint32_t)w.sl * 2u * (uint32_t)src.kv_dim + 16u * w.c;
  w.chunk_off = 16u * w.c;
  w.last = first + ((te - 1 - first) / stride) * stride;
  w.stride = stride;
  w.lim = lim;
  w.wmin = wmin;
  w.kst = st;
  w.qop = qop;
  mfma_chunk<DPH, CHUNK, true>(src, w, first, qr, qsc, rq, m_run, l_run, o, balance);
  for (int c0 = first + CHUNK * stride; c0 < te; c0 += CHUNK * stride)
    mfma_chunk<DPH, CHUNK, false>(src, w, c0, qr, qsc, rq, m_run, l_run, o, balance);
  if (balance) __builtin_amdgcn_s_setprio(0);
}

// LDS of the MFMA tile path: per wave, its staged K and V tiles; once the
// wave's tiles are done the same bytes hold its records (up to 16 rows).
// Then the workgroup's packed q operand (hi and lo parts, 16 rows).
template <int DPH, int WAVES>
struct MfmaLds {
  static constexpr int kRows = 16;
  static_assert(kRows * (DPH + 2) * 4 <= MfmaShape<DPH>::WAVEB, "records fit the staging area");
  static_assert(kRows * kTile * 4 <= MfmaShape<DPH>::TILEB, "probabilities fit a K tile");
  char st[WAVES * MfmaShape<DPH>::WAVEB] __attribute__((aligned(16)));
  h8_t qop[2 * MfmaShape<DPH>::KS * 64];
  int last;
  int extra;
  __device__ char* staging(int w) { return st + w * MfmaShape<DPH>::WAVEB; }
  __device__ float* acc_at(int w, int r) {
    return reinterpret_cast<float*>(staging(w)) + r * DPH;
  }
  __device__ float2& ml_at(int w, int r) {
    return reinterpret_cast<float2*>(staging(w) + kRows * DPH * 4)[r];
  }
};

// The window's K / V rows of KV head kvh from the gathered tables, rounded
// to fp16 (RNE, as kv_cache_append) into the pool by the whole workgroup;
// returns once the stores are visible to the workgroup's loads.
template <int DPH>
__device__ __forceinline__ void gather_append_slice(const AttnArgs& a, const GatherArgs& g,
                                                    int kvh) {
  const int M = a.R / a.G;
  const int kvd = a.src.kv_dim;
  const int bs = a.src.bs;
  for (int t = item_tid(); t < M * DPH; t += blockDim.x) {
    const int m = t / DPH;
    const int d = t - m * DPH;
    const int pos = a.pos_base + m;
    const int lb = pos / bs;
    const int slot = pos - lb * bs;
    const size_t src = (size_t)g.tok[m] * kvd + (size_t)kvh * DPH + d;
    uint16_t* kd = g.pool + ((size_t)(uint32_t)a.src.table[lb] * 2u * bs + slot) * kvd +
                   (size_t)kvh * DPH + d;
    kd[0] = __builtin_bit_cast(uint16_t, (_Float16)g.k_table[src]);
    kd[(size_t)bs * kvd] = __builtin_bit_cast(uint16_t, (_Float16)g.v_table[src]);
  }
  __syncthreads();
}

// Partition `part` of (KV head kvh, row group rg) on the calling workgroup:
// waves 0..nwaves-1 (nwaves <= WAVES) take tiles tb+w, tb+w+nwaves, ...
// (further waves idle), merge their states through LDS, and either write
// the normalised output (one partition) or publish a partial and count the
// arrival; the last arrival combines all partitions (with WAVES waves).
// SPLIT (libsde_paged's kernels, one item per workgroup, arrival counters
// a line apart): a group of more than slice_rows rows is combined in
// slices of up to slice_rows rows, slice s by the workgroup that arrived s
// places before the last -- the last arrival takes slice 0 at once, the
// ones before it wait (bounded) for it -- so several CUs read the partials
// at once (one CU reads them at ~35 GB/s); see slice_arrive.
// Every thread of the workgroup calls it.
// GATHER: the window comes from `ga` (GatherArgs) instead of a.q and
// earlier appends.
template <int DPH, int RPW, int CHUNK, int WAVES, bool ROPE = false, class Lds,
          bool GATHER = false, bool SPLIT = false>
__device__ __forceinline__ void stream_item(const AttnArgs& a, int part, int kvh, int rg,
                                            Lds& lds, int nwaves = WAVES,
                                            const RopeArgs* rp = nullptr,
                                            const GatherArgs* ga = nullptr) {
  static_assert(DPH == 64 || DPH == 128, "head_dim");
  static_assert(RPW == 2 || RPW == 4 || RPW == 8 || RPW == 16, "rows per group");
  using Mh = MfmaShape<DPH>;

  const int tid = item_tid();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r0 = rg * RPW;
  const int nrows = min(RPW, a.R - r0);
  const int n_tiles = (a.src.L_max + kTile - 1) / kTile;
  // (a plan may leave up to one extra tile per wave past its whole
  // partitions, see stream_plan)
  int tb = part * a.tiles_per_part;
  int te = part == a.n_parts - 1 ? n_tiles : min(n_tiles, tb + a.tiles_per_part);
  {
    // The partition holding the window also masks the window's causal tail
    // and, in the fused and gathered steps, appends the window first: the
    // extra tiles go to the first partition instead (measured on MI355X:
    // Qwen2.5-7B fused 9-query window 19.5 -> 18.1 us, a fused 5-query
    // window at 16K 28.7 -> 26.9, its unfused window 29.5 -> 29.1).
    const int rem = n_tiles - a.n_parts * a.tiles_per_part;
    if (rem > 0) {
      tb = part == 0 ? 0 : rem + part * a.tiles_per_part;
      te = rem + (part + 1) * a.tiles_per_part;
    }
  }

  if constexpr (ROPE) {
    // A partition that reads window positions first writes the window's K
    // (rotated) and V slice of this KV head itself, so no other workgroup
    // has to finish first; partitions sharing the window write the same
    // bytes.  (q rotates in mfma_pack_q, behind the first tile loads.)
    if (te * kTile > a.pos_base) rope_append_slice<DPH>(a, *rp, kvh);
  }
  if constexpr (GATHER) {
    // (as above: a partition reading window positions writes them first)
    if (te * kTile > a.pos_base) gather_append_slice<DPH>(a, *ga, kvh);
  }

  if (wave < nwaves) {
    // Lane l serves row r0 + l%16 (rows past nrows are padding: zero q,
    // nothing visible).
    const int l16 = lane & 15, grp = lane >> 4;
    const bool real = l16 < nrows;
    const int gr = min(r0 + l16, a.R - 1);
    const int m = gr / a.G;
    const int h = kvh * a.G + (gr - m * a.G);
    const float* qrow;
    if constexpr (GATHER)
      qrow = ga->q_table + (size_t)ga->tok[m] * a.nh * DPH;
    else
      qrow = a.q + (size_t)m * a.nh * DPH;
    const float2* qp = reinterpret_cast<const float2*>(qrow + (size_t)h * DPH + 8 * grp);
    QRope rq_v;
    if constexpr (ROPE) rq_v.fr = rp->inv_freq[lane % (DPH / 2)];  // (before q: see QRope)
    float2 qr[Mh::KS][4];
#pragma unroll
    for (int ks = 0; ks < Mh::KS; ks++)
#pragma unroll
      for (int w = 0; w < 4; w++) qr[ks][w] = qp[16 * ks + w];
    if constexpr (GATHER) {
      if (ga->q_add) {  // the residual, added in fp32 as the window's q rows are built
        const float2* ap = reinterpret_cast<const float2*>(ga->q_add + (size_t)m * a.nh * DPH +
                                                           (size_t)h * DPH + 8 * grp);
#pragma unroll
        for (int ks = 0; ks < Mh::KS; ks++)
#pragma unroll
          for (int w = 0; w < 4; w++) {
            const float2 r = ap[16 * ks + w];
            qr[ks][w].x += r.x;
            qr[ks][w].y += r.y;
          }
      }
    }
    const QRope* rq = nullptr;
    if constexpr (ROPE) {
      const int m0 = r0 / a.G;
      rq_v.pos_div = rp->pos_div;
      rq_v.p0 = a.pos_base + m0;
      rq_v.nm = (r0 + nrows - 1) / a.G - m0 + 1;
      rq_v.mi = real ? m - m0 : 0;
      rq = &rq_v;
    }
    const int lim = real ? a.pos_base + (r0 + l16) / a.G : -1;
    const int wmin = a.pos_base + r0 / a.G;  // row r0 is the group's first query
    float m_run = -INFINITY, l_run = 0.f;
    f4_t o[Mh::DB];
#pragma unroll
    for (int db = 0; db < Mh::DB; db++) o[db] = f4_t{0.f, 0.f, 0.f, 0.f};
    // Several row groups per KV head: the first half of every chunk's tiles
    // runs at raised wave priority, so a wave past its midpoint yields issue
    // to the other wave of its SIMD that is behind -- for chunks of up to 3
    // tiles, and in the plain kernel for groups of fewer than 16 rows only.
    // Measured on MI355X (two runs each, us): a 5-query window over 16K keys
    // (16-row groups, chunks of 4) 29.0 -> 27.4 without, fused 26.7 -> 25.3;
    // the Qwen2.5-7B window (16-row groups, chunks of 2) 19.6 -> 19.2
    // without, but fused 17.7 with against 18.2 without; the 4K window and
    // TinyLlama (groups of 8 and 2) slower without.
    constexpr bool kBalanceable = CHUNK < 4 && (ROPE || RPW < 16);
    mfma_attend<DPH, CHUNK>(a.src, lane, kvh, tb + wave, te, nwaves, lim, wmin, qr,
                            real ? a.qscale : 0.f, rq, lds.staging(wave), lds.qop, m_run, l_run,
                            o, kBalanceable && a.row_groups > 1);
    const float l_row = groups_sum(l_run);
    // The staged tiles are dead: records go over them (DS operations of a
    // wave complete in order).
    if (real) {
#pragma unroll
      for (int db = 0; db < Mh::DB; db++)
        *reinterpret_cast<f4_t*>(lds.acc_at(wave, l16) + 16 * db + 4 * grp) = o[db];
      if (grp == 0) lds.ml_at(wave, l16) = make_float2(m_run, l_row);
    }
  }
  __syncthreads();

  // ---- workgroup merge: thread (row, feature pair) over the waves --------
  // Every wave's record is read up front (waves past nwaves re-read the
  // last one and weigh nothing), so the LDS reads overlap instead of
  // forming a chain of round trips; the sums run in wave order.
  constexpr int DP = DPH / 2;
  for (int idx = tid; idx < nrows * DP; idx += blockDim.x) {
    const int r = idx / DP;
    const int dcol = 2 * (idx - r * DP);
    float2 ml[WAVES], x[WAVES];
#pragma unroll
    for (int w = 0; w < WAVES; w++) {
      const int ws = min(w, nwaves - 1);
      ml[w] = lds.ml_at(ws, r);
      x[w] = *reinterpret_cast<const float2*>(lds.acc_at(ws, r) + dcol);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; w++)
      if (w < nwaves) mx = fmaxf(mx, ml[w].x);
    float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) {
      const float wt =
          (w >= nwaves || ml[w].x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ml[w].x - mx);
      l += ml[w].y * wt;
      o0 += x[w].x * wt;
      o1 += x[w].y * wt;
    }
    const int gr = r0 + r;
    if (a.n_parts == 1) {
      const float inv = finish_scale(l);
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      *reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH + dcol) =
          make_float2(o0 * inv, o1 * inv);
    } else {
      const size_t pr = ((size_t)kvh * a.R + gr) * a.n_parts + part;
      float* ml_base = a.partials + (size_t)a.nkv * a.R * a.n_parts * DPH;
      store_dev2(a.partials + pr * DPH + dcol, o0, o1);
      if (dcol == 0) store_dev2(ml_base + pr * 2, mx, l);
    }
  }
  if (a.n_parts == 1) return;

  // ---- the last workgroup(s) of (KV head, row group) combine ------------
  // Partials are device-scope stores; waiting for them (vmcnt) before the
  // arrival increment orders them before it (see store_dev2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Slices of a split combine (SPLIT, counters a line apart).
  int n_slices = 1;
  if constexpr (SPLIT)
    if (a.ctr_stride > 1)
      n_slices = min((nrows + slice_rows<RPW>() - 1) / slice_rows<RPW>(), a.n_parts);
  if (tid == 0) {
    uint32_t* ctr = a.counters + ((size_t)kvh * a.row_groups + rg) * a.ctr_stride;
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int slice = -1;  // the slice this workgroup combines (-1: none)
    int extra = 0;   // the last arrival's slices given up by their waits (bit s: slice s)
    if (n_slices == 1) {
      if (prev == (uint32_t)(a.n_parts - 1)) {
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        slice = 0;
      }
    } else {
      slice = slice_arrive(ctr, prev, a.n_parts, n_slices, a.slice_spin, extra);
    }
    lds.last = slice;
    lds.extra = extra;
  }
  __syncthreads();
  const int slice = lds.last;
  if (slice < 0) return;
  if (n_slices == 1) {
    stream_combine<DPH, RPW, WAVES>(a, tid, kvh, r0, nrows);
    return;
  }
  const int rs = (nrows + n_slices - 1) / n_slices;
  const int s0 = slice * rs;
  const int sn = min(rs, nrows - s0);
  if (rs <= kSliceRows)
    stream_combine<DPH, kSliceRows, WAVES>(a, tid, kvh, r0 + s0, sn);
  else
    stream_combine<DPH, RPW, WAVES>(a, tid, kvh, r0 + s0, sn);
  // (the last arrival only, after waits that gave up)
  for (int bits = lds.extra; bits != 0; bits &= bits - 1) {
    const int e0 = __builtin_ctz((unsigned)bits) * rs;
    stream_combine<DPH, RPW, WAVES>(a, tid, kvh, r0 + e0, min(rs, nrows - e0));
  }
}

// Partition sizing shared by libsde_paged and the grid API: at most
// `blocks` workgroups in all (one per CU for the library), as many
// partitions per (KV head, row group) as that allows (up to
// kStreamMaxParts, at least one tile per wave), then the fewest tiles per
// wave that cover the context.  A wave takes its tiles in chunks of `chunk`
// (1 to max_chunk, unrolled at compile time), several chunks when it has
// more than max_chunk tiles; a remainder of at most one tile per wave goes
// to the first partition (stream_item).  (Cutting the context evenly instead, with
// masked slots for the waves past a partition's last tile, measured slower
// on short contexts: the masked slots are not free.)  Rows per group:
// `rows` (2, 4, 8 or 16).
struct StreamPlan {
  int rpw;             // rows per group
  int row_groups;
  int chunk;
  int tiles_per_part;
  int n_parts;
};

__host__ __device__ inline StreamPlan stream_plan(int L_max, int nkv, int R, int blocks,
                                                  int waves, int max_chunk, int rows) {
  // (32-bit divisions: every quotient here is small, and a grid device
  // function's blocks each compute this plan before their first load)
  StreamPlan p;
  p.rpw = rows;
  p.row_groups = (R + p.rpw - 1) / p.rpw;
  const int n_tiles = (L_max + kTile - 1) / kTile;
  const int64_t units = (int64_t)nkv * p.row_groups;
  int parts = units >= blocks ? 1 : blocks / (int)units;
  if (parts > kStreamMaxParts) parts = kStreamMaxParts;
  const int by_len = (n_tiles + waves - 1) / waves;
  if (parts > by_len) parts = by_len;
  const int per_wave = (n_tiles + parts * waves - 1) / (parts * waves);
  // When the tiles exceed a whole number (2 or more) of tiles per wave by
  // at most one per wave (a window's few positions past a round context
  // length), one partition takes the extra tiles instead of every wave
  // taking one more (measured on MI355X: Qwen2.5-7B 9-query window at 8K
  // 21.6 -> 20.7 us, a 5-query window at 16K 34.6 -> 30.5; with one tile
  // per wave the extra tile doubles that partition's work: the grid
  // device function's 4K window took 22.3 us that way against 20.7).
  const int whole = n_tiles / (parts * waves);
  if (per_wave >= 3 && whole >= 2 && whole <= max_chunk &&
      n_tiles - whole * parts * waves <= waves) {
    p.chunk = whole;
    p.tiles_per_part = waves * p.chunk;
    p.n_parts = parts;
    return p;
  }
  p.chunk = per_wave < max_chunk ? (per_wave < 1 ? 1 : per_wave) : max_chunk;
  const int reps = (per_wave + p.chunk - 1) / p.chunk;
  p.tiles_per_part = waves * p.chunk * (reps < 1 ? 1 : reps);
  p.n_parts = (n_tiles + p.tiles_per_part - 1) / p.tiles_per_part;
  return p;
}

// Workgroup -> (partition, KV head, row group) of libsde_paged's kernels,
// whose grid is (n_parts, nkv, row_groups).  Long contexts (waves of four
// tiles or more) take the KV head fastest in the linear workgroup index:
// consecutive workgroups then read the adjacent KV-head slices of the same
// token rows at the same time, which the memory system serves faster than
// the same slices read by workgroups far apart in dispatch order.
template <int CHUNK>
__device__ __forceinline__ int3 stream_coords() {
  if constexpr (CHUNK < 4) {
    return make_int3(blockIdx.x, blockIdx.y, blockIdx.z);
  } else {
    const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    return make_int3((lin / gridDim.y) % gridDim.x, lin % gridDim.y,
                     lin / (gridDim.x * gridDim.y));
  }
}

// Rows per group of the 8-wave kernels (libsde_paged's and the 8-wave grid
// device function; an MFMA tile holds 16; measured on MI355X): up to 8 rows
// (decode) in groups of 4 (2 for up to 2), so a KV head's rows keep twice
// the workgroups pulling K/V; verify windows of up to 48 rows over contexts
// up to 16K in groups of 8, whose repeated K/V reads are cache hits; larger
// windows and longer contexts in groups of 16, the fewest repeated reads.
__host__ __device__ inline int stream_rows(int R, int L_max) {
  if (R <= 2) return 2;
  if (R <= 8) return 4;
  if (R <= 48 && L_max <= 16384) return 8;
  return 16;
}

// The plan of the 8-wave kernels: stream_rows' group size, or twice it (up
// to 16) when that leaves each wave fewer tiles -- a KV head's rows then
// share every tile they read, where the smaller groups' extra workgroups
// would have needed a second tile per wave (measured on MI355X: the
// Qwen2.5-7B draft step, 7 rows per KV head over 8K keys, two 4-row groups
// with two tiles per wave 15.9 us, one 8-row group with one 15.6 us).
__host__ __device__ inline StreamPlan stream_plan8(int L_max, int nkv, int R, int blocks) {
  const int rows = stream_rows(R, L_max);
  StreamPlan p = stream_plan(L_max, nkv, R, blocks, 8, 4, rows);
  if (rows < 16 && R > rows) {
    const StreamPlan w = stream_plan(L_max, nkv, R, blocks, 8, 4, 2 * rows);
    if (w.tiles_per_part < p.tiles_per_part) p = w;
  }
  return p;
}

// libsde_paged's plan (host side): stream_plan8's, then half-size groups
// (down to 2 rows) when each wave keeps its tiles and the grid still fits
// one workgroup per CU: more workgroups pull the same K/V (measured on
// MI355X: TinyLlama's 8 rows per KV head at 2K in groups of 2 instead of 4,
// attention 6.98 -> 6.84 us, fused step 7.36 -> 7.25; groups that would
// take more tiles per wave, such as the Qwen2.5-7B draft step's, measured
// 11.9 -> 13.8 and are not taken).  The grid device function keeps
// stream_plan8: every block computes its plan, and the third candidate's
// registers made its largest item variant spill.
inline StreamPlan stream_plan8_spread(int L_max, int nkv, int R, int blocks) {
  StreamPlan p = stream_plan8(L_max, nkv, R, blocks);
  if (p.rpw >= 4 && R > 2) {
    const StreamPlan h = stream_plan(L_max, nkv, R, blocks, 8, 4, p.rpw / 2);
    if (h.tiles_per_part <= p.tiles_per_part &&
        (int64_t)nkv * h.row_groups * h.n_parts <= blocks)
      p = h;
  }
  return p;
}

// Rows per group of the 4-wave device functions: 4 (decode of up to 4 q
// heads per KV head) or 16 (everything larger) -- the MFMA computes 16 rows
// either way; fewer rows per group give a KV head more workgroups.
__host__ __device__ inline int device_rows(int R) { return R <= 4 ? 4 : 16; }

// Static LDS shared by the device functions of one kernel (a function-scope
// __shared__ array is one allocation per kernel, whichever caller uses
// it): MaxWaves waves' staging at head_dim 128.
template <int MaxWaves>
__device__ __forceinline__ char* device_lds() {
  __shared__ __attribute__((aligned(16))) char buf[sizeof(MfmaLds<128, MaxWaves>)];
  return buf;
}

// The units (KV head, row group) of a call on the calling block alone, the
// whole context per unit (one partition: the output is written directly),
// its tiles spread over `nwaves` waves and merged through LDS.
template <int DPH, int RPW, int MaxWaves>
__device__ __forceinline__ void block_units(const AttnArgs& a, int nwaves) {
  auto& lds = *reinterpret_cast<MfmaLds<DPH, MaxWaves>*>(device_lds<MaxWaves>());
  for (int u = 0; u < a.nkv * a.row_groups; u++) {
    __syncthreads();  // the previous unit's readers of lds are done
    stream_item<DPH, RPW, 2, MaxWaves>(a, 0, u % a.nkv, u / a.nkv, lds, nwaves);
  }
}

// The items (partition, KV head, row group) of a call, taken by the grid's
// blocks in turns, CHUNK tiles per wave in flight; in libsde_paged's
// workgroup order (with four tiles per wave or more the KV head fastest:
// blocks that run together read the adjacent KV-head slices of the same
// token rows).
template <int DPH, int RPW, int CHUNK, int WAVES, int MaxWaves, bool GATHER = false>
__device__ __forceinline__ void grid_items(const AttnArgs& a, const GatherArgs* ga = nullptr) {
  auto& lds = *reinterpret_cast<MfmaLds<DPH, MaxWaves>*>(device_lds<MaxWaves>());
  const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
  const int block = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int items = a.nkv * a.row_groups * a.n_parts;
  for (int it = block; it < items; it += n_blocks) {
    int part, kvh, rg;
    if constexpr (CHUNK >= 4) {
      kvh = it % a.nkv;
      part = (it / a.nkv) % a.n_parts;
      rg = it / (a.nkv * a.n_parts);
    } else {
      part = it % a.n_parts;
      const int unit = it / a.n_parts;
      kvh = unit % a.nkv;
      rg = unit / a.nkv;
    }
    stream_item<DPH, RPW, CHUNK, WAVES, false, MfmaLds<DPH, MaxWaves>, GATHER>(
        a, part, kvh, rg, lds, WAVES, nullptr, ga);
    if (it + n_blocks < items) __syncthreads();  // this item's readers of lds are done
  }
}

// 4-wave blocks: rows per group 4 or 16, two tiles per wave in flight (on
// the MaxWaves-sized staging).
template <int DPH, int MaxWaves, bool GATHER = false>
__device__ __forceinline__ void grid_dispatch4(const AttnArgs& a, int rpw,
                                               const GatherArgs* ga = nullptr) {
  if (rpw == 4)
    grid_items<DPH, 4, 2, 4, MaxWaves, GATHER>(a, ga);
  else
    grid_items<DPH, 16, 2, 4, MaxWaves, GATHER>(a, ga);
}

// 8-wave blocks: stream_plan8, libsde_paged's plans without the host's
// half-size rule (2-16 rows per group,
// 1-4 tiles per wave in flight; a wave with one tile and a chunk of two
// loads and multiplies a second, masked tile: measured on MI355X at the 4K
// decode, 15.3 against 11.8 us with a chunk of one).
template <int DPH, int RPW>
__device__ __forceinline__ void grid_chunks8(const AttnArgs& a, int chunk) {
  switch (chunk) {
    case 1: grid_items<DPH, RPW, 1, 8, 8>(a); break;
    case 2: grid_items<DPH, RPW, 2, 8, 8>(a); break;
    case 3: grid_items<DPH, RPW, 3, 8, 8>(a); break;
    default: grid_items<DPH, RPW, 4, 8, 8>(a); break;
  }
}

template <int DPH>
__device__ __forceinline__ void grid_dispatch8(const AttnArgs& a, int rpw, int chunk) {
  switch (rpw) {
    case 2: grid_chunks8<DPH, 2>(a, chunk); break;
    case 4: grid_chunks8<DPH, 4>(a, chunk); break;
    case 8: grid_chunks8<DPH, 8>(a, chunk); break;
    default: grid_chunks8<DPH, 16>(a, chunk); break;
  }
}

}  // namespace attn

// ---- reference-named device API (block-cooperative) ---------------------

// kv_cache.h:70-72 / kv_cache.cu:70-93: fp32 k, v [kv_dim] -> fp16 (RNE) at
// position `current_seq_len` of `layer`.  Positions outside the layer's
// table are ignored (the reference does not check).
__device__ inline void kv_cache_append(const sde_kv_view& kv, int layer, const float* k,
                                       const float* v, int current_seq_len) {
  const int lb = current_seq_len / kv.block_size;
  if (layer >= 0 && layer < kv.n_layers && current_seq_len >= 0 && lb < kv.max_blocks_per_layer) {
    const int pb = kv.block_tables[(size_t)layer * kv.max_blocks_per_layer + lb];
    uint16_t* kd = kv.pool + ((size_t)pb * 2u * kv.block_size + (current_seq_len - lb * kv.block_size)) *
                                 (size_t)kv.kv_dim;
    uint16_t* vd = kd + (size_t)kv.block_size * kv.kv_dim;
    for (int i = threadIdx.x; i < kv.kv_dim; i += blockDim.x) {
      kd[i] = __builtin_bit_cast(uint16_t, (_Float16)k[i]);
      vd[i] = __builtin_bit_cast(uint16_t, (_Float16)v[i]);
    }
  }
  __syncthreads();
}

// kv_cache.h:74-75 / kv_cache.cu:95-114: K[pos], V[pos] of `layer`, widened
// exactly to fp32 [kv_dim].
__device__ inline void kv_cache_read(const sde_kv_view& kv, int layer, int pos, float* k_out,
                                     float* v_out) {
  const int lb = pos / kv.block_size;
  if (layer >= 0 && layer < kv.n_layers && pos >= 0 && lb < kv.max_blocks_per_layer) {
    const int pb = kv.block_tables[(size_t)layer * kv.max_blocks_per_layer + lb];
    const uint16_t* ks = kv.pool + ((size_t)pb * 2u * kv.block_size + (pos - lb * kv.block_size)) *
                                       (size_t)kv.kv_dim;
    const uint16_t* vs = ks + (size_t)kv.block_size * kv.kv_dim;
    for (int i = threadIdx.x; i < kv.kv_dim; i += blockDim.x) {
      k_out[i] = (float)__builtin_bit_cast(_Float16, ks[i]);
      v_out[i] = (float)__builtin_bit_cast(_Float16, vs[i]);
    }
  }
  __syncthreads();
}

// kv_cache.h:77-79 / kv_cache.cu:116-120: O(1) rewind, seq_len <-
// target_len, written by thread 0 of block 0; the pool keeps its bytes
// (positions >= target_len are overwritten by later appends).
__device__ inline void kv_cache_rollback(const sde_kv_view& kv, int target_len) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *kv.seq_len = target_len;
  __syncthreads();
}

// attention.h:21-127: attention of one query (q_all fp32 [nh*dph], RoPE
// applied; global or shared memory) over positions [0, total_len) of
// `layer`, by the calling block: q head h reads KV head h*nkv/nh, scale
// dph^-1/2; attn_out fp32 [nh*dph] (global or shared) is fully written
// (zeros when total_len is 0), so the caller need not zero it.  The units
// (KV head, up to 16 q heads) run one after another, each spread over
// min(blockDim.x/64, MaxWaves) waves that split its context and merge
// through LDS.  Uses sizeof(attn::MfmaLds<128, MaxWaves>) bytes of static
// LDS (64 KiB for the default 4 waves), shared with the grid function.
// Inlined into the caller; its tile loop needs up to ~240 VGPRs per lane,
// so the calling kernel should be declared __launch_bounds__(512) or
// smaller (two waves per SIMD), else the compiler spills.
// Other head sizes (up to 512) and block sizes run the generic fp32 path
// (sde/attention_generic_device.hpp: up to 256 of the block's threads, its
// LDS inside the same static area).  nkv | nh and blockDim.x a multiple of 64; returns
// SDE_ERR_UNSUPPORTED (writing nothing) otherwise, or for head_dim > 512.
template <int MaxWaves = 4>
__device__ __forceinline__ int device_flash_attention_gqa(const float* q_all, float* attn_out,
                                                          const sde_kv_view& kv, int layer, int nh,
                                                          int nkv, int dph, int total_len) {
  using namespace attn;
  static_assert(MaxWaves == 1 || MaxWaves == 2 || MaxWaves == 4 || MaxWaves == 8, "waves");
  if (nkv < 1 || nh % nkv != 0 || total_len < 0 || dph < 1 || dph > gen::kMaxDph ||
      blockDim.x % 64 != 0)
    return SDE_ERR_UNSUPPORTED;
  if (gen::needs_generic(dph, kv.block_size)) {
    if (total_len == 0) {
      for (int i = threadIdx.x; i < nh * dph; i += blockDim.x) attn_out[i] = 0.f;
      __syncthreads();
      return SDE_OK;
    }
    gen::GenArgs g;
    g.pool = kv.pool;
    g.table = kv.block_tables + (size_t)layer * kv.max_blocks_per_layer;
    g.q = q_all;
    g.out = attn_out;
    g.partials = nullptr;
    g.kv_dim = kv.kv_dim;
    g.bs = kv.block_size;
    g.nh = nh;
    g.nkv = nkv;
    g.dph = dph;
    g.G = nh / nkv;
    g.R = g.G;
    g.pos_base = total_len - 1;  // one query seeing [0, total_len)
    g.L_max = total_len;
    g.n_parts = 1;
    g.part_len = total_len;
    g.qscale = (float)(kLog2e / __builtin_sqrt((double)dph));
    static_assert(sizeof(gen::GenLds) <= sizeof(MfmaLds<128, MaxWaves>), "generic LDS fits");
    auto& lds = *reinterpret_cast<gen::GenLds*>(device_lds<MaxWaves>());
    const int nt = gen::gen_threads(blockDim.x);
    if (nt == 256)
      gen::gen_block_units<256>(g, lds);
    else if (nt == 128)
      gen::gen_block_units<128>(g, lds);
    else
      gen::gen_block_units<64>(g, lds);
    return SDE_OK;
  }
  const int G = nh / nkv;
  const int rows = device_rows(G);
  AttnArgs a;
  a.src = TileSource{kv.pool, kv.block_tables + (size_t)layer * kv.max_blocks_per_layer,
                     kv.kv_dim, kv.block_size, total_len};
  a.q = q_all;
  a.out = attn_out;
  a.partials = nullptr;
  a.counters = nullptr;
  a.nh = nh;
  a.nkv = nkv;
  a.G = G;
  a.R = G;
  a.row_groups = (G + rows - 1) / rows;
  a.pos_base = total_len - 1;  // one query seeing [0, total_len)
  a.n_parts = 1;
  a.tiles_per_part = (total_len + kTile - 1) / kTile;
  a.qscale = (float)(kLog2e / __builtin_sqrt((double)dph));
  const int nw = min((int)(blockDim.x >> 6), MaxWaves);
  if (total_len == 0) {
    for (int i = threadIdx.x; i < nh * dph; i += blockDim.x) attn_out[i] = 0.f;
  } else if (dph == 128) {
    rows == 4 ? block_units<128, 4, MaxWaves>(a, nw) : block_units<128, 16, MaxWaves>(a, nw);
  } else {
    rows == 4 ? block_units<64, 4, MaxWaves>(a, nw) : block_units<64, 16, MaxWaves>(a, nw);
  }
  __syncthreads();
  return SDE_OK;
}

// attention.h:21-29 with the reference's full argument list: blk_logits
// (KV_BLOCK_SIZE floats of the caller's shared scratch) and the five shared
// scalars are accepted for call-site compatibility and left untouched (this
// function keeps its state in registers and its own LDS).
template <int MaxWaves = 4>
__device__ __forceinline__ int device_flash_attention_gqa(const float* q_all, float* attn_out,
                                                          const sde_kv_view& kv, int layer, int nh,
                                                          int nkv, int dph, int total_len,
                                                          float* blk_logits, float& s_m, float& s_l,
                                                          float& s_tm, float& s_alpha,
                                                          float& s_inv) {
  (void)blk_logits;
  (void)s_m;
  (void)s_l;
  (void)s_tm;
  (void)s_alpha;
  (void)s_inv;
  return device_flash_attention_gqa<MaxWaves>(q_all, attn_out, kv, layer, nh, nkv, dph,
                                              total_len);
}

// attention.h:140-164: SDE_ATTN_SOFTMAX runs device_flash_attention_gqa; the
// types the reference reserves (and traps on) return SDE_ERR_UNSUPPORTED.
// attn_type takes the reference's AttentionType enum (config.h:51-56) or an
// sde_attention_type.
template <int MaxWaves = 4>
__device__ __forceinline__ int device_attention_dispatch(int attn_type, const float* q_all,
                                                         float* attn_out, const sde_kv_view& kv,
                                                         int layer, int nh, int nkv, int dph,
                                                         int total_len) {
  if (attn_type != SDE_ATTN_SOFTMAX) return SDE_ERR_UNSUPPORTED;
  return device_flash_attention_gqa<MaxWaves>(q_all, attn_out, kv, layer, nh, nkv, dph,
                                              total_len);
}

// attention.h:140-150 with the reference's full argument list.
template <int MaxWaves = 4>
__device__ __forceinline__ int device_attention_dispatch(int attn_type, const float* q_all,
                                                         float* attn_out, const sde_kv_view& kv,
                                                         int layer, int nh, int nkv, int dph,
                                                         int total_len, float* blk_logits,
                                                         float& s_m, float& s_l, float& s_tm,
                                                         float& s_alpha, float& s_inv) {
  if (attn_type != SDE_ATTN_SOFTMAX) return SDE_ERR_UNSUPPORTED;
  return device_flash_attention_gqa<MaxWaves>(q_all, attn_out, kv, layer, nh, nkv, dph,
                                              total_len, blk_logits, s_m, s_l, s_tm, s_alpha,
                                              s_inv);
}

// ---- grid-cooperative split-context attention (persistent kernels) -------

// The view with every field read into scalar registers (see wave_uniform).
__device__ __forceinline__ sde_kv_view uniform_view(const sde_kv_view& v) {
  sde_kv_view u;
  u.pool = wave_uniform(v.pool);
  u.block_tables = wave_uniform(v.block_tables);
  u.seq_len = wave_uniform(v.seq_len);
  u.n_layers = wave_uniform(v.n_layers);
  u.kv_dim = wave_uniform(v.kv_dim);
  u.block_size = wave_uniform(v.block_size);
  u.max_blocks_per_layer = wave_uniform(v.max_blocks_per_layer);
  u.pool_blocks = wave_uniform(v.pool_blocks);
  u.reserved = wave_uniform(v.reserved);
  return u;
}

// Arrival counters at the head of the grid function's workspace: a fixed
// area, so calls of different shapes sharing one workspace never find
// partial data where another shape keeps its counters.
constexpr int kGridCounters = 4096;
constexpr size_t kGridCounterBytes = kGridCounters * sizeof(uint32_t);

// Bytes of the workspace of device_flash_attention_gqa_grid for windows of
// up to n_queries queries over up to max_total_len positions: the arrival
// counters (zero-fill them once before the first call; each call leaves
// them zero) followed by the partials of at most kStreamMaxParts
// partitions.
__host__ __device__ inline size_t grid_attention_workspace_size(int nh, int nkv, int dph,
                                                                int n_queries, int max_total_len) {
  if (nh < 1 || nkv < 1 || nh % nkv != 0 || dph < 1 || n_queries < 1 || max_total_len < 1)
    return 0;
  const int R = n_queries * (nh / nkv);
  const int n_tiles = (max_total_len + attn::kTile - 1) / attn::kTile;
  const int by_len = (n_tiles + 3) / 4;  // 4-wave workgroups hold at least 4 tiles
  const int parts = by_len < attn::kStreamMaxParts ? by_len : attn::kStreamMaxParts;
  return kGridCounterBytes + (size_t)nkv * R * parts * (size_t)(dph + 2) * sizeof(float);
}

// Grid-cooperative form of cublas_attention_kernel (kernels.cu:904-940) for
// persistent (megakernel) decode loops, where the reference runs
// device_flash_attention_gqa on block 0 alone (kernels.cu:2727-2739): every
// block of the caller's grid (any size; blockDim.x >= 256, a multiple of 64)
// calls it with the same arguments.  q_all fp32 [n_queries][nh*dph]; query m
// attends causally to positions [0, pos_base+m] of `layer`; attn_out fp32
// [n_queries][nh*dph].  The context is split into partitions, one per block
// and (KV head, row group) -- the same kernel body as sde_paged_attention --
// and the last block to finish a (KV head, row group) combines its
// partitions, so the call has no grid barrier inside; the output is complete
// once every block has returned (the caller's next grid barrier).  Two calls
// that share a workspace need a grid barrier between them.  `workspace`
// (device memory of grid_attention_workspace_size(...) bytes or more)
// starts with arrival counters that must be zero before the first call.
// Blocks run 8 waves when MaxWaves is 8 and blockDim.x >= 512, else 4;
// static LDS sizeof(attn::MfmaLds<128, MaxWaves>) (64 KiB by default),
// shared with device_flash_attention_gqa.  Like it, the caller's kernel
// should be declared __launch_bounds__(512) or smaller.  Head sizes other
// than 64 / 128 (up to 512) and block sizes that are not multiples of 8 run
// the generic fp32 path on 256 threads of each block, with the same
// workspace layout (items taken in turns, the last block of a (KV head,
// group of 8 rows) merging its partitions).  Returns the same status in
// every thread: SDE_OK, SDE_ERR_UNSUPPORTED (dph above 512, blockDim.x <
// 256, more than kGridCounters (KV head, row group) pairs),
// SDE_ERR_INVALID_ARGUMENT, SDE_ERR_CAPACITY (window past the layer's
// table) or SDE_ERR_WORKSPACE; nothing is written on error.
template <int MaxWaves = 4>
__device__ __forceinline__ int device_flash_attention_gqa_grid(const float* q_all,
                                                               float* attn_out,
                                                               const sde_kv_view& kv_in, int layer,
                                                               int nh, int nkv, int dph,
                                                               int pos_base, int n_queries,
                                                               void* workspace,
                                                               size_t workspace_bytes) {
  using namespace attn;
  static_assert(MaxWaves == 4 || MaxWaves == 8, "grid workgroups of 4 or 8 waves");
  // The arguments are the same in every thread: in scalar registers also
  // where the caller is a function of its own.
  q_all = wave_uniform(q_all);
  attn_out = wave_uniform(attn_out);
  workspace = wave_uniform(workspace);
  workspace_bytes = wave_uniform(workspace_bytes);
  layer = wave_uniform(layer);
  nh = wave_uniform(nh);
  nkv = wave_uniform(nkv);
  dph = wave_uniform(dph);
  pos_base = wave_uniform(pos_base);
  n_queries = wave_uniform(n_queries);
  const sde_kv_view kv = uniform_view(kv_in);
  if (blockDim.x < 256 || blockDim.x % 64 != 0) return SDE_ERR_UNSUPPORTED;
  if (dph < 1 || dph > gen::kMaxDph) return SDE_ERR_UNSUPPORTED;
  if (nh < 1 || nkv < 1 || nh % nkv != 0 || nkv * dph != kv.kv_dim || layer < 0 ||
      layer >= kv.n_layers || pos_base < 0 || n_queries < 1 || !q_all || !attn_out || !workspace)
    return SDE_ERR_INVALID_ARGUMENT;
  const int L_max = pos_base + n_queries;
  if ((int64_t)L_max > (int64_t)kv.max_blocks_per_layer * kv.block_size) return SDE_ERR_CAPACITY;
  if (workspace_bytes < grid_attention_workspace_size(nh, nkv, dph, n_queries, L_max))
    return SDE_ERR_WORKSPACE;
  if (gen::needs_generic(dph, kv.block_size)) {
    gen::GenArgs g;
    g.pool = kv.pool;
    g.table = kv.block_tables + (size_t)layer * kv.max_blocks_per_layer;
    g.q = q_all;
    g.out = attn_out;
    g.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kGridCounterBytes);
    g.kv_dim = kv.kv_dim;
    g.bs = kv.block_size;
    g.nh = nh;
    g.nkv = nkv;
    g.dph = dph;
    g.G = nh / nkv;
    g.R = n_queries * g.G;
    g.pos_base = pos_base;
    g.L_max = L_max;
    // Partitions of 256 tokens or more, about one item per block, no more
    // than the workspace holds (its bound: a partition per 4 tiles, at most
    // kStreamMaxParts).
    const int rgs = (g.R + gen::kGenRows - 1) / gen::kGenRows;
    if ((int64_t)nkv * rgs > kGridCounters) return SDE_ERR_UNSUPPORTED;
    const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
    int parts = n_blocks / (nkv * rgs);
    const int by_len = (L_max + gen::kGenChunk - 1) / gen::kGenChunk;
    if (parts > by_len) parts = by_len;
    if (parts > attn::kStreamMaxParts) parts = attn::kStreamMaxParts;
    if (parts < 1) parts = 1;
    g.part_len = (L_max + parts - 1) / parts;
    g.n_parts = (L_max + g.part_len - 1) / g.part_len;
    g.qscale = (float)(attn::kLog2e / __builtin_sqrt((double)dph));
    static_assert(sizeof(gen::GenLds) <= sizeof(MfmaLds<128, MaxWaves>), "generic LDS fits");
    gen::gen_grid_items<256>(g, static_cast<uint32_t*>(workspace),
                             *reinterpret_cast<gen::GenLds*>(device_lds<MaxWaves>()));
    return SDE_OK;
  }

  const int waves = (MaxWaves == 8 && blockDim.x >= 512) ? 8 : 4;
  const int G = nh / nkv;
  const int R = n_queries * G;
  const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
  const StreamPlan p = waves == 8
                           ? stream_plan8(L_max, nkv, R, n_blocks)
                           : stream_plan(L_max, nkv, R, n_blocks, 4, 2, device_rows(R));
  if ((int64_t)nkv * p.row_groups > kGridCounters) return SDE_ERR_UNSUPPORTED;
  AttnArgs a;
  a.src = TileSource{kv.pool, kv.block_tables + (size_t)layer * kv.max_blocks_per_layer,
                     kv.kv_dim, kv.block_size, L_max};
  a.q = q_all;
  a.out = attn_out;
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kGridCounterBytes);
  a.nh = nh;
  a.nkv = nkv;
  a.G = G;
  a.R = R;
  a.row_groups = p.row_groups;
  a.pos_base = pos_base;
  a.n_parts = p.n_parts;
  a.tiles_per_part = p.tiles_per_part;
  a.qscale = (float)(kLog2e / __builtin_sqrt((double)dph));

  if constexpr (MaxWaves == 8) {
    if (waves == 8) {
      if (dph == 128)
        attn::grid_dispatch8<128>(a, p.rpw, p.chunk);
      else
        attn::grid_dispatch8<64>(a, p.rpw, p.chunk);
      __syncthreads();
      return SDE_OK;
    }
  }
  if (dph == 128)
    attn::grid_dispatch4<128, MaxWaves>(a, p.rpw);
  else
    attn::grid_dispatch4<64, MaxWaves>(a, p.rpw);
  __syncthreads();
  return SDE_OK;
}

// device_flash_attention_gqa_grid's 4-wave tile path over a gathered window
// (attn::GatherArgs: a persistent loop whose model builds q rows and K / V
// rows from per-token tables): no q buffer and no append phase, so the loop
// needs no grid barrier between building the window and attending to it.
// The same plans, workspace and results (bit for bit: the same q sums and
// fp16 roundings) as building q, appending and calling
// device_flash_attention_gqa_grid<4>.  Head sizes 64 / 128 with block sizes
// that are multiples of 8 only (SDE_ERR_UNSUPPORTED otherwise: the caller
// keeps the separate phases for the generic path); other errors as the grid
// function's.
__device__ __forceinline__ int device_attention_grid_gathered(const attn::GatherArgs& g_in,
                                                              float* attn_out,
                                                              const sde_kv_view& kv_in, int layer,
                                                              int nh, int nkv, int dph,
                                                              int pos_base, int n_queries,
                                                              void* workspace,
                                                              size_t workspace_bytes) {
  using namespace attn;
  GatherArgs g;
  g.tok = wave_uniform(g_in.tok);
  g.q_table = wave_uniform(g_in.q_table);
  g.q_add = wave_uniform(g_in.q_add);
  g.k_table = wave_uniform(g_in.k_table);
  g.v_table = wave_uniform(g_in.v_table);
  g.pool = wave_uniform(g_in.pool);
  attn_out = wave_uniform(attn_out);
  workspace = wave_uniform(workspace);
  workspace_bytes = wave_uniform(workspace_bytes);
  layer = wave_uniform(layer);
  nh = wave_uniform(nh);
  nkv = wave_uniform(nkv);
  dph = wave_uniform(dph);
  pos_base = wave_uniform(pos_base);
  n_queries = wave_uniform(n_queries);
  const sde_kv_view kv = uniform_view(kv_in);
  if (blockDim.x < 256 || blockDim.x % 64 != 0 || gen::needs_generic(dph, kv.block_size))
    return SDE_ERR_UNSUPPORTED;
  if (nh < 1 || nkv < 1 || nh % nkv != 0 || nkv * dph != kv.kv_dim || layer < 0 ||
      layer >= kv.n_layers || pos_base < 0 || n_queries < 1 || !g.tok || !g.q_table ||
      !g.k_table || !g.v_table || !g.pool || !attn_out || !workspace)
    return SDE_ERR_INVALID_ARGUMENT;
  const int L_max = pos_base + n_queries;
  if ((int64_t)L_max > (int64_t)kv.max_blocks_per_layer * kv.block_size) return SDE_ERR_CAPACITY;
  if (workspace_bytes < grid_attention_workspace_size(nh, nkv, dph, n_queries, L_max))
    return SDE_ERR_WORKSPACE;
  const int G = nh / nkv;
  const int R = n_queries * G;
  const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
  const StreamPlan p = stream_plan(L_max, nkv, R, n_blocks, 4, 2, device_rows(R));
  if ((int64_t)nkv * p.row_groups > kGridCounters) return SDE_ERR_UNSUPPORTED;
  AttnArgs a;
  a.src = TileSource{kv.pool, kv.block_tables + (size_t)layer * kv.max_blocks_per_layer,
                     kv.kv_dim, kv.block_size, L_max};
  a.q = nullptr;
  a.out = attn_out;
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kGridCounterBytes);
  a.nh = nh;
  a.nkv = nkv;
  a.G = G;
  a.R = R;
  a.row_groups = p.row_groups;
  a.pos_base = pos_base;
  a.n_parts = p.n_parts;
  a.tiles_per_part = p.tiles_per_part;
  a.qscale = (float)(kLog2e / __builtin_sqrt((double)dph));
  if (dph == 128)
    attn::grid_dispatch4<128, 4, true>(a, p.rpw, &g);
  else
    attn::grid_dispatch4<64, 4, true>(a, p.rpw, &g);
  __syncthreads();
  return SDE_OK;
}

}  // namespace sde
