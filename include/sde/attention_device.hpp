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
 * and table layout is the reference's (kv_cache.h:5-18).
 *
 * The functions in namespace sde are block-cooperative like the reference's:
 * every thread of the calling block calls them with the same arguments
 * (blockDim.x a multiple of 64).  They need no caller scratch.  Building
 * blocks of the streaming attention live in namespace sde::attn.
 */
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "sde_paged_kv.h"

namespace sde {
namespace attn {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kTile = 32;          // tokens per tile
constexpr int kStreamMaxRows = 4;  // rows (query, q head) per wave
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

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                __builtin_bit_cast(half2_t, b), c, false);
}

// dot2(a, b, 0) as one VOP3P instruction with an inline-constant addend (the
// builtin with a 0 addend becomes a register move plus the accumulating
// VOP2 form).
__device__ __forceinline__ float dot2_0(uint32_t a, uint32_t b) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Cross-lane moves (gfx950 lane semantics):
//  * DPP quad_perm [1,0,3,2] / [2,3,0,1] exchange lanes i^1 / i^2, and
//    row_ror:4 / row_ror:8 rotate each 16-lane row, so four steps reduce
//    every row of 16 lanes;
//  * v_permlane16_swap(x, x) returns rows {0,0,2,2} and {1,1,3,3}: one more
//    step reduces each 32-lane half without mixing the halves;
//  * v_permlane32_swap(a, b) returns [a.lo | b.lo] and [a.hi | b.hi], so
//    their sum holds a's half-sum in lanes 0-31 and b's in lanes 32-63.
__device__ __forceinline__ float dpp_f(float x, int ctrl_sel) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  switch (ctrl_sel) {
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true); break;   // i^1
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true); break;   // i^2
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, true); break;  // ror 4
    case 3: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, true); break;  // ror 8
    default: r = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, true); break; // i^7 in 8
  }
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


typedef const __attribute__((address_space(4))) int32_t* const_table_t;

// The block table is read-only during the kernel: reading it through the
// constant address space turns the entries into scalar loads (lgkmcnt),
// which never wait behind outstanding tile loads (vmcnt).
__device__ __forceinline__ const_table_t const_table(const TileSource& a) {
  return (const_table_t)a.table;
}

__device__ __forceinline__ uint32_t pack_h2(float x, float y) {
  const half2_t h = {(_Float16)x, (_Float16)y};
  return __builtin_bit_cast(uint32_t, h);
}

// All-reduce over the token slots (lanes with the same chunk c).
template <int DPH>
__device__ __forceinline__ float slot_sum(float x) {
  if constexpr (DPH == 64) x += dpp_f(x, 3);  // slots 2k, 2k+1 share a 16-lane row
  const float2 p = row_pair(x);
  x = p.x + p.y;
  return half_pair_total(x, x);
}

template <int DPH>
__device__ __forceinline__ float slot_max(float x) {
  if constexpr (DPH == 64) x = fmaxf(x, dpp_f(x, 3));
  const float2 p = row_pair(x);
  x = fmaxf(p.x, p.y);
  const auto q = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x),
                                                  __builtin_bit_cast(int, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (int)q[0]), __builtin_bit_cast(float, (int)q[1]));
}

__device__ __forceinline__ uint4 ld16(const char* p) { return *reinterpret_cast<const uint4*>(p); }

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

// Marks the point where a tile's registers are first consumed: the empty
// asm redefines them, so no use of the tile (and hence no wait for its
// loads) is hoisted above this point into the previous tile's work.  SITE
// makes the asm text differ per call site, so identical pins at the heads of
// two branches are not merged and hoisted into their common predecessor.
template <int NLD, int SITE>
__device__ __forceinline__ void pin_arrival(const uint4 (&x)[NLD]) {
  uint4(&y)[NLD] = const_cast<uint4(&)[NLD]>(x);
#pragma unroll
  for (int j = 0; j < NLD; j++) {
    if constexpr (SITE == 0) asm volatile("; tile 0" : "+v"(y[j].x), "+v"(y[j].y), "+v"(y[j].z), "+v"(y[j].w));
    else if constexpr (SITE == 1) asm volatile("; tile 1" : "+v"(y[j].x), "+v"(y[j].y), "+v"(y[j].z), "+v"(y[j].w));
    else if constexpr (SITE == 2) asm volatile("; tile 2" : "+v"(y[j].x), "+v"(y[j].y), "+v"(y[j].z), "+v"(y[j].w));
    else asm volatile("; tile 3" : "+v"(y[j].x), "+v"(y[j].y), "+v"(y[j].z), "+v"(y[j].w));
  }
}

// Lane roles of the streaming attention.  Load role: lane = (slot sl, chunk c),
// c = lane % CH.  After the transposing reduction of the logits a lane owns
// one (row r, token pair jp) of its slot: the NV = RPW*NLD partial logits of
// a lane are halved once per butterfly step (the lane keeps the half named
// by one bit of c and adds its partner's copy of that half), so after
// log2(NV)-1 steps a lane holds the full logits of tokens 2jp and 2jp+1 of
// row r, and the softmax does per-lane scalar work.
template <int DPH, int RPW>
struct StreamShape {
  static constexpr int CH = DPH / 8;                  // lanes per token
  static constexpr int S = CH == 16 ? 4 : 3;          // butterfly steps over CH lanes
  static constexpr int SL = 64 / CH;                  // slots
  static constexpr int NLD = kTile / SL;              // loads per tile (K and V each)
  static constexpr int NV = RPW * NLD;                // partial logits per lane
  static constexpr int T = (NV == 32 ? 5 : NV == 16 ? 4 : NV == 8 ? 3 : 2) - 1;  // halving steps
  static constexpr int RB = RPW == 4 ? 2 : 1;         // bits of r
  static constexpr int SF = CH == 16 ? RB : 1;        // select-free butterfly steps
  static_assert(T <= S, "more logits than lanes to spread them over");
  // chunk index of the lane owning (row r, pair jp) (its redundant bits 0)
  static constexpr int owner(int r, int jp) { return ((r << (T - RB)) | jp) << (S - T); }
};

// Butterfly step k over the CH lanes of a token: partner lane = c ^ mask,
// masks {8, 7, 2, 1} (dph 128) or {7, 2, 1} (dph 64) -- row_ror:8,
// row_half_mirror, quad_perm [2,3,0,1], quad_perm [1,0,3,2]; step k splits on
// bit S-1-k of c, which the later masks leave unchanged.
template <int CH>
__device__ __forceinline__ float bfly(float x, int k) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  switch (CH == 16 ? k : k + 1) {
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, true); break;
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, true); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true); break;
    default: r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true); break;
  }
  return __builtin_bit_cast(float, r);
}

// Value of lane n of this lane's 16-lane row (DPP row_newbcast:n).
__device__ __forceinline__ int row_bcast(int v, int n) {
  switch (n) {
    case 0: return __builtin_amdgcn_update_dpp(0, v, 0x150, 0xf, 0xf, true);
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0x151, 0xf, 0xf, true);
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x152, 0xf, 0xf, true);
    case 3: return __builtin_amdgcn_update_dpp(0, v, 0x153, 0xf, 0xf, true);
    case 4: return __builtin_amdgcn_update_dpp(0, v, 0x154, 0xf, 0xf, true);
    case 5: return __builtin_amdgcn_update_dpp(0, v, 0x155, 0xf, 0xf, true);
    case 6: return __builtin_amdgcn_update_dpp(0, v, 0x156, 0xf, 0xf, true);
    case 7: return __builtin_amdgcn_update_dpp(0, v, 0x157, 0xf, 0xf, true);
    case 8: return __builtin_amdgcn_update_dpp(0, v, 0x158, 0xf, 0xf, true);
    case 9: return __builtin_amdgcn_update_dpp(0, v, 0x159, 0xf, 0xf, true);
    case 10: return __builtin_amdgcn_update_dpp(0, v, 0x15A, 0xf, 0xf, true);
    case 11: return __builtin_amdgcn_update_dpp(0, v, 0x15B, 0xf, 0xf, true);
    case 12: return __builtin_amdgcn_update_dpp(0, v, 0x15C, 0xf, 0xf, true);
    case 13: return __builtin_amdgcn_update_dpp(0, v, 0x15D, 0xf, 0xf, true);
    case 14: return __builtin_amdgcn_update_dpp(0, v, 0x15E, 0xf, 0xf, true);
    default: return __builtin_amdgcn_update_dpp(0, v, 0x15F, 0xf, 0xf, true);
  }
}

// Value held by the owner of (row r, pair jp) in this lane's slot.  With
// dph 64 a 16-lane row holds two slots (lane bit 3 = odd slot).
template <int DPH, int RPW>
__device__ __forceinline__ uint32_t from_owner(uint32_t x, int r, int jp, bool odd_slot) {
  using Sh = StreamShape<DPH, RPW>;
  const int n = Sh::owner(r, jp);
  const int v = (int)x;
  if constexpr (DPH == 128) {
    return (uint32_t)row_bcast(v, n);
  } else {
    const int lo = row_bcast(v, n);
    const int hi = row_bcast(v, n + 8);
    return (uint32_t)(odd_slot ? hi : lo);
  }
}

template <int DPH, int RPW>
__device__ __forceinline__ float from_owner_f(float x, int r, int jp, bool odd_slot) {
  return __builtin_bit_cast(
      float, from_owner<DPH, RPW>(__builtin_bit_cast(uint32_t, x), r, jp, odd_slot));
}

// Logits of one tile (transposing reduction) and the online-softmax update
// of the lane's (row, pair): m_run / l_run are the lane's (row, slot) state
// (l_run a partial sum over the lane's token pairs).  Returns the rescale
// factor in al_out and the pair's probabilities as fp16x2 in pk_out.
template <int DPH, int RPW, int SITE>
__device__ __forceinline__ void stream_qk(int ts, int sl, int c, int min_lim, int my_lim,
                                          int my_jp, const uint4 (&qr)[RPW],
                                          const uint4 (&k)[kTile / (512 / DPH)], float& m_run,
                                          float& l_run, float& al_out, uint32_t& pk_out) {
  using Sh = StreamShape<DPH, RPW>;
  constexpr int CH = Sh::CH, S = Sh::S, SL = Sh::SL, NLD = Sh::NLD, NV = Sh::NV, T = Sh::T;
  pin_arrival<NLD, SITE>(k);
  float x[NV];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint4 q4 = qr[r];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
      float t = dot2_0(q4.x, k[j].x);
      t = dot2(q4.y, k[j].y, t);
      t = dot2(q4.z, k[j].z, t);
      t = dot2(q4.w, k[j].w, t);
      x[r * NLD + j] = t;
    }
  }
  // Transposing butterfly: step kk keeps the half of x whose top index bit
  // equals bit S-1-kk of c.  The first SF steps split on row bits, and the
  // lane's q rows arrive permuted by those same lane bits (qr[r] holds row
  // r ^ flip, see q_row_flip), so the half to keep is always the lower one
  // there -- no per-element select.
#pragma unroll
  for (int kk = 0; kk < T; kk++) {
    const bool f = (c >> (S - 1 - kk)) & 1;
    const int h = NV >> (kk + 1);
#pragma unroll
    for (int i = 0; i < (NV >> 1); i++) {
      if (i < h) {
        if (kk < Sh::SF) {
          x[i] += bfly<CH>(x[i + h], kk);
        } else {
          const float a = x[i], b = x[i + h];
          const float send = f ? a : b;
          const float keep = f ? b : a;
          x[i] = keep + bfly<CH>(send, kk);
        }
      }
    }
  }
#pragma unroll
  for (int kk = T; kk < S; kk++) {
    x[0] += bfly<CH>(x[0], kk);
    x[1] += bfly<CH>(x[1], kk);
  }
  float s0 = x[0], s1 = x[1];
  // Causal / length mask: token g is visible to the lane's row iff g <= my_lim.
  if (ts + kTile - 1 > min_lim) {
    const int g0 = ts + 2 * my_jp * SL + sl;
    if (g0 > my_lim) s0 = -INFINITY;
    if (g0 + SL > my_lim) s1 = -INFINITY;
  }
  float tmax = fmaxf(s0, s1);
#pragma unroll
  for (int kk = Sh::RB; kk < S; kk++) tmax = fmaxf(tmax, bfly<CH>(tmax, kk));
  const float m_new = fmaxf(m_run, tmax);
  // Nothing visible yet: base 0 makes every weight exp2(-inf) = 0.
  const float base = m_new == -INFINITY ? 0.f : m_new;
  const float al = __builtin_amdgcn_exp2f(m_run - base);
  const float p0 = __builtin_amdgcn_exp2f(s0 - base);
  const float p1 = __builtin_amdgcn_exp2f(s1 - base);
  l_run = l_run * al + (p0 + p1);
  m_run = m_new;
  al_out = al;
  pk_out = pack_h2(p0, p1);
  // Finish this tile's logits here, in program order (see pin_arrival).
  asm volatile("" : "+v"(m_run), "+v"(l_run), "+v"(al_out), "+v"(pk_out));
}

// P.V of one tile: rescales acc by each row's factor and accumulates the
// probability pairs (from their owners) against the byte-permuted V pairs.
template <int DPH, int RPW, int SITE>
__device__ __forceinline__ void stream_pv(int sl, float al, uint32_t pk,
                                          const uint4 (&v)[kTile / (512 / DPH)],
                                          float (&acc)[RPW][8]) {
  constexpr int NLD = StreamShape<DPH, RPW>::NLD;
  pin_arrival<NLD, SITE>(v);
  const bool odd_slot = sl & 1;
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const float a_r = from_owner_f<DPH, RPW>(al, r, 0, odd_slot);
#pragma unroll
    for (int e = 0; e < 8; e++) acc[r][e] *= a_r;
  }
#pragma unroll
  for (int jp = 0; jp < NLD / 2; jp++) {
    uint32_t pp[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) pp[r] = from_owner<DPH, RPW>(pk, r, jp, odd_slot);
    const uint32_t v0[4] = {v[2 * jp].x, v[2 * jp].y, v[2 * jp].z, v[2 * jp].w};
    const uint32_t v1[4] = {v[2 * jp + 1].x, v[2 * jp + 1].y, v[2 * jp + 1].z, v[2 * jp + 1].w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const uint32_t lo = __builtin_amdgcn_perm(v1[w], v0[w], 0x05040100u);
      const uint32_t hi = __builtin_amdgcn_perm(v1[w], v0[w], 0x07060302u);
#pragma unroll
      for (int r = 0; r < RPW; r++) {
        acc[r][2 * w] = dot2(pp[r], lo, acc[r][2 * w]);
        acc[r][2 * w + 1] = dot2(pp[r], hi, acc[r][2 * w + 1]);
      }
    }
  }
  // Finish this tile's P.V here, in program order, so it is not sunk past
  // the following tiles' work (which would keep its V registers live).
#pragma unroll
  for (int r = 0; r < RPW; r++)
    asm volatile("" : "+v"(acc[r][0]), "+v"(acc[r][1]), "+v"(acc[r][2]), "+v"(acc[r][3]),
                 "+v"(acc[r][4]), "+v"(acc[r][5]), "+v"(acc[r][6]), "+v"(acc[r][7]));
}


// Streams the tiles first, first+stride, ... (< te) of KV head kvh through
// this wave: the online softmax of the wave's rows (q_raw: this lane's
// chunk, features 8c..8c+7, of each row in fp32) accumulates into
// (m_run, l_run, acc).  Rows r >= nrows and positions past each row's limit
// (my_lim for the lane's own row, min_lim the smallest over rows) are
// masked.  Tiles are taken in chunks of CHUNK, unrolled at compile time:
// K of tile i+1 is issued before tile i's logits and V of tile i+1 before
// tile i's P.V, so a tile of loads stays in flight while the wave computes,
// and no in-flight register is carried across a loop edge (the compiler
// would copy it, which waits for it).  Chunk slots past the wave's last tile
// re-read that tile (an L2 hit) and are fully masked.
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

__device__ __forceinline__ float rope_angle(const RopeArgs& rp, int pos, int j) {
  return ((float)pos / rp.pos_div) * rp.inv_freq[j];
}

// Window rows the fused path supports: its (cos, sin) table lives in LDS.
constexpr int kRopeMaxQueries = 32;

// (cos, sin) of every (window query m, rotation pair j), m-major, into LDS
// by the whole workgroup (one sincos per entry), then a barrier.
template <int DPH>
__device__ __forceinline__ void rope_table(const RopeArgs& rp, int pos_base, int M,
                                           float2* cs) {
  constexpr int HALF = DPH / 2;
  for (int t = threadIdx.x; t < M * HALF; t += blockDim.x) {
    const int m = t / HALF;
    float sn, c;
    sincosf(rope_angle(rp, pos_base + m, t - m * HALF), &sn, &c);
    cs[t] = make_float2(c, sn);
  }
  __syncthreads();
}

// The lane's row permutation for stream_qk's select-free butterfly steps:
// bit (RB-1-kk) of the flip is bit (S-1-kk) of the chunk index c, for the
// first SF steps.  A step can go select-free only if its partner lanes
// differ in its own flip bit and agree on the earlier ones: with 16 lanes
// per token the first two partners are c^8 and the 8-lane mirror (both row
// bits); with 8 lanes the first partner is the 8-lane mirror, which also
// flips the second bit, so only the first step qualifies.
template <int DPH, int RPW>
__device__ __forceinline__ int q_row_flip(int c) {
  using Sh = StreamShape<DPH, RPW>;
  int flip = 0;
#pragma unroll
  for (int kk = 0; kk < Sh::SF; kk++) flip |= ((c >> (Sh::S - 1 - kk)) & 1) << (Sh::RB - 1 - kk);
  return flip;
}

// qr[r] <- packed row r ^ flip (selects on whole rows, once per packing).
template <int RPW>
__device__ __forceinline__ void permute_rows(uint4 (&qr)[RPW], int flip) {
#pragma unroll
  for (int bit = RPW / 2; bit >= 1; bit >>= 1) {
    const bool f = flip & bit;
    uint4 t[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const uint4 a = qr[r], b = qr[r ^ bit];
      t[r] = make_uint4(f ? b.x : a.x, f ? b.y : a.y, f ? b.z : a.z, f ? b.w : a.w);
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) qr[r] = t[r];
  }
}

template <int DPH, int RPW, int CHUNK>
__device__ __forceinline__ void wave_attend(const TileSource& src, int kvh, int first, int te,
                                            int stride, int nrows, int min_lim, int my_lim,
                                            float qscale, const float2 (&q_raw)[RPW][4],
                                            float& m_run, float& l_run, float (&acc)[RPW][8],
                                            bool balance = false) {
  using Sh = StreamShape<DPH, RPW>;
  constexpr int CH = Sh::CH, SL = Sh::SL, NLD = Sh::NLD;
  const int lane = threadIdx.x & 63;
  const int sl = lane / CH;
  const int c = lane % CH;
  const int my_jp = (c >> (Sh::S - Sh::T)) & ((1 << (Sh::T - Sh::RB)) - 1);
  const const_table_t table = const_table(src);
  const char* head_base = reinterpret_cast<const char*>(src.pool) + (size_t)kvh * DPH * 2u;
  const uint32_t lane_off = (uint32_t)sl * 2u * (uint32_t)src.kv_dim + 16u * c;
  const uint32_t chunk_off = 16u * c;
  if (first >= te) return;
  const int last = first + ((te - 1 - first) / stride) * stride;
  uint4 qr[RPW];
  for (int c0 = first; c0 < te; c0 += CHUNK * stride) {
    uint4 kbuf[2][NLD], vbuf[2][NLD];
    int blk[2][NLD], slot[2][NLD];
    float al;
    uint32_t pk;
    tile_groups<NLD, SL>(src, table, min(c0, last) * kTile, blk[0], slot[0]);
    stream_load<DPH>(src, head_base, min(c0, last) * kTile, sl, lane_off, chunk_off, false,
                     blk[0], slot[0], kbuf[0]);
    stream_load<DPH>(src, head_base, min(c0, last) * kTile, sl, lane_off, chunk_off, true,
                     blk[0], slot[0], vbuf[0]);
    if (CHUNK > 1)
      tile_groups<NLD, SL>(src, table, min(c0 + stride, last) * kTile, blk[1], slot[1]);
#pragma unroll
    for (int i = 0; i < CHUNK; i++) {
      const int t = c0 + i * stride;
      const int b = i & 1, nb = b ^ 1;
      const int tn = min(t + stride, last);
      if (i + 1 < CHUNK)
        stream_load<DPH>(src, head_base, tn * kTile, sl, lane_off, chunk_off, false, blk[nb],
                         slot[nb], kbuf[nb]);
      if (i == 0) {
        // q is scaled into the exp2 domain and rounded to fp16 pairs once
        // this chunk's loads are in flight (q was loaded before them, so
        // this waits for no tile data).
#pragma unroll
        for (int r = 0; r < RPW; r++) {
          const float sc = r < nrows ? qscale : 0.f;
          qr[r] = make_uint4(pack_h2(q_raw[r][0].x * sc, q_raw[r][0].y * sc),
                             pack_h2(q_raw[r][1].x * sc, q_raw[r][1].y * sc),
                             pack_h2(q_raw[r][2].x * sc, q_raw[r][2].y * sc),
                             pack_h2(q_raw[r][3].x * sc, q_raw[r][3].y * sc));
        }
        permute_rows<RPW>(qr, q_row_flip<DPH, RPW>(c));
      }
      // A slot past the wave's last tile: every token masked (no-op).
      const int ts_mask = t <= last ? t * kTile : INT_MAX / 2;
      // Balanced issue: the first half of every chunk's tiles runs at raised
      // wave priority, so a wave past its midpoint, or in its epilogue,
      // yields VALU issue to the other wave of its SIMD that is behind.
      if (balance) {
        if (2 * i < CHUNK) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      stream_qk<DPH, RPW, 0>(ts_mask, sl, c, min_lim, my_lim, my_jp, qr, kbuf[b], m_run, l_run,
                             al, pk);
      if (i + 1 < CHUNK) {
        stream_load<DPH>(src, head_base, tn * kTile, sl, lane_off, chunk_off, true, blk[nb],
                         slot[nb], vbuf[nb]);
        if (i + 2 < CHUNK)
          tile_groups<NLD, SL>(src, table, min(t + 2 * stride, last) * kTile, blk[b], slot[b]);
      }
      stream_pv<DPH, RPW, 0>(sl, al, pk, vbuf[b], acc);
    }
  }
  if (balance) __builtin_amdgcn_s_setprio(0);
}

// Totals over the four 16-lane rows of four values at once: afterwards lanes
// of row j hold the total of v[j] (per column).  permlane16_swap exchanges
// the odd rows of its first operand with the even rows of its second,
// permlane32_swap the upper half of its first with the lower half of its
// second, so two row-pair sums and one half-pair sum leave each row with the
// total of one of the four.
__device__ __forceinline__ float rows_total4(float v0, float v1, float v2, float v3) {
  const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v0),
                                                  __builtin_bit_cast(int, v1), false, false);
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v2),
                                                  __builtin_bit_cast(int, v3), false, false);
  const float s01 = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
  const float s23 = __builtin_bit_cast(float, (int)q[0]) + __builtin_bit_cast(float, (int)q[1]);
  return half_pair_total(s01, s23);
}

// Where wave_merge_slots leaves the slot totals: 16-lane row j holds row
// merged_row(j) of the record, features 8c + merged_col(j) + e for
// e < 2*RPW.
template <int RPW>
__device__ __forceinline__ int merged_row(int j) { return RPW == 4 ? j : (j & 1); }
template <int RPW>
__device__ __forceinline__ int merged_col(int j) { return RPW == 4 ? 0 : 4 * (j >> 1); }

// Merges the token slots' softmax states of this wave.  Every lane gets
// m_row / l_row, the max and sum of its own row my_r over all slots, and
// out[e] (e < 2*RPW), the accumulators rescaled to that max and summed over
// the slots, spread over the 16-lane rows j = lane/16: row j holds row
// merged_row(j), features 8c + merged_col(j) + e (c = lane % CH; with
// dph 64 both halves of a 16-lane row hold the same values).  Four values
// share each pair of row swaps, so the merge costs a quarter of the
// cross-lane moves of one all-reduce per value.
template <int DPH, int RPW>
__device__ __forceinline__ void wave_merge_slots(float m_run, float l_run,
                                                 const float (&acc)[RPW][8], float& m_row,
                                                 float& l_row, float (&out)[2 * RPW]) {
  using Sh = StreamShape<DPH, RPW>;
  constexpr int CH = Sh::CH;
  const int lane = threadIdx.x & 63;
  const int c = lane % CH;
  const bool odd_slot = (lane / CH) & 1;
  // Lanes of one chunk c share the row my_r, so the slot max of m_run is
  // the row's max and f_own rescales this lane's (row, slot) state to it.
  m_row = slot_max<DPH>(m_run);
  const float f_own = m_row == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_row);
  // l of (row, slot): sum over the row's token-pair owners (redundant lanes
  // hold copies and contribute 0).
  const bool redundant = (c & ((1 << (Sh::S - Sh::T)) - 1)) != 0;
  float lsum = redundant ? 0.f : l_run;
#pragma unroll
  for (int kk = Sh::RB; kk < Sh::S; kk++) lsum += bfly<CH>(lsum, kk);
  l_row = slot_sum<DPH>(lsum * f_own);
  float x[RPW][8];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const float f = from_owner_f<DPH, RPW>(f_own, r, 0, odd_slot);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      x[r][e] = acc[r][e] * f;
      if constexpr (DPH == 64) x[r][e] += dpp_f(x[r][e], 3);  // slots 2k, 2k+1 of a row
    }
  }
#pragma unroll
  for (int e = 0; e < 2 * RPW; e++) {
    if constexpr (RPW == 4)
      out[e] = rows_total4(x[0][e], x[1][e], x[2][e], x[3][e]);
    else
      out[e] = rows_total4(x[0][e], x[1][e], x[0][e + 4], x[1][e + 4]);
  }
}

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
  int row_groups;  // ceil(R / rows per wave)
  int pos_base;    // query m sees positions [0, pos_base+m]
  int n_parts;
  int tiles_per_part;
  float qscale;    // log2(e) / sqrt(dph)
};

constexpr int kStreamWaves = 8;      // waves per workgroup of libsde_paged's kernel
constexpr int kStreamMaxParts = 64;  // partitions per (KV head, row group)

// Device-scope (agent) relaxed atomic accesses for the partition partials:
// the stores write through to the device coherence point and the loads do
// not hit stale lines of another XCD's L2, so publishing partials needs no
// L2 writeback/invalidate fence (those cost microseconds per workgroup).
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
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)bytes, kRsrcWord3);
  // Bit-cast the whole vector: extracting elements of the builtin's integer
  // vector result makes this compiler shrink the load to one dword.
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v v = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
  return make_float4(v.x, v.y, v.z, v.w);
}

// One pass of the partition combine over NIT row slices: thread
// (row, float4 column c4, quarter sub) of slice it loads (max, sum, acc[c4])
// of partitions sub, sub+4, ... for all of its slices first -- every
// partial of the pass in one round trip, no LDS -- then weights them by
// exp2(m_p - max), and the four quarters of a (row, column) (adjacent
// lanes) reduce through DPP in a fixed order, so the result does not
// depend on arrival order.  (max, sum) of partition p is loaded once per
// wave, by lane p (a wave's lanes serve one row), and read across lanes.
// Within a live slice every load is issued unconditionally (indices past
// P re-read partition P-1, then weigh 0), so they all travel in one round
// trip: a load under `if (p < P)` would get a wait of its own at the join.
template <int DPH, int PMAX, int NIT, int WAVES>
__device__ __forceinline__ void combine_pass(const AttnArgs& a, int kvh, int r0, int nrows,
                                             int it0) {
  constexpr int C4 = DPH / 4;
  constexpr int SUB = 4;
  constexpr int NT = 64 * WAVES;
  const int P = a.n_parts;
  const int lane = threadIdx.x & 63;
  const int sub = threadIdx.x & (SUB - 1);
  const int col4 = (threadIdx.x / SUB) % C4;
  const size_t acc_floats = (size_t)a.nkv * a.R * P * DPH;
  const uint32_t acc_bytes = (uint32_t)(acc_floats * 4);
  float4 v[NIT][PMAX];
  float2 mine[NIT];
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int r = (threadIdx.x + (it0 + it) * NT) / (SUB * C4);  // uniform per wave
    if (r < nrows) {
      const size_t row = (size_t)kvh * a.R + r0 + r;
      const uint32_t acc_off = (uint32_t)((row * P * DPH + 4 * col4) * 4);
#pragma unroll
      for (int i = 0; i < PMAX; i++) {
        const int p = min(sub + i * SUB, P - 1);
        v[it][i] = load_dev16(a.partials, acc_bytes, acc_off + (uint32_t)p * (DPH * 4));
      }
      mine[it] = load_dev2(a.partials + acc_floats + row * P * 2 + (size_t)min(lane, P - 1) * 2);
    }
  }
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int r = (threadIdx.x + (it0 + it) * NT) / (SUB * C4);
    if (r >= nrows) break;
    float2 e[PMAX];
#pragma unroll
    for (int i = 0; i < PMAX; i++) {
      e[i].x = __shfl(mine[it].x, sub + i * SUB);
      e[i].y = __shfl(mine[it].y, sub + i * SUB);
      if (sub + i * SUB >= P) {
        e[i] = make_float2(-INFINITY, 0.f);
        v[it][i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PMAX; i++) mx = fmaxf(mx, e[i].x);
    mx = fmaxf(mx, dpp_f(mx, 0));
    mx = fmaxf(mx, dpp_f(mx, 1));
    float l = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < PMAX; i++) {
      const float w = e[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(e[i].x - mx);
      l += e[i].y * w;
      o.x += w * v[it][i].x;
      o.y += w * v[it][i].y;
      o.z += w * v[it][i].z;
      o.w += w * v[it][i].w;
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
      l += dpp_f(l, k);
      o.x += dpp_f(o.x, k);
      o.y += dpp_f(o.y, k);
      o.z += dpp_f(o.z, k);
      o.w += dpp_f(o.w, k);
    }
    if (sub == 0) {
      const float inv = finish_scale(l);
      const int gr = r0 + r;
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      float2* dst = reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH +
                                              4 * col4);
      dst[0] = make_float2(o.x * inv, o.y * inv);
      dst[1] = make_float2(o.z * inv, o.w * inv);
    }
  }
}

// Passes of up to 32 in-flight partial loads per thread.
template <int DPH, int RPW, int PMAX, int WAVES>
__device__ __forceinline__ void combine_rows(const AttnArgs& a, int kvh, int r0, int nrows) {
  constexpr int SLICES = (RPW * DPH + 64 * WAVES - 1) / (64 * WAVES);  // RPW*C4*SUB / threads
  constexpr int CAP = 32 / PMAX;
  constexpr int NIT = SLICES < CAP ? SLICES : CAP;
#pragma unroll
  for (int it0 = 0; it0 < SLICES; it0 += NIT)
    combine_pass<DPH, PMAX, NIT, WAVES>(a, kvh, r0, nrows, it0);
}

// Partition combine, run by the last workgroup of a (KV head, row group) to
// finish (the rows r0 .. r0+nrows-1 of KV head kvh).
template <int DPH, int RPW, int WAVES>
__device__ __forceinline__ void stream_combine(const AttnArgs& a, int kvh, int r0, int nrows) {
  static_assert(kStreamMaxParts == 64, "combine buckets");
  static_assert((4 * (DPH / 4)) % 64 == 0, "each wave's lanes serve one row");
  if ((int)threadIdx.x >= 64 * WAVES) return;  // waves past WAVES idle
  const int P = a.n_parts;
  if (P <= 16)
    combine_rows<DPH, RPW, 4, WAVES>(a, kvh, r0, nrows);
  else if (P <= 32)
    combine_rows<DPH, RPW, 8, WAVES>(a, kvh, r0, nrows);
  else
    combine_rows<DPH, RPW, 16, WAVES>(a, kvh, r0, nrows);
}

// The window's rows (positions pos_base .. pos_base+M-1) of KV head kvh:
// k rotated by RoPE, k and v rounded to fp16 (RNE) into the pool
// (kv_cache_append, kv_cache.cu:70-93), by the whole workgroup; returns
// once the stores are visible to the workgroup's loads.
template <int DPH>
__device__ __forceinline__ void rope_append_slice(const AttnArgs& a, const RopeArgs& rp,
                                                  const float2* rope_cs, int kvh) {
  constexpr int HALF = DPH / 2;
  const int M = a.R / a.G;
  const int kvd = a.src.kv_dim;
  const int bs = a.src.bs;
  for (int t = threadIdx.x; t < M * HALF; t += blockDim.x) {
    const int m = t / HALF;
    const int j = t - m * HALF;
    const int pos = a.pos_base + m;
    const float* kin = rp.k_new + (size_t)m * kvd + (size_t)kvh * DPH;
    const float x0 = kin[j], x1 = kin[j + HALF];
    const float cs = rope_cs[t].x, sn = rope_cs[t].y;
    const int lb = pos / bs;
    const int slot = pos - lb * bs;
    uint16_t* kd = rp.pool + ((size_t)(uint32_t)a.src.table[lb] * 2u * bs + slot) * kvd +
                   (size_t)kvh * DPH;
    kd[j] = __builtin_bit_cast(uint16_t, (_Float16)(x0 * cs - x1 * sn));
    kd[j + HALF] = __builtin_bit_cast(uint16_t, (_Float16)(x0 * sn + x1 * cs));
  }
  for (int t = threadIdx.x; t < M * DPH; t += blockDim.x) {
    const int m = t / DPH;
    const int d = t - m * DPH;
    const int pos = a.pos_base + m;
    const int lb = pos / bs;
    const int slot = pos - lb * bs;
    uint16_t* vd = rp.pool + ((size_t)(uint32_t)a.src.table[lb] * 2u * bs + bs + slot) * kvd +
                   (size_t)kvh * DPH;
    vd[d] = __builtin_bit_cast(uint16_t, (_Float16)rp.v_new[(size_t)m * kvd + (size_t)kvh * DPH + d]);
  }
  __syncthreads();
}

// ---- MFMA tile path (v_mfma_f32_16x16x32_f16, up to 16 rows per wave) ----
//
// K and V stream in with the same loads as the VALU path (a token's slice
// read by CH lanes, 16 bytes each) and are staged per wave in LDS, row-major
// by token with the 16-byte units of row t stored at unit u ^ (t % UNITS),
// which keeps both the stores and the operand reads below free of bank
// conflicts.  Per tile of 32 tokens:
//  * logits S^T[token][row] = K . Q^T: A = K read from LDS in the operand
//    layout (lane l: token l%16 of a 16-token block, features
//    32ks + 8(l/16) .. +7), B = Q^T (row l%16, the same features).  The C
//    layout leaves lane l the logits of row l%16 for tokens 4(l/16) + i and
//    16 + 4(l/16) + i (i < 4), so the online softmax is lane-local per row:
//    one cross-group max per tile (two lane swaps), sums reduced once.
//  * O^T[feature][row] += V^T . P^T: B = P^T straight from the logits'
//    registers (k order: tokens 4(l/16)+i, then 16+4(l/16)+i), A = V^T read
//    with ds_read_b64_tr_b16: in each 16-lane group lane 4b+t receives
//    element t of the 8-byte pieces addressed by lanes b, b+4, b+8, b+12, so
//    lane m' addressing token base + m'/4, features 16db + 4(m'%4) gives
//    lane m feature 16db + m of tokens base..base+3 (the A layout).
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
// update and the rescale of o; returns P^T as the output product's B.
// kst: this wave's staged K tile.
template <int DPH>
__device__ __forceinline__ h8_t mfma_logits(int ts, int q, int l16, int lim,
                                            const h8_t (&qb)[MfmaShape<DPH>::KS],
                                            const char* kst, float& m_run, float& l_run,
                                            f4_t (&o)[MfmaShape<DPH>::DB]) {
  using Sh = MfmaShape<DPH>;
  f4_t s[2];
#pragma unroll
  for (int tb = 0; tb < 2; tb++) {
    s[tb] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < Sh::KS; ks++) {
      const uint4 kx =
          *reinterpret_cast<const uint4*>(kst + staged<DPH>(16 * tb + l16, 4 * ks + q));
      s[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, kx), qb[ks], s[tb],
                                                     0, 0, 0);
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
  float p[8];
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
  return h8_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
              (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
}

// o += V^T . P^T for a tile; vst: this wave's staged V tile.
template <int DPH>
__device__ __forceinline__ void mfma_pv(int q, int l16, const h8_t pb, const char* vst,
                                        f4_t (&o)[MfmaShape<DPH>::DB]) {
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
    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, both), pb, o[db], 0,
                                                   0, 0);
  }
}

// This lane's q operand (row l%16, features 32ks + 8(l/16) + e) from its
// raw fp32 values: rotated by RoPE when cs (the row's (cos, sin) table
// entries, feature-pair-indexed) is given -- the partner of feature f is
// f +- dph/2, k-step ks +- KS/2 of the same lane -- then scaled into the
// exp2 domain and rounded to fp16.
template <int DPH>
__device__ __forceinline__ void mfma_pack_q(const float2 (&qr)[MfmaShape<DPH>::KS][4], float sc,
                                            const float2* cs, int grp,
                                            h8_t (&qb)[MfmaShape<DPH>::KS]) {
  constexpr int KS = MfmaShape<DPH>::KS;
  float x[KS][8];
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int w = 0; w < 4; w++) {
      x[ks][2 * w] = qr[ks][w].x;
      x[ks][2 * w + 1] = qr[ks][w].y;
    }
  if (cs) {
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
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int e = 0; e < 8; e++) qb[ks][e] = (_Float16)(x[ks][e] * sc);
}

// Per-wave constants of the MFMA tile loop.
struct MfmaWave {
  const char* head_base;  // this KV head's slice in the pool
  const_table_t table;
  uint32_t lane_off, chunk_off;
  int sl, c, l16, q;      // load role (slot, chunk) and operand role (row, group)
  int last, stride, lim;
  char* kst;              // staged K tile; the V tile follows
};

// One chunk of a wave's tiles, starting at tile c0, pipelined a tile ahead
// like wave_attend.  FIRST: the wave's first chunk, which packs q once its
// first loads are in flight (q was loaded before them, so this waits for no
// tile data); the raw q registers are dead after it.
template <int DPH, int CHUNK, bool FIRST>
__device__ __forceinline__ void mfma_chunk(const TileSource& src, const MfmaWave& w, int c0,
                                           const float2 (&qr)[MfmaShape<DPH>::KS][4], float qsc,
                                           const float2* cs, h8_t (&qb)[MfmaShape<DPH>::KS],
                                           float& m_run, float& l_run,
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
    if (FIRST && i == 0) mfma_pack_q<DPH>(qr, qsc, cs, w.q, qb);
    if (balance) {
      if (2 * i < CHUNK) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // A slot past the wave's last tile: every token masked (no-op).
    const int ts_mask = t <= w.last ? t * kTile : INT_MAX / 2;
    stage_tile<DPH>(w.kst, w.sl, w.c, kbuf[b]);
    const h8_t pb = mfma_logits<DPH>(ts_mask, w.q, w.l16, w.lim, qb, w.kst, m_run, l_run, o);
    if (i + 1 < CHUNK) {
      stream_load<DPH>(src, w.head_base, tn * kTile, w.sl, w.lane_off, w.chunk_off, true,
                       blk[nb], slot[nb], vbuf[nb]);
      if (i + 2 < CHUNK)
        tile_groups<NLD, SL>(src, w.table, min(t + 2 * w.stride, w.last) * kTile, blk[b],
                             slot[b]);
    }
    stage_tile<DPH>(vst, w.sl, w.c, vbuf[b]);
    mfma_pv<DPH>(w.q, w.l16, pb, vst, o);
  }
}

// A wave's tiles first, first+stride, ... < te of KV head kvh on the MFMA
// path.  lim: last visible position of this lane's row (-1: a padding
// row).  qr, qsc, cs: the lane's raw q values, their scale and RoPE table
// (mfma_pack_q).  st: this wave's LDS (K tile, then V tile).
template <int DPH, int CHUNK>
__device__ __forceinline__ void mfma_attend(const TileSource& src, int kvh, int first, int te,
                                            int stride, int lim,
                                            const float2 (&qr)[MfmaShape<DPH>::KS][4], float qsc,
                                            const float2* cs, char* st, float& m_run,
                                            float& l_run, f4_t (&o)[MfmaShape<DPH>::DB],
                                            bool balance) {
  constexpr int CH = DPH / 8;
  if (first >= te) return;
  const int lane = threadIdx.x & 63;
  MfmaWave w;
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
  w.kst = st;
  h8_t qb[MfmaShape<DPH>::KS];
  mfma_chunk<DPH, CHUNK, true>(src, w, first, qr, qsc, cs, qb, m_run, l_run, o, balance);
  for (int c0 = first + CHUNK * stride; c0 < te; c0 += CHUNK * stride)
    mfma_chunk<DPH, CHUNK, false>(src, w, c0, qr, qsc, cs, qb, m_run, l_run, o, balance);
  if (balance) __builtin_amdgcn_s_setprio(0);
}

// LDS of stream_item: per-wave records of every row, acc[DPH] and
// (max, sum).
template <int DPH, int RPW, int WAVES>
struct StreamLds {
  float acc[WAVES * RPW * DPH] __attribute__((aligned(16)));
  float2 ml[WAVES * RPW];
  int last;
  __device__ float* acc_at(int w, int r) { return acc + (w * RPW + r) * DPH; }
  __device__ float2& ml_at(int w, int r) { return ml[w * RPW + r]; }
};

// LDS of the MFMA tile path: per wave, its staged K and V tiles; once the
// wave's tiles are done the same bytes hold its records (up to 16 rows).
template <int DPH, int WAVES>
struct MfmaLds {
  static constexpr int kRows = 16;
  static_assert(kRows * (DPH + 2) * 4 <= MfmaShape<DPH>::WAVEB, "records fit the staging area");
  char st[WAVES * MfmaShape<DPH>::WAVEB] __attribute__((aligned(16)));
  int last;
  __device__ char* staging(int w) { return st + w * MfmaShape<DPH>::WAVEB; }
  __device__ float* acc_at(int w, int r) {
    return reinterpret_cast<float*>(staging(w)) + r * DPH;
  }
  __device__ float2& ml_at(int w, int r) {
    return reinterpret_cast<float2*>(staging(w) + kRows * DPH * 4)[r];
  }
};

// Partition `part` of (KV head kvh, row group rg) on the calling workgroup:
// waves 0..WAVES-1 take tiles tb+w, tb+w+WAVES, ... (further waves idle),
// merge their states through LDS, and either write the normalised output
// (one partition) or publish a partial and count the arrival; the last
// arrival combines all partitions.  Every thread of the workgroup calls it.
template <int DPH, int RPW, int CHUNK, int WAVES, bool ROPE = false, bool MF = false,
          class Lds>
__device__ __forceinline__ void stream_item(const AttnArgs& a, int part, int kvh, int rg,
                                            Lds& lds, const RopeArgs* rp = nullptr,
                                            float2* rope_cs = nullptr) {
  static_assert(DPH == 64 || DPH == 128, "head_dim");
  static_assert(RPW == 2 || RPW == 4 || (MF && (RPW == 8 || RPW == 16)), "rows per wave");
  static_assert(MF || !ROPE, "fused RoPE runs on the MFMA tile path");
  constexpr int CH = DPH / 8;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int sl = lane / CH;
  const int c = lane % CH;
  const int r0 = rg * RPW;
  const int nrows = min(RPW, a.R - r0);
  const int n_tiles = (a.src.L_max + kTile - 1) / kTile;
  const int tb = part * a.tiles_per_part;
  const int te = min(n_tiles, tb + a.tiles_per_part);

  if constexpr (ROPE) {
    rope_table<DPH>(*rp, a.pos_base, a.R / a.G, rope_cs);
    // A partition that reads window positions first writes the window's K
    // (rotated) and V slice of this KV head itself, so no other workgroup
    // has to finish first; partitions sharing the window write the same
    // bytes.
    if (te * kTile > a.pos_base) rope_append_slice<DPH>(a, *rp, rope_cs, kvh);
  }

  if constexpr (MF) {
    if (wave < WAVES) {
      // MFMA tile path: lane l serves row r0 + l%16 (rows past nrows are
      // padding: zero q, nothing visible).
      using Mh = MfmaShape<DPH>;
      const int l16 = lane & 15, grp = lane >> 4;
      const bool real = l16 < nrows;
      const int gr = min(r0 + l16, a.R - 1);
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      const float2* qp = reinterpret_cast<const float2*>(a.q + (size_t)m * a.nh * DPH +
                                                         (size_t)h * DPH + 8 * grp);
      float2 qr[Mh::KS][4];
#pragma unroll
      for (int ks = 0; ks < Mh::KS; ks++)
#pragma unroll
        for (int w = 0; w < 4; w++) qr[ks][w] = qp[16 * ks + w];
      const float2* cs = nullptr;
      if constexpr (ROPE) cs = rope_cs + m * (DPH / 2);
      const int lim = real ? a.pos_base + (r0 + l16) / a.G : -1;
      float m_run = -INFINITY, l_run = 0.f;
      f4_t o[Mh::DB];
#pragma unroll
      for (int db = 0; db < Mh::DB; db++) o[db] = f4_t{0.f, 0.f, 0.f, 0.f};
      mfma_attend<DPH, CHUNK>(a.src, kvh, tb + wave, te, WAVES, lim, qr,
                              real ? a.qscale : 0.f, cs, lds.staging(wave), m_run, l_run, o,
                              a.row_groups > 1);
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
  } else if (wave < WAVES) {
    using Sh = StreamShape<DPH, RPW>;
    const int my_r = (c >> (Sh::S - Sh::T)) >> (Sh::T - Sh::RB);
    // This lane's q chunk (features 8c..8c+7) of every row, loaded before
    // any K/V load so that waiting for it never waits for tile data.
    float2 q_raw[RPW][4];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const int gr = min(r0 + r, a.R - 1);  // rows past nrows: zeroed by wave_attend
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      const float2* qp = reinterpret_cast<const float2*>(a.q + (size_t)m * a.nh * DPH +
                                                         (size_t)h * DPH + 8 * c);
#pragma unroll
      for (int w = 0; w < 4; w++) q_raw[r][w] = qp[w];
    }
    // Last visible position of each row (query m sees pos_base + m); rows
    // past nrows see nothing.
    int min_lim = INT_MAX, my_lim = -1;
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const int lim = r < nrows ? a.pos_base + (r0 + r) / a.G : -1;
      min_lim = min(min_lim, lim);
      if (r == my_r) my_lim = lim;
    }

    float m_run = -INFINITY, l_run = 0.f, acc[RPW][8];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
      for (int e = 0; e < 8; e++) acc[r][e] = 0.f;
    // Several row groups per KV head make the step VALU-bound per SIMD
    // (each K/V byte serves several workgroups from L2): balance the waves
    // of a SIMD (4K 5-query window 14.9 -> 14.5 us; a long one-group decode
    // is HBM-bound and measured 0.3 us slower with it).
    wave_attend<DPH, RPW, CHUNK>(a.src, kvh, tb + wave, te, WAVES, nrows, min_lim, my_lim,
                                 a.qscale, q_raw, m_run, l_run, acc, a.row_groups > 1);

    // ---- merge the slot states of this wave; record per row -------------
    float m_row, l_row, o[2 * RPW];
    wave_merge_slots<DPH, RPW>(m_run, l_run, acc, m_row, l_row, o);
    if (sl == 0 && c == Sh::owner(my_r, 0)) lds.ml_at(wave, my_r) = make_float2(m_row, l_row);
    const int j = lane >> 4;
    if (DPH == 128 || (lane & 8) == 0) {
      float4* dst = reinterpret_cast<float4*>(lds.acc_at(wave, merged_row<RPW>(j)) +
                                              8 * c + merged_col<RPW>(j));
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      if constexpr (RPW == 4) dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
  __syncthreads();

  // ---- workgroup merge: thread (row, feature pair) over the waves --------
  constexpr int DP = DPH / 2;
  for (int idx = threadIdx.x; idx < nrows * DP; idx += blockDim.x) {
    const int r = idx / DP;
    const int dcol = 2 * (idx - r * DP);
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; w++) mx = fmaxf(mx, lds.ml_at(w, r).x);
    float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) {
      const float2 ml = lds.ml_at(w, r);
      const float wt = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
      l += ml.y * wt;
      const float2 x = *reinterpret_cast<const float2*>(lds.acc_at(w, r) + dcol);
      o0 += x.x * wt;
      o1 += x.y * wt;
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

  // ---- the last workgroup of (KV head, row group) combines --------------
  // Partials are device-scope stores; waiting for them (vmcnt) before the
  // arrival increment orders them before it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* ctr = a.counters + (size_t)kvh * a.row_groups + rg;
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)(a.n_parts - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds.last = last;
  }
  __syncthreads();
  if (!lds.last) return;
  stream_combine<DPH, RPW, WAVES>(a, kvh, r0, nrows);
}

// Partition sizing shared by libsde_paged and the grid API: at most
// `blocks` workgroups in all (one per CU for the library), as many
// partitions per (KV head, row group) as that allows (up to
// kStreamMaxParts, at least one tile per wave), then the fewest tiles per
// wave that cover the context.  A wave takes its tiles in chunks of `chunk`
// (1 to max_chunk, unrolled at compile time), several chunks when it has
// more than max_chunk tiles.  (Cutting the context evenly instead, with
// masked slots for the waves past a partition's last tile, measured slower
// on short contexts: the masked slots are not free.)  Rows per group:
// `rows`, or (0) 2 for windows of at most 2 rows and kStreamMaxRows
// otherwise.
struct StreamPlan {
  int rpw;             // rows per group
  int row_groups;
  int chunk;
  int tiles_per_part;
  int n_parts;
};

__host__ __device__ inline StreamPlan stream_plan(int L_max, int nkv, int R, int blocks,
                                                  int waves, int max_chunk, int rows = 0) {
  StreamPlan p;
  p.rpw = rows > 0 ? rows : R <= 2 ? 2 : kStreamMaxRows;
  p.row_groups = (R + p.rpw - 1) / p.rpw;
  const int n_tiles = (L_max + kTile - 1) / kTile;
  const int64_t units = (int64_t)nkv * p.row_groups;
  int64_t parts = blocks / units;
  if (parts < 1) parts = 1;
  if (parts > kStreamMaxParts) parts = kStreamMaxParts;
  const int64_t by_len = (n_tiles + waves - 1) / waves;
  if (parts > by_len) parts = by_len;
  const int per_wave = (int)((n_tiles + parts * waves - 1) / (parts * waves));
  p.chunk = per_wave < max_chunk ? (per_wave < 1 ? 1 : per_wave) : max_chunk;
  const int reps = (per_wave + p.chunk - 1) / p.chunk;
  p.tiles_per_part = waves * p.chunk * (reps < 1 ? 1 : reps);
  p.n_parts = (n_tiles + p.tiles_per_part - 1) / p.tiles_per_part;
  return p;
}

// One query, all heads, all of [0, total_len) on one block (no split):
// wave w takes the (KV head, group of up to four q heads) units w, w+nw, ...
template <int DPH>
__device__ __forceinline__ void block_attend(const float* q_all, float* out, const sde_kv_view& kv,
                                             int layer, int nh, int nkv, int total_len) {
  constexpr int RPW = kStreamMaxRows;
  constexpr int CH = DPH / 8;
  const int G = nh / nkv;
  const int groups = (G + RPW - 1) / RPW;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c = lane % CH;
  const TileSource src{kv.pool, kv.block_tables + (size_t)layer * kv.max_blocks_per_layer,
                       kv.kv_dim, kv.block_size, total_len};
  const int n_tiles = (total_len + kTile - 1) / kTile;
  const float qscale = (float)(kLog2e / __builtin_sqrt((double)DPH));
  using Sh = StreamShape<DPH, RPW>;
  const int my_r = (c >> (Sh::S - Sh::T)) >> (Sh::T - Sh::RB);
  for (int u = wave; u < nkv * groups; u += nw) {
    const int kvh = u / groups;
    const int h0 = kvh * G + (u - kvh * groups) * RPW;
    const int nrows = min(RPW, kvh * G + G - h0);
    float2 q_raw[RPW][4];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const float2* qp = reinterpret_cast<const float2*>(q_all + (size_t)min(h0 + r, nh - 1) * DPH +
                                                         8 * c);
#pragma unroll
      for (int w = 0; w < 4; w++) q_raw[r][w] = qp[w];
    }
    const int min_lim = nrows < RPW ? -1 : total_len - 1;
    const int my_lim = my_r < nrows ? total_len - 1 : -1;
    float m_run = -INFINITY, l_run = 0.f, acc[RPW][8];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
      for (int e = 0; e < 8; e++) acc[r][e] = 0.f;
    wave_attend<DPH, RPW, 2>(src, kvh, 0, n_tiles, 1, nrows, min_lim, my_lim, qscale, q_raw,
                             m_run, l_run, acc);
    float m_row, l_row, o[2 * RPW];
    wave_merge_slots<DPH, RPW>(m_run, l_run, acc, m_row, l_row, o);
    // 16-lane row j holds row rr of the output; its sum sits in the lanes
    // of chunk owner(rr, 0).
    const int j = lane >> 4;
    const int rr = merged_row<RPW>(j);
    float l_mine = 0.f;
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const float lr = from_owner_f<DPH, RPW>(l_row, r, 0, false);
      if (r == rr) l_mine = lr;
    }
    if (rr < nrows && (DPH == 128 || (lane & 8) == 0)) {
      const float inv = finish_scale(l_mine);
      float4* dst = reinterpret_cast<float4*>(out + (size_t)(h0 + rr) * DPH + 8 * c +
                                              merged_col<RPW>(j));
      dst[0] = make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
      if constexpr (RPW == 4) dst[1] = make_float4(o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv);
    }
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
// applied) over positions [0, total_len) of `layer`: q head h reads KV head
// h*nkv/nh, scale dph^-1/2; attn_out fp32 [nh*dph] is fully written
// (zeros when total_len is 0).  head_dim 64 or 128, block_size a multiple
// of 8, nkv | nh; returns SDE_ERR_UNSUPPORTED (writing nothing) otherwise.
__device__ inline int device_flash_attention_gqa(const float* q_all, float* attn_out,
                                                 const sde_kv_view& kv, int layer, int nh, int nkv,
                                                 int dph, int total_len) {
  if (nkv < 1 || nh % nkv != 0 || kv.block_size % 8 != 0 || total_len < 0) return SDE_ERR_UNSUPPORTED;
  if (dph == 128)
    attn::block_attend<128>(q_all, attn_out, kv, layer, nh, nkv, total_len);
  else if (dph == 64)
    attn::block_attend<64>(q_all, attn_out, kv, layer, nh, nkv, total_len);
  else
    return SDE_ERR_UNSUPPORTED;
  __syncthreads();
  return SDE_OK;
}

// attention.h:140-164: SDE_ATTN_SOFTMAX runs device_flash_attention_gqa; the
// types the reference reserves (and traps on) return SDE_ERR_UNSUPPORTED.
__device__ inline int device_attention_dispatch(int attn_type, const float* q_all, float* attn_out,
                                                const sde_kv_view& kv, int layer, int nh, int nkv,
                                                int dph, int total_len) {
  if (attn_type != SDE_ATTN_SOFTMAX) return SDE_ERR_UNSUPPORTED;
  return device_flash_attention_gqa(q_all, attn_out, kv, layer, nh, nkv, dph, total_len);
}

// ---- grid-cooperative split-context attention (persistent kernels) -------

// Bytes of the workspace of device_flash_attention_gqa_grid for windows of
// up to n_queries queries over up to max_total_len positions: the arrival
// counters (one per (KV head, row group), padded to 256 bytes; zero-fill
// them once before the first call, each call leaves them zero) followed by
// the partials of at most kStreamMaxParts partitions.
__host__ __device__ inline size_t grid_attention_workspace_size(int nh, int nkv, int dph,
                                                                int n_queries, int max_total_len) {
  if (nh < 1 || nkv < 1 || nh % nkv != 0 || dph < 1 || n_queries < 1 || max_total_len < 1)
    return 0;
  const int R = n_queries * (nh / nkv);
  const int rpw = R <= 2 ? 2 : attn::kStreamMaxRows;
  const size_t counters = ((size_t)nkv * ((R + rpw - 1) / rpw) * 4 + 255) / 256 * 256;
  const int n_tiles = (max_total_len + attn::kTile - 1) / attn::kTile;
  const int by_len = (n_tiles + 3) / 4;  // 4-wave workgroups hold at least 4 tiles
  const int parts = by_len < attn::kStreamMaxParts ? by_len : attn::kStreamMaxParts;
  return counters + (size_t)nkv * R * parts * (size_t)(dph + 2) * sizeof(float);
}

namespace attn {
template <int DPH, int RPW, int WAVES>
__device__ __forceinline__ void grid_items(const AttnArgs& a, int units_rg, void* lds_raw) {
  auto& lds = *reinterpret_cast<StreamLds<DPH, RPW, WAVES>*>(lds_raw);
  const int n_blocks = gridDim.x * gridDim.y * gridDim.z;
  const int block = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int items = a.nkv * units_rg * a.n_parts;
  for (int it = block; it < items; it += n_blocks) {
    const int part = it % a.n_parts;
    const int unit = it / a.n_parts;
    __syncthreads();  // the previous item's readers of lds are done
    stream_item<DPH, RPW, 2, WAVES>(a, part, unit % a.nkv, unit / a.nkv, lds);
  }
}
}  // namespace attn

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
// Uses 17 KiB of LDS.  Returns the same status in every thread: SDE_OK,
// SDE_ERR_UNSUPPORTED (dph not 64/128, block_size not a multiple of 8,
// blockDim.x < 256), SDE_ERR_INVALID_ARGUMENT, SDE_ERR_CAPACITY (window past
// the layer's table) or SDE_ERR_WORKSPACE; nothing is written on error.
__device__ inline int device_flash_attention_gqa_grid(const float* q_all, float* attn_out,
                                                      const sde_kv_view& kv, int layer, int nh,
                                                      int nkv, int dph, int pos_base,
                                                      int n_queries, void* workspace,
                                                      size_t workspace_bytes) {
  using namespace attn;
  if (blockDim.x < 256 || blockDim.x % 64 != 0) return SDE_ERR_UNSUPPORTED;
  if ((dph != 64 && dph != 128) || kv.block_size % 8 != 0) return SDE_ERR_UNSUPPORTED;
  if (nh < 1 || nkv < 1 || nh % nkv != 0 || nkv * dph != kv.kv_dim || layer < 0 ||
      layer >= kv.n_layers || pos_base < 0 || n_queries < 1 || !q_all || !attn_out || !workspace)
    return SDE_ERR_INVALID_ARGUMENT;
  const int L_max = pos_base + n_queries;
  if ((int64_t)L_max > (int64_t)kv.max_blocks_per_layer * kv.block_size) return SDE_ERR_CAPACITY;
  if (workspace_bytes < grid_attention_workspace_size(nh, nkv, dph, n_queries, L_max))
    return SDE_ERR_WORKSPACE;

  const int waves = blockDim.x >= 512 ? kStreamWaves : 4;
  const int G = nh / nkv;
  const int R = n_queries * G;
  const StreamPlan p =
      stream_plan(L_max, nkv, R, gridDim.x * gridDim.y * gridDim.z, waves, 2);
  AttnArgs a;
  a.src = TileSource{kv.pool, kv.block_tables + (size_t)layer * kv.max_blocks_per_layer,
                     kv.kv_dim, kv.block_size, L_max};
  a.q = q_all;
  a.out = attn_out;
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        ((size_t)nkv * p.row_groups * 4 + 255) / 256 * 256);
  a.nh = nh;
  a.nkv = nkv;
  a.G = G;
  a.R = R;
  a.row_groups = p.row_groups;
  a.pos_base = pos_base;
  a.n_parts = p.n_parts;
  a.tiles_per_part = p.tiles_per_part;
  a.qscale = (float)(kLog2e / __builtin_sqrt((double)dph));

  __shared__ __attribute__((aligned(16))) char lds[sizeof(StreamLds<128, 4, kStreamWaves>)];
  const bool w8 = waves == kStreamWaves;
  if (dph == 128) {
    if (p.rpw == 2)
      w8 ? grid_items<128, 2, kStreamWaves>(a, p.row_groups, lds)
         : grid_items<128, 2, 4>(a, p.row_groups, lds);
    else
      w8 ? grid_items<128, 4, kStreamWaves>(a, p.row_groups, lds)
         : grid_items<128, 4, 4>(a, p.row_groups, lds);
  } else {
    if (p.rpw == 2)
      w8 ? grid_items<64, 2, kStreamWaves>(a, p.row_groups, lds)
         : grid_items<64, 2, 4>(a, p.row_groups, lds);
    else
      w8 ? grid_items<64, 4, kStreamWaves>(a, p.row_groups, lds)
         : grid_items<64, 4, 4>(a, p.row_groups, lds);
  }
  __syncthreads();
  return SDE_OK;
}

}  // namespace sde
