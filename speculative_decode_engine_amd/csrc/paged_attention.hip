// Paged GQA decode / speculative-verify attention for gfx950 (wave64).
//
// Computes what cublas_attention_kernel (kernels.cu:904-940) computes with
// device_flash_attention_gqa (attention.h:21-127): for query m of a window,
// out[m][h] = softmax(q[m][h] . K[0..pos_base+m]^T * dph^-1/2) V, with query
// head h reading KV head h*nkv/nh, keys gathered through the block table.
//
// No MFMA: decode and small-k verify are GEMV-shaped and HBM-bound.  The
// "rows" of a KV head are its (query, head-in-group) pairs; a row group of up
// to four rows shares every K/V byte it loads.  The context of each (KV
// head, row group) is split into partitions, one 8-wave workgroup each
// (about one per CU); a single-partition context writes the normalised
// output directly, otherwise per-row partials go to the workspace and the
// last workgroup of a (KV head, row group) to finish -- found with one
// arrival counter per pair -- merges all partitions with a log-sum-exp
// combine in partition order, so the result does not depend on arrival
// order and one call is one launch.
//
// attn_stream_kernel: K and V stream from HBM straight into VGPRs in the
// coalesced load layout (lane = token slot x 16-byte feature chunk),
// software-pipelined a tile (32 tokens) ahead; logits are reduced across
// the lanes of a token with a transposing DPP butterfly that leaves each
// lane one (row, token pair), so the online softmax is a handful of scalar
// ops per lane; P.V dot2-accumulates fp16 probability pairs against
// byte-permuted V pairs.  Row groups of a larger verify window are separate
// workgroups reading the same K/V (the repeats are L2 hits).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdlib>

#include "sde_internal.hpp"

namespace sde {
namespace attn {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kTile = 32;  // tokens per tile
constexpr double kLog2e = 1.4426950408889634;

struct AttnArgs {
  const uint16_t* pool;
  const int32_t* table;  // this layer's block table
  const float* q;        // [M][nh*dph]
  float* out;            // [M][nh*dph]
  float* partials;       // [nkv][R][n_parts][dph+2] = (max, sum, acc[dph])
  uint32_t* counters;    // [nkv][row_groups] arrival counters, zero at rest
  int kv_dim;
  int bs;
  int nh;
  int G;         // query heads per KV head
  int R;         // rows per KV head = M * G (row = m*G + g)
  int pos_base;  // query m sees positions [0, pos_base+m]
  int L_max;     // pos_base + M
  int n_parts;
  int tiles_per_part;  // attn_stream_kernel: tiles per partition
  float qscale;  // log2(e) / sqrt(dph)
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                __builtin_bit_cast(half2_t, b), c, false);
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
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false); break;   // i^1
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false); break;   // i^2
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false); break;  // ror 4
    case 3: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false); break;  // ror 8
    default: r = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false); break; // i^7 in 8
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

typedef const __attribute__((address_space(4))) int32_t* const_table_t;

// The block table is read-only during the kernel: reading it through the
// constant address space turns the entries into scalar loads (lgkmcnt),
// which never wait behind outstanding tile loads (vmcnt).
__device__ __forceinline__ const_table_t const_table(const AttnArgs& a) {
  return (const_table_t)a.table;
}

// ---------------------------------------------------------------------------
// attn_stream_kernel: decode and short windows (<= kStreamMaxRows rows per
// wave).  K and V stream from HBM straight into VGPRs in the load layout --
// lane (slot sl, chunk c) holds features 8c..8c+7 of token j*SL + sl of load
// j -- software-pipelined across tiles: K of tile i+1 is issued before tile
// i's logits and V of tile i+1 before tile i's P.V, so each wave keeps a
// tile of loads in flight while it computes; no LDS holds K or V.
//  * Q.K: each lane takes dot2 products of its K chunk with the same chunk of
//    every q row; a transposing butterfly over the CH lanes of a token
//    leaves each lane the full logits of one (row, token pair);
//  * softmax: each token slot keeps its own online-softmax state (running
//    max and sum per row), so a tile needs no cross-slot traffic; the SL
//    states merge once, when the wave is done;
//  * P.V: the probability pair of loads 2j', 2j'+1 (fp16x2, broadcast from
//    its owner lane) dot2-accumulates against the byte-permuted V pairs,
//    fp32 accumulators.
// One workgroup of kStreamWaves waves per (partition, KV head, row group),
// about one workgroup per CU; the partition combine reads every partial in
// a single round trip.
// ---------------------------------------------------------------------------
constexpr int kStreamWaves = 8;
constexpr int kStreamMaxRows = 4;
constexpr int kStreamMaxParts = 64;

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

__device__ __forceinline__ float4 load_dev4(const float* p) {
  const float2 lo = load_dev2(p);
  const float2 hi = load_dev2(p + 2);
  return make_float4(lo.x, lo.y, hi.x, hi.y);
}

__device__ __forceinline__ uint4 ld16(const char* p) { return *reinterpret_cast<const uint4*>(p); }

// Physical block and in-block slot of the first token of each load group of
// tile ts (SL tokens per group, SL divides block_size).  Groups at or past
// L_max are pinned to token L_max-1 so every address stays on written data.
template <int NLD, int SL>
__device__ __forceinline__ void tile_groups(const AttnArgs& a, const_table_t table, int ts,
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
__device__ __forceinline__ void stream_load(const AttnArgs& a, const char* head_base, int ts,
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

// Lane roles of attn_stream_kernel.  Load role: lane = (slot sl, chunk c),
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
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false); break;
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false); break;
  }
  return __builtin_bit_cast(float, r);
}

// Value of lane n of this lane's 16-lane row (DPP row_newbcast:n).
__device__ __forceinline__ int row_bcast(int v, int n) {
  switch (n) {
    case 0: return __builtin_amdgcn_update_dpp(0, v, 0x150, 0xf, 0xf, false);
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0x151, 0xf, 0xf, false);
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x152, 0xf, 0xf, false);
    case 3: return __builtin_amdgcn_update_dpp(0, v, 0x153, 0xf, 0xf, false);
    case 4: return __builtin_amdgcn_update_dpp(0, v, 0x154, 0xf, 0xf, false);
    case 5: return __builtin_amdgcn_update_dpp(0, v, 0x155, 0xf, 0xf, false);
    case 6: return __builtin_amdgcn_update_dpp(0, v, 0x156, 0xf, 0xf, false);
    case 7: return __builtin_amdgcn_update_dpp(0, v, 0x157, 0xf, 0xf, false);
    case 8: return __builtin_amdgcn_update_dpp(0, v, 0x158, 0xf, 0xf, false);
    case 9: return __builtin_amdgcn_update_dpp(0, v, 0x159, 0xf, 0xf, false);
    case 10: return __builtin_amdgcn_update_dpp(0, v, 0x15A, 0xf, 0xf, false);
    case 11: return __builtin_amdgcn_update_dpp(0, v, 0x15B, 0xf, 0xf, false);
    case 12: return __builtin_amdgcn_update_dpp(0, v, 0x15C, 0xf, 0xf, false);
    case 13: return __builtin_amdgcn_update_dpp(0, v, 0x15D, 0xf, 0xf, false);
    case 14: return __builtin_amdgcn_update_dpp(0, v, 0x15E, 0xf, 0xf, false);
    default: return __builtin_amdgcn_update_dpp(0, v, 0x15F, 0xf, 0xf, false);
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
      float t = dot2(q4.x, k[j].x, 0.f);
      t = dot2(q4.y, k[j].y, t);
      t = dot2(q4.z, k[j].z, t);
      t = dot2(q4.w, k[j].w, t);
      x[r * NLD + j] = t;
    }
  }
  // Transposing butterfly: step kk keeps the half of x whose top index bit
  // equals bit S-1-kk of c.
#pragma unroll
  for (int kk = 0; kk < T; kk++) {
    const bool f = (c >> (S - 1 - kk)) & 1;
    const int h = NV >> (kk + 1);
#pragma unroll
    for (int i = 0; i < (NV >> 1); i++) {
      if (i < h) {
        const float a = x[i], b = x[i + h];
        const float send = f ? a : b;
        const float keep = f ? b : a;
        x[i] = keep + bfly<CH>(send, kk);
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

// Partition combine of attn_stream_kernel, run by the last workgroup of a
// (KV head, row group): thread (row r, float4 column c4, quarter sub) loads
// (max, sum, acc[c4]) of partitions sub, sub+4, ... -- every partial in one
// round trip, no LDS -- weights them by exp2(m_p - max) and the four
// quarters of a (row, column) (adjacent lanes) reduce through DPP in a fixed
// order, so the result does not depend on arrival order.
template <int DPH, int RPW>
__device__ __forceinline__ void stream_combine(const AttnArgs& a, int kvh, int r0, int nrows) {
  constexpr int C4 = DPH / 4;
  constexpr int SUB = 4;
  constexpr int PMAX = kStreamMaxParts / SUB;
  static_assert(RPW * C4 * SUB <= 64 * kStreamWaves, "one thread per (row, column, quarter)");
  const int tid = threadIdx.x;
  const int sub = tid & (SUB - 1);
  const int col4 = (tid / SUB) % C4;
  const int r = tid / (SUB * C4);  // uniform per wave
  if (r >= nrows) return;
  const int P = a.n_parts;
  const size_t row = (size_t)kvh * a.R + r0 + r;
  const float* ml = a.partials + row * P * 2;
  const float* accp = a.partials + (size_t)gridDim.y * a.R * P * 2 + row * P * DPH + 4 * col4;
  float2 e[PMAX];
  float4 v[PMAX];
#pragma unroll
  for (int i = 0; i < PMAX; i++) {
    const int p = sub + i * SUB;
    e[i] = make_float2(-INFINITY, 0.f);
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p < P) {
      e[i] = load_dev2(ml + (size_t)p * 2);
      v[i] = load_dev4(accp + (size_t)p * DPH);
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
    o.x += w * v[i].x;
    o.y += w * v[i].y;
    o.z += w * v[i].z;
    o.w += w * v[i].w;
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
    // attention.h:120-126: normalise unless the sum is tiny or not finite.
    const float inv = (l > 1e-20f && isfinite(l)) ? 1.f / l : 0.f;
    const int gr = r0 + r;
    const int m = gr / a.G;
    const int h = kvh * a.G + (gr - m * a.G);
    float2* dst = reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH +
                                            4 * col4);
    dst[0] = make_float2(o.x * inv, o.y * inv);
    dst[1] = make_float2(o.z * inv, o.w * inv);
  }
}

template <int DPH, int RPW, int CHUNK>
__global__ __launch_bounds__(64 * kStreamWaves) void attn_stream_kernel(AttnArgs a) {
  static_assert(DPH == 64 || DPH == 128, "head_dim");
  static_assert(RPW == 2 || RPW == 4, "rows per wave");
  constexpr int CH = DPH / 8;
  constexpr int SL = 64 / CH;
  constexpr int NLD = kTile / SL;
  constexpr int REC = DPH + 2;
  // Per-wave records (max, sum, acc[DPH]) of every row.
  __shared__ __attribute__((aligned(16))) float s_buf[kStreamWaves * RPW * REC];
  __shared__ int s_last;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int sl = lane / CH;
  const int c = lane % CH;
  const int part = blockIdx.x;
  const int kvh = blockIdx.y;
  const int r0 = blockIdx.z * RPW;
  const int nrows = min(RPW, a.R - r0);
  const int n_tiles = (a.L_max + kTile - 1) / kTile;
  const int tb = part * a.tiles_per_part;
  const int te = min(n_tiles, tb + a.tiles_per_part);

  using Sh = StreamShape<DPH, RPW>;
  // This lane's (row, pair) in the transposed layout, and its redundancy.
  const int prefix = c >> (Sh::S - Sh::T);
  const int my_r = prefix >> (Sh::T - Sh::RB);
  const int my_jp = prefix & ((1 << (Sh::T - Sh::RB)) - 1);
  const bool redundant = (c & ((1 << (Sh::S - Sh::T)) - 1)) != 0;

  // This lane's q chunk (features 8c..8c+7) of every row, loaded before any
  // K/V load so that waiting for it never waits for tile data; it is scaled
  // into the exp2 domain and rounded to fp16 pairs once the first tile's
  // loads are in flight.
  float2 q_raw[RPW][4];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int gr = min(r0 + r, a.R - 1);  // rows past nrows: zeroed below
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

  const const_table_t table = const_table(a);
  const char* head_base = reinterpret_cast<const char*>(a.pool) + (size_t)kvh * DPH * 2u;
  const uint32_t lane_off = (uint32_t)sl * 2u * (uint32_t)a.kv_dim + 16u * c;
  const uint32_t chunk_off = 16u * c;
  // Wave w takes tiles tb+w, tb+w+W, ... in chunks of CHUNK tiles.  Within
  // a chunk the code is straight-line (unrolled at compile time): K of tile
  // i+1 is issued before tile i's logits and V of tile i+1 before tile i's
  // P.V, so a tile of loads stays in flight while the wave computes, and the
  // compiler's waits before each use are exact (no loop-carried buffers,
  // no register copies of in-flight data).  Chunk slots past the wave's
  // last tile re-read that tile (an L2 hit) and are fully masked.
  constexpr int W = kStreamWaves;
  const int first = tb + wave;
  if (first < te) {
    const int last = first + ((te - 1 - first) / W) * W;
    uint4 qr[RPW];
    for (int c0 = first; c0 < te; c0 += CHUNK * W) {
      uint4 kbuf[2][NLD], vbuf[2][NLD];
      int blk[2][NLD], slot[2][NLD];
      float al;
      uint32_t pk;
      tile_groups<NLD, SL>(a, table, min(c0, last) * kTile, blk[0], slot[0]);
      stream_load<DPH>(a, head_base, min(c0, last) * kTile, sl, lane_off, chunk_off, false,
                       blk[0], slot[0], kbuf[0]);
      stream_load<DPH>(a, head_base, min(c0, last) * kTile, sl, lane_off, chunk_off, true,
                       blk[0], slot[0], vbuf[0]);
      if (CHUNK > 1)
        tile_groups<NLD, SL>(a, table, min(c0 + W, last) * kTile, blk[1], slot[1]);
#pragma unroll
      for (int i = 0; i < CHUNK; i++) {
        const int t = c0 + i * W;
        const int b = i & 1, nb = b ^ 1;
        const int tn = min(t + W, last);
        if (i + 1 < CHUNK)
          stream_load<DPH>(a, head_base, tn * kTile, sl, lane_off, chunk_off, false, blk[nb],
                           slot[nb], kbuf[nb]);
        if (i == 0) {
#pragma unroll
          for (int r = 0; r < RPW; r++) {
            const float sc = r < nrows ? a.qscale : 0.f;
            qr[r] = make_uint4(pack_h2(q_raw[r][0].x * sc, q_raw[r][0].y * sc),
                               pack_h2(q_raw[r][1].x * sc, q_raw[r][1].y * sc),
                               pack_h2(q_raw[r][2].x * sc, q_raw[r][2].y * sc),
                               pack_h2(q_raw[r][3].x * sc, q_raw[r][3].y * sc));
          }
        }
        // A slot past the wave's last tile: every token masked (no-op).
        const int ts_mask = t <= last ? t * kTile : INT_MAX / 2;
        stream_qk<DPH, RPW, 0>(ts_mask, sl, c, min_lim, my_lim, my_jp, qr, kbuf[b], m_run, l_run,
                               al, pk);
        if (i + 1 < CHUNK) {
          stream_load<DPH>(a, head_base, tn * kTile, sl, lane_off, chunk_off, true, blk[nb],
                           slot[nb], vbuf[nb]);
          if (i + 2 < CHUNK)
            tile_groups<NLD, SL>(a, table, min(t + 2 * W, last) * kTile, blk[b], slot[b]);
        }
        stream_pv<DPH, RPW, 0>(sl, al, pk, vbuf[b], acc);
      }
    }
  }

  // ---- merge the SL slot states of this wave; record per row ------------
  // l of (row, slot): sum over the row's token-pair owners (redundant lanes
  // hold copies and contribute 0).
  float lsum = redundant ? 0.f : l_run;
#pragma unroll
  for (int kk = Sh::RB; kk < Sh::S; kk++) lsum += bfly<CH>(lsum, kk);
  const bool odd_slot = sl & 1;
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const float m_s = from_owner_f<DPH, RPW>(m_run, r, 0, odd_slot);
    const float l_s = from_owner_f<DPH, RPW>(lsum, r, 0, odd_slot);
    const float mx = slot_max<DPH>(m_s);
    const float f = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_s - mx);
    const float l = slot_sum<DPH>(l_s * f);
#pragma unroll
    for (int e = 0; e < 8; e++) acc[r][e] = slot_sum<DPH>(acc[r][e] * f);
    float* rec = s_buf + (wave * RPW + r) * REC;
    if (lane == 0) {
      rec[0] = mx;
      rec[1] = l;
    }
    if (sl == 0) {
      float2* dst = reinterpret_cast<float2*>(rec + 2 + 8 * c);
      dst[0] = make_float2(acc[r][0], acc[r][1]);
      dst[1] = make_float2(acc[r][2], acc[r][3]);
      dst[2] = make_float2(acc[r][4], acc[r][5]);
      dst[3] = make_float2(acc[r][6], acc[r][7]);
    }
  }
  __syncthreads();

  // ---- workgroup merge: thread (row, feature pair) over the waves --------
  constexpr int DP = DPH / 2;
  if ((int)threadIdx.x < nrows * DP) {
    const int r = threadIdx.x / DP;
    const int dcol = 2 * (threadIdx.x - r * DP);
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kStreamWaves; w++) mx = fmaxf(mx, s_buf[(w * RPW + r) * REC]);
    float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < kStreamWaves; w++) {
      const float* rec = s_buf + (w * RPW + r) * REC;
      const float wt = rec[0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(rec[0] - mx);
      l += rec[1] * wt;
      const float2 x = *reinterpret_cast<const float2*>(rec + 2 + dcol);
      o0 += x.x * wt;
      o1 += x.y * wt;
    }
    const int gr = r0 + r;
    if (a.n_parts == 1) {
      // attention.h:120-126: normalise unless the sum is tiny or not finite.
      const float inv = (l > 1e-20f && isfinite(l)) ? 1.f / l : 0.f;
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      *reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH + dcol) =
          make_float2(o0 * inv, o1 * inv);
    } else {
      const size_t pr = ((size_t)kvh * a.R + gr) * a.n_parts + part;
      float* acc_base = a.partials + (size_t)gridDim.y * a.R * a.n_parts * 2;
      store_dev2(acc_base + pr * DPH + dcol, o0, o1);
      if (dcol == 0) store_dev2(a.partials + pr * 2, mx, l);
    }
  }
  if (a.n_parts == 1) return;

  // ---- the last workgroup of (KV head, row group) combines --------------
  // Partials are device-scope stores; waiting for them (vmcnt) before the
  // arrival increment orders them before it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* ctr = a.counters + (size_t)kvh * gridDim.z + blockIdx.z;
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)(a.n_parts - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  stream_combine<DPH, RPW>(a, kvh, r0, nrows);
}

}  // namespace attn
}  // namespace sde

namespace {

using namespace sde::attn;

struct Plan {
  int rpw;             // rows per wave (2 or kStreamMaxRows)
  int row_groups;
  int chunk;           // tiles per unrolled chunk (1, 2 or 4)
  int tiles_per_part;  // tiles per partition (workgroup)
  int n_parts;
};

int rows_per_wave(int R) { return R <= 2 ? 2 : kStreamMaxRows; }

// Each wave takes its tiles in chunks of `chunk` (1, 2 or 4, a compile-time
// unroll).  The largest chunk that still gives at least one workgroup per CU
// is used; past kStreamMaxParts partitions per (KV head, row group) the
// waves take several chunks.
Plan make_plan(int L_max, int nkv, int R, int n_cus) {
  Plan p;
  p.rpw = rows_per_wave(R);
  p.row_groups = (R + p.rpw - 1) / p.rpw;
  const int n_tiles = (L_max + kTile - 1) / kTile;
  const int64_t units = (int64_t)nkv * p.row_groups;
  p.chunk = 1;
  for (int ch : {4, 2}) {
    const int per = kStreamWaves * ch;
    if ((int64_t)((n_tiles + per - 1) / per) * units >= n_cus) {
      p.chunk = ch;
      break;
    }
  }
  const int per_chunk = kStreamWaves * p.chunk;
  const int chunks = (n_tiles + per_chunk - 1) / per_chunk;
  const int reps = (chunks + kStreamMaxParts - 1) / kStreamMaxParts;
  p.tiles_per_part = per_chunk * reps;
  p.n_parts = (n_tiles + p.tiles_per_part - 1) / p.tiles_per_part;
  return p;
}

// Upper bound of make_plan(L).n_parts over every L <= max_total_len: a
// partition holds at least kStreamWaves tiles and there are at most
// kStreamMaxParts of them.
int parts_bound(int max_total_len) {
  const int n_tiles = (max_total_len + kTile - 1) / kTile;
  const int by_len = (n_tiles + kStreamWaves - 1) / kStreamWaves;
  return by_len < kStreamMaxParts ? by_len : kStreamMaxParts;
}

size_t partial_bytes(int nkv, int R, int n_parts, int dph) {
  return n_parts > 1 ? (size_t)nkv * R * n_parts * (size_t)(dph + 2) * sizeof(float) : 0;
}

template <int DPH>
int launch(const Plan& p, const AttnArgs& a, int nkv, hipStream_t s) {
  const dim3 grid(p.n_parts, nkv, p.row_groups);
  const dim3 block(64 * kStreamWaves);
#define SDE_STREAM(R, C)                                     \
  if (p.rpw == R && p.chunk == C) {                          \
    attn_stream_kernel<DPH, R, C><<<grid, block, 0, s>>>(a); \
    return sde::launch_status();                             \
  }
  SDE_STREAM(2, 1)
  SDE_STREAM(2, 2)
  SDE_STREAM(2, 4)
  SDE_STREAM(4, 1)
  SDE_STREAM(4, 2)
  SDE_STREAM(4, 4)
#undef SDE_STREAM
  return SDE_ERR_UNSUPPORTED;
}

int check_attention(const sde_kv_cache* c, int layer, const float* d_q,
                    const float* d_out, int nh, int nkv, int dph, int pos_base,
                    int n_queries) {
  if (!c || !d_q || !d_out) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= c->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  if (nh < 1 || nkv < 1 || dph < 1 || nh % nkv != 0) return SDE_ERR_INVALID_ARGUMENT;
  if ((int64_t)nkv * dph != c->cfg.kv_dim) return SDE_ERR_INVALID_ARGUMENT;
  if (pos_base < 0 || n_queries < 1 || n_queries > 4096) return SDE_ERR_INVALID_ARGUMENT;
  if (dph != 64 && dph != 128) return SDE_ERR_UNSUPPORTED;
  if (c->cfg.block_size % 8 != 0) return SDE_ERR_UNSUPPORTED;
  if ((((uintptr_t)d_q) & 7u) != 0 || (((uintptr_t)d_out) & 7u) != 0)
    return SDE_ERR_INVALID_ARGUMENT;
  if ((int64_t)pos_base + n_queries > sde::mapped_tokens(c, layer)) return SDE_ERR_CAPACITY;
  return SDE_OK;
}

}  // namespace

extern "C" {

size_t sde_paged_attention_workspace_size(const sde_kv_cache* cache, int nh,
                                          int nkv, int dph, int n_queries,
                                          int max_total_len) {
  if (!cache || nh < 1 || nkv < 1 || nh % nkv != 0 || n_queries < 1 || max_total_len < 1)
    return 0;
  const int R = n_queries * (nh / nkv);
  return partial_bytes(nkv, R, parts_bound(max_total_len), dph);
}

int sde_paged_attention(sde_kv_cache* cache, int layer, const float* d_q,
                        float* d_out, int nh, int nkv, int dph, int pos_base,
                        int n_queries, void* d_workspace, size_t workspace_bytes,
                        sde_stream_t stream) {
  int st = check_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base, n_queries);
  if (st != SDE_OK) return st;
  sde::DeviceGuard guard(cache->device);
  if (!guard.ok()) return SDE_ERR_HIP;

  const int G = nh / nkv;
  const int R = n_queries * G;
  const int L_max = pos_base + n_queries;
  const Plan plan = make_plan(L_max, nkv, R, cache->n_cus);
  if ((int64_t)nkv * plan.row_groups > sde::kMaxAttnCounters) return SDE_ERR_UNSUPPORTED;
  const size_t need = partial_bytes(nkv, R, plan.n_parts, dph);
  float* partials = nullptr;
  if (need > 0) {
    if (d_workspace) {
      if (workspace_bytes < need) return SDE_ERR_WORKSPACE;
      partials = static_cast<float*>(d_workspace);
    } else {
      if (cache->workspace_bytes < need) {
        // Grow the cache-owned workspace (not for use under graph capture).
        if (cache->workspace) {
          if (hipDeviceSynchronize() != hipSuccess) return SDE_ERR_HIP;
          (void)hipFree(cache->workspace);
          cache->workspace = nullptr;
          cache->workspace_bytes = 0;
        }
        if (hipMalloc(&cache->workspace, need) != hipSuccess) return SDE_ERR_HIP;
        cache->workspace_bytes = need;
      }
      partials = static_cast<float*>(cache->workspace);
    }
  }

  AttnArgs a;
  a.pool = cache->pool;
  a.table = sde::layer_table(cache, layer);
  a.q = d_q;
  a.out = d_out;
  a.partials = partials;
  a.counters = cache->d_counters;
  a.kv_dim = cache->cfg.kv_dim;
  a.bs = cache->cfg.block_size;
  a.nh = nh;
  a.G = G;
  a.R = R;
  a.pos_base = pos_base;
  a.L_max = L_max;
  a.n_parts = plan.n_parts;
  a.tiles_per_part = plan.tiles_per_part;
  a.qscale = (float)(kLog2e / std::sqrt((double)dph));

  const hipStream_t s = (hipStream_t)stream;
  return dph == 128 ? launch<128>(plan, a, nkv, s) : launch<64>(plan, a, nkv, s);
}

int sde_attention_dispatch(int attn_type, sde_kv_cache* cache, int layer,
                           const float* d_q, float* d_out, int nh, int nkv,
                           int dph, int pos_base, int n_queries,
                           void* d_workspace, size_t workspace_bytes,
                           sde_stream_t stream) {
  if (attn_type != SDE_ATTN_SOFTMAX) return SDE_ERR_UNSUPPORTED;
  return sde_paged_attention(cache, layer, d_q, d_out, nh, nkv, dph, pos_base,
                             n_queries, d_workspace, workspace_bytes, stream);
}

}  // extern "C"
