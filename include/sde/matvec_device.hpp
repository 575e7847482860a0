// Output-projection GEMV (Wo) on gfx950: out[m][c] (+)= sum_r x[m][r] * W[r][c]
// with fp16 weights W [d_in][d_out] (row-major, the reference's layout,
// utils.h:410-416 and model.h:19) and fp32 activations and accumulation.
//
//   device_matvec_partial        utils.h:417-433
//   device_matvec_partial_accum  utils.h:437-452 (Wo / W_down in
//                                coop_layer_forward, kernels.cu:2742-2747)
//   device_matvec_batched        utils.h:248-280 (the verify window's Wo,
//                                model.cu:717, 892)
//   device_matvec_grid           all blocks of a persistent kernel share one
//                                projection (the step after attention)
//
// Layout of the work (libsde_paged's sde_matvec and device_matvec_grid):
// the columns are cut into tiles of kCols = 256 (32 lanes x 8 fp16: a
// wave's 16-byte loads cover two rows of 512 B, lane groups of 32 taking
// the two row phases) and the rows into `splits` ranges, one workgroup per
// (column tile, row range).  Its waves stream rows of the range, two
// batches of eight 16-byte loads in flight per lane; x[m][r] is
// wave-uniform per row phase (scalar loads).  The waves' sums meet in
// LDS; each row range publishes a partial per column, and the last
// workgroup of a column tile to finish (one arrival counter per tile) adds
// the partials in row-range order, so the result does not depend on
// arrival order.  HBM-bound: d_in * d_out * 2 bytes of weights per call.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "sde_paged_kv.h"
#include "sde/wave_uniform.hpp"

namespace sde {
namespace mv {

constexpr int kRowPhases = 2;   // rows per wave load (lane groups of 64/kRowPhases)
constexpr int kLanesPerRow = 64 / kRowPhases;
constexpr int kCols = 8 * kLanesPerRow;  // columns per tile: 8 fp16 per lane
constexpr int kUnroll = 8;      // rows in flight per wave
constexpr int kMaxSplit = 64;   // row ranges per column tile
constexpr int kMaxRows = 16;    // rows of x (the verify window is <= 9)
constexpr int kChunkRows = 8;   // rows of x per pass (unrolled in registers)

struct MvArgs {
  const float* x;       // [M][d_in]
  const uint16_t* W;    // [d_in][d_out] fp16 bits
  float* out;           // [M][d_out]
  float* partials;      // [splits][M][d_out]
  uint32_t* counters;   // [col_tiles] arrival counters, zero at rest
  int d_in;
  int d_out;
  int M;
  int splits;
  int rows_per_split;
  int accumulate;       // out += (1) or out = (0)
};

struct MvPlan {
  int col_tiles;
  int splits;
  int rows_per_split;
};

// Row ranges so that col_tiles * splits fills `blocks` workgroups, each wave
// keeping at least kUnroll rows (one full batch of loads in flight).
// Rows of x of a pass as unrolled (every count 1..kChunkRows has its own
// instantiation: the multiply-adds are the streaming loop's issue cost, so
// a 5-row verify window must not pay for 8).
__host__ __device__ inline int mv_row_bucket(int rows) {
  return rows <= 1 ? 1 : rows >= kChunkRows ? kChunkRows : rows;
}

// splits <= 4 * (kMaxSplit / 4 / bucket): the combining workgroup then holds
// every partial of its columns in registers (one round trip; four quarters
// of kMaxSplit / 4 / bucket loads per row of x).
__host__ __device__ inline MvPlan mv_plan(int d_in, int d_out, int blocks, int waves, int M) {
  MvPlan p;
  p.col_tiles = (d_out + kCols - 1) / kCols;
  int s = blocks / p.col_tiles;
  const int by_rows = d_in / (waves * kUnroll * kRowPhases);
  if (s > by_rows) s = by_rows;
  const int cap = 4 * (kMaxSplit / 4 / mv_row_bucket(M < kChunkRows ? M : kChunkRows));
  if (s > cap) s = cap;
  if (s < 1) s = 1;
  p.rows_per_split = (d_in + s - 1) / s;
  p.splits = (d_in + p.rows_per_split - 1) / p.rows_per_split;
  return p;
}

// Rows of x are taken kChunkRows at a time; each pass has its own arrival
// counters and partials.  Bytes of the workspace (counters, then partials)
// for any call with these shapes and at most kMaxSplit row ranges.
__host__ __device__ inline int mv_passes(int M) { return (M + kChunkRows - 1) / kChunkRows; }
__host__ __device__ inline int mv_pass_rows(int M) { return M < kChunkRows ? M : kChunkRows; }
__host__ __device__ inline size_t mv_counter_bytes(int d_out, int M) {
  return ((size_t)mv_passes(M) * ((d_out + kCols - 1) / kCols) * 4 + 255) / 256 * 256;
}
__host__ __device__ inline size_t mv_pass_partial_floats(int d_out, int M) {
  return (size_t)kMaxSplit * mv_pass_rows(M) * d_out;
}
__host__ __device__ inline size_t mv_workspace_size(int d_in, int d_out, int M) {
  (void)d_in;
  return mv_counter_bytes(d_out, M) +
         (size_t)mv_passes(M) * mv_pass_partial_floats(d_out, M) * sizeof(float);
}

// The arguments of pass j (rows 8j .. 8j+7 of x) of a call whose whole-call
// arguments are `a` (a.partials / a.counters at the workspace's areas).
__host__ __device__ inline MvArgs mv_pass(const MvArgs& a, int j) {
  MvArgs p = a;
  p.x = a.x + (size_t)j * kChunkRows * a.d_in;
  p.out = a.out + (size_t)j * kChunkRows * a.d_out;
  p.M = a.M - j * kChunkRows < kChunkRows ? a.M - j * kChunkRows : kChunkRows;
  p.counters = a.counters ? a.counters + (size_t)j * ((a.d_out + kCols - 1) / kCols) : nullptr;
  p.partials = a.partials ? a.partials + (size_t)j * mv_pass_partial_floats(a.d_out, a.M)
                          : nullptr;
  return p;
}

// 16-byte device-scope (sc1) store / load of the partials through a raw
// buffer over the partial area (`bytes` long): written through to the
// device coherence point and read past other XCDs' L2, as agent-scope
// relaxed atomics are.
__device__ __forceinline__ void mv_store_dev16(float* base, uint32_t bytes, uint32_t off,
                                               float4 v) {
  constexpr int kSc1 = 16;
  constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer, 32-bit data format
  typedef float f4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(wave_uniform(base), 0, (int)wave_uniform(bytes),
                                        kRsrcWord3);
  const f4v d = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, d), r, off, 0, kSc1);
}
__device__ __forceinline__ float4 mv_load_dev16(const float* base, uint32_t bytes, uint32_t off) {
  constexpr int kSc1 = 16;
  constexpr int kRsrcWord3 = 0x00020000;
  typedef float f4v __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(wave_uniform(base)), 0,
                                        (int)wave_uniform(bytes), kRsrcWord3);
  const f4v v = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
  return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float h_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// The row range [r0, r1) of W as a raw buffer.  A wave's load covers
// kRowPhases consecutive rows (lane group rp = lane / kLanesPerRow takes row
// rb + rp); the whole byte offset is the lane's 32-bit VGPR offset, so rows
// past r1 fall outside the buffer and load zeros.
struct MvRows {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t lane_off;   // the lane's column chunk and row phase, bytes
  uint32_t row_bytes;  // d_out * 2
  int r0, r1;
};

__device__ __forceinline__ MvRows mv_rows(const MvArgs& a, int r0, int r1, int colc, int rp) {
  constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer, 32-bit data format
  MvRows t;
  t.row_bytes = (uint32_t)a.d_out * 2u;
  t.rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(wave_uniform(a.W + (size_t)r0 * a.d_out)), 0,
      (int)wave_uniform((uint32_t)(r1 - r0) * t.row_bytes), kRsrcWord3);
  t.lane_off = (uint32_t)colc * 2u + (uint32_t)rp * t.row_bytes;
  t.r0 = r0;
  t.r1 = r1;
  return t;
}

// The U row blocks rb(u) = r + u * WAVES * kRowPhases of a batch (r the
// wave's first row block): the lane's 16-byte chunk of row rb(u) + rp.
template <int WAVES, int U>
__device__ __forceinline__ void mv_load_batch(const MvRows& t, int r, uint4 (&w)[U]) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t rb = (uint32_t)(r + u * WAVES * kRowPhases - t.r0);
    const u4v v = __builtin_bit_cast(
        u4v, __builtin_amdgcn_raw_buffer_load_b128(t.rsrc, t.lane_off + rb * t.row_bytes, 0, 0));
    w[u] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// acc[m][j] += x[m][row] * w[row][j] for the lane's rows of the batch
// (row rb(u) + rp; rows at or past r1 weigh 0).  When FULL every row of the
// batch is below r1.  x of the batch's rows is read with scalar loads (the
// row blocks are wave-uniform) and picked per lane group.
// x of the lane's row: from xl (the row range staged in LDS as
// [m][row - r0], `rows` long) when given, else a scalar load per row phase
// picked per lane group (a single row of x: the whole batch's scalars are
// loaded ahead).
template <int MB, int WAVES, int U, bool FULL>
__device__ __forceinline__ void mv_fma_batch(const struct MvArgs& a, int r, int r0, int r1,
                                             int rp, const float* xl, int rows,
                                             const uint4 (&w)[U], float (&acc)[MB][8]) {
  float xs[U][kRowPhases];
  if (MB == 1 && !xl) {
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int p = 0; p < kRowPhases; p++)
        xs[u][p] = a.x[min(r + u * WAVES * kRowPhases + p, a.d_in - 1)];
  }
  // LDS-staged x: the values of UP row blocks are read up front, so their
  // LDS round trips overlap instead of sitting in the multiply-add chain
  // (UP = U unless that would need more than 48 registers).
  constexpr int UP = MB * U <= 48 ? U : U / 2;
  float xpre[UP][MB];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int rb = r + u * WAVES * kRowPhases;
    if (xl && u % UP == 0) {
#pragma unroll
      for (int v = 0; v < UP; v++)
#pragma unroll
        for (int m = 0; m < MB; m++)
          xpre[v][m] = xl[m * rows + min(rb + v * WAVES * kRowPhases + rp, r1 - 1) - r0];
    }
    const bool live = FULL || rb + rp < r1;
    const uint32_t wd[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
    for (int m = 0; m < MB; m++) {
      if (m < a.M) {
        float xv;
        if (xl) {
          xv = xpre[u % UP][m];
        } else if (MB == 1) {
          xv = xs[u][0];
#pragma unroll
          for (int p = 1; p < kRowPhases; p++) xv = rp == p ? xs[u][p] : xv;
        } else {
          xv = a.x[(size_t)m * a.d_in + min(rb + rp, r1 - 1)];
        }
        if (!FULL) xv = live ? xv : 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          acc[m][2 * k] = fmaf(xv, h_lo(wd[k]), acc[m][2 * k]);
          acc[m][2 * k + 1] = fmaf(xv, h_hi(wd[k]), acc[m][2 * k + 1]);
        }
      }
    }
  }
}

// Sum over the row phases of a wave (lane groups kLanesPerRow apart): every
// lane gets the total of its column chunk.
__device__ __forceinline__ float mv_phase_sum(float v) {
  if constexpr (kRowPhases >= 4) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v),
                                                    __builtin_bit_cast(int, v), false, false);
    v = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
  }
  if constexpr (kRowPhases >= 2) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v),
                                                    __builtin_bit_cast(int, v), false, false);
    v = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
  }
  return v;
}

// out[m][c..c+3] = v (+ out when accumulating); out may be 4-byte aligned.
__device__ __forceinline__ void mv_write_out(const struct MvArgs& a, int m, int c, float4 v) {
  float* o = a.out + (size_t)m * a.d_out + c;
  if (a.accumulate) {
    v.x += o[0];
    v.y += o[1];
    v.z += o[2];
    v.w += o[3];
  }
  o[0] = v.x;
  o[1] = v.y;
  o[2] = v.z;
  o[3] = v.w;
}

// LDS of one workgroup item: the waves' column sums and the last-arrival flag.
constexpr int kXStage = 4096;  // floats of x staged per workgroup item

template <int WAVES>
struct MvLds {
  float red[WAVES * kCols] __attribute__((aligned(16)));
  float xs[kXStage];
  int last;
};

// ---- matrix-core form for three or more rows of x ------------------------
//
// out^T[c][m] += W^T[c][r] . x^T[r][m] with v_mfma_f32_16x16x16_f16: each
// wave stores a batch of its loads (16 rows of W x the tile's 256 columns,
// in the load layout) into 8 KiB of its own LDS, with the 16-byte units of
// row r at u ^ (r % 16), and reads it back transposed with
// ds_read_b64_tr_b16: for column block cb, lane l (group g = l / 16, L =
// l % 16) addresses row 4g + L/4, columns 16cb + 4(L%4) .. +3, and receives
// column 16cb + L of rows 4g .. 4g+3 -- the A operand (i = column, k = row).
// B = x^T: lane l holds x[l % 16][rows 4g .. 4g+3] as fp16 hi + lo parts
// (two MFMAs, so the products carry x to ~2^-22 relative; the VALU form's
// fp32 multiply-adds are exact products).  D leaves lane l columns 16cb +
// 4g .. 4g+3 of row l % 16 of x.  Rows of a batch at or past the range end
// load zeros (the raw buffer) and take x = 0.  Per batch and wave: 16 LDS
// stores, 16 transposed reads and 32 MFMA, where the VALU form spends 8
// multiply-adds per row of x and loaded 16 bytes.
typedef _Float16 mv_h4 __attribute__((ext_vector_type(4)));
typedef float mv_f4 __attribute__((ext_vector_type(4)));
typedef short mv_s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) mv_s4 mv_lds_s4;
constexpr int kStageRows = kUnroll * kRowPhases;
constexpr int kStageBytes = kStageRows * kCols * 2;
constexpr int kColBlocks = kCols / 16;
// The VALU form's LDS plus every wave's W staging area (which the
// epilogue reuses for the rows' sums).
template <int WAVES>
struct MvMfmaLds {
  MvLds<WAVES> base;
  uint4 wst[WAVES][kStageBytes / 16];
  float xmax[WAVES][kMaxRows];  // per wave: max |x| of each row over the item's range
  float xscale[kMaxRows];       // per row of x: the power-of-two scale (1 in fp16 range)
};

// Per row of x, a power of two s with max |x| * s < 2^14 over the item's
// rows [r0, r1) (s = 1 when x already fits, and for non-finite x, which
// then propagates as in fp32), so the fp16 hi + lo split below never
// overflows; the sums are multiplied by 1/s, exactly, before they leave
// the item.  Scaling by a power of two commutes with every fp16 and fp32
// rounding here, so the result equals the unscaled computation's wherever
// that one is finite.  Every thread calls it; ends with a barrier.
template <int WAVES>
__device__ __forceinline__ void mv_row_scales(const MvArgs& a, const float* xl, int xrows,
                                              int r0, int r1, MvMfmaLds<WAVES>& L) {
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  for (int m = 0; m < a.M; m++) {
    float mx = 0.f;
    if (wave < WAVES)
      for (int i = wave * 64 + lane; i < xrows; i += WAVES * 64)
        mx = fmaxf(mx, fabsf(xl ? xl[m * xrows + i] : a.x[(size_t)m * a.d_in + r0 + i]));
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (wave < WAVES && lane == 0) L.xmax[wave][m] = mx;
  }
  __syncthreads();
  if ((int)threadIdx.x < a.M) {
    float mx = 0.f;
    for (int w = 0; w < WAVES; w++) mx = fmaxf(mx, L.xmax[w][threadIdx.x]);
    float sc = 1.f;
    if (mx >= 16384.f && mx <= 3.0e38f) {  // (finite and past the fp16-safe range)
      int e;
      (void)frexpf(mx, &e);          // mx < 2^e
      sc = ldexpf(1.f, 14 - e);      // mx * sc < 2^14
    }
    L.xscale[threadIdx.x] = sc;
  }
  __syncthreads();
}
__device__ __forceinline__ int mv_staged(int r, int u) { return r * (kCols * 2) + 16 * (u ^ (r & 15)); }
template <int WAVES>
__device__ __forceinline__ void mv_x_operand(const MvArgs& a, const float* xl, int xrows, int r0,
                                             int r1, int rbase, int lane, float sc, mv_h4& xh,
                                             mv_h4& xo) {
  const int m = lane & 15, g = lane >> 4;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int lr = 4 * g + q;
    const int row = rbase + (lr >> 1) * WAVES * kRowPhases + (lr & 1);
    float v = 0.f;
    if (m < a.M && row < r1) v = (xl ? xl[m * xrows + row - r0] : a.x[(size_t)m * a.d_in + row]) * sc;
    asm("" : "+v"(v));  // rounded once: hi = fp16(v), lo = fp16(v - hi)
    const _Float16 h = (_Float16)v;
    xh[q] = h;
    xo[q] = (_Float16)(v - (float)h);
  }
}
template <int U>
__device__ __forceinline__ void mv_stage(char* st, int rp, int lc, const uint4 (&w)[U]) {
#pragma unroll
  for (int u = 0; u < U; u++) *reinterpret_cast<uint4*>(st + mv_staged(2 * u + rp, lc)) = w[u];
}
__device__ __forceinline__ void mv_mfma_batch(const char* st, int lane, mv_h4 xh, mv_h4 xo,
                                              mv_f4 (&c)[kColBlocks]) {
  const int L = lane & 15, g = lane >> 4;
  const int row = 4 * g + (L >> 2);
  const int u0 = (L & 3) >> 1, sub = 8 * (L & 1);
#pragma unroll
  for (int cb = 0; cb < kColBlocks; cb++) {
    const mv_s4 s = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (mv_lds_s4*)(st + mv_staged(row, 2 * cb + u0) + sub));
    const mv_h4 w = __builtin_bit_cast(mv_h4, s);
    c[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(w, xh, c[cb], 0, 0, 0);
    c[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(w, xo, c[cb], 0, 0, 0);
  }
}

// (column tile ct, row range ks) on the calling workgroup; every thread
// calls it.  MB >= a.M rows of x are unrolled; waves at or past WAVES idle.
template <int MB, int WAVES, bool MFMA = false, class Lds>
__device__ __forceinline__ void mv_item(const MvArgs& a, int ct, int ks, Lds& L) {
  MvLds<WAVES>* lds_p;
  if constexpr (MFMA)
    lds_p = &L.base;
  else
    lds_p = &L;
  MvLds<WAVES>& lds = *lds_p;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int rp = lane / kLanesPerRow;  // row phase
  const int lc = lane % kLanesPerRow;  // 16-byte column chunk
  const int col = ct * kCols + lc * 8;
  // Lanes past d_out load the tile's last valid 16 bytes (results unused).
  const int colc = col < a.d_out ? col : a.d_out - 8;
  const int r0 = ks * a.rows_per_split;
  const int r1 = min(a.d_in, r0 + a.rows_per_split);
  float acc[MB][8];
  mv_f4 cm[MFMA ? kColBlocks : 1];
  if constexpr (MFMA) {
#pragma unroll
    for (int cb = 0; cb < kColBlocks; cb++) cm[cb] = mv_f4{0.f, 0.f, 0.f, 0.f};
  } else {
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int j = 0; j < 8; j++) acc[m][j] = 0.f;
  }

  // Several rows of x: stage the range's x in LDS when it fits.
  const int xrows = r1 - r0;
  const float* xl = nullptr;
  if (MB > 1 && a.M * xrows <= kXStage) {
    for (int i = threadIdx.x; i < a.M * xrows; i += blockDim.x) {
      const int m = i / xrows;
      lds.xs[i] = a.x[(size_t)m * a.d_in + r0 + (i - m * xrows)];
    }
    __syncthreads();
    xl = lds.xs;
  }
  if constexpr (MFMA) mv_row_scales<WAVES>(a, xl, xrows, r0, r1, L);

  if (wave < WAVES) {
    // Row blocks of kRowPhases rows: the wave takes blocks wave, wave +
    // WAVES, ... of the range, two batches of U per iteration: both
    // batches' loads are issued before the first batch's multiply-adds.
    constexpr int U = kUnroll;
    const MvRows rows = mv_rows(a, r0, r1, colc, rp);
    const int step = WAVES * U * kRowPhases;   // rows per batch of the workgroup
    const int last = (U - 1) * WAVES * kRowPhases + kRowPhases - 1;  // a batch's last row
    const int first = r0 + wave * kRowPhases;
    if constexpr (MFMA) {
      char* st = reinterpret_cast<char*>(L.wst[wave]);
      const float sc = L.xscale[min(lane & 15, a.M - 1)];  // this lane's row of x
      for (int r = first; r < r1; r += 2 * step) {
        uint4 wa[U], wb[U];
        mv_load_batch<WAVES, U>(rows, r, wa);
        mv_load_batch<WAVES, U>(rows, r + step, wb);
        mv_h4 xh, xo;
        mv_x_operand<WAVES>(a, xl, xrows, r0, r1, r, lane, sc, xh, xo);
        mv_stage<U>(st, rp, lc, wa);
        mv_mfma_batch(st, lane, xh, xo, cm);
        if (r + step < r1) {
          mv_x_operand<WAVES>(a, xl, xrows, r0, r1, r + step, lane, sc, xh, xo);
          mv_stage<U>(st, rp, lc, wb);  // (a wave's LDS operations complete in order)
          mv_mfma_batch(st, lane, xh, xo, cm);
        }
      }
    } else {
    for (int r = first; r < r1; r += 2 * step) {
      uint4 wa[U], wb[U];
      mv_load_batch<WAVES, U>(rows, r, wa);
      mv_load_batch<WAVES, U>(rows, r + step, wb);
      if (r + last < r1)
        mv_fma_batch<MB, WAVES, U, true>(a, r, r0, r1, rp, xl, xrows, wa, acc);
      else
        mv_fma_batch<MB, WAVES, U, false>(a, r, r0, r1, rp, xl, xrows, wa, acc);
      if (r + step + last < r1)
        mv_fma_batch<MB, WAVES, U, true>(a, r + step, r0, r1, rp, xl, xrows, wb, acc);
      else if (r + step < r1)
        mv_fma_batch<MB, WAVES, U, false>(a, r + step, r0, r1, rp, xl, xrows, wb, acc);
    }
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int j = 0; j < 8; j++) acc[m][j] = mv_phase_sum(acc[m][j]);
    }
  }

  // ---- waves -> one partial per (row of x, column) --------------------
  // Thread t < kCols/4 (64) sums 4 adjacent columns over the waves; a
  // partial is one 16-byte device-scope store.  Rows alternate between two LDS buffers
  // (the x staging area is free once every wave is past the streaming
  // loop), so one barrier per row orders its stores before the sums, and
  // the barrier of row m+1 orders row m's sums before row m+2's stores.
  static_assert(kXStage >= WAVES * kCols, "second reduction buffer");
  const uint32_t part_bytes = (uint32_t)((size_t)a.splits * a.M * a.d_out * sizeof(float));
  if constexpr (MFMA) {
    // every row of x at once: lane l writes its columns of row l % 16 into
    // [m][wave][kCols] over the W staging area (free once every wave is past
    // the streaming loop), 16-byte unit u of row m at u ^ (m % 16) so the
    // 16 rows of a store do not share banks; one barrier, then thread
    // t < kCols/4 sums 4 columns over the waves for each row of x
    static_assert(sizeof(L.wst) >= 8 * WAVES * kCols * sizeof(float), "row buffers");
    float* red = reinterpret_cast<float*>(L.wst);
    __syncthreads();
    if (wave < WAVES && (lane & 15) < a.M) {
      const float inv = 1.f / L.xscale[lane & 15];  // a power of two: exact
#pragma unroll
      for (int cb = 0; cb < kColBlocks; cb++)
        *reinterpret_cast<mv_f4*>(red + ((lane & 15) * WAVES + wave) * kCols +
                                  4 * ((4 * cb + (lane >> 4)) ^ (lane & 15))) = cm[cb] * inv;
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int c = ct * kCols + 4 * t;
    if (t < kCols / 4 && c < a.d_out) {
#pragma unroll
      for (int m = 0; m < MB; m++) {
        if (m >= a.M) break;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < WAVES; w++) {
          const float4 r =
              *reinterpret_cast<const float4*>(red + (m * WAVES + w) * kCols + 4 * (t ^ (m & 15)));
          v.x += r.x;
          v.y += r.y;
          v.z += r.z;
          v.w += r.w;
        }
        if (a.splits == 1)
          mv_write_out(a, m, c, v);
        else
          mv_store_dev16(a.partials, part_bytes,
                         (uint32_t)((((size_t)ks * a.M + m) * a.d_out + c) * sizeof(float)), v);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MB; m++) {
    if constexpr (MFMA) break;
    if (m >= a.M) break;
    if (m == 0) __syncthreads();  // every wave is past the streaming loop
    float* red = (m & 1) ? lds.xs : lds.red;
    if constexpr (MFMA) {
      if (wave < WAVES && (lane & 15) == m) {
#pragma unroll
        for (int cb = 0; cb < kColBlocks; cb++)
          *reinterpret_cast<mv_f4*>(red + wave * kCols + 16 * cb + 4 * (lane >> 4)) = cm[cb];
      }
    } else if (wave < WAVES && rp == 0) {
      float4* d = reinterpret_cast<float4*>(red + wave * kCols + lc * 8);
      d[0] = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
      d[1] = make_float4(acc[m][4], acc[m][5], acc[m][6], acc[m][7]);
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int c = ct * kCols + 4 * t;
    if (t < kCols / 4 && c < a.d_out) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int w = 0; w < WAVES; w++) {
        const float4 r = *reinterpret_cast<const float4*>(red + w * kCols + 4 * t);
        v.x += r.x;
        v.y += r.y;
        v.z += r.z;
        v.w += r.w;
      }
      if (a.splits == 1) {
        mv_write_out(a, m, c, v);
      } else {
        mv_store_dev16(a.partials, part_bytes,
                       (uint32_t)((((size_t)ks * a.M + m) * a.d_out + c) * sizeof(float)), v);
      }
    }
  }
  if (a.splits == 1) return;

  // ---- the last row range of this column tile adds the partials -------
  // The partials are device-scope stores; waiting for them (vmcnt) before
  // the arrival increment orders them before it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* ctr = a.counters + ct;
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)(a.splits - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds.last = last;
  }
  __syncthreads();
  if (!lds.last) return;
  // Thread (4 columns col4, quarter sub) loads the partials of row ranges
  // sub, sub+4, ... of every row of x in one round trip (splits * MB <=
  // kMaxSplit, indices past the last range re-read it and are dropped),
  // sums them in order, and the quarters of a column (adjacent lanes) add up
  // through two lane exchanges in a fixed order.
  constexpr int Q = kMaxSplit / 4 / MB;  // loads per row of x
  const int S = a.splits;
#pragma unroll 1
  for (int t = threadIdx.x; t < kCols; t += blockDim.x) {
    const int sub = t & 3;
    const int c = ct * kCols + 4 * (t >> 2);
    const int cc = c < a.d_out ? c : a.d_out - 4;
    float4 pv[MB][Q];
#pragma unroll
    for (int m = 0; m < MB; m++) {
#pragma unroll
      for (int i = 0; i < Q; i++) {
        if (m < a.M && i * 4 < S) {
          const int k = min(sub + 4 * i, S - 1);
          pv[m][i] = mv_load_dev16(
              a.partials, part_bytes,
              (uint32_t)((((size_t)k * a.M + m) * a.d_out + cc) * sizeof(float)));
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) {
      if (m >= a.M) break;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < Q; i++) {
        if (sub + 4 * i < S) {
          v.x += pv[m][i].x;
          v.y += pv[m][i].y;
          v.z += pv[m][i].z;
          v.w += pv[m][i].w;
        }
      }
#pragma unroll
      for (int x = 1; x <= 2; x *= 2) {
        v.x += __shfl_xor(v.x, x);
        v.y += __shfl_xor(v.y, x);
        v.z += __shfl_xor(v.z, x);
        v.w += __shfl_xor(v.w, x);
      }
      if (sub == 0 && c < a.d_out) mv_write_out(a, m, c, v);
    }
  }
}

// Rows of x rounded up to an unrolled instantiation.
template <int WAVES>
__device__ __forceinline__ void mv_item_any(const MvArgs& a, int ct, int ks, MvLds<WAVES>& lds) {
  switch (mv_row_bucket(a.M)) {
    case 1: mv_item<1, WAVES>(a, ct, ks, lds); break;
    case 2: mv_item<2, WAVES>(a, ct, ks, lds); break;
    case 3: mv_item<3, WAVES>(a, ct, ks, lds); break;
    case 4: mv_item<4, WAVES>(a, ct, ks, lds); break;
    case 5: mv_item<5, WAVES>(a, ct, ks, lds); break;
    case 6: mv_item<6, WAVES>(a, ct, ks, lds); break;
    case 7: mv_item<7, WAVES>(a, ct, ks, lds); break;
    default: mv_item<8, WAVES>(a, ct, ks, lds); break;
  }
}

}  // namespace mv

// ---- reference-named device API ------------------------------------------

// utils.h:417-452: out[c] (+)= sum_r x[r] * W[r*d_out + c] for c in
// [col_start, col_start+col_count), by the calling block alone (any
// blockDim that is a multiple of 64, no LDS).  The stripe's 8-column groups
// are spread over the waves, and each wave's lanes split the rows of its
// groups into phases whose sums meet through a lane butterfly; 16-byte
// weight loads.  Requires d_out % 8 == 0, col_start % 8 == 0 and a
// 16-byte-aligned W (the reference's shapes); each thread returns once its
// wave's columns are written (no block barrier, as in the reference).
namespace mv {
template <bool ACCUM>
__device__ __forceinline__ void block_matvec(const float* __restrict__ x,
                                             const uint16_t* __restrict__ W, float* out,
                                             int d_in, int d_out, int col_start, int col_count) {
  const int waves = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int groups = (col_count + 7) / 8;
  // Groups per wave (a power of two <= 64) and row phases per wave.
  int gpw = 1;
  while (gpw < 64 && gpw * waves < groups) gpw *= 2;
  const int phases = 64 / gpw;
  for (int g0 = wave * gpw; g0 < groups; g0 += waves * gpw) {
    const int g = g0 + (lane % gpw);
    const int p = lane / gpw;
    const bool live = g < groups;
    const int col = col_start + 8 * (live ? g : g0);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = p; r < d_in; r += phases * 4) {
      uint4 w[4];
      float xv[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int rr = r + u * phases;
        xv[u] = rr < d_in ? x[rr] : 0.f;
        w[u] = *reinterpret_cast<const uint4*>(W + (size_t)min(rr, d_in - 1) * d_out + col);
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint32_t wd[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          acc[2 * k] = fmaf(xv[u], h_lo(wd[k]), acc[2 * k]);
          acc[2 * k + 1] = fmaf(xv[u], h_hi(wd[k]), acc[2 * k + 1]);
        }
      }
    }
    // Sum over the phases (lanes gpw, 2*gpw, ... apart).
    for (int s = gpw; s < 64; s *= 2)
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] += __shfl_xor(acc[j], s);
    if (p == 0 && live) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int c = col + j;
        if (c < col_start + col_count) out[c] = ACCUM ? out[c] + acc[j] : acc[j];
      }
    }
  }
}
}  // namespace mv

__device__ inline void device_matvec_partial(const float* __restrict__ x,
                                             const uint16_t* __restrict__ W, float* out,
                                             int d_in, int d_out, int col_start,
                                             int col_count) {
  mv::block_matvec<false>(x, W, out, d_in, d_out, col_start, col_count);
}

__device__ inline void device_matvec_partial_accum(const float* __restrict__ x,
                                                   const uint16_t* __restrict__ W, float* out,
                                                   int d_in, int d_out, int col_start,
                                                   int col_count) {
  mv::block_matvec<true>(x, W, out, d_in, d_out, col_start, col_count);
}

// utils.h:248-280: g_out[b][c] = sum_r g_x[b*d_in + r] * W[r][c] for b < B,
// every column, by the calling block.
__device__ inline void device_matvec_batched(const float* g_x, const uint16_t* W, float* g_out,
                                             int d_in, int d_out, int B) {
  for (int b = 0; b < B; b++)
    mv::block_matvec<false>(g_x + (size_t)b * d_in, W, g_out + (size_t)b * d_out, d_in, d_out,
                            0, d_out);
}

// Grid-cooperative projection for persistent kernels: every block of the
// grid calls it with the same arguments (blockDim.x >= 256, a multiple of
// 64; any grid size) and blocks take the (column tile, row range) items in
// turns; out[m][c] (+)= sum_r x[m][r] W[r][c] for m < M <= 16.  The
// workspace (sde_matvec_workspace_size bytes) starts with arrival counters
// that must be zero before the first call (every call leaves them zero).
// Returns SDE_OK in every thread, or an error code before any work; out is
// complete once the grid has synchronized after the call.
__device__ __forceinline__ int device_matvec_grid(const float* x, const uint16_t* W, float* out,
                                                  int d_in, int d_out, int M, int accumulate,
                                                  void* workspace, size_t workspace_bytes) {
  using namespace mv;
  // The arguments are the same in every thread: in scalar registers also
  // where the caller is a function of its own.
  x = wave_uniform(x);
  W = wave_uniform(W);
  out = wave_uniform(out);
  d_in = wave_uniform(d_in);
  d_out = wave_uniform(d_out);
  M = wave_uniform(M);
  accumulate = wave_uniform(accumulate);
  workspace = wave_uniform(workspace);
  workspace_bytes = wave_uniform(workspace_bytes);
  if (blockDim.x < 256 || blockDim.x % 64 != 0) return SDE_ERR_UNSUPPORTED;
  if (d_out % 8 != 0 || (reinterpret_cast<uintptr_t>(W) & 15u) != 0) return SDE_ERR_UNSUPPORTED;
  if (!x || !W || !out || !workspace || d_in < 1 || d_out < 8 || M < 1 || M > kMaxRows)
    return SDE_ERR_INVALID_ARGUMENT;
  if (workspace_bytes < mv_workspace_size(d_in, d_out, M)) return SDE_ERR_WORKSPACE;
  const bool w8 = blockDim.x >= 512;
  const MvPlan p = mv_plan(d_in, d_out, gridDim.x * gridDim.y * gridDim.z, w8 ? 8 : 4, M);
  // A row range is addressed with 32-bit byte offsets.
  if ((size_t)p.rows_per_split * d_out * 2 >= ((size_t)1 << 31)) return SDE_ERR_UNSUPPORTED;
  MvArgs a;
  a.x = x;
  a.W = W;
  a.out = out;
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        mv_counter_bytes(d_out, M));
  a.d_in = d_in;
  a.d_out = d_out;
  a.M = M;
  a.splits = p.splits;
  a.rows_per_split = p.rows_per_split;
  a.accumulate = accumulate;
  __shared__ MvLds<8> lds;
  const int blk = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int nblk = gridDim.x * gridDim.y * gridDim.z;
  const int per_pass = p.col_tiles * p.splits;
  const int items = mv_passes(M) * per_pass;
  for (int it = blk; it < items; it += nblk) {
    const int j = it / per_pass;
    const int ct = (it - j * per_pass) % p.col_tiles;
    const int ks = (it - j * per_pass) / p.col_tiles;
    const MvArgs pa = mv_pass(a, j);
    if (w8)
      mv_item_any<8>(pa, ct, ks, lds);
    else
      mv_item_any<4>(pa, ct, ks, *reinterpret_cast<MvLds<4>*>(&lds));
    __syncthreads();  // LDS reuse by the block's next item
  }
  return SDE_OK;
}

}  // namespace sde
