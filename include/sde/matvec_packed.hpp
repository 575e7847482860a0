// Panel-packed output projection: out[m][c] (+)= sum_r x[m][r] W[r][c] over
// a one-time re-layout of W [d_in][d_out] (fp16, row-major, the SDEC
// layout) in which every workgroup streams whole output columns from
// contiguous memory.
//
// Why a second layout.  In the row-major layout a workgroup that owns a few
// output columns reads a few dozen bytes per row at a d_out-element stride,
// which HBM serves at a fraction of its rate; so sde_matvec splits d_in over
// the CUs and pays a split reduction (partial stores, arrival counters, one
// combining workgroup's round trips: ~4 us of a 13 us 4096 x 4096 call).  In
// the packed layout the columns of a panel (8 or 16 of them) are stored
// together for all rows, so one workgroup per panel reads one contiguous
// slab, reduces in registers and LDS, and writes its columns: no partials,
// no counters, no workspace, one launch.
//
// Layout.  A panel is PW = 8 * LPR output columns (LPR = 16-byte column
// chunks per row: 2 when d_out is a multiple of 16 and at least 4096, which
// gives one panel per CU or more at the reference models' widths, else 1).
// Its rows are cut into batches of BR = (64 / LPR) * 8 rows.  Within batch b
// of panel p, the 16-byte unit of lane l (0..63) and step j (0..7) is
//     unit ((p * n_batches + b) * 8 + j) * 64 + l
// holding W[r][c0 .. c0 + 7] for
//     r  = b * BR + (l / LPR) * 8 + j,   c0 = p * PW + 8 * (l % LPR);
// rows past d_in are zero.  So step j of a batch is one contiguous 1 KiB
// wave load, and lane l's eight rows of a batch are consecutive (its x
// values are two 16-byte loads).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sde {
namespace mvp {

constexpr int kWaves = 8;          // waves per workgroup
constexpr int kSteps = 8;          // 16-byte units of a lane per batch (rows)
constexpr int kMaxPassRows = 9;    // rows of x per launch pass (a verify window of k <= 8)

struct PackedShape {
  int lpr;         // 16-byte column chunks per row of a panel (1 or 2)
  int panel_cols;  // 8 * lpr
  int batch_rows;  // (64 / lpr) * kSteps
  int n_batches;
  int panels;
  size_t units;    // 16-byte units of the packed matrix
};

// The packed layout of a d_in x d_out matrix; panels == 0 when the shape is
// not supported (d_in or d_out not a positive multiple of 8).
__host__ __device__ inline PackedShape packed_shape(int d_in, int d_out) {
  PackedShape s;
  s.lpr = (d_out % 16 == 0 && d_out >= 4096) ? 2 : 1;
  s.panel_cols = 8 * s.lpr;
  s.batch_rows = (64 / s.lpr) * kSteps;
  if (d_in < 8 || d_out < 8 || d_in % 8 != 0 || d_out % 8 != 0) {
    s.n_batches = 0;
    s.panels = 0;
    s.units = 0;
    return s;
  }
  s.n_batches = (d_in + s.batch_rows - 1) / s.batch_rows;
  s.panels = d_out / s.panel_cols;
  s.units = (size_t)s.panels * s.n_batches * 64 * kSteps;
  return s;
}

// Rows of x per pass for M rows: passes of at most kMaxPassRows, balanced
// (16 rows run as 8 + 8, 10 as 5 + 5).
__host__ __device__ inline int packed_passes(int M) {
  return (M + kMaxPassRows - 1) / kMaxPassRows;
}
__host__ __device__ inline int packed_pass_rows(int M) {
  const int n = packed_passes(M);
  return (M + n - 1) / n;
}

// Passes of one host launch of M rows (the grid's second dimension).  The
// passes of one panel are workgroups p, p + panels, ...; with the panel
// count a multiple of 8 they run on one XCD, so when the whole packed
// matrix fits the 8 XCDs' L2 (at most 28 MiB of their 8 x 4 MiB) the later
// passes re-read the panel from that L2, and passes of up to 3 rows (97
// VGPRs: several workgroups per CU) beat one pass of up to 9 rows (up to 212
// VGPRs: one workgroup per CU) when that one-pass grid takes more than one
// round of the CUs or holds more than 5 rows.  Measured on MI355X, us, one
// pass vs 3-row passes: 3584 x 3584 with 9 rows 18.0 vs 14.5, 5 rows 12.4
// vs 11.4; 2048 x 2048 with 9 rows 8.1 vs 7.5, 5 rows 5.9 vs 6.1 (kept at
// one pass); 4096 x 4096 (32 MiB) with 9 rows 13.7 vs 14.3; 14336 x 4096
// with 9 rows 31.5 vs 50.7.
inline int packed_launch_passes(int M, const PackedShape& s, int n_cus) {
  const int one = packed_passes(M);
  if (M <= 3 || one > 1 || s.panels % 8 != 0) return one;
  if (s.units * 16 > ((size_t)28 << 20)) return one;
  if (s.panels <= n_cus && M <= 5) return one;
  return (M + 2) / 3;
}

struct PackedArgs {
  const uint4* W;   // packed units
  const float* x;   // [M][d_in], 16-byte aligned
  float* out;       // [M][d_out]
  int d_in, d_out, M, pass_rows, n_batches, accumulate;
};

// Unit u of the packed matrix from the row-major W (16-byte loads; d_out a
// multiple of 8 and W 16-byte aligned keep them aligned).
__device__ __forceinline__ uint4 packed_unit(const uint16_t* __restrict__ W, int d_in, int d_out,
                                             const PackedShape& s, size_t u) {
  const int l = (int)(u % 64);
  const size_t q = u / 64;
  const int j = (int)(q % kSteps);
  const size_t pb = q / kSteps;
  const int b = (int)(pb % (size_t)s.n_batches);
  const int p = (int)(pb / (size_t)s.n_batches);
  const int r = b * s.batch_rows + (l / s.lpr) * kSteps + j;
  if (r >= d_in) return make_uint4(0u, 0u, 0u, 0u);
  const int c0 = p * s.panel_cols + 8 * (l % s.lpr);
  return *reinterpret_cast<const uint4*>(W + (size_t)r * d_out + c0);
}

// (static: every source file that includes this header gets its own copy)
static __global__ void __launch_bounds__(256) matvec_pack_kernel(const uint16_t* __restrict__ W,
                                                           uint4* __restrict__ P, int d_in,
                                                           int d_out) {
  const PackedShape s = packed_shape(d_in, d_out);
  for (size_t u = blockIdx.x * (size_t)blockDim.x + threadIdx.x; u < s.units;
       u += (size_t)gridDim.x * blockDim.x)
    P[u] = packed_unit(W, d_in, d_out, s, u);
}

__device__ __forceinline__ float half_lo(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

// One step of a lane: JR units (rows r0 .. r0 + JR - 1 of its column chunk)
// and the matching x of every row of the pass (zero past d_in or past the
// pass's rows).
template <int MB, int JR>
struct PackedStep {
  uint4 w[JR];
  float x[MB][JR];
};

// Eight zero floats (device globals are zero-initialized; nothing writes
// them): the x operand of rows past d_in (one copy per source file).
static __device__ __attribute__((aligned(16))) float packed_zero_x[kSteps];

template <int MB, int LPR, int JR>
__device__ __forceinline__ void packed_load(const PackedArgs& a, const uint4* __restrict__ P,
                                            int m0, int mc, int s, int lane,
                                            PackedStep<MB, JR>& st) {
  constexpr int kHalves = kSteps / JR;
  constexpr int BR = (64 / LPR) * kSteps;
  const int b = s / kHalves, hf = s % kHalves;
  const uint4* q = P + ((size_t)b * kSteps + hf * JR) * 64 + lane;
#pragma unroll
  for (int j = 0; j < JR; j++) st.w[j] = q[j * 64];
  const int r0 = b * BR + (lane / LPR) * kSteps + hf * JR;
  // Every load is unconditional (no branch or select on loaded values, so
  // nothing waits on a load before its step's multiply-adds): lanes whose
  // rows are past d_in (d_in % 8 == 0: all of a lane's rows or none) read
  // zeros from packed_zero_x -- never x, whose values could turn the padded
  // zero weights into NaN -- and rows of x past the pass re-read the pass's
  // first row (their sums are never written).
  const bool in = r0 < a.d_in;
#pragma unroll
  for (int m = 0; m < MB; m++) {
    const int mm = m < mc ? m : 0;
    const float4* xp = reinterpret_cast<const float4*>(
        in ? a.x + (size_t)(m0 + mm) * a.d_in + r0 : packed_zero_x);
#pragma unroll
    for (int h = 0; h < JR / 4; h++) {
      const float4 v = xp[h];
      st.x[m][4 * h + 0] = v.x;
      st.x[m][4 * h + 1] = v.y;
      st.x[m][4 * h + 2] = v.z;
      st.x[m][4 * h + 3] = v.w;
    }
  }
}

template <int MB, int JR>
__device__ __forceinline__ void packed_fma(const PackedStep<MB, JR>& st, float (&acc)[MB][8]) {
#pragma unroll
  for (int j = 0; j < JR; j++) {
    const float w[8] = {half_lo(st.w[j].x), half_hi(st.w[j].x), half_lo(st.w[j].y),
                        half_hi(st.w[j].y), half_lo(st.w[j].z), half_hi(st.w[j].z),
                        half_lo(st.w[j].w), half_hi(st.w[j].w)};
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int c = 0; c < 8; c++) acc[m][c] = __builtin_fmaf(w[c], st.x[m][j], acc[m][c]);
  }
}

// v + the value of the lane selected by a DPP control (all lanes active).
template <int CTRL>
__device__ __forceinline__ float dpp_plus(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
  return v + __builtin_bit_cast(float, s);
}

// Sum over the lanes of a wave with the same l % LPR, in every such lane:
// within each 16-lane row by DPP (quad_perm [1,0,3,2] when LPR == 1, then
// quad_perm [2,3,0,1], row_ror 4, row_ror 8), then across the four rows by
// permlane16 / permlane32 swaps.
template <int LPR>
__device__ __forceinline__ float packed_wave_sum(float v) {
  if constexpr (LPR == 1) v = dpp_plus<0xB1>(v);
  v = dpp_plus<0x4E>(v);
  v = dpp_plus<0x124>(v);
  v = dpp_plus<0x128>(v);
  auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                            false, false);
  v = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
  p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                       false, false);
  return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}

// Workgroup (panel blockIdx.x, pass blockIdx.y): the waves take the panel's
// steps (batches, or half batches when JR == 4) in turn, two in flight per
// wave (ping-pong registers, no loop-carried copies); each lane accumulates
// its 8 columns over its rows, the wave sums its lanes, and the 8 waves'
// sums are added in wave order through LDS.  Deterministic.
// ext_red: when not null, the waves' sums go through this caller-provided
// LDS (at least MB * kWaves * 8 * LPR floats) instead of the function's own
// array (one per instantiation): a kernel running several row counts can
// give them one array.
template <int MB, int LPR, int JR, bool EXT_RED = false>
__device__ __forceinline__ void packed_item(const PackedArgs& a, int panel, int pass,
                                            float* ext_red = nullptr) {
  constexpr int PW = 8 * LPR;
  using Red = float[MB][kWaves][PW];
  Red* red_p;
  if constexpr (EXT_RED) {
    red_p = reinterpret_cast<Red*>(ext_red);
  } else {
    __shared__ float own[MB][kWaves][PW];
    red_p = &own;
  }
  Red& red = *red_p;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int m0 = pass * a.pass_rows;
  const int mc = min(a.pass_rows, a.M - m0);
  const uint4* P = a.W + (size_t)panel * a.n_batches * kSteps * 64;
  const int n_steps = a.n_batches * (kSteps / JR);
  float acc[MB][8];
#pragma unroll
  for (int m = 0; m < MB; m++)
#pragma unroll
    for (int c = 0; c < 8; c++) acc[m][c] = 0.f;
  // The wave's ns steps run as pairs with the next step's loads issued
  // before the current step's multiply-adds; the loop body's loads are
  // unconditional (a conditional load would make the compiler's wait before
  // the multiply-adds cover the new loads too) and the last one or two
  // steps are peeled.  The scheduling barriers keep each load batch ahead of
  // the multiply-adds it overlaps (measured: 5 rows of a 4096 x 4096
  // projection 10.4 us against 10.9-11.5 for the same code without them or
  // with a non-peeled loop).
  PackedStep<MB, JR> sa, sb;
  const int ns = wave < n_steps ? (n_steps - wave + kWaves - 1) / kWaves : 0;
  if (ns > 0) {
    packed_load<MB, LPR, JR>(a, P, m0, mc, wave, lane, sa);
    int k = 0;
    for (; k + 2 < ns; k += 2) {
      packed_load<MB, LPR, JR>(a, P, m0, mc, wave + (k + 1) * kWaves, lane, sb);
      __builtin_amdgcn_sched_barrier(0);
      packed_fma<MB, JR>(sa, acc);
      packed_load<MB, LPR, JR>(a, P, m0, mc, wave + (k + 2) * kWaves, lane, sa);
      __builtin_amdgcn_sched_barrier(0);
      packed_fma<MB, JR>(sb, acc);
    }
    if (ns - k == 2) {
      packed_load<MB, LPR, JR>(a, P, m0, mc, wave + (k + 1) * kWaves, lane, sb);
      __builtin_amdgcn_sched_barrier(0);
      packed_fma<MB, JR>(sa, acc);
      packed_fma<MB, JR>(sb, acc);
    } else {
      packed_fma<MB, JR>(sa, acc);
    }
  }
#pragma unroll
  for (int m = 0; m < MB; m++)
#pragma unroll
    for (int c = 0; c < 8; c++) acc[m][c] = packed_wave_sum<LPR>(acc[m][c]);
  if (lane < LPR) {
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int c = 0; c < 8; c++) red[m][wave][8 * lane + c] = acc[m][c];
  }
  __syncthreads();
  if ((int)threadIdx.x < MB * PW) {
    const int m = threadIdx.x / PW, c = threadIdx.x % PW;
    if (m < mc) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) t += red[m][w][c];
      float* o = a.out + (size_t)(m0 + m) * a.d_out + panel * PW + c;
      *o = a.accumulate ? *o + t : t;
    }
  }
}

}  // namespace mvp
}  // namespace sde
