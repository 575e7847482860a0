// Paged GQA decode / speculative-verify attention for gfx950 (wave64).
//
// Computes what cublas_attention_kernel (kernels.cu:904-940) computes with
// device_flash_attention_gqa (attention.h:21-127): for query m of a window,
// out[m][h] = softmax(q[m][h] . K[0..pos_base+m]^T * dph^-1/2) V, with query
// head h reading KV head h*nkv/nh, keys gathered through the block table.
//
// Work decomposition (no MFMA: decode and small-k verify are GEMV-shaped):
//  * one workgroup of kWaves wave64s per (context partition, KV head, row
//    group).  The "rows" are the (query, head-in-group) pairs sharing one KV
//    head, so each K/V byte is read from HBM once for all G*n_queries rows;
//  * a partition is kWaves * tiles_per_wave tiles of 32 tokens; wave w takes
//    tiles w, w+kWaves, ...  Each tile's K and V head slices land in the
//    wave's LDS with direct-to-LDS 16-byte loads (16 lanes cover a 256 B
//    row for dph 128), K chunk-swizzled so the transposed reads below are
//    bank-conflict free;
//  * Q.K: lane (t, half) owns token t and half of the head dimension, reads
//    its K chunks from LDS and takes fp16 dot2 products with the q group
//    (scaled by log2(e)/sqrt(dph), rounded to fp16, broadcast from LDS);
//    the two halves are summed across lanes, leaving row 2i+half's logit;
//  * online softmax in the exp2 domain with 32-lane max/sum reductions;
//    probabilities go to LDS as fp16;
//  * P.V: lane owns a pair of head features; V rows of two tokens are
//    byte-permuted into (token0, token1) fp16 pairs and dot2-accumulated
//    against the probability pairs, fp32 accumulators;
//  * the waves' (max, sum, acc) merge through LDS; a single-partition
//    context writes the normalised output directly, otherwise per-row
//    partials go to the workspace and the last workgroup to finish a (KV
//    head, row group) -- found with one arrival counter per pair -- merges
//    all partitions with a log-sum-exp combine in partition order, so the
//    result does not depend on arrival order and one call is one launch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>

#include "sde_internal.hpp"

namespace sde {
namespace attn {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kTile = 32;  // tokens per tile
constexpr int kWaves = 4;  // waves per workgroup
constexpr int kMaxRowsPerWave = 32;
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
  int tiles_per_wave;
  float qscale;  // log2(e) / sqrt(dph)
};

// LDS of one wave: K tile, V tile, P tile; after the tile loop the same bytes
// hold the wave's merge record (max, sum, acc[dph]) per row.
template <int DPH, int RPW>
struct WaveLds {
  static constexpr int kTileBytes = kTile * DPH * 2;
  static constexpr int kWork = 2 * kTileBytes + RPW * kTile * 2;
  static constexpr int kMerge = RPW * (DPH + 2) * 4;
  static constexpr int kBytes = ((kWork > kMerge ? kWork : kMerge) + 15) / 16 * 16;
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                __builtin_bit_cast(half2_t, b), c, false);
}

// All-reduce within each 32-lane half of the wave.
__device__ __forceinline__ float half_max(float x) {
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float half_sum(float x) {
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

__device__ __forceinline__ uint16_t f2h_bits(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Device-scope (agent) relaxed atomic accesses for the partition partials:
// the stores write through to the device coherence point and the loads do
// not hit stale lines of another XCD's L2, so publishing partials needs no
// L2 writeback/invalidate fence (those cost microseconds per workgroup).
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_dev2(float* p, float x, float y) {
  const uint64_t bits = (uint64_t)__builtin_bit_cast(uint32_t, x) |
                        ((uint64_t)__builtin_bit_cast(uint32_t, y) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 load_dev2(const float* p) {
  const uint64_t bits = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__builtin_bit_cast(float, (uint32_t)bits),
                     __builtin_bit_cast(float, (uint32_t)(bits >> 32)));
}

// Physical 16-byte chunk of logical chunk c of tile token t is c ^ kswz(t):
// the 16 lanes of a QK read then touch 16 distinct chunk columns.
template <int DPH>
__device__ __forceinline__ int kswz(int t) {
  if constexpr (DPH == 128)
    return t & 15;
  else
    return (t >> 1) & 7;
}

template <int DPH, int RPW>
__global__ __launch_bounds__(64 * kWaves) void attn_partition_kernel(AttnArgs a) {
  static_assert(DPH == 64 || DPH == 128, "head_dim");
  static_assert(RPW % 2 == 0 && RPW <= kMaxRowsPerWave, "rows per wave");
  constexpr int CH = DPH / 8;       // 16-byte chunks per head row
  constexpr int TPL = 64 / CH;      // tokens per direct-to-LDS instruction
  constexpr int NLD = kTile / TPL;  // instructions per tile (per K and per V)
  constexpr int HCH = CH / 2;       // chunks per lane in Q.K
  constexpr int RP = RPW / 2;       // row pairs
  constexpr int DP = DPH / 2;       // fp16 pairs per head row
  using W = WaveLds<DPH, RPW>;

  __shared__ __attribute__((aligned(16))) uint16_t sQ[RPW * DPH];
  __shared__ __attribute__((aligned(16))) unsigned char sWave[kWaves][W::kBytes];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint16_t* const sK = reinterpret_cast<uint16_t*>(sWave[wave]);
  uint16_t* const sV = sK + kTile * DPH;
  uint16_t* const sP = sV + kTile * DPH;
  const uint32_t* const sV32 = reinterpret_cast<const uint32_t*>(sV);
  const uint32_t* const sP32 = reinterpret_cast<const uint32_t*>(sP);

  const int part = blockIdx.x;
  const int kvh = blockIdx.y;
  const int r0 = blockIdx.z * RPW;
  const int nrows = min(RPW, a.R - r0);
  const int t_begin = part * a.tiles_per_wave * kWaves * kTile;
  const int t_end = min(a.L_max, t_begin + a.tiles_per_wave * kWaves * kTile);

  // q rows of this group -> fp16 in LDS, pre-scaled into the exp2 domain.
  for (int idx = threadIdx.x; idx < RPW * DP; idx += 64 * kWaves) {
    const int r = idx / DP;
    const int d2 = idx - r * DP;
    uint32_t packed = 0;
    if (r < nrows) {
      const int gr = r0 + r;
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      const float2 qv = *reinterpret_cast<const float2*>(
          a.q + (size_t)m * a.nh * DPH + (size_t)h * DPH + 2 * d2);
      const half2_t hv = {(_Float16)(qv.x * a.qscale), (_Float16)(qv.y * a.qscale)};
      packed = __builtin_bit_cast(uint32_t, hv);
    }
    reinterpret_cast<uint32_t*>(sQ)[idx] = packed;
  }

  // Q.K role: token t of the tile, feature half hh.  After the half-sum a
  // lane holds the logit of row 2i+hh for pair i.
  const int t = lane & 31;
  const int hh = lane >> 5;
  int lim[RP];  // last visible position of row 2i+hh (-1: padding row)
  float m_run[RP], l_run[RP];
#pragma unroll
  for (int i = 0; i < RP; i++) {
    const int r = 2 * i + hh;
    lim[i] = (r < nrows) ? a.pos_base + (r0 + r) / a.G : -1;
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }
  float acc[RPW][2];
#pragma unroll
  for (int r = 0; r < RPW; r++) acc[r][0] = acc[r][1] = 0.f;

  __syncthreads();  // sQ complete

  // The waves run different numbers of tiles: only wave-local ordering is
  // used inside this loop (LDS operations of one wave complete in order).
  // The table is read-only during the kernel: read it through the constant
  // address space so entries arrive by scalar loads (lgkmcnt), which do not
  // wait behind the outstanding direct-to-LDS loads (vmcnt).
  const __attribute__((address_space(4))) int32_t* const table =
      (const __attribute__((address_space(4))) int32_t*)a.table;

  for (int ts = t_begin + wave * kTile; ts < t_end; ts += kWaves * kTile) {
    // ---- K and V head slices of tokens ts..ts+31 -> this wave's LDS -------
    int blk[NLD];  // physical block of each instruction group (wave-uniform)
#pragma unroll
    for (int j = 0; j < NLD; j++) {
      const int g0 = min(ts + j * TPL, a.L_max - 1);
      blk[j] = table[g0 / a.bs];
    }
#pragma unroll
    for (int j = 0; j < NLD; j++) {
      const int g0 = ts + j * TPL;  // wave-uniform; the group shares a block
      if (g0 < a.L_max) {
        const int lb = g0 / a.bs;
        const int tl = j * TPL + lane / CH;
        const int pc = lane % CH;
        const int slot = g0 - lb * a.bs + lane / CH;
        const uint16_t* rowk = a.pool +
                               ((size_t)blk[j] * 2u * a.bs + slot) * (size_t)a.kv_dim +
                               (size_t)kvh * DPH;
        const uint16_t* rowv = rowk + (size_t)a.bs * a.kv_dim;
        __builtin_amdgcn_global_load_lds((const void*)(rowk + (pc ^ kswz<DPH>(tl)) * 8),
                                         (lds_ptr_t)(sK + j * 512), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(rowv + pc * 8),
                                         (lds_ptr_t)(sV + j * 512), 16, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    // Rows past the context may hold stale (even non-finite) bytes; their
    // probabilities are 0 but 0 * NaN is not, so clear those V rows.
    const int nvalid = a.L_max - ts;
    if (nvalid < kTile) {
      uint32_t* v32 = reinterpret_cast<uint32_t*>(sV);
      for (int idx = nvalid * DP + lane; idx < kTile * DP; idx += 64) v32[idx] = 0u;
    }

    // ---- logits ----------------------------------------------------------
    float s[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) s[r] = 0.f;
#pragma unroll
    for (int jj = 0; jj < HCH; jj++) {
      const int c = hh * HCH + jj;
      const uint4 kc =
          *reinterpret_cast<const uint4*>(sK + t * DPH + (c ^ kswz<DPH>(t)) * 8);
#pragma unroll
      for (int r = 0; r < RPW; r++) {
        const uint4 qc = *reinterpret_cast<const uint4*>(sQ + r * DPH + c * 8);
        s[r] = dot2(qc.x, kc.x, s[r]);
        s[r] = dot2(qc.y, kc.y, s[r]);
        s[r] = dot2(qc.z, kc.z, s[r]);
        s[r] = dot2(qc.w, kc.w, s[r]);
      }
    }

    // ---- online softmax (exp2 domain) ------------------------------------
    const int tok = ts + t;
    float alpha[RP];
#pragma unroll
    for (int i = 0; i < RP; i++) {
      const float x0 = s[2 * i] + __shfl_xor(s[2 * i], 32);
      const float x1 = s[2 * i + 1] + __shfl_xor(s[2 * i + 1], 32);
      const float x = hh ? x1 : x0;
      const bool valid = tok <= lim[i];
      const float tmax = half_max(valid ? x : -INFINITY);
      const float m_new = fmaxf(m_run[i], tmax);
      const bool any = m_new != -INFINITY;
      const float al = any ? __builtin_amdgcn_exp2f(m_run[i] - m_new) : 1.f;
      const float p = (valid && any) ? __builtin_amdgcn_exp2f(x - m_new) : 0.f;
      l_run[i] = l_run[i] * al + p;
      m_run[i] = m_new;
      alpha[i] = al;
      sP[(2 * i + hh) * kTile + t] = f2h_bits(p);
    }

    // ---- P.V ---------------------------------------------------------------
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const float al = lane_value(alpha[r / 2], (r & 1) ? 32 : 0);
      acc[r][0] *= al;
      acc[r][1] *= al;
    }
    if constexpr (DPH == 128) {
#pragma unroll 2
      for (int jp = 0; jp < kTile / 2; jp++) {
        const uint32_t v0 = sV32[(2 * jp) * DP + lane];
        const uint32_t v1 = sV32[(2 * jp + 1) * DP + lane];
        const uint32_t lo = __builtin_amdgcn_perm(v1, v0, 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(v1, v0, 0x07060302u);
#pragma unroll
        for (int r = 0; r < RPW; r++) {
          const uint32_t pp = sP32[r * (kTile / 2) + jp];
          acc[r][0] = dot2(pp, lo, acc[r][0]);
          acc[r][1] = dot2(pp, hi, acc[r][1]);
        }
      }
    } else {
      // 32 feature pairs: lanes 0-31 take even token pairs, 32-63 odd ones.
      const int dp = lane & 31;
      const int tp = lane >> 5;
#pragma unroll 2
      for (int jj = 0; jj < kTile / 4; jj++) {
        const int jp = 2 * jj + tp;
        const uint32_t v0 = sV32[(2 * jp) * DP + dp];
        const uint32_t v1 = sV32[(2 * jp + 1) * DP + dp];
        const uint32_t lo = __builtin_amdgcn_perm(v1, v0, 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(v1, v0, 0x07060302u);
#pragma unroll
        for (int r = 0; r < RPW; r++) {
          const uint32_t pp = sP32[r * (kTile / 2) + jp];
          acc[r][0] = dot2(pp, lo, acc[r][0]);
          acc[r][1] = dot2(pp, hi, acc[r][1]);
        }
      }
    }
    // Every LDS read of this tile has returned before the next iteration's
    // direct-to-LDS loads may overwrite the tile.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // ---- per-wave row statistics -> this wave's merge record in LDS --------
  float* const rec = reinterpret_cast<float*>(sWave[wave]);
#pragma unroll
  for (int i = 0; i < RP; i++) {
    const float lt = half_sum(l_run[i]);
    if (lane == 0 || lane == 32) {
      rec[(2 * i + hh) * (DPH + 2)] = m_run[i];
      rec[(2 * i + hh) * (DPH + 2) + 1] = lt;
    }
  }
  if constexpr (DPH == 64) {
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      acc[r][0] += __shfl_xor(acc[r][0], 32);
      acc[r][1] += __shfl_xor(acc[r][1], 32);
    }
  }
  const int dcol = (DPH == 128 ? lane : (lane & 31)) * 2;
  if (DPH == 128 || lane < 32) {
#pragma unroll
    for (int r = 0; r < RPW; r++)
      *reinterpret_cast<float2*>(rec + r * (DPH + 2) + 2 + dcol) =
          make_float2(acc[r][0], acc[r][1]);
  }
  __syncthreads();

  // ---- merge the waves; wave w finalises rows w, w+kWaves, ... ------------
  for (int r = wave; r < nrows; r += kWaves) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++)
      mx = fmaxf(mx, reinterpret_cast<const float*>(sWave[w])[r * (DPH + 2)]);
    float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float* rw = reinterpret_cast<const float*>(sWave[w]) + r * (DPH + 2);
      const float mw = rw[0];
      const float wt = (mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
      l += rw[1] * wt;
      if (DPH == 128 || lane < 32) {
        const float2 aw = *reinterpret_cast<const float2*>(rw + 2 + dcol);
        o0 += aw.x * wt;
        o1 += aw.y * wt;
      }
    }
    if (DPH == 128 || lane < 32) {
      const int gr = r0 + r;
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      if (a.n_parts == 1) {
        // attention.h:120-126: normalise unless the sum is tiny or not finite.
        const float inv = (l > 1e-20f && isfinite(l)) ? 1.f / l : 0.f;
        *reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH + dcol) =
            make_float2(o0 * inv, o1 * inv);
      } else {
        float* pr = a.partials +
                    (((size_t)kvh * a.R + gr) * a.n_parts + part) * (size_t)(DPH + 2);
        store_dev2(pr + 2 + dcol, o0, o1);
        if (lane == 0) {
          store_dev(pr, mx);
          store_dev(pr + 1, l);
        }
      }
    }
  }
  if (a.n_parts == 1) return;

  // ---- fused partition combine: the last workgroup of (kvh, row group) ----
  // Every partial was stored at device scope; waiting for their completion
  // (vmcnt) before the arrival increment orders them before it, and the last
  // arriver reads them back with device-scope loads.
  __shared__ int s_last;
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

  // Latency-tolerant merge: lane p reads partition p's (max, sum); the
  // accumulator rows are loaded kBatch partitions at a time before use.
  constexpr int kBatch = 16;
  for (int r = wave; r < nrows; r += kWaves) {
    const int gr = r0 + r;
    const float* base = a.partials + ((size_t)kvh * a.R + gr) * a.n_parts * (size_t)(DPH + 2);
    float mx = -INFINITY;
    for (int p0 = 0; p0 < a.n_parts; p0 += 64) {
      const int p = p0 + lane;
      const float mp = p < a.n_parts ? load_dev(base + (size_t)p * (DPH + 2)) : -INFINITY;
      mx = fmaxf(mx, half_max(mp));
    }
    mx = fmaxf(lane_value(mx, 0), lane_value(mx, 32));
    float l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int p0 = 0; p0 < a.n_parts; p0 += 64) {
      const int p = p0 + lane;
      float wt = 0.f;  // weight of partition p0+lane (0: absent or no visible key)
      if (p < a.n_parts) {
        const float mp = load_dev(base + (size_t)p * (DPH + 2));
        if (mp != -INFINITY) {
          wt = __builtin_amdgcn_exp2f(mp - mx);
          l += load_dev(base + (size_t)p * (DPH + 2) + 1) * wt;
        }
      }
      const int n = min(64, a.n_parts - p0);
      for (int b0 = 0; b0 < n; b0 += kBatch) {
        float2 v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
          v[u] = make_float2(0.f, 0.f);
          if (b0 + u < n && (DPH == 128 || lane < 32))
            v[u] = load_dev2(base + (size_t)(p0 + b0 + u) * (DPH + 2) + 2 + dcol);
        }
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
          if (b0 + u < n) {
            const float wu = lane_value(wt, b0 + u);
            o0 += v[u].x * wu;
            o1 += v[u].y * wu;
          }
        }
      }
    }
    l = half_sum(l);
    l = lane_value(l, 0) + lane_value(l, 32);
    if (DPH == 128 || lane < 32) {
      const int m = gr / a.G;
      const int h = kvh * a.G + (gr - m * a.G);
      const float inv = (l > 1e-20f && isfinite(l)) ? 1.f / l : 0.f;
      *reinterpret_cast<float2*>(a.out + (size_t)m * a.nh * DPH + (size_t)h * DPH + dcol) =
          make_float2(o0 * inv, o1 * inv);
    }
  }
}

}  // namespace attn
}  // namespace sde

namespace {

using namespace sde::attn;

struct Plan {
  int rpw;
  int row_groups;
  int tiles_per_wave;
  int n_parts;
};

int env_int(const char* name, int fallback) {
  const char* s = std::getenv(name);
  if (!s || !*s) return fallback;
  const int v = std::atoi(s);
  return v > 0 ? v : fallback;
}

int rows_per_wave(int R) {
  static const int kChoices[] = {2, 4, 8, 12, 16, 20, 24, 28, 32};
  if (R > kMaxRowsPerWave) return kMaxRowsPerWave;
  for (int c : kChoices)
    if (c >= R) return c;
  return kMaxRowsPerWave;
}

int target_waves() { return env_int("SDE_ATTN_TARGET_WAVES", 2048); }

// Tiles per wave: the fewest that keep the total near target_waves() waves.
Plan make_plan(int L_max, int nkv, int R) {
  Plan p;
  p.rpw = rows_per_wave(R);
  p.row_groups = (R + p.rpw - 1) / p.rpw;
  const int n_tiles = (L_max + kTile - 1) / kTile;
  const int64_t work = (int64_t)n_tiles * nkv * p.row_groups;
  const int64_t tw = target_waves();
  p.tiles_per_wave = (int)((work + tw - 1) / tw);
  if (p.tiles_per_wave < 1) p.tiles_per_wave = 1;
  const int per_part = p.tiles_per_wave * kWaves;
  p.n_parts = (n_tiles + per_part - 1) / per_part;
  return p;
}

// Upper bound of make_plan(L).n_parts over every L <= max_total_len: with one
// tile per wave n_parts = ceil(n_tiles / kWaves); with more, n_tiles/tpw is
// at most target/(nkv*row_groups).
int parts_bound(int max_total_len, int nkv, int row_groups) {
  const int n_tiles = (max_total_len + kTile - 1) / kTile;
  const int by_len = (n_tiles + kWaves - 1) / kWaves;
  const int64_t per = (int64_t)nkv * row_groups * kWaves;
  const int by_target = (int)((target_waves() + per - 1) / per);
  return by_len < by_target ? by_len : by_target;
}

size_t partial_bytes(int nkv, int R, int n_parts, int dph) {
  return n_parts > 1 ? (size_t)nkv * R * n_parts * (size_t)(dph + 2) * sizeof(float) : 0;
}

template <int DPH>
int launch_partition(const Plan& p, const AttnArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(64 * kWaves);
  switch (p.rpw) {
#define SDE_CASE(N)                                              \
  case N:                                                        \
    attn_partition_kernel<DPH, N><<<grid, block, 0, s>>>(a);     \
    break;
    SDE_CASE(2)
    SDE_CASE(4)
    SDE_CASE(8)
    SDE_CASE(12)
    SDE_CASE(16)
    SDE_CASE(20)
    SDE_CASE(24)
    SDE_CASE(28)
    SDE_CASE(32)
#undef SDE_CASE
    default:
      return SDE_ERR_UNSUPPORTED;
  }
  return sde::launch_status();
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
  const int rpw = rows_per_wave(R);
  const int row_groups = (R + rpw - 1) / rpw;
  return partial_bytes(nkv, R, parts_bound(max_total_len, nkv, row_groups), dph);
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
  const Plan plan = make_plan(L_max, nkv, R);
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
  a.tiles_per_wave = plan.tiles_per_wave;
  a.qscale = (float)(kLog2e / std::sqrt((double)dph));

  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid(plan.n_parts, nkv, plan.row_groups);
  return dph == 128 ? launch_partition<128>(plan, a, grid, s)
                    : launch_partition<64>(plan, a, grid, s);
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
