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

#include "sde/attention_device.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace attn {

struct AttnArgs {
  TileSource src;        // pool, this layer's table, kv_dim, block_size, L_max
  const float* q;        // [M][nh*dph]
  float* out;            // [M][nh*dph]
  float* partials;       // [nkv][R][n_parts][dph+2] = (max, sum, acc[dph])
  uint32_t* counters;    // [nkv][row_groups] arrival counters, zero at rest
  int nh;
  int G;         // query heads per KV head
  int R;         // rows per KV head = M * G (row = m*G + g)
  int pos_base;  // query m sees positions [0, pos_base+m]
  int n_parts;
  int tiles_per_part;  // attn_stream_kernel: tiles per partition
  float qscale;  // log2(e) / sqrt(dph)
};

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

__device__ __forceinline__ float4 load_dev4(const float* p) {
  const float2 lo = load_dev2(p);
  const float2 hi = load_dev2(p + 2);
  return make_float4(lo.x, lo.y, hi.x, hi.y);
}

constexpr int kStreamWaves = 8;      // waves per workgroup
constexpr int kStreamMaxParts = 64;  // partitions per (KV head, row group)

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

template <int DPH, int RPW, int CHUNK>
__global__ __launch_bounds__(64 * kStreamWaves) void attn_stream_kernel(AttnArgs a) {
  static_assert(DPH == 64 || DPH == 128, "head_dim");
  static_assert(RPW == 2 || RPW == 4, "rows per wave");
  constexpr int CH = DPH / 8;
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
  const int n_tiles = (a.src.L_max + kTile - 1) / kTile;
  const int tb = part * a.tiles_per_part;
  const int te = min(n_tiles, tb + a.tiles_per_part);

  using Sh = StreamShape<DPH, RPW>;
  const int my_r = (c >> (Sh::S - Sh::T)) >> (Sh::T - Sh::RB);

  // This lane's q chunk (features 8c..8c+7) of every row, loaded before any
  // K/V load so that waiting for it never waits for tile data.
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
  // Wave w takes tiles tb+w, tb+w+W, ... of the partition.
  wave_attend<DPH, RPW, CHUNK>(a.src, kvh, tb + wave, te, kStreamWaves, nrows, min_lim, my_lim,
                               a.qscale, q_raw, m_run, l_run, acc);

  // ---- merge the slot states of this wave; record per row ---------------
  float mx[RPW], lw[RPW];
  wave_merge_slots<DPH, RPW>(m_run, l_run, acc, mx, lw);
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    float* rec = s_buf + (wave * RPW + r) * REC;
    if (lane == 0) {
      rec[0] = mx[r];
      rec[1] = lw[r];
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
      const float inv = finish_scale(l);
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
  int chunk;           // tiles per unrolled chunk (1 to 4)
  int tiles_per_part;  // tiles per partition (workgroup)
  int n_parts;
};

int rows_per_wave(int R) { return R <= 2 ? 2 : kStreamMaxRows; }

// Sizing: at most one workgroup per CU (a second round of workgroups would
// double the latency of a latency-bound call), as many partitions as that
// allows (up to kStreamMaxParts, at least one tile per wave), then the
// fewest tiles per wave that cover the context.  A wave takes its tiles in
// chunks of `chunk` (1 to 4, unrolled at compile time), several chunks
// when it has more than four tiles.
Plan make_plan(int L_max, int nkv, int R, int n_cus) {
  Plan p;
  p.rpw = rows_per_wave(R);
  p.row_groups = (R + p.rpw - 1) / p.rpw;
  const int n_tiles = (L_max + kTile - 1) / kTile;
  const int64_t units = (int64_t)nkv * p.row_groups;
  int64_t parts = n_cus / units;
  if (parts < 1) parts = 1;
  if (parts > kStreamMaxParts) parts = kStreamMaxParts;
  const int64_t by_len = (n_tiles + kStreamWaves - 1) / kStreamWaves;
  if (parts > by_len) parts = by_len;
  const int per_wave = (int)((n_tiles + parts * kStreamWaves - 1) / (parts * kStreamWaves));
  p.chunk = per_wave <= 3 ? per_wave : 4;
  const int reps = (per_wave + p.chunk - 1) / p.chunk;
  p.tiles_per_part = kStreamWaves * p.chunk * reps;
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
  SDE_STREAM(2, 3)
  SDE_STREAM(2, 4)
  SDE_STREAM(4, 1)
  SDE_STREAM(4, 2)
  SDE_STREAM(4, 3)
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
  a.src.pool = cache->pool;
  a.src.table = sde::layer_table(cache, layer);
  a.src.kv_dim = cache->cfg.kv_dim;
  a.src.bs = cache->cfg.block_size;
  a.src.L_max = L_max;
  a.q = d_q;
  a.out = d_out;
  a.partials = partials;
  a.counters = cache->d_counters;
  a.nh = nh;
  a.G = G;
  a.R = R;
  a.pos_base = pos_base;
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
