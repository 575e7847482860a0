// Measurement kernels for bench.py's roofline object (libsde_measure.so):
// reference points measured in the same process as the attention kernel.
// Nothing on the attention path calls them.
//
//  * sde_measure_stream_read: a plain streaming read of a device buffer
//    (16-byte loads, eight in flight per thread, grid-stride), the HBM read
//    rate this part reaches with the simplest access pattern.
//  * sde_measure_attention_loads: the load skeleton of sde_paged_attention
//    for one call -- the same plan, grid, workgroup -> (partition, KV head,
//    row group) mapping, per-wave tile sequence, block-table lookups and
//    16-byte K/V loads, pipelined a tile ahead in the same order -- with the
//    arithmetic, LDS staging, merge and combine taken out.  Its time is the
//    floor of the kernel's own access pattern over the paged pool.
#include <hip/hip_runtime.h>

#include <vector>

#include "sde/attention_device.hpp"
#include "sde_paged_kv.h"

namespace {

using namespace sde::attn;

constexpr uint32_t kSinkMagic = 0x9E3779B9u;  // never the xor of real data in practice

__device__ __forceinline__ uint32_t fold(const uint4& x) { return x.x ^ x.y ^ x.z ^ x.w; }

__global__ __launch_bounds__(512) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          uint32_t* sink) {
  constexpr int kInFlight = 8;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kInFlight - 1) * stride < n16; i += kInFlight * stride) {
    uint4 x[kInFlight];
#pragma unroll
    for (int j = 0; j < kInFlight; j++) x[j] = p[i + j * stride];
#pragma unroll
    for (int j = 0; j < kInFlight; j++) acc ^= fold(x[j]);
  }
  for (; i < n16; i += stride) acc ^= fold(p[i]);
  if (acc == kSinkMagic) sink[0] = acc;  // keeps the loads
}

// A tile's data consumed here (a volatile use: the compiler waits for its
// loads at this point and cannot sink the use past the next tile's loads),
// as the kernel consumes it where it stages the tile.
template <int N>
__device__ __forceinline__ uint32_t consume(const uint4 (&x)[N]) {
  uint32_t acc = 0;
#pragma unroll
  for (int j = 0; j < N; j++) {
    asm volatile("" ::"v"(x[j].x), "v"(x[j].y), "v"(x[j].z), "v"(x[j].w) : "memory");
    acc ^= fold(x[j]);
  }
  return acc;
}

// mfma_chunk's loads (sde/attention_device.hpp) in the same order -- the
// first tile's K and V, then per tile: the next tile's K, this tile's K
// consumed, the next tile's V, this tile's V consumed -- so at most two
// tiles are in flight per wave, as in the kernel.
template <int DPH, int CHUNK>
__device__ __forceinline__ uint32_t pattern_chunk(const TileSource& src, const MfmaWave& w,
                                                  int c0) {
  constexpr int SL = 512 / DPH, NLD = kTile / SL;
  uint4 kbuf[2][NLD], vbuf[2][NLD];
  int blk[2][NLD], slot[2][NLD];
  uint32_t acc = 0;
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
    acc ^= consume(kbuf[b]);
    if (i + 1 < CHUNK) {
      stream_load<DPH>(src, w.head_base, tn * kTile, w.sl, w.lane_off, w.chunk_off, true,
                       blk[nb], slot[nb], vbuf[nb]);
      if (i + 2 < CHUNK)
        tile_groups<NLD, SL>(src, w.table, min(t + 2 * w.stride, w.last) * kTile, blk[b],
                             slot[b]);
    }
    acc ^= consume(vbuf[b]);
  }
  return acc;
}

// One workgroup of sde_paged_attention's grid, loads only (stream_item's
// tile assignment: wave w of partition `part` takes tiles tb+w, tb+w+8, ...).
// It reserves the kernel's LDS (MfmaLds), so the dispatcher places its
// workgroups as it places the kernel's: one per CU.
template <int DPH, int CHUNK>
__global__ __launch_bounds__(64 * kStreamWaves) void attn_pattern_kernel(AttnArgs a,
                                                                        uint32_t* sink) {
  __shared__ MfmaLds<DPH, kStreamWaves> lds;
  const int3 c = stream_coords<CHUNK>();
  const int part = c.x, kvh = c.y;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n_tiles = (a.src.L_max + kTile - 1) / kTile;
  const int tb = part * a.tiles_per_part;
  const int te = part == a.n_parts - 1 ? n_tiles : min(n_tiles, tb + a.tiles_per_part);
  const int first = tb + wave;
  if (first >= te) return;
  constexpr int CH = DPH / 8;
  MfmaWave w;
  w.lane = lane;
  w.sl = lane / CH;
  w.c = lane % CH;
  w.table = const_table(a.src);
  w.head_base = reinterpret_cast<const char*>(a.src.pool) + (size_t)kvh * DPH * 2u;
  w.lane_off = (uint32_t)w.sl * 2u * (uint32_t)a.src.kv_dim + 16u * w.c;
  w.chunk_off = 16u * w.c;
  w.stride = kStreamWaves;
  w.last = first + ((te - 1 - first) / kStreamWaves) * kStreamWaves;
  uint32_t acc = 0;
  for (int c0 = first; c0 < te; c0 += CHUNK * kStreamWaves) acc ^= pattern_chunk<DPH, CHUNK>(a.src, w, c0);
  if (acc == kSinkMagic) {  // (a use of the staging area keeps its reservation)
    lds.st[threadIdx.x * 64 + lane] = (char)acc;
    sink[0] = acc + (uint32_t)lds.st[threadIdx.x * 64];
  }
}

template <int DPH>
int launch_pattern(const StreamPlan& p, const AttnArgs& a, int nkv, uint32_t* sink,
                   hipStream_t s) {
  const dim3 grid(p.n_parts, nkv, p.row_groups);
  switch (p.chunk) {
    case 1: attn_pattern_kernel<DPH, 1><<<grid, 64 * kStreamWaves, 0, s>>>(a, sink); break;
    case 2: attn_pattern_kernel<DPH, 2><<<grid, 64 * kStreamWaves, 0, s>>>(a, sink); break;
    case 3: attn_pattern_kernel<DPH, 3><<<grid, 64 * kStreamWaves, 0, s>>>(a, sink); break;
    default: attn_pattern_kernel<DPH, 4><<<grid, 64 * kStreamWaves, 0, s>>>(a, sink); break;
  }
  return hipGetLastError() == hipSuccess ? SDE_OK : SDE_ERR_HIP;
}

}  // namespace

extern "C" {

// Streaming read of `bytes` (a multiple of 16, 16-byte aligned) at d_buf by
// `blocks` workgroups of 512 threads.  d_sink: one device word (written only
// in the unlikely case the data fold to the sink pattern).
int sde_measure_stream_read(const void* d_buf, size_t bytes, int blocks, uint32_t* d_sink,
                            void* stream) {
  if (!d_buf || !d_sink || bytes == 0 || (bytes & 15) != 0 || ((uintptr_t)d_buf & 15) != 0 ||
      blocks < 1 || blocks > (1 << 20))
    return SDE_ERR_INVALID_ARGUMENT;
  stream_read_kernel<<<blocks, 512, 0, (hipStream_t)stream>>>(
      static_cast<const uint4*>(d_buf), bytes / 16, d_sink);
  return hipGetLastError() == hipSuccess ? SDE_OK : SDE_ERR_HIP;
}

// The load skeleton of sde_paged_attention(cache, layer, ..., nh, nkv, dph,
// pos_base, n_queries) on `n_cus` compute units (head sizes 64 / 128 and
// block sizes that are multiples of 8: the tile kernels' shapes).
int sde_measure_attention_loads(const sde_kv_cache* cache, int layer, int nh, int nkv, int dph,
                                int pos_base, int n_queries, int n_cus, uint32_t* d_sink,
                                void* stream) {
  sde_kv_view v;
  if (!d_sink || sde_kv_get_view(cache, &v) != SDE_OK) return SDE_ERR_INVALID_ARGUMENT;
  if (layer < 0 || layer >= v.n_layers || nh < 1 || nkv < 1 || nh % nkv != 0 ||
      nkv * dph != v.kv_dim || pos_base < 0 || n_queries < 1 || n_cus < 1)
    return SDE_ERR_INVALID_ARGUMENT;
  if ((dph != 64 && dph != 128) || v.block_size % 8 != 0) return SDE_ERR_UNSUPPORTED;
  const int L_max = pos_base + n_queries;
  if ((int64_t)L_max > (int64_t)v.max_blocks_per_layer * v.block_size) return SDE_ERR_CAPACITY;
  // Every block the loads touch must be mapped into the pool.
  const int nblk = (L_max + v.block_size - 1) / v.block_size;
  std::vector<int32_t> table(nblk);
  if (sde_kv_get_block_table(cache, layer, table.data(), nblk) != SDE_OK)
    return SDE_ERR_INVALID_ARGUMENT;
  for (int b = 0; b < nblk; b++)
    if (table[b] < 0 || table[b] >= v.pool_blocks) return SDE_ERR_CAPACITY;
  const int R = n_queries * (nh / nkv);
  const StreamPlan p = stream_plan8_spread(L_max, nkv, R, n_cus);
  AttnArgs a{};
  a.src.pool = v.pool;
  a.src.table = v.block_tables + (size_t)layer * v.max_blocks_per_layer;
  a.src.kv_dim = v.kv_dim;
  a.src.bs = v.block_size;
  a.src.L_max = L_max;
  a.nh = nh;
  a.nkv = nkv;
  a.G = nh / nkv;
  a.R = R;
  a.row_groups = p.row_groups;
  a.pos_base = pos_base;
  a.n_parts = p.n_parts;
  a.tiles_per_part = p.tiles_per_part;
  const hipStream_t s = (hipStream_t)stream;
  return dph == 128 ? launch_pattern<128>(p, a, nkv, d_sink, s)
                    : launch_pattern<64>(p, a, nkv, d_sink, s);
}

}  // extern "C"
