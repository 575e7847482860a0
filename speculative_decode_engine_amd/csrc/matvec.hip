// The output projection after attention (Wo), across all CUs, behind the
// C-ABI: sde_matvec replaces the reference's column-striped
// device_matvec_partial_accum over the blocks of coop_layer_forward
// (utils.h:437-452, kernels.cu:2742-2747), device_matvec_batched for the
// verify window (utils.h:248-280, model.cu:717) and the multi-kernel path's
// Wo GEMM + residual add (kernels.cu:1069-1075, with fp32 activations as in
// the other two).  The work layout and its reduction are described in
// include/sde/matvec_device.hpp.  sde_matvec_pack / sde_matvec_packed run
// the same product over a one-time panel-packed copy of W
// (include/sde/matvec_packed.hpp): one workgroup per panel of output
// columns, no split reduction.
#include <hip/hip_runtime.h>

#include "sde/matvec_device.hpp"
#include "sde/matvec_packed.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace mv {

constexpr int kWaves = 8;

// Workgroup (column tile x, row range y) of pass z (rows 8z.. of x): one or
// two rows of x on the VALU (8 or 16 multiply-adds per loaded 16 bytes keep
// up with the loads), three or more on the matrix cores (measured: 5 rows
// of a 4096 x 4096 projection 25.6 -> 21.6 us, 9 rows 34.4 -> 23.8, 5 rows
// of the 14336 x 4096 W_down 103 -> 40.3; 2 rows 16.7 either way).
template <int MB>
__global__ __launch_bounds__(64 * kWaves) void matvec_kernel(MvArgs a) {
  if constexpr (MB <= 2) {
    __shared__ MvLds<kWaves> lds;
    mv_item<MB, kWaves>(mv_pass(a, blockIdx.z), blockIdx.x, blockIdx.y, lds);
  } else {
    __shared__ MvMfmaLds<kWaves> lds;
    mv_item<MB, kWaves, true>(mv_pass(a, blockIdx.z), blockIdx.x, blockIdx.y, lds);
  }
}

}  // namespace mv

namespace mvp {

// Workgroup (panel, pass).  One row of x takes whole batches per step (8
// units in flight per lane and step); several rows take half batches, whose
// multiply-adds overlap more of the streaming (measured on MI355X, 5 rows
// of the 14336 x 4096 W_down: 24.2 vs 25.2 us) and whose doubled step
// registers stay within 256 VGPRs up to 9 rows.
template <int MB, int LPR>
__global__ __launch_bounds__(64 * kWaves) void matvec_packed_kernel(PackedArgs a) {
  packed_item<MB, LPR, (MB == 1 ? 8 : 4)>(a, blockIdx.x, blockIdx.y);
}

}  // namespace mvp
}  // namespace sde

namespace {

using namespace sde::mv;

// Compute units of the current device, cached per device.
int current_cus(int* status) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    *status = SDE_ERR_NO_DEVICE;
    return 0;
  }
  if (dev < 64 && cus[dev] > 0) return cus[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1) {
    *status = SDE_ERR_HIP;
    return 0;
  }
  if (dev < 64) cus[dev] = n;
  return n;
}

}  // namespace

extern "C" {

size_t sde_matvec_workspace_size(int d_in, int d_out, int M) {
  if (d_in < 1 || d_out < 8 || M < 1 || M > kMaxRows) return 0;
  return mv_workspace_size(d_in, d_out, M);
}

int sde_matvec(const float* d_x, const uint16_t* d_W, float* d_out, int d_in, int d_out_dim,
               int M, int accumulate, void* d_workspace, size_t workspace_bytes,
               sde_stream_t stream) {
  if (!d_x || !d_W || !d_out || d_in < 1 || d_out_dim < 8 || M < 1 || M > kMaxRows)
    return SDE_ERR_INVALID_ARGUMENT;
  if (d_out_dim % 8 != 0 || (reinterpret_cast<uintptr_t>(d_W) & 15u) != 0)
    return SDE_ERR_UNSUPPORTED;
  int st = SDE_OK;
  const int n_cus = current_cus(&st);
  if (st != SDE_OK) return st;
  const MvPlan p = mv_plan(d_in, d_out_dim, n_cus, kWaves, M);
  // A row range is addressed with 32-bit byte offsets.
  if ((size_t)p.rows_per_split * d_out_dim * 2 >= ((size_t)1 << 31)) return SDE_ERR_UNSUPPORTED;
  MvArgs a;
  a.x = d_x;
  a.W = d_W;
  a.out = d_out;
  a.counters = nullptr;
  a.partials = nullptr;
  a.d_in = d_in;
  a.d_out = d_out_dim;
  a.M = M;
  a.splits = p.splits;
  a.rows_per_split = p.rows_per_split;
  a.accumulate = accumulate ? 1 : 0;
  if (p.splits > 1) {
    if (!d_workspace || workspace_bytes < mv_workspace_size(d_in, d_out_dim, M))
      return SDE_ERR_WORKSPACE;
    a.counters = static_cast<uint32_t*>(d_workspace);
    a.partials = reinterpret_cast<float*>(static_cast<char*>(d_workspace) +
                                          mv_counter_bytes(d_out_dim, M));
  }
  const dim3 grid(p.col_tiles, p.splits, mv_passes(M));
  const dim3 block(64 * kWaves);
  const hipStream_t s = (hipStream_t)stream;
  switch (mv_row_bucket(mv_pass_rows(M))) {
    case 1: sde::mv::matvec_kernel<1><<<grid, block, 0, s>>>(a); break;
    case 2: sde::mv::matvec_kernel<2><<<grid, block, 0, s>>>(a); break;
    case 3: sde::mv::matvec_kernel<3><<<grid, block, 0, s>>>(a); break;
    case 4: sde::mv::matvec_kernel<4><<<grid, block, 0, s>>>(a); break;
    case 5: sde::mv::matvec_kernel<5><<<grid, block, 0, s>>>(a); break;
    case 6: sde::mv::matvec_kernel<6><<<grid, block, 0, s>>>(a); break;
    case 7: sde::mv::matvec_kernel<7><<<grid, block, 0, s>>>(a); break;
    default: sde::mv::matvec_kernel<8><<<grid, block, 0, s>>>(a); break;
  }
  return sde::launch_status();
}

size_t sde_matvec_packed_size(int d_in, int d_out) {
  return sde::mvp::packed_shape(d_in, d_out).units * 16;
}

int sde_matvec_pack(const uint16_t* d_W, int d_in, int d_out_dim, void* d_packed,
                    size_t packed_bytes, sde_stream_t stream) {
  if (!d_W || !d_packed || d_in < 1 || d_out_dim < 1) return SDE_ERR_INVALID_ARGUMENT;
  const sde::mvp::PackedShape sh = sde::mvp::packed_shape(d_in, d_out_dim);
  if (sh.panels == 0 || (reinterpret_cast<uintptr_t>(d_W) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(d_packed) & 15u) != 0)
    return SDE_ERR_UNSUPPORTED;
  if (packed_bytes < sh.units * 16) return SDE_ERR_WORKSPACE;
  int st = SDE_OK;
  const int n_cus = current_cus(&st);
  if (st != SDE_OK) return st;
  const size_t want = (sh.units + 255) / 256;
  const int blocks = (int)(want < (size_t)n_cus * 16 ? want : (size_t)n_cus * 16);
  sde::mvp::matvec_pack_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
      d_W, static_cast<uint4*>(d_packed), d_in, d_out_dim);
  return sde::launch_status();
}

int sde_matvec_packed(const float* d_x, const void* d_packed, float* d_out, int d_in,
                      int d_out_dim, int M, int accumulate, sde_stream_t stream) {
  if (!d_x || !d_packed || !d_out || d_in < 1 || d_out_dim < 1 || M < 1 || M > kMaxRows)
    return SDE_ERR_INVALID_ARGUMENT;
  const sde::mvp::PackedShape sh = sde::mvp::packed_shape(d_in, d_out_dim);
  if (sh.panels == 0 || (reinterpret_cast<uintptr_t>(d_x) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(d_packed) & 15u) != 0)
    return SDE_ERR_UNSUPPORTED;
  sde::mvp::PackedArgs a;
  a.W = static_cast<const uint4*>(d_packed);
  a.x = d_x;
  a.out = d_out;
  a.d_in = d_in;
  a.d_out = d_out_dim;
  a.M = M;
  int st = SDE_OK;
  const int n_cus = current_cus(&st);
  if (st != SDE_OK) return st;
  const int passes = sde::mvp::packed_launch_passes(M, sh, n_cus);
  a.pass_rows = (M + passes - 1) / passes;
  a.n_batches = sh.n_batches;
  a.accumulate = accumulate ? 1 : 0;
  const dim3 grid(sh.panels, passes);
  const dim3 block(64 * sde::mvp::kWaves);
  const hipStream_t s = (hipStream_t)stream;
#define SDE_MVP(MB)                                                                  \
  case MB:                                                                           \
    if (sh.lpr == 2)                                                                 \
      sde::mvp::matvec_packed_kernel<MB, 2><<<grid, block, 0, s>>>(a);               \
    else                                                                             \
      sde::mvp::matvec_packed_kernel<MB, 1><<<grid, block, 0, s>>>(a);               \
    break;
  switch (a.pass_rows) {
    SDE_MVP(1) SDE_MVP(2) SDE_MVP(3) SDE_MVP(4) SDE_MVP(5) SDE_MVP(6) SDE_MVP(7) SDE_MVP(8)
    default:
      if (sh.lpr == 2)
        sde::mvp::matvec_packed_kernel<9, 2><<<grid, block, 0, s>>>(a);
      else
        sde::mvp::matvec_packed_kernel<9, 1><<<grid, block, 0, s>>>(a);
      break;
  }
#undef SDE_MVP
  return sde::launch_status();
}

}  // extern "C"
