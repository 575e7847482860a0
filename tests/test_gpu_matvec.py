"""GPU parity of the output projection (Wo) through the C-ABI (sde_matvec):
out[m][c] (+)= sum_r x[m][r] W[r][c] with fp16 W [d_in][d_out] and fp32
accumulation -- device_matvec_partial(_accum) / device_matvec_batched
(utils.h:248-280, 417-452; kernels.cu:2742-2747; model.cu:717).

Checked against the float64 product within 1e-5 x sum_r |x_r W_rc| (an
fp32 summation bound; the C restatement of the reference's per-column loop
sits within the same bound), on the closed forms (identity weights exactly
for one or two rows of x, which run on the VALU, and within 2^-21 of x for
three or more, which reach the matrix cores as fp16 hi + lo parts (or
2^-25 absolute where lo is an fp16 subnormal); one-hot
inputs exactly on both), bit-identically across repeated calls (the partial
sums are added in a fixed order), and at the reference's shapes: Llama-3-8B Wo
(4096 x 4096) and W_down (14336 -> 4096), Qwen2.5-7B (3584), TinyLlama
(2048), the tiny model (256), a verify window of 9 rows."""
import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import SDEError, matvec, matvec_workspace
from speculative_decode_engine_amd import _native as N

pytestmark = pytest.mark.gpu
MV_TOL = 1e-5


def _case(rng, M, d_in, d_out, wscale=0.05):
    x = rng.standard_normal((M, d_in)).astype(np.float32)
    Wb = (rng.standard_normal((d_in, d_out)) * wscale).astype(np.float16).view(np.uint16)
    return x, Wb


def _run(gpu, x, Wb, out0=None, accumulate=False):
    xt = torch.from_numpy(x).to(gpu)
    Wt = torch.from_numpy(Wb.view(np.float16)).to(gpu)
    out = torch.from_numpy(out0.copy()).to(gpu) if out0 is not None else None
    got = matvec(xt, Wt, out=out, accumulate=accumulate)
    torch.cuda.synchronize()
    return got.cpu().numpy()


SHAPES = [
    (1, 4096, 4096),     # Llama-3-8B Wo, decode
    (5, 4096, 4096),     # Llama-3-8B verify window
    (1, 14336, 4096),    # Llama-3-8B W_down (same function in coop_layer_forward)
    (9, 3584, 3584),     # Qwen2.5-7B verify window
    (1, 2048, 2048),     # TinyLlama
    (1, 256, 256),       # tiny model
    (3, 1000, 1032),     # ragged: rows not a multiple of the tiling, partial column tile
    (1, 7, 8),           # fewer rows than one wave's batch
    (16, 640, 520),      # the largest row count
    (2, 4096, 1024),     # every row count has its own unrolled instantiation:
    (3, 14336, 1024),    #   3 rows split 20 ways (the combine's quarters hold 5 each)
    (4, 2048, 2048),
    (6, 8192, 512),      #   6 and 7 rows: 8 row ranges at most
    (7, 8192, 512),
    (2, 200, 264),       # d_in < 256: one row range, so 2/4/8 rows take the direct
    (4, 120, 512),       #   single-split write, odd rows through the second LDS
    (8, 255, 1032),      #   reduction buffer
]


@pytest.mark.parametrize("M,d_in,d_out", SHAPES)
def test_matvec_matches_float64(gpu, oracle, M, d_in, d_out):
    case_banner("matvec", M, d_in, d_out)
    rng = np.random.default_rng(d_in * 31 + d_out + M)
    x, Wb = _case(rng, M, d_in, d_out)
    got = _run(gpu, x, Wb)
    y, mag = oracle.matvec_f64(x, Wb)
    err = np.abs(got - y)
    assert np.all(err <= MV_TOL * mag + 1e-30), float((err / mag).max())


@pytest.mark.parametrize("M,d_in,d_out", [(1, 4096, 4096), (9, 3584, 3584), (2, 300, 24)])
def test_matvec_accumulate_matches_reference_restatement(gpu, oracle, M, d_in, d_out):
    case_banner("matvec accumulate", M, d_in, d_out)
    rng = np.random.default_rng(7 + M)
    x, Wb = _case(rng, M, d_in, d_out)
    out0 = rng.standard_normal((M, d_out)).astype(np.float32)
    got = _run(gpu, x, Wb, out0, accumulate=True)
    ref = oracle.matvec_ref(x, Wb, out0, accumulate=True)
    y, mag = oracle.matvec_f64(x, Wb, out0)
    assert np.all(np.abs(got - y) <= MV_TOL * mag)
    assert np.all(np.abs(ref - y) <= MV_TOL * mag)


def test_matvec_closed_forms_are_exact(gpu):
    case_banner("matvec closed forms")
    rng = np.random.default_rng(3)
    d = 4096
    eye = np.eye(d, dtype=np.float16).view(np.uint16)
    x = rng.standard_normal((2, d)).astype(np.float32)
    assert np.array_equal(_run(gpu, x, eye), x)            # VALU: exact products
    x5 = rng.standard_normal((5, d)).astype(np.float32)
    got5 = _run(gpu, x5, eye)                              # matrix cores: x as hi + lo
    # |x - hi - lo| <= 2^-22 |x| for normal lo, half an fp16 subnormal step (2^-25) below
    assert np.all(np.abs(got5 - x5) <= np.maximum(2.0 ** -21 * np.abs(x5), 2.0 ** -25))
    assert not np.array_equal(got5, x5)  # (the lo part's rounding shows: this is the MFMA path)
    _, Wb = _case(rng, 1, 3584, 3584)
    for k in (0, 1791, 3583):
        e = np.zeros((1, 3584), np.float32)
        e[0, k] = 1.0
        assert np.array_equal(_run(gpu, e, Wb)[0], Wb[k].view(np.float16).astype(np.float32))
    e5 = np.zeros((5, 3584), np.float32)
    for m, k in enumerate((0, 900, 1791, 2700, 3583)):
        e5[m, k] = 1.0
    got = _run(gpu, e5, Wb)
    for m, k in enumerate((0, 900, 1791, 2700, 3583)):
        assert np.array_equal(got[m], Wb[k].view(np.float16).astype(np.float32))


@pytest.mark.parametrize("M,d_in,d_out", [(5, 4096, 4096), (3, 14336, 1024), (9, 3584, 3584)])
def test_matvec_large_inputs_beyond_fp16_range(gpu, oracle, M, d_in, d_out):
    """Rows of x past the fp16 range (|x| up to 1e9) on the matrix-core form
    (three or more rows): every row is scaled by a power of two for the
    fp16 hi + lo split and scaled back, so the result stays within the fp32
    summation bound of the float64 product, with no Inf; scaling x by 2^k
    scales the result by exactly 2^k."""
    case_banner("matvec large x", M, d_in, d_out)
    rng = np.random.default_rng(M * 7 + d_in)
    x, Wb = _case(rng, M, d_in, d_out)
    x[0] *= np.float32(1e9)               # row 0: every element past 65504
    x[1, ::97] = np.float32(3.0e5)        # row 1: a few elements past it
    got = _run(gpu, x, Wb)
    assert np.all(np.isfinite(got))
    y, mag = oracle.matvec_f64(x, Wb)
    err = np.abs(got - y)
    assert np.all(err <= MV_TOL * mag + 1e-30), float((err / mag).max())
    # Rows past the range are normalized by their power-of-two scale, so two
    # power-of-two multiples of a row give exactly proportional results (an
    # in-range row keeps scale 1 and its own fp16 rounding of the lo part).
    x2, x3 = x.copy(), x.copy()
    x2[2] *= np.float32(2.0 ** 20)
    x3[2] *= np.float32(2.0 ** 24)
    got2, got3 = _run(gpu, x2, Wb), _run(gpu, x3, Wb)
    assert np.array_equal(got3[2], got2[2] * np.float32(16.0))
    y2, mag2 = oracle.matvec_f64(x2, Wb)
    assert np.all(np.abs(got2 - y2) <= MV_TOL * mag2 + 1e-30)
    assert np.array_equal(got2[3:], got[3:]) and np.array_equal(got2[:2], got[:2])


def test_matvec_is_deterministic(gpu):
    case_banner("matvec determinism")
    rng = np.random.default_rng(5)
    x, Wb = _case(rng, 5, 4096, 4096)
    xt = torch.from_numpy(x).to(gpu)
    Wt = torch.from_numpy(Wb.view(np.float16)).to(gpu)
    ws = matvec_workspace(4096, 4096, 5, gpu)
    a = matvec(xt, Wt, workspace=ws)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = matvec(xt, Wt, workspace=ws, stream=s)
    s.synchronize()
    c = matvec(xt, Wt, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)


def test_matvec_errors(gpu):
    case_banner("matvec errors")
    lib = N.load()
    x = torch.zeros(1, 64, device=gpu)
    W = torch.zeros(64, 64, dtype=torch.float16, device=gpu)
    out = torch.zeros(1, 64, device=gpu)
    need = lib.sde_matvec_workspace_size(64, 64, 1)
    assert need > 0 and lib.sde_matvec_workspace_size(64, 12, 1) > 0
    assert lib.sde_matvec_workspace_size(64, 64, 17) == 0
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    p = lambda t: t.data_ptr()
    assert lib.sde_matvec(p(x), p(W), p(out), 64, 64, 1, 0, p(ws), need, None) == 0
    assert lib.sde_matvec(p(x), p(W), p(out), 64, 60, 1, 0, p(ws), need, None) == 4  # d_out % 8
    assert lib.sde_matvec(p(x), p(W) + 2, p(out), 64, 64, 1, 0, p(ws), need, None) == 4
    assert lib.sde_matvec(p(x), p(W), p(out), 64, 64, 17, 0, p(ws), need, None) == 1
    assert lib.sde_matvec(None, p(W), p(out), 64, 64, 1, 0, p(ws), need, None) == 1
    assert lib.sde_matvec(p(x), p(W), p(out), 0, 64, 1, 0, p(ws), need, None) == 1
    big_x = torch.zeros(1, 4096, device=gpu)
    big_W = torch.zeros(4096, 4096, dtype=torch.float16, device=gpu)
    big_out = torch.zeros(1, 4096, device=gpu)
    assert lib.sde_matvec(p(big_x), p(big_W), p(big_out), 4096, 4096, 1, 0, p(ws), need,
                          None) == 5  # workspace too small for the split plan
    torch.cuda.synchronize()
    with pytest.raises(SDEError):
        matvec(big_x, big_W, workspace=ws)


# ---- the device-side API (include/sde/matvec_device.hpp) -----------------------
# Kernels in tests/device/device_api_test.hip call the reference-named
# block-level functions the way coop_layer_forward does (GEMV_COL_TILE = 128
# column stripes taken by blocks in turns, config.h:29, kernels.cu:2742-2747),
# device_matvec_batched from one block, and the grid-cooperative projection
# from every block of arbitrary grids.

DEV_LIB = Path(__file__).resolve().parent / "device" / "libsde_device_test.so"


@pytest.fixture(scope="module")
def mvdev(gpu):
    if not DEV_LIB.exists():
        pytest.fail(f"{DEV_LIB} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(DEV_LIB))
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.sdet_stripe_matvec.argtypes = [vp, vp, vp, i, i, i, i, i, i, vp]
    lib.sdet_batched_matvec.argtypes = [vp, vp, vp, i, i, i, i, vp]
    lib.sdet_grid_matvec.argtypes = [vp, vp, vp, i, i, i, i, i, i, vp, sz, vp, vp]
    for f in (lib.sdet_stripe_matvec, lib.sdet_batched_matvec, lib.sdet_grid_matvec):
        f.restype = i
    return lib


def _dev_tensors(gpu, x, Wb, out0):
    return (torch.from_numpy(x).to(gpu), torch.from_numpy(Wb.view(np.float16)).to(gpu),
            torch.from_numpy(out0.copy()).to(gpu))


@pytest.mark.parametrize("d_in,d_out,tile,blocks,threads,acc", [
    (4096, 4096, 128, 256, 256, 1),    # Llama-3-8B Wo, the reference's stripes
    (3584, 3584, 128, 19, 512, 1),     # Qwen2.5-7B, fewer blocks than stripes
    (14336, 4096, 128, 64, 1024, 1),   # W_down
    (1000, 1032, 128, 5, 64, 0),       # ragged last stripe, one-wave blocks
    (256, 256, 48, 3, 320, 0),         # stripes not a power of two, five-wave blocks
])
def test_block_matvec_stripes(gpu, mvdev, oracle, d_in, d_out, tile, blocks, threads, acc):
    case_banner("block matvec", d_in, d_out, tile, blocks, threads, acc)
    rng = np.random.default_rng(d_in + tile)
    x, Wb = _case(rng, 1, d_in, d_out)
    out0 = rng.standard_normal((1, d_out)).astype(np.float32)
    xt, Wt, ot = _dev_tensors(gpu, x, Wb, out0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert mvdev.sdet_stripe_matvec(xt.data_ptr(), Wt.data_ptr(), ot.data_ptr(), d_in, d_out,
                                    tile, acc, blocks, threads, s) == 0
    torch.cuda.synchronize()
    y, mag = oracle.matvec_f64(x, Wb, out0 if acc else None)
    got = ot.cpu().numpy()
    assert np.all(np.abs(got - y) <= MV_TOL * mag + 1e-30)


@pytest.mark.parametrize("B,d_in,d_out,threads", [(5, 4096, 4096, 1024), (9, 3584, 3584, 256),
                                                  (2, 64, 8, 64)])
def test_block_matvec_batched(gpu, mvdev, oracle, B, d_in, d_out, threads):
    case_banner("batched matvec", B, d_in, d_out, threads)
    rng = np.random.default_rng(B * 7 + d_in)
    x, Wb = _case(rng, B, d_in, d_out)
    xt, Wt, ot = _dev_tensors(gpu, x, Wb, np.full((B, d_out), np.nan, np.float32))
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert mvdev.sdet_batched_matvec(xt.data_ptr(), Wt.data_ptr(), ot.data_ptr(), d_in, d_out, B,
                                     threads, s) == 0
    torch.cuda.synchronize()
    y, mag = oracle.matvec_f64(x, Wb)
    assert np.all(np.abs(ot.cpu().numpy() - y) <= MV_TOL * mag + 1e-30)


def _grid_mv(mvdev, gpu, xt, Wt, ot, M, d_in, d_out, acc, blocks, threads, ws, ws_bytes=None):
    status = torch.full((blocks,), -1, dtype=torch.int32, device=gpu)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert mvdev.sdet_grid_matvec(xt.data_ptr(), Wt.data_ptr(), ot.data_ptr(), d_in, d_out, M,
                                  acc, blocks, threads, ws.data_ptr(),
                                  ws.numel() if ws_bytes is None else ws_bytes,
                                  status.data_ptr(), s) == 0
    torch.cuda.synchronize()
    return status.cpu().numpy()


@pytest.mark.parametrize("M,d_in,d_out,acc,blocks,threads", [
    (1, 4096, 4096, 1, 256, 512),     # decode Wo on a one-block-per-CU persistent grid
    (9, 3584, 3584, 0, 300, 256),     # Qwen verify window, 4-wave blocks, two row passes
    (16, 640, 520, 1, 7, 1024),       # the largest row count, fewer blocks than items
    (1, 7, 8, 0, 3, 320),             # fewer rows than one batch
    (2, 200, 2048, 1, 3, 512),        # d_in < 256 (single split): 2, 4 and 8 rows, odd
    (4, 120, 1032, 0, 2, 256),        #   rows through the second reduction buffer, blocks
    (8, 255, 4096, 1, 5, 512),        #   taking several column tiles each
])
def test_grid_matvec(gpu, mvdev, oracle, M, d_in, d_out, acc, blocks, threads):
    case_banner("grid matvec", M, d_in, d_out, acc, blocks, threads)
    rng = np.random.default_rng(M + d_in + blocks)
    x, Wb = _case(rng, M, d_in, d_out)
    out0 = rng.standard_normal((M, d_out)).astype(np.float32)
    xt, Wt, _ = _dev_tensors(gpu, x, Wb, out0)
    ws = matvec_workspace(d_in, d_out, M, gpu)
    y, mag = oracle.matvec_f64(x, Wb, out0 if acc else None)
    first = None
    for call in range(2):   # the second call finds the counters the first left at zero
        ot = torch.from_numpy(out0.copy()).to(gpu)
        status = _grid_mv(mvdev, gpu, xt, Wt, ot, M, d_in, d_out, acc, blocks, threads, ws)
        assert (status == 0).all()
        got = ot.cpu().numpy()
        assert np.all(np.abs(got - y) <= MV_TOL * mag + 1e-30)
        if first is None:
            first = got
        else:
            assert np.array_equal(got, first)
    host = matvec(xt, Wt, out=torch.from_numpy(out0.copy()).to(gpu), accumulate=bool(acc))
    torch.cuda.synchronize()
    assert np.all(np.abs(host.cpu().numpy() - y) <= MV_TOL * mag + 1e-30)


def test_grid_matvec_errors_write_nothing(gpu, mvdev):
    case_banner("grid matvec errors")
    rng = np.random.default_rng(1)
    x, Wb = _case(rng, 1, 4096, 4096)
    xt, Wt, _ = _dev_tensors(gpu, x, Wb, np.zeros((1, 4096), np.float32))
    ws = matvec_workspace(4096, 4096, 1, gpu)
    nan = torch.full((1, 4096), float("nan"), device=gpu)
    ot = nan.clone()
    st = _grid_mv(mvdev, gpu, xt, Wt, ot, 1, 4096, 4096, 0, 8, 512, ws, ws.numel() // 2)
    assert (st == N.SDE_ERR_WORKSPACE).all() and torch.isnan(ot).all()
    st = _grid_mv(mvdev, gpu, xt, Wt, ot, 1, 4096, 4096, 0, 8, 192, ws)
    assert (st == N.SDE_ERR_UNSUPPORTED).all() and torch.isnan(ot).all()
    st = _grid_mv(mvdev, gpu, xt, Wt, ot, 17, 4096, 4096, 0, 8, 512, ws)
    assert (st == N.SDE_ERR_INVALID_ARGUMENT).all() and torch.isnan(ot).all()
