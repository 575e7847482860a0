"""GPU parity of the panel-packed output projection through the C-ABI
(sde_matvec_pack once, then sde_matvec_packed): the same product as
sde_matvec -- device_matvec_partial(_accum) / device_matvec_batched
(utils.h:248-280, 417-452; kernels.cu:2742-2747; model.cu:717) -- over a
one-time re-layout of W in which one workgroup streams whole output columns.

Checked: the packed bytes equal a numpy restatement of the layout (bit for
bit, zero rows past d_in included); the product is within 1e-5 x
sum_r |x_r W_rc| of float64 (the fp32 summation bound the row-major path and
the C restatement of the reference's per-column loop meet) at the
reference's shapes -- Llama-3-8B Wo and W_down with one row and the verify
window, Qwen2.5-7B, TinyLlama, 16 rows -- and on ragged shapes of both panel
widths; accumulation follows the restatement; identity weights and one-hot
inputs are exact (fp32 products of fp16 weights, sums of zeros); repeated
calls are bit-identical; unsupported shapes and alignments are rejected
before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import (PackedWeight, SDEError, matvec, matvec_packed)
from speculative_decode_engine_amd import _native as N

pytestmark = pytest.mark.gpu
MV_TOL = 1e-5


def packed_layout(Wb: np.ndarray) -> np.ndarray:
    """The documented packed layout of uint16 W [d_in][d_out], as uint16 units
    of 8: unit ((p * nb + b) * 8 + j) * 64 + l holds W[r][c0:c0+8] with
    r = b*BR + (l // LPR)*8 + j, c0 = p*PW + 8*(l % LPR)."""
    d_in, d_out = Wb.shape
    lpr = 2 if (d_out % 16 == 0 and d_out >= 4096) else 1
    pw, br = 8 * lpr, (64 // lpr) * 8
    nb = -(-d_in // br)
    panels = d_out // pw
    Wp = np.zeros((nb * br, d_out), np.uint16)
    Wp[:d_in] = Wb
    # [b][g][j][p][h][8] -> [p][b][j][g][h][8]
    t = Wp.reshape(nb, 64 // lpr, 8, panels, lpr, 8)
    return np.ascontiguousarray(t.transpose(3, 0, 2, 1, 4, 5)).reshape(-1)


def _case(rng, M, d_in, d_out, wscale=0.05):
    x = rng.standard_normal((M, d_in)).astype(np.float32)
    Wb = (rng.standard_normal((d_in, d_out)) * wscale).astype(np.float16).view(np.uint16)
    return x, Wb


def _run(gpu, x, Wb, out0=None, accumulate=False):
    Wp = PackedWeight(torch.from_numpy(Wb.view(np.float16)).to(gpu))
    xt = torch.from_numpy(x).to(gpu)
    out = torch.from_numpy(out0.copy()).to(gpu) if out0 is not None else None
    got = matvec_packed(xt, Wp, out=out, accumulate=accumulate)
    torch.cuda.synchronize()
    return got.cpu().numpy()


@pytest.mark.parametrize("d_in,d_out", [(4096, 4096), (1000, 1032), (264, 4112), (8, 8),
                                        (14336, 4096), (520, 16)])
def test_pack_matches_layout(gpu, d_in, d_out):
    case_banner("matvec pack", d_in, d_out)
    rng = np.random.default_rng(d_in + d_out)
    Wb = rng.integers(0, 1 << 16, size=(d_in, d_out), dtype=np.uint16)
    Wt = torch.from_numpy(Wb.view(np.int16)).to(gpu).view(torch.float16)
    Wp = PackedWeight(Wt)
    torch.cuda.synchronize()
    got = Wp.data.cpu().numpy().view(np.uint16)
    want = packed_layout(Wb)
    assert got.size == want.size == N.load().sde_matvec_packed_size(d_in, d_out) // 2
    assert np.array_equal(got, want)


SHAPES = [
    (1, 4096, 4096),     # Llama-3-8B Wo, decode (16-column panels, one per CU)
    (5, 4096, 4096),     # Llama-3-8B verify window
    (1, 14336, 4096),    # Llama-3-8B W_down
    (5, 14336, 4096),
    (9, 3584, 3584),     # Qwen2.5-7B verify window: three passes of 3 rows, 8-column panels
    (5, 3584, 3584),     # passes of 3 + 2 rows (448 panels, more than one round of the CUs)
    (7, 2048, 2048),     # passes of 3 + 3 + 1 rows (more than 5 rows, 2048 x 2048 fits L2)
    (1, 2048, 2048),     # TinyLlama
    (1, 256, 256),       # tiny model
    (16, 640, 520),      # the largest row count: two passes of 8
    (6, 1000, 1032),     # ragged: d_in not a multiple of a batch, 6 and 7 rows
    (7, 264, 4112),      # 16-column panels with d_in shorter than one batch
    (3, 8, 8),           # one unit row
    (2, 4096, 1024),
    (4, 2048, 2048),     # one pass of 4 rows
    (8, 8192, 512),      # passes of 3 + 3 + 2 rows
]


@pytest.mark.parametrize("M,d_in,d_out", SHAPES)
def test_matvec_packed_matches_float64(gpu, oracle, M, d_in, d_out):
    case_banner("matvec packed", M, d_in, d_out)
    rng = np.random.default_rng(d_in * 17 + d_out + M)
    x, Wb = _case(rng, M, d_in, d_out)
    got = _run(gpu, x, Wb)
    y, mag = oracle.matvec_f64(x, Wb)
    err = np.abs(got - y)
    assert np.all(err <= MV_TOL * mag + 1e-30), float((err / mag).max())


@pytest.mark.parametrize("M,d_in,d_out", [(1, 4096, 4096), (9, 3584, 3584), (2, 304, 24)])
def test_matvec_packed_accumulate(gpu, oracle, M, d_in, d_out):
    case_banner("matvec packed accumulate", M, d_in, d_out)
    rng = np.random.default_rng(11 + M)
    x, Wb = _case(rng, M, d_in, d_out)
    out0 = rng.standard_normal((M, d_out)).astype(np.float32)
    got = _run(gpu, x, Wb, out0, accumulate=True)
    ref = oracle.matvec_ref(x, Wb, out0, accumulate=True)
    y, mag = oracle.matvec_f64(x, Wb, out0)
    assert np.all(np.abs(got - y) <= MV_TOL * mag)
    assert np.all(np.abs(ref - y) <= MV_TOL * mag)


def test_matvec_packed_closed_forms_are_exact(gpu):
    case_banner("matvec packed closed forms")
    rng = np.random.default_rng(5)
    for d, M in ((4096, 5), (2048, 9)):
        eye = np.eye(d, dtype=np.float16).view(np.uint16)
        x = rng.standard_normal((M, d)).astype(np.float32)
        assert np.array_equal(_run(gpu, x, eye), x)
    _, Wb = _case(rng, 1, 3584, 3584)
    ks = (0, 900, 1791, 2700, 3583)
    e = np.zeros((len(ks), 3584), np.float32)
    for m, k in enumerate(ks):
        e[m, k] = 1.0
    got = _run(gpu, e, Wb)
    for m, k in enumerate(ks):
        assert np.array_equal(got[m], Wb[k].view(np.float16).astype(np.float32))


def test_matvec_packed_is_deterministic_and_agrees_with_row_major(gpu, oracle):
    case_banner("matvec packed determinism")
    rng = np.random.default_rng(8)
    x, Wb = _case(rng, 5, 4096, 4096)
    xt = torch.from_numpy(x).to(gpu)
    Wt = torch.from_numpy(Wb.view(np.float16)).to(gpu)
    Wp = PackedWeight(Wt)
    a = matvec_packed(xt, Wp)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = matvec_packed(xt, Wp, stream=s)
    s.synchronize()
    c = matvec_packed(xt, Wp)
    r = matvec(xt, Wt)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    y, mag = oracle.matvec_f64(x, Wb)
    # the two layouts add in different orders: both meet the bound, not the same bits
    assert np.all(np.abs(r.cpu().numpy() - y) <= MV_TOL * mag)
    assert np.all(np.abs(a.cpu().numpy() - y) <= MV_TOL * mag)


def test_matvec_packed_errors(gpu):
    case_banner("matvec packed errors")
    lib = N.load()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib.sde_matvec_packed_size(64, 64) > 0
    for d_in, d_out in ((60, 64), (64, 60), (0, 64), (64, 0), (4, 8)):
        assert lib.sde_matvec_packed_size(d_in, d_out) == 0
    W = torch.zeros(64, 64, dtype=torch.float16, device=gpu)
    need = lib.sde_matvec_packed_size(64, 64)
    buf = torch.zeros(need + 16, dtype=torch.uint8, device=gpu)
    assert lib.sde_matvec_pack(p(W), 64, 64, p(buf), need, None) == 0
    assert lib.sde_matvec_pack(p(W), 64, 64, p(buf), need - 16, None) == 5   # too small
    assert lib.sde_matvec_pack(p(W), 64, 60, p(buf), need, None) == 4        # d_out % 8
    assert lib.sde_matvec_pack(ctypes.c_void_p(W.data_ptr() + 2), 64, 64, p(buf), need,
                               None) == 4                                    # alignment
    assert lib.sde_matvec_pack(None, 64, 64, p(buf), need, None) == 1
    x = torch.zeros(17, 64, device=gpu)
    out = torch.full((17, 64), 7.0, device=gpu)
    assert lib.sde_matvec_packed(p(x), p(buf), p(out), 64, 64, 17, 0, None) == 1   # > 16 rows
    assert lib.sde_matvec_packed(p(x), p(buf), p(out), 64, 64, 0, 0, None) == 1
    assert lib.sde_matvec_packed(ctypes.c_void_p(x.data_ptr() + 4), p(buf), p(out), 64, 64, 1,
                                 0, None) == 4                               # x alignment
    assert lib.sde_matvec_packed(p(x), p(buf), p(out), 60, 64, 1, 0, None) == 4    # d_in % 8
    assert lib.sde_matvec_packed(p(x), None, p(out), 64, 64, 1, 0, None) == 1
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)  # nothing launched
    with pytest.raises(ValueError):
        PackedWeight(torch.zeros(60, 64, dtype=torch.float16, device=gpu))
    with pytest.raises(SDEError):
        matvec_packed(torch.zeros(17, 64, device=gpu), PackedWeight(W))
