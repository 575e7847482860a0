"""GPU parity of the output projection (Wo) through the C-ABI (sde_matvec):
out[m][c] (+)= sum_r x[m][r] W[r][c] with fp16 W [d_in][d_out] and fp32
accumulation -- device_matvec_partial(_accum) / device_matvec_batched
(utils.h:248-280, 417-452; kernels.cu:2742-2747; model.cu:717).

Checked against the float64 product within 1e-5 x sum_r |x_r W_rc| (an
fp32 summation bound; the C restatement of the reference's per-column loop
sits within the same bound), exactly on the closed forms (identity weights,
one-hot inputs), bit-identically across repeated calls (the partial sums
are added in a fixed order), and at the reference's shapes: Llama-3-8B Wo
(4096 x 4096) and W_down (14336 -> 4096), Qwen2.5-7B (3584), TinyLlama
(2048), the tiny model (256), a verify window of 9 rows."""
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
    assert np.array_equal(_run(gpu, x, eye), x)
    _, Wb = _case(rng, 1, 3584, 3584)
    for k in (0, 1791, 3583):
        e = np.zeros((1, 3584), np.float32)
        e[0, k] = 1.0
        assert np.array_equal(_run(gpu, e, Wb)[0], Wb[k].view(np.float16).astype(np.float32))


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
