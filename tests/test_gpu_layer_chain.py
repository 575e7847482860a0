"""The attention half of a decoder layer composed from the library, with
weights from an SDEC file: q, k, v = x @ Wq, Wk, Wv (sde_matvec), RoPE +
append + causal attention in one launch (sde_rope_append_attention), then
hidden += attn @ Wo (sde_matvec, accumulate; and sde_matvec_packed over a
packed copy of the loaded Wo) -- the reference's
model_layer_kv_phase + attention + Wo residual (model.cu:346-435,
kernels.cu:2700-2747) for a decode step and a 5-row verify window.

Each stage is checked against float64 on the inputs the device actually
produced at the previous stage: the projections within the fp32 summation
bound (1e-5 x sum|x W|), the attention within the north_star tolerance
(2e-3 abs + 1e-2 rel) of fp64 attention over the cache and the rows the
kernel stored, and the residual update within the summation bound."""
import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import PackedWeight, matvec, matvec_packed
from speculative_decode_engine_amd import sdec
from test_gpu_attention import assert_close
from test_gpu_fused_rope import build

pytestmark = pytest.mark.gpu
MV_TOL = 1e-5


@pytest.mark.parametrize("d,nh,nkv,ctx,M,theta", [
    (1024, 8, 2, 1500, 1, 500000.0),    # decode step, GQA 4, head_dim 128
    (1024, 8, 2, 1500, 5, 500000.0),    # k = 4 verify window
    (512, 8, 4, 300, 9, 1000000.0),     # 9-row window, head_dim 64
])
def test_attention_sublayer_from_sdec_weights(gpu, oracle, tmp_path, d, nh, nkv, ctx, M, theta):
    case_banner("layer chain", d, nh, nkv, ctx, M)
    dph = d // nh
    kv = nkv * dph
    cfg = dict(n_layers=1, d_model=d, n_heads=nh, n_kv_heads=nkv, d_ff=256, vocab_size=32,
               rope_theta=theta, has_qkv_bias=0)
    rng = np.random.default_rng(d + M)
    t = {n: (rng.standard_normal(s) * (0.6 / np.sqrt(s[0]) if len(s) == 2 else 1.0)
             ).astype(np.float16) for n, s in sdec.tensor_shapes(cfg).items()}
    path = tmp_path / "layer.sdec"
    sdec.write_sdec(path, cfg, t, 5)
    model = sdec.load_sdec(path)
    cache, table, pool_blocks, K, V, rng2 = build(nh, nkv, dph, 16, ctx, M, ctx + M)
    try:
        assert model.config["rope_theta"] == np.float32(theta)
        lw = model.layer(0)
        x = rng.standard_normal((M, d)).astype(np.float32)
        hidden0 = rng.standard_normal((M, d)).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        q = matvec(xd, lw["Wq"])
        k = matvec(xd, lw["Wk"])
        v = matvec(xd, lw["Wv"])
        torch.cuda.synchronize()
        for name, got in (("Wq", q), ("Wk", k), ("Wv", v)):
            y, mag = oracle.matvec_f64(x, t[f"L0.{name}"].view(np.uint16))
            assert np.all(np.abs(got.cpu().numpy() - y) <= MV_TOL * mag + 1e-30), name
        attn = cache.rope_append_attention(0, q, k, v, nh, nkv, dph, ctx,
                                           theta=model.config["rope_theta"])
        hidden = torch.from_numpy(hidden0.copy()).cuda()
        matvec(attn, lw["Wo"], out=hidden, accumulate=True)
        hidden_p = torch.from_numpy(hidden0.copy()).cuda()
        matvec_packed(attn, PackedWeight(lw["Wo"]), out=hidden_p, accumulate=True)
        torch.cuda.synchronize()
        pos = np.arange(ctx, ctx + M)
        gk, gv = cache.read(0, ctx, M)
        gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
        qr = oracle.rope_rotate_half_f64(q.cpu().numpy(), nh, dph, pos, theta=theta)
        ref = oracle.attention_f64_np(qr, np.concatenate([K, gk]), np.concatenate([V, gv]),
                                      nh, nkv, dph, ctx)
        a = attn.cpu().numpy()
        assert_close(a, ref, "attention of the projected, rotated rows")
        y, mag = oracle.matvec_f64(a, t["L0.Wo"].view(np.uint16), hidden0)
        assert np.all(np.abs(hidden.cpu().numpy() - y) <= MV_TOL * mag)
        assert np.all(np.abs(hidden_p.cpu().numpy() - y) <= MV_TOL * mag)
    finally:
        model.free()
        cache.free()
