"""GPU parity of the attention path for head sizes other than 64 / 128 and
block sizes that are not a multiple of 8 (the reference's
device_flash_attention_gqa, attention.h:21-126, loops over any dph), through
the same C-ABI entry points: sde_paged_attention, sde_attention_dispatch,
sde_rope_append_attention and sde_paged_attention_noalloc.

Checked against the fp64 oracle (oracle.attention_f64_np over the gathered
fp16 K/V) within the north_star tolerance, at head sizes 32, 48, 80, 96,
100, 112, 160, 256, 512 and 7 (odd), block sizes 1, 3, 4, 12, 16 and 20,
contexts from none (a window alone) to 20000 keys (multi-partition
combine), GQA ratios 1-8, windows of 1-9 queries; a window equals the
single-query calls at the same positions; Inf / NaN V rows the causal rule
hides from earlier queries stay out of their outputs; the fused RoPE entry
point stores V bit-exactly and K within one fp16 ulp of the float64
rotation; a head size above 512 is rejected."""
import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import KVCache, SDEError
from speculative_decode_engine_amd import _native as N
from speculative_decode_engine_amd import workloads as W
from test_gpu_attention import assert_close, build_layer

pytestmark = pytest.mark.gpu

CASES = [
    # nh, nkv, dph, bs, ctx, M
    (8, 2, 96, 16, 1000, 1),      # head size 96 (Phi-3-mini), decode
    (8, 2, 96, 16, 1000, 5),      # verify window
    (32, 32, 80, 16, 2047, 1),    # head size 80 (Phi-2), MHA
    (16, 2, 256, 16, 4096, 1),    # head size 256 (Gemma)
    (16, 2, 256, 16, 600, 9),     # 9-query window over 256-wide heads
    (8, 8, 32, 16, 300, 3),       # head size 32
    (12, 4, 48, 12, 777, 4),      # head size 48, block size 12
    (8, 1, 112, 3, 500, 2),       # block size 3, G = 8
    (4, 2, 100, 20, 1234, 1),     # head size not a multiple of 8
    (4, 4, 7, 4, 333, 5),         # odd head size
    (2, 1, 160, 1, 257, 1),       # block size 1
    (8, 2, 64, 12, 3000, 5),      # head size 64 with a block size the tile kernels reject
    (8, 2, 128, 20, 20000, 1),    # 20000 keys: a multi-partition combine
    (4, 2, 512, 16, 2000, 2),     # the largest head size
    (8, 2, 96, 16, 0, 6),         # no context: the window alone
    # partials capped to the no-allocation array (plans that asked for
    # 4.23 MB at 16129 keys before the cap)
    (16, 8, 256, 16, 16125, 4),   # head size 256, 4-query window
    (64, 8, 256, 16, 16128, 1),   # head size 256, 64 q heads
    (32, 4, 512, 16, 16128, 1),   # head size 512
]


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M", CASES)
def test_generic_attention_matches_float64(gpu, oracle, nh, nkv, dph, bs, ctx, M):
    case_banner("generic attention", nh, nkv, dph, bs, ctx, M)
    nblk = -(-(ctx + M) // bs)
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, nblk + 17, dph * 7 + bs + ctx)
    q = W.queries(rng, M, nh, dph)
    qt = torch.from_numpy(q).cuda()
    out = cache.attention(0, qt, nh, nkv, dph, ctx)
    ref = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
    assert_close(out.cpu().numpy(), ref, f"dph {dph} bs {bs}")
    # sde_attention_dispatch and the allocation-free entry point run the same path
    out2 = cache.attention(0, qt, nh, nkv, dph, ctx, attn_type=N.SDE_ATTN_SOFTMAX)
    out3 = cache.attention_noalloc(0, qt, nh, nkv, dph, ctx,
                                   out=torch.full_like(out, float("nan")))
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(out, out3)
    cache.free()


def test_generic_window_equals_single_query_calls(gpu, oracle):
    case_banner("generic window vs single queries")
    nh, nkv, dph, bs, ctx, M = 8, 2, 96, 12, 900, 5
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, -(-(ctx + M) // bs) + 3, 5)
    q = W.queries(rng, M, nh, dph)
    win = cache.attention(0, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx).cpu().numpy()
    for m in range(M):
        one = cache.attention(0, torch.from_numpy(q[m:m + 1]).cuda(), nh, nkv, dph, ctx + m)
        ref = oracle.attention_f64_np(q[m:m + 1], K[:ctx + m + 1], V[:ctx + m + 1], nh, nkv,
                                      dph, ctx + m)
        assert_close(one.cpu().numpy(), ref, f"query {m} alone")
        assert np.allclose(one.cpu().numpy()[0], win[m], rtol=0, atol=2e-6)
    cache.free()


def test_generic_hidden_nonfinite_window_rows(gpu, oracle):
    """Window rows 2-4 hold Inf / NaN V (and K); queries 0 and 1 must not see
    them (attention.h:52-63 reads only positions < total_len)."""
    case_banner("generic hidden non-finite rows")
    nh, nkv, dph, bs, ctx, M = 8, 2, 80, 12, 500, 5
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, -(-(ctx + M) // bs) + 3, 9)
    bad_k = np.full((3, nkv * dph), np.inf, np.float32)
    bad_v = np.full((3, nkv * dph), np.nan, np.float32)
    bad_v[0] = np.inf
    cache.append(0, torch.from_numpy(bad_k).cuda(), torch.from_numpy(bad_v).cuda(), ctx + 2)
    q = W.queries(rng, M, nh, dph)
    out = cache.attention(0, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx).cpu().numpy()
    ref = oracle.attention_f64_np(q[:2], K[:ctx + 2], V[:ctx + 2], nh, nkv, dph, ctx)
    assert_close(out[:2], ref, "queries before the non-finite rows")
    assert not np.isfinite(out[2:]).all()  # later queries see them, as in the reference
    cache.free()


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M,stype,factor,theta", [
    (8, 2, 96, 16, 1000, 5, 0, 1.0, 10000.0),
    (16, 2, 256, 12, 700, 3, 2, 4.0, 500000.0),   # NTK
    (4, 4, 80, 3, 300, 9, 1, 2.0, 10000.0),       # linear scaling, block size 3
    (8, 2, 64, 12, 2000, 1, 3, 2.0, 0.0),         # YaRN, default theta, tile-rejected block size
])
def test_generic_fused_rope_append_attention(gpu, oracle, nh, nkv, dph, bs, ctx, M, stype,
                                             factor, theta):
    case_banner("generic fused rope", nh, nkv, dph, bs, ctx, M, stype)
    from test_gpu_fused_rope import build
    cache, table, pool_blocks, K, V, rng = build(nh, nkv, dph, bs, ctx, M, dph + bs)
    kv_dim = nkv * dph
    q = W.queries(rng, M, nh, dph)
    k = rng.standard_normal((M, kv_dim)).astype(np.float32)
    v = rng.standard_normal((M, kv_dim)).astype(np.float32)
    before = cache.pool.clone()
    out = cache.rope_append_attention(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                      torch.from_numpy(v).cuda(), nh, nkv, dph, ctx,
                                      theta=theta, scaling_type=stype, scaling_factor=factor)
    torch.cuda.synchronize()
    pos = np.arange(ctx, ctx + M)
    kr = oracle.rope_rotate_half_f64(k, nkv, dph, pos, theta, stype, factor)
    qr = oracle.rope_rotate_half_f64(q, nh, dph, pos, theta, stype, factor)
    gk, gv = cache.read(0, ctx, M)
    gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
    assert np.array_equal(gv, v.astype(np.float16).astype(np.float32))
    want = kr.astype(np.float16)
    got16 = gk.astype(np.float16)
    ulp = np.abs(got16.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1 and (ulp == 0).mean() >= 0.99
    ref = oracle.attention_f64_np(qr, np.concatenate([K, gk]), np.concatenate([V, gv]), nh, nkv,
                                  dph, ctx)
    assert_close(out.cpu().numpy(), ref, "generic fused")
    # only the window's rows changed
    after = cache.pool
    changed = (after != before).nonzero().flatten().cpu().numpy()
    blk = 2 * bs * kv_dim
    rows = set()
    for e in changed:
        b, off = divmod(int(e), blk)
        slot = (off % (bs * kv_dim)) // kv_dim
        rows.add((b, slot))
    allowed = {(int(table[p // bs]), p % bs) for p in pos}
    assert rows <= allowed
    cache.free()


def test_generic_rejects_head_size_above_512(gpu):
    case_banner("generic head size limit")
    cache = KVCache(1, 520, 4, 16, pool_blocks=4)
    with pytest.raises(SDEError) as e:
        cache.attention(0, torch.zeros(1, 520, device="cuda"), 1, 1, 520, 0)
    assert e.value.status == N.SDE_ERR_UNSUPPORTED
    cache.free()
