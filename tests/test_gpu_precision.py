"""GPU parity of attention at the edges of its arithmetic, through the C-ABI.

1. Sharp attention: q scaled x8 and x16 (logits spanning about +-50 to
   +-70) at the 32K decode and the Qwen2.5-7B 9-query verify shapes.  The
   reference multiplies fp32 q by the widened fp16 K and fp32 weights by
   the widened V (attention.h:61-62, 103-112); the kernels feed q and the
   weights to the matrix cores as fp16 hi + lo pairs, so the contract (2e-3
   abs + 1e-2 rel against fp64) holds here too, and a tighter bound (2e-4 of
   the output's scale) catches a lost lo part: fp16 q alone errs by about
   |logit| * 2^-11 ~ 3 % in the weights at these scales.

2. Non-finite K/V in a verify window's own rows: query m of a window sees
   positions [0, pos_base+m] (kernels.cu:904-940); the reference never
   reads a hidden row (attention.h:52, 98-115).  Rows 2-4 of the window
   hold +-Inf (fp32 values past the fp16 range, rounded by the append) and
   NaN.  Queries 0-1 must match the fp64 oracle; later queries, which see
   the poisoned rows, must be non-finite exactly where the oracle's literal
   fp32 restatement of attention.h (mode "tiled") is, and in tolerance
   elsewhere.
"""
import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import KVCache
from speculative_decode_engine_amd import workloads as W
from test_gpu_attention import assert_close

pytestmark = pytest.mark.gpu


def _cache_with_context(nh, nkv, dph, bs, ctx, M, seed):
    rng = np.random.default_rng(seed)
    kv_dim = nkv * dph
    nblk = -(-(ctx + M) // bs)
    pool_blocks = nblk + 37
    table = W.make_tables(rng, 1, nblk, pool_blocks)[0]
    cache = KVCache(1, kv_dim, nblk, bs, pool_blocks)
    cache.set_block_table(0, table)
    kc, vc = W.context_kv(rng, ctx, kv_dim)
    cache.write_fp16(0, torch.from_numpy(kc.view(np.int16)).cuda(),
                     torch.from_numpy(vc.view(np.int16)).cuda(), 0)
    return cache, table, pool_blocks, kc, vc, rng


SHARP = [
    # name, nh, nkv, dph, bs, ctx, M
    ("llama3_8b_32k", 32, 8, 128, 16, 32767, 1),
    ("qwen25_7b_verify", 28, 4, 128, 32, 8192, 9),
]


@pytest.mark.parametrize("scale", [8.0, 16.0])
@pytest.mark.parametrize("name,nh,nkv,dph,bs,ctx,M", SHARP)
def test_sharp_logits(gpu, oracle, name, nh, nkv, dph, bs, ctx, M, scale):
    case_banner("sharp logits", name, scale)
    cache, table, pool_blocks, kc, vc, rng = _cache_with_context(nh, nkv, dph, bs, ctx, M,
                                                                 int(scale) + ctx)
    k, v = W.new_kv(rng, M, nkv * dph)
    cache.append(0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), ctx)
    K = np.concatenate([kc.astype(np.float32), k.astype(np.float16).astype(np.float32)])
    V = np.concatenate([vc.astype(np.float32), v.astype(np.float16).astype(np.float32)])
    q = (W.queries(rng, M, nh, dph) * np.float32(scale)).astype(np.float32)
    logits = (q.reshape(M, nh, dph)[:, 0] @ K[:, :dph].T) / np.sqrt(dph)
    assert np.abs(logits).max() > 4 * scale  # the shape is as sharp as intended
    out = cache.attention(0, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx)
    torch.cuda.synchronize()
    ref = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
    got = out.cpu().numpy()
    assert_close(got, ref, f"{name} x{scale}")
    err = np.abs(got.astype(np.float64) - ref).max()
    assert err <= 2e-4 * np.abs(ref).max(), f"{name} x{scale}: max abs err {err:.3e}"
    cache.free()


def test_sharp_logits_fused_rope(gpu, oracle):
    """The fused RoPE + append + attention step at the Qwen2.5-7B verify
    shape with q x16: the rotated q enters the matrix cores split too."""
    case_banner("sharp logits fused")
    nh, nkv, dph, bs, ctx, M = 28, 4, 128, 32, 8192, 9
    cache, table, pool_blocks, kc, vc, rng = _cache_with_context(nh, nkv, dph, bs, ctx, M, 716)
    q = (rng.standard_normal((M, nh * dph), dtype=np.float32) * np.float32(16.0))
    k = rng.standard_normal((M, nkv * dph), dtype=np.float32)
    v = rng.standard_normal((M, nkv * dph), dtype=np.float32)
    out = cache.rope_append_attention(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                      torch.from_numpy(v).cuda(), nh, nkv, dph, ctx,
                                      theta=1000000.0)
    torch.cuda.synchronize()
    gk, gv = cache.read(0, ctx, M)
    qr = oracle.rope_rotate_half_f64(q, nh, dph, np.arange(ctx, ctx + M), theta=1000000.0)
    ref = oracle.attention_f64_np(qr, np.concatenate([kc.astype(np.float32), gk.cpu().numpy()]),
                                  np.concatenate([vc.astype(np.float32), gv.cpu().numpy()]),
                                  nh, nkv, dph, ctx)
    got = out.cpu().numpy()
    assert_close(got, ref, "fused x16")
    err = np.abs(got.astype(np.float64) - ref).max()
    assert err <= 2e-4 * np.abs(ref).max(), f"fused x16: max abs err {err:.3e}"
    cache.free()


def poisoned_window(rng, M, kv_dim, poison_k):
    """Window rows with non-finite values from row 2 on: V +Inf (1e6 rounds
    to fp16 +Inf), NaN, -Inf; with poison_k also NaN and +Inf in K."""
    k, v = W.new_kv(rng, M, kv_dim)
    v[2, ::3] = 1e6
    v[3, 5::7] = np.nan
    v[4, 1::5] = -1e6
    if poison_k:
        k[3, 9::13] = np.nan
        k[4, ::11] = 7e4
    return k, v


def check_poisoned(got, f64, tiled, what, first=2):
    """Queries < first: finite and in tolerance; the others: non-finite
    exactly where the reference restatement is, in tolerance elsewhere."""
    got = np.asarray(got, np.float64)
    assert_close(got[:first], f64[:first], f"{what}: queries before the poisoned rows")
    mask = np.isfinite(tiled[first:])
    assert (~mask).any(), f"{what}: the poisoned rows must reach the later queries"
    bad = np.isfinite(got[first:]) != mask
    assert not bad.any(), f"{what}: {bad.sum()} entries differ in finiteness from the reference"
    fin = mask & np.isfinite(f64[first:])
    err = np.abs(got[first:][fin] - f64[first:][fin])
    assert (err <= 2e-3 + 1e-2 * np.abs(f64[first:][fin])).all(), f"{what}: finite entries"


WINDOWS = [
    # nh, nkv, dph, bs, ctx, M
    (32, 8, 128, 16, 1500, 5),     # Llama-3-8B verify (8-row groups: queries 0-1 together)
    (28, 4, 128, 32, 8192, 9),     # Qwen2.5-7B verify (16-row groups straddle queries)
    (8, 2, 64, 16, 700, 5),        # head_dim 64
    (32, 8, 128, 16, 30, 5),       # window across a tile boundary, one partition
]


@pytest.mark.parametrize("poison_k", [False, True])
@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M", WINDOWS)
def test_nonfinite_window_rows_stay_hidden(gpu, oracle, nh, nkv, dph, bs, ctx, M, poison_k):
    case_banner("non-finite window", nh, nkv, dph, bs, ctx, M, poison_k)
    kv_dim = nkv * dph
    cache, table, pool_blocks, kc, vc, rng = _cache_with_context(nh, nkv, dph, bs, ctx, M,
                                                                 ctx + M + int(poison_k))
    k, v = poisoned_window(rng, M, kv_dim, poison_k)
    cache.append(0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), ctx)
    q = W.queries(rng, M, nh, dph)
    out = cache.attention(0, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx)
    torch.cuda.synchronize()
    K = np.concatenate([kc.astype(np.float32), k.astype(np.float16).astype(np.float32)])
    V = np.concatenate([vc.astype(np.float32), v.astype(np.float16).astype(np.float32)])
    model = oracle.PagedKVModel(1, kv_dim, len(table), bs, pool_blocks)
    model.set_block_table(0, table)
    model.write_fp16(0, kc, vc, 0)
    model.append(0, k, v, ctx)
    with np.errstate(invalid="ignore", over="ignore"):
        f64 = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
        tiled = model.attention(0, q, nh, nkv, dph, ctx, mode="tiled")
    check_poisoned(out.cpu().numpy(), f64, tiled, f"window {nh}/{nkv} M{M} k={poison_k}")
    cache.free()


def test_nonfinite_window_rows_stay_hidden_fused(gpu, oracle):
    """The same through the fused RoPE + append + attention step, whose
    workgroups write the window themselves: v of rows 2-4 non-finite."""
    case_banner("non-finite window fused")
    nh, nkv, dph, bs, ctx, M = 32, 8, 128, 16, 2500, 5
    kv_dim = nkv * dph
    cache, table, pool_blocks, kc, vc, rng = _cache_with_context(nh, nkv, dph, bs, ctx, M, 99)
    k, v = poisoned_window(rng, M, kv_dim, False)
    q = rng.standard_normal((M, nh * dph), dtype=np.float32)
    out = cache.rope_append_attention(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                      torch.from_numpy(v).cuda(), nh, nkv, dph, ctx,
                                      theta=500000.0)
    torch.cuda.synchronize()
    gk, gv = cache.read(0, ctx, M)
    gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
    qr = oracle.rope_rotate_half_f64(q, nh, dph, np.arange(ctx, ctx + M),
                                     theta=500000.0).astype(np.float32)
    model = oracle.PagedKVModel(1, kv_dim, len(table), bs, pool_blocks)
    model.set_block_table(0, table)
    model.write_fp16(0, kc, vc, 0)
    model.write_fp16(0, gk.astype(np.float16), gv.astype(np.float16), ctx)
    with np.errstate(invalid="ignore", over="ignore"):
        f64 = oracle.attention_f64_np(qr, np.concatenate([kc.astype(np.float32), gk]),
                                      np.concatenate([vc.astype(np.float32), gv]), nh, nkv, dph,
                                      ctx)
        tiled = model.attention(0, qr, nh, nkv, dph, ctx, mode="tiled")
    check_poisoned(out.cpu().numpy(), f64, tiled, "fused window")
    cache.free()
