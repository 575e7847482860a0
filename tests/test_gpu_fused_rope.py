"""GPU parity of sde_rope_append_attention: RoPE + append + attention fused
in one launch (model.cu:346-384 with cublas_rope_kernel kernels.cu:797-817,
cublas_kv_append_kernel kernels.cu:826-844 and cublas_attention_kernel
kernels.cu:904-940).

Oracle: oracle.rope_rotate_half_f64 (rope_apply_inplace, model.cu:281-323,
with the library's stated frequency rule) rotates q and k in float64.
  * V rows of the window: bit-exact fp16 (RNE) of v.
  * K rows: within one fp16 ulp of the float64-rotated k rounded to fp16
    (the kernel rotates in fp32 with rope_sincos -- a reduction by 2 pi,
    then the hardware's sin / cos, pinned against float64 below; the
    reference's fast-math fp32 RoPE is not reproducible bit for bit), and at
    least 99 % exact.
  * Every other pool byte unchanged.
  * Output within 2e-3 abs + 1e-2 rel of fp64 attention of the rotated q
    over the context and the window rows the kernel stored.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import KVCache
from speculative_decode_engine_amd import _native as N
from speculative_decode_engine_amd import workloads as W
from test_gpu_attention import assert_close

pytestmark = pytest.mark.gpu


def build(nh, nkv, dph, bs, ctx, M, seed):
    rng = np.random.default_rng(seed)
    kv_dim = nkv * dph
    nblk = -(-(ctx + M) // bs)
    pool_blocks = nblk + 40
    table = W.make_tables(rng, 1, nblk, pool_blocks)[0]
    cache = KVCache(1, kv_dim, nblk, bs, pool_blocks)
    cache.set_block_table(0, table)
    if ctx:
        kc, vc = W.context_kv(rng, ctx, kv_dim)
        cache.write_fp16(0, torch.from_numpy(kc.view(np.int16)).cuda(),
                         torch.from_numpy(vc.view(np.int16)).cuda(), 0)
        K, V = kc.astype(np.float32), vc.astype(np.float32)
    else:
        K = V = np.zeros((0, kv_dim), np.float32)
    return cache, table, pool_blocks, K, V, rng


CASES = [
    # nh, nkv, dph, bs, ctx, M, scaling type, factor, theta
    (32, 8, 128, 16, 4096, 5, 0, 1.0, 500000.0),   # Llama-3-8B verify window
    (32, 8, 128, 16, 32767, 1, 0, 1.0, 500000.0),  # 32K decode
    (28, 4, 128, 32, 8192, 9, 0, 1.0, 1000000.0),  # Qwen2.5-7B verify (G = 7, bs 32)
    (32, 4, 64, 16, 2048, 1, 0, 1.0, 10000.0),     # TinyLlama decode
    (4, 2, 64, 16, 128, 1, 0, 1.0, 10000.0),       # config 1 shape
    (32, 8, 128, 16, 1000, 5, 1, 2.0, 10000.0),    # linear scaling
    (32, 8, 128, 16, 1000, 5, 2, 4.0, 10000.0),    # NTK scaling
    (28, 4, 128, 32, 777, 3, 3, 2.0, 0.0),         # YaRN scaling, default theta
    (8, 8, 128, 8, 30, 4, 0, 1.0, 10000.0),        # window across a tile boundary
    (8, 2, 64, 16, 0, 32, 0, 1.0, 10000.0),        # empty context, 32-row window
    (32, 8, 128, 16, 17000, 5, 0, 1.0, 500000.0),  # window past 16K keys: 16-row groups
    (32, 8, 128, 16, 16384, 5, 0, 1.0, 500000.0),  # 513 tiles: the extra one in partition 0
    # one q head per KV head: a 16-row group spans 16 window queries, the
    # largest per-wave (cos, sin) table (16 queries x dph/2 pairs)
    (8, 8, 128, 16, 17000, 20, 0, 1.0, 500000.0),
    (4, 4, 64, 16, 17000, 24, 1, 2.0, 10000.0),
]


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M,stype,factor,theta", CASES)
def test_fused_rope_append_attention(gpu, oracle, nh, nkv, dph, bs, ctx, M, stype, factor,
                                     theta):
    case_banner("fused rope", nh, nkv, dph, bs, ctx, M, stype, factor, theta)
    kv_dim = nkv * dph
    cache, table, pool_blocks, K, V, rng = build(nh, nkv, dph, bs, ctx, M, ctx + M + nh)
    before = cache.pool.cpu().numpy().view(np.uint16).copy()
    q = rng.standard_normal((M, nh * dph), dtype=np.float32)
    k = rng.standard_normal((M, kv_dim), dtype=np.float32)
    v = rng.standard_normal((M, kv_dim), dtype=np.float32)
    out = cache.rope_append_attention(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                      torch.from_numpy(v).cuda(), nh, nkv, dph, ctx, theta=theta,
                                      scaling_type=stype, scaling_factor=factor)
    torch.cuda.synchronize()
    pos = np.arange(ctx, ctx + M)
    kw = dict(theta=theta, scaling_type=stype, factor=factor)
    gk, gv = cache.read(0, ctx, M)
    gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
    # V: bit-exact append
    assert np.array_equal(gv, v.astype(np.float16).astype(np.float32))
    # K: rotated, within one fp16 ulp of the float64 rotation
    kref = oracle.rope_rotate_half_f64(k, nkv, dph, pos, **kw).astype(np.float16)
    ulp = np.spacing(np.abs(kref)).astype(np.float32)
    diff = np.abs(gk - kref.astype(np.float32))
    assert (diff <= ulp).all(), f"max diff {diff.max()} at {np.argmax(diff)}"
    assert (diff == 0).mean() >= 0.99
    # every other pool byte unchanged
    m = oracle.PagedKVModel(1, kv_dim, len(table), bs, pool_blocks)
    m.pool = before.reshape(m.pool.shape)
    m.set_block_table(0, table)
    m.write_fp16(0, gk.astype(np.float16), gv.astype(np.float16), ctx)
    after = cache.pool.cpu().numpy().view(np.uint16).reshape(m.pool.shape)
    assert np.array_equal(after, m.pool)
    # attention of the rotated q over context + stored window
    qr = oracle.rope_rotate_half_f64(q, nh, dph, pos, **kw)
    ref = oracle.attention_f64_np(qr, np.concatenate([K, gk]), np.concatenate([V, gv]),
                                  nh, nkv, dph, ctx)
    assert_close(out.cpu().numpy(), ref, "fused rope+append+attention")
    cache.free()


def test_fused_equals_unfused_steps(gpu, oracle):
    """The fused call against the unfused calls on the same inputs: append
    of the stored rotated rows + attention of the fp64-rotated q."""
    case_banner("fused vs unfused")
    nh, nkv, dph, bs, ctx, M = 32, 8, 128, 16, 3000, 5
    cache, table, pool_blocks, K, V, rng = build(nh, nkv, dph, bs, ctx, M, 11)
    q = rng.standard_normal((M, nh * dph), dtype=np.float32)
    k = rng.standard_normal((M, nkv * dph), dtype=np.float32)
    v = rng.standard_normal((M, nkv * dph), dtype=np.float32)
    fused = cache.rope_append_attention(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                        torch.from_numpy(v).cuda(), nh, nkv, dph, ctx,
                                        theta=500000.0)
    qr = oracle.rope_rotate_half_f64(q, nh, dph, np.arange(ctx, ctx + M), theta=500000.0)
    unfused = cache.attention(0, torch.from_numpy(qr.astype(np.float32)).cuda(), nh, nkv, dph, ctx)
    torch.cuda.synchronize()
    assert_close(fused.cpu().numpy(), unfused.cpu().numpy().astype(np.float64), "fused vs unfused")
    cache.free()


def test_fused_argument_errors_do_no_device_work(gpu):
    case_banner("fused rope errors")
    lib = N.load()
    nh, nkv, dph, ctx = 8, 2, 64, 100
    cache, table, pool_blocks, K, V, rng = build(nh, nkv, dph, 16, ctx, 40, 3)
    before = cache.pool.clone()
    q = torch.zeros(40, nh * dph, device="cuda")
    kv = torch.zeros(40, nkv * dph, device="cuda")
    out = torch.full((40, nh * dph), float("nan"), device="cuda")
    vp = ctypes.c_void_p
    good = N.RopeConfig(10000.0, 0, 1.0)

    def call(M, k_ptr, rope):
        return lib.sde_rope_append_attention(cache.handle, 0, vp(q.data_ptr()), k_ptr,
                                             vp(kv.data_ptr()), vp(out.data_ptr()), nh, nkv,
                                             dph, ctx, M, rope, None, 0, None)
    assert call(33, vp(kv.data_ptr()), ctypes.byref(good)) == N.SDE_ERR_UNSUPPORTED
    assert call(4, None, ctypes.byref(good)) == N.SDE_ERR_INVALID_ARGUMENT
    assert call(4, vp(kv.data_ptr()), None) == N.SDE_ERR_INVALID_ARGUMENT
    bad = N.RopeConfig(10000.0, 7, 1.0)
    assert call(4, vp(kv.data_ptr()), ctypes.byref(bad)) == N.SDE_ERR_INVALID_ARGUMENT
    assert call(4, vp(kv.data_ptr() + 2), ctypes.byref(good)) == N.SDE_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and torch.equal(cache.pool, before)
    cache.free()


def test_rope_sincos_against_float64(gpu):
    """sde::attn::rope_sincos, the fused step's sin / cos (Cody-Waite
    reduction by 2 pi, then the hardware's sin / cos of the revolutions;
    sincosf from 2^17 on), against float64 sin / cos of the same fp32
    angles: every angle the step forms for positions up to 2^17 + 2^12 at
    the benchmark models' frequencies (dph 64 and 128, theta 1e4, 5e5, 1e6),
    random angles of either sign, points around multiples of pi/2 (where
    the reduction's cancellation is largest) and large angles."""
    lib = ctypes.CDLL(str(Path(__file__).resolve().parent / "device" / "libsde_device_test.so"))
    lib.sdet_rope_sincos.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p]
    lib.sdet_rope_sincos.restype = ctypes.c_int
    rng = np.random.default_rng(7)
    pos = np.arange(0, 2 ** 17 + 2 ** 12, 7, dtype=np.float32)
    parts = []
    for theta in (1e4, 5e5, 1e6):
        for dph in (64, 128):
            inv = (theta ** (-np.arange(0, dph, 2, dtype=np.float64) / dph)).astype(np.float32)
            parts.append((pos[:, None] * inv[None, :]).ravel())
    k = np.arange(-40000, 40000, dtype=np.float64)
    near = (k * (np.pi / 2)).astype(np.float32)
    parts += [rng.uniform(-2.0 ** 17, 2.0 ** 17, 1 << 20).astype(np.float32), near,
              np.nextafter(near, np.float32(np.inf)), np.nextafter(near, np.float32(-np.inf)),
              rng.uniform(2.0 ** 17, 1e7, 1 << 16).astype(np.float32)]
    x = np.concatenate(parts).astype(np.float32)
    case_banner("rope_sincos", x.size)
    xt = torch.from_numpy(x).cuda()
    sn = torch.empty_like(xt)
    cs = torch.empty_like(xt)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.sdet_rope_sincos(xt.data_ptr(), sn.data_ptr(), cs.data_ptr(), x.size, stream) == 0
    torch.cuda.synchronize()
    x64 = x.astype(np.float64)
    es = np.abs(sn.cpu().numpy().astype(np.float64) - np.sin(x64))
    ec = np.abs(cs.cpu().numpy().astype(np.float64) - np.cos(x64))
    small = np.abs(x) < 2.0 ** 17
    print(f"rope_sincos max abs error: below 2^17 sin {es[small].max():.3g} cos "
          f"{ec[small].max():.3g}; above sin {es[~small].max():.3g} cos {ec[~small].max():.3g}")
    assert es[small].max() <= 1e-6 and ec[small].max() <= 1e-6
    assert es[~small].max() <= 2e-7 and ec[~small].max() <= 2e-7
