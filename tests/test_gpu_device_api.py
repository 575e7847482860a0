"""GPU parity of the device-side API (include/sde/attention_device.hpp):
kv_cache_append / kv_cache_read / kv_cache_rollback and
device_flash_attention_gqa / device_attention_dispatch called from inside a
caller's kernel (tests/device/device_api_test.hip), the way the reference's
persistent decode loop calls them (kv_cache.h:70-79, attention.h:21-164).

Append and read are checked bit-exact against the C-ABI path and the oracle
byte model; attention against the oracle's fp64 attention with the same
tolerance as the host entry point (2e-3 abs + 1e-2 rel).
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
from test_gpu_attention import assert_close, build_layer

pytestmark = pytest.mark.gpu
LIB = Path(__file__).resolve().parent / "device" / "libsde_device_test.so"


@pytest.fixture(scope="module")
def dev(gpu):
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB))
    vp, i = ctypes.c_void_p, ctypes.c_int
    view_p = ctypes.POINTER(N.KVView)
    lib.sdet_attention.argtypes = [view_p, i, vp, vp, i, i, i, i, i, i, i, vp, vp]
    lib.sdet_append.argtypes = [view_p, i, vp, vp, i, i, i, vp]
    lib.sdet_read.argtypes = [view_p, i, i, i, vp, vp, i, vp]
    lib.sdet_rollback.argtypes = [view_p, i, vp]
    for f in (lib.sdet_attention, lib.sdet_append, lib.sdet_read, lib.sdet_rollback):
        f.restype = i
    return lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def device_attention(dev, cache, q, nh, nkv, dph, pos_base, threads=256, attn_type=0):
    M = q.shape[0]
    out = torch.full((M, nh * dph), float("nan"), device="cuda")
    status = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    view = cache.view()
    rc = dev.sdet_attention(ctypes.byref(view), 0, q.data_ptr(), out.data_ptr(), nh, nkv, dph,
                            pos_base, M, threads, attn_type, status.data_ptr(), _stream())
    assert rc == 0
    torch.cuda.synchronize()
    return out, status.cpu().numpy()


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M", [
    (4, 2, 64, 16, 128, 1),       # config 1 shape
    (32, 4, 64, 16, 2048, 1),     # TinyLlama: G = 8 -> two row groups per KV head
    (32, 8, 128, 16, 4096, 5),    # Llama-3-8B verify window
    (28, 4, 128, 32, 1000, 9),    # Qwen2.5-7B (G = 7), block size 32
    (8, 8, 128, 8, 77, 2),        # MHA, block size 8, ragged last tile
    # the generic fp32 path: other head sizes and block sizes
    (8, 2, 96, 16, 300, 1),       # head size 96
    (16, 4, 256, 12, 500, 3),     # head size 256 (Gemma), block size 12
    (4, 1, 80, 10, 1000, 2),      # head size 80, block size 10
    (8, 2, 512, 16, 200, 1),      # the largest head size
    (4, 4, 32, 5, 77, 1),         # head size 32, block size 5
    (32, 8, 64, 12, 600, 5),      # head size 64 with block size 12
])
def test_device_attention_matches_oracle(dev, oracle, nh, nkv, dph, bs, ctx, M):
    case_banner("device attention", nh, nkv, dph, bs, ctx, M)
    nblk = -(-(ctx + M) // bs)
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, nblk + 40, nh + ctx)
    q = W.queries(rng, M, nh, dph)
    qd = torch.from_numpy(q).cuda()
    out, status = device_attention(dev, cache, qd, nh, nkv, dph, ctx)
    assert (status == 0).all()
    ref = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
    assert_close(out.cpu().numpy(), ref, "device_flash_attention_gqa")
    host = cache.attention(0, qd, nh, nkv, dph, ctx)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), host.cpu().numpy().astype(np.float64), "device vs host entry")
    cache.free()


@pytest.mark.parametrize("threads", [64, 192, 256, 512])
@pytest.mark.parametrize("dph", [128, 96])
def test_device_attention_any_block_size(dev, oracle, threads, dph):
    """Any multiple of 64 threads: the tile path spreads over the block's
    waves; the generic path (head size 96) uses 64, 128 or 256 threads."""
    case_banner("device attention threads", threads, dph)
    nh, nkv, ctx = 32, 8, 700
    cache, K, V, rng = build_layer(nh, nkv, dph, 16, ctx, 1, 80, threads)
    q = W.queries(rng, 1, nh, dph)
    out, status = device_attention(dev, cache, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx,
                                   threads=threads)
    assert (status == 0).all()
    assert_close(out.cpu().numpy(), oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx), "threads")
    cache.free()


def _ref_fns(dev):
    vp, i = ctypes.c_void_p, ctypes.c_int
    view_p = ctypes.POINTER(N.KVView)
    dev.sdet_ref_layer_attention.argtypes = [view_p, i, vp, vp, i, i, i, i, i, i, i, vp, vp]
    dev.sdet_ref_megakernel_step.argtypes = [view_p, i, vp, vp, vp, vp, i, i, i, i, i, i, vp,
                                             vp]
    dev.sdet_ref_layer_attention.restype = i
    dev.sdet_ref_megakernel_step.restype = i


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M,threads", [
    (32, 8, 128, 16, 3000, 5, 256),    # Llama-3-8B, the reference's 256-thread blocks
    (28, 4, 128, 32, 1000, 2, 512),    # Qwen2.5-7B (G = 7)
    (32, 4, 64, 16, 2048, 1, 256),     # TinyLlama
])
def test_reference_signature_layer_attention(dev, oracle, nh, nkv, dph, bs, ctx, M, threads):
    """model.cu:400-432's call, verbatim but for the cache type: q_all and
    attn_out in the caller's dynamic shared memory, blk_logits and the five
    __shared__ scalars passed through device_attention_dispatch's
    reference argument list."""
    case_banner("reference-signature layer attention", nh, nkv, dph, bs, ctx, M, threads)
    _ref_fns(dev)
    nblk = -(-(ctx + M) // bs)
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, nblk + 11, 5 * nh + ctx)
    q = W.queries(rng, M, nh, dph)
    qd = torch.from_numpy(q).cuda()
    out = torch.full((M, nh * dph), float("nan"), device="cuda")
    status = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    view = cache.view()
    assert dev.sdet_ref_layer_attention(ctypes.byref(view), 0, qd.data_ptr(), out.data_ptr(), nh,
                                        nkv, dph, ctx, M, threads, 0, status.data_ptr(),
                                        _stream()) == 0
    torch.cuda.synchronize()
    assert (status.cpu().numpy() == 0).all()
    ref = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
    assert_close(out.cpu().numpy(), ref, "reference-signature dispatch")
    cache.free()


def test_reference_signature_megakernel_step(dev, oracle):
    """kernels.cu:2727-2739 on block 0 of a 256-thread grid: append the
    token at seq, zero g_attn, dispatch over seq + 1 positions with the
    reference's arguments (s_scratch, five __shared__ scalars); the pool
    bytes are the oracle's and the output matches its attention."""
    case_banner("reference-signature megakernel step")
    _ref_fns(dev)
    nh, nkv, dph, bs, ctx = 32, 8, 128, 16, 1200
    kv_dim = nkv * dph
    nblk = -(-(ctx + 1) // bs)
    rng = np.random.default_rng(2739)
    tables = W.make_tables(rng, 2, nblk, 2 * nblk + 5)
    cache = KVCache(2, kv_dim, nblk, bs, 2 * nblk + 5)
    model = oracle.PagedKVModel(2, kv_dim, nblk, bs, 2 * nblk + 5)
    kc, vc = W.context_kv(rng, ctx, kv_dim)
    for l in range(2):
        cache.set_block_table(l, tables[l])
        model.set_block_table(l, tables[l])
    cache.write_fp16(1, torch.from_numpy(kc.view(np.int16)).cuda(),
                     torch.from_numpy(vc.view(np.int16)).cuda(), 0)
    model.write_fp16(1, kc, vc, 0)
    k, v = W.new_kv(rng, 1, kv_dim)
    q = W.queries(rng, 1, nh, dph)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    attn = torch.full((nh * dph,), float("nan"), device="cuda")
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    view = cache.view()
    assert dev.sdet_ref_megakernel_step(ctypes.byref(view), 1, kd.data_ptr(), vd.data_ptr(),
                                        qd.data_ptr(), attn.data_ptr(), nh, nkv, dph, ctx, 4, 0,
                                        status.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    assert status.item() == 0
    model.append(1, k, v, ctx)
    pool = cache.pool.cpu().numpy().view(np.uint16).reshape(model.pool.shape)
    assert np.array_equal(pool, model.pool)
    ref = model.attention(1, q, nh, nkv, dph, ctx, mode="f64")
    assert_close(attn.cpu().numpy()[None], ref, "megakernel step")
    cache.free()


def test_device_attention_empty_context_gives_zeros(dev):
    case_banner("device attention total_len 0")
    nh, nkv, dph = 8, 2, 64
    cache = KVCache(1, nkv * dph, 4, 16, 8)
    q = torch.randn(1, nh * dph, device="cuda")
    # pos_base -1: query 0 sees positions [0, 0) -- attention.h:120-126 -> zeros
    out, status = device_attention(dev, cache, q, nh, nkv, dph, -1)
    assert (status == 0).all()
    assert torch.count_nonzero(out).item() == 0
    cache.free()


def test_device_dispatch_rejects_reserved_types(dev):
    case_banner("device dispatch reserved types")
    nh, nkv, dph = 8, 2, 64
    cache = KVCache(1, nkv * dph, 4, 16, 8)
    q = torch.randn(1, nh * dph, device="cuda")
    for t in (N.SDE_ATTN_SLIDING_WINDOW, N.SDE_ATTN_KDA, N.SDE_ATTN_LINEAR):
        out, status = device_attention(dev, cache, q, nh, nkv, dph, 10, attn_type=t)
        assert (status == N.SDE_ERR_UNSUPPORTED).all()
        assert torch.isnan(out).all()  # nothing written
    cache.free()


@pytest.mark.parametrize("kv_dim,bs,n", [(128, 16, 37), (1024, 16, 9), (512, 32, 70), (96, 8, 5)])
def test_device_append_and_read_bit_exact(dev, oracle, kv_dim, bs, n):
    case_banner("device append/read", kv_dim, bs, n)
    rng = np.random.default_rng(kv_dim + n)
    nblk = -(-(n + 3) // bs)
    pool_blocks = 2 * nblk + 3
    tables = W.make_tables(rng, 2, nblk, pool_blocks)
    host = KVCache(2, kv_dim, nblk, bs, pool_blocks)
    devc = KVCache(2, kv_dim, nblk, bs, pool_blocks)
    for l in range(2):
        host.set_block_table(l, tables[l])
        devc.set_block_table(l, tables[l])
    k, v = W.new_kv(rng, n, kv_dim)
    k[0, :4] = [65519.0, 65520.0, 1e-8, -0.0]          # overflow boundary, underflow, -0
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    host.append(1, kd, vd, 3)
    view = devc.view()
    assert dev.sdet_append(ctypes.byref(view), 1, kd.data_ptr(), vd.data_ptr(), 3, n, 128,
                           _stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(devc.pool, host.pool)          # same bytes as the C-ABI append
    m = oracle.PagedKVModel(2, kv_dim, nblk, bs, pool_blocks)
    for l in range(2):
        m.set_block_table(l, tables[l])
    m.append(1, k, v, 3)
    assert np.array_equal(devc.pool.cpu().numpy().view(np.uint16).reshape(m.pool.shape), m.pool)
    ko = torch.empty(n, kv_dim, device="cuda")
    vo = torch.empty(n, kv_dim, device="cuda")
    assert dev.sdet_read(ctypes.byref(view), 1, 3, n, ko.data_ptr(), vo.data_ptr(), 256,
                         _stream()) == 0
    gk, gv = host.read(1, 3, n)
    torch.cuda.synchronize()
    assert torch.equal(ko, gk) and torch.equal(vo, gv)
    host.free()
    devc.free()


def test_device_rollback_writes_seq_len_only(dev):
    case_banner("device rollback")
    cache = KVCache(1, 128, 8, 16, 8)
    cache.set_seq_len(100)
    before = cache.pool.clone()
    view = cache.view()
    assert dev.sdet_rollback(ctypes.byref(view), 61, _stream()) == 0
    torch.cuda.synchronize()
    assert cache.device_seq_len() == 61
    assert torch.equal(cache.pool, before)
    cache.free()


def test_cpp_host_names_match_the_c_abi(dev, oracle):
    """sde/kv_cache.hpp (kv_cache_alloc, cublas_kv_append_kernel,
    cublas_attention_kernel, set_seq_len_kernel, kv_cache_rollback) run end to
    end in C++ give the same pool bytes, outputs and seq_len as the same
    steps through the Python binding of the C-ABI."""
    case_banner("C++ host names")
    nl, nh, nkv, dph, bs, ctx, M = 2, 32, 8, 128, 16, 300, 5
    kv_dim = nkv * dph
    nblk = -(-(ctx + M) // bs)
    pool_blocks = nl * nblk + 7
    rng = np.random.default_rng(77)
    tables = W.make_tables(rng, nl, nblk, pool_blocks).astype(np.int32)
    k, v = W.new_kv(rng, ctx + M, kv_dim)
    q = W.queries(rng, M, nh, dph)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    # C++: append all ctx+M rows at 0, window of M queries at ctx, rewind to ctx+2
    pool_out = torch.empty(pool_blocks * 2 * bs * kv_dim, dtype=torch.int16, device="cuda")
    out_cpp = torch.empty(M, nh * dph, device="cuda")
    seq = ctypes.c_int(-1)
    f = dev.sdet_cpp_pipeline
    f.restype = ctypes.c_int
    rc = f(nl, kv_dim, nblk, bs, pool_blocks, tables.ctypes.data_as(ctypes.c_void_p), 1,
           ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()), 0, ctx + M,
           ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(out_cpp.data_ptr()), nh, nkv, dph,
           ctx, M, ctx + 2, ctypes.c_void_p(pool_out.data_ptr()), ctypes.byref(seq))
    assert rc == 0
    torch.cuda.synchronize()
    # the same through the Python binding
    cache = KVCache(nl, kv_dim, nblk, bs, pool_blocks, pool="library")
    for l in range(nl):
        cache.set_block_table(l, tables[l])
    cache.append(1, kd, vd, 0)
    cache.set_seq_len(ctx + M)
    out_py = cache.attention(1, qd, nh, nkv, dph, ctx)
    cache.rollback(ctx + 2)
    torch.cuda.synchronize()
    assert seq.value == ctx + 2 == cache.device_seq_len()
    assert torch.equal(out_cpp, out_py)
    gk, gv = cache.read(1, 0, ctx + M)
    torch.cuda.synchronize()
    assert np.array_equal(gk.cpu().numpy(), k.astype(np.float16).astype(np.float32))
    pool_cpp = pool_out.cpu().numpy().view(np.uint16).reshape(pool_blocks, 2, bs, kv_dim)
    m = oracle.PagedKVModel(nl, kv_dim, nblk, bs, pool_blocks)
    for l in range(nl):
        m.set_block_table(l, tables[l])
    m.append(1, k, v, 0)
    assert np.array_equal(pool_cpp, m.pool)           # C++ append: oracle bytes
    cache.free()


# ---- grid-cooperative attention (device_flash_attention_gqa_grid) ----------

def _grid_ws(nh, nkv, dph, M, L):
    n = N.load().sde_grid_attention_workspace_size(nh, nkv, dph, M, L)
    assert n > 0
    return torch.zeros(n // 4 + 1, dtype=torch.int32, device="cuda")


def grid_attention(dev, cache, q, nh, nkv, dph, pos_base, blocks, threads, ws, layer=0,
                   max_waves=4):
    M = q.shape[0]
    out = torch.full((M, nh * dph), float("nan"), device="cuda")
    status = torch.full((blocks,), -1, dtype=torch.int32, device="cuda")
    view = cache.view()
    f = dev.sdet_grid_attention
    f.restype = ctypes.c_int
    vp, i = ctypes.c_void_p, ctypes.c_int
    f.argtypes = [ctypes.POINTER(N.KVView), i, vp, vp, i, i, i, i, i, i, i, i, vp,
                  ctypes.c_size_t, vp, vp]
    assert f(ctypes.byref(view), layer, q.data_ptr(), out.data_ptr(), nh, nkv, dph, pos_base, M,
             blocks, threads, max_waves, ws.data_ptr(), ws.numel() * 4, status.data_ptr(),
             _stream()) == 0
    torch.cuda.synchronize()
    return out, status.cpu().numpy()


@pytest.mark.parametrize("nh,nkv,dph,bs,ctx,M,blocks,threads,max_waves", [
    (32, 8, 128, 16, 32767, 1, 256, 512, 8),   # Llama-3-8B 32K decode, one block per CU
    (32, 8, 128, 16, 32767, 1, 256, 512, 4),   # the same with 4-wave staging
    (32, 8, 128, 16, 4096, 5, 300, 256, 4),    # verify window, 4-wave blocks
    (28, 4, 128, 32, 8192, 9, 64, 512, 8),     # Qwen2.5-7B verify, fewer blocks than items
    (32, 4, 64, 16, 2048, 1, 37, 320, 4),      # TinyLlama, odd grid, a wave past the four
    (4, 2, 64, 16, 128, 1, 1, 256, 4),         # config 1 shape on a single block
    (8, 8, 128, 8, 77, 2, 512, 512, 8),        # ragged last tile, more blocks than work
    (32, 8, 128, 16, 4096, 5, 256, 512, 8),    # 4K verify window, 8-wave: 8-row groups, 2 tiles
    (4, 2, 64, 16, 40, 1, 256, 512, 8),        # G = 2 decode, 8-wave: 2-row groups, 1 tile
    (32, 8, 128, 16, 17000, 5, 256, 512, 8),   # window past 16K, 8-wave: 16-row groups
    # the generic fp32 path (other head sizes, block sizes not a multiple of 8)
    (8, 2, 96, 16, 3000, 3, 256, 512, 4),      # head size 96, 8-row groups, partitions
    (16, 4, 256, 12, 2000, 5, 64, 512, 8),     # head size 256, block size 12, few blocks
    (4, 1, 80, 10, 700, 1, 300, 256, 4),       # head size 80, more blocks than items
    (32, 8, 256, 16, 4096, 5, 256, 512, 8),    # Gemma-like verify window
    (28, 4, 64, 12, 1500, 9, 256, 512, 4),     # head size 64 with block size 12
    (8, 2, 512, 16, 900, 2, 40, 256, 4),       # the largest head size
])
def test_grid_attention_matches_oracle_and_host_entry(dev, oracle, nh, nkv, dph, bs, ctx, M,
                                                      blocks, threads, max_waves):
    case_banner("grid attention", nh, nkv, dph, bs, ctx, M, blocks, threads, max_waves)
    nblk = -(-(ctx + M) // bs)
    cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, nblk + 40, nh + ctx + M)
    q = W.queries(rng, M, nh, dph)
    qd = torch.from_numpy(q).cuda()
    ws = _grid_ws(nh, nkv, dph, M, ctx + M)
    ref = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
    host = cache.attention(0, qd, nh, nkv, dph, ctx)
    torch.cuda.synchronize()
    first = None
    for call in range(2):   # the second call finds the counters the first left at zero
        out, status = grid_attention(dev, cache, qd, nh, nkv, dph, ctx, blocks, threads, ws,
                                     max_waves=max_waves)
        assert (status == 0).all()
        assert_close(out.cpu().numpy(), ref, f"grid call {call}")
        assert_close(out.cpu().numpy(), host.cpu().numpy().astype(np.float64), "grid vs host")
        if first is None:
            first = out
        else:
            assert torch.equal(out, first)   # deterministic
    assert torch.count_nonzero(ws[:4096]).item() == 0   # counters back at zero
    cache.free()


def test_grid_attention_nonfinite_window_rows_stay_hidden(dev, oracle):
    """Rows 2-4 of a 5-query window hold Inf/NaN V: on the grid-cooperative
    path too, queries 0-1 match the oracle and later queries are non-finite
    exactly where the reference's restatement is."""
    from test_gpu_precision import _cache_with_context, check_poisoned, poisoned_window
    case_banner("grid attention non-finite window")
    nh, nkv, dph, bs, ctx, M = 32, 8, 128, 16, 4096, 5
    kv_dim = nkv * dph
    cache, table, pool_blocks, kc, vc, rng = _cache_with_context(nh, nkv, dph, bs, ctx, M, 404)
    k, v = poisoned_window(rng, M, kv_dim, False)
    cache.append(0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), ctx)
    K = np.concatenate([kc.astype(np.float32), k.astype(np.float16).astype(np.float32)])
    V = np.concatenate([vc.astype(np.float32), v.astype(np.float16).astype(np.float32)])
    q = W.queries(rng, M, nh, dph)
    ws = _grid_ws(nh, nkv, dph, M, ctx + M)
    out, status = grid_attention(dev, cache, torch.from_numpy(q).cuda(), nh, nkv, dph, ctx, 256,
                                 512, ws, max_waves=8)
    assert (status == 0).all()
    model = oracle.PagedKVModel(1, kv_dim, len(table), bs, pool_blocks)
    model.set_block_table(0, table)
    model.write_fp16(0, kc, vc, 0)
    model.append(0, k, v, ctx)
    with np.errstate(invalid="ignore", over="ignore"):
        f64 = oracle.attention_f64_np(q, K, V, nh, nkv, dph, ctx)
        tiled = model.attention(0, q, nh, nkv, dph, ctx, mode="tiled")
    check_poisoned(out.cpu().numpy(), f64, tiled, "grid window")
    cache.free()


def test_grid_attention_errors_write_nothing(dev):
    case_banner("grid attention errors")
    nh, nkv, dph, ctx = 32, 8, 128, 1000
    cache, K, V, rng = build_layer(nh, nkv, dph, 16, ctx, 1, 80, 5)
    q = torch.from_numpy(W.queries(rng, 1, nh, dph)).cuda()
    ws = _grid_ws(nh, nkv, dph, 1, ctx + 1)
    small = ws[: ws.numel() // 2]
    out, status = grid_attention(dev, cache, q, nh, nkv, dph, ctx, 16, 512, small)
    assert (status == N.SDE_ERR_WORKSPACE).all() and torch.isnan(out).all()
    out, status = grid_attention(dev, cache, q, nh, nkv, dph, ctx, 16, 192, ws)
    assert (status == N.SDE_ERR_UNSUPPORTED).all() and torch.isnan(out).all()
    out, status = grid_attention(dev, cache, q, nh, nkv, dph, ctx + 5000, 16, 512, ws)
    assert (status == N.SDE_ERR_CAPACITY).all() and torch.isnan(out).all()
    big = torch.zeros(1, 600, device="cuda")   # head size above 512
    out, status = grid_attention(dev, cache, big, 1, 1, 600, ctx, 16, 512, ws)
    assert (status == N.SDE_ERR_UNSUPPORTED).all() and torch.isnan(out).all()
    cache.free()


def test_persistent_loop_append_verify_rewind(dev, oracle):
    """One cooperative persistent kernel runs three verify steps of k+1 = 5
    tokens over 2 layers -- append (block 0), grid barrier, grid attention,
    grid barrier -- rewinding seq_len between steps to a partial accept; the
    pool bytes equal the oracle's after the same appends, every window's
    output matches the oracle's attention, and seq_len ends at pos + M."""
    case_banner("persistent loop")
    nl, nh, nkv, dph, bs, M = 2, 32, 8, 128, 16, 5
    kv_dim = nkv * dph
    ctx = 3000
    pos = [ctx, ctx + 3, ctx + 3 + 1]   # 2 then 0 drafts accepted
    nblk = -(-(pos[-1] + M) // bs)
    pool_blocks = nl * nblk + 9
    rng = np.random.default_rng(123)
    tables = W.make_tables(rng, nl, nblk, pool_blocks)
    cache = KVCache(nl, kv_dim, nblk, bs, pool_blocks)
    model = oracle.PagedKVModel(nl, kv_dim, nblk, bs, pool_blocks)
    kc, vc = W.context_kv(rng, ctx, kv_dim)
    for l in range(nl):
        cache.set_block_table(l, tables[l])
        model.set_block_table(l, tables[l])
        cache.write_fp16(l, torch.from_numpy(kc.view(np.int16)).cuda(),
                         torch.from_numpy(vc.view(np.int16)).cuda(), 0)
        model.write_fp16(l, kc, vc, 0)
    S = len(pos)
    k = rng.standard_normal((S, nl, M, kv_dim), dtype=np.float32)
    v = rng.standard_normal((S, nl, M, kv_dim), dtype=np.float32)
    q = rng.standard_normal((S, nl, M, nh * dph), dtype=np.float32)
    out = torch.full((S, nl, M, nh * dph), float("nan"), device="cuda")
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    posd = torch.tensor(pos, dtype=torch.int32, device="cuda")
    ws = _grid_ws(nh, nkv, dph, M, pos[-1] + M)
    blocks = 256
    status = torch.full((blocks,), -1, dtype=torch.int32, device="cuda")
    f = dev.sdet_persistent_loop
    f.restype = ctypes.c_int
    view = cache.view()
    vp = ctypes.c_void_p
    rc = f(ctypes.byref(view), vp(posd.data_ptr()), S, M, nh, nkv, dph, vp(kd.data_ptr()),
           vp(vd.data_ptr()), vp(qd.data_ptr()), vp(out.data_ptr()), vp(ws.data_ptr()),
           ctypes.c_size_t(ws.numel() * 4), vp(status.data_ptr()), blocks, 512, _stream())
    if rc == 2:
        pytest.skip("device cannot hold the cooperative grid")
    assert rc == 0
    torch.cuda.synchronize()
    assert (status.cpu().numpy() == 0).all()
    assert cache.device_seq_len() == pos[-1] + M
    outs = out.cpu().numpy()
    for s in range(S):
        for l in range(nl):
            model.append(l, k[s, l], v[s, l], pos[s])
            ref = model.attention(l, q[s, l], nh, nkv, dph, pos[s], mode="f64")
            assert_close(outs[s, l], ref, f"step {s} layer {l}")
    pool = cache.pool.cpu().numpy().view(np.uint16).reshape(model.pool.shape)
    assert np.array_equal(pool, model.pool)
    cache.free()
