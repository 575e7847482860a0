"""sde_paged_attention_noalloc through the C-ABI: the allocation-free
variant of sde_paged_attention (partials in the library's static per-device
array) gives the same bytes as the workspace entry point on the same inputs,
on two calls in a row -- the Qwen2.5-7B 9-query verify window, whose
partials are the largest of the configurations (~2.1 MB on 256 CUs), then a
smaller Llama-3-8B decode step -- and agrees with the fp64 oracle.  The
array keeps the last call's contents; a call writes every partial it
reads, so the second call's result must not depend on the first's."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import _native as N
from test_gpu_attention import assert_close, build_layer
from speculative_decode_engine_amd import workloads as W

pytestmark = pytest.mark.gpu


def _noalloc(lib, cache, q, out, nh, nkv, dph, pos_base):
    return lib.sde_paged_attention_noalloc(
        cache.handle, 0, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(out.data_ptr()), nh, nkv,
        dph, pos_base, q.shape[0], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("shapes", [
    [(28, 4, 128, 32, 8192, 9), (32, 8, 128, 16, 4096, 1)],
])
def test_noalloc_equals_workspace_entry_point(gpu, oracle, shapes):
    lib = N.load()
    for i, (nh, nkv, dph, bs, ctx, M) in enumerate(shapes):
        case_banner("noalloc call", i, nh, nkv, dph, bs, ctx, M)
        nblk = -(-(ctx + M) // bs)
        cache, K, V, rng = build_layer(nh, nkv, dph, bs, ctx, M, nblk + 17, 90 + i)
        q = torch.from_numpy(W.queries(rng, M, nh, dph)).cuda()
        out = torch.full((M, nh * dph), float("nan"), device="cuda")
        assert _noalloc(lib, cache, q, out, nh, nkv, dph, ctx) == N.SDE_OK
        need = cache.workspace_size(nh, nkv, dph, M, ctx + M)
        assert need > 0
        ws = torch.empty(need // 4 + 1, dtype=torch.float32, device="cuda")
        ref = cache.attention(0, q, nh, nkv, dph, ctx, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: differs from sde_paged_attention"
        f64 = oracle.attention_f64_np(q.cpu().numpy(), K, V, nh, nkv, dph, ctx)
        assert_close(out.cpu().numpy(), f64, f"noalloc call {i}")
        cache.free()


def test_noalloc_rejects_arguments_like_the_workspace_entry_point(gpu):
    case_banner("noalloc errors")
    lib = N.load()
    cache, K, V, rng = build_layer(8, 2, 64, 16, 40, 1, 8, 3)
    q = torch.zeros(1, 8 * 64, device="cuda")
    out = torch.full((1, 8 * 64), float("nan"), device="cuda")
    assert _noalloc(lib, cache, q, out, 8, 2, 64, 4096) == N.SDE_ERR_CAPACITY
    assert _noalloc(lib, cache, q, out, 8, 3, 64, 0) == N.SDE_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    cache.free()
