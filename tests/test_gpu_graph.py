"""HIP-graph capture of the library's launches (the way a serving loop runs
them): after capture, replays interleaved with eager calls on the same cache
and host synchronizations must reproduce the eager result bit for bit --
the arrival counters return to zero after every call and a caller
workspace carries no state from one call to the next."""
import numpy as np
import pytest
import torch

from conftest import case_banner
from speculative_decode_engine_amd import matvec, matvec_workspace
from test_gpu_attention import build_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nh,nkv,dph,ctx,M", [
    (32, 8, 128, 3000, 1),    # decode: 4-row groups, split context
    (32, 8, 128, 3000, 5),    # verify window: 8-row groups
    (28, 4, 128, 8192, 9),    # 63 rows: 16-row groups
    (32, 4, 64, 2047, 1),     # head_dim 64
])
def test_attention_graph_replays_match_eager(gpu, nh, nkv, dph, ctx, M):
    case_banner("graph attention", nh, nkv, dph, ctx, M)
    cache, _, _, rng = build_layer(nh, nkv, dph, 16, ctx, M, -(-(ctx + M) // 16) + 8, ctx + M)
    q = torch.from_numpy(rng.standard_normal((M, nh * dph), dtype=np.float32)).cuda()
    q_other = torch.from_numpy(rng.standard_normal((1, nh * dph), dtype=np.float32)).cuda()
    ws_bytes = cache.workspace_size(nh, nkv, dph, M, ctx + M)
    ws = torch.zeros(max(1, -(-ws_bytes // 4)), dtype=torch.float32, device="cuda")
    ref = cache.attention(0, q, nh, nkv, dph, ctx, workspace=ws)
    torch.cuda.synchronize()
    out = torch.empty_like(ref)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        cache.attention(0, q, nh, nkv, dph, ctx, out=out, workspace=ws, stream=side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        cache.attention(0, q, nh, nkv, dph, ctx, out=out, workspace=ws, stream=side)
    for rep in range(4):
        out.zero_()
        # eager work on the same cache and workspace between replays
        cache.attention(0, q_other, nh, nkv, dph, ctx // 2, workspace=ws)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
    cache.free()


@pytest.mark.parametrize("M,d_in,d_out", [(1, 4096, 4096), (5, 4096, 4096)])
def test_matvec_graph_replays_match_eager(gpu, M, d_in, d_out):
    case_banner("graph matvec", M, d_in, d_out)
    gen = torch.Generator(device="cuda").manual_seed(M + d_in)
    x = torch.randn(M, d_in, device="cuda", generator=gen)
    W = (torch.randn(d_in, d_out, device="cuda", generator=gen) * 0.05).half()
    ws = matvec_workspace(d_in, d_out, M, "cuda")
    ref = matvec(x, W, workspace=ws)
    torch.cuda.synchronize()
    out = torch.empty_like(ref)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        matvec(x, W, out=out, workspace=ws, stream=side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        matvec(x, W, out=out, workspace=ws, stream=side)
    for rep in range(4):
        out.zero_()
        matvec(x[:1] * 2, W, workspace=ws)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"


@pytest.mark.parametrize("nh,nkv,dph,ctx,M", [(32, 8, 128, 3000, 5), (32, 4, 64, 2047, 1)])
def test_fused_rope_graph_replays_match_eager(gpu, nh, nkv, dph, ctx, M):
    """The fused step appends the window itself: every replay rewrites the
    same rotated K and V and must give the eager output again."""
    case_banner("graph fused", nh, nkv, dph, ctx, M)
    cache, _, _, rng = build_layer(nh, nkv, dph, 16, ctx, M, -(-(ctx + M) // 16) + 8, ctx + 3 * M)
    kv_dim = nkv * dph
    q = torch.from_numpy(rng.standard_normal((M, nh * dph), dtype=np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((M, kv_dim), dtype=np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal((M, kv_dim), dtype=np.float32)).cuda()
    q_other = torch.from_numpy(rng.standard_normal((1, nh * dph), dtype=np.float32)).cuda()
    ws_bytes = cache.workspace_size(nh, nkv, dph, M, ctx + M)
    ws = torch.zeros(max(1, -(-ws_bytes // 4)), dtype=torch.float32, device="cuda")
    ref = cache.rope_append_attention(0, q, k, v, nh, nkv, dph, ctx, theta=500000.0, workspace=ws)
    torch.cuda.synchronize()
    out = torch.empty_like(ref)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        cache.rope_append_attention(0, q, k, v, nh, nkv, dph, ctx, theta=500000.0, out=out,
                                    workspace=ws, stream=side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        cache.rope_append_attention(0, q, k, v, nh, nkv, dph, ctx, theta=500000.0, out=out,
                                    workspace=ws, stream=side)
    for rep in range(4):
        out.zero_()
        cache.attention(0, q_other, nh, nkv, dph, ctx + M - 1, workspace=ws)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
    cache.free()
