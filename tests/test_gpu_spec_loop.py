"""The persistent speculative loop (sde_spec_loop_greedy) against its CPU
restatement (oracle.spec_loop_greedy), through the C-ABI.

One cooperative launch runs every round on the device (megakernel_speculative,
kernels.cu:2864-3106): drafting with the prefix layers, the window's verify
(model.cu:838-890), greedy acceptance on device tokens and the O(1) rewind;
each round starts at the device seq_len the previous one wrote.  Checked:
  * emitted tokens, per-round acceptances, the final device seq_len and the
    SHA-256 of the whole pool (stale rejected drafts included) equal the
    oracle's, for greedy decoding (k = 0) and self-speculation;
  * speculation emits the greedy tokens (the reference's invariant,
    main.cu:311-337) and leaves the greedy run's K/V bytes below seq_len;
  * a window past the mapped blocks stops the loop with SDE_ERR_CAPACITY
    after the rounds that fit; bad arguments are rejected before any work.

The sampling loop (sde_spec_loop_stochastic, kernels.cu:3108-3481) against
oracle.spec_loop_stochastic: the same tokens, acceptances, seq_len, pool
SHA-256, final call index and (adapted) draft temperature, for seeds whose
every accept test and sample lies at least 1e-4 from its decision boundary
(the oracle reports that distance; device and oracle logits differ by
rounding, ~1e-5 of a probability here), with and without adaptation, and
k = 0 (plain sampling).
"""
import hashlib

import numpy as np
import pytest
import torch

from conftest import case_banner
from loop_model import make_loop_model, prefill, prompt_tokens
from speculative_decode_engine_amd import KVCache, SDEError
from speculative_decode_engine_amd.spec_loop import (SpecLoopModel, spec_loop_greedy,
                                                     spec_loop_stochastic)

pytestmark = pytest.mark.gpu


class DeviceKV:
    """prefill()'s cache interface over a KVCache."""

    def __init__(self, cache):
        self.c = cache

    def append(self, layer, k, v, pos):
        self.c.append(layer, torch.from_numpy(np.ascontiguousarray(k)).cuda(),
                      torch.from_numpy(np.ascontiguousarray(v)).cuda(), pos)

    def set_seq_len(self, n):
        self.c.set_seq_len(n)


def device_model(m):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return SpecLoopModel(t(m.emb_q), t(m.emb_k), t(m.emb_v), t(m.head.view(np.float16)),
                         m.nh, m.nkv, m.dph)


def run_both(oracle, m, k, n_draft, max_new, seed, P0, nblk=None):
    nblk = nblk or -(-(P0 + max_new + k + 1) // 16)
    kvd = m.nkv * m.dph
    cache = KVCache(m.n_layers, kvd, nblk, 16, m.n_layers * nblk)
    model = oracle.PagedKVModel(m.n_layers, kvd, nblk, 16, m.n_layers * nblk)
    prompt = prompt_tokens(seed, P0, m.vocab)
    prefill(DeviceKV(cache), m, prompt)
    prefill(model, m, prompt)
    anchor = int(np.random.default_rng(seed).integers(0, m.vocab))
    res = spec_loop_greedy(cache, device_model(m), anchor, k, n_draft, max_new)
    return res, cache, model, anchor


def pool_sha(cache):
    torch.cuda.synchronize()
    return hashlib.sha256(cache.pool.cpu().numpy().tobytes()).hexdigest()


CASES = [
    # seed, (L, nh, nkv, dph, V), P0, k, n_draft
    (3, (4, 4, 2, 64, 256), 40, 4, 2),
    (6, (4, 4, 2, 64, 256), 40, 7, 1),
    (5, (3, 8, 2, 128, 512), 700, 4, 1),
    (9, (2, 32, 8, 128, 1024), 2000, 5, 1),   # Llama-3-8B heads, multi-partition windows
    (7, (3, 8, 2, 64, 512), 300, 15, 1),      # the largest window: the head in two passes of 8
    (8, (2, 8, 2, 128, 256), 100, 9, 1),      # 10 rows: two passes of 5
    (11, (2, 8, 2, 64, 4096), 120, 4, 1),     # vocab 4096: 16-column head panels into the argmax
    (13, (3, 4, 2, 96, 256), 300, 3, 1),      # head size 96: the grid attention's generic path
]


@pytest.mark.parametrize("seed,shape,P0,k,n_draft", CASES)
def test_spec_loop_matches_oracle_and_greedy(gpu, oracle, seed, shape, P0, k, n_draft):
    L, nh, nkv, dph, V = shape
    case_banner("spec loop", seed, shape, P0, k, n_draft)
    m = make_loop_model(seed, n_layers=L, nh=nh, nkv=nkv, dph=dph, vocab=V, noise=0.1,
                        q_scale=2.0)
    max_new = 32
    greedy, gcache, gmodel, anchor = run_both(oracle, m, 0, 0, max_new, seed, P0,
                                              nblk=-(-(P0 + max_new + k + 1) // 16))
    g_toks, g_acc, _ = oracle.spec_loop_greedy(gmodel, m.emb_q, m.emb_k, m.emb_v, m.head, nh,
                                               nkv, dph, anchor, 0, 0, max_new)
    assert greedy.status == 0
    assert greedy.tokens == g_toks and greedy.accepted == g_acc == [0] * max_new
    assert greedy.seq_len == gmodel.seq_len == P0 + max_new
    assert pool_sha(gcache) == gmodel.pool_sha256()

    spec, scache, smodel, _ = run_both(oracle, m, k, n_draft, max_new, seed, P0)
    s_toks, s_acc, _ = oracle.spec_loop_greedy(smodel, m.emb_q, m.emb_k, m.emb_v, m.head, nh,
                                               nkv, dph, anchor, k, n_draft, max_new)
    assert spec.status == 0
    assert spec.tokens == s_toks and spec.accepted == s_acc
    assert spec.seq_len == smodel.seq_len == P0 + len(spec.tokens)
    assert pool_sha(scache) == smodel.pool_sha256()
    # the reference's invariant, on the device: speculation emits the greedy
    # tokens and keeps the greedy run's K/V bytes below seq_len
    assert spec.tokens[:max_new] == greedy.tokens
    assert spec.rounds < max_new and any(a > 0 for a in spec.accepted)
    n = P0 + max_new
    for l in range(L):
        gk, gv = gcache.read(l, 0, n)
        sk, sv = scache.read(l, 0, n)
        assert torch.equal(gk, sk) and torch.equal(gv, sv)
    gcache.free()
    scache.free()


@pytest.mark.parametrize("stochastic", [False, True])
def test_spec_loop_rejects_out_of_vocabulary_anchor(gpu, stochastic):
    """An anchor outside [0, vocab) reaches the device through the C-ABI
    (the Python wrappers refuse it): the launch records
    SDE_ERR_INVALID_ARGUMENT and stops at its first round check, before any
    table read -- no token, no append, seq_len unchanged."""
    case_banner("spec loop bad anchor", stochastic)
    import ctypes
    from speculative_decode_engine_amd import _native as N
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    cache = KVCache(m.n_layers, m.nkv * m.dph, 8, 16, m.n_layers * 8)
    cache.set_seq_len(10)
    dm = device_model(m)
    with pytest.raises(ValueError):
        spec_loop_greedy(cache, dm, m.vocab, 2, 1, 4)
    lib = N.load()
    state = torch.zeros(8, dtype=torch.int32, device="cuda")
    state[0] = m.vocab + 5
    em = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    ac = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    ws = torch.empty(lib.sde_spec_loop_workspace_size(cache.handle, ctypes.byref(dm.c), 2),
                     dtype=torch.uint8, device="cuda")
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    before = cache.pool.clone()
    if stochastic:
        off = torch.zeros(1, dtype=torch.int64, device="cuda")
        smp = N.LoopSampling(1.0, 0, 0.1, 2.0, 0.7, 0.1, 0.2, 5)
        rc = lib.sde_spec_loop_stochastic(cache.handle, ctypes.byref(dm.c), 2, 1, 4,
                                          ctypes.byref(smp), vp(off), vp(state), vp(em), vp(ac),
                                          vp(ws), ws.numel(), None)
    else:
        rc = lib.sde_spec_loop_greedy(cache.handle, ctypes.byref(dm.c), 2, 1, 4, vp(state),
                                      vp(em), vp(ac), vp(ws), ws.numel(), None)
    assert rc == 0  # the launch itself is valid; the device rejects the anchor
    torch.cuda.synchronize()
    st = state.cpu().tolist()
    assert st[3] == N.SDE_ERR_INVALID_ARGUMENT and st[1] == 0 and st[2] == 0
    assert torch.equal(cache.pool, before) and cache.device_seq_len() == 10
    assert (em == -1).all() and (ac == -1).all()
    cache.free()


def test_spec_loop_stops_at_capacity(gpu, oracle):
    case_banner("spec loop capacity")
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    P0, k = 40, 4
    # 4 blocks = 64 positions: rounds run while P + k + 1 <= 64
    res, cache, model, anchor = run_both(oracle, m, k, 2, 64, 3, P0, nblk=4)
    assert res.status == 2  # SDE_ERR_CAPACITY
    assert res.seq_len + k + 1 > 64 and res.seq_len <= 64
    toks, acc, _ = oracle.spec_loop_greedy(model, m.emb_q, m.emb_k, m.emb_v, m.head, m.nh, m.nkv,
                                           m.dph, anchor, k, 2, len(res.tokens))
    assert res.tokens == toks[:len(res.tokens)] and res.accepted == acc[:len(res.accepted)]
    cache.free()


def test_spec_loop_rejects_bad_arguments(gpu):
    case_banner("spec loop errors")
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    cache = KVCache(m.n_layers, m.nkv * m.dph, 8, 16, m.n_layers * 8)
    cache.set_seq_len(10)
    dm = device_model(m)
    before = cache.pool.clone()
    for k, n_draft, status in ((16, 1, 3), (4, 0, 1), (4, m.n_layers, 1), (-1, 1, 3)):
        with pytest.raises(SDEError) as e:
            spec_loop_greedy(cache, dm, 5, k, n_draft, 8)
        assert e.value.status == status
    odd = SpecLoopModel(dm.emb_q[:, :250].contiguous(), dm.emb_k[:, :250].contiguous(),
                        dm.emb_v[:, :250].contiguous(), dm.head[:, :250].contiguous(),
                        m.nh, m.nkv, m.dph)
    with pytest.raises(SDEError) as e:
        spec_loop_greedy(cache, odd, 5, 2, 1, 8)
    assert e.value.status == 4  # vocab not a multiple of 8
    torch.cuda.synchronize()
    assert torch.equal(cache.pool, before) and cache.device_seq_len() == 10
    cache.free()


STOCH_CASES = [
    # seed, (L, nh, nkv, dph, V), P0, k, n_draft, draft temp, adaptive, rng seed
    (3, (4, 4, 2, 64, 256), 40, 4, 2, 1.0, False, 14),
    (3, (4, 4, 2, 64, 256), 40, 4, 2, 1.0, False, 16),
    (6, (4, 4, 2, 64, 256), 40, 7, 1, 0.8, True, 9),
    (6, (4, 4, 2, 64, 256), 40, 7, 1, 0.8, True, 36),
    (5, (3, 8, 2, 128, 512), 300, 4, 1, 1.0, False, 25),
    (3, (4, 4, 2, 64, 256), 40, 0, 0, 1.0, False, 1),   # k = 0: plain sampling
    (7, (3, 8, 2, 64, 512), 60, 15, 1, 0.8, True, 19),  # the largest window: two head passes
    (8, (2, 8, 2, 128, 256), 40, 9, 1, 1.0, False, 2),  # 10 rows
]


@pytest.mark.parametrize("seed,shape,P0,k,n_draft,temp,adaptive,rseed,head_scale",
                         [c + (8.0,) for c in STOCH_CASES] +
                         # vocab 8192: two vocabulary slices per row (a sharper head keeps
                         # every decision clear of its boundary at this vocabulary size)
                         [(12, (2, 8, 2, 64, 8192), 60, 4, 1, 1.0, False, 8, 32.0)])
def test_stochastic_loop_matches_oracle(gpu, oracle, seed, shape, P0, k, n_draft, temp,
                                        adaptive, rseed, head_scale):
    L, nh, nkv, dph, V = shape
    case_banner("spec loop stochastic", seed, shape, P0, k, n_draft, temp, adaptive, rseed)
    m = make_loop_model(seed, n_layers=L, nh=nh, nkv=nkv, dph=dph, vocab=V, noise=0.1,
                        q_scale=2.0, head_scale=head_scale)
    max_new = 16
    nblk = -(-(P0 + max_new + k + 1) // 16)
    kvd = nkv * dph
    cache = KVCache(L, kvd, nblk, 16, L * nblk)
    model = oracle.PagedKVModel(L, kvd, nblk, 16, L * nblk)
    prompt = prompt_tokens(seed, P0, V)
    prefill(DeviceKV(cache), m, prompt)
    prefill(model, m, prompt)
    anchor = int(np.random.default_rng(seed).integers(0, V))
    toks, acc, rounds, t_fin, ewma, off, margin = oracle.spec_loop_stochastic(
        model, m.emb_q, m.emb_k, m.emb_v, m.head, nh, nkv, dph, anchor, k, n_draft, max_new,
        rseed, 0, temp, adaptive)
    assert margin > 1e-4  # the case's decisions are all clear of their boundaries
    offset = torch.zeros(1, dtype=torch.int64, device="cuda")
    res = spec_loop_stochastic(cache, device_model(m), anchor, k, n_draft, max_new, rseed,
                               draft_temp=temp, adaptive=adaptive, offset=offset)
    assert res.status == 0
    assert res.tokens == toks and res.accepted == acc and res.rounds == rounds
    assert res.seq_len == model.seq_len == P0 + len(toks)
    assert int(offset.item()) == off == rounds * (k + 1)
    assert pool_sha(cache) == model.pool_sha256()
    assert abs(res.draft_temp - t_fin) <= 1e-5 * max(1.0, abs(t_fin))
    if adaptive:
        assert res.draft_temp != temp and abs(res.accept_ewma - ewma) <= 1e-5
    else:
        assert res.draft_temp == np.float32(temp) and res.accept_ewma == -1.0
    cache.free()


def test_stochastic_loop_rejects_bad_arguments(gpu):
    case_banner("spec loop stochastic errors")
    import ctypes
    from speculative_decode_engine_amd import _native as N
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    cache = KVCache(m.n_layers, m.nkv * m.dph, 8, 16, m.n_layers * 8)
    cache.set_seq_len(10)
    dm = device_model(m)
    lib = N.load()
    state = torch.zeros(8, dtype=torch.int32, device="cuda")
    em = torch.zeros(16, dtype=torch.int32, device="cuda")
    ac = torch.zeros(8, dtype=torch.int32, device="cuda")
    off = torch.zeros(1, dtype=torch.int64, device="cuda")
    ws = torch.empty(lib.sde_spec_loop_workspace_size(cache.handle, ctypes.byref(dm.c), 2),
                     dtype=torch.uint8, device="cuda")
    vp = lambda t: ctypes.c_void_p(t.data_ptr())

    def call(smp, offp):
        return lib.sde_spec_loop_stochastic(cache.handle, ctypes.byref(dm.c), 2, 1, 4, smp, offp,
                                            vp(state), vp(em), vp(ac), vp(ws), ws.numel(), None)
    good = N.LoopSampling(1.0, 0, 0.1, 2.0, 0.7, 0.1, 0.2, 5)
    assert call(None, vp(off)) == N.SDE_ERR_INVALID_ARGUMENT
    assert call(ctypes.byref(good), None) == N.SDE_ERR_INVALID_ARGUMENT
    bad = N.LoopSampling(float("nan"), 0, 0.1, 2.0, 0.7, 0.1, 0.2, 5)
    assert call(ctypes.byref(bad), vp(off)) == N.SDE_ERR_INVALID_ARGUMENT
    bad = N.LoopSampling(1.0, 1, 2.0, 0.1, 0.7, 0.1, 0.2, 5)  # min > max, adaptive
    assert call(ctypes.byref(bad), vp(off)) == N.SDE_ERR_INVALID_ARGUMENT
    assert call(ctypes.byref(good), ctypes.c_void_p(off.data_ptr() + 4)) == \
        N.SDE_ERR_INVALID_ARGUMENT  # offset alignment
    torch.cuda.synchronize()
    assert cache.device_seq_len() == 10 and int(off.item()) == 0
    cache.free()
