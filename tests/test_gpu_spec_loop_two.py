"""The persistent loops with a separate draft model over a cache of its own,
and the EOS stop, through the C-ABI (sde_spec_loop), against the oracle's
two-cache restatements (oracle.spec_loop_greedy_two / _stochastic_two).

megakernel_speculative(_stochastic)_kernel with shared_kv false
(kernels.cu:2864-3106, 3108-3481): the draft model drafts k tokens into its
own cache from its device seq_len D, the target verifies the window at P,
the accept rewinds the target to P + n + 1 and the draft to D + n
(draft_save + n_accepted), and the draft's catch-up forward appends the last
draft (all k accepted) or the bonus at D + n (kernels.cu:3079-3093).
eos_token ends the loop after a round whose bonus is that token
(kernels.cu:3095, 3471).  Checked, per case: emitted tokens, per-round
acceptances, both device seq_lens and the SHA-256 of both pools (stale
rejected drafts included) equal the oracle's; greedy speculation emits the
target's greedy tokens whatever the draft (the reference's invariant,
main.cu:311-337) and leaves the greedy run's K/V bytes below seq_len.
"""
import ctypes
import hashlib

import numpy as np
import pytest
import torch

from conftest import case_banner
from loop_model import LoopModelNp, make_loop_model, prefill, prompt_tokens
from speculative_decode_engine_amd import KVCache, SDEError
from speculative_decode_engine_amd import _native as N
from speculative_decode_engine_amd.spec_loop import (SpecLoopModel, spec_loop_greedy,
                                                     spec_loop_stochastic)

pytestmark = pytest.mark.gpu


class DeviceKV:
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


def pool_sha(cache):
    torch.cuda.synchronize()
    return hashlib.sha256(cache.pool.cpu().numpy().tobytes()).hexdigest()


def lm(m):
    return (m.emb_q, m.emb_k, m.emb_v, m.head, m.nh, m.nkv, m.dph)


def draft_of(m, kind, V, head_scale=8.0):
    if kind == "prefix":     # the target's first two layers over a cache of its own
        return LoopModelNp(m.emb_q[:2], m.emb_k[:2], m.emb_v[:2], m.head, m.nh, m.nkv, m.dph)
    if kind == "same":       # the target itself: every draft accepted
        return m
    if kind == "zero":       # a zero head: proposes token 0, every draft rejected
        return LoopModelNp(m.emb_q[:1], m.emb_k[:1], m.emb_v[:1], np.zeros_like(m.head), m.nh,
                           m.nkv, m.dph)
    if kind == "other":      # another model, another shape (kv_dim 64)
        return make_loop_model(50, n_layers=2, nh=4, nkv=1, dph=64, vocab=V, noise=0.1,
                               q_scale=2.0, head_scale=head_scale)
    if kind == "dph96":      # head size 96: the draft side on the generic attention path
        return make_loop_model(52, n_layers=2, nh=4, nkv=2, dph=96, vocab=V, noise=0.1,
                               q_scale=2.0, head_scale=head_scale)
    return make_loop_model(51, n_layers=1, nh=4, nkv=2, dph=64, vocab=V, noise=0.1,
                           q_scale=2.0, head_scale=head_scale)  # "small": dph 64 under dph 128


class Pair:
    """Target and draft caches on the device and in the oracle, prefilled
    with the same prompt (both at seq_len P0)."""

    def __init__(self, oracle, tm, dm, P0, max_new, k, seed, nblk_draft=None):
        nblk = -(-(P0 + 2 * max_new + k + 2) // 16)
        nd = nblk_draft or nblk
        self.cache = KVCache(tm.n_layers, tm.nkv * tm.dph, nblk, 16, tm.n_layers * nblk)
        self.dcache = KVCache(dm.n_layers, dm.nkv * dm.dph, nd, 16, dm.n_layers * nd)
        self.tmod = oracle.PagedKVModel(tm.n_layers, tm.nkv * tm.dph, nblk, 16,
                                        tm.n_layers * nblk)
        self.dmod = oracle.PagedKVModel(dm.n_layers, dm.nkv * dm.dph, nd, 16, dm.n_layers * nd)
        prompt = prompt_tokens(seed, P0, tm.vocab)
        for c, mm in ((DeviceKV(self.cache), tm), (DeviceKV(self.dcache), dm),
                      (self.tmod, tm), (self.dmod, dm)):
            prefill(c, mm, prompt)
        self.anchor = int(np.random.default_rng(seed).integers(0, tm.vocab))
        self.tdev, self.ddev = device_model(tm), device_model(dm)

    def check(self, res, toks, acc, rounds):
        assert res.status == 0
        assert res.tokens == toks and res.accepted == acc and res.rounds == rounds
        assert res.seq_len == self.tmod.seq_len
        assert res.draft_seq_len == self.dmod.seq_len
        assert pool_sha(self.cache) == self.tmod.pool_sha256()
        assert pool_sha(self.dcache) == self.dmod.pool_sha256()

    def free(self):
        self.cache.free()
        self.dcache.free()


GREEDY_CASES = [
    # seed, target (L, nh, nkv, dph, V), draft kind, P0, k
    (3, (4, 4, 2, 64, 256), "prefix", 40, 4),
    (3, (4, 4, 2, 64, 256), "prefix", 40, 1),
    (3, (4, 4, 2, 64, 256), "same", 40, 4),     # all accepted: catch-up of the last draft
    (3, (4, 4, 2, 64, 256), "zero", 40, 2),     # none accepted: catch-up of the bonus
    (6, (4, 4, 2, 64, 256), "other", 40, 3),    # draft kv_dim 64 under target kv_dim 128
    (5, (3, 8, 2, 128, 512), "small", 700, 5),  # dph 64 draft, dph 128 multi-partition target
    (11, (2, 8, 2, 64, 4096), "prefix", 120, 4),  # vocab 4096: 16-column head panels
    (6, (3, 4, 2, 64, 256), "dph96", 200, 3),   # a generic-path draft: separate q / append phases
]


@pytest.mark.parametrize("seed,shape,kind,P0,k", GREEDY_CASES)
def test_two_cache_greedy_loop_matches_oracle_and_greedy(gpu, oracle, seed, shape, kind, P0, k):
    L, nh, nkv, dph, V = shape
    case_banner("two-cache greedy loop", seed, shape, kind, P0, k)
    m = make_loop_model(seed, n_layers=L, nh=nh, nkv=nkv, dph=dph, vocab=V, noise=0.1,
                        q_scale=2.0)
    d = draft_of(m, kind, V, head_scale=1.0)
    max_new = 32
    p = Pair(oracle, m, d, P0, max_new, k, seed)
    toks, acc, rounds = oracle.spec_loop_greedy_two(p.tmod, p.dmod, lm(m), lm(d), p.anchor, k,
                                                    max_new)
    res = spec_loop_greedy(p.cache, p.tdev, p.anchor, k, 0, max_new, draft_cache=p.dcache,
                           draft_model=p.ddev)
    p.check(res, toks, acc, rounds)
    if kind == "same":
        assert acc == [k] * rounds
    if kind == "zero" and 0 not in toks:
        assert acc == [0] * rounds
    # the invariant: the target's greedy tokens and K/V bytes, whatever the draft
    g = KVCache(L, nkv * dph, p.cache.max_blocks_per_layer, 16, L * p.cache.max_blocks_per_layer)
    prefill(DeviceKV(g), m, prompt_tokens(seed, P0, V))
    greedy = spec_loop_greedy(g, p.tdev, p.anchor, 0, 0, max_new)
    assert greedy.status == 0 and res.tokens[:max_new] == greedy.tokens
    n = P0 + max_new
    for l in range(L):
        gk, gv = g.read(l, 0, n)
        sk, sv = p.cache.read(l, 0, n)
        assert torch.equal(gk, sk) and torch.equal(gv, sv)
    g.free()
    p.free()


STOCH_CASES = [
    # seed, target shape, draft kind, P0, k, draft temp, adaptive, rng seed
    (3, (4, 4, 2, 64, 256), "prefix", 40, 4, 1.0, False, 1),
    (3, (4, 4, 2, 64, 256), "prefix", 40, 4, 1.0, False, 9),
    (6, (4, 4, 2, 64, 256), "other", 40, 3, 0.8, True, 3),
    (5, (3, 8, 2, 128, 512), "small", 300, 4, 1.0, False, 19),
]


@pytest.mark.parametrize("seed,shape,kind,P0,k,temp,adaptive,rseed", STOCH_CASES)
def test_two_cache_stochastic_loop_matches_oracle(gpu, oracle, seed, shape, kind, P0, k, temp,
                                                  adaptive, rseed):
    L, nh, nkv, dph, V = shape
    case_banner("two-cache stochastic loop", seed, shape, kind, P0, k, temp, adaptive, rseed)
    m = make_loop_model(seed, n_layers=L, nh=nh, nkv=nkv, dph=dph, vocab=V, noise=0.1,
                        q_scale=2.0, head_scale=8.0)
    d = draft_of(m, kind, V)
    max_new = 16
    p = Pair(oracle, m, d, P0, max_new, k, seed)
    toks, acc, rounds, t_fin, ewma, off, margin = oracle.spec_loop_stochastic_two(
        p.tmod, p.dmod, lm(m), lm(d), p.anchor, k, max_new, rseed, 0, temp, adaptive)
    assert margin > 1e-4  # every decision clear of its boundary
    offset = torch.zeros(1, dtype=torch.int64, device="cuda")
    res = spec_loop_stochastic(p.cache, p.tdev, p.anchor, k, 0, max_new, rseed, draft_temp=temp,
                               adaptive=adaptive, offset=offset, draft_cache=p.dcache,
                               draft_model=p.ddev)
    p.check(res, toks, acc, rounds)
    assert int(offset.item()) == off == rounds * (k + 1)
    assert abs(res.draft_temp - t_fin) <= 1e-5 * max(1.0, abs(t_fin))
    if adaptive:
        assert abs(res.accept_ewma - ewma) <= 1e-5
    p.free()


def _round_ends(acc):
    return np.cumsum([a + 1 for a in acc])


@pytest.mark.parametrize("two", [False, True])
def test_greedy_loop_stops_on_the_eos_bonus(gpu, oracle, two):
    """eos_token = the bonus of round 3 of the unstopped run: the loop ends
    after the first round whose bonus it is, with fewer than max_new tokens,
    and cache, seq_len and tokens equal the oracle's stopped run."""
    case_banner("loop eos greedy", two)
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    max_new, k = 40, 4
    if two:
        d = draft_of(m, "prefix", m.vocab)
        p = Pair(oracle, m, d, 40, max_new, k, 3)
        toks, acc, _ = oracle.spec_loop_greedy_two(p.tmod, p.dmod, lm(m), lm(d), p.anchor, k,
                                                   max_new)
        p.free()
    else:
        p = Pair(oracle, m, m, 40, max_new, k, 3)
        toks, acc, _ = oracle.spec_loop_greedy(p.tmod, *lm(m), p.anchor, k, 2, max_new)
        p.free()
    ends = _round_ends(acc)
    eos = toks[ends[3] - 1]
    first = next(i for i in range(len(acc)) if toks[ends[i] - 1] == eos)
    d = draft_of(m, "prefix", m.vocab) if two else m
    p = Pair(oracle, m, d, 40, max_new, k, 3)
    if two:
        t2, a2, r2 = oracle.spec_loop_greedy_two(p.tmod, p.dmod, lm(m), lm(d), p.anchor, k,
                                                 max_new, eos_token=eos)
        res = spec_loop_greedy(p.cache, p.tdev, p.anchor, k, 0, max_new, eos_token=eos,
                               draft_cache=p.dcache, draft_model=p.ddev)
        p.check(res, t2, a2, r2)
    else:
        t2, a2, r2 = oracle.spec_loop_greedy(p.tmod, *lm(m), p.anchor, k, 2, max_new,
                                             eos_token=eos)
        res = spec_loop_greedy(p.cache, p.tdev, p.anchor, k, 2, max_new, eos_token=eos)
        assert res.status == 0 and res.tokens == t2 and res.accepted == a2
        assert res.seq_len == p.tmod.seq_len
        assert pool_sha(p.cache) == p.tmod.pool_sha256()
    assert r2 == first + 1 and t2 == toks[:ends[first]] and len(t2) < max_new
    assert res.tokens[-1] == eos
    p.free()


def test_self_speculative_stochastic_loop_stops_on_the_eos_bonus(gpu, oracle):
    """The self-speculative sampling loop's EOS stop (kernels.cu:3471)."""
    case_banner("loop eos stochastic self")
    m = make_loop_model(3, noise=0.1, q_scale=2.0, head_scale=8.0)
    max_new, k, nd = 16, 4, 2
    p = Pair(oracle, m, m, 40, max_new, k, 3)
    toks, acc, *_ = oracle.spec_loop_stochastic(p.tmod, *lm(m), p.anchor, k, nd, max_new, 14)
    p.free()
    ends = _round_ends(acc)
    eos = toks[ends[1] - 1]
    p = Pair(oracle, m, m, 40, max_new, k, 3)
    t2, a2, r2, _, _, off, margin = oracle.spec_loop_stochastic(p.tmod, *lm(m), p.anchor, k, nd,
                                                                max_new, 14, eos_token=eos)
    assert margin > 1e-4 and t2[-1] == eos and len(t2) < max_new
    offset = torch.zeros(1, dtype=torch.int64, device="cuda")
    res = spec_loop_stochastic(p.cache, p.tdev, p.anchor, k, nd, max_new, 14, offset=offset,
                               eos_token=eos)
    assert res.status == 0 and res.tokens == t2 and res.accepted == a2 and res.rounds == r2
    assert res.seq_len == p.tmod.seq_len and pool_sha(p.cache) == p.tmod.pool_sha256()
    assert int(offset.item()) == off
    p.free()


def test_stochastic_loop_stops_on_the_eos_bonus(gpu, oracle):
    case_banner("loop eos stochastic")
    m = make_loop_model(3, noise=0.1, q_scale=2.0, head_scale=8.0)
    d = draft_of(m, "prefix", m.vocab)
    max_new, k = 16, 4
    p = Pair(oracle, m, d, 40, max_new, k, 3)
    toks, acc, *_ = oracle.spec_loop_stochastic_two(p.tmod, p.dmod, lm(m), lm(d), p.anchor, k,
                                                    max_new, 1)
    p.free()
    ends = _round_ends(acc)
    eos = toks[ends[2] - 1]
    p = Pair(oracle, m, d, 40, max_new, k, 3)
    t2, a2, r2, _, _, off, margin = oracle.spec_loop_stochastic_two(
        p.tmod, p.dmod, lm(m), lm(d), p.anchor, k, max_new, 1, eos_token=eos)
    assert margin > 1e-4 and t2[-1] == eos and r2 <= 3
    offset = torch.zeros(1, dtype=torch.int64, device="cuda")
    res = spec_loop_stochastic(p.cache, p.tdev, p.anchor, k, 0, max_new, 1, offset=offset,
                               eos_token=eos, draft_cache=p.dcache, draft_model=p.ddev)
    p.check(res, t2, a2, r2)
    assert int(offset.item()) == off
    p.free()


def test_two_cache_loop_stops_at_the_draft_capacity(gpu, oracle):
    """A draft cache mapping fewer positions than the target's: the loop
    stops with SDE_ERR_CAPACITY once a draft window D + k + 1 would pass
    them, after the rounds that fit (the oracle's first rounds)."""
    case_banner("two-cache draft capacity")
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    d = draft_of(m, "prefix", m.vocab)
    k = 4
    p = Pair(oracle, m, d, 40, 32, k, 3, nblk_draft=4)   # 64 draft positions
    res = spec_loop_greedy(p.cache, p.tdev, p.anchor, k, 0, 32, draft_cache=p.dcache,
                           draft_model=p.ddev)
    assert res.status == N.SDE_ERR_CAPACITY
    assert res.draft_seq_len + k + 1 > 64 and res.draft_seq_len <= 64
    toks, acc, _ = oracle.spec_loop_greedy_two(p.tmod, p.dmod, lm(m), lm(d), p.anchor, k,
                                               len(res.tokens))
    assert res.tokens == toks[:len(res.tokens)] and res.accepted == acc[:len(res.accepted)]
    p.free()


def test_two_cache_loop_rejects_bad_configurations(gpu):
    case_banner("two-cache loop errors")
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    cache = KVCache(m.n_layers, m.nkv * m.dph, 8, 16, m.n_layers * 8)
    dcache = KVCache(2, m.nkv * m.dph, 8, 16, 16)
    cache.set_seq_len(10)
    dcache.set_seq_len(10)
    tm = device_model(m)
    dm = device_model(draft_of(m, "prefix", m.vocab))
    with pytest.raises(ValueError):
        spec_loop_greedy(cache, tm, 5, 2, 0, 4, draft_model=dm)
    lib = N.load()
    state = torch.zeros(8, dtype=torch.int32, device="cuda")
    state[0] = 5
    em = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    ac = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    vp = lambda t: ctypes.c_void_p(t.data_ptr())

    def call(k, dc, dmod):
        cfg = N.LoopConfig(k, 1, 4, -1, dc, ctypes.pointer(dmod.c) if dmod else None)
        size = lib.sde_spec_loop_config_workspace_size(cache.handle, ctypes.byref(tm.c),
                                                       ctypes.byref(cfg))
        ws = torch.empty(max(size, 1 << 20), dtype=torch.uint8, device="cuda")
        return lib.sde_spec_loop(cache.handle, ctypes.byref(tm.c), ctypes.byref(cfg), None, None,
                                 vp(state), vp(em), vp(ac), vp(ws), ws.numel(), None)
    other_v = draft_of(m, "other", 512)
    bad_v = device_model(other_v)
    bad_cache = KVCache(2, 64, 8, 16, 16)
    assert call(2, cache.handle, dm) == N.SDE_ERR_INVALID_ARGUMENT      # the target's own cache
    assert call(0, dcache.handle, dm) == N.SDE_ERR_INVALID_ARGUMENT     # k = 0 with a draft
    assert call(2, dcache.handle, None) == N.SDE_ERR_INVALID_ARGUMENT   # a cache, no model
    assert call(2, bad_cache.handle, bad_v) == N.SDE_ERR_INVALID_ARGUMENT  # another vocabulary
    assert call(2, bad_cache.handle, dm) == N.SDE_ERR_INVALID_ARGUMENT  # kv_dim != the cache's
    assert lib.sde_spec_loop_config_workspace_size(
        cache.handle, ctypes.byref(tm.c),
        ctypes.byref(N.LoopConfig(2, 1, 4, -1, dcache.handle, None))) == 0
    torch.cuda.synchronize()
    assert cache.device_seq_len() == 10 and dcache.device_seq_len() == 10
    assert (em == -1).all() and (ac == -1).all()
    with pytest.raises(SDEError) as e:  # the same through the wrapper
        spec_loop_greedy(cache, tm, 5, 2, 0, 4, draft_cache=bad_cache, draft_model=dm)
    assert e.value.status == N.SDE_ERR_INVALID_ARGUMENT
    for c in (cache, dcache, bad_cache):
        c.free()
