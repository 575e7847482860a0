"""Greedy speculative decoding == greedy decoding, on the CPU oracle cache.

The reference's end-to-end pin for its KV cache (main.cu:311-337,
cli/benchmark.py:73-80) restated with a tiny random model
(tests/tiny_llama.py): two-model speculation with a perturbed draft (most
drafts rejected), with an identical draft (every draft accepted, so the draft
cache takes the extra append of d_k, kernels.cu:2466-2476), and self-
speculation over one shared cache.  Positions come from the caches' seq_len,
so the rewind is what places the next round's appends.  The planted-mistake
tests show the check fails for a rewind that keeps one rejected draft or
drops one accepted token.
"""
import numpy as np
import pytest

from tiny_llama import (OracleCache, TinyConfig, TinyLlama, greedy, host_accept, spec_self,
                        spec_two_model, spec_two_model_reference)

CFG = TinyConfig()
PROMPT = [3, 17, 101, 250, 9, 44, 300, 7]
N_NEW = 40
POSITIONS = 128  # room for a broken rewind that keeps rejected drafts
K = 4


def _models(seed, mode):
    target = TinyLlama(CFG, seed)
    if mode == "perturbed":
        return target, TinyLlama(CFG, seed + 100, base=target, noise=0.05, n_layers=2)
    return target, target


def run_spec(oracle, seed, mode, cache_cls=OracleCache, stats=None):
    target, draft = _models(seed, mode)
    if mode == "self":
        return spec_self(target, cache_cls(oracle, CFG, CFG.n_layers, POSITIONS, seed), PROMPT,
                         N_NEW, K, n_draft=3, stats=stats)
    tc = cache_cls(oracle, CFG, CFG.n_layers, POSITIONS, seed)
    dc = cache_cls(oracle, CFG, draft.n_layers, POSITIONS, seed + 1)
    return spec_two_model(target, draft, tc, dc, PROMPT, N_NEW, K, stats=stats)


@pytest.mark.parametrize("seed", [1, 2])
@pytest.mark.parametrize("mode", ["perturbed", "identical", "self"])
def test_greedy_speculation_emits_greedy_tokens(oracle, seed, mode):
    ref = greedy(TinyLlama(CFG, seed), OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed),
                 PROMPT, N_NEW)
    stats = {}
    out = run_spec(oracle, seed, mode, stats=stats)
    assert out == ref
    acc = stats["accepted"]
    if mode == "identical":
        assert all(a == K for a in acc[:-1])          # every draft accepted
    else:
        assert any(a < K for a in acc) and any(a > 0 for a in acc)


class _KeepsOneRejected(OracleCache):
    def rollback(self, n):
        super().rollback(min(n + 1, self.seq_len))


class _DropsOneAccepted(OracleCache):
    def rollback(self, n):
        super().rollback(max(n - 1, 0))


@pytest.mark.parametrize("broken", [_KeepsOneRejected, _DropsOneAccepted])
@pytest.mark.parametrize("mode", ["perturbed", "self"])
def test_planted_rewind_mistakes_break_the_invariant(oracle, broken, mode):
    seed = 1
    ref = greedy(TinyLlama(CFG, seed), OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed),
                 PROMPT, N_NEW)
    assert run_spec(oracle, seed, mode, cache_cls=broken) != ref


@pytest.mark.parametrize("mode", ["perturbed", "identical"])
def test_reference_host_loop_with_oracle_accept_rule(oracle, mode):
    """The reference's host loop (draft rewound to save + n_acc) with the
    oracle's acceptance rule emits the greedy tokens too."""
    seed = 2
    ref = greedy(TinyLlama(CFG, seed), OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed),
                 PROMPT, N_NEW)
    target, draft = _models(seed, mode)
    tc = OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed)
    dc = OracleCache(oracle, CFG, draft.n_layers, POSITIONS, seed + 1)
    stats = {}
    out = spec_two_model_reference(target, draft, tc, dc, PROMPT, N_NEW, K,
                                   host_accept(oracle, tc, dc), stats)
    assert out == ref
    if mode == "identical":
        assert all(a == K for a in stats["accepted"][:-1])


def test_accept_rule_cases(oracle):
    # no match, partial, all; shared cache
    assert oracle.spec_accept_greedy([5, 6, 7], [1, 2, 3, 4], 3, 10, 10, False) == \
        (0, 1, 11, 10, [1])
    assert oracle.spec_accept_greedy([5, 6, 7], [5, 6, 3, 4], 3, 10, 8, False) == \
        (2, 3, 13, 10, [5, 6, 3])
    assert oracle.spec_accept_greedy([5, 6, 7], [5, 6, 7, 9], 3, 10, 10, True) == \
        (3, 9, 14, 14, [5, 6, 7, 9])
    assert oracle.spec_accept_greedy([], [4], 0, 3, 3, False) == (0, 4, 4, 3, [4])


def test_planted_accept_rule_mistake_breaks_the_loop(oracle):
    # target rewound to save + n_acc (the bonus position lost) must fail
    seed = 1
    ref = greedy(TinyLlama(CFG, seed), OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed),
                 PROMPT, N_NEW)
    target, draft = _models(seed, "perturbed")
    tc = OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed)
    dc = OracleCache(oracle, CFG, draft.n_layers, POSITIONS, seed + 1)
    good = host_accept(oracle, tc, dc)

    def bad(drafts, tt, k, ts, ds):
        n, b, t_seq, d_seq, em = good(drafts, tt, k, ts, ds)
        tc.rollback(t_seq - 1)
        return n, b, t_seq - 1, d_seq, em
    assert spec_two_model_reference(target, draft, tc, dc, PROMPT, N_NEW, K, bad) != ref


# ---- speculative sampling oracle (stochastic acceptance) -------------------

def test_philox_known_answers(oracle):
    # Random123's known-answer vectors for philox4x32-10
    kat = [([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
           ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
           ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
            [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1])]
    for ctr, key, want in kat:
        assert oracle.philox4x32_10(ctr, key) == want


def test_spec_draws_are_uniform(oracle):
    u = np.array([oracle.spec_draws(7, off, b) for off in range(400) for b in range(5)])
    assert ((u > 0) & (u < 1)).all()
    hist, _ = np.histogram(u.ravel(), bins=10, range=(0, 1))
    chi2 = ((hist - len(u.ravel()) / 10) ** 2 / (len(u.ravel()) / 10)).sum()
    assert chi2 < 27.9   # 9 dof, p = 0.001


def test_speculative_sampling_preserves_the_target_distribution(oracle):
    """The theorem speculative sampling rests on (Leviathan et al. 2023):
    the first emitted token is distributed as p, whatever the draft q."""
    rng = np.random.default_rng(8)
    V, trials = 8, 6000
    tl = rng.standard_normal((2, V)) * 1.5
    dl = rng.standard_normal((1, V)) * 1.5
    p = np.exp(tl[0] - tl[0].max()); p /= p.sum()
    q = np.exp(dl[0] - dl[0].max()); q /= q.sum()
    counts = np.zeros(V)
    for off in range(trials):
        # the draft token is sampled from q with an independent Philox draw
        u = oracle.spec_draws(99, off, 7)[0]
        d = int(np.searchsorted(np.cumsum(q), u))
        r = oracle.spec_accept_stochastic(tl, dl, [d], 1, 1.0, 1.0, 5, off, 10, 10, False)
        counts[r["emitted"][0]] += 1
    chi2 = ((counts - trials * p) ** 2 / (trials * p)).sum()
    assert chi2 < 24.3   # 7 dof, p = 0.001
    # planted mistake: always emitting the draft token (no rejection) is q, not p
    bad = np.zeros(V)
    for off in range(trials):
        u = oracle.spec_draws(99, off, 7)[0]
        bad[int(np.searchsorted(np.cumsum(q), u))] += 1
    assert ((bad - trials * p) ** 2 / (trials * p)).sum() > 100


def test_speculative_sampling_special_cases(oracle):
    V = 6
    tl = np.log(np.array([[.5, .2, .1, .1, .05, .05], [.1, .1, .1, .1, .1, .5]]))
    # q == p: the residual is empty and every draft is accepted (cap 1)
    r = oracle.spec_accept_stochastic(tl, tl[:1], [2], 1, 1.0, 1.0, 3, 0, 4, 4, True)
    assert r["flags"] == [True] and r["n_accepted"] == 1 and r["target_seq"] == 6
    # a draft token with p = 0 is always rejected; the correction excludes it
    tl0 = tl.copy()
    tl0[0, 3] = -np.inf
    for off in range(50):
        r = oracle.spec_accept_stochastic(tl0, tl[:1], [3], 1, 1.0, 1.0, 3, off, 4, 4, False)
        assert r["n_accepted"] == 0 and r["token"] != 3 and r["draft_seq"] == 4


# ---- the persistent loop's restatement (oracle.spec_loop_greedy) ------------
# sde_spec_loop_greedy's algorithm on the CPU byte model: self-speculation
# over one cache must emit the greedy tokens (k = 0) and leave the greedy
# run's K/V bytes below seq_len; a rewind one position off either way breaks
# it, so the check is sharp.

def loop_run(oracle, m, k, n_draft, max_new, seed, P0=40, shift=0):
    from loop_model import prefill, prompt_tokens
    nblk = -(-(P0 + 2 * max_new + k + 1) // 16)
    model = oracle.PagedKVModel(m.n_layers, m.nkv * m.dph, nblk, 16, m.n_layers * nblk)
    prefill(model, m, prompt_tokens(seed, P0, m.vocab))
    anchor = int(np.random.default_rng(seed).integers(0, m.vocab))
    toks, acc, _ = oracle.spec_loop_greedy(model, m.emb_q, m.emb_k, m.emb_v, m.head, m.nh,
                                           m.nkv, m.dph, anchor, k, n_draft, max_new, shift)
    return toks, acc, model


@pytest.mark.parametrize("seed,k,n_draft", [(3, 4, 2), (6, 7, 1), (5, 4, 3)])
def test_loop_restatement_speculation_emits_greedy_tokens(oracle, seed, k, n_draft):
    from loop_model import make_loop_model
    m = make_loop_model(seed, noise=0.1, q_scale=2.0)
    base, base_acc, bm = loop_run(oracle, m, 0, 0, 40, seed)
    assert base_acc == [0] * 40 and bm.seq_len == 80
    spec, acc, sm = loop_run(oracle, m, k, n_draft, 40, seed)
    assert spec[:40] == base
    assert any(a > 0 for a in acc) and any(a < k for a in acc)  # both rewind paths
    assert sm.seq_len == 40 + sum(a + 1 for a in acc) == 40 + len(spec)
    for l in range(m.n_layers):
        kb, vb = bm.gather(l, 0, 80)
        ks, vs = sm.gather(l, 0, 80)
        assert np.array_equal(kb, ks) and np.array_equal(vb, vs)


@pytest.mark.parametrize("shift", [-1, 1])
def test_loop_restatement_planted_rewind_mistake(oracle, shift):
    from loop_model import make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    base, _, _ = loop_run(oracle, m, 0, 0, 40, 3)
    spec, _, _ = loop_run(oracle, m, 4, 2, 40, 3, shift=shift)
    assert spec[:40] != base


# ---- the sampling loop's restatement (oracle.spec_loop_stochastic) ----------
# With one-hot distributions (logits thousands apart, draft temperature
# 1e-6) speculative sampling picks every argmax: the sampling loop must then
# emit exactly the greedy loop's tokens, acceptances and K/V bytes -- the
# window, the accept rule, the corrected sample and the rewind all line up.
# Its call indices advance by k + 1 per round, and the adaptive temperature
# follows its float32 rule.

def stoch_run(oracle, m, k, n_draft, max_new, seed, P0=40, **kw):
    from loop_model import prefill, prompt_tokens
    nblk = -(-(P0 + 2 * max_new + k + 1) // 16)
    model = oracle.PagedKVModel(m.n_layers, m.nkv * m.dph, nblk, 16, m.n_layers * nblk)
    prefill(model, m, prompt_tokens(seed, P0, m.vocab))
    anchor = int(np.random.default_rng(seed).integers(0, m.vocab))
    out = oracle.spec_loop_stochastic(model, m.emb_q, m.emb_k, m.emb_v, m.head, m.nh, m.nkv,
                                      m.dph, anchor, k, n_draft, max_new, 11, 0, **kw)
    return out, model


@pytest.mark.parametrize("seed,k,n_draft", [(3, 4, 2), (6, 7, 1), (3, 0, 0)])
def test_sampling_loop_restatement_with_one_hot_distributions_is_greedy(oracle, seed, k,
                                                                         n_draft):
    from loop_model import make_loop_model
    m = make_loop_model(seed, noise=0.1, q_scale=2.0, head_scale=4000.0)
    greedy, g_acc, gm = loop_run(oracle, m, k, n_draft, 24, seed)
    (toks, acc, rounds, temp, ewma, off, _), sm = stoch_run(oracle, m, k, n_draft, 24, seed,
                                                             draft_temp=1e-6)
    assert toks == greedy and acc == g_acc and sm.seq_len == gm.seq_len
    assert off == rounds * (k + 1) and temp == np.float32(1e-6) and ewma == -1.0
    if k:
        assert any(a > 0 for a in acc) and any(a < k for a in acc)
    assert sm.pool_sha256() == gm.pool_sha256()


def test_sampling_loop_restatement_adapts_the_draft_temperature(oracle):
    from loop_model import make_loop_model
    m = make_loop_model(6, noise=0.1, q_scale=2.0, head_scale=8.0)
    k = 7
    (toks, acc, rounds, temp, ewma, off, _), _ = stoch_run(
        oracle, m, k, 1, 16, 6, draft_temp=0.8, adaptive=True, min_temp=0.1, max_temp=2.0,
        target_accept=0.7, gain=0.1, ewma_mix=0.2)
    f = np.float32
    t, e = f(0.8), f(-1.0)
    # (the closed forms of test_sampling_loop_temperature_rule_closed_forms
    # pin the rule; here: it moved, within its clamp, with the call indices)
    assert 0.1 <= temp <= 2.0 and temp != np.float32(0.8) and 0.0 <= ewma <= 1.0
    assert off == rounds * (k + 1) and len(acc) == rounds


def test_sampling_loop_temperature_rule_closed_forms(oracle):
    """The adaptive draft temperature (kernels.cu:3441-3458) by closed forms
    instead of a restatement, on the two-cache sampling loop with one-hot
    distributions: a draft identical to the target accepts every draft
    (rate 1), so T_d rises by gain * (1 - target) per round up to max_temp; a
    draft that proposes only token 0 (a zero head) is rejected every round
    (rate 0), so T_d falls by gain * target per round down to min_temp; with
    gain 0 T_d stays put."""
    from loop_model import LoopModelNp, make_loop_model
    m = make_loop_model(6, noise=0.1, q_scale=2.0, head_scale=4000.0)
    k, gain, tgt = 3, 0.1, 0.7
    kw = dict(draft_temp=1.0, adaptive=True, min_temp=0.1, max_temp=2.0, target_accept=tgt,
              gain=gain, ewma_mix=0.2)
    (toks, acc, rounds, temp, ewma, off, _), _, _, _ = two_run(oracle, m, m, k, 24, 6, stoch=kw)
    assert acc == [k] * rounds and ewma == 1.0 and off == rounds * (k + 1)
    assert abs(temp - min(2.0, 1.0 + rounds * gain * (1 - tgt))) < 1e-5
    zero = LoopModelNp(m.emb_q[:1], m.emb_k[:1], m.emb_v[:1], np.zeros_like(m.head), m.nh,
                       m.nkv, m.dph)
    (toks, acc, rounds, temp, ewma, _, _), _, _, _ = two_run(oracle, m, zero, 1, 12, 6,
                                                             stoch=dict(kw, draft_temp=1e-6))
    assert acc == [0] * rounds and ewma == 0.0 and rounds == 12
    assert abs(temp - max(0.1, 1e-6 - rounds * gain * tgt)) < 1e-5
    (_, acc, rounds, temp, _, _, _), _, _, _ = two_run(oracle, m, zero, 1, 12, 6,
                                                       stoch=dict(kw, draft_temp=0.5, gain=0.0))
    assert temp == np.float32(0.5)


# ---- the two-cache loops (a separate draft model and cache) ---------------
# megakernel_speculative(_stochastic)_kernel with shared_kv false: the draft
# model drafts into its own cache, rewinds to draft_save + n, and catches up
# with the last draft (all accepted) or the bonus token (kernels.cu:3066-3093).

def two_run(oracle, tm, dm, k, max_new, seed, P0=40, eos=-1, shift=0, stoch=None):
    from loop_model import prefill, prompt_tokens
    nblk = -(-(P0 + 2 * max_new + k + 2) // 16)
    tmod = oracle.PagedKVModel(tm.n_layers, tm.nkv * tm.dph, nblk, 16, tm.n_layers * nblk)
    dmod = oracle.PagedKVModel(dm.n_layers, dm.nkv * dm.dph, nblk, 16, dm.n_layers * nblk)
    prompt = prompt_tokens(seed, P0, tm.vocab)
    prefill(tmod, tm, prompt)
    prefill(dmod, dm, prompt)
    anchor = int(np.random.default_rng(seed).integers(0, tm.vocab))
    T = (tm.emb_q, tm.emb_k, tm.emb_v, tm.head, tm.nh, tm.nkv, tm.dph)
    D = (dm.emb_q, dm.emb_k, dm.emb_v, dm.head, dm.nh, dm.nkv, dm.dph)
    if stoch is None:
        out = oracle.spec_loop_greedy_two(tmod, dmod, T, D, anchor, k, max_new, eos, shift)
    else:
        out = oracle.spec_loop_stochastic_two(tmod, dmod, T, D, anchor, k, max_new, 11, 0,
                                              eos_token=eos, **stoch)
    return out, tmod, dmod, anchor


def _drafts(m, kind):
    from loop_model import LoopModelNp, make_loop_model
    if kind == "prefix":       # the target's first two layers, its own cache
        return LoopModelNp(m.emb_q[:2], m.emb_k[:2], m.emb_v[:2], m.head, m.nh, m.nkv, m.dph)
    return make_loop_model(50, n_layers=2, nh=4, nkv=1, dph=64, vocab=m.vocab)  # other shape


@pytest.mark.parametrize("kind,k", [("prefix", 4), ("prefix", 1), ("other", 3)])
def test_two_cache_loop_restatement_emits_greedy_tokens(oracle, kind, k):
    from loop_model import make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    base, _, bm = loop_run(oracle, m, 0, 0, 40, 3)
    (toks, acc, rounds), tm, dm, _ = two_run(oracle, m, _drafts(m, kind), k, 40, 3)
    assert toks[:40] == base
    # both rewinds add n + 1 per round (the draft's catch-up included)
    assert tm.seq_len == 40 + len(toks) and dm.seq_len == tm.seq_len
    if kind == "prefix":
        assert any(a > 0 for a in acc) and any(a < k for a in acc)
    for l in range(m.n_layers):  # the target's bytes below seq_len are the greedy run's
        kb, vb = bm.gather(l, 0, 80)
        ks, vs = tm.gather(l, 0, 80)
        assert np.array_equal(kb, ks) and np.array_equal(vb, vs)


def test_two_cache_identical_draft_accepts_every_draft(oracle):
    """A draft model identical to the target (own cache, same prompt)
    proposes the target's tokens: every round accepts all k, the catch-up
    writes the last draft, and the draft cache then holds the target's bytes
    at every position below the common seq_len."""
    from loop_model import make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    (toks, acc, rounds), tm, dm, _ = two_run(oracle, m, m, 4, 30, 3)
    assert acc == [4] * rounds and dm.seq_len == tm.seq_len
    for l in range(m.n_layers):
        kt, vt = tm.gather(l, 0, tm.seq_len)
        kd, vd = dm.gather(l, 0, dm.seq_len)
        assert np.array_equal(kt, kd) and np.array_equal(vt, vd)


def test_two_cache_rejected_drafts_catch_up_with_the_bonus(oracle):
    """A draft with a zero head proposes token 0 every time; the target never
    emits 0 on this prompt, so every round accepts nothing, and the catch-up
    writes the round's bonus at draft_save + 0 -- where the round's anchor
    was (the reference's rule, kernels.cu:3081-3090): after R rounds the draft
    cache holds bonus_0 .. bonus_{R-1} at positions P0 .. P0+R-1."""
    from loop_model import LoopModelNp, make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    zero = LoopModelNp(m.emb_q[:1], m.emb_k[:1], m.emb_v[:1], np.zeros_like(m.head), m.nh,
                       m.nkv, m.dph)
    (toks, acc, rounds), tm, dm, _ = two_run(oracle, m, zero, 2, 16, 3)
    assert 0 not in toks and acc == [0] * rounds and rounds == 16
    assert dm.seq_len == 40 + rounds and tm.seq_len == 40 + rounds
    k16, v16 = dm.gather(0, 40, rounds)
    bon = np.array(toks)  # one token per round: the bonus
    assert np.array_equal(k16, zero.emb_k[0][bon].astype(np.float16).astype(np.float32))
    assert np.array_equal(v16, zero.emb_v[0][bon].astype(np.float16).astype(np.float32))


def test_two_cache_planted_draft_rewind_mistake_changes_the_draft_cache(oracle):
    from loop_model import make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    d = _drafts(m, "prefix")
    (toks, acc, _), tm, dm, _ = two_run(oracle, m, d, 4, 30, 3)
    (toks2, acc2, _), tm2, dm2, _ = two_run(oracle, m, d, 4, 30, 3, shift=1)
    assert toks2[:30] == toks[:30]                       # the output cannot tell
    assert dm2.pool_sha256() != dm.pool_sha256() or dm2.seq_len != dm.seq_len


@pytest.mark.parametrize("two", [False, True])
def test_loops_stop_on_the_eos_bonus(oracle, two):
    """eos_token ends the loop after the round whose bonus it is
    (kernels.cu:3095); an accepted draft equal to it does not."""
    from loop_model import make_loop_model
    m = make_loop_model(3, noise=0.1, q_scale=2.0)
    if two:
        (toks, acc, rounds), _, _, _ = two_run(oracle, m, _drafts(m, "prefix"), 4, 40, 3)
    else:
        toks, acc, _ = loop_run(oracle, m, 4, 2, 40, 3)[:3]
    ends = np.cumsum([a + 1 for a in acc])
    r = 3
    eos = toks[ends[r] - 1]                              # round r's bonus
    first = next(i for i in range(len(acc)) if toks[ends[i] - 1] == eos)
    if two:
        (t2, a2, r2), _, _, _ = two_run(oracle, m, _drafts(m, "prefix"), 4, 40, 3, eos=eos)
    else:
        from loop_model import prefill, prompt_tokens
        nblk = -(-(40 + 80 + 5) // 16)
        model = oracle.PagedKVModel(m.n_layers, m.nkv * m.dph, nblk, 16, m.n_layers * nblk)
        prefill(model, m, prompt_tokens(3, 40, m.vocab))
        anchor = int(np.random.default_rng(3).integers(0, m.vocab))
        t2, a2, r2 = oracle.spec_loop_greedy(model, m.emb_q, m.emb_k, m.emb_v, m.head, m.nh,
                                             m.nkv, m.dph, anchor, 4, 2, 40, eos_token=eos)
    assert r2 == first + 1 and t2 == toks[:ends[first]] and t2[-1] == eos
