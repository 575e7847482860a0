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
