"""Greedy speculative decoding through libsde_paged.so emits the greedy tokens.

The end-to-end pin of the append / causal verify attention / O(1) rewind path
in its real control flow (main.cu:311-337, kernels.cu:2314-2475), with the
tiny random model of tests/tiny_llama.py computing everything but the cache
in float64 on the GPU.  For each draft mode:
  * greedy decoding on the library's cache == greedy decoding on the CPU
    oracle's cache (same tokens);
  * speculative decoding on the library's caches == that greedy output;
  * the target cache's final seq_len (host mirror and device word) is the
    emitted length, and its layer-0 K/V bytes for every kept position equal
    the greedy run's (layer 0 depends on tokens and positions only), deeper
    layers within fp16 rounding of them.
"""
import numpy as np
import pytest
import torch

from conftest import case_banner
from test_spec_decode import CFG, K, N_NEW, POSITIONS, PROMPT
from tiny_llama import (DeviceCache, OracleCache, TinyLlama, greedy, spec_self,
                        spec_two_model)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [1, 2])
@pytest.mark.parametrize("mode", ["perturbed", "identical", "self"])
def test_library_speculation_emits_greedy_tokens(gpu, oracle, seed, mode):
    case_banner("spec decode", mode, seed)
    target = TinyLlama(CFG, seed, device="cuda")
    gcache = DeviceCache(CFG, CFG.n_layers, POSITIONS, seed)
    margins = []
    ref = greedy(target, gcache, PROMPT, N_NEW, margins)
    cpu = greedy(TinyLlama(CFG, seed), OracleCache(oracle, CFG, CFG.n_layers, POSITIONS, seed),
                 PROMPT, N_NEW)
    assert ref == cpu

    stats = {}
    tc = DeviceCache(CFG, CFG.n_layers, POSITIONS, seed)
    caches = [tc]
    if mode == "self":
        out = spec_self(target, tc, PROMPT, N_NEW, K, n_draft=3, stats=stats)
    else:
        draft = target if mode == "identical" else TinyLlama(
            CFG, seed + 100, device="cuda", base=target, noise=0.05, n_layers=2)
        dc = DeviceCache(CFG, draft.n_layers, POSITIONS, seed + 1)
        caches.append(dc)
        out = spec_two_model(target, draft, tc, dc, PROMPT, N_NEW, K, stats=stats)
    assert out == ref, f"accepted per round {stats['accepted']}, min greedy margin {min(margins)}"

    final = len(PROMPT) + sum(a + 1 for a in stats["accepted"])
    assert tc.seq_len == final and tc.c.device_seq_len() == final
    kept = min(final, gcache.seq_len)
    k0, v0 = tc.gather(0, 0, kept)
    gk0, gv0 = gcache.gather(0, 0, kept)
    assert np.array_equal(k0, gk0) and np.array_equal(v0, gv0)
    for l in range(1, CFG.n_layers):
        k, v = tc.gather(l, 0, kept)
        gk, gv = gcache.gather(l, 0, kept)
        np.testing.assert_allclose(k, gk, rtol=2e-3, atol=2e-3)
        np.testing.assert_allclose(v, gv, rtol=2e-3, atol=2e-3)
    for c in caches + [gcache]:
        c.free()
