"""The persistent loop's model for the tests (TEST INFRASTRUCTURE).

sde_spec_loop_greedy's model (include/sde_paged_kv.h): per-layer embedding
tables for q, k, v and an fp16 head.  Layers share base tables plus a
per-layer perturbation, so the first layers' outputs predict the last
layer's often but not always: the self-speculative loop then accepts some
drafts and rejects others, and both paths of the rewind run.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class LoopModelNp:
    emb_q: np.ndarray   # fp32 [L][V][nh*dph]
    emb_k: np.ndarray   # fp32 [L][V][kv_dim]
    emb_v: np.ndarray   # fp32 [L][V][kv_dim]
    head: np.ndarray    # uint16 fp16 bits [nh*dph][V]
    nh: int
    nkv: int
    dph: int

    @property
    def n_layers(self) -> int:
        return self.emb_q.shape[0]

    @property
    def vocab(self) -> int:
        return self.emb_q.shape[1]


def make_loop_model(seed: int, n_layers=4, nh=4, nkv=2, dph=64, vocab=256,
                    noise=0.3, q_scale=0.5, head_scale=1.0) -> LoopModelNp:
    rng = np.random.default_rng(seed)
    d, kvd = nh * dph, nkv * dph

    def tables(width, scale):
        base = rng.standard_normal((vocab, width)).astype(np.float32) * np.float32(scale)
        per = rng.standard_normal((n_layers, vocab, width)).astype(np.float32)
        return (base[None] + np.float32(noise * scale) * per).astype(np.float32)

    head = (rng.standard_normal((d, vocab)) * head_scale / np.sqrt(d)).astype(np.float16)
    return LoopModelNp(tables(d, q_scale), tables(kvd, 1.0), tables(kvd, 1.0),
                       head.view(np.uint16), nh, nkv, dph)


def prompt_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    return np.random.default_rng(seed + 7).integers(0, vocab, size=n)


def prefill(cache, m: LoopModelNp, prompt) -> None:
    """Context K/V of `prompt` at positions 0.. in every layer (the loop's
    K/V depend on (token, position) alone) and seq_len = len(prompt); `cache`
    is an oracle PagedKVModel or a DeviceKV wrapper with the same append."""
    toks = np.asarray(prompt)
    for l in range(m.n_layers):
        cache.append(l, m.emb_k[l][toks], m.emb_v[l][toks], 0)
    cache.set_seq_len(len(toks))
