"""Tiny LLaMA-shaped model and speculative-decoding loops (TEST INFRASTRUCTURE).

The reference's one behavioural invariant for its paged KV cache is that
greedy speculative decoding emits exactly the target model's greedy tokens
(main.cu:311-337, binding.cu:104-108, cli/benchmark.py:73-80).  It holds only
if every verify window appends at the right positions, the rejected drafts are
rewound by an O(1) seq_len assignment, and the next round's appends overwrite
the stale entries behind seq_len -- i.e. the whole append / attention /
rollback path in its real control flow.

The model here is plumbing for that check: embedding, RMSNorm, q/k/v/o
projections, rotate-half RoPE (model.cu:281-323), SwiGLU MLP and an output
head, in float64 torch on whatever device the cache lives on.  Only append,
attention and rollback go through the cache object, which is either
`DeviceCache` (libsde_paged.so through the Python binding) or `OracleCache`
(the CPU oracle's byte-level paged pool and its fp64 brute-force attention).

Loops (reference host loop kernels.cu:2314-2475):
  * `greedy`: prefill the prompt as one causal window, then one token per
    step (model.cu:391-432: query at seq_pos sees seq_pos+1 keys).
  * `spec_two_model`: a draft model with its own cache proposes k tokens one
    at a time; the target verifies the window [last, d1..dk] at positions
    S..S+k in one causal call (model.cu:657-714); n_acc = leading matches;
    target seq_len <- S+n_acc+1 (kernels.cu:2457-2459).  The draft cache
    keeps the n_acc+1 accepted tokens it holds (S+n_acc+1), or, when all k
    were accepted, appends d_k, which it never wrote (kernels.cu:2466-2476).
  * `spec_self`: one shared cache; the first n_draft layers plus the output
    head draft k tokens (writing those layers' K/V and saving the hidden
    after layer n_draft-1, kernels.cu:1274-1305), then layers
    [n_draft, n_layers) verify the k+1 saved hiddens as one window
    (cublas_forward_from_hidden, kernels.cu:1308-1370) and seq_len rewinds
    to S+n_acc+1 for the whole cache.
The draft's cache bookkeeping affects only the acceptance rate; the emitted
tokens depend on the target cache alone.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class TinyConfig:
    n_layers: int = 4
    d_model: int = 256
    n_heads: int = 4
    n_kv_heads: int = 2
    d_ff: int = 512
    vocab: int = 512
    theta: float = 10000.0
    eps: float = 1e-5

    @property
    def dph(self) -> int:
        return self.d_model // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.dph


class TinyLlama:
    """Random-init weights (float64).  `base` + `noise` makes a draft model
    that agrees with `base` on part of its greedy choices."""

    def __init__(self, cfg: TinyConfig, seed: int, device="cpu", base: "TinyLlama | None" = None,
                 noise: float = 0.0, n_layers: int | None = None):
        self.cfg = cfg
        self.n_layers = n_layers or cfg.n_layers
        g = torch.Generator().manual_seed(seed)
        d, kv, ff, V = cfg.d_model, cfg.kv_dim, cfg.d_ff, cfg.vocab

        def rnd(*shape, scale):
            return torch.randn(*shape, generator=g, dtype=torch.float64) * scale

        w = {"emb": rnd(V, d, scale=1.0), "head": rnd(d, V, scale=2.0 / math.sqrt(d)),
             "norm_f": 1.0 + rnd(d, scale=0.1)}
        for l in range(self.n_layers):
            w[f"wq{l}"] = rnd(d, d, scale=1.0 / math.sqrt(d))
            w[f"wk{l}"] = rnd(d, kv, scale=1.0 / math.sqrt(d))
            w[f"wv{l}"] = rnd(d, kv, scale=1.0 / math.sqrt(d))
            w[f"wo{l}"] = rnd(d, d, scale=1.0 / math.sqrt(d))
            w[f"w1{l}"] = rnd(d, ff, scale=1.0 / math.sqrt(d))
            w[f"w3{l}"] = rnd(d, ff, scale=1.0 / math.sqrt(d))
            w[f"w2{l}"] = rnd(ff, d, scale=1.0 / math.sqrt(ff))
            w[f"n1{l}"] = 1.0 + rnd(d, scale=0.1)
            w[f"n2{l}"] = 1.0 + rnd(d, scale=0.1)
        if base is not None:
            for name in w:
                b = base.w[name].cpu()
                w[name] = b + noise * w[name] * (b.std() / w[name].std())
        self.w = {name: t.to(device) for name, t in w.items()}
        self.device = torch.device(device)
        # rotate-half RoPE tables (model.cu:281-323, no position scaling)
        j = torch.arange(cfg.dph // 2, dtype=torch.float64)
        self.inv_freq = torch.exp(-math.log(cfg.theta) * 2.0 * j / cfg.dph).to(device)

    def embed(self, tokens) -> torch.Tensor:
        t = torch.as_tensor(tokens, dtype=torch.long, device=self.device).reshape(-1)
        return self.w["emb"][t]

    def _rms(self, x, weight):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + self.cfg.eps) * weight

    def _rope(self, x, n_heads, pos_base):
        M = x.shape[0]
        dph = self.cfg.dph
        pos = torch.arange(pos_base, pos_base + M, dtype=torch.float64, device=self.device)
        ang = pos[:, None] * self.inv_freq[None, :]
        c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
        x = x.reshape(M, n_heads, dph)
        x0, x1 = x[..., : dph // 2], x[..., dph // 2:]
        return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1).reshape(M, n_heads * dph)

    def layers(self, x: torch.Tensor, cache, pos_base: int, lo: int, hi: int) -> torch.Tensor:
        """Layers [lo, hi) on hidden rows x [M][d] at positions pos_base..:
        append the window's K/V, then causal attention (query m sees
        pos_base+m+1 keys)."""
        cfg, w = self.cfg, self.w
        for l in range(lo, hi):
            h = self._rms(x, w[f"n1{l}"])
            q = self._rope(h @ w[f"wq{l}"], cfg.n_heads, pos_base)
            k = self._rope(h @ w[f"wk{l}"], cfg.n_kv_heads, pos_base)
            v = h @ w[f"wv{l}"]
            cache.append(l, k, v, pos_base)
            att = cache.attention(l, q, pos_base)
            x = x + att @ w[f"wo{l}"]
            h = self._rms(x, w[f"n2{l}"])
            x = x + (torch.nn.functional.silu(h @ w[f"w1{l}"]) * (h @ w[f"w3{l}"])) @ w[f"w2{l}"]
        return x

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        return self._rms(x, self.w["norm_f"]) @ self.w["head"]


class OracleCache:
    """The CPU oracle's paged pool (bytes + tables + seq_len) with fp64
    brute-force attention read through the block tables."""

    def __init__(self, oracle, cfg: TinyConfig, n_layers: int, n_positions: int, seed: int,
                 block_size: int = 16):
        self.cfg = cfg
        nblk = -(-n_positions // block_size)
        pool_blocks = n_layers * nblk + 5
        self.m = oracle.PagedKVModel(n_layers, cfg.kv_dim, nblk, block_size, pool_blocks)
        perm = np.random.default_rng(seed).permutation(pool_blocks).astype(np.int32)
        for l in range(n_layers):
            self.m.set_block_table(l, perm[l * nblk:(l + 1) * nblk])

    def append(self, layer, k, v, pos_base):
        self.m.append(layer, k.float().cpu().numpy(), v.float().cpu().numpy(), pos_base)

    def attention(self, layer, q, pos_base):
        c = self.cfg
        out = self.m.attention(layer, q.float().cpu().numpy(), c.n_heads, c.n_kv_heads, c.dph,
                               pos_base, mode="f64")
        return torch.from_numpy(out)

    @property
    def seq_len(self):
        return self.m.seq_len

    def set_seq_len(self, n):
        self.m.set_seq_len(n)

    def rollback(self, n):
        self.m.rollback(n)

    def gather(self, layer, pos, n):
        return self.m.gather(layer, pos, n)


class DeviceCache:
    """libsde_paged.so's cache through the Python binding of the C-ABI, with
    the same seeded fragmented block tables as OracleCache."""

    def __init__(self, cfg: TinyConfig, n_layers: int, n_positions: int, seed: int,
                 block_size: int = 16):
        from speculative_decode_engine_amd import KVCache
        self.cfg = cfg
        nblk = -(-n_positions // block_size)
        pool_blocks = n_layers * nblk + 5
        self.c = KVCache(n_layers, cfg.kv_dim, nblk, block_size, pool_blocks)
        perm = np.random.default_rng(seed).permutation(pool_blocks).astype(np.int32)
        for l in range(n_layers):
            self.c.set_block_table(l, perm[l * nblk:(l + 1) * nblk])

    def append(self, layer, k, v, pos_base):
        self.c.append(layer, k.float().contiguous(), v.float().contiguous(), pos_base)

    def attention(self, layer, q, pos_base):
        c = self.cfg
        return self.c.attention(layer, q.float().contiguous(), c.n_heads, c.n_kv_heads, c.dph,
                                pos_base).double()

    @property
    def seq_len(self):
        return self.c.seq_len

    def set_seq_len(self, n):
        self.c.set_seq_len(n)

    def rollback(self, n):
        self.c.rollback(n)

    def gather(self, layer, pos, n):
        k, v = self.c.read(layer, pos, n)
        torch.cuda.synchronize()
        return k.cpu().numpy(), v.cpu().numpy()

    def free(self):
        self.c.free()


def _argmax(logits: torch.Tensor) -> list[int]:
    return [int(t) for t in torch.argmax(logits, dim=-1).reshape(-1).cpu()]


def prefill(model: TinyLlama, cache, prompt) -> int:
    x = model.layers(model.embed(prompt), cache, 0, 0, model.n_layers)
    cache.set_seq_len(len(prompt))
    return _argmax(model.logits(x[-1:]))[0]


def greedy(model: TinyLlama, cache, prompt, n_new: int, margins: list | None = None) -> list[int]:
    tok = prefill(model, cache, prompt)
    out, pos = [tok], len(prompt)
    while len(out) < n_new:
        x = model.layers(model.embed([tok]), cache, pos, 0, model.n_layers)
        pos += 1
        cache.set_seq_len(pos)
        lg = model.logits(x)
        if margins is not None:
            top = torch.topk(lg.reshape(-1), 2).values
            margins.append(float(top[0] - top[1]))
        tok = _argmax(lg)[0]
        out.append(tok)
    return out


def _n_accepted(drafts, targets) -> int:
    n = 0
    for d, t in zip(drafts, targets):
        if d != t:
            break
        n += 1
    return n


def spec_two_model(target: TinyLlama, draft: TinyLlama, tcache, dcache, prompt, n_new: int,
                   k: int, stats: dict | None = None) -> list[int]:
    last = prefill(target, tcache, prompt)
    prefill(draft, dcache, prompt)
    out = [last]
    while len(out) < n_new:
        # positions come from the caches' seq_len: a wrong rewind shifts them
        S = tcache.seq_len
        assert dcache.seq_len == S
        cur_k = min(k, n_new - len(out))
        drafts, cur = [], last
        for i in range(cur_k):
            x = draft.layers(draft.embed([cur]), dcache, S + i, 0, draft.n_layers)
            dcache.set_seq_len(S + i + 1)
            cur = _argmax(draft.logits(x))[0]
            drafts.append(cur)
        x = target.layers(target.embed([last] + drafts), tcache, S, 0, target.n_layers)
        tcache.set_seq_len(S + cur_k + 1)
        tt = _argmax(target.logits(x))
        n_acc = _n_accepted(drafts, tt)
        out += drafts[:n_acc] + [tt[n_acc]]
        tcache.rollback(S + n_acc + 1)
        if n_acc == cur_k:
            draft.layers(draft.embed([drafts[-1]]), dcache, S + cur_k, 0, draft.n_layers)
            dcache.set_seq_len(S + cur_k + 1)
        else:
            dcache.rollback(S + n_acc + 1)
        if stats is not None:
            stats.setdefault("accepted", []).append(n_acc)
        last = tt[n_acc]
    return out[:n_new]


def spec_self(model: TinyLlama, cache, prompt, n_new: int, k: int, n_draft: int,
              stats: dict | None = None) -> list[int]:
    last = prefill(model, cache, prompt)
    out = [last]
    while len(out) < n_new:
        S = cache.seq_len
        cur_k = min(k, n_new - len(out))
        hid, drafts, cur = [], [], last
        for i in range(cur_k + 1):
            h = model.layers(model.embed([cur]), cache, S + i, 0, n_draft)
            hid.append(h)
            if i < cur_k:
                cur = _argmax(model.logits(h))[0]
                drafts.append(cur)
        x = model.layers(torch.cat(hid), cache, S, n_draft, model.n_layers)
        cache.set_seq_len(S + cur_k + 1)
        tt = _argmax(model.logits(x))
        n_acc = _n_accepted(drafts, tt)
        out += drafts[:n_acc] + [tt[n_acc]]
        cache.rollback(S + n_acc + 1)
        if stats is not None:
            stats.setdefault("accepted", []).append(n_acc)
        last = tt[n_acc]
    return out[:n_new]


def spec_two_model_reference(target: TinyLlama, draft: TinyLlama, tcache, dcache, prompt,
                             n_new: int, k: int, accept, stats: dict | None = None) -> list[int]:
    """The reference's multi-kernel host loop (kernels.cu:2314-2475) step for
    step: host-side seq positions, the draft rewound to draft_save + n_acc
    (and, when every draft was accepted, one extra draft forward of d_k,
    kernels.cu:2466-2476), the target to target_save + n_acc + 1.  `accept`
    does the acceptance and both rewinds: accept(draft_tokens, target_tokens,
    k, target_save, draft_save) -> (n_acc, bonus, target_seq, draft_seq,
    emitted), either the oracle's rule plus host rewinds or the device
    entry point."""
    last = prefill(target, tcache, prompt)
    prefill(draft, dcache, prompt)
    out = [last]
    target_seq = draft_seq = len(prompt)
    while len(out) < n_new:
        cur_k = min(k, n_new - len(out))
        target_save, draft_save = target_seq, draft_seq
        drafts, cur = [], last
        for _ in range(cur_k):
            x = draft.layers(draft.embed([cur]), dcache, draft_seq, 0, draft.n_layers)
            draft_seq += 1
            dcache.set_seq_len(draft_seq)
            cur = _argmax(draft.logits(x))[0]
            drafts.append(cur)
        x = target.layers(target.embed([last] + drafts), tcache, target_seq, 0, target.n_layers)
        target_seq += cur_k + 1
        tcache.set_seq_len(target_seq)
        tt = torch.argmax(target.logits(x), dim=-1)
        n_acc, bonus, target_seq, draft_seq, emitted = accept(drafts, tt, cur_k, target_save,
                                                              draft_save)
        out += emitted
        if n_acc == cur_k:
            draft.layers(draft.embed([drafts[-1]]), dcache, draft_seq, 0, draft.n_layers)
            draft_seq += 1
            dcache.set_seq_len(draft_seq)
        if stats is not None:
            stats.setdefault("accepted", []).append(n_acc)
        last = bonus
    return out[:n_new]


def host_accept(oracle, tcache, dcache):
    """The oracle's greedy rule with the rewinds done from the host."""
    def accept(drafts, tt, k, target_save, draft_save):
        r = oracle.spec_accept_greedy(drafts, [int(t) for t in tt.reshape(-1).cpu()], k,
                                      target_save, draft_save, shared=False)
        tcache.rollback(r[2])
        dcache.rollback(r[3])
        return r
    return accept
