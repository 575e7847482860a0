"""The five BASELINE workloads and their seeded synthetic inputs.

Shapes follow the five `configs` of BASELINE.json.  Every input comes from
numpy's PCG64 `default_rng(seed)` so the GPU path and the CPU oracle see the
same bytes:
  * pre-filled context K/V: fp16 values float16(N(0,1));
  * appended k/v and queries q: fp32 N(0,1);
  * block tables: `perm = rng.permutation(pool_blocks)` assigned layer-major,
    table[l][j] = perm[l*n_blocks + j] (the fragmented pools of the configs);
  * rollback counts: rng.integers(0, k+1).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    n_layers: int
    nh: int
    nkv: int
    dph: int
    block_size: int
    ctx: int          # pre-filled context tokens
    pool_blocks: int  # physical blocks in the shared pool
    n_queries: int    # 1 = decode step, k+1 = verify window
    seed: int
    draft_layers: int = 0  # self-speculative: layers the draft runs
    rope_theta: float = 10000.0  # the model family's RoPE base (fused-path bench)
    note: str = ""

    @property
    def kv_dim(self) -> int:
        return self.nkv * self.dph

    @property
    def G(self) -> int:
        return self.nh // self.nkv

    @property
    def k(self) -> int:
        return self.n_queries - 1

    @property
    def l_max(self) -> int:
        """Keys visible to the last query of one layer-step."""
        return self.ctx + self.n_queries

    def blocks_per_layer(self, tokens: int | None = None) -> int:
        t = self.l_max if tokens is None else tokens
        return math.ceil(t / self.block_size)

    def algorithmic_bytes(self, l_max: int | None = None, n_app: int | None = None,
                          n_queries: int | None = None) -> int:
        """Bytes one layer-step must move (HBM lower bound):
        K+V fp16 once per visible position, appended fp16 writes, fp32 k/v
        inputs, fp32 q and out, int32 table entries."""
        L = self.l_max if l_max is None else l_max
        a = self.n_queries if n_app is None else n_app
        Q = self.n_queries if n_queries is None else n_queries
        return (4 * self.kv_dim * L + 4 * self.kv_dim * a + 8 * self.kv_dim * a
                + 8 * self.nh * self.dph * Q + 4 * math.ceil(L / self.block_size))

    def attention_flops(self, pos_base: int | None = None, n_queries: int | None = None) -> int:
        """Q.K and P.V multiply-adds (2 flops each) over the causal window."""
        Q = self.n_queries if n_queries is None else n_queries
        pb = self.ctx if pos_base is None else pos_base
        keys = sum(pb + m + 1 for m in range(Q))
        return 4 * self.dph * self.nh * keys


CONFIGS: dict[str, Workload] = {
    "tiny": Workload(
        "tiny", n_layers=4, nh=4, nkv=2, dph=64, block_size=16, ctx=128, pool_blocks=64,
        n_queries=1, seed=1,
        note="tiny dummy LLaMA: append 1 token, single-query attention with RoPE-applied q"),
    "tinyllama": Workload(
        "tinyllama", n_layers=22, nh=32, nkv=4, dph=64, block_size=16, ctx=2048,
        pool_blocks=4096, n_queries=1, seed=2,
        note="TinyLlama-1.1B-shaped decode: one append + one single-query attention"),
    "llama3_8b_verify": Workload(
        "llama3_8b_verify", n_layers=32, nh=32, nkv=8, dph=128, block_size=16, ctx=4096,
        pool_blocks=32 * 257, n_queries=5, seed=3, rope_theta=500000.0,
        note="Llama-3-8B-shaped verify: append k+1=5, causal attention, rollback, re-append"),
    "llama3_8b_32k": Workload(
        "llama3_8b_32k", n_layers=32, nh=32, nkv=8, dph=128, block_size=16, ctx=32767,
        pool_blocks=131072, n_queries=1, seed=4, rope_theta=500000.0,
        note="Llama-3-8B-shaped 32K decode: attention over 32768 keys in a fragmented "
             "131072-block pool"),
    "qwen25_7b_selfspec": Workload(
        "qwen25_7b_selfspec", n_layers=28, nh=28, nkv=4, dph=128, block_size=32, ctx=8192,
        pool_blocks=28 * 257, n_queries=9, seed=5, draft_layers=8, rope_theta=1000000.0,
        note="Qwen2.5-7B-shaped self-spec: 8 draft layers x 8 decode steps, then 9-query "
             "full-depth verify with partial rollback"),
}


def make_tables(rng: np.random.Generator, n_layers: int, n_blocks: int,
                pool_blocks: int) -> np.ndarray:
    """Seeded fragmented block tables, int32 [n_layers][n_blocks]."""
    if n_layers * n_blocks > pool_blocks:
        raise ValueError("pool too small for the requested tables")
    perm = rng.permutation(pool_blocks).astype(np.int32)
    return perm[: n_layers * n_blocks].reshape(n_layers, n_blocks).copy()


def context_kv(rng: np.random.Generator, n_tokens: int, kv_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """Pre-filled context rows, fp16 [n_tokens][kv_dim] each for K and V."""
    k = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32).astype(np.float16)
    return k, v


def new_kv(rng: np.random.Generator, n_tokens: int, kv_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """Rows to append, fp32 [n_tokens][kv_dim] each for K and V."""
    k = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32)
    v = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32)
    return k, v


def queries(rng: np.random.Generator, n_queries: int, nh: int, dph: int) -> np.ndarray:
    """fp32 [n_queries][nh*dph]."""
    return rng.standard_normal((n_queries, nh * dph), dtype=np.float32)


def scripted_pool_blocks(w: Workload, n_layers: int, rounds: int = 2) -> int:
    """Pool size of a scripted run: the workload's pool at full depth; with
    fewer layers, twice the blocks those layers map (still fragmented, but
    small enough to hash on the CPU)."""
    nblk = w.blocks_per_layer(w.ctx + rounds * w.n_queries)
    if n_layers >= w.n_layers:
        return w.pool_blocks
    return min(w.pool_blocks, max(2 * n_layers * nblk, n_layers * nblk))


def scripted_rounds(w: Workload, n_layers: int | None = None, rounds: int = 2,
                    draft_layers: int | None = None,
                    seed_offset: int = 0) -> tuple[np.ndarray, list[tuple]]:
    """A seeded speculative-decoding script over a cache of `n_layers` layers
    with `w`'s per-layer shapes (pool: scripted_pool_blocks).  Returns
    (tables, ops).  Ops:
      ("write_fp16", layer, pos, k16, v16)   pre-filled context rows
      ("append", layer, pos, k32, v32)       kv_cache_append of fp32 rows
      ("set_seq_len", n)                     set_seq_len_kernel
      ("rollback", n)                        O(1) rewind
      ("checkpoint", label)                  compare cache state here
      ("attend", layer, pos_base, M)         an attention call of the step
    Greedy rounds follow kernels.cu:2362-2466: the k+1 verify tokens are
    appended at seq..seq+k (model.cu:657-684), seq_len += k+1, then rewound
    to save + n_acc + 1.  A self-speculative workload (draft_layers > 0)
    follows kernels.cu:661-720: k single-token draft steps plus the bonus
    prefix step on the draft layers, then the k+1-token verify on the others.
    """
    L = w.n_layers if n_layers is None else n_layers
    rng = np.random.default_rng(w.seed + seed_offset)
    k = w.k
    nblk = w.blocks_per_layer(w.ctx + rounds * (k + 1))
    tables = make_tables(rng, L, nblk, scripted_pool_blocks(w, L, rounds))
    ops: list[tuple] = []
    for layer in range(L):
        kc, vc = context_kv(rng, w.ctx, w.kv_dim)
        ops.append(("write_fp16", layer, 0, kc, vc))
    seq = w.ctx
    ops.append(("set_seq_len", seq))
    ops.append(("checkpoint", "prefill"))
    draft = w.draft_layers if draft_layers is None else draft_layers
    if draft >= L:
        raise ValueError("a self-speculative script needs layers beyond the draft layers")
    for rnd in range(rounds):
        save = seq
        if draft:
            for i in range(k + 1):  # k draft steps + bonus prefix step
                for layer in range(draft):
                    kk, vv = new_kv(rng, 1, w.kv_dim)
                    ops.append(("append", layer, save + i, kk, vv))
                    ops.append(("attend", layer, save + i, 1))
            ops.append(("checkpoint", f"round{rnd}-draft"))
            verify_layers = range(draft, L)
        else:
            verify_layers = range(L)
        for layer in verify_layers:
            kk, vv = new_kv(rng, k + 1, w.kv_dim)
            ops.append(("append", layer, save, kk, vv))
            ops.append(("attend", layer, save, k + 1))
        seq = save + k + 1
        ops.append(("set_seq_len", seq))
        ops.append(("checkpoint", f"round{rnd}-verify"))
        rejected = int(rng.integers(0, k + 1))
        n_acc = k - rejected
        seq = save + n_acc + 1
        ops.append(("rollback", seq))
        ops.append(("checkpoint", f"round{rnd}-rollback"))
    return tables, ops


def rope_rotate_half(x: np.ndarray, n_heads: int, dph: int, pos: int,
                     theta: float = 10000.0) -> np.ndarray:
    """Rotary embedding as rope_apply_inplace with no position scaling
    (model.cu:281-323): dim j pairs with j + dph/2, inv_freq =
    exp(-ln(theta) * 2j / dph), angle = pos * inv_freq; fp32 arithmetic.
    Input preparation only (config "tiny" applies it to q)."""
    x = np.asarray(x, dtype=np.float32).reshape(-1, n_heads, dph).copy()
    pairs = dph // 2
    j = np.arange(pairs, dtype=np.float32)
    inv_freq = np.exp(-np.float32(math.log(theta)) * (np.float32(2) * j) / np.float32(dph))
    angle = np.float32(pos) * inv_freq
    c = np.cos(angle).astype(np.float32)
    s = np.sin(angle).astype(np.float32)
    x0 = x[..., :pairs].copy()
    x1 = x[..., pairs:].copy()
    x[..., :pairs] = x0 * c - x1 * s
    x[..., pairs:] = x0 * s + x1 * c
    return x.reshape(-1, n_heads * dph)
