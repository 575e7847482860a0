"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The reference ships no golden vectors, known-answer tests or fixtures for
this path (its only pin is "greedy speculative == greedy baseline" at run
time, main.cu:311-337), so these fixtures come from this repository's
oracle (oracle/sde_oracle.c), itself pinned by tests/test_oracle.py.

  tiny_decode.npz        config "tiny": 4 layers, seeded fragmented tables
                         over 64 blocks, 128 fp16 context tokens, one fp32
                         append at 128, RoPE-applied q; expected outputs
                         (fp64 brute force and the fp32 tile restatement).
  scripted_hashes.json   SHA-256 of the whole pool after every checkpoint of
                         seeded append / seq_len / rollback / re-append
                         scripts for configs tiny, llama3_8b_verify (2 layers)
                         and qwen25_7b_selfspec (4 layers, 2 draft layers).

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import paged_kv as O  # noqa: E402
from speculative_decode_engine_amd import workloads as W  # noqa: E402

# (config, layers, draft layers, rounds)
SCRIPTS = [
    ("tiny", 4, None, 2),
    ("llama3_8b_verify", 2, None, 2),
    ("qwen25_7b_selfspec", 4, 2, 2),
]


def tiny_decode_case():
    """Inputs and expected outputs of one config-"tiny" decode step."""
    w = W.CONFIGS["tiny"]
    rng = np.random.default_rng(w.seed)
    nblk = w.blocks_per_layer()  # 129 tokens -> 9 blocks
    tables = W.make_tables(rng, w.n_layers, nblk, w.pool_blocks)
    model = O.PagedKVModel(w.n_layers, w.kv_dim, nblk, w.block_size, w.pool_blocks)
    ctx_k = np.empty((w.n_layers, w.ctx, w.kv_dim), np.float16)
    ctx_v = np.empty_like(ctx_k)
    new_k = np.empty((w.n_layers, 1, w.kv_dim), np.float32)
    new_v = np.empty_like(new_k)
    q = np.empty((w.n_layers, 1, w.nh * w.dph), np.float32)
    for layer in range(w.n_layers):
        model.set_block_table(layer, tables[layer])
        ctx_k[layer], ctx_v[layer] = W.context_kv(rng, w.ctx, w.kv_dim)
        new_k[layer], new_v[layer] = W.new_kv(rng, 1, w.kv_dim)
        q[layer] = W.rope_rotate_half(W.queries(rng, 1, w.nh, w.dph), w.nh, w.dph, w.ctx)
    out_f64 = np.empty((w.n_layers, 1, w.nh * w.dph), np.float64)
    out_tiled = np.empty((w.n_layers, 1, w.nh * w.dph), np.float32)
    for layer in range(w.n_layers):
        model.write_fp16(layer, ctx_k[layer], ctx_v[layer], 0)
        model.append(layer, new_k[layer], new_v[layer], w.ctx)
        out_f64[layer] = model.attention(layer, q[layer], w.nh, w.nkv, w.dph, w.ctx, mode="f64")
        out_tiled[layer] = model.attention(layer, q[layer], w.nh, w.nkv, w.dph, w.ctx,
                                           mode="tiled")
    return dict(tables=tables, ctx_k=ctx_k.view(np.uint16), ctx_v=ctx_v.view(np.uint16),
                new_k=new_k, new_v=new_v, q=q, out_f64=out_f64, out_tiled=out_tiled,
                pool_sha256=np.frombuffer(bytes.fromhex(model.pool_sha256()), np.uint8))


def scripted_hashes():
    out = {}
    for name, layers, draft, rounds in SCRIPTS:
        w = W.CONFIGS[name]
        tables, ops = W.scripted_rounds(w, layers, rounds, draft_layers=draft)
        pool_blocks = W.scripted_pool_blocks(w, layers, rounds)
        model = O.PagedKVModel(layers, w.kv_dim, tables.shape[1], w.block_size, pool_blocks)
        for layer in range(layers):
            model.set_block_table(layer, tables[layer])
        marks = O.run_script(model, ops)
        out[name] = dict(n_layers=layers, draft_layers=draft, rounds=rounds,
                         pool_blocks=pool_blocks,
                         checkpoints=[dict(label=l, seq_len=s, sha256=h) for l, s, h in marks])
    return out


def main():
    O.build()
    np.savez_compressed(HERE / "tiny_decode.npz", **tiny_decode_case())
    (HERE / "scripted_hashes.json").write_text(json.dumps(scripted_hashes(), indent=1) + "\n")
    print("wrote", HERE / "tiny_decode.npz", HERE / "scripted_hashes.json")


if __name__ == "__main__":
    main()
