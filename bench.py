#!/usr/bin/env python3
"""Benchmark of the paged-KV decode/verify hot path on one MI355X.

Metric: paged decode-attention us/layer + HBM GB/s (% of
peak) at 4K/32K context, verify k=4.  The headline `value` is the achieved
algorithmic HBM throughput (GB/s) of a Llama-3-8B-shaped 32K-context decode
layer-step (attention of one query over 32768 keys, 32 q / 8 KV heads,
head_dim 128, block_size 16, fragmented 131072-block pool).  A step is one
such layer-step; steps rotate over 16 layers of 128 MiB of K/V each (2 GiB,
eight times the 256 MB Infinity Cache), every other config over >= 2 GiB
too when its steps reach that many layers.

Timing: the K timed steps are captured once into a HIP graph (rotating over
the layers) and replayed between two HIP events on the launch stream, so a
step costs its kernels plus the graph's inter-kernel gaps, without Python or
launch overhead; eager per-launch event durations are reported beside it.

Also reported: us per layer-step for all five BASELINE configs, each beside
the CPU oracle's time for the same layer-step (oracle/sde_oracle.c, OpenMP,
a bounded sample), the verify (k=4) / single-query step ratio at 4K, the cost
of an O(1) rollback, the grid-cooperative device function
(sde::device_flash_attention_gqa_grid, through its test kernel) at the 4K
verify and 32K shapes, the roofline of the dominant kernel against both the
8 TB/s peak and a device copy measured in the same process, and the
persistent speculative loop's time per round.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       [--calibrate-copy MiB]  (adds plain device copies of known size, the
       reference point for rocprofv3 FETCH_SIZE / WRITE_SIZE)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E spec sheet
ROTATE_BYTES = 2 << 30  # K/V bytes the timed steps rotate over (8x the Infinity Cache)
DTYPE = ("fp16 K/V; q and the softmax weights enter the MFMA as fp16 hi+lo pairs "
         "(fp32-level products), fp32 accumulate")
HEADLINE = "llama3_8b_32k"
# configs entries named differently from their workload
CONFIG_WORKLOAD = {"llama3_8b_4k_decode": "llama3_8b_verify",
                   "llama3_8b_4k_attn": "llama3_8b_verify",
                   "llama3_8b_verify_fused": "llama3_8b_verify",
                   "llama3_8b_4k_decode_fused": "llama3_8b_verify",
                   "tinyllama_decode_fused": "tinyllama",
                   "qwen25_7b_selfspec_verify": "qwen25_7b_selfspec",
                   "qwen25_7b_selfspec_draft": "qwen25_7b_selfspec",
                   "qwen25_7b_selfspec_verify_fused": "qwen25_7b_selfspec"}
KERNEL = "attn_mfma_kernel"  # the headline (1-query, GQA 4) path


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="approximate CPU work of the baseline sample")
    p.add_argument("--only-headline", action="store_true")
    p.add_argument("--only", default=None, metavar="CONFIG",
                   help="time one configs entry (e.g. llama3_8b_verify, "
                        "qwen25_7b_selfspec_verify_fused) and print its JSON (profiling)")
    p.add_argument("--only-shares", action="store_true",
                   help="time only the headline's per-GPU shares (KV-head and context "
                        "sharding) and print their JSON")
    p.add_argument("--only-matvec", action="store_true",
                   help="time only the output projection (sde_matvec) and print its JSON")
    p.add_argument("--matvec-shape", default=None,
                   help="with --only-matvec: one shape name (e.g. llama3_8b_wo) and no load timing")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MiB",
                   help="after the benchmark, copy a MiB-sized buffer 5 times")
    return p.parse_args()


class Timer:
    """Per-launch HIP events on the current stream + a bracket around all."""

    def __init__(self, torch, n):
        self.torch = torch
        self.ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(n)]
        self.t0 = torch.cuda.Event(enable_timing=True)
        self.t1 = torch.cuda.Event(enable_timing=True)

    def run(self, fn, steps, warmup, per_launch=True):
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        self.t0.record()
        for i in range(steps):
            if per_launch:
                self.ev[i][0].record()
            fn(i)
            if per_launch:
                self.ev[i][1].record()
        self.t1.record()
        torch.cuda.synchronize()
        total_ms = self.t0.elapsed_time(self.t1)
        launch_ms = [s.elapsed_time(e) for s, e in self.ev[:steps]] if per_launch else []
        return total_ms / steps, (float(np.mean(launch_ms)) if launch_ms else None)


def graph_step_ms(torch, step, steps, warmup):
    """ms per step of `steps` steps captured into one HIP graph and replayed
    (after `warmup` eager steps and one untimed replay) between two events
    on the capture/launch stream."""
    for i in range(max(warmup, 1)):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                step(i)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def make_rotation_cache(torch, W, w, n_layers, l_max, pool_blocks, seed):
    """A cache of n_layers layers of l_max tokens each, tables a seeded
    permutation of the pool, the whole pool filled with N(0,1) fp16."""
    from speculative_decode_engine_amd import KVCache
    nblk = -(-l_max // w.block_size)
    rng = np.random.default_rng(seed)
    tables = W.make_tables(rng, n_layers, nblk, pool_blocks)
    cache = KVCache(n_layers, w.kv_dim, nblk, w.block_size, pool_blocks)
    for l in range(n_layers):
        cache.set_block_table(l, tables[l])
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    cache.pool.view(torch.float16).normal_(generator=g)
    torch.cuda.synchronize()
    return cache


def bench_config(torch, W, w, steps, warmup, mode):
    """Times one layer-step of workload w.  mode: 'attn' (attention only),
    'decode' (append 1 + 1-query attention), 'verify' (append k+1 +
    (k+1)-query causal attention), and 'decode_fused' / 'verify_fused'
    (the same steps with RoPE of q and k, append and attention in one
    sde_rope_append_attention launch).  Returns a dict."""
    fused = mode.endswith("_fused")
    n_q = 1 if mode in ("attn", "decode", "decode_fused") else w.n_queries
    n_app = 0 if mode == "attn" else n_q
    pos_base = w.ctx if mode != "attn" else w.l_max - 1
    l_max = pos_base + n_q
    # rotate over distinct layers holding ROTATE_BYTES of K/V in all
    per_layer = 4 * w.kv_dim * l_max
    n_layers = max(1, min(4096, math.ceil(ROTATE_BYTES / per_layer)))
    nblk = -(-l_max // w.block_size)
    pool_blocks = max(w.pool_blocks, n_layers * nblk)
    cache = make_rotation_cache(torch, W, w, n_layers, l_max, pool_blocks, w.seed)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(w.seed + 100)
    q = torch.randn(n_layers, n_q, w.nh * w.dph, device="cuda", generator=gen)
    k = torch.randn(n_layers, max(n_app, 1), w.kv_dim, device="cuda", generator=gen)
    v = torch.randn(n_layers, max(n_app, 1), w.kv_dim, device="cuda", generator=gen)
    out = torch.empty(n_q, w.nh * w.dph, device="cuda")
    ws = torch.empty(max(cache.workspace_size(w.nh, w.nkv, w.dph, n_q, l_max), 4) // 4 + 1,
                     device="cuda")

    def step(i):
        l = i % n_layers
        if fused:
            cache.rope_append_attention(l, q[l], k[l], v[l], w.nh, w.nkv, w.dph, pos_base,
                                        theta=w.rope_theta, out=out, workspace=ws)
            return
        if n_app:
            cache.append(l, k[l], v[l], pos_base)
        cache.attention(l, q[l], w.nh, w.nkv, w.dph, pos_base, out=out, workspace=ws)

    # eager: per-launch HIP events (attention only) and the bracket
    timer = Timer(torch, steps)
    eager_ms, launch_ms = timer.run(step, steps, warmup, per_launch=(n_app == 0 or fused))
    # timed: the steps captured into one HIP graph, replayed between events
    ms = graph_step_ms(torch, step, steps, warmup)
    nbytes = w.algorithmic_bytes(l_max=l_max, n_app=n_app, n_queries=n_q)
    res = dict(mode=mode, n_queries=n_q, keys=l_max, rotated_layers=n_layers,
               us_per_layer_step=round(ms * 1e3, 3), algorithmic_bytes=nbytes,
               gbps=round(nbytes / (ms * 1e-3) / 1e9, 1),
               frac_of_hbm_peak=round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
               flops=w.attention_flops(pos_base, n_q),
               us_per_layer_step_eager=round(eager_ms * 1e3, 3))
    if launch_ms is not None:
        res["kernel_us_events"] = round(launch_ms * 1e3, 3)
    cache.free()
    return res


def bench_shares(torch, W, steps, warmup):
    """The headline layer-step as one GPU of N would run it (N = 2, 4, 8;
    the sharding is design only, every box here has one GPU): by KV head
    (nkv/N KV heads with their q heads over the whole 32K context, a pool
    of kv_dim/N, no exchange) and by context (all heads over 32768/N keys,
    whose partials one all-gather would combine).  Each share is timed like
    the headline (attention only, graph-replayed over a 2 GiB rotation);
    `frac_of_hbm_peak` is the share's own algorithmic bytes over its time."""
    import dataclasses
    w = W.CONFIGS[HEADLINE]
    out = {}
    for n in (2, 4, 8):
        heads = dataclasses.replace(w, name=f"{w.name}_heads_of_{n}", nh=w.nh // n,
                                    nkv=w.nkv // n)
        ctx = dataclasses.replace(w, name=f"{w.name}_context_of_{n}",
                                  ctx=w.l_max // n - 1,
                                  pool_blocks=max(w.pool_blocks // n, 1))
        r = {}
        for kind, sw in (("heads", heads), ("context", ctx)):
            res = bench_config(torch, W, sw, steps, warmup, "attn")
            r[kind] = dict(nh=sw.nh, nkv=sw.nkv, keys=res["keys"],
                           us=res["us_per_layer_step"], gbps=res["gbps"],
                           frac_of_hbm_peak=res["frac_of_hbm_peak"])
        out[f"n{n}"] = r
    return out


def bench_rollback(torch, W, steps=2000):
    """us per O(1) rollback (host bookkeeping + one stream-ordered 4-byte
    device write) at 4K and 32K context: must not depend on context."""
    from speculative_decode_engine_amd import KVCache
    out = {}
    for ctx in (4096, 32768):
        cache = KVCache(1, 1024, ctx // 16 + 1, 16, pool_blocks=ctx // 16 + 1, pool="library")
        cache.set_seq_len(ctx + 5)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for i in range(steps):
            cache.rollback(ctx + 1 + (i % 5) if i % 2 == 0 else ctx + 1)
            cache.set_seq_len(ctx + 5)
        torch.cuda.synchronize()
        out[f"ctx{ctx}"] = round((time.perf_counter() - t) / (2 * steps) * 1e6, 3)
        cache.free()
    return out


def bench_accept(torch, steps=200, k=4, vocab=128256):
    """us per on-device acceptance + rewind of a k=4 verify window: greedy
    (sde_spec_accept_greedy) and speculative sampling over a Llama-3-sized
    vocabulary (sde_spec_accept_stochastic), graph-replayed like the
    attention steps."""
    from speculative_decode_engine_amd import KVCache, spec_accept_greedy, spec_accept_stochastic
    tc = KVCache(1, 1024, 8, 16, 8, pool="library")
    dc = KVCache(1, 1024, 8, 16, 8, pool="library")
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    tl = torch.randn(k + 1, vocab, device="cuda", generator=g) * 4
    dl = tl[:k] + torch.randn(k, vocab, device="cuda", generator=g)
    dl = dl.contiguous()
    drafts = torch.argmax(dl, dim=-1).to(torch.int32)
    targets = torch.argmax(tl, dim=-1).to(torch.int32)
    off = torch.zeros(1, dtype=torch.int64, device="cuda")
    res = torch.empty(k + 5, dtype=torch.int32, device="cuda")
    out = {}
    for name, fn in (
            ("greedy", lambda i: spec_accept_greedy(tc, dc, drafts, targets, k, 64, 60, out=res)),
            ("stochastic", lambda i: spec_accept_stochastic(tc, dc, tl, dl, drafts, k, 64, 60, 5,
                                                            off, 1.0, 1.0, out=res))):
        out[name] = round(graph_step_ms(torch, fn, steps, 10) * 1e3, 3)
    out["k"] = k
    out["vocab"] = vocab
    tc.free()
    dc.free()
    return out


def bench_matvec(torch, steps, warmup, only=None):
    """The output projection after attention: us per call and algorithmic
    GB/s (fp16 weights once + fp32 x, out read when accumulating, out
    written) at the reference models' Wo / W_down shapes, for W in the
    reference's row-major layout (sde_matvec) and in the panel-packed layout
    (sde_matvec_packed, W packed once beforehand), each graph-replayed over
    >= 512 MiB of distinct weight matrices (beyond the 256 MB Infinity
    Cache); the C restatement of the reference's per-column loop
    (oracle_matvec, OpenMP on the host cores) timed beside the Llama-3-8B Wo."""
    from speculative_decode_engine_amd import PackedWeight, matvec, matvec_packed, matvec_workspace
    shapes = [("llama3_8b_wo", 1, 4096, 4096, 1), ("llama3_8b_wo_verify", 5, 4096, 4096, 0),
              ("llama3_8b_w_down", 1, 14336, 4096, 1), ("llama3_8b_w_down_verify", 5, 14336, 4096, 0),
              ("qwen25_7b_wo", 1, 3584, 3584, 1), ("qwen25_7b_wo_verify", 9, 3584, 3584, 0),
              ("tinyllama_wo", 1, 2048, 2048, 1)]
    out = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    for name, M, d_in, d_out, acc in shapes:
        if only and name != only:
            continue
        wbytes = d_in * d_out * 2
        n_mats = max(4, -(-(512 << 20) // wbytes))
        Ws = [(torch.randn(d_in, d_out, device="cuda", generator=g) * 0.02).half()
              for _ in range(n_mats)]
        x = torch.randn(M, d_in, device="cuda", generator=g)
        y = torch.zeros(M, d_out, device="cuda")
        ws = matvec_workspace(d_in, d_out, M, "cuda")
        us = graph_step_ms(torch, lambda i: matvec(x, Ws[i % n_mats], out=y, accumulate=bool(acc),
                                                    workspace=ws), steps, warmup) * 1e3
        nbytes = wbytes + M * d_in * 4 + M * d_out * 4 * (2 if acc else 1)
        gbps = nbytes / (us * 1e-6) / 1e9
        Ps = [PackedWeight(W) for W in Ws]
        del Ws
        pus = graph_step_ms(torch, lambda i: matvec_packed(x, Ps[i % n_mats], out=y,
                                                           accumulate=bool(acc)),
                            steps, warmup) * 1e3
        pgbps = nbytes / (pus * 1e-6) / 1e9
        out[name] = dict(n_rows=M, d_in=d_in, d_out=d_out, accumulate=acc, us=round(us, 3),
                         algorithmic_bytes=nbytes, gbps=round(gbps, 1),
                         frac_of_hbm_peak=round(gbps / HBM_PEAK_GBPS, 4),
                         packed_us=round(pus, 3), packed_gbps=round(pgbps, 1),
                         packed_frac_of_hbm_peak=round(pgbps / HBM_PEAK_GBPS, 4))
        del Ps
        torch.cuda.empty_cache()
    if only:
        return out
    try:
        from oracle import paged_kv as O
        O.lib()
        rng = np.random.default_rng(0)
        xs = rng.standard_normal((1, 4096)).astype(np.float32)
        Wb = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float16).view(np.uint16)
        o = np.zeros((1, 4096), np.float32)
        O.matvec_ref(xs, Wb, o, True)
        t = time.perf_counter()
        reps = 5
        for _ in range(reps):
            O.matvec_ref(xs, Wb, o, True)
        cpu_us = (time.perf_counter() - t) / reps * 1e6
        out["cpu_llama3_8b_wo"] = dict(us=round(cpu_us, 1), cores=int(O.lib().oracle_max_threads()),
                                       kind="port", sample="5 x the 4096x4096 Wo of one decode "
                                       "token, the reference's per-column fp32 loop in C")
    except Exception as e:  # the CPU leg is a reported baseline only
        out["cpu_llama3_8b_wo"] = dict(error=str(e))
    return out


def bench_sdec_load(torch, layers=2):
    """Seconds and GB/s of sde_model_load for a Llama-3-8B-shaped SDEC v5
    file of `layers` layers (d 4096, 8 KV heads, d_ff 14336, vocab 32000:
    ~0.83 GB per two layers + 0.52 GB of embeddings), written to a
    temporary file first, so the read comes from the page cache: the time
    is the staged host-to-device path, not the disk."""
    import shutil
    import tempfile
    from speculative_decode_engine_amd import sdec
    cfg = dict(n_layers=layers, d_model=4096, n_heads=32, n_kv_heads=8, d_ff=14336,
               vocab_size=32000, rope_theta=500000.0, has_qkv_bias=0)
    tmp = tempfile.mkdtemp(prefix="sde_sdec_")
    try:
        path = os.path.join(tmp, "llama_like.sdec")
        shapes = sdec.tensor_shapes(cfg)
        # Same bytes for every tensor (a repeated pattern): the loader's work
        # does not depend on the values.
        pattern = (np.arange(1 << 20, dtype=np.float32) % 97 * 1e-3).astype(np.float16)
        with open(path, "wb") as f:
            import struct
            f.write(b"SDEC" + struct.pack("<IIIIIIIfifii", 5, layers, 4096, 32, 8, 14336, 32000,
                                          500000.0, 0, 1.0, 0, 0))
            for name, shape in shapes.items():
                n = int(np.prod(shape))
                f.write(struct.pack("<I", n))
                for off in range(0, n, pattern.size):
                    f.write(pattern[:min(pattern.size, n - off)].tobytes())
        nbytes = os.path.getsize(path)
        times = []
        for _ in range(3):
            torch.cuda.synchronize()
            t = time.perf_counter()
            m = sdec.load_sdec(path)
            times.append(time.perf_counter() - t)
            m.free()
        best = min(times)
        return dict(file_bytes=nbytes, seconds=round(best, 4), gbps=round(nbytes / best / 1e9, 2),
                    layers=layers, source="page cache (file written just before)")
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def measure_lib():
    """libsde_measure.so: the streaming-read and load-skeleton kernels."""
    import ctypes
    from speculative_decode_engine_amd import _native
    _native.load()
    path = ROOT / "speculative_decode_engine_amd" / "libsde_measure.so"
    if not path.exists():
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.sde_measure_stream_read.argtypes = [vp, sz, ctypes.c_int, vp, vp]
    lib.sde_measure_stream_read.restype = ctypes.c_int
    ci = ctypes.c_int
    lib.sde_measure_attention_loads.argtypes = [vp, ci, ci, ci, ci, ci, ci, ci, vp, vp]
    lib.sde_measure_attention_loads.restype = ctypes.c_int
    return lib


def measured_hbm(torch, nbytes=2 << 30, reps=5):
    """Same-process reference points for the HBM roofline: a hand-written
    HIP streaming read of an nbytes buffer (sde_measure_stream_read:
    16-byte loads, eight in flight per thread; the best of `reps` runs at
    each of several grid sizes, read bytes over the time) and the best of
    `reps` device-to-device copies (torch copy_, read + write bytes), each
    between HIP events on the current stream."""
    import ctypes
    lib = measure_lib()
    src = torch.ones(nbytes // 4, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count

    def best(fn):
        fn()
        torch.cuda.synchronize()
        t = []
        for _ in range(reps):
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            t.append(e0.elapsed_time(e1) * 1e-3)
        return min(t)

    def read(blocks):
        rc = lib.sde_measure_stream_read(ctypes.c_void_p(src.data_ptr()), nbytes, blocks,
                                         ctypes.c_void_p(sink.data_ptr()),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"sde_measure_stream_read: {rc}")
    t_read = {b: best(lambda b=b: read(b)) for b in (n_cus * 2, n_cus * 4, n_cus * 8, n_cus * 16)}
    blocks = min(t_read, key=t_read.get)
    dst = torch.empty_like(src)
    t_copy = best(lambda: dst.copy_(src))
    del src, dst
    torch.cuda.empty_cache()
    return dict(read_gbps=round(nbytes / t_read[blocks] / 1e9, 1),
                copy_gbps=round(2 * nbytes / t_copy / 1e9, 1), bytes=nbytes,
                read_blocks=blocks,
                how="HIP streaming read (sde_measure_stream_read, 512-thread workgroups, best "
                    "grid of 2-16 per CU, best of 5) of a 2 GiB buffer, read bytes; torch "
                    "copy_ of it, read + write bytes")


def bench_pattern_floor(torch, W, w, steps, warmup):
    """The load skeleton of the headline's attention call
    (sde_measure_attention_loads: the kernel's plan, grid, workgroup
    mapping, per-wave tiles, table lookups and K/V loads in the same order,
    no arithmetic, staging, merge or combine), graph-replayed over the same
    2 GiB rotation as the kernel: the floor of the kernel's access pattern,
    measured in the same process."""
    import ctypes
    lib = measure_lib()
    pos_base = w.l_max - 1
    l_max = pos_base + 1
    per_layer = 4 * w.kv_dim * l_max
    n_layers = max(1, min(4096, math.ceil(ROTATE_BYTES / per_layer)))
    nblk = -(-l_max // w.block_size)
    cache = make_rotation_cache(torch, W, w, n_layers, l_max,
                                max(w.pool_blocks, n_layers * nblk), w.seed)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count

    def step(i):
        rc = lib.sde_measure_attention_loads(
            cache.handle, i % n_layers, w.nh, w.nkv, w.dph, pos_base, 1,
            n_cus, ctypes.c_void_p(sink.data_ptr()),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"sde_measure_attention_loads: {rc}")
    ms = graph_step_ms(torch, step, steps, warmup)
    cache.free()
    nbytes = w.algorithmic_bytes(l_max=l_max, n_app=0, n_queries=1)
    return dict(us=round(ms * 1e3, 3), gbps=round(nbytes / (ms * 1e-3) / 1e9, 1),
                rotated_layers=n_layers,
                how="load skeleton of the same call (sde_measure_attention_loads), "
                    "graph-replayed like the kernel")


def cpu_threads():
    """Host threads for the CPU baseline: the box's CPU share (its
    OMP_NUM_THREADS, else the process's CPU affinity), not every core the
    host reports."""
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    try:
        share = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        share = os.cpu_count() or 1
    return min(env, share) if env else share


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it (model name, family / model /
    stepping, logical CPUs the host reports)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                info.setdefault(k.strip(), v.strip())
    except OSError:
        return "unknown"
    return (f"{info.get('model name', 'unknown')} (vendor {info.get('vendor_id', '?')}, family "
            f"{info.get('cpu family', '?')} model {info.get('model', '?')} stepping "
            f"{info.get('stepping', '?')}; {os.cpu_count()} logical CPUs on the host)")


def cpu_step(W, w, mode, seconds, reps_min=5):
    """One layer-step of `mode` (bench_config's modes) at workload w's shape
    on the CPU, the torch-CPU restatement of the reference semantics that
    the baseline names (oracle.attention_torch_cpu: block-table index_select gather,
    fp32 q.K^T * dph^-1/2, causal mask, softmax, .V; the window's append as
    an fp32 -> fp16 scatter into the pool), torch on cpu_threads() threads.
    2 warm-ups, then at least reps_min repetitions and about `seconds`;
    the median per step.  Fused modes time the same steps (RoPE excluded)."""
    import torch
    from oracle import paged_kv as O
    threads = cpu_threads()
    torch.set_num_threads(threads)
    n_q = 1 if mode.startswith(("attn", "decode")) else w.n_queries
    n_app = 0 if mode == "attn" else n_q
    pos_base = w.ctx if mode != "attn" else w.l_max - 1
    l_max = pos_base + n_q
    rng = np.random.default_rng(w.seed)
    nblk = -(-l_max // w.block_size)
    pool_blocks = 2 * nblk
    pool = torch.from_numpy(rng.standard_normal((pool_blocks, 2, w.block_size, w.kv_dim),
                                                dtype=np.float32).astype(np.float16))
    table = torch.from_numpy(rng.permutation(pool_blocks)[:nblk].astype(np.int64))
    q = torch.from_numpy(W.queries(rng, n_q, w.nh, w.dph))
    k, v = (torch.from_numpy(x) for x in W.new_kv(rng, max(n_app, 1), w.kv_dim))
    pos = torch.arange(pos_base, pos_base + n_app)
    blk, slot = table[pos // w.block_size], pos % w.block_size

    def step():
        if n_app:  # kv_cache_append: fp32 -> fp16 (RNE) at (table[pos/BS], pos%BS)
            pool[blk, 0, slot] = k[:n_app].half()
            pool[blk, 1, slot] = v[:n_app].half()
        return O.attention_torch_cpu(pool, table, q, w.nh, w.nkv, w.dph, w.block_size, pos_base)

    for _ in range(2):
        step()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < reps_min or time.perf_counter() < t_end:
        t = time.perf_counter()
        step()
        times.append(time.perf_counter() - t)
    dt = float(np.median(times))
    nbytes = w.algorithmic_bytes(l_max=l_max, n_app=n_app, n_queries=n_q)
    return dict(us_per_layer_step=round(dt * 1e6, 1), gbps=round(nbytes / dt / 1e9, 3),
                reps=len(times), cores=threads, kind="port",
                how="torch-CPU gather + fp32 softmax attention (oracle.attention_torch_cpu)")


def cpu_config(W, w, mode, seconds):
    """cpu_step for a configs entry (a bounded sample)."""
    return cpu_step(W, w, mode, seconds)


def bench_grid_device_fn(torch, W, steps, warmup):
    """sde::device_flash_attention_gqa_grid as a persistent kernel would
    call it (every block of a one-block-per-CU grid of 512 threads; 8-wave
    staging), launched by the device-API test library's grid_attention
    kernel, at the 4K verify window (5 queries over 4101 keys) and the 32K
    decode (1 query over 32768 keys), graph-replayed over >= 2 GiB like the
    library's kernel."""
    import ctypes
    from speculative_decode_engine_amd import _native
    lib_path = ROOT / "tests" / "device" / "libsde_device_test.so"
    if not lib_path.exists():
        return dict(error=f"{lib_path} not built")
    lib = ctypes.CDLL(str(lib_path))
    fn = lib.sdet_grid_attention
    fn.restype = ctypes.c_int
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = {}
    for name, mode in (("llama3_8b_verify", "verify"), ("llama3_8b_32k", "attn")):
        w = W.CONFIGS[name]
        n_q = 1 if mode == "attn" else w.n_queries
        pos_base = w.ctx if mode != "attn" else w.l_max - 1
        l_max = pos_base + n_q
        per_layer = 4 * w.kv_dim * l_max
        n_layers = max(1, min(4096, math.ceil(ROTATE_BYTES / per_layer)))
        nblk = -(-l_max // w.block_size)
        cache = make_rotation_cache(torch, W, w, n_layers, l_max,
                                    max(w.pool_blocks, n_layers * nblk), w.seed)
        view = cache.view()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(w.seed + 200)
        q = torch.randn(n_layers, n_q, w.nh * w.dph, device="cuda", generator=gen)
        o = torch.empty(n_q, w.nh * w.dph, device="cuda")
        ws_bytes = int(_native.load().sde_grid_attention_workspace_size(w.nh, w.nkv, w.dph, n_q,
                                                                        l_max))
        ws = torch.zeros(ws_bytes // 4 + 1, dtype=torch.int32, device="cuda")
        status = torch.zeros(n_cus, dtype=torch.int32, device="cuda")

        def step(i):
            l = i % n_layers
            s = torch.cuda.current_stream().cuda_stream
            rc = fn(ctypes.byref(view), l, ctypes.c_void_p(q[l].data_ptr()),
                    ctypes.c_void_p(o.data_ptr()), w.nh, w.nkv, w.dph, pos_base, n_q, n_cus, 512,
                    8, ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws_bytes),
                    ctypes.c_void_p(status.data_ptr()), ctypes.c_void_p(s))
            if rc != 0:
                raise RuntimeError(f"sdet_grid_attention: {rc}")
        ms = graph_step_ms(torch, step, steps, warmup)
        torch.cuda.synchronize()
        st = int(status.abs().max().item())
        nbytes = w.algorithmic_bytes(l_max=l_max, n_app=0, n_queries=n_q)
        out[f"{name}_{mode}"] = dict(us=round(ms * 1e3, 3), queries=n_q, keys=l_max,
                                     gbps=round(nbytes / (ms * 1e-3) / 1e9, 1), blocks=n_cus,
                                     threads=512, status=st)
        cache.free()
    return out


def bench_spec_loop(torch, max_new=64):
    """The persistent speculative loops (sde_spec_loop_greedy and
    sde_spec_loop_stochastic, one cooperative launch each): us per round and
    per emitted token at a Llama-3-8B head shape (32 q / 8 KV heads, dph
    128), 4 layers, 4K context, vocabulary 4096, greedy (k = 0) and
    self-speculative (k = 4, one draft layer); the sampling loop at draft
    temperature 1 with adaptation."""
    from speculative_decode_engine_amd import KVCache
    from speculative_decode_engine_amd.spec_loop import (SpecLoopModel, spec_loop_greedy,
                                                         spec_loop_stochastic)
    L, nh, nkv, dph, V, P0 = 4, 32, 8, 128, 4096, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(31)
    base_q = torch.randn(V, nh * dph, device="cuda", generator=g) * 2.0
    base_k = torch.randn(V, nkv * dph, device="cuda", generator=g)
    base_v = torch.randn(V, nkv * dph, device="cuda", generator=g)
    mk = lambda b: (b[None] + 0.1 * b.abs().mean() * torch.randn(L, *b.shape, device="cuda",
                                                                   generator=g)).contiguous()
    model = SpecLoopModel(mk(base_q), mk(base_k), mk(base_v),
                          (torch.randn(nh * dph, V, device="cuda", generator=g) /
                           math.sqrt(nh * dph)).half(), nh, nkv, dph)
    # the same model cut to its first two layers (the per-layer cost below)
    model2 = SpecLoopModel(model.emb_q[:2].contiguous(), model.emb_k[:2].contiguous(),
                           model.emb_v[:2].contiguous(), model.head, nh, nkv, dph)
    out = {}

    def run(name, k, n_new, m=model):
        nl = m.n_layers
        nblk = -(-(P0 + n_new + k + 1) // 16)
        cache = KVCache(nl, nkv * dph, nblk, 16, nl * nblk)
        toks = torch.randint(0, V, (P0,), device="cuda", generator=g)
        for l in range(nl):
            cache.append(l, m.emb_k[l][toks].contiguous(), m.emb_v[l][toks].contiguous(), 0)
        cache.set_seq_len(P0)
        torch.cuda.synchronize()
        t = time.perf_counter()
        if name.startswith("sampling"):
            res = spec_loop_stochastic(cache, m, 7, k, 1 if k else 0, n_new, seed=5,
                                       draft_temp=1.0, adaptive=True)
        else:
            res = spec_loop_greedy(cache, m, 7, k, 1 if k else 0, n_new)
        dt = time.perf_counter() - t
        cache.free()
        return res, dt

    # one short untimed run of each kernel first: its first launch in the
    # process loads the code object
    run("k0", 0, 2)
    run("sampling_k0", 0, 2)
    for name, k in (("k0", 0), ("k4", 4), ("sampling_k0", 0), ("sampling_k4", 4)):
        res, dt = run(name, k, max_new)
        out[name] = dict(rounds=res.rounds, tokens=len(res.tokens),
                            accepted=sum(res.accepted), status=res.status,
                            us_per_round=round(dt / max(res.rounds, 1) * 1e6, 1),
                            us_per_token=round(dt / max(len(res.tokens), 1) * 1e6, 1))
    # Per layer of a greedy k = 0 round: the 4-layer round minus the 2-layer
    # round of the same model, halved (one layer's append + q phase, its grid
    # attention phase and their two grid barriers), best of 3 each.
    t4 = min(run("k0", 0, max_new)[1] for _ in range(3))
    t2 = min(run("k0", 0, max_new, model2)[1] for _ in range(3))
    out["k0_per_layer_us"] = round((t4 - t2) / max_new / 2 * 1e6, 1)
    out["shape"] = dict(layers=L, nh=nh, nkv=nkv, dph=dph, vocab=V, context=P0,
                        n_draft=1, note="wall time of one launch incl. launch and sync")
    return out


def cpu_baseline(W, w, seconds):
    """The headline layer-step (one query over 32768 keys, Llama-3-8B
    heads) on the host cores: cpu_step's torch-CPU restatement, median over
    about `seconds` of repetitions."""
    c = cpu_step(W, w, "attn", seconds)
    nbytes = w.algorithmic_bytes(l_max=w.l_max, n_app=0, n_queries=1)
    return dict(value=round(nbytes / (c["us_per_layer_step"] * 1e-6) / 1e9, 3), unit="GB/s",
                cores=c["cores"], kind="port", us_per_layer_step=c["us_per_layer_step"],
                sample=f"median of {c['reps']} x one {w.l_max}-key layer-step ({w.nh}q/{w.nkv}kv "
                       f"heads, dph {w.dph}, bs {w.block_size}, fragmented table): torch-CPU "
                       f"index_select gather of the fp16 blocks, fp32 q.K^T, softmax, .V "
                       f"(oracle.attention_torch_cpu), {c['cores']} torch threads, "
                       f"{cpu_model()}")


def measured_traffic(workload: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), if present."""
    f = ROOT / "profiles" / f"{KERNEL}_{workload}_traffic.md"
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build's "
              "path is single-GPU (the design notes describe how it would shard).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from speculative_decode_engine_amd import _native
    from speculative_decode_engine_amd import workloads as W
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _native.load()
    torch.cuda.set_device(0)
    steps, warmup = args.steps, args.warmup
    if args.only_matvec:
        if args.matvec_shape:
            print(json.dumps({"matvec": bench_matvec(torch, steps, warmup, args.matvec_shape)}),
                  flush=True)
        else:
            print(json.dumps({"matvec": bench_matvec(torch, steps, warmup),
                              "sdec_load": bench_sdec_load(torch)}), flush=True)
        if args.calibrate_copy:
            n = args.calibrate_copy * 2 ** 20 // 4
            src = torch.ones(n, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(5):
                dst.copy_(src)
            torch.cuda.synchronize()
        return

    if args.only_shares:
        print(json.dumps({"shares": bench_shares(torch, W, steps, warmup)}), flush=True)
        return
    if args.only:
        modes = {"llama3_8b_verify": "verify", "llama3_8b_4k_decode": "decode",
                 "llama3_8b_4k_attn": "attn", "llama3_8b_verify_fused": "verify_fused",
                 "llama3_8b_4k_decode_fused": "decode_fused", "tiny": "decode",
                 "tinyllama": "decode", "tinyllama_decode_fused": "decode_fused",
                 "qwen25_7b_selfspec_verify": "verify",
                 "qwen25_7b_selfspec_draft": "decode",
                 "qwen25_7b_selfspec_verify_fused": "verify_fused", HEADLINE: "attn"}
        wl = W.CONFIGS[CONFIG_WORKLOAD.get(args.only, args.only)]
        res = bench_config(torch, W, wl, steps, warmup, modes[args.only])
        print(json.dumps({args.only: res}), flush=True)
        if args.calibrate_copy:
            n = args.calibrate_copy * 2 ** 20 // 4
            src = torch.ones(n, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(5):
                dst.copy_(src)
            torch.cuda.synchronize()
        return

    w = W.CONFIGS[HEADLINE]
    log(f"[bench] headline {HEADLINE}: {steps} steps, {warmup} warmup")
    head = bench_config(torch, W, w, steps, warmup, "attn")
    log("[bench]", json.dumps(head))

    configs = {HEADLINE: head}
    extra = {}
    if not args.only_headline:
        w3 = W.CONFIGS["llama3_8b_verify"]
        ver = bench_config(torch, W, w3, steps, warmup, "verify")
        dec = bench_config(torch, W, w3, steps, warmup, "decode")
        att4 = bench_config(torch, W, w3, steps, warmup, "attn")
        configs["llama3_8b_verify"] = ver
        configs["llama3_8b_4k_decode"] = dec
        configs["llama3_8b_4k_attn"] = att4
        extra["verify_over_decode"] = round(ver["us_per_layer_step"] / dec["us_per_layer_step"], 3)
        verf = bench_config(torch, W, w3, steps, warmup, "verify_fused")
        decf = bench_config(torch, W, w3, steps, warmup, "decode_fused")
        configs["llama3_8b_verify_fused"] = verf
        configs["llama3_8b_4k_decode_fused"] = decf
        extra["verify_over_decode_fused"] = round(verf["us_per_layer_step"] /
                                                  decf["us_per_layer_step"], 3)
        for name in ("tiny", "tinyllama"):
            configs[name] = bench_config(torch, W, W.CONFIGS[name], steps, warmup, "decode")
        configs["tinyllama_decode_fused"] = bench_config(torch, W, W.CONFIGS["tinyllama"], steps,
                                                         warmup, "decode_fused")
        w5 = W.CONFIGS["qwen25_7b_selfspec"]
        configs["qwen25_7b_selfspec_verify"] = bench_config(torch, W, w5, steps, warmup, "verify")
        configs["qwen25_7b_selfspec_draft"] = bench_config(torch, W, w5, steps, warmup, "decode")
        configs["qwen25_7b_selfspec_verify_fused"] = bench_config(torch, W, w5, steps, warmup,
                                                                  "verify_fused")
        extra["rollback_us"] = bench_rollback(torch, W)
        extra["accept_us"] = bench_accept(torch)
        log("[bench] accept", json.dumps(extra["accept_us"]))
        extra["matvec"] = bench_matvec(torch, steps, warmup)
        log("[bench] matvec", json.dumps(extra["matvec"]))
        extra["sdec_load"] = bench_sdec_load(torch)
        log("[bench] sdec load", json.dumps(extra["sdec_load"]))
        extra["grid_device_fn"] = bench_grid_device_fn(torch, W, steps, warmup)
        log("[bench] grid device fn", json.dumps(extra["grid_device_fn"]))
        extra["shares"] = bench_shares(torch, W, steps, warmup)
        log("[bench] shares", json.dumps(extra["shares"]))
        extra["spec_loop"] = bench_spec_loop(torch)
        # a loop layer (same heads, 4K context, one query) against the
        # library's decode step (append + attention launches, graph-replayed)
        extra["spec_loop"]["k0_per_layer_over_decode_step"] = round(
            extra["spec_loop"]["k0_per_layer_us"] / configs["llama3_8b_4k_decode"]["us_per_layer_step"], 3)
        log("[bench] spec loop", json.dumps(extra["spec_loop"]))
        for k_, v_ in configs.items():
            log(f"[bench] {k_}: {v_['us_per_layer_step']} us/layer-step, {v_['gbps']} GB/s")

    # One launch per headline step: the graph-replayed step time is the
    # kernel's average launch duration (plus the graph's inter-kernel gap).
    kernel_us = head["us_per_layer_step"]
    nbytes = head["algorithmic_bytes"]
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    hbm = measured_hbm(torch)
    log("[bench] hbm", json.dumps(hbm))
    floor = bench_pattern_floor(torch, W, w, steps, warmup)
    log("[bench] pattern floor", json.dumps(floor))
    roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBPS, 4),
                    traffic=measured_traffic(HEADLINE), kernel=KERNEL,
                    bytes_per_launch=nbytes, kernel_us=kernel_us,
                    kernel_us_eager_events=head.get("kernel_us_events"),
                    measured_read_gbps=hbm["read_gbps"], measured_copy_gbps=hbm["copy_gbps"],
                    frac_of_measured_read=round(achieved / hbm["read_gbps"], 4),
                    frac_of_measured_copy=round(achieved / hbm["copy_gbps"], 4),
                    pattern_floor_us=floor["us"], pattern_floor_gbps=floor["gbps"],
                    kernel_over_pattern_floor=round(kernel_us / floor["us"], 4),
                    reference_points=dict(read=hbm["how"], pattern_floor=floor["how"]))

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline(W, w, args.cpu_seconds)
        log("[bench] cpu", json.dumps(cpu))
        # every other config's layer-step on the CPU oracle too (bounded samples)
        for name, res in configs.items():
            if name == HEADLINE:
                continue
            wl = W.CONFIGS[CONFIG_WORKLOAD.get(name, name)]
            c = cpu_config(W, wl, res["mode"], min(3.0, args.cpu_seconds))
            res["cpu"] = c
            res["gpu_over_cpu"] = round(c["us_per_layer_step"] / res["us_per_layer_step"], 1)
            log(f"[bench] cpu {name}: {c['us_per_layer_step']} us")

    line = {
        "metric": "paged decode-attn us/layer + HBM GB/s (% peak) at ctx 4K/32K, verify k=4",
        "value": head["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["us_per_layer_step"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "data": "synthetic: N(0,1) fp16 K/V filling the pool, N(0,1) fp32 q, seeded "
                "fragmented block tables",
        "config": {"workload": HEADLINE, "keys": head["keys"], "nh": w.nh, "nkv": w.nkv,
                   "head_dim": w.dph, "block_size": w.block_size, "pool_blocks": w.pool_blocks,
                   "rotated_layers": head["rotated_layers"], "us_per_layer_step":
                       head["us_per_layer_step"], "frac_of_hbm_peak": head["frac_of_hbm_peak"]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "configs": configs,
        **extra,
    }
    if args.calibrate_copy:
        n = args.calibrate_copy * 2 ** 20 // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration: 5 copies of {args.calibrate_copy} MiB")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
