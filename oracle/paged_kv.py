"""CPU oracle for the paged-KV hot path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline.

Two layers:
  * `lib()`: the C restatement in oracle/sde_oracle.c (built by
    oracle/Makefile into oracle/_build/libsde_oracle.so): fp16 conversion,
    append / gather on a raw pool, the literal tile-by-tile attention of
    attention.h:21-127, and an fp64 brute force.
  * `PagedKVModel`: the cache state as numpy bytes (pool + tables + seq_len)
    driven through the C functions, for scripted append / rollback / re-append
    sequences checked bit for bit (kv_cache.cu:70-120, kernels.cu:2457-2466).
And `attention_f64_np`, an independent vectorised numpy softmax attention
over gathered (contiguous) K/V.

Reference: arkhamHack/speculative_decode_engine, cuda/include/kv_cache.h,
cuda/src/kv_cache.cu, cuda/include/attention.h, cuda/src/kernels.cu.
"""
from __future__ import annotations

import ctypes
import math
import hashlib
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libsde_oracle.so"

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_ci = ctypes.c_int


def build() -> Path:
    """Compiles the C oracle (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} missing; run `make -C oracle` or __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB_PATH))
    L.oracle_f32_to_f16.restype = ctypes.c_uint16
    L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    L.oracle_f16_to_f32.restype = ctypes.c_float
    L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.oracle_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
    L.oracle_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
    L.oracle_kv_append.argtypes = [_u16p, _i32p, _ci, _ci, _f32p, _f32p, _ci, _ci]
    L.oracle_kv_write_fp16.argtypes = [_u16p, _i32p, _ci, _ci, _u16p, _u16p, _ci, _ci]
    L.oracle_kv_gather.argtypes = [_u16p, _i32p, _ci, _ci, _ci, _ci, _f32p, _f32p]
    L.oracle_attention_tiled.argtypes = [_f32p, _f32p, _u16p, _i32p, _ci, _ci, _ci, _ci, _ci, _ci]
    L.oracle_attention_f64.argtypes = [_f32p, _f64p, _u16p, _i32p, _ci, _ci, _ci, _ci, _ci, _ci]
    L.oracle_paged_attention.restype = _ci
    L.oracle_paged_attention.argtypes = [_f32p, _f32p, _f64p, _u16p, _i32p, _ci, _ci, _ci, _ci,
                                         _ci, _ci, _ci, _ci, _ci]
    L.oracle_max_threads.restype = _ci
    L.oracle_matvec.argtypes = [_f32p, _u16p, _f32p, _ci, _ci, _ci, _ci]
    _lib = L
    return L


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


class PagedKVModel:
    """Cache state on the CPU: the pool as uint16 bits with the reference
    layout [pool_blocks][2 (K,V)][block_size][kv_dim], per-layer tables, and
    the seq_len integer (kv_cache.h:27-51)."""

    def __init__(self, n_layers: int, kv_dim: int, max_blocks_per_layer: int,
                 block_size: int = 16, pool_blocks: int = 0):
        self.n_layers = n_layers
        self.kv_dim = kv_dim
        self.max_blocks = max_blocks_per_layer
        self.bs = block_size
        self.pool_blocks = pool_blocks or n_layers * max_blocks_per_layer
        # kv_cache_alloc zeroes the pool and assigns blocks statically when
        # they fit (kv_cache.cu:16-37).
        self.pool = np.zeros((self.pool_blocks, 2, block_size, kv_dim), dtype=np.uint16)
        self.tables = np.full((n_layers, max_blocks_per_layer), -1, dtype=np.int32)
        self.n_mapped = np.zeros(n_layers, dtype=np.int64)
        if n_layers * max_blocks_per_layer <= self.pool_blocks:
            self.tables[:] = np.arange(n_layers * max_blocks_per_layer,
                                       dtype=np.int32).reshape(n_layers, -1)
            self.n_mapped[:] = max_blocks_per_layer
        self.seq_len = 0

    def set_block_table(self, layer: int, table) -> None:
        t = np.asarray(table, dtype=np.int32)
        assert t.ndim == 1 and t.size <= self.max_blocks
        assert np.all((t >= 0) & (t < self.pool_blocks))
        self.tables[layer, : t.size] = t
        self.n_mapped[layer] = t.size

    def _table(self, layer: int) -> np.ndarray:
        return np.ascontiguousarray(self.tables[layer])

    def append(self, layer: int, k: np.ndarray, v: np.ndarray, pos_base: int) -> None:
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1, self.kv_dim)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1, self.kv_dim)
        assert pos_base >= 0 and pos_base + k.shape[0] <= self.n_mapped[layer] * self.bs
        t = self._table(layer)
        lib().oracle_kv_append(_p(self.pool, _u16p), _p(t, _i32p), self.kv_dim, self.bs,
                               _p(k, _f32p), _p(v, _f32p), pos_base, k.shape[0])

    def write_fp16(self, layer: int, k16: np.ndarray, v16: np.ndarray, pos_base: int) -> None:
        k16 = np.ascontiguousarray(k16).view(np.uint16).reshape(-1, self.kv_dim)
        v16 = np.ascontiguousarray(v16).view(np.uint16).reshape(-1, self.kv_dim)
        assert pos_base >= 0 and pos_base + k16.shape[0] <= self.n_mapped[layer] * self.bs
        t = self._table(layer)
        lib().oracle_kv_write_fp16(_p(self.pool, _u16p), _p(t, _i32p), self.kv_dim, self.bs,
                                   _p(k16, _u16p), _p(v16, _u16p), pos_base, k16.shape[0])

    def gather(self, layer: int, pos: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        assert pos >= 0 and pos + n <= self.n_mapped[layer] * self.bs
        k = np.empty((n, self.kv_dim), dtype=np.float32)
        v = np.empty((n, self.kv_dim), dtype=np.float32)
        t = self._table(layer)
        lib().oracle_kv_gather(_p(self.pool, _u16p), _p(t, _i32p), self.kv_dim, self.bs,
                               pos, n, _p(k, _f32p), _p(v, _f32p))
        return k, v

    def set_seq_len(self, n: int) -> None:
        assert 0 <= n <= self.max_blocks * self.bs
        self.seq_len = n

    def rollback(self, target_len: int) -> None:
        """kv_cache_rollback / set_seq_len_kernel: an integer assignment."""
        assert 0 <= target_len <= self.seq_len
        self.seq_len = target_len

    def pool_sha256(self) -> str:
        return hashlib.sha256(self.pool.tobytes()).hexdigest()

    def attention(self, layer: int, q: np.ndarray, nh: int, nkv: int, dph: int,
                  pos_base: int, mode: str = "tiled", threads: int = 1) -> np.ndarray:
        """cublas_attention_kernel semantics (kernels.cu:904-940): q fp32
        [M][nh*dph]; query m sees pos_base+m+1 keys.  mode 'tiled' = the
        literal fp32 restatement of attention.h; 'f64' = fp64 brute force."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1, nh * dph)
        M = q.shape[0]
        assert pos_base + M <= self.n_mapped[layer] * self.bs
        t = self._table(layer)
        out = np.zeros((M, nh * dph), dtype=np.float32)
        out64 = np.zeros((M, nh * dph), dtype=np.float64)
        lib().oracle_paged_attention(_p(q, _f32p), _p(out, _f32p), _p(out64, _f64p),
                                     _p(self.pool, _u16p), _p(t, _i32p), self.kv_dim, self.bs,
                                     nh, nkv, dph, pos_base, M, 0 if mode == "tiled" else 1,
                                     threads)
        return out if mode == "tiled" else out64

    def attention_one(self, layer: int, q: np.ndarray, nh: int, nkv: int, dph: int,
                      total_len: int) -> np.ndarray:
        """device_flash_attention_gqa with an explicit total_len (any value
        >= 0, including 0) for one query."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(nh * dph)
        out = np.zeros(nh * dph, dtype=np.float32)
        t = self._table(layer)
        lib().oracle_attention_tiled(_p(q, _f32p), _p(out, _f32p), _p(self.pool, _u16p),
                                     _p(t, _i32p), self.kv_dim, self.bs, nh, nkv, dph, total_len)
        return out


def run_script(model: PagedKVModel, ops, on_checkpoint=None, on_attend=None) -> list:
    """Executes a workloads.scripted_rounds op list on the CPU model.
    Returns [(label, seq_len, pool_sha256)] at every checkpoint."""
    marks = []
    for op in ops:
        kind = op[0]
        if kind == "write_fp16":
            model.write_fp16(op[1], op[3], op[4], op[2])
        elif kind == "append":
            model.append(op[1], op[3], op[4], op[2])
        elif kind == "set_seq_len":
            model.set_seq_len(op[1])
        elif kind == "rollback":
            model.rollback(op[1])
        elif kind == "checkpoint":
            marks.append((op[1], model.seq_len, model.pool_sha256()))
            if on_checkpoint is not None:
                on_checkpoint(op[1], model)
        elif kind == "attend":
            if on_attend is not None:
                on_attend(model, op[1], op[2], op[3])
        else:
            raise ValueError(f"unknown op {kind}")
    return marks


def spec_accept_greedy(draft_tokens, target_tokens, k: int, target_save: int,
                       draft_save: int, shared: bool):
    """Greedy acceptance and rewind of the reference's loop
    (kernels.cu:2428-2466; megakernel kernels.cu:3050-3072): n = leading
    drafts equal to the target's argmaxes, emit drafts[:n] + [bonus =
    target[n]], target seq_len = target_save + n + 1, draft seq_len =
    draft_save + n (the target's value for one shared cache).  Returns
    (n, bonus, target_seq, draft_seq, emitted)."""
    n = 0
    while n < k and int(draft_tokens[n]) == int(target_tokens[n]):
        n += 1
    target_seq = target_save + n + 1
    draft_seq = target_seq if shared else draft_save + n
    emitted = [int(t) for t in draft_tokens[:n]] + [int(target_tokens[n])]
    return n, int(target_tokens[n]), target_seq, draft_seq, emitted


def spec_loop_greedy(model: PagedKVModel, emb_q, emb_k, emb_v, head_bits, nh: int, nkv: int,
                     dph: int, anchor: int, k: int, n_draft: int, max_new: int,
                     shift_rewind: int = 0, eos_token: int = -1):
    """The persistent self-speculative greedy loop (megakernel_speculative,
    kernels.cu:2864-3106; self-speculative verify model.cu:838-890) over the
    byte model, with the loop model of sde_spec_loop_greedy: layer l of token
    t has q, k, v rows emb_q/emb_k/emb_v[l][t] (fp32), q adds the previous
    layer's attention output (rounded to fp32, as the device keeps it), and
    the logits are that output of the last layer (fp64) times head (fp16
    bits [nh*dph][V], widened exactly), argmax taking the lowest index.

    Each round from P = model.seq_len: for i = 0..k (k > 0) the prefix layers
    [0, n_draft) append window token i at P+i and attend (one query); the
    first k of them propose window token i+1 from their head logits.  Then
    layers [n_draft, n_layers) (all layers when k = 0) append the window
    [anchor, drafts] at P.. and attend it causally; the target's tokens are
    the argmaxes of every row; spec_accept_greedy emits the accepted drafts
    and the bonus and seq_len <- P + n + 1 (kernels.cu:3050-3072).
    `shift_rewind` plants a rewind mistake (for the tests that must catch
    one).  The loop stops after a round whose bonus is eos_token >= 0
    (kernels.cu:3095).  Returns (tokens, accepted per round, rounds)."""
    L = model.n_layers
    d = nh * dph
    head = f16_bits_to_f32(np.asarray(head_bits, dtype=np.uint16)).astype(np.float64)
    M = k + 1
    tokens_out, accepted = [], []
    cur = int(anchor)
    while len(tokens_out) < max_new:
        P = model.seq_len
        window = [cur] + [0] * k
        h = np.zeros((M, d), dtype=np.float32)

        def layers(lo, hi, r0, n):
            for l in range(lo, hi):
                toks = window[r0:r0 + n]
                model.append(l, emb_k[l][toks], emb_v[l][toks], P + r0)
                q = emb_q[l][toks].astype(np.float32)
                if l > 0:
                    q = q + h[r0:r0 + n]
                out = model.attention(l, q, nh, nkv, dph, P + r0, mode="f64")
                h[r0:r0 + n] = out.astype(np.float32)
            return h[r0:r0 + n].astype(np.float64) @ head

        lo = 0
        if k > 0:
            for i in range(M):
                logits = layers(0, n_draft, i, 1)
                if i < k:
                    window[i + 1] = int(np.argmax(logits[0]))
            lo = n_draft
        logits = layers(lo, L, 0, M)
        target = [int(np.argmax(logits[m])) for m in range(M)]
        n, bonus, t_seq, _, emitted = spec_accept_greedy(window[1:], target, k, P, P, True)
        tokens_out += emitted
        accepted.append(n)
        model.seq_len = t_seq + shift_rewind
        cur = bonus
        if eos_token >= 0 and bonus == eos_token:
            break
    return tokens_out, accepted, len(accepted)


def _forward_rows(model: PagedKVModel, lm, window, h, lo: int, hi: int, r0: int, n: int,
                  pos0: int):
    """Layers [lo, hi) of loop model lm = (emb_q, emb_k, emb_v, head_bits, nh, nkv, dph)
    over window rows [r0, r0+n) at positions pos0 + row: append each row's
    K/V, q = emb_q (+ the previous layer's output in h), fp64 attention
    rounded to fp32 into h.  Returns the rows' logits (fp64, h @ head)."""
    emb_q, emb_k, emb_v, head_bits, nh, nkv, dph = lm
    for l in range(lo, hi):
        toks = window[r0:r0 + n]
        model.append(l, emb_k[l][toks], emb_v[l][toks], pos0 + r0)
        q = emb_q[l][toks].astype(np.float32)
        if l > 0:
            q = q + h[r0:r0 + n]
        out = model.attention(l, q, nh, nkv, dph, pos0 + r0, mode="f64")
        h[r0:r0 + n] = out.astype(np.float32)
    head = f16_bits_to_f32(np.asarray(head_bits, dtype=np.uint16)).astype(np.float64)
    return h[r0:r0 + n].astype(np.float64) @ head


def _catch_up(draft: PagedKVModel, dm, tok: int, pos: int) -> None:
    """The draft model's forward of one token at `pos` as the cache sees it
    (kernels.cu:3079-3093): its K/V rows in every layer (the K/V of the loop
    model depend on (token, position) only; the forward's logits are unused)."""
    _, emb_k, emb_v = dm[0], dm[1], dm[2]
    for l in range(draft.n_layers):
        draft.append(l, emb_k[l][[tok]], emb_v[l][[tok]], pos)


def spec_loop_greedy_two(target: PagedKVModel, draft: PagedKVModel, tm, dm, anchor: int, k: int,
                         max_new: int, eos_token: int = -1, shift_draft_rewind: int = 0):
    """The persistent greedy loop with a separate draft model and cache
    (megakernel_speculative_kernel with shared_kv false, kernels.cu:2864-3106).
    tm, dm: (emb_q, emb_k, emb_v, head_bits, nh, nkv, dph) of the target and
    draft models.  Each round from P = target.seq_len, D = draft.seq_len:
      * draft steps i = 0..k-1 (kernels.cu:2948-2958): the draft model appends
        window token i (the anchor, then each draft) at D+i in all its layers,
        attends with one query, and its head's argmax is window token i+1;
      * verify (model_batch_forward_logits, model.cu:657-714): the target
        appends the window [anchor, drafts] at P.. and attends causally; the
        argmax of every row is the target's token;
      * accept (kernels.cu:3050-3076): n leading matches, emit drafts[:n] and
        the bonus target[n]; target seq_len <- P+n+1, draft seq_len <- D+n;
      * catch-up (kernels.cu:3079-3093): the draft model's forward of the
        last draft when all k were accepted (its K/V were never written) or
        of the bonus otherwise, at D+n; draft seq_len <- D+n+1.  (In the
        second case the bonus lands where the last accepted draft was, as in
        the reference: the draft cache then trails the true sequence by that
        token, which costs acceptance, never output.)
      * stop once max_new tokens are out, or after a round whose bonus is
        eos_token >= 0 (kernels.cu:3095: the bonus is checked, not the
        accepted drafts).
    `shift_draft_rewind` plants a draft-rewind mistake for the tests.
    Returns (tokens, accepted per round, rounds)."""
    assert k >= 1
    M = k + 1
    dt = dm[4] * dm[6]
    tt = tm[4] * tm[6]
    tokens_out, accepted = [], []
    cur = int(anchor)
    while len(tokens_out) < max_new:
        P, D = target.seq_len, draft.seq_len
        window = [cur] + [0] * k
        hd = np.zeros((M, dt), dtype=np.float32)
        for i in range(k):
            logits = _forward_rows(draft, dm, window, hd, 0, draft.n_layers, i, 1, D)
            window[i + 1] = int(np.argmax(logits[0]))
        ht = np.zeros((M, tt), dtype=np.float32)
        logits = _forward_rows(target, tm, window, ht, 0, target.n_layers, 0, M, P)
        tgt = [int(np.argmax(logits[m])) for m in range(M)]
        n, bonus, t_seq, d_seq, emitted = spec_accept_greedy(window[1:], tgt, k, P, D, False)
        tokens_out += emitted
        accepted.append(n)
        target.seq_len = t_seq
        d_seq += shift_draft_rewind
        _catch_up(draft, dm, window[k] if n == k else bonus, d_seq)
        draft.seq_len = d_seq + 1
        cur = bonus
        if eos_token >= 0 and bonus == eos_token:
            break
    return tokens_out, accepted, len(accepted)


def spec_loop_stochastic_two(target: PagedKVModel, draft: PagedKVModel, tm, dm, anchor: int,
                             k: int, max_new: int, seed: int, offset: int = 0,
                             draft_temp: float = 1.0, adaptive: bool = False,
                             min_temp: float = 0.1, max_temp: float = 2.0,
                             target_accept: float = 0.7, gain: float = 0.1,
                             ewma_mix: float = 0.2, eos_token: int = -1):
    """The sampling loop with a separate draft model and cache
    (megakernel_speculative_stochastic_kernel with shared_kv false,
    kernels.cu:3108-3481), on spec_loop_greedy_two's rounds: draft token i+1
    is sampled (spec_accept_stochastic with no drafts, its bonus row) from
    the draft model's logits of row i at T_d, one call index each; the
    window's target logits (temperature 1) and the draft rows' logits (T_d)
    go to spec_accept_stochastic for the accept tests and the corrected or
    bonus sample, one more call index; target seq_len <- P+n+1, draft
    seq_len <- D+n, then the draft catch-up of spec_loop_greedy_two; T_d
    adapts as in spec_loop_stochastic; the EOS stop as in the greedy loop.
    (The target rewinds like the batched verify path, without the
    reference's extra target forward of a rejection's corrected token.)
    Returns spec_loop_stochastic's tuple."""
    assert k >= 1
    M = k + 1
    f32 = np.float32
    temp, ewma = f32(draft_temp), f32(-1.0)
    mix = min(max(f32(ewma_mix), f32(1e-6)), f32(1.0) - f32(1e-6))
    dt = dm[4] * dm[6]
    tt = tm[4] * tm[6]
    tokens_out, accepted = [], []
    margin = float("inf")
    cur = int(anchor)
    while len(tokens_out) < max_new:
        P, D = target.seq_len, draft.seq_len
        window = [cur] + [0] * k
        hd = np.zeros((M, dt), dtype=np.float32)
        dlog = []
        for i in range(k):
            logits = _forward_rows(draft, dm, window, hd, 0, draft.n_layers, i, 1, D)
            r = spec_accept_stochastic(logits, None, [], 0, float(temp), 1.0, seed, offset, 0, 0,
                                       True)
            offset += 1
            margin = min(margin, r["sample_margin"][0])
            window[i + 1] = r["token"]
            dlog.append(logits[0])
        ht = np.zeros((M, tt), dtype=np.float32)
        logits = _forward_rows(target, tm, window, ht, 0, target.n_layers, 0, M, P)
        r = spec_accept_stochastic(logits, np.array(dlog), window[1:], k, 1.0, float(temp), seed,
                                   offset, P, D, False)
        offset += 1
        n = r["n_accepted"]
        margin = min([margin] + r["accept_margin"][:min(n + 1, k)] + [r["sample_margin"][n]])
        tokens_out += r["emitted"]
        accepted.append(n)
        target.seq_len = r["target_seq"]
        bonus = r["token"]
        _catch_up(draft, dm, window[k] if n == k else bonus, r["draft_seq"])
        draft.seq_len = r["draft_seq"] + 1
        cur = bonus
        if adaptive:
            rr = f32(n) / f32(k)
            ewma = rr if ewma < 0 else f32((f32(1.0) - mix) * ewma + mix * rr)
            temp = f32(temp + f32(gain) * f32(ewma - f32(target_accept)))
            temp = f32(max(f32(min_temp), min(f32(max_temp), temp)))
        if eos_token >= 0 and bonus == eos_token:
            break
    return tokens_out, accepted, len(accepted), float(temp), float(ewma), offset, margin


_PHILOX_M = (0xD2511F53, 0xCD9E8D57)   # Salmon et al., SC'11 (Philox4x32)
_PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def spec_loop_stochastic(model: PagedKVModel, emb_q, emb_k, emb_v, head_bits, nh: int,
                         nkv: int, dph: int, anchor: int, k: int, n_draft: int, max_new: int,
                         seed: int, offset: int = 0, draft_temp: float = 1.0,
                         adaptive: bool = False, min_temp: float = 0.1, max_temp: float = 2.0,
                         target_accept: float = 0.7, gain: float = 0.1, ewma_mix: float = 0.2,
                         eos_token: int = -1):
    """The persistent self-speculative sampling loop
    (megakernel_speculative_stochastic_kernel, kernels.cu:3108-3481) over
    the byte model, with spec_loop_greedy's model and rounds: draft token
    i+1 = spec_accept_stochastic with no drafts (its bonus sample) on the
    prefix layers' logits of row i at the draft temperature T_d, one call
    index each; then the window's target logits (temperature 1) and the
    draft rows' logits (T_d) go to spec_accept_stochastic for the accept
    tests and the corrected / bonus sample, one more call index; seq_len <-
    P + n + 1.  With `adaptive`, after each round (kernels.cu:3441-3458,
    in float32): r = n / k, ewma = r the first time else (1 - mix) ewma +
    mix r with mix clamped to [1e-6, 1 - 1e-6], T_d += gain (ewma -
    target_accept), clamped to [min_temp, max_temp].  Returns (tokens,
    accepted per round, rounds, final T_d, final ewma, final offset, the
    smallest distance of any accept test / sample from its boundary)."""
    L = model.n_layers
    d = nh * dph
    head = f16_bits_to_f32(np.asarray(head_bits, dtype=np.uint16)).astype(np.float64)
    M = k + 1
    f32 = np.float32
    temp, ewma = f32(draft_temp), f32(-1.0)
    mix = min(max(f32(ewma_mix), f32(1e-6)), f32(1.0) - f32(1e-6))
    tokens_out, accepted = [], []
    margin = float("inf")
    cur = int(anchor)
    while len(tokens_out) < max_new:
        P = model.seq_len
        window = [cur] + [0] * k
        h = np.zeros((M, d), dtype=np.float32)

        def layers(lo, hi, r0, n):
            for l in range(lo, hi):
                toks = window[r0:r0 + n]
                model.append(l, emb_k[l][toks], emb_v[l][toks], P + r0)
                q = emb_q[l][toks].astype(np.float32)
                if l > 0:
                    q = q + h[r0:r0 + n]
                out = model.attention(l, q, nh, nkv, dph, P + r0, mode="f64")
                h[r0:r0 + n] = out.astype(np.float32)
            return h[r0:r0 + n].astype(np.float64) @ head

        lo = 0
        dlog = []
        if k > 0:
            for i in range(M):
                logits = layers(0, n_draft, i, 1)
                if i < k:
                    r = spec_accept_stochastic(logits, None, [], 0, float(temp), 1.0, seed,
                                               offset, 0, 0, True)
                    offset += 1
                    margin = min(margin, r["sample_margin"][0])
                    window[i + 1] = r["token"]
                    dlog.append(logits[0])
            lo = n_draft
        logits = layers(lo, L, 0, M)
        r = spec_accept_stochastic(logits, np.array(dlog) if k else None, window[1:], k, 1.0,
                                   float(temp), seed, offset, P, P, True)
        offset += 1
        n = r["n_accepted"]
        margin = min([margin] + r["accept_margin"][:min(n + 1, k)] + [r["sample_margin"][n]])
        tokens_out += r["emitted"]
        accepted.append(n)
        model.seq_len = r["target_seq"]
        cur = r["token"]
        if adaptive and k > 0:
            rr = f32(n) / f32(k)
            ewma = rr if ewma < 0 else f32((f32(1.0) - mix) * ewma + mix * rr)
            temp = f32(temp + f32(gain) * f32(ewma - f32(target_accept)))
            temp = f32(max(f32(min_temp), min(f32(max_temp), temp)))
        if eos_token >= 0 and cur == eos_token:
            break
    return tokens_out, accepted, len(accepted), float(temp), float(ewma), offset, margin


def philox4x32_10(ctr, key) -> list:
    """Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
    as easy as 1, 2, 3", SC'11), the counter-based generator of
    sde_spec_accept_stochastic: 10 rounds of two 32x32->64 multiplies,
    Weyl key schedule.  ctr: 4 uint32, key: 2 uint32; returns 4 uint32."""
    c = [int(x) & 0xFFFFFFFF for x in ctr]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for _ in range(10):
        p0 = _PHILOX_M[0] * c[0]
        p1 = _PHILOX_M[1] * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k0) & 0xFFFFFFFF, p1 & 0xFFFFFFFF,
             ((p0 >> 32) ^ c[3] ^ k1) & 0xFFFFFFFF, p0 & 0xFFFFFFFF]
        k0 = (k0 + _PHILOX_W[0]) & 0xFFFFFFFF
        k1 = (k1 + _PHILOX_W[1]) & 0xFFFFFFFF
    return c


def spec_draws(seed: int, offset: int, b: int) -> tuple:
    """(u_accept, u_sample) of window row b of call `offset`: counter
    (b, offset lo, offset hi, 0), key = seed; u = ((x >> 8) + 0.5) / 2^24."""
    r = philox4x32_10([b, offset & 0xFFFFFFFF, (offset >> 32) & 0xFFFFFFFF, 0],
                      [seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF])
    return tuple(float(np.float32(((x >> 8) + 0.5) / 16777216.0)) for x in r[:2])


def spec_accept_stochastic(target_logits, draft_logits, draft_tokens, k: int,
                           temp_target: float, temp_draft: float, seed: int, offset: int,
                           target_save: int, draft_save: int, shared: bool) -> dict:
    """Speculative sampling with the reference's rules, in float64:
    draft token i is accepted iff u_i < min(1, p_i / max(q_i, 1e-36)) with
    p = softmax(target_logits[i] / T_t), q = softmax(draft_logits[i] / T_d)
    (batch_stochastic_accept_kernel, kernels.cu:550-572; temperatures below
    1e-6 act as 1e-6); the first rejection at i emits a token sampled from
    norm(max(0, p - q)), or from p when that is empty
    (device_corrected_adjusted_sample, kernels.cu:319-380); with every draft
    accepted the bonus is sampled from p of row k.  A sample is the first
    token, in the order below, whose cumulative weight reaches u * total
    (and has a positive weight): tokens ordered by vocabulary slice (S =
    min(ceil(V/4096), 64) slices of L = ceil(V/S) tokens), then by
    (l % 1024, l // 1024) of the offset l in the slice -- the library's
    coalescing-friendly inverse-CDF order (index order for V <= 1024; any
    fixed order samples the same distribution).  Rewinds as
    spec_accept_greedy.  Returns the result and, per row, the distance of
    the accept test and of the sample from their decision boundaries."""
    tl = np.asarray(target_logits, np.float64)
    dl = np.asarray(draft_logits, np.float64) if k else None
    it, idr = 1.0 / max(temp_target, 1e-6), 1.0 / max(temp_draft, 1e-6)

    def softmax(x):
        e = np.exp(x - x.max())
        return e / e.sum()
    flags, tokens, acc_margin, smp_margin = [], [], [], []
    for b in range(k + 1):
        ua, us = spec_draws(seed, offset, b)
        p = softmax(tl[b] * it)
        if b < k:
            q = softmax(dl[b] * idr)
            d = int(draft_tokens[b])
            cap = min(1.0, p[d] / max(q[d], 1e-36))
            flags.append(ua < cap)
            acc_margin.append(abs(ua - cap))
            w = np.maximum(p - q, 0.0)
            if w.sum() <= 1e-20:
                w = p
        else:
            w = p
        V = w.shape[0]
        S = min((V + 4095) // 4096, 64)
        L = (V + S - 1) // S
        i = np.arange(V)
        loc = i % L
        order = np.lexsort((loc // 1024, loc % 1024, i // L))
        wo = w[order]
        cdf = np.cumsum(wo)
        goal = us * cdf[-1]
        idx = np.nonzero((cdf >= goal) & (wo > 0))[0]
        pos = int(idx[0]) if idx.size else int(np.nonzero(wo > 0)[0][-1])
        tokens.append(int(order[pos]))
        lo = cdf[pos] - wo[pos]
        smp_margin.append(min(abs(goal - lo), abs(cdf[pos] - goal)) / cdf[-1])
    n = 0
    while n < k and flags[n]:
        n += 1
    t_seq = target_save + n + 1
    return dict(n_accepted=n, token=tokens[n], target_seq=t_seq,
                draft_seq=t_seq if shared else draft_save + n,
                emitted=[int(t) for t in draft_tokens[:n]] + [tokens[n]],
                flags=flags, tokens=tokens, accept_margin=acc_margin, sample_margin=smp_margin)


ROPE_NONE, ROPE_LINEAR, ROPE_NTK, ROPE_YARN = 0, 1, 2, 3  # config.h:42-47


def rope_inv_freq(dph: int, theta: float = 10000.0, scaling_type: int = ROPE_NONE,
                  factor: float = 1.0) -> np.ndarray:
    """Inverse frequencies of rope_apply_inplace (model.cu:281-323): theta
    (10000 when <= 1e-6), times factor^(dph/(dph-2)) for NTK with factor > 1;
    inv_freq[j] = exp(-ln(theta) * 2j / dph), in float64 rounded to float32
    (the rule sde_rope_append_attention states for its table)."""
    th = float(np.float32(theta))
    th = th if th > 1e-6 else 10000.0
    f = float(np.float32(factor))
    if scaling_type == ROPE_NTK and f > 1.0:
        th *= f ** (dph / (dph - 2.0))
    j = np.arange(dph // 2, dtype=np.float64)
    return np.exp(-np.log(th) * 2.0 * j / dph).astype(np.float32)


def rope_rotate_half_f64(x: np.ndarray, n_heads: int, dph: int, positions,
                         theta: float = 10000.0, scaling_type: int = ROPE_NONE,
                         factor: float = 1.0) -> np.ndarray:
    """Rotate-half RoPE of rows x [M][n_heads*dph] at positions[m]
    (rope_apply_inplace, model.cu:281-323): dim j pairs with j + dph/2,
    (x0, x1) -> (x0 c - x1 s, x0 s + x1 c) with c, s = cos, sin(angle);
    angle = float32(float32(pos) / div) * inv_freq[j] as a float32 product,
    div = factor for linear / YaRN with factor > 1 (else 1).  The rotation
    is evaluated in float64."""
    x = np.asarray(x, dtype=np.float64).reshape(-1, n_heads, dph)
    pos = np.asarray(positions, dtype=np.int64).reshape(-1)
    assert pos.shape[0] == x.shape[0]
    inv = rope_inv_freq(dph, theta, scaling_type, factor)
    f = np.float32(factor)
    div = f if scaling_type in (ROPE_LINEAR, ROPE_YARN) and f > 1 else np.float32(1.0)
    ps = (pos.astype(np.float32) / div).astype(np.float32)
    angle = (ps[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    c, sn = np.cos(angle)[:, None, :], np.sin(angle)[:, None, :]
    half = dph // 2
    x0, x1 = x[..., :half], x[..., half:]
    out = np.concatenate([x0 * c - x1 * sn, x0 * sn + x1 * c], axis=-1)
    return out.reshape(-1, n_heads * dph)


def attention_f64_np(q: np.ndarray, K: np.ndarray, V: np.ndarray, nh: int, nkv: int,
                     dph: int, pos_base: int) -> np.ndarray:
    """softmax(q K^T / sqrt(dph)) V in fp64 with numpy, on contiguous
    (already gathered) K, V [L][nkv*dph]; query m sees pos_base+m+1 keys;
    head h uses KV head h*nkv//nh.  Returns float64 [M][nh*dph]."""
    q = np.asarray(q, dtype=np.float64).reshape(-1, nh, dph)
    M = q.shape[0]
    L_all = pos_base + M
    K = np.asarray(K[:L_all], dtype=np.float64).reshape(L_all, nkv, dph)
    V = np.asarray(V[:L_all], dtype=np.float64).reshape(L_all, nkv, dph)
    kvh_of = (np.arange(nh) * nkv) // nh
    out = np.zeros((M, nh, dph), dtype=np.float64)
    scale = 1.0 / np.sqrt(dph)
    for kvh in range(nkv):
        heads = np.nonzero(kvh_of == kvh)[0]
        Kg = K[:, kvh, :]  # [L][dph]
        Vg = V[:, kvh, :]
        for m in range(M):
            L = pos_base + m + 1
            logits = (q[m, heads] @ Kg[:L].T) * scale  # [heads][L]
            logits -= logits.max(axis=1, keepdims=True)
            w = np.exp(logits)
            w /= w.sum(axis=1, keepdims=True)
            out[m, heads] = w @ Vg[:L]
    return out.reshape(M, nh * dph)


def attention_torch_cpu(pool, table, q, nh: int, nkv: int, dph: int, block_size: int,
                        pos_base: int):
    """The reference's paged attention semantics as a torch-CPU step
    (attention.h:21-127 driven by cublas_attention_kernel, kernels.cu:904-940):
    block-table gather (index_select) of the fp16 K/V blocks, fp32
    q.K^T * dph^-1/2, causal mask per query (query m sees pos_base+m+1 keys),
    softmax, .V.  The timed CPU baseline of bench.py (torch's own threads);
    the tile loop and the fp64 brute force stay the parity checkers.

    pool: torch.int16/float16 [pool_blocks][2][block_size][nkv*dph] (fp16
    bits); table: torch int64 [>= ceil(L/block_size)]; q: torch float32
    [M][nh*dph].  Returns float32 [M][nh*dph]."""
    import torch
    M = q.shape[0]
    L = pos_base + M
    G = nh // nkv
    nblk = -(-L // block_size)
    blocks = pool.view(torch.float16).index_select(0, table[:nblk])  # [nblk][2][BS][kv_dim]
    K = blocks[:, 0].reshape(nblk * block_size, nkv, dph)[:L].float().permute(1, 0, 2)
    V = blocks[:, 1].reshape(nblk * block_size, nkv, dph)[:L].float().permute(1, 0, 2)
    # rows of KV head g: (query m, head-in-group j) -> q head g*G + j
    qg = q.reshape(M, nkv, G, dph).permute(1, 0, 2, 3).reshape(nkv, M * G, dph)
    s = torch.bmm(qg, K.transpose(1, 2).contiguous()) * (1.0 / math.sqrt(dph))
    if M > 1:
        lim = pos_base + torch.arange(M).repeat_interleave(G)  # last visible key per row
        hidden = torch.arange(L)[None, :] > lim[:, None]
        s = s.masked_fill(hidden[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    out = torch.bmm(p, V.contiguous())  # [nkv][M*G][dph]
    return out.reshape(nkv, M, G, dph).permute(1, 0, 2, 3).reshape(M, nh * dph)


# ---- the output projection (Wo) -------------------------------------------

def matvec_ref(x: np.ndarray, W_bits: np.ndarray, out: np.ndarray | None = None,
               accumulate: bool = False) -> np.ndarray:
    """device_matvec_partial(_accum) / device_matvec_batched (utils.h:248-280,
    417-452) restated in C (oracle_matvec): fp32, per column in row order.
    x fp32 [M][d_in], W_bits uint16 fp16 bits [d_in][d_out]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, W_bits.shape[0])
    W_bits = np.ascontiguousarray(W_bits, dtype=np.uint16)
    M, d_in = x.shape
    d_out = W_bits.shape[1]
    if out is None:
        out = np.zeros((M, d_out), dtype=np.float32)
    else:
        out = np.ascontiguousarray(out, dtype=np.float32).reshape(M, d_out).copy()
    lib().oracle_matvec(_p(x, _f32p), _p(W_bits, _u16p), _p(out, _f32p), d_in, d_out, M,
                        int(bool(accumulate)))
    return out


def matvec_f64(x: np.ndarray, W_bits: np.ndarray, out0: np.ndarray | None = None) -> tuple:
    """Exact-ish float64 product x @ W (W decoded from fp16 bits), plus the
    per-output magnitude sum_r |x[m][r] * W[r][c]| that bounds an fp32
    summation's rounding error; out0 (fp32) is added when given."""
    x64 = np.asarray(x, dtype=np.float64).reshape(-1, W_bits.shape[0])
    W64 = W_bits.view(np.float16).astype(np.float64)
    y = x64 @ W64
    mag = np.abs(x64) @ np.abs(W64)
    if out0 is not None:
        o = np.asarray(out0, dtype=np.float64).reshape(y.shape)
        y = y + o
        mag = mag + np.abs(o)
    return y, mag
