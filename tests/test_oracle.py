"""Pins the CPU oracle (oracle/) before anything is checked against it.

The reference has no golden vectors for this path, so each oracle function
is pinned by an independent formulation or a closed form:
  * fp16 conversion: numpy's IEEE binary16 cast, exhaustively for fp16->fp32
    and on random + boundary + tie values for fp32->fp16;
  * paged layout (kv_cache.h:5-18, kv_cache.cu:58-93): numpy fancy indexing
    of the [block][K|V][slot][kv_dim] pool, block-table permutation
    invariance, the contiguous special case block_size=1, untouched bytes;
  * rollback (kernels.cu:2457-2466): pool bytes unchanged, re-append only
    rewrites [target, target+n);
  * attention (attention.h:21-127): the fp32 tile restatement against an
    fp64 brute force in C, a vectorised numpy softmax, and torch's
    scaled_dot_product_attention (float64, CPU); closed forms (total_len=0,
    one key, uniform logits, one-hot logits); causal window = independent
    single-query calls; and planted mistakes (head mapping, scale,
    off-by-one length, K/V swap) that the 2e-3 tolerance must catch.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from speculative_decode_engine_amd import workloads as W

GOLDEN = Path(__file__).resolve().parent / "golden"
ATOL, RTOL = 2e-3, 1e-2  # north_star tolerance for attention outputs


# ---- fp16 conversion ------------------------------------------------------------

def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    parts = [
        rng.standard_normal(200_000).astype(np.float32),
        (rng.standard_normal(50_000) * 1e4).astype(np.float32),
        (rng.standard_normal(50_000) * 1e-5).astype(np.float32),   # fp16 subnormals
        np.exp(rng.uniform(-30, 12, 100_000)).astype(np.float32),  # all exponents
        np.array([0.0, -0.0, 65504, 65519.996, 65520, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 6.1e-5], np.float32),
    ]
    # exact ties: halfway between adjacent fp16 values (both parities)
    h = np.arange(0, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(0, 0x7bff, 7, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    parts.append(((h + nxt) / 2).astype(np.float32))
    x = np.concatenate(parts)
    x = np.concatenate([x, -x])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_bits(x)
    assert np.array_equal(got, want)


def test_f32_to_f16_nan_stays_nan(oracle):
    x = np.array([np.nan, -np.nan], np.float32)
    got = oracle.f32_to_f16_bits(x).view(np.float16)
    assert np.all(np.isnan(got))


# ---- layout / append / gather / rollback -----------------------------------------

def _model_with_tables(oracle, n_layers=3, kv_dim=24, nblk=5, bs=4, pool=40, seed=1):
    rng = np.random.default_rng(seed)
    tables = W.make_tables(rng, n_layers, nblk, pool)
    m = oracle.PagedKVModel(n_layers, kv_dim, nblk, bs, pool)
    for l in range(n_layers):
        m.set_block_table(l, tables[l])
    return m, tables, rng


def test_append_layout_against_numpy_indexing(oracle):
    m, tables, rng = _model_with_tables(oracle)
    n = 5 * 4
    k, v = W.new_kv(rng, n, m.kv_dim)
    before = m.pool.copy()
    m.append(1, k, v, 0)
    pos = np.arange(n)
    blk = tables[1][pos // m.bs]
    slot = pos % m.bs
    assert np.array_equal(m.pool[blk, 0, slot], k.astype(np.float16).view(np.uint16))
    assert np.array_equal(m.pool[blk, 1, slot], v.astype(np.float16).view(np.uint16))
    touched = np.zeros(m.pool.shape[0], bool)
    touched[tables[1]] = True
    assert np.array_equal(m.pool[~touched], before[~touched])  # other blocks untouched


def test_append_gather_roundtrip_and_offsets(oracle):
    m, tables, rng = _model_with_tables(oracle)
    k, v = W.new_kv(rng, 7, m.kv_dim)
    m.append(2, k, v, 9)  # crosses a block boundary (bs=4)
    gk, gv = m.gather(2, 9, 7)
    assert np.array_equal(gk, k.astype(np.float16).astype(np.float32))
    assert np.array_equal(gv, v.astype(np.float16).astype(np.float32))
    # positions before 9 of that layer are still zero
    zk, zv = m.gather(2, 0, 9)
    assert not zk.any() and not zv.any()


def test_permutation_invariance(oracle):
    rng = np.random.default_rng(5)
    a = oracle.PagedKVModel(1, 16, 6, 8, 20)
    b = oracle.PagedKVModel(1, 16, 6, 8, 20)
    ta = rng.permutation(20)[:6]
    tb = rng.permutation(20)[:6]
    a.set_block_table(0, ta)
    b.set_block_table(0, tb)
    k, v = W.new_kv(rng, 48, 16)
    a.append(0, k, v, 0)
    b.append(0, k, v, 0)
    for x, y in zip(a.gather(0, 0, 48), b.gather(0, 0, 48)):
        assert np.array_equal(x, y)
    assert np.array_equal(a.pool[ta], b.pool[tb])


def test_block_size_one_is_contiguous(oracle):
    rng = np.random.default_rng(6)
    m = oracle.PagedKVModel(1, 8, 10, 1, 10)
    m.set_block_table(0, np.arange(10))
    k, v = W.new_kv(rng, 10, 8)
    m.append(0, k, v, 0)
    assert np.array_equal(m.pool[:, 0, 0], k.astype(np.float16).view(np.uint16))
    assert np.array_equal(m.pool[:, 1, 0], v.astype(np.float16).view(np.uint16))


def test_static_assignment_matches_reference_alloc(oracle):
    m = oracle.PagedKVModel(3, 8, 4, 16)  # pool = n_layers * max_blocks
    assert np.array_equal(m.tables, np.arange(12).reshape(3, 4))  # kv_cache.cu:32-37


def test_rollback_moves_no_bytes_and_reappend_is_local(oracle):
    m, tables, rng = _model_with_tables(oracle, n_layers=1, nblk=6, bs=4, pool=12)
    k, v = W.new_kv(rng, 20, m.kv_dim)
    m.append(0, k, v, 0)
    m.set_seq_len(20)
    before = m.pool.copy()
    m.rollback(13)
    assert m.seq_len == 13 and np.array_equal(m.pool, before)
    with pytest.raises(AssertionError):
        m.rollback(14)  # beyond seq_len
    k2, v2 = W.new_kv(rng, 3, m.kv_dim)
    m.append(0, k2, v2, 13)
    gk, gv = m.gather(0, 0, 20)
    exp_k = k.astype(np.float16).astype(np.float32)
    exp_k[13:16] = k2.astype(np.float16)
    exp_v = v.astype(np.float16).astype(np.float32)
    exp_v[13:16] = v2.astype(np.float16)
    assert np.array_equal(gk, exp_k) and np.array_equal(gv, exp_v)


# ---- attention ---------------------------------------------------------------------

def _attn_case(oracle, nh=4, nkv=2, dph=64, bs=16, L=77, M=1, seed=3, q_scale=1.0):
    rng = np.random.default_rng(seed)
    kv_dim = nkv * dph
    nblk = -(-(L + M) // bs)
    pool = 2 * nblk + 3
    m = oracle.PagedKVModel(1, kv_dim, nblk, bs, pool)
    m.set_block_table(0, rng.permutation(pool)[:nblk])
    kc, vc = W.context_kv(rng, L + M, kv_dim)
    m.write_fp16(0, kc, vc, 0)
    q = W.queries(rng, M, nh, dph) * np.float32(q_scale)
    K, V = m.gather(0, 0, L + M)
    return m, q, K, V


@pytest.mark.parametrize("nh,nkv,dph,bs", [(4, 2, 64, 16), (32, 8, 128, 16), (28, 4, 128, 32),
                                           (8, 8, 64, 8), (6, 1, 64, 1)])
def test_tiled_vs_bruteforce_vs_numpy_vs_torch(oracle, nh, nkv, dph, bs):
    M = 3
    m, q, K, V = _attn_case(oracle, nh, nkv, dph, bs, L=70, M=M)
    pos_base = 70
    tiled = m.attention(0, q, nh, nkv, dph, pos_base, mode="tiled")
    f64 = m.attention(0, q, nh, nkv, dph, pos_base, mode="f64")
    npy = oracle.attention_f64_np(q, K, V, nh, nkv, dph, pos_base)
    np.testing.assert_allclose(f64, npy, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(tiled, f64, rtol=1e-5, atol=2e-6)
    # torch SDPA, fp64 on the CPU, GQA by repeating KV heads
    G = nh // nkv
    for mq in range(M):
        Lq = pos_base + mq + 1
        qt = torch.from_numpy(q[mq].astype(np.float64)).view(nh, 1, dph)
        kt = torch.from_numpy(K[:Lq].astype(np.float64)).view(Lq, nkv, dph).permute(1, 0, 2)
        vt = torch.from_numpy(V[:Lq].astype(np.float64)).view(Lq, nkv, dph).permute(1, 0, 2)
        kt = kt.repeat_interleave(G, dim=0).contiguous()
        vt = vt.repeat_interleave(G, dim=0).contiguous()
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).reshape(-1).numpy()
        np.testing.assert_allclose(f64[mq], ref, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("nh,nkv,dph,bs,M", [(4, 2, 64, 16, 1), (32, 8, 128, 16, 5),
                                             (28, 4, 128, 32, 9), (6, 1, 64, 1, 3)])
def test_torch_cpu_baseline_matches_bruteforce(oracle, nh, nkv, dph, bs, M):
    """The benchmark's torch-CPU restatement (the timed CPU baseline) against
    the fp64 brute force, on the same fragmented pool; a planted K/V head
    mix-up (KV head h % nkv instead of h * nkv // nh) must fail."""
    m, q, K, V = _attn_case(oracle, nh, nkv, dph, bs, L=70, M=M)
    pos_base = 70
    f64 = m.attention(0, q, nh, nkv, dph, pos_base, mode="f64")
    pool = torch.from_numpy(m.pool.view(np.int16))
    table = torch.from_numpy(m.tables[0].astype(np.int64))
    got = oracle.attention_torch_cpu(pool, table, torch.from_numpy(q), nh, nkv, dph, bs,
                                     pos_base).numpy()
    np.testing.assert_allclose(got, f64, rtol=1e-5, atol=2e-6)
    if nkv > 1 and nh // nkv > 1:
        Kp = K.reshape(-1, nkv, dph)
        Vp = V.reshape(-1, nkv, dph)
        G = nh // nkv
        perm = [h % nkv for h in range(nh)]  # wrong head mapping
        Kw = np.stack([Kp[:, perm[g * G], :] for g in range(nkv)], axis=1).reshape(K.shape)
        Vw = np.stack([Vp[:, perm[g * G], :] for g in range(nkv)], axis=1).reshape(V.shape)
        bad = oracle.attention_f64_np(q, Kw, Vw, nh, nkv, dph, pos_base)
        assert not _close(got, bad)


def test_total_len_zero_gives_zeros(oracle):
    m, q, K, V = _attn_case(oracle)
    out = m.attention_one(0, q[0], 4, 2, 64, 0)
    assert not out.any()  # attention.h:120-126 (l = 0 -> inv = 0)


def test_single_key_returns_its_value(oracle):
    m, q, K, V = _attn_case(oracle, nh=4, nkv=2, dph=64)
    out = m.attention_one(0, q[0], 4, 2, 64, 1)
    for h in range(4):
        kvh = h * 2 // 4
        np.testing.assert_allclose(out[h * 64:(h + 1) * 64], V[0, kvh * 64:(kvh + 1) * 64],
                                   rtol=1e-6, atol=1e-7)


def test_uniform_logits_give_mean_of_values(oracle):
    m, q, K, V = _attn_case(oracle, nh=4, nkv=2, dph=64, L=50)
    zq = np.zeros_like(q[0])
    out = m.attention_one(0, zq, 4, 2, 64, 41)
    for h in range(4):
        kvh = h * 2 // 4
        np.testing.assert_allclose(out[h * 64:(h + 1) * 64],
                                   V[:41, kvh * 64:(kvh + 1) * 64].mean(axis=0), rtol=1e-5,
                                   atol=1e-6)


def test_one_hot_logits_select_one_value(oracle):
    """q aligned with one key and scaled up: softmax -> one-hot on that key."""
    rng = np.random.default_rng(9)
    dph, nkv, nh, L = 64, 1, 1, 40
    m = oracle.PagedKVModel(1, dph, 4, 16, 4)
    m.set_block_table(0, [2, 0, 3, 1])
    kc = np.zeros((L, dph), np.float16)
    kc[np.arange(L), np.arange(L) % dph] = 1.0  # orthogonal unit keys
    vc = rng.standard_normal((L, dph)).astype(np.float16)
    m.write_fp16(0, kc, vc, 0)
    j = 23
    q = np.zeros(dph, np.float32)
    q[j % dph] = 400.0  # logit gap 400/8 = 50 -> weight ratio e^-50
    out = m.attention_one(0, q, nh, nkv, dph, L)
    np.testing.assert_allclose(out, vc[j].astype(np.float32), rtol=1e-6, atol=1e-6)


def test_causal_window_equals_single_query_calls(oracle):
    M = 5
    m, q, K, V = _attn_case(oracle, nh=8, nkv=2, dph=64, L=60, M=M)
    win = m.attention(0, q, 8, 2, 64, 60, mode="tiled")
    for mq in range(M):
        one = m.attention_one(0, q[mq], 8, 2, 64, 60 + mq + 1)
        assert np.array_equal(win[mq], one)


def _close(a, b):
    return np.all(np.abs(a - b) <= ATOL + RTOL * np.abs(b))


def test_planted_mistakes_exceed_tolerance(oracle):
    """Mistakes a kernel could plausibly make, planted in a CPU restatement,
    must all fail the attention tolerance against the oracle."""
    nh, nkv, dph, pb, M = 8, 2, 64, 90, 3
    m, q, K, V = _attn_case(oracle, nh, nkv, dph, 16, L=pb, M=M, q_scale=2.0)
    ref = m.attention(0, q, nh, nkv, dph, pb, mode="f64")
    good = oracle.attention_f64_np(q, K, V, nh, nkv, dph, pb)
    assert _close(good, ref)

    def variant(kvh_map=None, scale=None, off=0, swap=False):
        Kx, Vx = (V, K) if swap else (K, V)
        qh = q.astype(np.float64).reshape(M, nh, dph)
        Kh = Kx.astype(np.float64).reshape(-1, nkv, dph)
        Vh = Vx.astype(np.float64).reshape(-1, nkv, dph)
        mp = kvh_map if kvh_map is not None else (np.arange(nh) * nkv) // nh
        sc = scale if scale is not None else 1 / np.sqrt(dph)
        out = np.zeros((M, nh, dph))
        for mq in range(M):
            L = pb + mq + 1 + off
            lg = np.einsum("hd,lhd->hl", qh[mq], Kh[:L, mp]) * sc
            w = np.exp(lg - lg.max(1, keepdims=True))
            w /= w.sum(1, keepdims=True)
            out[mq] = np.einsum("hl,lhd->hd", w, Vh[:L, mp])
        return out.reshape(M, -1)

    assert _close(variant(), ref)
    assert not _close(variant(kvh_map=np.arange(nh) % nkv), ref)  # h % nkv mapping
    assert not _close(variant(scale=1.0), ref)                      # scale dropped
    assert not _close(variant(scale=1 / dph), ref)                  # 1/d, not 1/sqrt(d)
    assert not _close(variant(off=-1), ref)                         # total_len off by one
    assert not _close(variant(swap=True), ref)                      # K and V regions swapped


def test_rope_rotate_half_is_a_rotation():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 4 * 64)).astype(np.float32)
    assert np.array_equal(W.rope_rotate_half(x, 4, 64, 0), x)  # angle 0
    y = W.rope_rotate_half(x, 4, 64, 129).reshape(4, 64).astype(np.float64)
    xr = x.reshape(4, 64).astype(np.float64)
    # as complex numbers z_j = x_j + i x_{j+32}, rotation by pos*theta^(-2j/64)
    z = xr[:, :32] + 1j * xr[:, 32:]
    ang = 129 * 10000.0 ** (-np.arange(32) * 2 / 64)
    zr = z * np.exp(1j * ang)
    np.testing.assert_allclose(y[:, :32], zr.real, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(y[:, 32:], zr.imag, rtol=1e-4, atol=1e-4)


# ---- golden fixtures -----------------------------------------------------------------

def test_tiny_decode_fixture_reproduces(oracle):
    g = np.load(GOLDEN / "tiny_decode.npz")
    w = W.CONFIGS["tiny"]
    m = oracle.PagedKVModel(w.n_layers, w.kv_dim, g["tables"].shape[1], w.block_size,
                            w.pool_blocks)
    for layer in range(w.n_layers):
        m.set_block_table(layer, g["tables"][layer])
        m.write_fp16(layer, g["ctx_k"][layer], g["ctx_v"][layer], 0)
        m.append(layer, g["new_k"][layer], g["new_v"][layer], w.ctx)
        tiled = m.attention(layer, g["q"][layer], w.nh, w.nkv, w.dph, w.ctx, mode="tiled")
        assert np.array_equal(tiled, g["out_tiled"][layer])
        f64 = m.attention(layer, g["q"][layer], w.nh, w.nkv, w.dph, w.ctx, mode="f64")
        np.testing.assert_allclose(f64, g["out_f64"][layer], rtol=1e-12, atol=1e-14)
    assert m.pool_sha256() == bytes(g["pool_sha256"]).hex()


@pytest.mark.parametrize("name", ["tiny", "llama3_8b_verify", "qwen25_7b_selfspec"])
def test_scripted_hashes_reproduce(oracle, name):
    spec = json.loads((GOLDEN / "scripted_hashes.json").read_text())[name]
    w = W.CONFIGS[name]
    tables, ops = W.scripted_rounds(w, spec["n_layers"], spec["rounds"],
                                    draft_layers=spec["draft_layers"])
    m = oracle.PagedKVModel(spec["n_layers"], w.kv_dim, tables.shape[1], w.block_size,
                            spec["pool_blocks"])
    for layer in range(spec["n_layers"]):
        m.set_block_table(layer, tables[layer])
    marks = oracle.run_script(m, ops)
    assert [(c["label"], c["seq_len"], c["sha256"]) for c in spec["checkpoints"]] == marks
    # rollback checkpoints: same bytes as the verify checkpoint before them
    for a, b in zip(marks, marks[1:]):
        if b[0].endswith("rollback"):
            assert a[2] == b[2] and b[1] <= a[1]


# ---- RoPE restatement (rope_apply_inplace, model.cu:281-323) ----------------

def _rope(oracle, x, nh, dph, pos, **kw):
    return oracle.rope_rotate_half_f64(x, nh, dph, pos, **kw)


def test_rope_f64_is_a_rotation_and_identity_at_zero(oracle):
    rng = np.random.default_rng(3)
    nh, dph = 4, 64
    x = rng.standard_normal((5, nh * dph))
    pos = np.array([0, 1, 17, 1000, 4095])
    y = _rope(oracle, x, nh, dph, pos)
    xr, yr = x.reshape(5, nh, 2, dph // 2), y.reshape(5, nh, 2, dph // 2)
    np.testing.assert_allclose((yr ** 2).sum(2), (xr ** 2).sum(2), rtol=1e-12)
    np.testing.assert_array_equal(y[0], x[0])


def test_rope_f64_first_pair_turns_by_the_position(oracle):
    # inv_freq[0] = 1: pair (0, dph/2) of every head turns by exactly pos radians
    dph = 128
    x = np.zeros((3, dph))
    x[:, 0] = 1.0
    pos = np.array([1, 7, 300])
    y = _rope(oracle, x, 1, dph, pos)
    np.testing.assert_allclose(y[:, 0], np.cos(pos), atol=1e-12)
    np.testing.assert_allclose(y[:, dph // 2], np.sin(pos), atol=1e-12)


def test_rope_f64_logits_depend_on_relative_position(oracle):
    # RoPE's defining property: <R(m) q, R(n) k> depends on m - n only
    rng = np.random.default_rng(4)
    dph = 128
    q, k = rng.standard_normal((1, dph)), rng.standard_normal((1, dph))
    def logit(m, n):
        return float((_rope(oracle, q, 1, dph, [m]) @ _rope(oracle, k, 1, dph, [n]).T)[0, 0])
    for m, n, s in [(10, 3, 100), (500, 499, 1000), (64, 0, 7)]:
        assert abs(logit(m, n) - logit(m + s, n + s)) < 2e-3 * (1 + abs(logit(m, n)))


def test_rope_f64_matches_the_fp32_restatement(oracle):
    from speculative_decode_engine_amd import workloads as W
    rng = np.random.default_rng(5)
    nh, dph = 2, 64
    x = rng.standard_normal((1, nh * dph)).astype(np.float32)
    for pos in [0, 3, 129, 2000]:
        a = _rope(oracle, x, nh, dph, [pos])
        b = W.rope_rotate_half(x, nh, dph, pos)
        np.testing.assert_allclose(a, b, atol=2e-4 * (1 + pos / 1000))


def test_rope_f64_scaling_modes(oracle):
    rng = np.random.default_rng(6)
    nh, dph = 2, 64
    x = rng.standard_normal((1, nh * dph))
    # linear and YaRN divide the position (exact here: 96 / 4 = 24)
    for t in (oracle.ROPE_LINEAR, oracle.ROPE_YARN):
        np.testing.assert_allclose(_rope(oracle, x, nh, dph, [96], scaling_type=t, factor=4.0),
                                   _rope(oracle, x, nh, dph, [24]), atol=1e-12)
    # NTK scales theta; a factor <= 1 changes nothing
    th = 10000.0 * 2.0 ** (dph / (dph - 2.0))
    np.testing.assert_allclose(oracle.rope_inv_freq(dph, 10000.0, oracle.ROPE_NTK, 2.0),
                               oracle.rope_inv_freq(dph, th), rtol=1e-6)
    np.testing.assert_array_equal(_rope(oracle, x, nh, dph, [50], scaling_type=oracle.ROPE_NTK,
                                        factor=1.0), _rope(oracle, x, nh, dph, [50]))
    # theta <= 1e-6 selects 10000 (model.cu:290)
    np.testing.assert_array_equal(oracle.rope_inv_freq(dph, 0.0), oracle.rope_inv_freq(dph))


def test_rope_f64_planted_interleaved_pairing_fails(oracle):
    # GPT-J pairing (2j, 2j+1) is not the reference's rotate-half pairing
    from speculative_decode_engine_amd import workloads as W
    rng = np.random.default_rng(7)
    dph = 64
    x = rng.standard_normal((1, dph)).astype(np.float32)
    perm = np.concatenate([np.arange(0, dph, 2), np.arange(1, dph, 2)])
    inter = np.empty(dph)
    inter[perm] = _rope(oracle, x[:, perm], 1, dph, [40])[0]
    assert np.abs(inter - W.rope_rotate_half(x, 1, dph, 40)[0]).max() > 1e-2


# ---- the output projection (Wo) -------------------------------------------------
# oracle_matvec restates device_matvec_partial(_accum) (utils.h:417-452) in C;
# it is pinned by closed forms (identity weights, one-hot inputs), by the
# float64 product, and by planted mistakes (transposed weights, dropped
# row) that the fp32-summation tolerance must catch.

MV_TOL = 1e-5  # x magnitude sum_r |x_r W_rc|: fp32 summation error bound used by the GPU tests


def _mv_case(rng, M, d_in, d_out):
    x = rng.standard_normal((M, d_in)).astype(np.float32)
    Wb = (rng.standard_normal((d_in, d_out)) * 0.05).astype(np.float16).view(np.uint16)
    return x, Wb


def test_matvec_identity_and_one_hot_are_exact(oracle):
    rng = np.random.default_rng(11)
    d = 96
    eye = np.eye(d, dtype=np.float16).view(np.uint16)
    x = rng.standard_normal((2, d)).astype(np.float32)
    assert np.array_equal(oracle.matvec_ref(x, eye), x)
    _, Wb = _mv_case(rng, 1, d, 40)
    for k in (0, 17, d - 1):
        e = np.zeros((1, d), np.float32)
        e[0, k] = 1.0
        got = oracle.matvec_ref(e, Wb)
        assert np.array_equal(got[0], Wb[k].view(np.float16).astype(np.float32))


def test_matvec_accumulate_adds_to_out(oracle):
    rng = np.random.default_rng(12)
    x, Wb = _mv_case(rng, 3, 130, 24)
    out0 = rng.standard_normal((3, 24)).astype(np.float32)
    prod = oracle.matvec_ref(x, Wb)
    acc = oracle.matvec_ref(x, Wb, out0, accumulate=True)
    assert np.array_equal(acc, out0 + prod)  # out[c] += acc: one fp32 add of the same acc
    y, mag = oracle.matvec_f64(x, Wb, out0)
    assert np.all(np.abs(acc - y) <= MV_TOL * mag)


@pytest.mark.parametrize("M,d_in,d_out", [(1, 1, 8), (1, 4096, 64), (9, 512, 48), (2, 1000, 16)])
def test_matvec_matches_float64(oracle, M, d_in, d_out):
    rng = np.random.default_rng(M * 1000 + d_in)
    x, Wb = _mv_case(rng, M, d_in, d_out)
    got = oracle.matvec_ref(x, Wb)
    y, mag = oracle.matvec_f64(x, Wb)
    assert np.all(np.abs(got - y) <= MV_TOL * mag + 1e-30)
    # Linearity in x (exact in float64 terms up to the same bound).
    got2 = oracle.matvec_ref(2.0 * x, Wb)
    assert np.array_equal(got2, 2.0 * got)  # scaling by 2 is exact in fp32


def test_matvec_planted_mistakes_exceed_tolerance(oracle):
    rng = np.random.default_rng(13)
    x, Wb = _mv_case(rng, 1, 256, 256)
    y, mag = oracle.matvec_f64(x, Wb)
    transposed = oracle.matvec_ref(x, np.ascontiguousarray(Wb.T))
    assert np.any(np.abs(transposed - y) > MV_TOL * mag)
    dropped = oracle.matvec_ref(x[:, :-1], np.ascontiguousarray(Wb[:-1]))
    assert np.any(np.abs(dropped - y) > MV_TOL * mag)
