"""The SDEC header reader (sde_model_read_header, host only) against files
of every version written by speculative_decode_engine_amd.sdec.write_sdec,
byte-for-byte against the layout of model.cu:68-179 /
tools/export_model.py:19-35, and its rejections (model.cu:89-192)."""
import struct

import numpy as np
import pytest

from speculative_decode_engine_amd import _native as N
from speculative_decode_engine_amd import sdec

CFG = dict(n_layers=2, d_model=64, n_heads=4, n_kv_heads=2, d_ff=96, vocab_size=40,
           rope_theta=500000.0, rope_scaling_type=1, rope_scaling_factor=2.0,
           attention_type=0, has_qkv_bias=1)


def random_tensors(cfg, seed=0):
    rng = np.random.default_rng(seed)
    return {n: rng.standard_normal(s).astype(np.float16)
            for n, s in sdec.tensor_shapes(cfg).items()}


def cfg_for(version):
    c = dict(CFG)
    if version <= 2:
        c["n_kv_heads"] = c["n_heads"]
    if version < 5:
        c["has_qkv_bias"] = 0
    return c


@pytest.mark.parametrize("version", [1, 2, 3, 4, 5])
def test_header_round_trip(tmp_path, version):
    c = cfg_for(version)
    p = tmp_path / f"m{version}.sdec"
    sdec.write_sdec(p, c, random_tensors(c), version)
    h = sdec.read_header(p)
    assert h["version"] == version
    for k in ("n_layers", "d_model", "n_heads", "n_kv_heads", "d_ff", "vocab_size"):
        assert h[k] == c[k], k
    assert h["rope_theta"] == (c["rope_theta"] if version >= 2 else 10000.0)
    assert h["rope_scaling_type"] == (c["rope_scaling_type"] if version >= 3 else 0)
    assert h["rope_scaling_factor"] == (c["rope_scaling_factor"] if version >= 3 else 1.0)
    assert h["has_qkv_bias"] == (1 if version >= 5 else 0)


def test_writer_layout_matches_the_format(tmp_path):
    """Header bytes and the first tensor record of a v5 file, packed by hand
    from the documented layout (export_model.py:177-186, 66-74)."""
    c = cfg_for(5)
    t = random_tensors(c, 3)
    p = tmp_path / "m.sdec"
    sdec.write_sdec(p, c, t, 5)
    raw = p.read_bytes()
    head = b"SDEC" + struct.pack("<IIIIIIIfifii", 5, 2, 64, 4, 2, 96, 40, 500000.0, 1, 2.0, 0, 1)
    assert raw[:len(head)] == head
    first = struct.pack("<I", 40 * 64) + t["token_embedding"].tobytes()
    assert raw[len(head):len(head) + len(first)] == first
    total = len(head) + sum(4 + a.size * 2 for a in t.values())
    assert len(raw) == total


def _mutated(tmp_path, name, fn):
    c = cfg_for(5)
    p = tmp_path / "ok.sdec"
    sdec.write_sdec(p, c, random_tensors(c), 5)
    raw = bytearray(p.read_bytes())
    fn(raw)
    q = tmp_path / name
    q.write_bytes(bytes(raw))
    return q


def test_header_rejections(tmp_path):
    lib = N.load()
    cfg = N.ModelConfig()
    def st(path):
        return lib.sde_model_read_header(str(path).encode(), cfg)
    assert st(tmp_path / "missing.sdec") == N.SDE_ERR_IO
    assert st(_mutated(tmp_path, "magic", lambda r: r.__setitem__(slice(0, 4), b"SDEX"))) == N.SDE_ERR_FORMAT
    assert st(_mutated(tmp_path, "v0", lambda r: r.__setitem__(slice(4, 8), struct.pack("<I", 0)))) == N.SDE_ERR_FORMAT
    assert st(_mutated(tmp_path, "v6", lambda r: r.__setitem__(slice(4, 8), struct.pack("<I", 6)))) == N.SDE_ERR_FORMAT
    trunc = tmp_path / "trunc.sdec"
    trunc.write_bytes(_mutated(tmp_path, "t", lambda r: None).read_bytes()[:20])
    assert st(trunc) == N.SDE_ERR_IO
    # n_layers > MAX_LAYERS (40), d_model % n_heads, n_heads % n_kv_heads, zero heads
    for name, off, val in (("layers", 8, 41), ("dmodel", 12, 66), ("kv", 20, 3), ("h0", 16, 0),
                           ("kv0", 20, 0)):
        q = _mutated(tmp_path, name, lambda r, o=off, v=val: r.__setitem__(slice(o, o + 4),
                                                                            struct.pack("<I", v)))
        assert st(q) == N.SDE_ERR_FORMAT, name
    assert lib.sde_model_read_header(None, cfg) == N.SDE_ERR_INVALID_ARGUMENT


def test_weights_bytes_is_the_aligned_sum():
    for v in (1, 3, 5):
        c = cfg_for(v)
        want = sum(-(-int(np.prod(s)) * 2 // 256) * 256 for s in sdec.tensor_shapes(c).values())
        assert sdec.weights_bytes(dict(c, version=v)) == want
    assert sdec.weights_bytes(dict(CFG, n_heads=0)) == 0
    # A 2^30 x 2^30 embedding has more elements than the file's uint32 count
    # can state: rejected before any arena is sized from it.
    huge = dict(CFG, d_model=1 << 30, n_heads=1, n_kv_heads=1, vocab_size=1 << 30)
    assert sdec.weights_bytes(huge) == 0
