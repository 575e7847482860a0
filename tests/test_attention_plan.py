"""CPU checks of the tile path's partition plans (sde_debug_attention_plan,
host arithmetic only): over decode, verify and long-context shapes, device
sizes and context lengths around tile and partition boundaries, every plan
has the properties the kernels rely on --

  * rows per group 2, 4, 8 or 16, and the row groups cover the rows;
  * 1-4 tiles per wave in flight, whole chunks per partition;
  * the partitions cover the context's tiles: each is nonempty and the
    tiles past the whole partitions are at most one per wave (the kernel
    gives them to the first partition);
  * at most one workgroup per compute unit unless the (KV head, row group)
    units alone outnumber the units, and at most 64 partitions (the
    combine's buckets);
  * the workspace sized for a maximum length holds the partials of every
    shorter call (the partition count never exceeds the bound of the
    maximum)."""
import ctypes

import pytest

from speculative_decode_engine_amd import _native as N

TILE = 32
WAVES = 8


@pytest.fixture(scope="module")
def lib():
    return N.load()


def plan(lib, total_len, nkv, rows, n_cus):
    out = (ctypes.c_int32 * 6)()
    assert lib.sde_debug_attention_plan(total_len, nkv, rows, n_cus, out) == N.SDE_OK
    return tuple(out)


def lengths():
    base = [1, 2, 31, 32, 33, 100, 257, 1000, 2049, 4096, 4097, 4101, 8192, 8193, 8201,
            16384, 16385, 16389, 17005, 32768, 32769, 65536, 131072]
    return sorted(set(base + [n * TILE * WAVES + d for n in (1, 3, 16, 64, 128)
                              for d in (-1, 0, 1, 8, 9)]))


SHAPES = [(nkv, rows) for nkv in (1, 2, 4, 8, 16) for rows in (1, 2, 3, 4, 5, 7, 8, 9, 12,
                                                              16, 20, 36, 40, 63, 64)]


@pytest.mark.parametrize("n_cus", [256, 304, 80, 8])
def test_plan_properties(lib, n_cus):
    for L in lengths():
        for nkv, rows in SHAPES:
            rpw, groups, chunk, tpp, parts, bound = plan(lib, L, nkv, rows, n_cus)
            what = f"L={L} nkv={nkv} rows={rows} cus={n_cus}: {rpw, groups, chunk, tpp, parts}"
            assert rpw in (2, 4, 8, 16), what
            assert groups == -(-rows // rpw), what
            assert 1 <= chunk <= 4 and tpp % (WAVES * chunk) == 0, what
            n_tiles = -(-L // TILE)
            extra = n_tiles - parts * tpp
            # nonempty partitions; at most one extra tile per wave
            assert -tpp < extra <= WAVES, what
            units = nkv * groups
            assert 1 <= parts <= 64, what
            assert units * parts <= max(n_cus, units), what
            assert parts <= bound, what


@pytest.mark.parametrize("max_len", [4101, 8201, 32768, 131072])
def test_workspace_bound_covers_shorter_calls(lib, max_len):
    bound = plan(lib, max_len, 8, 4, 256)[5]
    for L in range(1, max_len + 1, 97):
        for nkv, rows in ((8, 4), (8, 20), (4, 63), (4, 8), (2, 2)):
            assert plan(lib, L, nkv, rows, 256)[4] <= bound, (L, nkv, rows)


def test_benchmark_shapes_take_the_documented_plans(lib):
    # (rows per group, row groups, chunk, tiles per partition, partitions)
    assert plan(lib, 32768, 8, 4, 256)[:5] == (4, 1, 4, 32, 32)      # 32K decode
    assert plan(lib, 4097, 8, 4, 256)[:5] == (4, 1, 1, 8, 17)        # 4K decode
    assert plan(lib, 4101, 8, 20, 256)[:5] == (8, 3, 2, 16, 9)       # 4K 5-query window
    assert plan(lib, 8201, 4, 63, 256)[:5] == (16, 4, 2, 16, 16)     # Qwen2.5-7B window
    assert plan(lib, 8193, 4, 7, 256)[:5] == (8, 1, 1, 8, 33)        # its draft step
    assert plan(lib, 2049, 4, 8, 256)[:5] == (2, 4, 1, 8, 9)         # TinyLlama decode


def test_invalid_sizes_rejected(lib):
    out = (ctypes.c_int32 * 6)()
    assert lib.sde_debug_attention_plan(0, 8, 4, 256, out) == N.SDE_ERR_INVALID_ARGUMENT
    assert lib.sde_debug_attention_plan(100, 0, 4, 256, out) == N.SDE_ERR_INVALID_ARGUMENT
    assert lib.sde_debug_attention_plan(100, 8, 0, 256, out) == N.SDE_ERR_INVALID_ARGUMENT
    assert lib.sde_debug_attention_plan(100, 8, 4, 0, out) == N.SDE_ERR_INVALID_ARGUMENT
    assert lib.sde_debug_attention_plan(100, 8, 4, 256, None) == N.SDE_ERR_INVALID_ARGUMENT
