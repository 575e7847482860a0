"""ctypes binding of libsde_paged.so (the C-ABI of include/sde_paged_kv.h).

torch is imported before the library is loaded: both the library and torch
need libamdhip64.so.7, and loading torch's copy first makes the library bind
to it, so device pointers and hipStream_t handles from torch are valid here.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch  # noqa: F401  (see module docstring: load order matters)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libsde_paged.so"
HEADER_PATH = PKG_DIR.parent / "include" / "sde_paged_kv.h"

SDE_OK = 0
SDE_ERR_INVALID_ARGUMENT = 1
SDE_ERR_CAPACITY = 2
SDE_ERR_RANGE = 3
SDE_ERR_UNSUPPORTED = 4
SDE_ERR_WORKSPACE = 5
SDE_ERR_HIP = 6
SDE_ERR_NO_DEVICE = 7
SDE_ERR_IO = 8
SDE_ERR_FORMAT = 9

# SDE_NOALLOC_SCRATCH_BYTES: sde_paged_attention_noalloc's static partials array
NOALLOC_SCRATCH_BYTES = 4 << 20

SDE_ATTN_SOFTMAX = 0
SDE_ATTN_SLIDING_WINDOW = 1
SDE_ATTN_KDA = 2
SDE_ATTN_LINEAR = 3

SDE_ROPE_NONE = 0
SDE_ROPE_LINEAR = 1
SDE_ROPE_NTK = 2
SDE_ROPE_YARN = 3


class KVConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int32),
        ("kv_dim", ctypes.c_int32),
        ("max_blocks_per_layer", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("pool_blocks", ctypes.c_int32),
    ]


class RopeConfig(ctypes.Structure):
    _fields_ = [
        ("theta", ctypes.c_float),
        ("scaling_type", ctypes.c_int32),
        ("scaling_factor", ctypes.c_float),
    ]


class KVView(ctypes.Structure):
    _fields_ = [
        ("pool", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_len", ctypes.c_void_p),
        ("n_layers", ctypes.c_int32),
        ("kv_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_layer", ctypes.c_int32),
        ("pool_blocks", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class ModelConfig(ctypes.Structure):
    """sde_model_config: ModelConfig (config.h:67-83) + the SDEC version."""
    _fields_ = [
        ("n_layers", ctypes.c_int32),
        ("d_model", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("d_ff", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
        ("rope_scaling_type", ctypes.c_int32),
        ("rope_scaling_factor", ctypes.c_float),
        ("attention_type", ctypes.c_int32),
        ("has_qkv_bias", ctypes.c_int32),
        ("version", ctypes.c_uint32),
    ]


LAYER_TENSORS = ("rms_attn_weight", "Wq", "Wk", "Wv", "Wo", "rms_mlp_weight", "W_gate", "W_up",
                 "W_down", "Wq_bias", "Wk_bias", "Wv_bias")
GLOBAL_TENSORS = ("token_embedding", "rms_final_weight", "output_proj")


class LoopModel(ctypes.Structure):
    """sde_loop_model: the persistent loop's embedding tables and head."""
    _fields_ = [
        ("emb_q", ctypes.c_void_p),
        ("emb_k", ctypes.c_void_p),
        ("emb_v", ctypes.c_void_p),
        ("head", ctypes.c_void_p),
        ("vocab", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
    ]


class LoopSampling(ctypes.Structure):
    """sde_loop_sampling: the stochastic loop's temperature schedule and seed."""
    _fields_ = [
        ("draft_temp", ctypes.c_float),
        ("adaptive", ctypes.c_int32),
        ("min_temp", ctypes.c_float),
        ("max_temp", ctypes.c_float),
        ("target_accept", ctypes.c_float),
        ("gain", ctypes.c_float),
        ("ewma_mix", ctypes.c_float),
        ("seed", ctypes.c_uint64),
    ]


class LayerWeights(ctypes.Structure):
    """sde_layer_weights: device pointers (model.h:32-47)."""
    _fields_ = [(n, ctypes.c_void_p) for n in LAYER_TENSORS]


class ModelGlobals(ctypes.Structure):
    """sde_model_globals: device pointers (model.h:49-55)."""
    _fields_ = [(n, ctypes.c_void_p) for n in GLOBAL_TENSORS]


class LoopConfig(ctypes.Structure):
    """sde_spec_loop_config: GenerationParams' spec_k, max_new_tokens, eos_token
    and self_speculative (config.h:139-160); the draft cache handle and draft
    model (NULL: self-speculative)."""
    _fields_ = [
        ("k", ctypes.c_int32),
        ("n_draft", ctypes.c_int32),
        ("max_new", ctypes.c_int32),
        ("eos_token", ctypes.c_int32),
        ("draft_cache", ctypes.c_void_p),
        ("draft_model", ctypes.POINTER(LoopModel)),
    ]


_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_cfg_p = ctypes.POINTER(KVConfig)
_i32_p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); must match include/sde_paged_kv.h
PROTOTYPES = {
    "sde_status_string": (ctypes.c_char_p, [_c_int]),
    "sde_kv_config_validate": (_c_int, [_cfg_p]),
    "sde_kv_pool_bytes": (_sz, [_cfg_p]),
    "sde_kv_cache_create": (_c_int, [_cfg_p, ctypes.POINTER(_vp)]),
    "sde_kv_cache_create_external": (_c_int, [_cfg_p, _vp, _sz, ctypes.POINTER(_vp)]),
    "sde_kv_cache_destroy": (_c_int, [_vp]),
    "sde_kv_reset": (_c_int, [_vp, _vp]),
    "sde_kv_set_block_table": (_c_int, [_vp, _c_int, _i32_p, _c_int]),
    "sde_kv_get_block_table": (_c_int, [_vp, _c_int, _i32_p, _c_int]),
    "sde_kv_seq_len": (_c_int, [_vp, ctypes.POINTER(_c_int)]),
    "sde_kv_device_seq_len": (_c_int, [_vp, ctypes.POINTER(_c_int)]),
    "sde_kv_set_seq_len": (_c_int, [_vp, _c_int, _vp]),
    "sde_kv_rollback": (_c_int, [_vp, _c_int, _vp]),
    "sde_kv_append": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _vp]),
    "sde_kv_write_fp16": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _vp]),
    "sde_kv_gather": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "sde_kv_get_view": (_c_int, [_vp, ctypes.POINTER(KVView)]),
    "sde_paged_attention_workspace_size": (_sz, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "sde_grid_attention_workspace_size": (_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "sde_paged_attention": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                     _c_int, _vp, _sz, _vp]),
    "sde_paged_attention_noalloc": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _vp]),
    "sde_debug_set_slice_spin": (ctypes.c_uint32, [ctypes.c_uint32]),
    "sde_debug_attention_plan": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_int, ctypes.POINTER(ctypes.c_int32)]),
    "sde_spec_accept_stochastic": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                            ctypes.c_float, ctypes.c_float, ctypes.c_uint64, _vp,
                                            _c_int, _c_int, _vp, _vp]),
    "sde_spec_accept_greedy": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "sde_rope_append_attention": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                           _c_int, _c_int, _c_int, _vp, _vp, _sz, _vp]),
    "sde_attention_dispatch": (_c_int, [_c_int, _vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int,
                                        _c_int, _c_int, _vp, _sz, _vp]),
    "sde_matvec_workspace_size": (_sz, [_c_int, _c_int, _c_int]),
    "sde_model_read_header": (_c_int, [ctypes.c_char_p, ctypes.POINTER(ModelConfig)]),
    "sde_model_weights_bytes": (_sz, [ctypes.POINTER(ModelConfig)]),
    "sde_model_load": (_c_int, [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(ModelConfig)]),
    "sde_model_get_config": (_c_int, [_vp, ctypes.POINTER(ModelConfig)]),
    "sde_model_get_layer": (_c_int, [_vp, _c_int, ctypes.POINTER(LayerWeights)]),
    "sde_model_get_globals": (_c_int, [_vp, ctypes.POINTER(ModelGlobals)]),
    "sde_model_free": (_c_int, [_vp]),
    "sde_matvec": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _sz, _vp]),
    "sde_matvec_packed_size": (_sz, [_c_int, _c_int]),
    "sde_matvec_pack": (_c_int, [_vp, _c_int, _c_int, _vp, _sz, _vp]),
    "sde_matvec_packed": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "sde_spec_loop_workspace_size": (_sz, [_vp, ctypes.POINTER(LoopModel), _c_int]),
    "sde_spec_loop_greedy": (_c_int, [_vp, ctypes.POINTER(LoopModel), _c_int, _c_int, _c_int,
                                      _vp, _vp, _vp, _vp, _sz, _vp]),
    "sde_spec_loop_stochastic": (_c_int, [_vp, ctypes.POINTER(LoopModel), _c_int, _c_int,
                                          _c_int, ctypes.POINTER(LoopSampling), _vp, _vp, _vp,
                                          _vp, _vp, _sz, _vp]),
    "sde_spec_loop_config_workspace_size": (_sz, [_vp, ctypes.POINTER(LoopModel),
                                                  ctypes.POINTER(LoopConfig)]),
    "sde_spec_loop": (_c_int, [_vp, ctypes.POINTER(LoopModel), ctypes.POINTER(LoopConfig),
                               ctypes.POINTER(LoopSampling), _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
}

_LIB = None


class SDEError(RuntimeError):
    """A non-zero sde_status returned by the library."""

    def __init__(self, status: int, where: str):
        self.status = status
        msg = status_string(status) if _LIB is not None else str(status)
        super().__init__(f"{where}: {msg} (status {status})")


def header_functions(header: Path = HEADER_PATH) -> list[str]:
    """Names of the functions declared in the C-ABI header."""
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sde_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    """Loads libsde_paged.so (built by __graft_entry__.build()); fails loudly."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def status_string(status: int) -> str:
    return load().sde_status_string(status).decode()


def check(status: int, where: str) -> None:
    if status != SDE_OK:
        raise SDEError(status, where)


def hip_runtime_paths() -> list[str]:
    """Paths of every libamdhip64 mapped into this process (expect one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    return sorted(paths)
