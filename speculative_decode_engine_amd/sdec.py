"""SDEC weight files: the loader of libsde_paged (sde_model_* in
include/sde_paged_kv.h, the reference's model_load_weights, model.cu:68-260)
and a writer of the same format (tools/export_model.py:19-35, 170-210 writes
it from HuggingFace checkpoints; this one writes numpy arrays, for tests and
conversions).

File layout: "SDEC", uint32 version (1-5), then uint32 n_layers, d_model,
n_heads, [n_kv_heads (v3+)], d_ff, vocab_size, [float32 rope_theta (v2+)],
[int32 rope_scaling_type, float32 rope_scaling_factor (v3+)],
[int32 attention_type (v4+)], [int32 has_qkv_bias (v5)]; then each tensor
as a uint32 element count followed by that many fp16 values, in the order
token_embedding [V][d], rms_final_weight [d], output_proj [d][V], and per
layer rms_attn [d], Wq [d][d], Wk [d][kv], Wv [d][kv], Wo [d][d], rms_mlp
[d], W_gate [d][ff], W_up [d][ff], W_down [ff][d] (+ Wq_bias [d], Wk_bias
[kv], Wv_bias [kv] when has_qkv_bias).  Versions 1-2 store Wk/Wv expanded
to [d][d] (n_kv_heads = n_heads)."""
from __future__ import annotations

import ctypes
import struct
from pathlib import Path
from typing import Dict, Mapping, Optional

import numpy as np
import torch

from . import _native
from ._native import GLOBAL_TENSORS, LAYER_TENSORS, LayerWeights, ModelConfig, ModelGlobals, check

CONFIG_FIELDS = ("n_layers", "d_model", "n_heads", "n_kv_heads", "d_ff", "vocab_size",
                 "rope_theta", "rope_scaling_type", "rope_scaling_factor", "attention_type",
                 "has_qkv_bias", "version")


def _cfg_dict(c: ModelConfig) -> dict:
    return {f: getattr(c, f) for f in CONFIG_FIELDS}


def kv_dim(cfg: Mapping) -> int:
    return cfg["n_kv_heads"] * (cfg["d_model"] // cfg["n_heads"])


def tensor_shapes(cfg: Mapping) -> Dict[str, tuple]:
    """name -> shape of every tensor of a file, in file order ("L{l}.name"
    for layer tensors)."""
    d, ff, V, kd = cfg["d_model"], cfg["d_ff"], cfg["vocab_size"], kv_dim(cfg)
    out = {"token_embedding": (V, d), "rms_final_weight": (d,), "output_proj": (d, V)}
    for l in range(cfg["n_layers"]):
        out.update({f"L{l}.rms_attn_weight": (d,), f"L{l}.Wq": (d, d), f"L{l}.Wk": (d, kd),
                    f"L{l}.Wv": (d, kd), f"L{l}.Wo": (d, d), f"L{l}.rms_mlp_weight": (d,),
                    f"L{l}.W_gate": (d, ff), f"L{l}.W_up": (d, ff), f"L{l}.W_down": (ff, d)})
        if cfg.get("has_qkv_bias"):
            out.update({f"L{l}.Wq_bias": (d,), f"L{l}.Wk_bias": (kd,), f"L{l}.Wv_bias": (kd,)})
    return out


def write_sdec(path, cfg: Mapping, tensors: Mapping[str, np.ndarray], version: int = 5) -> None:
    """Writes an SDEC file of `version` from fp16-convertible arrays named
    as tensor_shapes(cfg).  Versions 1-2 need n_kv_heads == n_heads."""
    if not 1 <= version <= 5:
        raise ValueError("SDEC versions are 1..5")
    if version <= 2 and cfg["n_kv_heads"] != cfg["n_heads"]:
        raise ValueError("SDEC v1/v2 store expanded K/V (n_kv_heads == n_heads)")
    shapes = tensor_shapes(dict(cfg, has_qkv_bias=cfg.get("has_qkv_bias", 0) if version >= 5
                                else 0))
    with open(path, "wb") as f:
        f.write(b"SDEC")
        f.write(struct.pack("<I", version))
        if version <= 2:
            f.write(struct.pack("<5I", cfg["n_layers"], cfg["d_model"], cfg["n_heads"],
                                cfg["d_ff"], cfg["vocab_size"]))
        else:
            f.write(struct.pack("<6I", cfg["n_layers"], cfg["d_model"], cfg["n_heads"],
                                cfg["n_kv_heads"], cfg["d_ff"], cfg["vocab_size"]))
        if version >= 2:
            f.write(struct.pack("<f", cfg.get("rope_theta", 10000.0)))
        if version >= 3:
            f.write(struct.pack("<if", cfg.get("rope_scaling_type", 0),
                                cfg.get("rope_scaling_factor", 1.0)))
        if version >= 4:
            f.write(struct.pack("<i", cfg.get("attention_type", 0)))
        if version >= 5:
            f.write(struct.pack("<i", 1 if cfg.get("has_qkv_bias") else 0))
        for name, shape in shapes.items():
            a = np.ascontiguousarray(np.asarray(tensors[name]).astype(np.float16))
            if a.shape != tuple(shape):
                raise ValueError(f"{name}: shape {a.shape}, expected {shape}")
            f.write(struct.pack("<I", a.size))
            f.write(a.tobytes())


def read_header(path) -> dict:
    """sde_model_read_header: the validated header as a dict."""
    c = ModelConfig()
    check(_native.load().sde_model_read_header(str(path).encode(), ctypes.byref(c)),
          "sde_model_read_header")
    return _cfg_dict(c)


def weights_bytes(cfg: Mapping) -> int:
    c = ModelConfig(**{f: cfg.get(f, 0) for f in CONFIG_FIELDS})
    return int(_native.load().sde_model_weights_bytes(ctypes.byref(c)))


class _DevArray:
    """A device fp16 buffer viewed through __cuda_array_interface__."""

    def __init__(self, ptr: int, shape: tuple):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": "<f2",
                                         "data": (ptr, False), "version": 2}


class SDECModel:
    """The weights of an SDEC file on the current GPU (sde_model_load).
    Tensors are zero-copy torch views into the model's device arena; they
    are valid until free()."""

    def __init__(self, path):
        self._lib = _native.load()
        self.handle = ctypes.c_void_p()
        c = ModelConfig()
        check(self._lib.sde_model_load(str(Path(path)).encode(), ctypes.byref(self.handle),
                                       ctypes.byref(c)), "sde_model_load")
        self.config = _cfg_dict(c)

    def _view(self, ptr: Optional[int], shape: tuple) -> Optional[torch.Tensor]:
        if not ptr:
            return None
        return torch.as_tensor(_DevArray(ptr, shape), device="cuda")

    def layer(self, l: int) -> Dict[str, Optional[torch.Tensor]]:
        w = LayerWeights()
        check(self._lib.sde_model_get_layer(self.handle, l, ctypes.byref(w)),
              "sde_model_get_layer")
        shapes = tensor_shapes(self.config)
        return {n: self._view(getattr(w, n), shapes.get(f"L{l}.{n}", (0,)))
                for n in LAYER_TENSORS}

    def globals(self) -> Dict[str, torch.Tensor]:
        g = ModelGlobals()
        check(self._lib.sde_model_get_globals(self.handle, ctypes.byref(g)),
              "sde_model_get_globals")
        shapes = tensor_shapes(self.config)
        return {n: self._view(getattr(g, n), shapes[n]) for n in GLOBAL_TENSORS}

    def free(self) -> None:
        if self.handle:
            check(self._lib.sde_model_free(self.handle), "sde_model_free")
            self.handle = ctypes.c_void_p()


def load_sdec(path) -> SDECModel:
    """model_load_weights (model.cu:83-260)."""
    return SDECModel(path)
