"""The persistent speculative decoding loop (sde_spec_loop_greedy) from Python.

Reference (arkhamHack/speculative_decode_engine): megakernel_speculative,
cuda/src/kernels.cu:2864-3106 (loop) and 3593-3755 (host launcher), in its
self-speculative form (model.cu:838-890).  One cooperative launch runs every
round on the device: the first n_draft layers draft k tokens one at a time,
the remaining layers verify the window [last token, drafts], the leading
matches plus the target's next token are emitted, and seq_len rewinds to
save + n_accepted + 1.  k = 0 is plain greedy decoding.

The loop's model is the paged-KV path's: layer l of token t has q, k, v rows
emb_q/emb_k/emb_v[l][t] (q adds the previous layer's attention output of
the same row), and fp16 `head` weights [n_heads*head_dim][vocab] turn the
last layer's attention output into logits.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _native
from ._native import LoopModel, check
from .kv_cache import KVCache, _stream_handle

STATE_WORDS = 8


@dataclass
class LoopResult:
    tokens: list          # emitted tokens, in order (at least max_new)
    accepted: list        # drafts accepted per round
    rounds: int
    seq_len: int          # the cache's device seq_len afterwards
    status: int


class SpecLoopModel:
    """Device tensors of the loop's model: emb_q fp32 [L][V][nh*dph],
    emb_k / emb_v fp32 [L][V][kv_dim], head fp16 [nh*dph][V]."""

    def __init__(self, emb_q: torch.Tensor, emb_k: torch.Tensor, emb_v: torch.Tensor,
                 head: torch.Tensor, n_heads: int, n_kv_heads: int, head_dim: int):
        L, V, d = emb_q.shape
        if d != n_heads * head_dim:
            raise ValueError("emb_q rows must be n_heads * head_dim wide")
        kvd = n_kv_heads * head_dim
        for name, t, shape, dt in (("emb_q", emb_q, (L, V, d), torch.float32),
                                   ("emb_k", emb_k, (L, V, kvd), torch.float32),
                                   ("emb_v", emb_v, (L, V, kvd), torch.float32),
                                   ("head", head, (d, V), torch.float16)):
            if t.device.type != "cuda" or t.dtype != dt or not t.is_contiguous():
                raise TypeError(f"{name} must be a contiguous CUDA {dt} tensor")
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
        self.emb_q, self.emb_k, self.emb_v, self.head = emb_q, emb_k, emb_v, head
        self.n_layers, self.vocab = L, V
        self.c = LoopModel(emb_q.data_ptr(), emb_k.data_ptr(), emb_v.data_ptr(),
                           head.data_ptr(), V, n_heads, n_kv_heads, head_dim)


def workspace_size(cache: KVCache, model: SpecLoopModel, k: int) -> int:
    return int(_native.load().sde_spec_loop_workspace_size(cache.handle, ctypes.byref(model.c),
                                                           k))


def spec_loop_greedy(cache: KVCache, model: SpecLoopModel, anchor: int, k: int, n_draft: int,
                     max_new: int, stream: Optional[torch.cuda.Stream] = None,
                     workspace: Optional[torch.Tensor] = None) -> LoopResult:
    """Runs the loop from the cache's device seq_len (positions below it hold
    the context) with `anchor` the last emitted token; synchronizes and
    returns the emitted tokens and per-round acceptances."""
    dev = cache.device
    state = torch.zeros(STATE_WORDS, dtype=torch.int32, device=dev)
    state[0] = anchor
    emitted = torch.full((max(max_new + k, 1),), -1, dtype=torch.int32, device=dev)
    accepted = torch.full((max(max_new, 1),), -1, dtype=torch.int32, device=dev)
    if workspace is None:
        # (an invalid k gives size 0: the call below then reports the status)
        workspace = torch.empty(max(workspace_size(cache, model, k), 256), dtype=torch.uint8,
                                device=dev)
    lib = _native.load()
    check(lib.sde_spec_loop_greedy(
        cache.handle, ctypes.byref(model.c), k, n_draft, max_new,
        ctypes.c_void_p(state.data_ptr()), ctypes.c_void_p(emitted.data_ptr()),
        ctypes.c_void_p(accepted.data_ptr()), ctypes.c_void_p(workspace.data_ptr()),
        workspace.numel() * workspace.element_size(), _stream_handle(stream)),
        "spec_loop_greedy")
    torch.cuda.synchronize(dev)
    st = state.cpu().tolist()
    n = st[1]
    rounds = st[2]
    return LoopResult(tokens=emitted[:n].cpu().tolist(),
                      accepted=accepted[:rounds].cpu().tolist(), rounds=rounds,
                      seq_len=cache.device_seq_len(), status=st[3])
