"""The persistent speculative decoding loops (sde_spec_loop_greedy,
sde_spec_loop_stochastic) from Python.

Reference (arkhamHack/speculative_decode_engine): megakernel_speculative,
cuda/src/kernels.cu:2864-3106 (loop) and 3593-3755 (host launcher), in its
self-speculative form (model.cu:838-890).  One cooperative launch runs every
round on the device: the first n_draft layers draft k tokens one at a time,
the remaining layers verify the window [last token, drafts], the leading
matches plus the target's next token are emitted, and seq_len rewinds to
save + n_accepted + 1.  k = 0 is plain greedy decoding.  The stochastic
loop (megakernel_speculative_stochastic_kernel, kernels.cu:3108-3481)
samples the drafts at a draft temperature and accepts by speculative
sampling; k = 0 is plain sampling at temperature 1.  Both loops also take a
separate draft model over a cache of its own (the megakernel's
self_speculative false: draft rewind to draft_save + n_accepted and the
catch-up forward, kernels.cu:3066-3095) and an EOS token that ends the loop.

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
from ._native import LoopConfig, LoopModel, LoopSampling, check
from .kv_cache import KVCache, _stream_handle

STATE_WORDS = 8


@dataclass
class LoopResult:
    tokens: list          # emitted tokens, in order (at least max_new)
    accepted: list        # drafts accepted per round
    rounds: int
    seq_len: int          # the cache's device seq_len afterwards
    status: int
    draft_temp: float = 0.0   # stochastic loop: the final draft temperature
    accept_ewma: float = -1.0  # stochastic loop: the acceptance-rate average (< 0: none)
    draft_seq_len: Optional[int] = None  # the draft cache's device seq_len (draft model only)


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


def _check_anchor(model: SpecLoopModel, anchor: int) -> None:
    # The anchor indexes the embedding tables (the device also rejects it,
    # with SDE_ERR_INVALID_ARGUMENT in the status word).
    if not 0 <= int(anchor) < model.vocab:
        raise ValueError(f"anchor token {anchor} is outside the vocabulary [0, {model.vocab})")


def workspace_size(cache: KVCache, model: SpecLoopModel, k: int,
                   draft_cache: Optional[KVCache] = None,
                   draft_model: Optional[SpecLoopModel] = None) -> int:
    lib = _native.load()
    if draft_cache is None and draft_model is None:
        return int(lib.sde_spec_loop_workspace_size(cache.handle, ctypes.byref(model.c), k))
    cfg = _config(k, 0, 1, -1, draft_cache, draft_model)
    return int(lib.sde_spec_loop_config_workspace_size(cache.handle, ctypes.byref(model.c),
                                                       ctypes.byref(cfg)))


def _config(k, n_draft, max_new, eos_token, draft_cache, draft_model) -> LoopConfig:
    return LoopConfig(k, n_draft, max_new, eos_token,
                      draft_cache.handle if draft_cache is not None else None,
                      ctypes.pointer(draft_model.c) if draft_model is not None else None)


def _run(cache, model, anchor, k, n_draft, max_new, eos_token, draft_cache, draft_model,
         smp, offset, stream, workspace, what) -> LoopResult:
    _check_anchor(model, anchor)
    if (draft_cache is None) != (draft_model is None):
        raise ValueError("a draft model needs its own draft cache, and the reverse")
    dev = cache.device
    state = torch.zeros(STATE_WORDS, dtype=torch.int32, device=dev)
    state[0] = anchor
    emitted = torch.full((max(max_new + k, 1),), -1, dtype=torch.int32, device=dev)
    accepted = torch.full((max(max_new, 1),), -1, dtype=torch.int32, device=dev)
    if workspace is None:
        # (an invalid configuration gives size 0: the call then reports the status)
        workspace = torch.empty(max(workspace_size(cache, model, k, draft_cache, draft_model),
                                    256), dtype=torch.uint8, device=dev)
    ws = (ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size())
    bufs = (ctypes.c_void_p(state.data_ptr()), ctypes.c_void_p(emitted.data_ptr()),
            ctypes.c_void_p(accepted.data_ptr()))
    off = ctypes.c_void_p(offset.data_ptr()) if offset is not None else None
    lib = _native.load()
    if draft_cache is not None or eos_token >= 0:
        cfg = _config(k, n_draft, max_new, eos_token, draft_cache, draft_model)
        st = lib.sde_spec_loop(cache.handle, ctypes.byref(model.c), ctypes.byref(cfg),
                               ctypes.byref(smp) if smp is not None else None, off, *bufs, *ws,
                               _stream_handle(stream))
    elif smp is None:
        st = lib.sde_spec_loop_greedy(cache.handle, ctypes.byref(model.c), k, n_draft, max_new,
                                      *bufs, *ws, _stream_handle(stream))
    else:
        st = lib.sde_spec_loop_stochastic(cache.handle, ctypes.byref(model.c), k, n_draft,
                                          max_new, ctypes.byref(smp), off, *bufs, *ws,
                                          _stream_handle(stream))
    check(st, what)
    torch.cuda.synchronize(dev)
    words = state.cpu()
    n, rounds = int(words[1]), int(words[2])
    fl = words[6:8].view(torch.float32).tolist()
    return LoopResult(tokens=emitted[:n].cpu().tolist(),
                      accepted=accepted[:rounds].cpu().tolist(), rounds=rounds,
                      seq_len=cache.device_seq_len(), status=int(words[3]),
                      draft_temp=fl[0] if smp is not None else 0.0,
                      accept_ewma=fl[1] if smp is not None else -1.0,
                      draft_seq_len=draft_cache.device_seq_len() if draft_cache is not None
                      else None)


def spec_loop_greedy(cache: KVCache, model: SpecLoopModel, anchor: int, k: int, n_draft: int,
                     max_new: int, stream: Optional[torch.cuda.Stream] = None,
                     workspace: Optional[torch.Tensor] = None, eos_token: int = -1,
                     draft_cache: Optional[KVCache] = None,
                     draft_model: Optional[SpecLoopModel] = None) -> LoopResult:
    """Runs the loop from the cache's device seq_len (positions below it hold
    the context) with `anchor` the last emitted token; synchronizes and
    returns the emitted tokens and per-round acceptances.  With draft_cache
    and draft_model, the draft model drafts over its own cache (its device
    seq_len the draft's start, n_draft unused); eos_token >= 0 stops after a
    round whose bonus token is it."""
    return _run(cache, model, anchor, k, n_draft, max_new, eos_token, draft_cache, draft_model,
                None, None, stream, workspace, "spec_loop_greedy")


def spec_loop_stochastic(cache: KVCache, model: SpecLoopModel, anchor: int, k: int, n_draft: int,
                         max_new: int, seed: int, draft_temp: float = 1.0, adaptive: bool = False,
                         min_temp: float = 0.1, max_temp: float = 2.0,
                         target_accept: float = 0.7, gain: float = 0.1, ewma_mix: float = 0.2,
                         offset: Optional[torch.Tensor] = None,
                         stream: Optional[torch.cuda.Stream] = None,
                         workspace: Optional[torch.Tensor] = None, eos_token: int = -1,
                         draft_cache: Optional[KVCache] = None,
                         draft_model: Optional[SpecLoopModel] = None) -> LoopResult:
    """spec_loop_greedy's rounds with speculative sampling.  `offset` is the
    device uint64 call index of the random stream (a fresh zero when None;
    the call advances it by k + 1 per round)."""
    if offset is None:
        offset = torch.zeros(1, dtype=torch.int64, device=cache.device)
    smp = LoopSampling(draft_temp, int(bool(adaptive)), min_temp, max_temp, target_accept, gain,
                       ewma_mix, seed & 0xFFFFFFFFFFFFFFFF)
    return _run(cache, model, anchor, k, n_draft, max_new, eos_token, draft_cache, draft_model,
                smp, offset, stream, workspace, "spec_loop_stochastic")
