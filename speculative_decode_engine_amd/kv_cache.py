"""Host-side mirror of the reference's paged KV cache API, over the C-ABI.

Reference (arkhamHack/speculative_decode_engine):
  KVCache / kv_cache_alloc / kv_cache_free / kv_cache_reset
                                   cuda/include/kv_cache.h:33-63, kv_cache.cu:8-52
  kv_cache_append, cublas_kv_append_kernel
                                   kv_cache.cu:70-93, kernels.cu:826-844
  kv_cache_read                    kv_cache.cu:95-114
  kv_cache_rollback, set_seq_len_kernel
                                   kv_cache.cu:116-120, kernels.cu:546-548
  cublas_attention_kernel / device_attention_dispatch
                                   kernels.cu:904-940, attention.h:140-164

Device buffers are torch tensors (plumbing only: every computation runs in
libsde_paged.so's HIP kernels).  Errors raise SDEError carrying the C status
code; the reference aborts instead (utils.h:387-395).
"""
from __future__ import annotations

import atexit
import ctypes
import sys
import weakref
from typing import Optional

import numpy as np
import torch

from . import _native
from ._native import KVConfig, KVView, SDEError, check

ATTN_SOFTMAX = _native.SDE_ATTN_SOFTMAX
ATTN_SLIDING_WINDOW = _native.SDE_ATTN_SLIDING_WINDOW
ATTN_KDA = _native.SDE_ATTN_KDA
ATTN_LINEAR = _native.SDE_ATTN_LINEAR

KV_BLOCK_SIZE = 16  # reference default (config.h:10)

# Caches still alive when the interpreter exits are destroyed by an exit
# handler, while the HIP runtime is still up; after it (and during the
# interpreter's own teardown, when module globals and the runtime may already
# be gone) a cache's destructor does nothing.
_LIVE: "weakref.WeakSet[KVCache]" = weakref.WeakSet()
_EXITING = False


def _free_live_caches() -> None:
    global _EXITING
    for cache in list(_LIVE):
        try:
            cache.free()
        except Exception:
            pass
    _EXITING = True


atexit.register(_free_live_caches)


def _stream_handle(stream: Optional[torch.cuda.Stream]) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dev_f32(t: torch.Tensor, name: str, shape: tuple) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise TypeError(f"{name} must be a CUDA tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if tuple(t.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


class KVCache:
    """One model's paged KV cache (reference KVCache, kv_cache.h:33-51).

    Layout (kv_cache.h:5-18): physical block b = K fp16[block_size][kv_dim]
    followed by V fp16[block_size][kv_dim]; token pos of layer l is in block
    table[l][pos // block_size], slot pos % block_size.

    `pool="library"` lets the library allocate (and zero) the pool like
    kv_cache_alloc; `pool="torch"` allocates it as a zeroed torch tensor
    (exposed as `.pool`) and hands it to sde_kv_cache_create_external.
    """

    def __init__(self, n_layers: int, d_head: int, max_blocks_per_layer: int,
                 block_size: int = KV_BLOCK_SIZE, pool_blocks: int = 0,
                 pool: str = "torch", device: Optional[torch.device] = None):
        self._lib = _native.load()
        self.cfg = KVConfig(n_layers, d_head, max_blocks_per_layer, block_size, pool_blocks)
        check(self._lib.sde_kv_config_validate(ctypes.byref(self.cfg)), "kv config")
        self.n_layers = n_layers
        self.d_head = d_head  # = kv_dim = n_kv_heads * head_dim (kv_cache.h:42-43)
        self.kv_dim = d_head
        self.max_blocks_per_layer = max_blocks_per_layer
        self.block_size = block_size
        self.pool_blocks = pool_blocks or n_layers * max_blocks_per_layer
        self.device = torch.device(device or "cuda")
        self._handle = ctypes.c_void_p()
        self.pool: Optional[torch.Tensor] = None
        nbytes = self._lib.sde_kv_pool_bytes(ctypes.byref(self.cfg))
        with torch.cuda.device(self.device):
            if pool == "torch":
                self.pool = torch.zeros(nbytes // 2, dtype=torch.int16, device=self.device)
                torch.cuda.synchronize(self.device)
                check(self._lib.sde_kv_cache_create_external(
                    ctypes.byref(self.cfg), ctypes.c_void_p(self.pool.data_ptr()),
                    nbytes, ctypes.byref(self._handle)), "kv_cache_alloc")
            elif pool == "library":
                check(self._lib.sde_kv_cache_create(ctypes.byref(self.cfg),
                                                    ctypes.byref(self._handle)),
                      "kv_cache_alloc")
            else:
                raise ValueError("pool must be 'torch' or 'library'")
        _LIVE.add(self)

    # ---- lifetime (kv_cache_free) -------------------------------------------
    def free(self) -> None:
        if self._handle:
            check(self._lib.sde_kv_cache_destroy(self._handle), "kv_cache_free")
            self._handle = ctypes.c_void_p()
        self.pool = None

    def __del__(self):
        if _EXITING or sys.is_finalizing():
            return
        try:
            self.free()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    @property
    def handle(self) -> ctypes.c_void_p:
        if not self._handle:
            raise RuntimeError("cache has been freed")
        return self._handle

    # ---- metadata -------------------------------------------------------------
    def pool_blocks_view(self) -> torch.Tensor:
        """The pool as int16 [pool_blocks][2][block_size][kv_dim] (torch pools)."""
        if self.pool is None:
            raise RuntimeError("pool is owned by the library; create with pool='torch'")
        return self.pool.view(self.pool_blocks, 2, self.block_size, self.kv_dim)

    def set_block_table(self, layer: int, table) -> None:
        arr = np.ascontiguousarray(np.asarray(table, dtype=np.int32))
        check(self._lib.sde_kv_set_block_table(
            self.handle, layer, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), arr.size),
            "set_block_table")

    def block_table(self, layer: int, n_blocks: Optional[int] = None) -> np.ndarray:
        n = self.max_blocks_per_layer if n_blocks is None else n_blocks
        out = np.empty(n, dtype=np.int32)
        check(self._lib.sde_kv_get_block_table(
            self.handle, layer, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n),
            "get_block_table")
        return out

    def view(self) -> KVView:
        v = KVView()
        check(self._lib.sde_kv_get_view(self.handle, ctypes.byref(v)), "get_view")
        return v

    # ---- seq_len bookkeeping ----------------------------------------------------
    @property
    def seq_len(self) -> int:
        out = ctypes.c_int()
        check(self._lib.sde_kv_seq_len(self.handle, ctypes.byref(out)), "seq_len")
        return out.value

    def set_seq_len(self, n: int, stream=None) -> None:
        """set_seq_len_kernel (kernels.cu:546-548)."""
        check(self._lib.sde_kv_set_seq_len(self.handle, n, _stream_handle(stream)),
              "set_seq_len")

    def reset(self, stream=None) -> None:
        """kv_cache_reset (kv_cache.cu:50-52)."""
        check(self._lib.sde_kv_reset(self.handle, _stream_handle(stream)), "kv_cache_reset")

    def rollback(self, target_len: int, stream=None) -> None:
        """O(1) rewind of rejected drafts (kernels.cu:2457-2459): no pool bytes move."""
        check(self._lib.sde_kv_rollback(self.handle, target_len, _stream_handle(stream)),
              "kv_cache_rollback")

    def device_seq_len(self) -> int:
        """The device-side seq_len word (synchronises the device)."""
        out = ctypes.c_int()
        check(self._lib.sde_kv_device_seq_len(self.handle, ctypes.byref(out)), "device_seq_len")
        return out.value

    # ---- data path ---------------------------------------------------------------
    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, pos_base: int,
               stream=None) -> None:
        """cublas_kv_append_kernel (kernels.cu:826-844): fp32 [M][kv_dim] rows
        -> fp16 (RNE) at positions pos_base..pos_base+M-1."""
        M = k.shape[0] if k.dim() == 2 else 1
        k = _dev_f32(k.reshape(M, self.kv_dim), "k", (M, self.kv_dim))
        v = _dev_f32(v.reshape(M, self.kv_dim), "v", (M, self.kv_dim))
        check(self._lib.sde_kv_append(self.handle, layer, ctypes.c_void_p(k.data_ptr()),
                                      ctypes.c_void_p(v.data_ptr()), pos_base, M,
                                      _stream_handle(stream)), "kv_cache_append")

    def write_fp16(self, layer: int, k16: torch.Tensor, v16: torch.Tensor, pos_base: int,
                   stream=None) -> None:
        """Lands fp16 rows ([M][kv_dim], float16 or int16 bits) unconverted."""
        M = k16.shape[0]
        for name, t in (("k16", k16), ("v16", v16)):
            if t.dtype not in (torch.float16, torch.int16) or tuple(t.shape) != (M, self.kv_dim) \
                    or not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError(f"{name} must be a contiguous CUDA fp16 [M][kv_dim] tensor")
        check(self._lib.sde_kv_write_fp16(self.handle, layer, ctypes.c_void_p(k16.data_ptr()),
                                          ctypes.c_void_p(v16.data_ptr()), pos_base, M,
                                          _stream_handle(stream)), "write_fp16")

    def read(self, layer: int, pos: int, n: int = 1, stream=None) -> tuple[torch.Tensor, torch.Tensor]:
        """kv_cache_read (kv_cache.cu:95-114) for positions pos..pos+n-1,
        widened exactly to fp32 [n][kv_dim]."""
        k = torch.empty(n, self.kv_dim, dtype=torch.float32, device=self.device)
        v = torch.empty(n, self.kv_dim, dtype=torch.float32, device=self.device)
        check(self._lib.sde_kv_gather(self.handle, layer, pos, n, ctypes.c_void_p(k.data_ptr()),
                                      ctypes.c_void_p(v.data_ptr()), _stream_handle(stream)),
              "kv_cache_read")
        return k, v

    def workspace_size(self, nh: int, nkv: int, dph: int, n_queries: int,
                       max_total_len: int) -> int:
        return int(self._lib.sde_paged_attention_workspace_size(
            self.handle, nh, nkv, dph, n_queries, max_total_len))

    def attention(self, layer: int, q: torch.Tensor, nh: int, nkv: int, dph: int,
                  pos_base: int, out: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None,
                  attn_type: int = ATTN_SOFTMAX, stream=None) -> torch.Tensor:
        """cublas_attention_kernel (kernels.cu:904-940) through
        device_attention_dispatch (attention.h:140-164): q fp32 [M][nh*dph];
        query m attends causally to positions [0, pos_base+m]."""
        M = q.shape[0] if q.dim() == 2 else 1
        q = _dev_f32(q.reshape(M, nh * dph), "q", (M, nh * dph))
        if out is None:
            out = torch.empty(M, nh * dph, dtype=torch.float32, device=self.device)
        _dev_f32(out, "out", (M, nh * dph))
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            if workspace.device.type != "cuda" or not workspace.is_contiguous():
                raise ValueError("workspace must be a contiguous CUDA tensor")
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.sde_attention_dispatch(
            attn_type, self.handle, layer, ctypes.c_void_p(q.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), nh, nkv, dph, pos_base, M,
            ctypes.c_void_p(ws_ptr), ws_bytes, _stream_handle(stream)),
            "paged_attention")
        return out

    def attention_noalloc(self, layer: int, q: torch.Tensor, nh: int, nkv: int, dph: int,
                          pos_base: int, out: Optional[torch.Tensor] = None,
                          stream=None) -> torch.Tensor:
        """attention() through sde_paged_attention_noalloc: the partials go
        to the library's static per-device array, so the call allocates no
        device memory (out must then be given by the caller)."""
        M = q.shape[0] if q.dim() == 2 else 1
        q = _dev_f32(q.reshape(M, nh * dph), "q", (M, nh * dph))
        if out is None:
            out = torch.empty(M, nh * dph, dtype=torch.float32, device=self.device)
        _dev_f32(out, "out", (M, nh * dph))
        check(self._lib.sde_paged_attention_noalloc(
            self.handle, layer, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(out.data_ptr()),
            nh, nkv, dph, pos_base, M, _stream_handle(stream)), "paged_attention_noalloc")
        return out

    def rope_append_attention(self, layer: int, q: torch.Tensor, k: torch.Tensor,
                              v: torch.Tensor, nh: int, nkv: int, dph: int, pos_base: int,
                              theta: float = 10000.0, scaling_type: int = 0,
                              scaling_factor: float = 1.0, out: Optional[torch.Tensor] = None,
                              workspace: Optional[torch.Tensor] = None,
                              stream=None) -> torch.Tensor:
        """RoPE + append + attention in one launch (model.cu:346-384 with
        cublas_rope_kernel, cublas_kv_append_kernel and
        cublas_attention_kernel): q fp32 [M][nh*dph], k and v fp32
        [M][nkv*dph], all before RoPE; q and k are rotated (rotate-half,
        model.cu:281-323) at positions pos_base+m, k and v appended there,
        and query m attends causally to [0, pos_base+m]."""
        M = q.shape[0] if q.dim() == 2 else 1
        q = _dev_f32(q.reshape(M, nh * dph), "q", (M, nh * dph))
        k = _dev_f32(k.reshape(M, self.kv_dim), "k", (M, self.kv_dim))
        v = _dev_f32(v.reshape(M, self.kv_dim), "v", (M, self.kv_dim))
        if out is None:
            out = torch.empty(M, nh * dph, dtype=torch.float32, device=self.device)
        _dev_f32(out, "out", (M, nh * dph))
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            if workspace.device.type != "cuda" or not workspace.is_contiguous():
                raise ValueError("workspace must be a contiguous CUDA tensor")
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        rope = _native.RopeConfig(theta, scaling_type, scaling_factor)
        check(self._lib.sde_rope_append_attention(
            self.handle, layer, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()),
            ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(out.data_ptr()), nh, nkv, dph,
            pos_base, M, ctypes.byref(rope), ctypes.c_void_p(ws_ptr), ws_bytes,
            _stream_handle(stream)), "rope_append_attention")
        return out


def spec_accept_greedy(target: KVCache, draft: Optional[KVCache], draft_tokens: torch.Tensor,
                       target_tokens: torch.Tensor, k: int, target_save: int, draft_save: int,
                       out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Greedy acceptance + O(1) rewind on the device (kernels.cu:2428-2466,
    3050-3072): returns the device int32 result [k+5] = (n_accepted, bonus,
    target seq_len, draft seq_len, emitted tokens...).  draft None or target
    = one shared cache (self-speculation)."""
    for name, t in (("draft_tokens", draft_tokens), ("target_tokens", target_tokens)):
        if t.device.type != "cuda" or t.dtype != torch.int32 or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous CUDA int32 tensor")
    if out is None:
        out = torch.empty(k + 5, dtype=torch.int32, device=target.device)
    lib = _native.load()
    check(lib.sde_spec_accept_greedy(
        target.handle, draft.handle if draft is not None else None,
        ctypes.c_void_p(draft_tokens.data_ptr()), ctypes.c_void_p(target_tokens.data_ptr()), k,
        target_save, draft_save, ctypes.c_void_p(out.data_ptr()), _stream_handle(stream)),
        "spec_accept_greedy")
    return out


def spec_accept_stochastic(target: KVCache, draft: Optional[KVCache],
                           target_logits: torch.Tensor, draft_logits: Optional[torch.Tensor],
                           draft_tokens: torch.Tensor, k: int, target_save: int,
                           draft_save: int, seed: int, rng_offset: torch.Tensor,
                           temp_target: float = 1.0, temp_draft: float = 1.0,
                           out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Speculative sampling acceptance + O(1) rewind on the device
    (kernels.cu:550-572, 319-380): target_logits fp32 [k+1][V], draft_logits
    fp32 [k][V], draft_tokens int32 [k], rng_offset a CUDA int64 [1] call
    counter the call increments.  Returns the device int32 result [k+5] like
    spec_accept_greedy."""
    V = target_logits.shape[-1]
    _dev_f32(target_logits, "target_logits", (k + 1, V))
    if k:
        _dev_f32(draft_logits, "draft_logits", (k, V))
    for name, t, dt in (("draft_tokens", draft_tokens, torch.int32),
                        ("rng_offset", rng_offset, torch.int64)):
        if t.device.type != "cuda" or t.dtype != dt or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous CUDA {dt} tensor")
    if out is None:
        out = torch.empty(k + 5, dtype=torch.int32, device=target.device)
    lib = _native.load()
    check(lib.sde_spec_accept_stochastic(
        target.handle, draft.handle if draft is not None else None,
        ctypes.c_void_p(target_logits.data_ptr()),
        ctypes.c_void_p(draft_logits.data_ptr() if k else 0),
        ctypes.c_void_p(draft_tokens.data_ptr()), k, V, temp_target, temp_draft,
        seed & 0xFFFFFFFFFFFFFFFF, ctypes.c_void_p(rng_offset.data_ptr()), target_save,
        draft_save, ctypes.c_void_p(out.data_ptr()), _stream_handle(stream)),
        "spec_accept_stochastic")
    return out


# Reference-named entry points (kv_cache.h:56-63).
def kv_cache_alloc(n_layers: int, d_head: int, max_blocks_per_layer: int,
                   block_size: int = KV_BLOCK_SIZE, pool_blocks: int = 0,
                   pool: str = "torch") -> KVCache:
    return KVCache(n_layers, d_head, max_blocks_per_layer, block_size, pool_blocks, pool)


def kv_cache_free(cache: KVCache) -> None:
    cache.free()


def kv_cache_reset(cache: KVCache, stream=None) -> None:
    cache.reset(stream)
