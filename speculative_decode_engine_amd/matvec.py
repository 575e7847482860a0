"""The output projection after attention (Wo) on the GPU: a ctypes mirror of
sde_matvec (include/sde_paged_kv.h), the replacement of the reference's
device_matvec_partial_accum / device_matvec_batched calls (utils.h:248-280,
437-452; kernels.cu:2742-2747, model.cu:717), and of its panel-packed form
(sde_matvec_pack once per weight, then sde_matvec_packed per call)."""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _native
from ._native import check
from .kv_cache import _stream_handle

_WORKSPACES: dict = {}
_RETIRED: list = []


def matvec_workspace(d_in: int, d_out: int, n_rows: int, device) -> torch.Tensor:
    """A zeroed workspace for sde_matvec calls of these shapes on `device`
    (its arrival counters must start at zero; every call leaves them zero)."""
    lib = _native.load()
    n = int(lib.sde_matvec_workspace_size(d_in, d_out, n_rows))
    if n == 0:
        raise ValueError(f"invalid matvec shape d_in={d_in} d_out={d_out} n_rows={n_rows}")
    return torch.zeros(n, dtype=torch.uint8, device=device)


def _cached_workspace(d_in: int, d_out: int, n_rows: int, device, stream) -> torch.Tensor:
    """One workspace per (device, stream): calls on one stream are ordered,
    so they may share its arrival counters; calls on different streams get
    different workspaces.  An outgrown workspace is kept alive (queued work
    or a captured graph may still use it)."""
    lib = _native.load()
    need = int(lib.sde_matvec_workspace_size(d_in, d_out, n_rows))
    key = (torch.device(device), _stream_handle(stream).value or 0)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def matvec(x: torch.Tensor, W: torch.Tensor, out: Optional[torch.Tensor] = None,
           accumulate: bool = False, workspace: Optional[torch.Tensor] = None,
           stream=None) -> torch.Tensor:
    """out[m][c] = (accumulate ? out[m][c] : 0) + sum_r x[m][r] * W[r][c].

    x: CUDA float32 [M][d_in] or [d_in]; W: CUDA float16 [d_in][d_out]
    (row-major, the reference's weight layout); out: CUDA float32
    [M][d_out] (allocated when None; required when accumulate).  The
    workspace defaults to one cached per (device, stream)."""
    squeeze = x.dim() == 1
    x2 = x.unsqueeze(0) if squeeze else x
    if x2.device.type != "cuda" or x2.dtype != torch.float32 or not x2.is_contiguous():
        raise TypeError("x must be a contiguous CUDA float32 tensor")
    if W.device.type != "cuda" or W.dtype != torch.float16 or not W.is_contiguous() or W.dim() != 2:
        raise TypeError("W must be a contiguous 2-D CUDA float16 tensor")
    M, d_in = x2.shape
    if W.shape[0] != d_in:
        raise ValueError(f"W has {W.shape[0]} rows, x has {d_in} columns")
    d_out = W.shape[1]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty((M, d_out) if not squeeze else (d_out,), dtype=torch.float32,
                          device=x.device)
    if out.device.type != "cuda" or out.dtype != torch.float32 or not out.is_contiguous() \
            or out.numel() != M * d_out:
        raise TypeError(f"out must be a contiguous CUDA float32 tensor of {M}x{d_out}")
    if workspace is None:
        workspace = _cached_workspace(d_in, d_out, M, x.device, stream)
    lib = _native.load()
    check(lib.sde_matvec(ctypes.c_void_p(x2.data_ptr()), ctypes.c_void_p(W.data_ptr()),
                         ctypes.c_void_p(out.data_ptr()), d_in, d_out, M, int(bool(accumulate)),
                         ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                         _stream_handle(stream)), "matvec")
    return out


class PackedWeight:
    """A panel-packed copy of a row-major fp16 W [d_in][d_out] (sde_matvec_pack),
    the operand of matvec_packed.  The source W is not kept."""

    def __init__(self, W: torch.Tensor, stream=None):
        if W.device.type != "cuda" or W.dtype != torch.float16 or not W.is_contiguous() \
                or W.dim() != 2:
            raise TypeError("W must be a contiguous 2-D CUDA float16 tensor")
        self.d_in, self.d_out = int(W.shape[0]), int(W.shape[1])
        lib = _native.load()
        n = int(lib.sde_matvec_packed_size(self.d_in, self.d_out))
        if n == 0:
            raise ValueError(f"packed matvec needs d_in and d_out multiples of 8, got "
                             f"{self.d_in} x {self.d_out}")
        self.data = torch.empty(n, dtype=torch.uint8, device=W.device)
        check(lib.sde_matvec_pack(ctypes.c_void_p(W.data_ptr()), self.d_in, self.d_out,
                                  ctypes.c_void_p(self.data.data_ptr()), n,
                                  _stream_handle(stream)), "matvec_pack")


def matvec_packed(x: torch.Tensor, Wp: PackedWeight, out: Optional[torch.Tensor] = None,
                  accumulate: bool = False, stream=None) -> torch.Tensor:
    """matvec over a PackedWeight: out[m][c] = (accumulate ? out[m][c] : 0) +
    sum_r x[m][r] * W[r][c], x CUDA float32 [M][d_in] or [d_in] (M <= 16)."""
    squeeze = x.dim() == 1
    x2 = x.unsqueeze(0) if squeeze else x
    if x2.device.type != "cuda" or x2.dtype != torch.float32 or not x2.is_contiguous():
        raise TypeError("x must be a contiguous CUDA float32 tensor")
    M, d_in = x2.shape
    if d_in != Wp.d_in:
        raise ValueError(f"W has {Wp.d_in} rows, x has {d_in} columns")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty((M, Wp.d_out) if not squeeze else (Wp.d_out,), dtype=torch.float32,
                          device=x.device)
    if out.device.type != "cuda" or out.dtype != torch.float32 or not out.is_contiguous() \
            or out.numel() != M * Wp.d_out:
        raise TypeError(f"out must be a contiguous CUDA float32 tensor of {M}x{Wp.d_out}")
    lib = _native.load()
    check(lib.sde_matvec_packed(ctypes.c_void_p(x2.data_ptr()), ctypes.c_void_p(Wp.data.data_ptr()),
                                ctypes.c_void_p(out.data_ptr()), d_in, Wp.d_out, M,
                                int(bool(accumulate)), _stream_handle(stream)), "matvec_packed")
    return out
