"""MI355X (gfx950) paged KV cache and paged GQA decode/verify attention.

The product is libsde_paged.so (C-ABI in include/sde_paged_kv.h, HIP kernels
in csrc/).  This package holds its ctypes binding, a host-side mirror of the
reference KVCache API (kv_cache.py) and the benchmark workloads.
"""
from .kv_cache import (ATTN_KDA, ATTN_LINEAR, ATTN_SLIDING_WINDOW, ATTN_SOFTMAX, KVCache,
                       kv_cache_alloc, kv_cache_free, kv_cache_reset, spec_accept_greedy,
                       spec_accept_stochastic)
from ._native import SDEError
from .matvec import PackedWeight, matvec, matvec_packed, matvec_workspace
from .sdec import SDECModel, load_sdec, read_header, write_sdec
from .spec_loop import SpecLoopModel, spec_loop_greedy, spec_loop_stochastic

__all__ = ["KVCache", "kv_cache_alloc", "kv_cache_free", "kv_cache_reset", "SDEError",
           "spec_accept_greedy", "spec_accept_stochastic", "matvec", "matvec_workspace", "PackedWeight", "matvec_packed",
           "SDECModel", "load_sdec", "read_header", "write_sdec",
           "SpecLoopModel", "spec_loop_greedy", "spec_loop_stochastic",
           "ATTN_SOFTMAX", "ATTN_SLIDING_WINDOW", "ATTN_KDA", "ATTN_LINEAR"]
