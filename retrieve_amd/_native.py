"""Loader of ``libretrieve_amd.so`` (the C ABI in ``include/retrieve_amd.h``) and the ctypes
plumbing every op shares: status → exception mapping, device pointers, the current stream.

The library is loaded after ``torch`` so it binds to the HIP runtime torch already holds
(both carry the SONAME ``libamdhip64.so.7``). There is no fallback: if the library is missing
or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libretrieve_amd.so")

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_sz = ctypes.c_size_t
_c_int = ctypes.c_int

# name -> (restype, argtypes); the symbol set include/retrieve_amd.h declares
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "rt_last_error": (ctypes.c_char_p, []),
    "rt_int8_scan_topk_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "rt_hamming_scan_topk_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "rt_hamming_scan_topk": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_int, _c_p,
         _c_sz, _c_p],
    ),
    "rt_dense_scan_topk_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "rt_dense_scan_topk": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_p, _c_p,
         _c_sz, _c_p],
    ),
    "rt_blocked_scan_topk_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "rt_blocked_scan_topk": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_p, _c_p,
         _c_sz, _c_p],
    ),
    "rt_profile_enable": (_c_int, [_c_int]),
    "rt_profile_collect": (_c_int, [_c_p, _c_p]),
    "rt_mfma_ceiling": (_c_int, [_c_int, _c_i64, _c_p, _c_p, _c_p]),
    "rt_clause_filter_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "rt_clause_filter": (
        _c_int,
        [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_p,
         _c_i64, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_scan_topk_clauses_workspace": (_c_sz, [_c_i64] * 6),
    "rt_scan_topk_clauses": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_int, _c_i64,
         _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_scan_topk_bloom_clauses": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_i64, _c_p, _c_int,
         _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_blocked_scan_topk_clauses_workspace": (_c_sz, [_c_i64] * 6),
    "rt_blocked_scan_topk_clauses": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_i64, _c_p, _c_int,
         _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_hamming_scan_topk_clauses_fused": (_c_int, [_c_i64, _c_i64, _c_i64]),
    "rt_hamming_scan_topk_clauses_workspace": (_c_sz, [_c_i64] * 6),
    "rt_hamming_scan_topk_clauses": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_int, _c_i64,
         _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_int, _c_p, _c_sz, _c_p],
    ),
    "rt_read_ceiling": (_c_int, [_c_p, _c_i64, _c_int, _c_p, _c_p]),
    "rt_bloom_bundle_terms": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "rt_bloom_build": (
        _c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p],
    ),
    "rt_bloom_search_workspace": (_c_sz, [_c_i64, _c_i64]),
    "rt_bloom_search": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
         _c_sz, _c_p],
    ),
    "rt_bloom_search_t": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
         _c_p, _c_sz, _c_p],
    ),
    "rt_bloom_compiled_bytes": (_c_sz, [_c_i64]),
    "rt_bloom_compile": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_sz, _c_p],
    ),
    "rt_bloom_search_compiled": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_sz,
         _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p],
    ),
    "rt_bloom_doc_bits": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "rt_bloom_probe_search": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p]),
    "rt_mask_compact_workspace": (_c_sz, [_c_i64, _c_i64]),
    "rt_mask_compact": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "rt_cand_topk_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "rt_cand_topk": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p,
         _c_sz, _c_p],
    ),
    "rt_gemv_scores": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "rt_quantize_int8_rows": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_int, _c_p]),
    "rt_pack_mask": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "rt_pack_signs": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "rt_quantize_int8_global": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "rt_int8_rerank_topk": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p,
         _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_clause_slots_filter": (
        _c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p],
    ),
    "rt_ivf_search_workspace": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "rt_ivf_search_payload_filters": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
         _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64,
         _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_ivf_search": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_p,
         _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
    "rt_search_epilogue": (
        _c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p],
    ),
    "rt_bloom_search_columns": (
        _c_int,
        [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p,
         _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p],
    ),
    "rt_fused_kmean_ann": (
        _c_int,
        [_c_p, _c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
         _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
         _c_p, _c_p, _c_p],
    ),
    "rt_int8_scan_topk_noalloc": (
        _c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p],
    ),
    "rt_int8_scan_topk": (
        _c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p],
    ),
}

_lib: ctypes.CDLL | None = None


class NativeMissing(RuntimeError):
    """``libretrieve_amd.so`` is not built or cannot be loaded."""


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeMissing(
                f"{LIB_PATH} is not built; build it with `make -C retrieve_amd/csrc` "
                "(or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


_STATUS_EXC = {1: ValueError, 2: TypeError, 3: RuntimeError, 4: RuntimeError}


def check(status: int) -> None:
    """Raise the mapped exception for a non-zero status, with the library's message."""
    if status != 0:
        msg = lib().rt_last_error().decode(errors="replace")
        raise _STATUS_EXC.get(status, RuntimeError)(msg)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` (torch's current stream)."""
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU; returns it. CPU tensors raise: there is no CPU path."""
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                f"retrieve_amd ops run on the GPU only; got a tensor on {t.device}"
            )
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch from torch's caching allocator (no hipMalloc per call once warm)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
