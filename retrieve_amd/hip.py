"""The ``"hip"`` op namespace: the reference's ``retrieve.ops.triton`` surface, re-implemented as
HIP kernels behind the C ABI and registered as ``torch.ops.retrieve.*``.

Importing this module registers the ops (the one side-effecting import, as the reference's
``retrieve.ops.triton``; ``import retrieve_amd`` registers nothing). Every op validates its
inputs here (``ValueError`` on shapes / contiguity, ``TypeError`` on dtypes, as
``retrieve/src/retrieve/ops/triton/_host.py:25-31`` and the preps do), allocates its outputs
and scratch from torch's caching allocator, and enqueues on torch's current stream.
"""

from __future__ import annotations

import torch
from torch import Tensor

from retrieve_amd import _native as nat


def _check_items(**tables: Tensor) -> None:
    """Item-side tables must arrive contiguous (``ops/triton/_host.py:25-31``)."""
    for name, t in tables.items():
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (copy it once at index build)")


# --- int8 full scan + top-k ---------------------------------------------------------------


def _int8_scan_prep(query_codes: Tensor, item_codes: Tensor, k: int, mask: Tensor | None):
    if query_codes.dim() != 2 or item_codes.dim() != 2:
        raise ValueError("query_codes must be [B, D] and item_codes [N, D]")
    if query_codes.dtype != torch.int8 or item_codes.dtype != torch.int8:
        raise TypeError("query_codes and item_codes must be int8")
    if query_codes.shape[1] != item_codes.shape[1]:
        raise ValueError(
            f"D mismatch: query D={query_codes.shape[1]} vs item D={item_codes.shape[1]}"
        )
    if not 1 <= k <= 1024:
        raise ValueError(f"k must be in [1, 1024], got {k}")
    _check_items(item_codes=item_codes)
    b, n = query_codes.shape[0], item_codes.shape[0]
    if mask is not None:
        if mask.dtype != torch.int64:
            raise TypeError("mask must be int64 words")
        if mask.dim() != 2 or mask.shape[0] != b or mask.shape[1] < (n + 63) // 64:
            raise ValueError(f"mask must be [B, ceil(N/64)] = [{b}, {(n + 63) // 64}]")
        mask = mask.contiguous()
    return query_codes.contiguous(), mask


@torch.library.custom_op("retrieve::int8_scan_topk", mutates_args=(), device_types="cuda")
def int8_scan_topk(
    query_codes: Tensor, item_codes: Tensor, k: int, mask: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """Exact int8 full-scan top-k: ``query_codes [B, D]`` int8 against ``item_codes [N, D]`` int8,
    int32 dot products, top ``k`` by (score desc, item index asc) → ``(ids int64 [B, k], scores
    int32 [B, k])``, ``-1`` / ``INT32_MIN`` where fewer than ``k`` items pass ``mask``
    (``[B, ceil(N/64)]`` int64 words, item ``d`` at bit ``63 - d % 64``). The int8 scorer and
    radix select of ``st::search`` on a single cluster
    (``silvertorch/.../fork_search_cuda.cu:1256-1524``)."""
    q, mask = _int8_scan_prep(query_codes, item_codes, k, mask)
    dev = nat.require_device(q, item_codes)
    b, d = q.shape
    n = item_codes.shape[0]
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.int32, device=dev)
    lib = nat.lib()
    ws_bytes = lib.rt_int8_scan_topk_workspace(b, n, d, k)
    ws = nat.workspace(ws_bytes, dev)
    with torch.cuda.device(dev):
        st = lib.rt_int8_scan_topk(
            nat.ptr(q), b, nat.ptr(item_codes), n, d, k, nat.ptr(mask),
            0 if mask is None else mask.shape[1],
            nat.ptr(ids), nat.ptr(scores), nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@int8_scan_topk.register_fake
def _(query_codes, item_codes, k, mask=None):
    b = query_codes.shape[0]
    return (
        query_codes.new_empty((b, k), dtype=torch.int64),
        query_codes.new_empty((b, k), dtype=torch.int32),
    )


__all__ = ["int8_scan_topk"]
