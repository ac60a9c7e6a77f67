"""Top-k above the fused kernels' bound (k > 1024).

The reference selects with ``at::topk`` over the scorer's raw ``[B, width]`` buffer above its
own radix select's 1024 (``silvertorch/silvertorch/ops/csrc/fork_search_cuda.cu:843-915``,
``docs/system/kernels.md:1201-1205``); ``retrieve``'s ``masked_topk`` has no bound
(``retrieve/src/retrieve/functional.py:22-85``). Here the raw scorer is this package's HIP
kernel (``torch.ops.st.fused_kmean_ann``'s, every probed slot scored in slot order), and each row
is selected by one ``torch.topk`` over int64 keys that hold the score's order in the high bits
and the slot in the low bits: the result is exact, ordered by (score desc, slot asc) as the
fused kernels order it, and the same on every call. Rows are processed in chunks whose buffers
take at most a quarter of the device's free memory.
"""

from __future__ import annotations

import torch
from torch import Tensor

from retrieve_amd import st

# Bytes per slot of one chunk's buffers: raw (4), slot index (4), key (8) and the key's
# temporaries (8).
_SLOT_BYTES = 24
_SLOT_BITS = 31


def order_keys(raw: Tensor, valid: Tensor) -> Tensor:
    """int64 keys of ``raw`` (int32, or a float type) ``[R, W]``: the score's order as an
    unsigned 32-bit value times 2**31 plus ``2**31 - 1 - slot``, ``-1`` where ``valid`` is false.
    Larger key = better: higher score, then lower slot."""
    if raw.dtype == torch.int32:
        key = raw.to(torch.int64) + 2**31
    else:
        bits = raw.to(torch.float32).contiguous().view(torch.int32).to(torch.int64)
        key = torch.where(bits >= 0, bits + 2**31, -bits - 1)
    slots = torch.arange(raw.shape[1], device=raw.device, dtype=torch.int64)
    key = key * 2**_SLOT_BITS + (2**_SLOT_BITS - 1 - slots)
    return torch.where(valid, key, -1)


def raw_topk(raw: Tensor, idx: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """The best ``min(k, W)`` slots of each row of a raw buffer (``idx < 0``: no candidate) →
    ``(raw values [R, k], slots int64 [R, k])``, slot ``-1`` past a row's candidates (its raw
    value then unspecified)."""
    rows, width = raw.shape
    kk = min(k, width)
    top_raw = raw.new_empty((rows, k))
    top_slot = torch.full((rows, k), -1, dtype=torch.int64, device=raw.device)
    if rows == 0 or kk == 0:
        return top_raw, top_slot
    keys = order_keys(raw, idx >= 0)
    v = torch.topk(keys, kk, dim=1).values
    slot = 2**_SLOT_BITS - 1 - (v & (2**_SLOT_BITS - 1))
    slot = torch.where(v >= 0, slot, -1)
    top_slot[:, :kk] = slot
    top_raw[:, :kk] = raw.gather(1, slot.clamp(min=0))
    return top_raw, top_slot


def chunk_rows(width: int, device: torch.device) -> int:
    """Rows per chunk: a quarter of the device's free memory (at least 2 GiB) over the bytes
    one row's buffers take."""
    free, _ = torch.cuda.mem_get_info(device)
    budget = max(2 << 30, free // 4)
    return max(1, budget // (_SLOT_BYTES * max(1, width)))


def full_scan_topk(queries: Tensor, items: Tensor, k: int, mask: Tensor | None,
                   pad_score) -> tuple[Tensor, Tensor]:
    """Top ``k`` items of every query over the whole table (one cluster ``[0, N)``, so slot =
    item position) → ``(ids int64 [B, k], scores [B, k])`` with ``-1`` / ``pad_score`` where
    fewer than ``k`` items pass ``mask`` (``[B, ceil(N/64)]`` words, item ``d`` at bit
    ``63 - d % 64``). int8 items give int32 dot products, bf16 / fp16 items fp32 ones."""
    b = queries.shape[0]
    n = items.shape[0]
    dev = items.device
    score_dtype = torch.int32 if items.dtype == torch.int8 else torch.float32
    ids = torch.full((b, k), -1, dtype=torch.int64, device=dev)
    scores = torch.full((b, k), pad_score, dtype=score_dtype, device=dev)
    if b == 0 or n == 0:
        return ids, scores
    offsets = torch.zeros(1, dtype=torch.int64, device=dev)
    step = chunk_rows(n, dev)
    for r0 in range(0, b, step):
        r1 = min(b, r0 + step)
        rows = r1 - r0
        cluster = torch.zeros((rows, 1), dtype=torch.int64, device=dev)
        length = torch.full((rows, 1), n, dtype=torch.int64, device=dev)
        raw, idx = st.raw_scores(offsets, cluster, length, items, queries[r0:r1].contiguous(), n,
                                 mask=None if mask is None else mask[r0:r1])
        top_raw, slot = raw_topk(raw, idx, k)
        ids[r0:r1] = torch.where(slot >= 0, idx.gather(1, slot.clamp(min=0)).to(torch.int64), -1)
        scores[r0:r1] = torch.where(slot >= 0, top_raw.to(score_dtype),
                                    torch.full_like(scores[r0:r1], pad_score))
    return ids, scores
