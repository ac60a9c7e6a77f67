"""CPU restatement of SilverTorch's search after phase 1 (test infrastructure only: the product
never imports it). Follows ``silvertorch/silvertorch/ops/csrc/fork_search_cuda.cu:1256-1524``:
quantize the rows (``:680-699``), number each row's probed docs as the GPU scorer writes them
(every probed cluster's full 32-doc warps in probe order, then every cluster's remaining docs in
probe order; at most ``width`` slots), score the int8 codes, keep the top ``k`` by (key desc,
slot asc), and write ``sort_perm[position]`` and the dequantized score (``:552-597``).

The slot order is the CUDA op's, not the CPU twin's: ``fused_kmean_ann_cpu``
(``fused_kmean_ann.cpp:181-220``) writes probe by probe in doc order and compacts filtered-out
docs, while the GPU scorer's warp payloads (``fork_search_cuda.cu:989-991``,
``fused_kmean_ann_cuda.cu:592-598``) and remainder payloads (``fork_search_cuda.cu:1051-1053``,
``fused_kmean_ann_cuda.cu:443-453``) write to fixed slots, a filtered-out doc leaving its slot
unwritten. Pinned by a hand-written slot table (``tests/test_oracle.py``) and, through ties,
by the GPU tests of ``st::search``."""

from __future__ import annotations

import numpy as np

from oracle.quantize import quantize_int8


def row_slots(probe_row, cluster_offsets, cluster_sizes, n, width) -> np.ndarray:
    """Sorted positions of one row's slots: the full 32-doc warps of each probed cluster in
    probe order, then each cluster's ``len % 32`` remaining docs in probe order, the first
    ``width`` of them. A probe of an invalid cluster (or one reaching outside the table) is
    empty."""
    full, rest = [], []
    for c in np.asarray(probe_row).tolist():
        if 0 <= c < len(cluster_offsets):
            s, ln = int(cluster_offsets[c]), int(cluster_sizes[c])
            if s >= 0 and ln >= 0 and s + ln <= n:
                w = ln // 32 * 32
                full.extend(range(s, s + w))
                rest.extend(range(s + w, s + ln))
    return np.array((full + rest)[:width], np.int64)


def search(query, probe_ids, cluster_offsets, cluster_sizes, item_codes, sort_perm, global_scale,
           k, max_tensor_size_per_row, divisor=-1, valid=None):
    """``valid`` [B, N] bool over sorted positions (any filter), or None. Returns ``(ids int64
    [B, k], scores float32 [B, k])`` with -1 / -inf pads."""
    codes, scales = quantize_int8(np.asarray(query, np.float32))
    width = (int(max_tensor_size_per_row) + 31) // 32 * 32
    items = np.asarray(item_codes, np.int64)
    n = items.shape[0]
    b = codes.shape[0]
    gs = np.float32(np.asarray(global_scale, np.float32).reshape(-1)[0])
    ids = np.full((b, k), -1, np.int64)
    out = np.full((b, k), -np.inf, np.float32)
    for r in range(b):
        pos = row_slots(probe_ids[r], cluster_offsets, cluster_sizes, n, width)
        slot = np.arange(pos.size)
        if valid is not None:
            keep = valid[r, pos]
            pos, slot = pos[keep], slot[keep]
        dots = items[pos] @ codes[r].astype(np.int64)
        if divisor == -1:
            key = dots.astype(np.float64)
        else:
            key = (dots.astype(np.float32) / np.float32(divisor)).astype(np.float16)
            key = key.astype(np.float64)
        order = np.lexsort((slot, -key))[:k]
        ids[r, : order.size] = np.asarray(sort_perm)[pos[order]]
        for i, o in enumerate(order):
            if divisor == -1:
                s = np.float32(np.float32(dots[o]) * scales[r]) * gs
            else:
                mult = np.float32(np.float32(scales[r] * np.float32(divisor)) * gs)
                s = np.float32(key[o]) * mult
            out[r, i] = np.float32(s)
    return ids, out
