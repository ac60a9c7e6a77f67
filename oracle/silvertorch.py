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


def _row_ranges(probe_ids_row, lengths_row, cluster_offsets, n):
    """``[(start, full, rest)]`` per probe: cluster ``c``'s first position, its full-warp docs
    (``len // 32 * 32``) and remainder; an invalid cluster (or one reaching outside the table)
    is empty."""
    out = []
    for c, ln in zip(np.asarray(probe_ids_row).tolist(), np.asarray(lengths_row).tolist()):
        s, ln = (int(cluster_offsets[c]), int(ln)) if 0 <= c < len(cluster_offsets) else (0, 0)
        if s < 0 or ln < 0 or s + ln > n:
            ln = 0
        out.append((s, ln // 32 * 32, ln - ln // 32 * 32))
    return out


def fused_kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                    max_tensor_size_per_row, valid=None, valid_index=None, invalid=-1,
                    divisor=-1, scale=None, partial=None):
    """The raw scorer ``st::fused_kmean_ann`` as the CUDA op lays it out
    (``fused_kmean_ann_cuda.cu:2126-2262``): ``(scores [B, W], indices int32 [B, W])``, ``W`` =
    ``max_tensor_size_per_row`` rounded up to 32. Row b's slots are its probes' full 32-doc warps
    in probe order (write index ``:592-598``), then their remainders in probe order (``:443-453``);
    slot ``s`` holds the doc at its position, scored, with the position as its index, unless the
    filter drops the doc. Unwritten slots hold the dtype's lowest value (``INT32_MIN``, fp16
    ``-65504``, ``-FLT_MAX``) and ``invalid``.

    Scores: int8 → exact int32 dot (``fused_kmean_ann.cpp:60-70``); ``divisor != -1`` →
    ``fp16(fp32(dot) / divisor)`` (``index_mm_helpers.cuh:48-65``); a per-doc fp16 ``scale`` →
    ``fp16(fp32(fp16(dot)) / fp32(scale))`` (the Half arithmetic of ``post_process`` with a Half
    divisor); float rows → the float64 dot rounded to the row type (``fused_kmean_ann.cpp:44-55``).

    Filters: ``valid [R, N]`` bool over positions, row ``valid_index[b]`` (or ``b``); or
    ``partial = (counts_cumsum, first_offsets, words)`` from the probed-column Bloom search:
    doc ``o`` of probe ``p`` is bit ``first[e] + o`` of the words from ``counts_cumsum[e - 1]``,
    ``e = mask_row * P + p`` (``fused_kmean_ann_cuda.cu:706-720``, ``:826-846``)."""
    emb = np.asarray(embeddings)
    q = np.asarray(queries)
    n = emb.shape[0]
    width = (int(max_tensor_size_per_row) + 31) // 32 * 32
    b, p = np.asarray(cluster_ids).shape
    if emb.dtype == np.int8:
        kind = np.int32 if divisor == -1 and scale is None else np.float16
    else:
        kind = emb.dtype
    pad = {np.dtype(np.int32): np.iinfo(np.int32).min, np.dtype(np.float16): -65504.0}.get(
        np.dtype(kind), -np.finfo(np.float32).max)
    scores = np.full((b, width), pad, dtype=kind)
    idx = np.full((b, width), invalid, dtype=np.int32)
    with np.errstate(over="ignore"):
        _fill_raw(scores, idx, emb, q, cluster_offsets, cluster_ids, cluster_length, n, width,
                  p, valid, valid_index, divisor, scale, partial)
    return scores, idx


def _fill_raw(scores, idx, emb, q, cluster_offsets, cluster_ids, cluster_length, n, width, p,
              valid, valid_index, divisor, scale, partial):
    """The slot loop of ``fused_kmean_ann``."""
    b = scores.shape[0]
    for r in range(b):
        ranges = _row_ranges(cluster_ids[r], cluster_length[r], cluster_offsets, n)
        slots = [(pi, s + i, i) for pi, (s, f, _) in enumerate(ranges) for i in range(f)]
        slots += [(pi, s + f + i, f + i) for pi, (s, f, rest) in enumerate(ranges)
                  for i in range(rest)]
        mrow = r if valid_index is None else int(valid_index[r])
        for slot, (pi, pos, off) in enumerate(slots[:width]):
            if valid is not None and not valid[mrow, pos]:
                continue
            if partial is not None:
                cum, first, words = partial
                e = mrow * p + pi
                w0 = 0 if e == 0 else int(cum[e - 1])
                bit = int(first[e]) + off
                word = int(np.asarray(words).view(np.uint64)[w0 + bit // 64])
                if not (word >> (63 - bit % 64)) & 1:
                    continue
            if emb.dtype == np.int8:
                dot = int(emb[pos].astype(np.int64) @ q[r].astype(np.int64))
                # fp16 conversions of |values| above 65504 give +-inf, as the device's do
                if scale is not None:
                    h = np.float16(np.float32(dot))
                    scores[r, slot] = np.float16(np.float32(h) / np.float32(scale[pos]))
                elif divisor != -1:
                    scores[r, slot] = np.float16(np.float32(dot) / np.float32(divisor))
                else:
                    scores[r, slot] = dot
            else:
                dot = float(emb[pos].astype(np.float64) @ q[r].astype(np.float64))
                scores[r, slot] = np.asarray(np.float32(dot)).astype(scores.dtype)
            idx[r, slot] = pos
