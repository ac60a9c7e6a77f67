"""Brute-force scans + top-k (test infrastructure; see ``oracle/__init__``).

Pinned by:
- int8: the reference's hand-computed known answer ``[1,2]·[5,6] = 17``, ``[3,4]·[5,6] = 39``
  (``silvertorch/.../tests/test_fused_kmean_ann.py:353-380``) and an element-by-element
  Python-int dot on small random inputs (``tests/test_oracle.py``). The float64 BLAS product
  used here is exact: ``|dot| <= 1024 * 128 * 128 = 2**24``.
- Hamming: the popcount known answer ``[0, 1, 2, 3, -1, 0x5555...] -> [0, 1, 1, 2, 64, 32]``
  (``retrieve/tests/correctness/test_quantize.py:195-199``), Python ``bin(x).count("1")`` on
  random words, and the identity ``64 W - 2 * hamming == dot of the ±1 expansions``.
- dense: float64 brute force; the GPU's float32 scores are compared to it with a tolerance.
- selection: ``oracle.select``.
"""

from __future__ import annotations

import numpy as np

from oracle.select import topk_rows

_CHUNK = 1 << 20


def int8_scores(q_codes: np.ndarray, item_codes: np.ndarray) -> np.ndarray:
    """``[B, D]`` int8 × ``[N, D]`` int8 → ``[B, N]`` int32 exact dot products (the int32
    accumulation of ``simple_index_mm.cuh:72-94`` / ``fused_kmean_ann.cpp:60-70``)."""
    if q_codes.shape[1] != item_codes.shape[1] or q_codes.shape[1] > 1024:
        raise ValueError("D mismatch or D > 1024 (the float64 product would not be exact)")
    out = np.asarray(q_codes, np.float64) @ np.asarray(item_codes, np.float64).T
    return out.astype(np.int32)


def int8_topk(
    q_codes: np.ndarray, item_codes: np.ndarray, k: int, valid: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Top-``k`` int32 dots per query, ties to the lower item index, ``-1`` / ``INT32_MIN``
    pads (the selection of ``fork_search_cuda.cu:142-440`` on a single cluster, where slot ==
    item index). ``valid [B, N]`` bool masks items out."""
    return topk_rows(int8_scores(q_codes, item_codes), k, valid)


def popcount64(x: np.ndarray) -> np.ndarray:
    """Popcount of int64 words as int32 (``retrieve/src/retrieve/functional.py:158-170``)."""
    return np.bitwise_count(np.asarray(x).view(np.uint64)).astype(np.int32)


def hamming_scores(q_bits: np.ndarray, item_bits: np.ndarray) -> np.ndarray:
    """``64 W - 2 * popcount(q ^ item)`` as int32 ``[B, N]``
    (``retrieve/src/retrieve/ops/reference/oporp_1bit_match_topk.py:9-17``)."""
    q = np.asarray(q_bits).view(np.uint64)
    it = np.asarray(item_bits).view(np.uint64)
    w = q.shape[1]
    out = np.empty((q.shape[0], it.shape[0]), dtype=np.int32)
    for r in range(q.shape[0]):
        ham = np.bitwise_count(it ^ q[r][None, :]).sum(axis=1, dtype=np.int32)
        out[r] = 64 * w - 2 * ham
    return out


def hamming_topk(
    q_bits: np.ndarray, item_bits: np.ndarray, k: int, valid: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Full-scan Hamming top-``k`` on the integer score, ties to the lower index
    (``ops/reference/oporp_1bit_match_topk.py:20-28`` with the lowest-index rule)."""
    return topk_rows(hamming_scores(q_bits, item_bits), k, valid)


def dense_scores(q: np.ndarray, items: np.ndarray) -> np.ndarray:
    """float64 ``q @ items.T`` (the exact reference the float32 scores are bounded against,
    ``retrieve/tests/parity/test_accumulation.py:31-32``)."""
    return np.asarray(q, np.float64) @ np.asarray(items, np.float64).T


def dense_topk(
    q: np.ndarray, items: np.ndarray, k: int, valid: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Exact float64 top-``k``, ties to the lower index, ``-1`` / ``-inf`` pads."""
    return topk_rows(dense_scores(q, items), k, valid)


def dense_topk_chunked(
    q: np.ndarray, items: np.ndarray, k: int, valid: np.ndarray | None = None,
    chunk: int = 1 << 15,
) -> tuple[np.ndarray, np.ndarray]:
    """``dense_topk`` computed over item chunks, for tables whose ``[B, N]`` float64 score
    matrix does not fit in memory: per chunk the entries at or above each row's chunk-local
    k-th largest score (the whole boundary tie group), then one lowest-id selection over the
    survivors. The chunk-then-merge structure of the reference's CPU oracle
    (``evaluation/bench/oracle.py:95-158``, ``ITEM_CHUNK``; the merge rule ``:83-92``), in
    float64 on torch's CPU kernels (the chunk's k-th value only: its tie order is irrelevant,
    every entry equal to it is kept). Pinned against ``dense_topk`` on small inputs with heavy
    ties (``tests/test_oracle.py``)."""
    import torch

    q64 = torch.from_numpy(np.ascontiguousarray(q, np.float64))
    b = q64.shape[0]
    n = items.shape[0]
    keep_s: list[list[np.ndarray]] = [[] for _ in range(b)]
    keep_i: list[list[np.ndarray]] = [[] for _ in range(b)]
    for s0 in range(0, n, chunk):
        part = torch.from_numpy(np.ascontiguousarray(items[s0 : s0 + chunk], np.float64))
        sc = q64 @ part.T
        m = sc.shape[1]
        if valid is not None:
            v = torch.from_numpy(np.ascontiguousarray(valid[:, s0 : s0 + m], bool))
            sc = sc.masked_fill(~v, float("-inf"))
        kk = min(k, m)
        thr = sc.topk(kk, dim=1).values[:, kk - 1 :]
        sc = sc.numpy()
        rows, cols = np.nonzero(((sc >= thr.numpy()) & np.isfinite(sc)))
        bounds = np.searchsorted(rows, np.arange(b + 1))
        for r in range(b):
            c = cols[bounds[r] : bounds[r + 1]]
            keep_s[r].append(sc[r, c])
            keep_i[r].append(c.astype(np.int64) + s0)
    ids = np.full((b, k), -1, np.int64)
    out = np.full((b, k), -np.inf)
    for r in range(b):
        s = np.concatenate(keep_s[r]) if keep_s[r] else np.empty(0)
        i = np.concatenate(keep_i[r]) if keep_i[r] else np.empty(0, np.int64)
        order = np.lexsort((i, -s))[:k]
        ids[r, : order.size] = i[order]
        out[r, : order.size] = s[order]
    return ids, out


def candidate_int8_topk(
    q_codes: np.ndarray,
    item_codes: np.ndarray,
    candidate_ids: np.ndarray,
    k: int,
) -> tuple[np.ndarray, np.ndarray]:
    """Re-rank ``candidate_ids [B, P]`` (``-1`` = padding, never scored) by the int32 dot;
    top ``min(k, P)`` by ``(score desc, id asc)``; short rows end in ``-1`` / ``INT32_MIN``.
    The selection order of ``modules/silvertorch.py:363-379`` with the lowest-id rule (the
    reference's ``torch.topk`` leaves tie order unspecified)."""
    b, p = candidate_ids.shape
    kk = min(k, p)
    ids = np.full((b, kk), -1, np.int64)
    sc = np.full((b, kk), np.iinfo(np.int32).min, np.int32)
    for r in range(b):
        c = candidate_ids[r]
        c = c[c >= 0]
        if c.size == 0:
            continue
        s = int8_scores(q_codes[r : r + 1], item_codes[c])[0]
        # primary: score desc; then id asc; then position (lexsort is stable)
        order = np.lexsort((c, -s.astype(np.int64)))[:kk]
        ids[r, : order.size] = c[order]
        sc[r, : order.size] = s[order]
    return ids, sc


def candidate_topk(
    scores_fn, candidate_ids: np.ndarray, counts: np.ndarray, k: int, *, pad_to_k: bool,
    empty_score,
) -> tuple[np.ndarray, np.ndarray]:
    """Top-k over ``candidate_ids[b, :counts[b]]`` by (score desc, item id asc); ``scores_fn(b,
    ids)`` scores one row's candidates. ``min(k, P)`` columns unless ``pad_to_k``; slots past a
    row's candidates hold ``-1`` / ``empty_score``. The selection of ``masked_topk`` with
    ``valid = counts_to_valid(counts, P)`` (``functional.py:52-85``;
    ``ops/reference/fused_masked_knn_topk.py:9-29``, ``oporp_1bit_match_topk.py:29-41``), ties
    by the lowest-id rule."""
    b, p = candidate_ids.shape
    kk = k if pad_to_k else min(k, p)
    ids = np.full((b, kk), -1, np.int64)
    sc = np.full((b, kk), empty_score)
    for r in range(b):
        c = candidate_ids[r, : max(0, min(int(counts[r]), p))]
        if c.size == 0:
            continue
        s = np.asarray(scores_fn(r, c))
        order = np.lexsort((c, -s))[: min(kk, c.size)]
        ids[r, : order.size] = c[order]
        sc[r, : order.size] = s[order]
    return ids, sc


def gemv_scores(q16: np.ndarray, e_t16: np.ndarray) -> np.ndarray:
    """``[D]`` fp16 query against the ``[D, N]`` fp16 table → ``[N]`` float32, acc =
    fma(q[k], e[k, :], acc) for k = 0 .. D-1 (``ops/triton/gemv_scores.py:19-28``). The product of
    two fp16 values is exact in float32, so each fma is one float32 add of the exact product."""
    q = np.asarray(q16, np.float16).astype(np.float32)
    e = np.asarray(e_t16, np.float16)
    acc = np.zeros(e.shape[1], np.float32)
    for k in range(e.shape[0]):
        acc = acc + q[k] * e[k].astype(np.float32)
    return acc
