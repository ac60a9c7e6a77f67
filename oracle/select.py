"""Exact top-k selection, ties to the lower index (test infrastructure; see ``oracle/__init__``).

The rule restated here is ``evaluation/bench/oracle.py:83-92`` (``_merge_topk``: equal
scores go to the lowest id) and ``silvertorch/.../fork_search_cuda.cu:50-81`` (keys equal to
the threshold are taken in index order; winners sorted by ``(key desc, slot asc)``).

Pinned by: the reference harness's tie known-answer test (two identical items 2 and 13, the
lower id first; ``evaluation/tests/bench/test_oracle.py:300-324``) kept as a fixture under
``tests/golden/``, and by brute force (a full Python ``sorted`` over ``(-score, id)``) on
small random inputs with heavy ties in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import numpy as np

INT32_MIN = -(2**31)


def topk_rows(
    scores: np.ndarray,
    k: int,
    valid: np.ndarray | None = None,
    *,
    pad_score=None,
) -> tuple[np.ndarray, np.ndarray]:
    """Row-wise top-``k`` of ``scores [B, N]`` by ``(score desc, column asc)``.

    Columns where ``valid`` is False are never selected. Rows with fewer than ``k`` selectable
    columns are padded with id ``-1`` and ``pad_score`` (default: ``INT32_MIN`` for integer
    scores, ``-inf`` for floating ones). Returns ``(ids int64 [B, k], scores [B, k])``."""
    scores = np.asarray(scores)
    b, n = scores.shape
    if pad_score is None:
        pad_score = INT32_MIN if np.issubdtype(scores.dtype, np.integer) else -np.inf
    out_ids = np.full((b, k), -1, dtype=np.int64)
    out_s = np.full((b, k), pad_score, dtype=scores.dtype)
    for r in range(b):
        s = scores[r]
        cols = np.arange(n, dtype=np.int64)
        if valid is not None:
            cols = cols[np.asarray(valid[r], dtype=bool)]
            s = s[cols]
        m = cols.shape[0]
        if m == 0:
            continue
        kk = min(k, m)
        if m > 4 * kk:
            # everything >= the kk-th largest value, so the whole boundary tie group is kept
            thr = np.partition(s, m - kk)[m - kk]
            keep = s >= thr
            cols, s = cols[keep], s[keep]
        # stable sort on the negated score keeps ascending column order inside a tie
        order = np.argsort(_neg(s), kind="stable")[:kk]
        out_ids[r, :kk] = cols[order]
        out_s[r, :kk] = s[order]
    return out_ids, out_s


def _neg(s: np.ndarray) -> np.ndarray:
    if np.issubdtype(s.dtype, np.integer):
        return -s.astype(np.int64)
    return -s.astype(np.float64)


class RepeatedRows:
    """``topk_rows`` for a table whose N rows each copy one of R distinct base rows, so that an
    item's score is its base row's: ``topk(base_scores[b], row_of_item, k, valid)`` equals
    ``topk_rows(base_scores[:, row_of_item], k, valid)`` without the ``[B, N]`` matrix. The items
    are taken score group by score group in descending order (a group = every base row of one
    score value), each group's items in ascending index, until k pass ``valid``: the same
    (score desc, index asc) order. Pinned against ``topk_rows`` on small tables with heavy ties
    across and within base rows (``tests/test_oracle.py``)."""

    def __init__(self, row_of_item: np.ndarray, n_base: int):
        rows = np.asarray(row_of_item, np.int64)
        self.n = rows.size
        self.order = np.argsort(rows, kind="stable")  # items of base row j, ascending index
        self.starts = np.searchsorted(rows[self.order], np.arange(n_base + 1))

    def items_of(self, base: np.ndarray) -> np.ndarray:
        parts = [self.order[self.starts[j]:self.starts[j + 1]] for j in np.asarray(base).tolist()]
        return np.sort(np.concatenate(parts)) if parts else np.empty(0, np.int64)

    def topk(self, base_scores: np.ndarray, k: int, valid: np.ndarray | None = None,
             pad_score=None) -> tuple[np.ndarray, np.ndarray]:
        """One query: ``base_scores [R]``, ``valid [N]`` bool → ``(ids [k], scores [k])``."""
        s = np.asarray(base_scores)
        if pad_score is None:
            pad_score = INT32_MIN if np.issubdtype(s.dtype, np.integer) else -np.inf
        neg = _neg(s)
        r = neg.size
        m = min(r, 64)
        while True:
            ids = np.full(k, -1, np.int64)
            out = np.full(k, pad_score, dtype=s.dtype)
            # the m best base rows; every row scoring above the worst of them is among them
            cand = np.argpartition(neg, m - 1)[:m] if m < r else np.arange(r)
            lim = neg[cand].max()
            got = 0
            for v in np.unique(neg[cand]).tolist():  # descending score
                # (the worst value's rows may lie partly outside the m: take all of them)
                rows = cand[neg[cand] == v] if v < lim else np.flatnonzero(neg == v)
                items = self.items_of(rows)
                if valid is not None:
                    items = items[np.asarray(valid, bool)[items]]
                take = min(k - got, items.size)
                ids[got:got + take] = items[:take]
                out[got:got + take] = s[rows[0]]
                got += take
                if got == k:
                    return ids, out
            if m == r:
                return ids, out
            m = min(r, 4 * m)


def merge_topk(
    s_a: np.ndarray, i_a: np.ndarray, s_b: np.ndarray, i_b: np.ndarray, k: int
) -> tuple[np.ndarray, np.ndarray]:
    """Top-``k`` of two candidate lists per row, equal scores to the lowest id: a stable sort
    by id, then a stable sort by descending score (``evaluation/bench/oracle.py:83-92``).
    Returns ``(scores, ids)`` like the reference."""
    cs = np.concatenate([s_a, s_b], axis=1)
    ci = np.concatenate([i_a, i_b], axis=1)
    by_id = np.argsort(ci, axis=1, kind="stable")
    cs = np.take_along_axis(cs, by_id, 1)
    ci = np.take_along_axis(ci, by_id, 1)
    by_score = np.argsort(_neg(cs), axis=1, kind="stable")[:, :k]
    return np.take_along_axis(cs, by_score, 1), np.take_along_axis(ci, by_score, 1)


def composite_key(score_i32: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """``(key desc, slot asc)`` in one uint64 that orders descending
    (``fork_search_cuda.cu:65-81``): high word = the int32 score with its sign bit flipped,
    low word = ``0xffffffff - idx``."""
    key = (np.asarray(score_i32).astype(np.int64) + 2**31).astype(np.uint64)
    return (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.asarray(idx).astype(np.uint64))
