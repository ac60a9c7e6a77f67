"""The reference's CPU path, timed by ``bench.py`` as the CPU baseline (test infrastructure; see
``oracle/__init__``). Restates ``evaluation/bench/oracle.py:95-158``: ``torch.mm`` over item
chunks of 2M rows (``ITEM_CHUNK``, ``oracle.py:20-22``), ``torch.topk`` per chunk, and the
lowest-id merge ``_merge_topk`` (``oracle.py:83-92``). int8 codes are cast to float32, which
is exact (``|dot| <= 512 * 127**2 < 2**24``).
"""

from __future__ import annotations

import time

import numpy as np
import torch

ITEM_CHUNK = 2_000_000


def _merge(best_s, best_i, s, i, k):
    cs, ci = torch.cat([best_s, s], 1), torch.cat([best_i, i], 1)
    by_id = ci.argsort(dim=1, stable=True)
    cs, ci = cs.gather(1, by_id), ci.gather(1, by_id)
    by_score = cs.argsort(dim=1, descending=True, stable=True)[:, :k]
    return cs.gather(1, by_score), ci.gather(1, by_score)


def int8_topk_cpu(q_codes: torch.Tensor, item_codes: torch.Tensor, k: int, chunk: int = ITEM_CHUNK,
                  valid_fn=None):
    """``(ids [B, k], scores float32 [B, k])`` of the int8 dot, ties to the lowest id.
    ``valid_fn(start, stop)`` (optional) gives the ``[B, stop - start]`` bool filter of a chunk:
    failing items score ``-inf`` before the chunk's ``topk`` (the postfilter gate of
    ``evaluation/bench/postfilter.py:41-59``)."""
    q = q_codes.float()
    b = q.shape[0]
    best_s = torch.full((b, k), float("-inf"))
    best_i = torch.full((b, k), -1, dtype=torch.long)
    for start in range(0, item_codes.shape[0], chunk):
        part = item_codes[start : start + chunk].float()
        scores = q @ part.t()
        if valid_fn is not None:
            scores = scores.masked_fill(~valid_fn(start, start + part.shape[0]), float("-inf"))
        top = torch.topk(scores, min(k, part.shape[0]), dim=1)
        best_s, best_i = _merge(best_s, best_i, top.values, top.indices + start, k)
    return best_i, best_s


def clause_sets_valid(item_attrs: torch.Tensor, query_sets: torch.Tensor):
    """``valid_fn`` of value-set clauses: ``[N, C, A]`` attrs, ``[B, C, V]`` sets (``-1``
    pads, an all ``-1`` clause inactive); clause ``c`` passes iff an item value is in the set."""

    def fn(start, stop):
        part = item_attrs[start:stop]
        out = torch.ones((query_sets.shape[0], part.shape[0]), dtype=torch.bool)
        for r in range(query_sets.shape[0]):
            for c in range(query_sets.shape[1]):
                vals = query_sets[r, c][query_sets[r, c] != -1]
                if vals.numel():
                    out[r] &= torch.isin(part[:, c, :], vals).any(1)
        return out

    return fn


def time_int8(q_codes, item_sample, k: int, reps: int = 3, valid_fn=None) -> tuple[float, int]:
    """Median seconds of ``int8_topk_cpu`` over ``reps`` runs, and the threads used."""
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        int8_topk_cpu(q_codes, item_sample, k, valid_fn=valid_fn)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], torch.get_num_threads()


def time_topk(q, item_sample, k: int, reps: int = 3, valid_fn=None) -> tuple[float, int]:
    """``time_int8`` for any item dtype (bf16 / fp16 items are scored in float32, as the
    reference's CPU branch of ``PostfilterKNN.score`` does, ``retrieve/src/retrieve/modules/
    knn.py:62-66``)."""
    return time_int8(q, item_sample, k, reps=reps, valid_fn=valid_fn)


_NO_SCORE = -(1 << 40)  # below every score, and safe to negate in the sort key


def hamming_topk_cpu(q_bits: np.ndarray, item_bits: np.ndarray, k: int,
                     valid: np.ndarray | None = None, chunk: int = 1 << 15):
    """The 1-bit top-k on the host: score ``64 W - 2 popcount(q ^ item)``
    (``retrieve/src/retrieve/ops/reference/oporp_1bit_match_topk.py:9-41``), failing items
    excluded, top ``k`` by (score desc, id asc). Returns ``(scores, ids)`` [B, k] (ids -1 and
    scores below every score where fewer items pass)."""
    b = q_bits.shape[0]
    n = item_bits.shape[0]
    qb = q_bits.view(np.uint64)
    ib = item_bits.view(np.uint64)
    w = ib.shape[1]
    best_s = np.full((b, k), _NO_SCORE, np.int64)
    best_i = np.full((b, k), -1, np.int64)
    for s in range(0, n, chunk):
        part = ib[s : s + chunk]
        pc = np.zeros((b, part.shape[0]), np.int64)
        for j in range(w):
            pc += np.bitwise_count(qb[:, None, j] ^ part[None, :, j]).astype(np.int64)
        sc = 64 * w - 2 * pc
        if valid is not None:
            sc[~valid[:, s : s + part.shape[0]]] = _NO_SCORE
        ids = np.broadcast_to(np.arange(s, s + part.shape[0]), sc.shape)
        cs = np.concatenate([best_s, sc], 1)
        ci = np.concatenate([best_i, ids], 1)
        order = np.lexsort((ci, -cs), axis=1)[:, :k]
        best_s = np.take_along_axis(cs, order, 1)
        best_i = np.take_along_axis(ci, order, 1)
    return best_s, best_i


def hamming_rerank_cpu(q_bits: np.ndarray, q_codes: np.ndarray, item_bits: np.ndarray,
                       item_codes: np.ndarray, k1: int, k: int, valid: np.ndarray | None = None,
                       chunk: int = 1 << 15):
    """The 1-bit retrieval with int8 re-rank on the host: the top ``k1`` of
    ``hamming_topk_cpu``, then the int8 dots of those candidates
    (``modules/silvertorch.py:363-379``), top ``k`` by (dot desc, id asc). Returns ids [B, k]."""
    b = q_bits.shape[0]
    best_s, best_i = hamming_topk_cpu(q_bits, item_bits, k1, valid, chunk)
    out = np.full((b, k), -1, np.int64)
    for r in range(b):
        cand = best_i[r][(best_i[r] >= 0) & (best_s[r] > _NO_SCORE)]
        dots = item_codes[cand].astype(np.int64) @ q_codes[r].astype(np.int64)
        order = np.lexsort((cand, -dots))[:k]
        out[r, : order.size] = cand[order]
    return out
