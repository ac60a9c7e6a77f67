"""Candidate-list top-k on the GPU against the oracle (``oracle.scan.candidate_topk``):
``fused_masked_knn_topk`` (fp16 / bf16 / fp32 items, fp32 dots within the float tolerance),
``oporp_1bit_match_topk_indirect`` and ``int8_candidates_topk`` (exact), ties to the lower
item id whatever the candidates' order."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from tests.conftest import rng

pytestmark = pytest.mark.gpu

RTOL = 1e-3


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _cands(g, b, p, n, counts_hi=None):
    cand = np.stack([g.permutation(n)[:p] for _ in range(b)]).astype(np.int64)
    counts = g.integers(0, (counts_hi or p) + 1, b).astype(np.int64)
    return cand, counts


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b,n,d,p,k", [(4, 5000, 128, 1000, 100), (3, 2000, 64, 64, 64),
                                       (5, 20000, 256, 4096, 10), (2, 300, 32, 200, 7)])
def test_fused_masked_knn(dev, dtype, b, n, d, p, k):
    g = rng(b * 31 + n + d + p + k)
    print(f"fused_masked_knn {dtype} B={b} N={n} D={d} P={p} k={k}", flush=True)
    q = g.standard_normal((b, d)).astype(np.float32)
    items = torch.from_numpy(g.standard_normal((n, d)).astype(np.float32)).to(dtype)
    cand, counts = _cands(g, b, p, n)
    counts[0] = p
    ids, sc = torch.ops.retrieve.fused_masked_knn_topk(_t(dev, q), items.to(dev), _t(dev, cand),
                                                       _t(dev, counts), k)
    ids, sc = ids.cpu().numpy(), sc.cpu().numpy()
    iv = items.float().numpy().astype(np.float64)
    exact = q.astype(np.float64) @ iv.T  # [b, n]
    want_ids, want_sc = osc.candidate_topk(lambda r, c: exact[r, c], cand, counts, k,
                                           pad_to_k=True, empty_score=-np.inf)
    for r in range(b):
        m = int(min(counts[r], k))
        assert (ids[r, m:] == -1).all() and np.isneginf(sc[r, m:]).all()
        got = ids[r, :m]
        assert set(got.tolist()) <= set(cand[r, : counts[r]].tolist())
        e = exact[r, got]
        scale = np.maximum(np.abs(e), 1.0)
        assert (np.abs(sc[r, :m] - e) <= RTOL * scale).all()
        if m:
            kth = want_sc[r, m - 1]
            band = RTOL * max(abs(kth), 1.0) * 2
            assert (e >= kth - band).all()
            for i in set(want_ids[r, :m].tolist()) - set(got.tolist()):
                assert exact[r, i] <= sc[r, m - 1] + band


def test_fused_masked_knn_ties_and_duplicates(dev):
    """Equal rows: every score ties, so the k lowest candidate ids win; a duplicated id is
    scored twice (as the reference's gather does)."""
    n, d, k = 500, 64, 20
    items = torch.ones((n, d), dtype=torch.float16)
    q = np.ones((1, d), np.float32)
    cand = np.arange(n - 1, -1, -1, dtype=np.int64)[None, :]  # descending order
    ids, sc = torch.ops.retrieve.fused_masked_knn_topk(
        _t(dev, q), items.to(dev), _t(dev, cand), _t(dev, np.array([n])), k)
    assert ids.cpu().tolist() == [list(range(k))]
    cand2 = np.array([[7, 7, 3, 9]], np.int64)
    ids2, _ = torch.ops.retrieve.fused_masked_knn_topk(
        _t(dev, q), items.to(dev), _t(dev, cand2), _t(dev, np.array([4])), 4)
    assert ids2.cpu().tolist() == [[3, 7, 7, 9]]


def test_duplicated_candidate_at_the_boundary(dev):
    """A candidate repeated many times ties with itself at the k-th place: the better item
    listed once must still win (the merge takes every entry above the k-th, then repeats)."""
    d = 64
    items = np.zeros((4, d), np.int8)
    items[1, :] = 2  # best
    items[2, :] = 1  # repeated
    q = np.ones((1, d), np.int8)
    for reps in (7, 300, 5000):
        cand = np.array([[2] * reps + [1] + [3] * 20], np.int64)
        ids, sc = torch.ops.retrieve_amd.int8_candidates_topk(
            _t(dev, q), _t(dev, items), _t(dev, cand), _t(dev, np.array([cand.shape[1]])), 5)
        assert ids.cpu().tolist() == [[1, 2, 2, 2, 2]], reps
        assert sc.cpu().tolist() == [[128, 64, 64, 64, 64]]


def test_oporp_indirect(dev):
    g = rng(92)
    b, n, w, p = 6, 30000, 8, 2000
    qb = g.integers(-(2**63), 2**63 - 1, (b, w), dtype=np.int64)
    ib = g.integers(-(2**63), 2**63 - 1, (n, w), dtype=np.int64)
    ib[100:200] = ib[100]  # a tie group
    cand, counts = _cands(g, b, p, n)
    cand[1, :150] = np.arange(199, 49, -1)  # the tie group, in descending id order
    counts[1] = 150
    for k, pp in ((100, p), (1000, p), (5000, 700)):  # k > P: min(k, P) columns
        cand_k = np.ascontiguousarray(cand[:, :pp])
        ids, sc = torch.ops.retrieve.oporp_1bit_match_topk_indirect(
            _t(dev, qb), _t(dev, ib), k, _t(dev, cand_k), _t(dev, counts))
        want_ids, want_sc = osc.candidate_topk(
            lambda r, c: osc.hamming_scores(qb[r:r + 1], ib[c])[0], cand_k, counts, k,
            pad_to_k=False, empty_score=-np.inf)
        assert ids.shape == (b, min(k, pp))
        assert np.array_equal(ids.cpu().numpy(), want_ids)
        assert np.array_equal(sc.cpu().numpy(), want_sc.astype(np.float32))


def test_int8_candidates_rerank(dev):
    """Config 5's second stage: Hamming top-1000 (score order) → int8 re-rank to top-100."""
    g = rng(93)
    b, n, d = 8, 50000, 512
    codes = g.integers(-128, 128, (n, d), dtype=np.int8)
    codes[1000:1100] = codes[1000]  # ties
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    bits = g.integers(-(2**63), 2**63 - 1, (n, 8), dtype=np.int64)
    qbits = g.integers(-(2**63), 2**63 - 1, (b, 8), dtype=np.int64)
    hids, _ = torch.ops.retrieve_amd.hamming_scan_topk(_t(dev, qbits), _t(dev, bits), 1000)
    hids[:, :100] = torch.arange(1099, 999, -1, device=dev)  # ties, descending ids
    counts = torch.full((b,), 1000, dtype=torch.int64, device=dev)
    ids, sc = torch.ops.retrieve_amd.int8_candidates_topk(_t(dev, q), _t(dev, codes), hids, counts,
                                                      100)
    cand = hids.cpu().numpy()
    want_ids, want_sc = osc.candidate_topk(
        lambda r, c: osc.int8_scores(q[r:r + 1], codes[c])[0], cand, np.full(b, 1000), 100,
        pad_to_k=False, empty_score=np.iinfo(np.int32).min)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(sc.cpu().numpy(), want_sc.astype(np.int32))


def test_large_p_and_bad_ids(dev):
    g = rng(94)
    b, n, d, p, k = 3, 400_000, 128, 300_000, 100
    codes = g.integers(-128, 128, (n, d), dtype=np.int8)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    cand, counts = _cands(g, b, p, n)
    counts[2] = p
    counts[0] = max(counts[0], 1000)  # enough valid candidates to fill k
    cand[0, 5] = -3  # outside the table: skipped
    cand[0, 6] = n + 10
    ids, sc = torch.ops.retrieve_amd.int8_candidates_topk(_t(dev, q), _t(dev, codes), _t(dev, cand),
                                                      _t(dev, counts), k)

    def score(r, c):
        s = np.full(c.size, -(2**40))  # below every int32 dot (and safe to negate)
        ok = (c >= 0) & (c < n)
        s[ok] = osc.int8_scores(q[r:r + 1], codes[c[ok]])[0]
        return s

    want_ids, want_sc = osc.candidate_topk(score, cand, counts, k, pad_to_k=False,
                                           empty_score=np.iinfo(np.int32).min)
    got = ids.cpu().numpy()
    for r in range(b):
        assert np.array_equal(got[r], want_ids[r]), (r, counts[r], got[r, :8], want_ids[r, :8])
    assert np.array_equal(sc.cpu().numpy(), want_sc.astype(np.int32))


def test_errors(dev):
    q = torch.zeros((2, 64), device=dev)
    items = torch.zeros((10, 64), dtype=torch.float16, device=dev)
    cand = torch.zeros((2, 5), dtype=torch.int64, device=dev)
    counts = torch.full((2,), 5, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        torch.ops.retrieve.fused_masked_knn_topk(q, items, cand, counts, 6)  # P < k
    with pytest.raises(TypeError):
        torch.ops.retrieve.fused_masked_knn_topk(q, items.int(), cand, counts, 3)
    with pytest.raises(ValueError):
        torch.ops.retrieve.fused_masked_knn_topk(q, items, cand[:, :, None], counts, 3)
    with pytest.raises(TypeError):
        torch.ops.retrieve.oporp_1bit_match_topk_indirect(q, items, 3, cand, counts)
