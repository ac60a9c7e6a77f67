"""Exact clause filter on the GPU against the oracle's predicate (``oracle.filters.clause_match``
/ ``clause_match_sets``): ``torch.ops.retrieve.clause_mask`` / ``clause_mask_scores`` /
``clause_compact`` with the reference's schemas, the packed ``clause_bits`` the scans take, and
``mask_compact``. Cases follow ``retrieve/tests/correctness/test_filters.py``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import filters as of
from oracle import scan as osc
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _attrs(g, n, c, a, vocab, pad_rate):
    x = g.integers(0, vocab, (n, c, a), dtype=np.int64)
    x[g.random((n, c, a)) < pad_rate] = -1
    return x


def _queries(g, b, c, vocab, inactive_rate):
    q = g.integers(0, vocab, (b, c), dtype=np.int64)
    q[g.random((b, c)) < inactive_rate] = -1
    return q


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _mask(dev, attrs, rev, q):
    print(f"clause_mask N={attrs.shape[0]} C={attrs.shape[1]} A={attrs.shape[2]} B={q.shape[0]}",
          flush=True)
    out = torch.ops.retrieve.clause_mask(_t(dev, attrs), _t(dev, rev), _t(dev, q))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_and_or_semantics(dev):
    """Per-clause OR over an item's values, AND across clauses, -1 inactive (the reference's
    hand-checked case, ``test_filters.py:14-43``)."""
    n = 200
    attrs = np.full((n, 2, 2), -1, np.int64)
    attrs[:100, 0, 0] = 1
    attrs[100:, 0, 0] = 2
    attrs[:, 1, 0] = 50
    attrs[50:70, 0, 1] = 3
    q = np.array([[1, 50], [2, 50], [3, -1], [-1, -1]], np.int64)
    m = _mask(dev, attrs, np.zeros(2, bool), q)
    assert m[0, :100].all() and not m[0, 100:].any()
    assert m[1, 100:].all() and not m[1, :100].any()
    assert m[2, 50:70].all() and not m[2, :50].any() and not m[2, 70:].any()
    assert m[3].all()
    assert np.array_equal(m, of.clause_match(attrs, np.zeros(2, bool), q))


@pytest.mark.parametrize(
    "n,c,a,vocab,b,rev",
    [(4096, 3, 4, 20, 8, (0, 0, 0)), (1024, 2, 3, 10, 4, (1, 0)), (1, 2, 2, 12, 3, (0, 1)),
     (100_003, 8, 1, 16, 5, (0, 0, 1, 0, 0, 0, 0, 0)), (777, 5, 4, 6, 70, (1, 1, 0, 0, 1)),
     (3000, 9, 2, 8, 3, (0,) * 9)],
)
def test_random_parity(dev, n, c, a, vocab, b, rev):
    """Pads, multi-value clauses, reverse and inactive clauses; C * A above 16 takes the path that
    reads attributes from memory."""
    g = rng(n + c * 7 + a * 13 + b)
    attrs = _attrs(g, n, c, a, vocab, 0.3)
    q = _queries(g, b, c, vocab, 0.3)
    rev = np.array(rev, bool)
    assert np.array_equal(_mask(dev, attrs, rev, q), of.clause_match(attrs, rev, q))


def test_all_reverse(dev):
    g = rng(51)
    attrs = _attrs(g, 256, 2, 2, 20, 0.0)
    q = _queries(g, 4, 2, 20, 0.0)
    m = _mask(dev, attrs, np.ones(2, bool), q)
    matched = (attrs[None] == q[:, None, :, None]).any(-1)
    assert np.array_equal(m, (~matched).all(-1))


def test_single_item(dev):
    attrs = np.array([[[5, -1], [10, -1]]], np.int64)
    q = np.array([[5, 10], [5, 11], [-1, -1]], np.int64)
    rev = np.zeros(2, bool)
    assert _mask(dev, attrs, rev, q)[:, 0].tolist() == [True, False, True]
    ids, counts = torch.ops.retrieve.clause_compact(_t(dev, attrs), _t(dev, rev), _t(dev, q))
    assert counts.tolist() == [1, 0, 1]
    assert ids[0, 0].item() == 0 and ids[2, 0].item() == 0


def test_mask_scores(dev):
    g = rng(52)
    attrs = _attrs(g, 5000, 3, 2, 9, 0.2)
    q = _queries(g, 6, 3, 9, 0.3)
    rev = np.array([0, 1, 0], bool)
    scores = g.standard_normal((6, 5000)).astype(np.float32)
    got = torch.ops.retrieve.clause_mask_scores(_t(dev, scores), _t(dev, attrs), _t(dev, rev),
                                                _t(dev, q)).cpu().numpy()
    want = np.where(of.clause_match(attrs, rev, q), scores, -np.inf).astype(np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [1, 63, 64, 65, 8191, 8192 * 3 + 17, 300_000])
def test_compact_ascending(dev, n):
    g = rng(53 + n)
    attrs = _attrs(g, n, 3, 2, 6, 0.2)
    q = _queries(g, 7, 3, 6, 0.2)
    q[0] = -1  # every item passes
    rev = np.array([0, 0, 1], bool)
    ids, counts = torch.ops.retrieve.clause_compact(_t(dev, attrs), _t(dev, rev), _t(dev, q))
    ids, counts = ids.cpu().numpy(), counts.cpu().numpy()
    want = of.clause_match(attrs, rev, q)
    assert counts.tolist() == want.sum(1).tolist()
    for r in range(7):
        assert np.array_equal(ids[r, : counts[r]], np.flatnonzero(want[r]))


def test_bits_layout_and_and_mask(dev):
    g = rng(54)
    n = 10_000
    attrs = _attrs(g, n, 4, 2, 7, 0.1)
    q = _queries(g, 9, 4, 7, 0.4)
    rev = np.array([1, 0, 0, 1], bool)
    want = of.clause_match(attrs, rev, q)
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, rev), _t(dev, q))
    assert np.array_equal(bits.cpu().numpy(), _pack(want))
    pre = g.random((9, n)) < 0.5
    bits2 = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, rev), _t(dev, q),
                                           _t(dev, _pack(pre)))
    assert np.array_equal(bits2.cpu().numpy(), _pack(want & pre))


def test_value_sets(dev):
    """``[B, C, V]`` value sets against ``clause_match_sets``; V == 1 equals the reference query."""
    g = rng(55)
    n, c = 20_000, 3
    attrs = _attrs(g, n, c, 2, 12, 0.2)
    sets = g.integers(0, 12, (11, c, 4), dtype=np.int64)
    sets[g.random(sets.shape) < 0.4] = -1
    sets[3] = -1  # no active clause
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, np.zeros(c, bool)),
                                          _t(dev, sets))
    assert np.array_equal(bits.cpu().numpy(), _pack(of.clause_match_sets(attrs, sets)))


def test_mask_compact_random_bits(dev):
    g = rng(56)
    n = 50_001
    valid = g.random((5, n)) < np.array([0.0, 0.01, 0.5, 0.99, 1.0])[:, None]
    words = _pack(valid)
    words[:, -1] |= np.int64(0x7FFF)  # bits past item n - 1 are ignored
    ids, counts = torch.ops.retrieve_amd.mask_compact(_t(dev, words), n)
    ids, counts = ids.cpu().numpy(), counts.cpu().numpy()
    for r in range(5):
        assert counts[r] == valid[r].sum()
        assert np.array_equal(ids[r, : counts[r]], np.flatnonzero(valid[r]))


def test_filtered_int8_scan(dev):
    """The packed clause mask gating the int8 scan equals the oracle's masked top-k."""
    g = rng(57)
    n, d, b, k = 40_000, 128, 6, 50
    attrs = _attrs(g, n, 2, 1, 10, 0.0)
    q = _queries(g, b, 2, 10, 0.2)
    rev = np.zeros(2, bool)
    codes = g.integers(-128, 128, (n, d), dtype=np.int8)
    qc = g.integers(-128, 128, (b, d), dtype=np.int8)
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, rev), _t(dev, q))
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk(_t(dev, qc), _t(dev, codes), k, bits)
    want_ids, want_sc = osc.int8_topk(qc, codes, k, of.clause_match(attrs, rev, q))
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


def test_errors(dev):
    attrs = torch.zeros((10, 2, 1), dtype=torch.int64, device=dev)
    rev = torch.zeros(2, dtype=torch.bool, device=dev)
    q = torch.zeros((3, 2), dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        torch.ops.retrieve.clause_mask(attrs[:, :, 0], rev, q)
    with pytest.raises(ValueError):
        torch.ops.retrieve.clause_mask(attrs, rev, q[:, :1])
    with pytest.raises(ValueError):
        torch.ops.retrieve.clause_mask(attrs.transpose(0, 1).contiguous().transpose(0, 1), rev, q)
    with pytest.raises(TypeError):
        torch.ops.retrieve.clause_mask(attrs.int(), rev, q)
    with pytest.raises(ValueError):
        torch.ops.retrieve.clause_mask_scores(torch.zeros(3, 9, device=dev), attrs, rev, q)


@pytest.mark.parametrize("dtype", [np.int16, np.int32])
def test_compact_attr_tables(dev, dtype):
    """``clause_bits`` over an int16 / int32 copy of the table equals the int64 oracle."""
    g = rng(58)
    n, c = 70_000, 8
    attrs = _attrs(g, n, c, 1, 1000, 0.1)
    sets = g.integers(0, 1000, (5, c, 3), dtype=np.int64)
    sets[g.random(sets.shape) < 0.6] = -1
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs.astype(dtype)),
                                          _t(dev, np.zeros(c, bool)), _t(dev, sets))
    assert np.array_equal(bits.cpu().numpy(), _pack(of.clause_match_sets(attrs, sets)))
    with pytest.raises(TypeError):
        torch.ops.retrieve.clause_mask(_t(dev, attrs.astype(dtype)), _t(dev, np.zeros(c, bool)),
                                       _t(dev, sets[:, :, 0]))


def test_large_and_negative_values(dev):
    """Rows whose values fall outside [0, 1024) walk their value lists; the others test bitmaps;
    item values outside the bitmap domain never match a bitmap row."""
    g = rng(59)
    n, c = 40_000, 4
    attrs = g.integers(-5, 3000, (n, c, 2), dtype=np.int64)
    attrs[:, :, 1] = g.integers(0, 40, (n, c))  # small values too
    sets = g.integers(0, 40, (8, c, 3), dtype=np.int64)
    sets[g.random(sets.shape) < 0.5] = -1
    sets[1, 0, 0] = 2500  # list rows
    sets[5, 2, 1] = -4
    rev = np.array([0, 1, 0, 0], bool)
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, rev), _t(dev, sets))
    assert np.array_equal(bits.cpu().numpy(), _pack(of.clause_match_sets(attrs, sets, rev)))


@pytest.mark.parametrize("c,a", [(8, 1), (3, 3), (18, 1)])
def test_row_groups_mixed_rows(dev, c, a):
    """More than 32 query rows (several row groups, the last partial), list rows among the
    bitmap rows, reverse clauses and an AND mask; C above 16 takes the per-row bitmap form."""
    g = rng(60 + c + a)
    n, b = 30_001, 45
    attrs = g.integers(-3, 60, (n, c, a), dtype=np.int64)
    sets = g.integers(0, 60, (b, c, 2), dtype=np.int64)
    sets[g.random(sets.shape) < 0.5] = -1
    sets[[2, 33, 40], 0, 0] = [5000, -7, 1024]  # list rows in two groups
    sets[10] = -1  # every clause inactive
    rev = (np.arange(c) % 3 == 1)
    want = of.clause_match_sets(attrs, sets, rev)
    pre = g.random((b, n)) < 0.7
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs), _t(dev, rev), _t(dev, sets),
                                          _t(dev, _pack(pre)))
    assert np.array_equal(bits.cpu().numpy(), _pack(want & pre))
    m = torch.ops.retrieve.clause_mask(_t(dev, attrs), _t(dev, rev), _t(dev, sets[:, :, 0]))
    assert np.array_equal(m.cpu().numpy(), of.clause_match(attrs, rev, sets[:, :, 0]))


@pytest.mark.parametrize("dtype", [np.int16, np.int64])
def test_wide_row_groups(dev, dtype):
    """Bit masks of more than 32 query rows go 64 rows to a workgroup: several groups (the last
    partial), list rows on either side of bit 32 of a group and in the last group, an AND mask."""
    g = rng(61)
    n, c, b = 20_011, 5, 150
    attrs = g.integers(-2, 50, (n, c, 1), dtype=np.int64)
    sets = g.integers(0, 50, (b, c, 3), dtype=np.int64)
    sets[g.random(sets.shape) < 0.55] = -1
    sets[[31, 32, 63, 64, 140], 1, 0] = [2000, -1, 4000, -9, 1500]  # -1 just pads
    sets[[5, 100]] = -1
    rev = np.array([0, 0, 1, 0, 1], bool)
    want = of.clause_match_sets(attrs, sets, rev)
    pre = g.random((b, n)) < 0.8
    bits = torch.ops.retrieve_amd.clause_bits(_t(dev, attrs.astype(dtype)), _t(dev, rev),
                                          _t(dev, sets), _t(dev, _pack(pre)))
    assert np.array_equal(bits.cpu().numpy(), _pack(want & pre))
