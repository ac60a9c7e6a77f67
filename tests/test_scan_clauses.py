"""Full scans with the exact clause filter tested inside the scan
(``torch.ops.retrieve_amd.int8_scan_topk_clauses`` / ``dense_scan_topk_clauses`` through
``rt_scan_topk_clauses``) against the oracle: the int8 top-k over the items that pass
``oracle.filters.clause_match_sets`` (and the optional mask), bit for bit; the dense forms equal
to the same kernel's scan over ``clause_bits``. Covers both set forms of the predicate (bitmaps for
values in [0, 1024), value lists otherwise), reverse and inactive clauses, rows with no active
clause, rows with fewer than k survivors, the sampled lower bound (N above 2**21), multi-valued
attributes, int16 / int32 / int64 tables, and the batches that fall back to the clause mask.
The blocked (large-batch) and 1-bit forms take the clauses with a mask: their lists hold the
candidates that pass the mask, filtered where a list is compacted and in the final merge; a
mask that passes everything makes every candidate a clause test and every compaction a filter."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import filters as of
from oracle import scan as osc
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _sets(g, b, c, v, vocab, active_rate, big=False):
    """[B, C, V] value sets, -1 pads; ``big`` puts values outside [0, 1024) in some rows."""
    s = np.full((b, c, v), -1, np.int64)
    for r in range(b):
        for ci in range(c):
            if g.random() < active_rate:
                m = int(g.integers(1, v + 1))
                s[r, ci, :m] = g.choice(vocab, m, replace=False)
        if big and r % 2 == 0:
            s[r][s[r] >= 0] += 5000
    return s


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _int8_case(dev, g, b, n, d, k, c, a, v, vocab, rev, active_rate=0.5, attr_dtype=np.int16,
               big=False, with_mask=False, pad_rate=0.1):
    print(f"int8 clause scan B={b} N={n} D={d} k={k} C={c} A={a} V={v} big={big} "
          f"mask={with_mask} attrs={np.dtype(attr_dtype).name}", flush=True)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    attrs = g.integers(0, vocab, (n, c, a)).astype(np.int64)
    attrs[g.random((n, c, a)) < pad_rate] = -1
    if big:
        attrs[g.random((n, c, a)) < 0.5] += 5000
    sets = _sets(g, b, c, v, vocab, active_rate, big)
    rev = np.array(rev, bool)
    valid = of.clause_match_sets(attrs, sets, rev)
    mask = g.random((b, n)) < 0.7 if with_mask else None
    if mask is not None:
        valid = valid & mask
    at = _t(dev, attrs.astype(attr_dtype))
    qt, it = _t(dev, q), _t(dev, items)
    mt = None if mask is None else _t(dev, _pack(mask))
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(qt, it, k, at, _t(dev, rev),
                                                        _t(dev, sets), mt)
    torch.cuda.synchronize()
    want_ids, want_sc = osc.int8_topk(q, items, k, valid)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    return qt, it, at, rev, sets, mt, ids, sc


@pytest.mark.parametrize(
    "b,n,d,k,c,a,v,vocab,rev",
    [(1, 5000, 64, 10, 3, 1, 2, 8, (0, 0, 0)),
     (16, 60_000, 512, 100, 8, 1, 4, 30, (0, 0, 1, 0, 0, 0, 0, 0)),
     (5, 777, 128, 1000, 2, 3, 3, 6, (1, 0)),
     (20, 100_003, 256, 64, 4, 2, 5, 12, (0, 1, 0, 0)),
     (31, 40_000, 64, 1, 1, 1, 1, 3, (0,))],
)
def test_int8_random_parity(dev, b, n, d, k, c, a, v, vocab, rev):
    g = rng(b * 7 + n + k)
    _int8_case(dev, g, b, n, d, k, c, a, v, vocab, rev)


def test_int8_value_lists_and_wide_tables(dev):
    """Values outside [0, 1024) (the value-list form) in half the rows, int32 and int64 tables."""
    g = rng(901)
    _int8_case(dev, g, 9, 20_000, 128, 50, 3, 2, 4, 20, (0, 1, 0), big=True,
               attr_dtype=np.int32)
    _int8_case(dev, g, 4, 9_000, 64, 30, 2, 1, 3, 10, (0, 0), big=True, attr_dtype=np.int64)


def test_int8_with_mask_and_few_survivors(dev):
    """The mask AND-ed in; sparse sets leave some rows fewer than k survivors (-1 pads)."""
    g = rng(902)
    _int8_case(dev, g, 12, 30_000, 64, 200, 4, 1, 1, 400, (0, 0, 0, 1), active_rate=0.9,
               with_mask=True)


def test_int8_seeded_path(dev):
    """N above the seed threshold: the sampled bound is a bound over passing items only."""
    g = rng(903)
    _int8_case(dev, g, 16, 2_300_000, 64, 100, 8, 1, 3, 16, (0,) * 8, active_rate=0.3)


def test_int8_equals_scan_over_clause_bits(dev):
    """The same answer as the scan over the packed clause mask (the unfused pipeline), also in
    the batches where the op falls back to it."""
    g = rng(904)
    for b in (3, 16, 40):
        q = _t(dev, g.integers(-128, 128, (b, 256), dtype=np.int8))
        items = _t(dev, g.integers(-128, 128, (50_000, 256), dtype=np.int8))
        attrs = _t(dev, g.integers(0, 12, (50_000, 5, 1)).astype(np.int16))
        rev = _t(dev, np.array([0, 1, 0, 0, 0], bool))
        sets = _t(dev, _sets(g, b, 5, 3, 12, 0.6))
        print(f"int8 clause scan vs clause_bits B={b}", flush=True)
        ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(q, items, 100, attrs, rev, sets)
        bits = torch.ops.retrieve_amd.clause_bits(attrs, rev, sets)
        want_ids, want_sc = torch.ops.retrieve_amd.int8_scan_topk(q, items, 100, bits)
        assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_equals_scan_over_clause_bits(dev, dtype):
    """bf16 / fp16: the fused filter returns what the same scan returns over the clause mask
    (same kernel, same scores), and every returned item passes the oracle's predicate."""
    g = rng(905)
    for b, n, d in ((1, 70_000, 128), (16, 300_000, 128), (7, 2_200_000, 64)):
        print(f"dense clause scan {dtype} B={b} N={n} D={d}", flush=True)
        q = torch.from_numpy(g.standard_normal((b, d)).astype(np.float32)).to(dev).to(dtype)
        items = torch.from_numpy(g.standard_normal((n, d)).astype(np.float32)).to(dev).to(dtype)
        attrs_np = g.integers(0, 10, (n, 3, 1)).astype(np.int64)
        sets_np = _sets(g, b, 3, 2, 10, 0.7)
        rev_np = np.array([0, 0, 1], bool)
        attrs, sets, rev = _t(dev, attrs_np.astype(np.int16)), _t(dev, sets_np), _t(dev, rev_np)
        ids, sc = torch.ops.retrieve_amd.dense_scan_topk_clauses(q, items, 100, attrs, rev, sets)
        bits = torch.ops.retrieve_amd.clause_bits(attrs, rev, sets)
        want_ids, want_sc = torch.ops.retrieve_amd.dense_scan_topk(q, items, 100, bits)
        assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)
        valid = of.clause_match_sets(attrs_np, sets_np, rev_np)
        got = ids.cpu().numpy()
        for r in range(b):
            row = got[r][got[r] >= 0]
            assert valid[r, row].all()
            assert len(row) == min(100, int(valid[r].sum()))


def test_empty_and_inactive_rows(dev):
    """N = 0 pads; a row with every clause inactive is the unfiltered scan."""
    g = rng(906)
    q = _t(dev, g.integers(-128, 128, (2, 64), dtype=np.int8))
    attrs0 = torch.zeros((0, 2, 1), dtype=torch.int16, device=dev)
    rev = _t(dev, np.zeros(2, bool))
    sets = _t(dev, np.full((2, 2, 1), -1, np.int64))
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(
        q, torch.zeros((0, 64), dtype=torch.int8, device=dev), 5, attrs0, rev, sets)
    assert (ids == -1).all() and (sc == torch.iinfo(torch.int32).min).all()
    items = _t(dev, g.integers(-128, 128, (3000, 64), dtype=np.int8))
    attrs = _t(dev, g.integers(0, 4, (3000, 2, 1)).astype(np.int16))
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(q, items, 50, attrs, rev, sets)
    want_ids, want_sc = torch.ops.retrieve_amd.int8_scan_topk(q, items, 50)
    assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)


def test_errors(dev):
    q = torch.zeros((2, 64), dtype=torch.int8, device=dev)
    items = torch.zeros((100, 64), dtype=torch.int8, device=dev)
    rev = torch.zeros(2, dtype=torch.bool, device=dev)
    sets = torch.full((2, 2, 1), -1, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.int8_scan_topk_clauses(
            q, items, 5, torch.zeros((99, 2, 1), dtype=torch.int16, device=dev), rev, sets)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.int8_scan_topk_clauses(
            q, items, 5, torch.zeros((100, 2, 1), dtype=torch.int16, device=dev), rev,
            sets[:1])
    with pytest.raises(TypeError):
        torch.ops.retrieve_amd.int8_scan_topk_clauses(
            q, items, 5, torch.zeros((100, 2, 1), dtype=torch.float32, device=dev), rev, sets)


def test_opcheck(dev):
    """Schema, fake tensor and dispatch registration of both ops."""
    g = rng(907)
    attrs = _t(dev, g.integers(0, 5, (4000, 2, 1)).astype(np.int16))
    rev = _t(dev, np.array([0, 1], bool))
    sets = _t(dev, _sets(g, 3, 2, 2, 5, 0.8))
    q8 = _t(dev, g.integers(-128, 128, (3, 64), dtype=np.int8))
    i8 = _t(dev, g.integers(-128, 128, (4000, 64), dtype=np.int8))
    qb = torch.randn((3, 64), device=dev).bfloat16()
    ib = torch.randn((4000, 64), device=dev).bfloat16()
    qh = _t(dev, g.integers(-2**63, 2**63 - 1, (3, 8), dtype=np.int64))
    ih = _t(dev, g.integers(-2**63, 2**63 - 1, (4000, 8), dtype=np.int64))
    for op, args in ((torch.ops.retrieve_amd.int8_scan_topk_clauses.default,
                      (q8, i8, 20, attrs, rev, sets)),
                     (torch.ops.retrieve_amd.dense_scan_topk_clauses.default,
                      (qb, ib, 20, attrs, rev, sets)),
                     (torch.ops.retrieve_amd.hamming_scan_topk_clauses.default,
                      (qh, ih, 20, attrs, rev, sets))):
        print(f"opcheck {op}", flush=True)
        torch.library.opcheck(op, args)


def _as_transposed(mask: torch.Tensor) -> torch.Tensor:
    """``mask`` [B, W] with its words stored transposed ([W, S], S = B rounded up to 256), as
    ``st.bloom_search_t`` returns them: the blocked scans read this layout directly."""
    b, w = mask.shape
    s = -(-b // 256) * 256
    out = torch.full((w, s), -1, dtype=mask.dtype, device=mask.device)  # (padding: never read)
    out[:, :b] = mask.t()
    return out.t()[:b]


def _unfused(dev, op, q, items, k, attrs, rev, sets, mask):
    bits = torch.ops.retrieve_amd.clause_bits(attrs, rev, sets, mask)
    return op(q, items, k, bits)


@pytest.mark.parametrize("b,n,d,k,dense_mask", [(40, 100_003, 128, 100, False),
                                                (256, 60_000, 256, 1000, False),
                                                (64, 50_000, 128, 5, True)])
def test_blocked_int8_parity(dev, b, n, d, k, dense_mask):
    """Large batches with a mask against the oracle; a mask of all ones leaves the clauses
    every decision (lists fill with failing candidates and are filtered when compacted)."""
    g = rng(b + n + k)
    print(f"blocked int8 clause scan B={b} N={n} D={d} k={k} all-ones mask={dense_mask}",
          flush=True)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    attrs = g.integers(0, 20, (n, 4, 1)).astype(np.int64)
    sets = _sets(g, b, 4, 3, 20, 0.6)
    rev = np.array([0, 0, 1, 0], bool)
    mask = np.ones((b, n), bool) if dense_mask else g.random((b, n)) < 0.6
    valid = of.clause_match_sets(attrs, sets, rev) & mask
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(
        _t(dev, q), _t(dev, items), k, _t(dev, attrs.astype(np.int16)), _t(dev, rev),
        _t(dev, sets), _t(dev, _pack(mask)))
    want_ids, want_sc = osc.int8_topk(q, items, k, valid)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


def test_blocked_adversarial_order(dev):
    """Scores rising with the item index and a mask of all ones: the sampled bound is far below
    the answer, so the lists fill and are filtered and compacted over and over."""
    n, b = 200_000, 48
    items = np.zeros((n, 128), np.int8)
    items[:, 0] = (np.arange(n) * 255 // n - 127).astype(np.int8)
    items[:, 1] = ((np.arange(n) * 7) % 5).astype(np.int8)
    q = np.zeros((b, 128), np.int8)
    q[:, 0] = 1
    q[1::2, 1] = 2
    g = rng(908)
    attrs = g.integers(0, 10, (n, 2, 1)).astype(np.int64)
    sets = _sets(g, b, 2, 2, 10, 0.8)
    rev = np.zeros(2, bool)
    mask = np.ones((b, n), bool)
    valid = of.clause_match_sets(attrs, sets, rev)
    print(f"blocked int8 clause scan, rising scores B={b} N={n}", flush=True)
    for k in (100, 1000):
        ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(
            _t(dev, q), _t(dev, items), k, _t(dev, attrs.astype(np.int16)), _t(dev, rev),
            _t(dev, sets), _t(dev, _pack(mask)))
        want_ids, want_sc = osc.int8_topk(q, items, k, valid)
        assert np.array_equal(sc.cpu().numpy(), want_sc)
        assert np.array_equal(ids.cpu().numpy(), want_ids)


@pytest.mark.parametrize("dtype,b,n,d", [(torch.bfloat16, 256, 300_000, 128),
                                         (torch.float16, 64, 2_200_000, 64),
                                         (torch.bfloat16, 512, 2_200_000, 128),
                                         (torch.float32, 64, 50_000, 64)])
def test_blocked_dense_equals_unfused(dev, dtype, b, n, d):
    """bf16 / fp16 / fp32 large batches with a mask equal the same scan over the clause mask:
    the seeded path (N above 2**21) with its rank-th bound."""
    g = rng(909 + b)
    print(f"blocked dense clause scan {dtype} B={b} N={n} D={d}", flush=True)
    q = torch.from_numpy(g.standard_normal((b, d)).astype(np.float32)).to(dev).to(dtype)
    items = torch.from_numpy(g.standard_normal((n, d)).astype(np.float32)).to(dev).to(dtype)
    attrs = _t(dev, g.integers(0, 12, (n, 3, 1)).astype(np.int16))
    sets = _t(dev, _sets(g, b, 3, 3, 12, 0.7))
    rev = _t(dev, np.array([0, 1, 0], bool))
    mask = _t(dev, _pack(g.random((b, n)) < 0.5))
    ids, sc = torch.ops.retrieve_amd.dense_scan_topk_clauses(q, items, 100, attrs, rev, sets, mask)
    want_ids, want_sc = _unfused(dev, torch.ops.retrieve_amd.dense_scan_topk, q, items, 100, attrs,
                                 rev, sets, mask)
    assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)
    # the same mask stored transposed
    ids_t, sc_t = torch.ops.retrieve_amd.dense_scan_topk_clauses(q, items, 100, attrs, rev, sets,
                                                             _as_transposed(mask))
    assert torch.equal(ids_t, ids) and torch.equal(sc_t, sc)


@pytest.mark.parametrize("b,n,k,ones", [(256, 200_000, 1000, False), (64, 2_200_000, 100, False),
                                        (96, 100_000, 50, True), (5, 50_000, 20, False)])
def test_hamming_parity(dev, b, n, k, ones):
    """512-bit codes: the matrix-core batches fused (B = 256, k = 1000 is the 1-bit
    configuration's shape), a small batch through the clause mask; against the oracle, and the
    seeded case against the unfused scan."""
    g = rng(910 + b + k)
    print(f"hamming clause scan B={b} N={n} k={k} all-ones mask={ones}", flush=True)
    q = g.integers(-2**63, 2**63 - 1, (b, 8), dtype=np.int64)
    items = g.integers(-2**63, 2**63 - 1, (n, 8), dtype=np.int64)
    attrs = g.integers(0, 16, (n, 3, 1)).astype(np.int64)
    sets = _sets(g, b, 3, 4, 16, 0.6)
    rev = np.array([0, 0, 1], bool)
    mask = np.ones((b, n), bool) if ones else g.random((b, n)) < 0.5
    args = (_t(dev, attrs.astype(np.int16)), _t(dev, rev), _t(dev, sets), _t(dev, _pack(mask)))
    qt, it = _t(dev, q), _t(dev, items)
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk_clauses(qt, it, k, *args, fused=True)
    ids2, sc2 = torch.ops.retrieve_amd.hamming_scan_topk_clauses(qt, it, k, *args, fused=False)
    assert torch.equal(ids, ids2) and torch.equal(sc, sc2)
    # the mask stored transposed (read directly by the blocked scan; copied elsewhere)
    args_t = args[:3] + (_as_transposed(args[3]),)
    for fused in (True, False):
        ids3, sc3 = torch.ops.retrieve_amd.hamming_scan_topk_clauses(qt, it, k, *args_t, fused=fused)
        assert torch.equal(ids, ids3) and torch.equal(sc, sc3)
    if n > 1_000_000:
        want_ids, want_sc = _unfused(dev, torch.ops.retrieve_amd.hamming_scan_topk, qt, it, k,
                                     *args)
        assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)
        return
    valid = of.clause_match_sets(attrs, sets, rev) & mask
    want_ids, want_sc = osc.hamming_topk(q, items, k, valid)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


def test_hamming_speculative_fallback(dev):
    """N >= 2.2M rows, clauses tested in the scan (the blocked 1-bit scan): query 0's 40 best
    rows that pass its clause sit at the start of 40 seed sample blocks, one a seed workgroup
    (items 16384 j: blocks 8 j of the seed's stride-8 sample), and 30 better rows that pass its
    mask but fail the clause sit in the first block. The seed's lists offer passing maxima only
    (the first block's, a failing row, offers none), so its rank-th best (35th at k = 100) is a
    planted row; the main pass ends with 35 passing entries, the flag rises, the fallback behind
    the seed's k-th runs, and the results match the oracle."""
    g = rng(916)
    b, n, k = 40, 2_200_000, 100
    print(f"hamming clause scan, speculative fallback B={b} N={n} k={k}", flush=True)
    q = g.integers(-2**63, 2**63 - 1, (b, 8), dtype=np.int64)
    base = g.integers(-2**63, 2**63 - 1, (4096, 8), dtype=np.int64)
    items = base[g.integers(0, 4096, n)]
    attrs = g.integers(0, 16, (n, 3, 1)).astype(np.int64)
    sets = _sets(g, b, 3, 4, 16, 0.6)
    sets[0] = -1
    sets[0, 0, 0] = 5  # query 0: attribute 0 equal to 5
    rev = np.array([0, 0, 1], bool)
    def off(d):  # q[0] with d of its bits flipped (up to 60 in word 0, the rest in word 1)
        x = q[0].copy()
        x[0] ^= np.int64((1 << min(d, 60)) - 1)
        if d > 60:
            x[1] ^= np.int64((1 << (d - 60)) - 1)
        return x

    planted = [16384 * j for j in range(1, 41)]
    for j, r in enumerate(planted):
        items[r] = off(31 + j)  # 31 .. 70 bits off
        attrs[r, 0, 0] = 5
    for r in range(1, 31):
        items[r] = off(r)  # 1 .. 30 bits off
        attrs[r, 0, 0] = 6
    mask = g.random((b, n)) < 0.5
    mask[0, planted] = True
    mask[0, 1:31] = True
    args = (_t(dev, attrs.astype(np.int16)), _t(dev, rev), _t(dev, sets), _t(dev, _pack(mask)))
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk_clauses(_t(dev, q), _t(dev, items), k, *args,
                                                           fused=True)
    valid = of.clause_match_sets(attrs, sets, rev) & mask
    want_ids, want_sc = osc.hamming_topk(q, items, k, valid)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert set(planted) <= set(ids[0].tolist())
