"""1-bit Hamming full scan + exact top-k on the GPU against the oracle (bit-exact integer
scores and ids, ties to the lower index): ``torch.ops.retrieve_amd.hamming_scan_topk`` and the
reference-schema ``torch.ops.retrieve.oporp_1bit_match_topk_full``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _codes(g, n, w):
    return g.integers(-(2**63), 2**63 - 1, (n, w), dtype=np.int64)


def _check(dev, q, items, k, mask=None):
    print(f"hamming scan B={q.shape[0]} N={items.shape[0]} W={q.shape[1]} k={k} "
          f"mask={mask is not None}", flush=True)
    qt = torch.from_numpy(q).to(dev)
    it = torch.from_numpy(items).to(dev)
    mt = None if mask is None else torch.from_numpy(_pack(mask)).to(dev)
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk(qt, it, k, mt)
    torch.cuda.synchronize()
    want_ids, want_sc = osc.hamming_topk(q, items, k, mask)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


def test_popcount_kat(dev, kat):
    """The reference's popcount words as one-word codes against a zero query: scores are
    64 - 2 * popcount."""
    a, _ = kat
    items = a["popcount_kat_in"].reshape(-1, 1)
    q = np.zeros((1, 1), np.int64)
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk(
        torch.from_numpy(q).to(dev), torch.from_numpy(items).to(dev), items.shape[0]
    )
    got = dict(zip(ids[0].tolist(), sc[0].tolist()))
    assert [got[i] for i in range(items.shape[0])] == \
        [64 - 2 * int(p) for p in a["popcount_kat_out"]]


@pytest.mark.parametrize(
    "b,n,w,k",
    [(1, 1, 8, 1), (1, 100, 1, 10), (5, 3000, 2, 50), (16, 20000, 8, 100),
     (65, 10000, 4, 100), (3, 50000, 16, 1000), (70, 4099, 8, 7), (9, 7000, 3, 64),
     (4, 5000, 5, 40), (33, 3000, 12, 100)],
)
def test_random_parity(dev, b, n, w, k):
    g = rng(b * 7 + n + w * 13 + k)
    _check(dev, _codes(g, b, w), _codes(g, n, w), k)


def test_heavy_ties_few_bits(dev):
    """W = 1 codes with only 8 distinct rows: huge tie groups at every boundary."""
    g = rng(31)
    base = _codes(g, 8, 1)
    items = base[g.integers(0, 8, 40000)]
    q = _codes(g, 9, 1)
    _check(dev, q, items, 100)
    _check(dev, q, items, 1000)


def test_masked(dev):
    g = rng(32)
    q = _codes(g, 6, 8)
    items = _codes(g, 30000, 8)
    mask = g.random((6, 30000)) < 0.1
    mask[1] = g.random(30000) < 0.001
    mask[3] = False
    _check(dev, q, items, 100, mask)


def test_seeded_path_k1000(dev):
    """N above the k = 1000 seed threshold (8 x 1024 x k rows): config 5's top-1000 over
    512-bit codes."""
    g = rng(33)
    q = _codes(g, 8, 8)
    items = _codes(g, 8_400_000, 8)
    _check(dev, q, items, 1000)


def test_unseeded_large_k(dev):
    """k = 1000 below the seed threshold: every wave's lists fill and compact from scratch."""
    g = rng(35)
    q = _codes(g, 20, 8)
    items = _codes(g, 2_200_000, 8)
    _check(dev, q, items, 1000)


@pytest.mark.parametrize("b,n,k,masked", [(8, 5000, 50, False), (16, 20000, 100, True),
                                          (64, 30000, 1000, True),
                                          (32, 9000, 1000, False), (33, 5000, 100, False),
                                          (37, 20000, 1000, True),
                                          (128, 9000, 100, False), (129, 20000, 100, True),
                                          (300, 7000, 1000, False), (64, 3000, 1, True)])
def test_matrix_core_path(dev, b, n, k, masked):
    """512-bit codes from 8 queries on run on the fp4 matrix cores (bits as e2m1 nibbles,
    the accumulator started at 64 W - 2 popcount(q)): wide and narrow layouts, k up to 1000,
    masks."""
    g = rng(b * 3 + n + k)
    q = _codes(g, b, 8)
    items = _codes(g, n, 8)
    items[7] = q[0]  # an exact match: the maximum score 512
    items[9] = ~q[1]  # the minimum -512
    mask = None
    if masked:
        mask = g.random((b, n)) < 0.2
        mask[0, 7] = True
    _check(dev, q, items, k, mask)


@pytest.mark.parametrize("b,masked", [(12, False), (12, True), (70, True)])
def test_matrix_core_skewed_queries(dev, b, masked):
    """Queries of every popcount (all zeros, all ones, a few bits, most bits) over 1M rows, seeded:
    the main pass's accumulators start at a fixed bias with the query's start 64 W - 2 |q| moved
    into each threshold, so the thresholds of these queries sit far from the scores' centre."""
    g = rng(41 + b + masked)
    q = _codes(g, b, 8)
    q[0] = 0
    q[1] = -1
    q[2] = np.int64(0x0101010101010101)
    q[3] = ~np.int64(0x0101010101010101)
    q[4, :4] = 0
    base = _codes(g, 4096, 8)
    items = base[g.integers(0, 4096, 1_000_000)]
    items[5] = q[0]
    items[11] = q[1]
    mask = g.random((b, items.shape[0])) < 0.3 if masked else None
    _check(dev, q, items, 100, mask)


@pytest.mark.parametrize("b,n,k,masked,wide_mask", [
    (1, 15, 20, False, False),
    (17, 16, 16, True, False),
    (48, 127, 100, True, True),
    (64, 129, 129, False, False),
    (65, 1000, 37, True, True),
    (100, 5000, 1, False, False),
    (128, 4099, 64, True, False),
])
def test_per_wave_bits_edges(dev, b, n, k, masked, wide_mask):
    """512-bit codes on the per-wave fp4 scan (1 to 128 queries): fewer rows than one 16-row
    group, partial groups and 128-row tiles (rows past the table read as zeros and are never
    kept), batches across the 16-query groups of a wave and the grid's second row of groups,
    k above N (padded), a query no item passes, and mask rows wider than ceil(N/64) words (the
    extra words all ones, past the table)."""
    g = rng(b * 11 + n + k)
    q = _codes(g, b, 8)
    items = _codes(g, n, 8)
    mask = None
    mt = None
    if masked:
        mask = g.random((b, n)) < 0.4
        mask[0] = False
        packed = _pack(mask)
        if wide_mask:
            packed = np.concatenate([packed, np.full((b, 3), -1, np.int64)], 1)
        mt = torch.from_numpy(packed).to(dev)
    print(f"per-wave bits B={b} N={n} k={k} mask={masked} wide={wide_mask}", flush=True)
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk(
        torch.from_numpy(q).to(dev), torch.from_numpy(items).to(dev), k, mt)
    torch.cuda.synchronize()
    want_ids, want_sc = osc.hamming_topk(q, items, k, mask)
    assert np.array_equal(sc.cpu().numpy(), want_sc)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


def test_matrix_core_ties(dev):
    """Few distinct 512-bit rows: every score ties in large groups, broken by the lower id."""
    g = rng(36)
    base = _codes(g, 5, 8)
    items = base[g.integers(0, 5, 30000)]
    q = np.concatenate([base[:3], _codes(g, 40, 8)])
    _check(dev, q, items, 1000)
    _check(dev, q[:9], items, 37)


def test_matrix_core_seeded_large_batch(dev):
    """B >= 512 over N >= 2.1M rows: the seed (its k-th and rank-th bounds) and the main pass."""
    g = rng(37)
    q = _codes(g, 520, 8)
    base = _codes(g, 4096, 8)
    items = base[g.integers(0, 4096, 2_200_000)]  # repeated rows keep the oracle's work small
    mask = g.random((520, 2_200_000)) < 0.5
    _check(dev, q, items, 100, mask)


@pytest.mark.parametrize("masked", [False, True])
def test_matrix_core_speculative_bound(dev, masked):
    """N >= 2.1M rows below 512 queries: the main pass runs behind the seed sample's rank-th best
    (23 at k = 100 over a 16th of the rows), and the results stay exact."""
    g = rng(38 + masked)
    q = _codes(g, 40, 8)
    base = _codes(g, 4096, 8)
    items = base[g.integers(0, 4096, 2_200_000)]  # repeated rows keep the oracle's work small
    mask = g.random((40, 2_200_000)) < 0.5 if masked else None
    _check(dev, q, items, 100, mask)
    _check(dev, q[:33], items, 1000, None if mask is None else mask[:33])


def _near(q: np.ndarray, d: int) -> np.ndarray:
    """``q`` with its lowest ``d`` bits flipped (d < 64): the score 64 W - 2 d against q."""
    x = q.copy()
    x[0] ^= np.int64((1 << d) - 1)
    return x


# Items at the first row of seed sample blocks far enough apart to fall in different seed lists,
# for N = 2.2M rows and k = 100: the blocked scan samples 256-row blocks every 8 blocks (stride
# 8, 2^18 rows, 128 sample rows a seed workgroup), the per-wave 1-bit scan every 16 (stride 16,
# 2^17 rows, 128 a seed wave), so items 16384 j start blocks 8 j and 4 j of the two samples.
SEED_SPREAD = [16384 * j for j in range(1, 41)]


@pytest.mark.parametrize("b", [40, 130])
def test_matrix_core_speculative_fallback(dev, b):
    """Query 0's 40 best rows sit at the start of 40 seed sample blocks, one a seed list: the
    seed's rank-th best (23rd at B = 40 on the per-wave scan, 35th at B = 130 on the blocked scan)
    is one of them, so the main pass keeps 23 / 35 rows for that query and ends short of k = 100,
    the flag rises, and the fallback pass (unbounded on the per-wave scan, behind the seed's k-th
    on the blocked one) gives every result exactly."""
    g = rng(40)
    q = _codes(g, b, 8)
    base = _codes(g, 4096, 8)
    items = base[g.integers(0, 4096, 2_200_000)]
    for j, r in enumerate(SEED_SPREAD):
        items[r] = _near(q[0], j + 1)
    _check(dev, q, items, 100)


def test_oporp_full_schema(dev):
    g = rng(34)
    q = torch.from_numpy(_codes(g, 4, 8)).to(dev)
    it = torch.from_numpy(_codes(g, 5000, 8)).to(dev)
    ids, sc = torch.ops.retrieve.oporp_1bit_match_topk_full(q, it, 64)
    assert ids.dtype == torch.int64 and sc.dtype == torch.float32 and sc.shape == (4, 64)
    ids2, sc2 = torch.ops.retrieve_amd.hamming_scan_topk(q, it, 64)
    assert torch.equal(ids, ids2) and torch.equal(sc, sc2.float())
    with pytest.raises(TypeError):
        torch.ops.retrieve.oporp_1bit_match_topk_full(q.int(), it, 3)
    with pytest.raises(ValueError):
        torch.ops.retrieve.oporp_1bit_match_topk_full(q[:, :4], it, 3)


@pytest.mark.parametrize(
    "b,n,w,k,masked,distinct",
    [(3, 20000, 8, 5000, False, 0), (9, 30000, 3, 2000, True, 0), (2, 30000, 8, 3000, False, 5),
     (4, 9000, 16, 8192, True, 0), (1, 1500, 2, 1100, False, 0), (5, 40000, 1, 4000, True, 3)],
)
def test_large_k(dev, b, n, w, k, masked, distinct):
    """k above 1024 (LiNR V3's candidate pools): selection by counting the 64 W + 1 scores, the
    ties at the cut resolved by id bins of 8192 (heavy ties span several bins), pads when fewer
    than k items pass."""
    g = rng(b * 5 + n + w + k)
    q = _codes(g, b, w)
    if distinct:
        base = _codes(g, distinct, w)
        items = base[g.integers(0, distinct, n)]
    else:
        items = _codes(g, n, w)
    mask = (g.random((b, n)) < 0.3) if masked else None
    _check(dev, q, items, k, mask)
