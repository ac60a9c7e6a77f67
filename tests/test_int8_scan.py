"""int8 full scan + exact top-k on the GPU against the oracle: bit-exact ids and int32 scores,
ties to the lower index (``torch.ops.retrieve_amd.int8_scan_topk`` through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from tests.conftest import rng

pytestmark = pytest.mark.gpu


def _run(dev, q, items, k, mask=None):
    qt = torch.from_numpy(q).to(dev)
    it = torch.from_numpy(items).to(dev)
    mt = None if mask is None else torch.from_numpy(_pack(mask)).to(dev)
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk(qt, it, k, mt)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), sc.cpu().numpy()


def _pack(valid: np.ndarray) -> np.ndarray:
    """[B, N] bool → [B, ceil(N/64)] int64, item d at bit 63 - d % 64."""
    b, n = valid.shape
    w = (n + 63) // 64
    pad = np.zeros((b, w * 64), bool)
    pad[:, :n] = valid
    bits = pad.reshape(b, w, 64).astype(np.uint64)
    shifts = np.uint64(63) - np.arange(64, dtype=np.uint64)
    return np.bitwise_or.reduce(bits << shifts, axis=2).view(np.int64)


def _check(dev, q, items, k, mask=None):
    print(f"int8 scan B={q.shape[0]} N={items.shape[0]} D={q.shape[1]} k={k} "
          f"mask={mask is not None}", flush=True)
    ids, sc = _run(dev, q, items, k, mask)
    want_ids, want_sc = osc.int8_topk(q, items, k, mask)
    assert np.array_equal(sc, want_sc)
    assert np.array_equal(ids, want_ids)


def test_kat(dev, kat):
    a, _ = kat
    q = np.zeros((1, 64), np.int8)
    q[:, :16] = a["int8_kat_query"]
    items = np.zeros((2, 64), np.int8)
    items[:, :16] = a["int8_kat_items"]
    ids, sc = _run(dev, q, items, 2)
    assert ids.tolist() == [[1, 0]] and sc.tolist() == [[39, 17]]


@pytest.mark.parametrize(
    "b,n,d,k",
    [(1, 1, 64, 1), (1, 15, 64, 10), (3, 1000, 128, 10), (16, 4097, 512, 100),
     (17, 20000, 256, 100), (33, 12345, 64, 1000), (5, 70000, 768, 7), (2, 3000, 1024, 64)],
)
def test_random_parity(dev, b, n, d, k):
    g = rng(b * 1000 + n + d + k)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    _check(dev, q, items, k)


def test_heavy_ties(dev):
    """Four distinct rows (the reference's heavy-tie setup, test_official.py:707-738): every
    boundary is a tie group, taken in index order."""
    g = rng(11)
    base = g.integers(-127, 128, (4, 128), dtype=np.int8)
    items = base[g.integers(0, 4, 50000)]
    q = g.integers(-127, 128, (9, 128), dtype=np.int8)
    _check(dev, q, items, 100)
    _check(dev, q, items, 1000)


def test_masked_and_short_rows(dev):
    g = rng(12)
    q = g.integers(-128, 128, (6, 64), dtype=np.int8)
    items = g.integers(-128, 128, (30000, 64), dtype=np.int8)
    mask = g.random((6, 30000)) < 0.1
    mask[1] = g.random(30000) < 0.001  # ~30 survivors < k: -1 / INT32_MIN pads
    mask[2] = False
    _check(dev, q, items, 100, mask)


@pytest.mark.parametrize("k", [1025, 3000])
def test_k_above_1024(dev, k):
    """Above the fused lists' 1024: the raw scorer's buffer and one key select per row
    (retrieve_amd.large_k), the same results, ties to the lower index, pads past the mask."""
    g = rng(14 + k)
    q = g.integers(-128, 128, (4, 64), dtype=np.int8)
    items = g.integers(-4, 5, (20000, 64), dtype=np.int8)  # small values: many tied dots
    mask = g.random((4, 20000)) < 0.5
    mask[1] = g.random(20000) < 0.02  # ~400 survivors < k
    _check(dev, q, items, k, mask)
    _check(dev, q, items, k)


def test_k_above_n_pads(dev):
    g = rng(13)
    q = g.integers(-128, 128, (2, 64), dtype=np.int8)
    items = g.integers(-128, 128, (7, 64), dtype=np.int8)
    _check(dev, q, items, 20)


def test_empty_items(dev):
    q = np.ones((3, 64), np.int8)
    ids, sc = _run(dev, q, np.zeros((0, 64), np.int8), 5)
    assert (ids == -1).all() and (sc == np.iinfo(np.int32).min).all()


def test_seeded_path_large_n(dev):
    """N above the seed threshold (8 x 2**18 rows): the sampled lower bound, then the scan."""
    g = rng(14)
    n = 2_300_000
    q = g.integers(-128, 128, (20, 64), dtype=np.int8)
    items = g.integers(-128, 128, (n, 64), dtype=np.int8)
    _check(dev, q, items, 100)


def test_seeded_path_adversarial_order(dev):
    """Scores rising with the item index: the sample's bound is far below the answer, so the
    waves' lists fill and compact over and over; the result must not change."""
    n = 2_200_000
    items = np.zeros((n, 64), np.int8)
    items[:, 0] = (np.arange(n) * 255 // n - 127).astype(np.int8)
    items[:, 1] = ((np.arange(n) * 7) % 5).astype(np.int8)
    q = np.zeros((3, 64), np.int8)
    q[0, 0] = 1
    q[1, 0] = -1
    q[2, :2] = [3, 1]
    _check(dev, q, items, 100)
    _check(dev, q, items, 1000)


def test_deterministic(dev):
    g = rng(15)
    q = torch.from_numpy(g.integers(-128, 128, (8, 512), dtype=np.int8)).to(dev)
    it = torch.from_numpy(g.integers(-128, 128, (100000, 512), dtype=np.int8)).to(dev)
    a = torch.ops.retrieve_amd.int8_scan_topk(q, it, 100)
    b = torch.ops.retrieve_amd.int8_scan_topk(q, it, 100)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_errors(dev):
    q = torch.zeros((2, 64), dtype=torch.int8, device=dev)
    it = torch.zeros((10, 64), dtype=torch.int8, device=dev)
    with pytest.raises(TypeError):
        torch.ops.retrieve_amd.int8_scan_topk(q.float(), it, 3)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.int8_scan_topk(q, it.t(), 3)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.int8_scan_topk(q, it, 0)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.int8_scan_topk(q[:, :32], it[:, :32].contiguous(), 3)


def test_full_size_properties(dev):
    """30M x 512 (config 4) at B = 16: ids unique and in range, scores sorted (ties by id), each
    returned score equals the recomputed dot of its id, and no sampled item beats the k-th."""
    n, d, b, k = 30_000_000, 512, 16, 100
    gen = torch.Generator(device=dev).manual_seed(21)
    items = torch.randint(-128, 128, (n, d), dtype=torch.int8, device=dev, generator=gen)
    q = torch.randint(-128, 128, (b, d), dtype=torch.int8, device=dev, generator=gen)
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk(q, items, k)
    torch.cuda.synchronize()
    assert (ids >= 0).all() and (ids < n).all()
    for r in range(b):
        assert torch.unique(ids[r]).numel() == k
    # recomputed dots (float32 products of int8 are exact here: |dot| < 2**24)
    rows = items[ids.reshape(-1)].float().reshape(b, k, d)
    dots = torch.bmm(rows, q.float().unsqueeze(2)).squeeze(2).to(torch.int32)
    assert torch.equal(dots, sc)
    # order: score desc, then id asc
    s64 = sc.long()
    assert (s64[:, :-1] >= s64[:, 1:]).all()
    tie = s64[:, :-1] == s64[:, 1:]
    assert (ids[:, :-1][tie] < ids[:, 1:][tie]).all()
    # a sample of 2M items: none beats the k-th (score, id)
    sample = torch.randint(0, n, (2_000_000,), device=dev, generator=gen)
    ss = (items[sample].float() @ q.float().t()).to(torch.int32).t()  # [b, S]
    kth_s, kth_i = sc[:, -1:].long(), ids[:, -1:]
    beats = (ss.long() > kth_s) | ((ss.long() == kth_s) & (sample.unsqueeze(0) < kth_i))
    for r in range(b):
        member = torch.isin(sample, ids[r])
        assert not (beats[r] & ~member).any()
    del items
    torch.cuda.empty_cache()


@pytest.mark.parametrize(
    "b,n,d,k", [(128, 5000, 512, 100), (300, 20000, 128, 10), (257, 30000, 256, 1000),
                (1024, 3000, 512, 7), (32, 9000, 512, 100), (45, 7000, 128, 50)],
)
def test_large_batch_parity(dev, b, n, d, k):
    """B >= 32 (rows of 128, 256 or 512 bytes) runs the register-blocked kernel: 256 queries per
    workgroup, waves whose 32-query column tiles hold only padding skip them."""
    g = rng(b * 3 + n + d + k)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    _check(dev, q, items, k)


def test_large_batch_seeded_ties_masked(dev):
    g = rng(16)
    base = g.integers(-127, 128, (64, 128), dtype=np.int8)
    items = base[g.integers(0, 64, 2_200_000)]
    q = g.integers(-128, 128, (200, 128), dtype=np.int8)
    _check(dev, q, items, 100)
    mask = g.random((130, 50000)) < 0.05
    mask[7] = False
    _check(dev, q[:130], items[:50000], 100, mask)


def test_large_batch_seeded_512b_rows(dev):
    """512-byte rows, B >= 512 over N >= 2.1M rows: the blocked scan's seed (its k-th and
    rank-th bounds) and main pass, heavy ties across sampled and unsampled rows, and a mask with
    an empty row and a row whose few passing items miss the sample."""
    g = rng(17)
    base = g.integers(-127, 128, (256, 512), dtype=np.int8)
    n = 2_100_000
    items = base[g.integers(0, 256, n)]
    q = g.integers(-128, 128, (512, 512), dtype=np.int8)
    _check(dev, q, items, 100)
    mask = g.random((512, n)) < 0.02
    mask[3] = False
    mask[5] = False
    mask[5, 64 * 9 : 64 * 9 + 40] = True  # only in an unsampled tile
    _check(dev, q, items, 100, mask)
