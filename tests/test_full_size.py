"""Full-size properties (the BASELINE shapes, too large for the oracle): the Bloom pre-filter has
no false negatives over 30M documents (every exact match survives it, so AND-ing the exact
post-check with it changes nothing), and the masked 1-bit top-1000 over 30M 512-bit codes returns
unique, mask-passing ids whose scores are the recomputed Hamming scores, in (score desc, id asc)
order, with no sampled passing item beating the k-th."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import retrieve_amd.hip  # noqa: F401
    import retrieve_amd.st  # noqa: F401

    return torch.device("cuda:0")


def test_bloom_no_false_negatives_30m(dev):
    import bench
    import retrieve_amd.st as st
    from retrieve_amd import bloom as bl

    n, b = 30_000_000, 16
    print(f"bloom full size N={n} B={b}", flush=True)
    attrs = bench.attr_table(n, 4321, dev)
    sets = bench.query_sets(attrs, b, 0.1, 77)
    fid, fo, fv = st.attrs_to_features(attrs.long())
    words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, bench.BLOOM_BITS,
                                                       bench.BLOOM_K)
    del fid, fo, fv
    blob, count, depth = st.prepare_plans(bl.sets_to_expressions(sets), bench.HASH_K, dev)
    pre = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, depth,
                                                         bench.BLOOM_K, bench.HASH_K)
    rev = torch.zeros(len(bench.CARDINALITIES), dtype=torch.bool, device=dev)
    qs = torch.from_numpy(sets).to(dev)
    exact = torch.ops.retrieve_amd.clause_bits(attrs, rev, qs)
    both = torch.ops.retrieve_amd.clause_bits(attrs, rev, qs, pre)
    nw = (n + 63) // 64
    # the search writes whole 2048-document bundles: words past the last document's are padding
    assert exact.shape == (b, nw) and pre.shape[0] == b and pre.shape[1] >= nw
    pre = pre[:, :nw].contiguous()
    assert not (exact & ~pre).any()  # no false negatives
    assert torch.equal(both, exact)
    # the pre-filter passes a superset, and rejects most non-matching documents
    counts = torch.ops.retrieve_amd.mask_compact(exact, n)[1].double()
    pcounts = torch.ops.retrieve_amd.mask_compact(pre, n)[1].double()
    assert (pcounts >= counts).all() and (counts > 0).all()
    assert float((pcounts / n).max()) < 0.9


def _popcount64(x: torch.Tensor) -> torch.Tensor:
    """Per-element popcount of int64 words (SWAR, two's-complement safe)."""
    x = x - ((x >> 1) & 0x5555555555555555)
    x = (x & 0x3333333333333333) + ((x >> 2) & 0x3333333333333333)
    x = (x + (x >> 4)) & 0x0F0F0F0F0F0F0F0F
    return ((x * 0x0101010101010101) >> 56) & 0xFF


def _check_binary(dev, n, w, b, k, masked, n_sample, seed):
    """The 1-bit scan at full size: every id distinct, valid and passing the mask, its score
    recomputed, descending order with lower ids first on ties, and no sampled passing item
    that beats the k-th left out."""
    print(f"binary full size N={n} W={w} B={b} k={k} masked={masked}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(seed)
    items = torch.randint(-2**63, 2**63 - 1, (n, w), dtype=torch.int64, device=dev,
                          generator=gen)
    q = torch.randint(-2**63, 2**63 - 1, (b, w), dtype=torch.int64, device=dev, generator=gen)
    if masked:
        valid = torch.rand((b, n), device=dev, generator=gen) < 0.1
        words = torch.ops.retrieve_amd.pack_mask(valid)
    else:
        valid = torch.ones((b, n), dtype=torch.bool, device=dev)
        words = None
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk(q, items, k, words)
    torch.cuda.synchronize()
    assert (ids >= 0).all() and (ids < n).all()
    for r in range(b):
        assert torch.unique(ids[r]).numel() == k
    assert torch.gather(valid, 1, ids).all()
    ham = _popcount64(items[ids.reshape(-1)].reshape(b, k, w) ^ q.unsqueeze(1)).sum(2)
    assert torch.equal((64 * w - 2 * ham).to(sc.dtype), sc)
    s64 = sc.long()
    assert (s64[:, :-1] >= s64[:, 1:]).all()
    tie = s64[:, :-1] == s64[:, 1:]
    assert (ids[:, :-1][tie] < ids[:, 1:][tie]).all()
    sample = torch.randint(0, n, (n_sample,), device=dev, generator=gen)
    hs = _popcount64(items[sample].unsqueeze(0) ^ q.unsqueeze(1)).sum(2)  # [b, S]
    ss = 64 * w - 2 * hs
    kth_s, kth_i = s64[:, -1:], ids[:, -1:]
    beats = ((ss > kth_s) | ((ss == kth_s) & (sample.unsqueeze(0) < kth_i))) & valid[:, sample]
    for r in range(b):
        assert not (beats[r] & ~torch.isin(sample, ids[r])).any()


def test_binary_masked_30m(dev):
    """64 queries over 30M rows at k = 1000 (a seed of 1,024,000 rows and its rank-th bound)."""
    _check_binary(dev, 30_000_000, 8, 64, 1000, True, 1_000_000, 31)


def test_binary_large_batch_9m(dev):
    """512 queries over 9M rows (the blocked scan behind its seed's rank-th bound), no mask."""
    _check_binary(dev, 9_000_000, 8, 512, 100, False, 200_000, 37)
