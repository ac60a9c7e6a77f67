"""Oracle parity at the sizes where the sampled paths run, bit for bit for the integer scans:

- the headline step exactly as ``bench.py`` times it: ``scan_topk_bloom_clauses`` (the Bloom
  plans probed per candidate, then the exact clauses, inside the scan) at B = 16, D = 512 over
  2.3M rows (the small-batch scan's seeded path) and over the benched 30M rows, the bench's Zipf
  attributes and 10 % value sets; and its ``--bloom-search`` form, ``int8_scan_topk_clauses`` under the words straight
  from ``st::bloom_index_search_batch_prepared`` with their bundle-padded width (more words
  than ceil(N / 64));
- the blocked scans over 4.3M rows, behind the seed sample's rank-th best: int8 at B = 1024,
  bf16 and fp16 at B = 1024 and 4096 (configuration 2's largest batch, clustered rows), and
  configuration 5's main path (512-bit codes, B = 256, k = 1000: a seed of 1,024,000 rows, the
  Bloom words stored transposed, the exact clauses fused);
- the small-batch scan's fallback when the seed's rank-th bound fails.

The tables repeat a set of distinct base rows, so the oracle scores only those and selects
through ``oracle.select.RepeatedRows`` (pinned against ``topk_rows`` in ``tests/test_oracle.py``).
Bloom ∧ exact equals exact (``retrieve/tests/parity/test_official.py:455-484``): each test checks
that the GPU's Bloom words have no false negative against the oracle's exact predicate, so the
oracle's exact predicate alone is the filter."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import filters as of
from oracle import scan as osc
from oracle import select as osel
from tests.conftest import rng

pytestmark = pytest.mark.gpu

N_SEEDED = 2_300_000  # above the small-batch scan's seed threshold (2**21 rows)
N_LARGE = 4_300_000  # the blocked scans' seed samples a 16th of it (k = 100), a 4th (k = 1000)


@pytest.fixture(scope="module")
def dev():
    import retrieve_amd.hip  # noqa: F401
    import retrieve_amd.st  # noqa: F401

    return torch.device("cuda:0")


def _unpack(words: np.ndarray, n: int) -> np.ndarray:
    """``[B, W]`` int64 words → ``[B, n]`` bool, item d at bit 63 - d % 64 of word d // 64."""
    be = np.ascontiguousarray(words).view(np.uint64).astype(">u8")
    return np.unpackbits(be.view(np.uint8), axis=1)[:, :n].astype(bool)


def _int8_rows(g, rows: int, d: int) -> np.ndarray:
    """Per-row int8 codes of N(0,1) rows (the bench's ``quantize_rows``)."""
    x = torch.from_numpy(g.standard_normal((rows, d)).astype(np.float32))
    return bench.quantize_rows(x).numpy()


def _check_exact(ids, sc, base_sc, rep, k, valid=None):
    ids, sc = ids.cpu().numpy(), sc.cpu().numpy()
    for r in range(ids.shape[0]):
        want_i, want_s = rep.topk(base_sc[r], k, None if valid is None else valid[r])
        assert np.array_equal(ids[r], want_i), f"row {r}: ids differ"
        assert np.array_equal(sc[r], want_s.astype(sc.dtype)), f"row {r}: scores differ"


def _filter_oracle(attrs: torch.Tensor, sets: np.ndarray, words: np.ndarray, n: int):
    """The oracle's exact predicate, after checking the Bloom words hold every exact match."""
    exact = of.clause_match_sets(attrs.cpu().numpy(), sets, np.zeros(attrs.shape[1], bool))
    assert not (exact & ~_unpack(words, n)).any(), "a Bloom false negative"
    return exact


@pytest.mark.timeout(400)
@pytest.mark.parametrize("n", [N_SEEDED, 30_000_000])
def test_headline_step_as_benched(dev, n):
    """At 2.3M rows (the default seed sample) and at the benched 30M rows (the doubled sample of
    one query group over 2^24 rows or more)."""
    b, d, k, n_base = 16, 512, 100, 8192
    print(f"headline step: int8 clause scan B={b} N={n} D={d} k={k}, bench filter", flush=True)
    g = rng(1300)
    base = _int8_rows(g, n_base, d)
    row_of = g.integers(0, n_base, n)
    q = _int8_rows(g, b, d)
    items = torch.from_numpy(base).to(dev)[torch.from_numpy(row_of).to(dev)]
    flt = bench.Filter(n, b, 0.1, dev)
    words = flt.bloom()
    assert words.shape == (b, -(-n // 2048) * 32) and words.shape[1] > -(-n // 64)
    qt = torch.from_numpy(q).to(dev)
    exact = _filter_oracle(flt.attrs, flt.sets.cpu().numpy(), words.cpu().numpy(), n)
    base_sc, rep = osc.int8_scores(q, base), osel.RepeatedRows(row_of, n_base)
    # bench.py's step: the Bloom plans probed per candidate inside the scan (Filter.scan), whose
    # plans the probe holds (no fallback to the search)
    import retrieve_amd.st as st

    depth = max(1, min(flt.max_stack, st.MAX_STACK))
    assert st._probe_tables(flt.offs, flt.blob, flt.plan_count, depth, bench.BLOOM_K,
                            bench.HASH_K) is not False
    ids, sc = flt.scan(qt, items, k)
    torch.cuda.synchronize()
    _check_exact(ids, sc, base_sc, rep, k, exact)
    # its --bloom-search form: the search's words, then the clause scan
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(qt, items, k, flt.attrs, flt.rev,
                                                            flt.sets, words)
    torch.cuda.synchronize()
    _check_exact(ids, sc, base_sc, rep, k, exact)


def test_int8_b1024_large(dev):
    n, b, d, k, n_base = N_LARGE, 1024, 512, 100, 1 << 16
    print(f"int8 scan B={b} N={n} D={d} k={k} (blocked, seeded)", flush=True)
    g = rng(1301)
    base = _int8_rows(g, n_base, d)
    row_of = g.integers(0, n_base, n)
    q = _int8_rows(g, b, d)
    items = torch.from_numpy(base).to(dev)[torch.from_numpy(row_of).to(dev)]
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk(torch.from_numpy(q).to(dev), items, k)
    torch.cuda.synchronize()
    _check_exact(ids, sc, osc.int8_scores(q, base), osel.RepeatedRows(row_of, n_base), k)


def _clustered(g, rows: int, d: int, centres: np.ndarray) -> np.ndarray:
    """Configuration 2's generator: centre[u] + 0.3 N(0,1), u uniform, L2-normalised."""
    x = centres[g.integers(0, centres.shape[0], rows)] + 0.3 * g.standard_normal((rows, d))
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("dtype,b", [(torch.bfloat16, 1024), (torch.bfloat16, 4096),
                                     (torch.float16, 4096)])
def test_dense_large_batch_large(dev, dtype, b):
    """Float scores: within 1e-3 relative of the float64 dot of the rounded values; the k-th
    boundary up to near ties; every item of a base row scoring clearly above the oracle's k-th
    returned; and the copies of one base row (equal scores on the GPU too) taken lowest index
    first, as the tie rule requires."""
    n, d, k, n_base, rtol = N_LARGE, 128, 100, 1 << 16, 1e-3
    print(f"dense scan {dtype} B={b} N={n} D={d} k={k} (blocked, seeded)", flush=True)
    g = rng(1302 + b)
    centres = g.standard_normal((1024, d))
    base = torch.from_numpy(_clustered(g, n_base, d, centres)).to(dtype)
    q = torch.from_numpy(_clustered(g, b, d, centres)).to(dtype)
    row_of = g.integers(0, n_base, n)
    items = base.to(dev)[torch.from_numpy(row_of).to(dev)]
    ids, sc = torch.ops.retrieve_amd.dense_scan_topk(q.to(dev), items, k)
    torch.cuda.synchronize()
    ids, sc = ids.cpu().numpy(), sc.cpu().numpy()
    rep = osel.RepeatedRows(row_of, n_base)
    base64, q64 = base.double().numpy(), q.double().numpy()
    for r0 in range(0, b, 512):
        exact = osc.dense_scores(q64[r0:r0 + 512], base64)  # [rows, n_base] float64
        for i, r in enumerate(range(r0, min(b, r0 + 512))):
            got = ids[r]
            assert (got >= 0).all() and np.unique(got).size == k
            e = exact[i, row_of[got]]
            assert (np.abs(sc[r] - e) <= rtol * np.maximum(np.abs(e), 1e-3)).all()
            _, want_s = rep.topk(exact[i], k)
            kth = want_s[-1]
            band = 2 * rtol * max(abs(kth), 1e-3)
            assert (e >= kth - band).all()
            above = np.flatnonzero(exact[i] > kth + band)
            assert np.isin(rep.items_of(above), got).all()
            for j in np.unique(row_of[got]).tolist():
                mine = np.sort(got[row_of[got] == j])
                assert np.array_equal(mine, rep.items_of([j])[:mine.size])


@pytest.mark.timeout(400)
def test_config5_main_path_large(dev):
    """512-bit codes, B = 256, k = 1000 over 4.3M rows under the Bloom words of the bench's 10 %
    value sets, stored transposed (read in place by the blocked scan), the exact clauses fused.
    (The oracle's clause predicate over 256 rows x 4.3M items takes about a minute of CPU.)"""
    import retrieve_amd.hip as hip
    import retrieve_amd.st as st
    from retrieve_amd import bloom as bl

    n, b, w, k, n_base = N_LARGE, 256, 8, 1000, 1 << 16
    print(f"1-bit clause scan B={b} N={n} W={w} k={k}, transposed Bloom words", flush=True)
    g = rng(1303)
    base = g.integers(-2**63, 2**63 - 1, (n_base, w), dtype=np.int64)
    q = g.integers(-2**63, 2**63 - 1, (b, w), dtype=np.int64)
    row_of = g.integers(0, n_base, n)
    items = torch.from_numpy(base).to(dev)[torch.from_numpy(row_of).to(dev)]
    attrs = bench.attr_table(n, 4321, dev)
    sets = bench.query_sets(attrs, b, 0.1, 78)
    fid, fo, fv = st.attrs_to_features(attrs.long())
    words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, bench.BLOOM_BITS,
                                                       bench.BLOOM_K)
    del fid, fo, fv
    blob, count, depth = st.prepare_plans(bl.sets_to_expressions(sets), bench.HASH_K, dev)
    mask_t = st.bloom_search_t(words, offs, blob, count, depth, bench.BLOOM_K, bench.HASH_K)
    assert hip._transposed_stride(mask_t, b) > 0  # the blocked scan reads it as it is
    rev = torch.zeros(len(bench.CARDINALITIES), dtype=torch.bool, device=dev)
    ids, sc = torch.ops.retrieve_amd.hamming_scan_topk_clauses(
        torch.from_numpy(q).to(dev), items, k, attrs, rev, torch.from_numpy(sets).to(dev),
        mask_t)
    torch.cuda.synchronize()
    exact = _filter_oracle(attrs, sets, mask_t.contiguous().cpu().numpy(), n)
    _check_exact(ids, sc, osc.hamming_scores(q, base), osel.RepeatedRows(row_of, n_base), k,
                 exact)


@pytest.mark.parametrize("clauses", [False, True])
def test_speculative_seed_bound_falls_back(dev, clauses):
    """The small-batch scan bounds its main pass by the seed sample's rank-th best (the 23rd of
    k = 100 here: 2^17 of 2.3M rows, 256-row blocks every 17 blocks, one seed workgroup a block),
    a bound that fails only when the sample holds more of the top k than chance allows. Query 0's
    30 best rows (its own code with 0 .. 29 leading dimensions zeroed, above every base row) sit
    at the start of sample blocks 1 .. 30, one a seed list, so the 23rd best list is one of them:
    that query's main pass keeps 23 entries and ends short, the flag rises and the fallback pass
    without the bound must give the exact top-k, bit for bit; the other queries are unaffected
    either way."""
    n, b, d, k, n_base = N_SEEDED, 4, 128, 100, 4096
    print(f"speculative seed fallback B={b} N={n} D={d} k={k} clauses={clauses}", flush=True)
    g = rng(1400 + clauses)
    base = _int8_rows(g, n_base, d)
    q = _int8_rows(g, b, d)
    best = np.repeat(q[:1], 30, axis=0)
    for c in range(30):
        best[c, :c] = 0
    base = np.concatenate([base, best])
    base_sc = osc.int8_scores(q, base)
    assert base_sc[0, n_base:].min() > base_sc[0, :n_base].max()
    row_of = g.integers(0, n_base, n)
    planted = 4352 * np.arange(1, 31)  # block j starts at item 256 * 17 * j
    row_of[planted] = n_base + np.arange(30)
    n_base += 30
    items = torch.from_numpy(base).to(dev)[torch.from_numpy(row_of).to(dev)]
    qt = torch.from_numpy(q).to(dev)
    rep = osel.RepeatedRows(row_of, n_base)
    if clauses:
        attrs = g.integers(0, 4, (n, 2, 1)).astype(np.int16)
        attrs[planted, 0, 0] = 0  # query 0's planted rows pass its clause (values 0, 2)
        sets = np.full((b, 2, 2), -1, np.int64)
        sets[:, 0, :2] = [0, 2]
        sets[1:, 1, 0] = 3
        rev = np.zeros(2, bool)
        valid = of.clause_match_sets(attrs, sets, rev)
        ids, sc = torch.ops.retrieve_amd.int8_scan_topk_clauses(
            qt, items, k, torch.from_numpy(attrs).to(dev), torch.from_numpy(rev).to(dev),
            torch.from_numpy(sets).to(dev))
    else:
        valid = None
        ids, sc = torch.ops.retrieve_amd.int8_scan_topk(qt, items, k)
    torch.cuda.synchronize()
    _check_exact(ids, sc, base_sc, rep, k, valid)
