"""Every BASELINE configuration's kernels at the batch shape the configuration runs, against the
oracle:

- configuration 1 (exact inner-product top-100, 100k x 128 fp32 L2-normalised rows, 1024
  queries; the reference runs it with torch.mm + torch.topk on the CPU): the same problem on the
  GPU in fp32 (the raw scorer and the key select), at full size, with duplicated rows whose
  equal scores must come back in index order;
- configuration 2 (bf16 10M x 128, B in {1, 64, 1024, 4096}): B = 512 / 1024 over 2.2M clustered
  rows, the narrow 256-byte-row layout with the seed pass (its k-th and rank-th bounds) and the
  main pass, masked and unmasked, bf16 and fp16, with rows whose only survivors sit in two
  64-row tiles, one of them outside every seed sample block;
- configuration 3 (filtered bf16, B = 256): the masked register-blocked bf16 / fp16 kernel at
  B in {40, 128, 256} with empty rows, rows of fewer than k survivors and rows whose survivors
  all score below zero (the float hit test's non-raw path), and the whole pipeline (Bloom
  pre-filter -> exact clause post-check -> scan) at 1 %, 10 % and 50 % selectivity;
- configuration 5 (filtered 1-bit top-1000 + int8 re-rank, B = 256): the masked narrow-layout
  512-bit Hamming kernel at k = 1000 with ties and the extreme scores +-512, and the whole
  pipeline (Bloom -> clause -> Hamming top-1000 -> int8 re-rank top-100).

Integer paths are bit-exact; bf16 / fp16 scores within 1e-3 relative of the float64 dot of the
returned ids, ids equal to the exact top-k outside a tolerance band at the k-th score."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import baseline as obase
from oracle import filters as ofl
from oracle import quantize as oq
from oracle import scan as osc
from tests.conftest import rng
from tests.test_dense_scan import RTOL, _check as _dense_check, _clustered
from tests.test_hamming_scan import _check as _hamming_check, _codes
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu

CARDINALITIES = (16, 32, 64, 128, 256, 512, 1000, 1000)
BLOOM_BITS, BLOOM_K, HASH_K = 64, 3, 7


def test_config1_exact_fp32(dev):
    g = rng(1001)
    n, d, b, k = 100_000, 128, 1024, 100
    x = g.standard_normal((n, d))
    items = (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)
    qx = g.standard_normal((b, d))
    q = (qx / np.linalg.norm(qx, axis=1, keepdims=True)).astype(np.float32)
    # exact ties: copies of a query's own direction at three indices
    items[[500, 70_000, 99_999]] = q[3]
    ids = _dense_check(dev, q, items, k, dtype=torch.float32)
    assert ids[3, :3].tolist() == [500, 70_000, 99_999]


# --- packed masks too large to unpack whole ----------------------------------------------------


class PackedMask:
    """``[B, ceil(N/64)]`` words (item d at bit 63 - d % 64) that unpack per column range, so a
    ``[B, N]`` bool matrix of a 2.2M-row table is never held whole (``valid[:, a:b]`` with
    ``a`` a multiple of 64, as ``osc.dense_topk_chunked`` slices)."""

    def __init__(self, words: np.ndarray, n: int):
        self.words = np.ascontiguousarray(words).view(np.uint64)
        self.n = n

    def __getitem__(self, idx):
        rows, cols = idx
        a, b = cols.start, min(cols.stop, self.n)
        assert a % 64 == 0
        w = self.words[rows, a // 64 : (b + 63) // 64]
        bits = np.unpackbits(w.astype(">u8").view(np.uint8), axis=-1)
        return bits[..., : b - a].astype(bool)

    def row_bits(self, r: int, ids: np.ndarray) -> np.ndarray:
        ids = np.asarray(ids, np.int64)
        return ((self.words[r, ids // 64] >> (np.uint64(63) - (ids % 64).astype(np.uint64)))
                & np.uint64(1)).astype(bool)


def _check_dense_large(dev, q32, it32, k, dtype, mask: PackedMask | None = None):
    """``tests.test_dense_scan._check`` for tables whose [B, N] score matrix does not fit: the
    exact top-k from the chunked float64 oracle, exact scores of the returned ids only."""
    print(f"dense scan {dtype} B={q32.shape[0]} N={it32.shape[0]} D={q32.shape[1]} k={k} "
          f"mask={mask is not None}", flush=True)
    qt = torch.from_numpy(q32).to(dev).to(dtype)
    it = torch.from_numpy(it32).to(dev).to(dtype)
    mt = None if mask is None else torch.from_numpy(mask.words.view(np.int64)).to(dev)
    ids, sc = torch.ops.retrieve_amd.dense_scan_topk(qt, it, k, mt)
    torch.cuda.synchronize()
    ids, sc = ids.cpu().numpy(), sc.cpu().numpy()
    qv = qt.float().cpu().numpy().astype(np.float64)
    iv = it.float().cpu().numpy()
    del it, qt
    want_ids, want_sc = osc.dense_topk_chunked(qv, iv, k, mask)
    for r in range(q32.shape[0]):
        m = int((want_ids[r] >= 0).sum())
        assert (ids[r, m:] == -1).all() and np.isneginf(sc[r, m:]).all(), r
        got = ids[r, :m]
        assert (got >= 0).all() and len(set(got.tolist())) == m, r
        if mask is not None:
            assert mask.row_bits(r, got).all(), r
        e = iv[got].astype(np.float64) @ qv[r]
        assert (np.abs(sc[r, :m] - e) <= RTOL * np.maximum(np.abs(e), 1e-3)).all(), r
        if m:
            assert (sc[r, : m - 1] >= sc[r, 1:m]).all(), r
            kth = want_sc[r, m - 1]
            band = RTOL * max(abs(kth), 1e-3) * 2
            assert (e >= kth - band).all(), r
            missing = np.array(sorted(set(want_ids[r, :m].tolist()) - set(got.tolist())),
                               np.int64)
            if missing.size:
                assert (iv[missing].astype(np.float64) @ qv[r] <= sc[r, m - 1] + band).all(), r
    return ids


def _large_mask(g, q32, it32, b, n) -> PackedMask:
    """Random 1/4-density rows plus rows the seed's bounds must not lose: no survivors, 37
    survivors, survivors only in tiles 1 and 17 (rows 64-127, inside the seed's first sample
    block, and 1088-1151, outside every block: the 64-row tiles of the narrow 256-byte-row
    layout), and survivors that all score below zero."""
    w = (n + 63) // 64
    words = g.integers(0, 2**64, (b, w), dtype=np.uint64) & g.integers(0, 2**64, (b, w),
                                                                        dtype=np.uint64)
    words[0] = 0
    words[1] = 0
    few = g.choice(n, 37, replace=False)
    for i in few:
        words[1, i // 64] |= np.uint64(1) << np.uint64(63 - i % 64)
    words[2] = 0
    words[2, 1] = ~np.uint64(0)
    words[2, 17] = ~np.uint64(0)
    s3 = it32 @ q32[3].astype(np.float32)
    neg = np.nonzero((s3 < 0) & (g.random(n) < 0.3))[0]
    words[3] = 0
    np.bitwise_or.at(words[3], neg // 64, np.uint64(1) << (np.uint64(63) - (neg % 64).astype(
        np.uint64)))
    if n % 64:
        words[:, -1] &= ~np.uint64(0) << np.uint64(64 - n % 64)
    return PackedMask(words, n)


@pytest.fixture(scope="module")
def config2_table():
    """configs[1]'s generator (Gaussian clusters, sigma 0.3, L2-normalised) at 2.2M rows: above
    the blocked scan's seed threshold (8 x 2^18 rows)."""
    g = rng(2)
    centres = g.standard_normal((1024, 128))
    it = _clustered(g, 2_200_000, 128, centres)
    q = _clustered(g, 1024, 128, centres)
    return g, q, it


@pytest.mark.parametrize("b,dtype,masked", [(512, torch.bfloat16, False),
                                            (1024, torch.bfloat16, True),
                                            (1024, torch.float16, False),
                                            (512, torch.float16, True)])
def test_config2_large_batch_seeded(dev, config2_table, b, dtype, masked):
    g, q, it = config2_table
    q = q[:b]
    mask = _large_mask(rng(b + int(masked)), q, it, b, it.shape[0]) if masked else None
    ids = _check_dense_large(dev, q, it, 100, dtype, mask)
    if masked:
        # every survivor of row 2 sits in tiles 1 and 17, 128 of them, so the top-100 is
        # entirely from those tiles
        assert ((64 <= ids[2]) & (ids[2] < 128) | (1088 <= ids[2]) & (ids[2] < 1152)).all()
        assert (ids[0] == -1).all() and (ids[1, :37] >= 0).all() and (ids[1, 37:] == -1).all()


@pytest.mark.parametrize("b", [40, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config3_masked_blocked(dev, b, dtype):
    """The masked register-blocked bf16 / fp16 kernel (configuration 3's main kernel at B = 256;
    wide row quarters at 40 and 128): float group maxima over the rows that pass, with the
    hit test's raw-bits path switched off by rows whose bound is below zero."""
    g = rng(300 + b)
    n = 60_000
    q = g.standard_normal((b, 128)).astype(np.float32)
    it = g.standard_normal((n, 128)).astype(np.float32)
    mask = g.random((b, n)) < 0.1
    mask[0] = False
    mask[1] = g.random(n) < 0.0005  # ~30 survivors < k
    s = it @ q[2]
    mask[2] = (s < 0) & (g.random(n) < 0.2)  # every survivor scores below zero
    mask[3] = (s < -5.0)  # a few strongly negative survivors
    mask[b - 1] = g.random(n) < 0.9
    _dense_check(dev, q, it, 100, dtype, mask)


# --- configuration 3 and 5 pipelines ------------------------------------------------------------


def _zipf_attrs(g, n):
    out = np.empty((n, len(CARDINALITIES), 1), np.int64)
    for c, card in enumerate(CARDINALITIES):
        p = 1.0 / np.arange(1, card + 1) ** 1.1
        out[:, c, 0] = g.choice(card, n, p=p / p.sum())
    return out


def _query_sets(g, attrs, b, selectivity):
    """Row r ANDs 1 + r % 3 attributes, each an OR over its most frequent values (from rank 0 or
    1) until the attribute's mass reaches selectivity ** (1 / attributes)."""
    n = attrs.shape[0]
    freq = [np.bincount(attrs[:, c, 0], minlength=card) / n
            for c, card in enumerate(CARDINALITIES)]
    rows = []
    for r in range(b):
        n_attr = 1 + r % 3
        target = selectivity ** (1.0 / n_attr)
        row = [[] for _ in CARDINALITIES]
        for c in g.choice(len(CARDINALITIES), n_attr, replace=False):
            order = np.roll(np.argsort(-freq[c], kind="stable"), -int(g.integers(0, 2)))
            mass = 0.0
            for v in order:
                if mass >= target:
                    break
                row[c].append(int(v))
                mass += freq[c][v]
        rows.append(row)
    v = max(len(x) for row in rows for x in row)
    out = np.full((b, len(CARDINALITIES), v), -1, np.int64)
    for r, row in enumerate(rows):
        for c, vals in enumerate(row):
            out[r, c, : len(vals)] = vals
    return out


def _filter_mask(dev, attrs, sets):
    """The configuration-3 filter on the GPU: the fixed-width Bloom index (64 bits, 3 hashes)
    searched with prepared plans of the value-set expressions, then the exact clause check
    AND-ed with the Bloom words. Returns (final words, Bloom words) as numpy."""
    import retrieve_amd.st as st
    from retrieve_amd import bloom as bl

    at = torch.from_numpy(attrs).to(dev)
    fid, fo, fv = st.attrs_to_features(at)
    words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, BLOOM_BITS, BLOOM_K)
    blob, count, stack = st.prepare_plans(bl.sets_to_expressions(sets), HASH_K, dev)
    pre = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, stack,
                                                         BLOOM_K, HASH_K)
    rev = torch.zeros(len(CARDINALITIES), dtype=torch.bool, device=dev)
    final = torch.ops.retrieve_amd.clause_bits(at.to(torch.int16), rev,
                                           torch.from_numpy(sets).to(dev), pre)
    torch.cuda.synchronize()
    return final, pre.cpu().numpy()


def _exact_valid(attrs, sets):
    return ofl.clause_match_sets(attrs, sets)


@pytest.mark.parametrize("selectivity", [0.01, 0.1, 0.5])
def test_config3_pipeline(dev, selectivity):
    """Bloom pre-filter -> exact clause post-check -> masked bf16 scan, B = 256, k = 100, over
    200k clustered rows, against the exact filter and the float64 oracle (bloom AND exact ==
    exact, so the result does not depend on the hash)."""
    g = rng(int(selectivity * 1000) + 3)
    n, b = 200_000, 256
    centres = g.standard_normal((1024, 128))
    it = _clustered(g, n, 128, centres)
    q = _clustered(g, b, 128, centres)
    attrs = _zipf_attrs(g, n)
    sets = _query_sets(g, attrs, b, selectivity)
    valid = _exact_valid(attrs, sets)
    final, bloom_words = _filter_mask(dev, attrs, sets)
    got_words = final.cpu().numpy()
    assert np.array_equal(got_words[:, : (n + 63) // 64], _pack(valid)), "exact post-check"
    bloom = PackedMask(bloom_words, n)[:, slice(0, n)]
    assert not (valid & ~bloom).any(), "the Bloom pre-filter dropped a passing item"
    _check_dense_large(dev, q, it, 100, torch.bfloat16, PackedMask(got_words, n))


def test_config5_masked_hamming_k1000(dev):
    """512-bit codes, B = 256 (the narrow layout, two stages beside the lists of k = 1000),
    masked at 0.2 density, exact matches (+512), complements (-512) and repeated rows."""
    g = rng(500)
    n, b = 200_000, 256
    q = _codes(g, b, 8)
    items = _codes(g, n, 8)
    items[100_000:100_500] = items[g.integers(0, 1000, 500)]  # repeated rows: tie groups
    items[7] = q[0]
    items[190_001] = q[0]
    items[9] = ~q[1]
    mask = g.random((b, n)) < 0.2
    mask[0, [7, 190_001]] = True
    mask[1, 9] = True
    mask[2] = False
    mask[3] = g.random(n) < 0.002  # ~400 survivors < k
    _hamming_check(dev, q, items, 1000, mask)


def test_config5_pipeline(dev):
    """SimHash codes of N(0,1) rows, Bloom + exact filter at 10 %, Hamming top-1000, then the int8
    re-rank of the same rows' codes to the top-100: bit-exact against the CPU path
    (``oracle.baseline.hamming_rerank_cpu``)."""
    g = rng(501)
    n, b, d = 200_000, 256, 512
    proj = g.standard_normal((d, d)).astype(np.float32)
    x = g.standard_normal((n, d)).astype(np.float32)
    xq = g.standard_normal((b, d)).astype(np.float32)
    item_bits = oq.simhash_bits(x, proj)
    q_bits = oq.simhash_bits(xq, proj)
    item_codes = oq.quantize_int8(x)[0]
    q_codes = oq.quantize_int8(xq)[0]
    del x
    attrs = _zipf_attrs(g, n)
    sets = _query_sets(g, attrs, b, 0.1)
    valid = _exact_valid(attrs, sets)
    final, _ = _filter_mask(dev, attrs, sets)
    print(f"config 5 pipeline B={b} N={n}", flush=True)
    qb = torch.from_numpy(q_bits).to(dev)
    ib = torch.from_numpy(item_bits).to(dev)
    ids1, s1 = torch.ops.retrieve_amd.hamming_scan_topk(qb, ib, 1000, final)
    counts = (ids1 >= 0).sum(1)
    qc = torch.from_numpy(q_codes).to(dev)
    ic = torch.from_numpy(item_codes).to(dev)
    ids, sc = torch.ops.retrieve_amd.int8_candidates_topk(qc, ic, ids1, counts, 100)
    torch.cuda.synchronize()
    want1, want_s1 = osc.hamming_topk(q_bits, item_bits, 1000, valid)
    assert np.array_equal(ids1.cpu().numpy(), want1)
    assert np.array_equal(s1.cpu().numpy(), want_s1)
    want = obase.hamming_rerank_cpu(q_bits, q_codes, item_bits, item_codes, 1000, 100, valid)
    got = ids.cpu().numpy()
    assert np.array_equal(got, want)
    sc = sc.cpu().numpy()
    for r in range(b):
        m = int((got[r] >= 0).sum())
        dots = item_codes[got[r, :m]].astype(np.int64) @ q_codes[r].astype(np.int64)
        assert np.array_equal(sc[r, :m], dots), r
