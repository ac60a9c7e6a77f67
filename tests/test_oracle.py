"""The CPU oracle against the reference's golden vectors, closed forms and brute force."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import filters as of
from oracle import quantize as oq
from oracle import scan as osc
from oracle import select as osel
from tests.conftest import rng


# --- int8 ---------------------------------------------------------------------------------


def test_int8_kat(kat):
    a, _ = kat
    s = osc.int8_scores(a["int8_kat_query"], a["int8_kat_items"])
    assert s.tolist() == [a["int8_kat_scores"].tolist()]
    ids, sc = osc.int8_topk(a["int8_kat_query"], a["int8_kat_items"], 2)
    assert ids.tolist() == [[1, 0]] and sc.tolist() == [[39, 17]]


def test_int8_scores_equal_python_int_dots():
    g = rng(1)
    q = g.integers(-128, 128, (3, 64), dtype=np.int8)
    it = g.integers(-128, 128, (50, 64), dtype=np.int8)
    got = osc.int8_scores(q, it)
    for b in range(3):
        for n in range(50):
            want = sum(int(x) * int(y) for x, y in zip(q[b], it[n]))
            assert got[b, n] == want


def test_int8_scores_extreme_accumulation():
    # the largest |dot| at D = 1024: (-128)(-128) * 1024 = 2**24, still exact
    q = np.full((1, 1024), -128, np.int8)
    it = np.full((2, 1024), -128, np.int8)
    it[1] = 127
    assert osc.int8_scores(q, it).tolist() == [[2**24, -128 * 127 * 1024]]


# --- popcount / Hamming -------------------------------------------------------------------


def test_popcount_kat(kat):
    a, _ = kat
    assert osc.popcount64(a["popcount_kat_in"]).tolist() == a["popcount_kat_out"].tolist()


def test_popcount_random_words():
    x = rng(2).integers(-(2**63), 2**63 - 1, 200, dtype=np.int64)
    want = [bin(int(v) & ((1 << 64) - 1)).count("1") for v in x]
    assert osc.popcount64(x).tolist() == want


def test_hamming_equals_pm1_dot():
    """``64 W - 2 * hamming`` is the dot product of the ±1 expansions of the bits."""
    g = rng(3)
    q = g.integers(-(2**63), 2**63 - 1, (4, 8), dtype=np.int64)
    it = g.integers(-(2**63), 2**63 - 1, (30, 8), dtype=np.int64)

    def pm1(words):
        u = words.view(np.uint64)
        bits = (u[..., None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)
        return bits.reshape(words.shape[0], -1).astype(np.int64) * 2 - 1

    assert np.array_equal(osc.hamming_scores(q, it), pm1(q) @ pm1(it).T)


# --- selection ----------------------------------------------------------------------------


def _brute_topk(scores, k, valid=None):
    out = []
    for r, row in enumerate(scores.tolist()):
        cand = [(-s, i) for i, s in enumerate(row) if valid is None or valid[r][i]]
        out.append([i for _, i in sorted(cand)[:k]])
    return out


@pytest.mark.parametrize("n,k", [(10, 3), (200, 50), (1000, 7), (37, 37), (5, 9)])
def test_topk_rows_brute_force_heavy_ties(n, k):
    g = rng(n * 31 + k)
    s = g.integers(-3, 4, (6, n)).astype(np.int32)
    valid = g.random((6, n)) > 0.2
    ids, sc = osel.topk_rows(s, k, valid)
    want = _brute_topk(s, k, valid)
    for r in range(6):
        m = len(want[r])
        assert ids[r, :m].tolist() == want[r]
        assert (ids[r, m:] == -1).all() and (sc[r, m:] == osel.INT32_MIN).all()
        assert sc[r, :m].tolist() == [s[r, i] for i in want[r]]


@pytest.mark.parametrize("n,k,chunk", [(1000, 7, 64), (300, 50, 37), (90, 100, 16),
                                       (5000, 20, 4096)])
def test_dense_topk_chunked_equals_brute_force(n, k, chunk):
    """Small-integer-valued rows give exact float64 scores with heavy ties across chunk
    boundaries: the chunked selection must equal the Python brute force (score desc, id asc),
    masks and short rows included."""
    g = rng(n + k + chunk)
    q = g.integers(-2, 3, (5, 8)).astype(np.float32)
    items = g.integers(-2, 3, (n, 8)).astype(np.float32)
    valid = g.random((5, n)) > 0.3
    valid[1] = False
    valid[2] = g.random(n) < 0.01
    s = q.astype(np.float64) @ items.T.astype(np.float64)
    want = _brute_topk(s, k, valid)
    ids, sc = osc.dense_topk_chunked(q, items, k, valid, chunk=chunk)
    for r in range(5):
        m = len(want[r])
        assert ids[r, :m].tolist() == want[r]
        assert (ids[r, m:] == -1).all() and np.isneginf(sc[r, m:]).all()
        assert sc[r, :m].tolist() == [s[r, i] for i in want[r]]
    ids2, _ = osc.dense_topk_chunked(q, items, k, None, chunk=chunk)
    assert np.array_equal(ids2, osc.dense_topk(q, items, k)[0])


def test_merge_topk_equals_topk_of_union():
    g = rng(4)
    s = g.integers(0, 5, (3, 40)).astype(np.float32)
    ids = np.tile(np.arange(40), (3, 1))
    a_s, a_i = osel.merge_topk(s[:, :17], ids[:, :17], s[:, 17:], ids[:, 17:], 9)
    want_i, want_s = osel.topk_rows(s, 9)
    assert np.array_equal(a_i, want_i) and np.array_equal(a_s, want_s)


def test_lowest_id_tie_kat(kat):
    """The reference harness's planted tie: items 2 and 13 identical; the lower id first."""
    a, meta = kat
    items, queries = a["tie_items"], a["tie_queries"]
    masks = a["tie_masks"][a["tie_qa"]]
    scores = (queries @ items.T).astype(np.float32)
    ids, _ = osel.topk_rows(scores, meta["tie_k"], masks)
    assert ids[5, 4:].tolist() == meta["tie_row5_tail"]


def test_composite_key_orders_score_desc_then_id_asc():
    s = np.array([5, 5, -3, 7, 5], np.int32)
    i = np.array([9, 2, 0, 100, 3])
    c = osel.composite_key(s, i)
    order = np.argsort(-c.astype(np.float64), kind="stable")  # exact for these magnitudes
    order = sorted(range(5), key=lambda j: -int(c[j]))
    assert [int(i[j]) for j in order] == [100, 2, 3, 9, 0]


# --- quantization -------------------------------------------------------------------------


def test_quantize_extremes(kat):
    a, _ = kat
    codes, scales = oq.quantize_int8(a["quant_extremes_in"])
    assert codes[:, 0].tolist() == [127, 127] and codes[:, 1].tolist() == [-127, -127]
    assert codes.max() <= 127 and codes.min() >= -127
    assert np.allclose(scales, np.array([1.0, 2.0]) / 127.0, atol=1e-6)


def test_quantize_half_to_even(kat):
    a, _ = kat
    codes, _ = oq.quantize_int8(a["quant_half_in"])
    assert codes.tolist() == a["quant_half_codes"].tolist()


def test_quantize_zero_and_tiny_rows():
    x = np.zeros((2, 16), np.float32)
    x[1, 3] = 1e-30
    codes, scales = oq.quantize_int8(x)
    assert (codes[0] == 0).all() and np.isfinite(scales).all()
    assert scales[0] == np.float32(1e-8) * (np.float32(1) / np.float32(127))
    assert codes[1, 3] == 0  # 1e-30 / 1e-8 * 127 rounds to 0


def _nearest_f32(fr) -> np.float32:
    """The float32 nearest the rational ``fr`` (ties to even), by exact comparison."""
    from fractions import Fraction

    lo = np.float32(float(fr))  # within one ulp of fr
    best = None
    for c in (np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - fr)
        key = (err, int(np.frombuffer(c.tobytes(), np.uint32)[0]) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


@pytest.mark.parametrize("shape", [(300, 32), (7, 5), (1, 1)])
def test_quantize_global_against_torch_eager(shape):
    """The reference's quantize_int8_global is torch eager fp32 ops (indexing/quantize.py:25-52):
    run those same ops on the CPU and compare bit for bit; plus the closed-form properties."""
    import torch

    from oracle import quantize as oq

    g = rng(31)
    x = (g.standard_normal(shape) * 3).astype(np.float32)
    x.flat[0] = -np.abs(x).max() * 1.5  # the extreme is negative: -min decides
    perm = g.permutation(shape[0])
    codes, abs_max = oq.quantize_int8_global(x, perm)
    t = torch.from_numpy(x)
    am = torch.maximum(t.amax(), -t.amin()).clamp(min=1e-8)
    want = (t[torch.from_numpy(perm)] / am * 127.0).round().clamp(-128, 127).to(torch.int8)
    assert np.array_equal(codes, want.numpy())
    assert abs_max == np.float32(am.item())
    # the extreme element maps to -127 exactly; every code reconstructs within half a step
    assert codes[np.argsort(perm)[0]].flat[0] == -127
    scale = np.float32(abs_max / np.float32(127))
    assert (np.abs(codes.astype(np.float64) * scale - x[perm]) <= scale / 2 * (1 + 1e-5)).all()
    plain, _ = oq.quantize_int8_global(x)
    assert np.array_equal(plain[perm], codes)


def test_quantize_global_zero_table():
    from oracle import quantize as oq

    codes, abs_max = oq.quantize_int8_global(np.zeros((3, 4), np.float32))
    assert abs_max == np.float32(1e-8) and not codes.any()


def test_quantize_divide_scale_is_the_rounded_quotient():
    """The ``divide`` scale is the float32 nearest ``abs_max / 127`` (exact rational), which
    differs from ``abs_max * fp32(1/127)`` for some ``abs_max``; the codes do not depend on it."""
    from fractions import Fraction

    g = rng(77)
    x = (g.standard_normal((400, 8)) * np.exp(3 * g.standard_normal((400, 1)))).astype(np.float32)
    codes_d, s_div = oq.quantize_int8(x, divide=True)
    codes_m, s_mul = oq.quantize_int8(x)
    assert np.array_equal(codes_d, codes_m)
    m = np.abs(x).max(axis=1)
    for i in range(x.shape[0]):
        assert s_div[i] == _nearest_f32(Fraction(float(m[i])) / 127)
    assert (s_div != s_mul).any()


def test_pack_signs_lsb_first():
    v = np.full((1, 128), -1.0, np.float32)
    v[0, 0] = 1.0  # word 0 bit 0
    v[0, 127] = 1.0  # word 1 bit 63
    w = oq.pack_signs(v).view(np.uint64)
    assert w[0, 0] == 1 and w[0, 1] == np.uint64(1) << np.uint64(63)


# --- filters ------------------------------------------------------------------------------


def test_clause_match_brute_force():
    g = rng(5)
    attrs = g.integers(-1, 4, (60, 3, 2))
    rev = np.array([False, True, False])
    q = g.integers(-1, 4, (7, 3))
    got = of.clause_match(attrs, rev, q)
    for b in range(7):
        for n in range(60):
            ok = True
            for c in range(3):
                if q[b, c] == -1:
                    continue
                m = any(v == q[b, c] for v in attrs[n, c])
                ok &= m != rev[c]
            assert got[b, n] == ok


def test_clause_sets_reduce_to_singletons():
    g = rng(6)
    attrs = g.integers(-1, 5, (80, 4, 1))
    q = g.integers(-1, 5, (9, 4))
    q = np.where(q == -1, -1, q)
    got = of.clause_match_sets(attrs, q[:, :, None])
    # an item value of -1 never matches a set, while clause_match compares -1 == -1 only
    # for inactive clauses (skipped), so the two agree
    assert np.array_equal(got, of.clause_match(attrs, np.zeros(4, bool), q))
    rev = np.array([True, False, True, False])
    assert np.array_equal(of.clause_match_sets(attrs, q[:, :, None], rev),
                          of.clause_match(attrs, rev, q))
    # a set is the OR of its singletons: two-value sets against a by-hand union
    two = g.integers(0, 5, (9, 4, 2))
    two[:, 1:, :] = -1  # only clause 0 active
    union = of.clause_match_sets(attrs, two[:, :, :1]) | of.clause_match_sets(attrs, two[:, :, 1:])
    assert np.array_equal(of.clause_match_sets(attrs, two), union)


def test_murmur_smhasher_verification(kat):
    _, meta = kat
    assert of.smhasher_verification() == meta["murmur3_x64_128_verification"]


def test_readme_bloom_kat(kat):
    a, meta = kat
    attrs = a["readme_attrs"]
    words, offs = of.bloom_build(attrs, meta["readme_build_k"],
                                 b_multiplier=meta["readme_b_multiplier"])
    for text, hits in zip(meta["readme_queries"], meta["readme_hits"]):
        m = of.bloom_expression_mask(words, offs, 4, text, meta["readme_build_k"],
                                     meta["readme_hash_k"])
        assert np.nonzero(m)[0].tolist() == hits
        assert np.nonzero(of.exact_expression_mask(attrs, text))[0].tolist() == hits


def test_expression_mapping_kat(kat):
    a, meta = kat
    assert of.queries_to_expressions(a["expr_kat_in"]) == meta["expr_kat_out"]
    assert of.queries_to_expressions(a["expr_kat_in"], [False, True]) == \
        meta["expr_kat_out_reverse"]


def test_bloom_layout_position():
    """Doc 70 sits in bundle 0, column 1, bit 57; doc 2050 in bundle 1, column 0, bit 61."""
    attrs = np.full((2100, 1, 1), -1, np.int64)
    attrs[70, 0, 0] = 5
    attrs[2050, 0, 0] = 5
    words, offs = of.bloom_build(attrs, 3, bits_per_doc=64)
    assert offs.tolist() == [0, 64, 128]
    pos = of.bit_positions(0, 5, 64, 3)
    w = words.view(np.uint64)
    want = {}
    for p in pos:
        want[p * 32 + 1] = np.uint64(1) << np.uint64(57)
        want[(64 + p) * 32 + 0] = np.uint64(1) << np.uint64(61)
    nz = {int(i): w[i] for i in np.nonzero(w)[0]}
    assert nz == want


def test_bloom_no_false_negatives():
    g = rng(7)
    attrs = g.integers(0, 20, (3000, 3, 1))
    words, offs = of.bloom_build(attrs, 3, bits_per_doc=64)
    for f in range(3):
        for v in range(0, 20, 3):
            m = of.term_mask(words, offs, 3000, f, v, 3, 7)
            exact = (attrs[:, f, 0] == v)
            assert (m | ~exact).all()  # every doc holding the token is found


@pytest.mark.parametrize("bits", [64, 40])
def test_bloom_doc_bits(bits):
    """The row view: each document's word is the OR of its tokens' build positions (computed
    from the tokens, not the words), and a term's test on it (all its search positions set) is
    ``term_mask``'s column-wise answer."""
    g = rng(bits)
    n = 4500  # three bundles, the last one partial
    attrs = g.integers(-1, 12, (n, 3, 2))
    words, offs = of.bloom_build(attrs, 3, bits_per_doc=bits)
    got = of.bloom_doc_bits(words, offs, n).view(np.uint64)
    want = np.zeros(n, np.uint64)
    for d in range(n):
        for c in range(3):
            for v in attrs[d, c]:
                if v != -1:
                    for p in of.bit_positions(c, int(v), bits, 3):
                        want[d] |= np.uint64(1) << np.uint64(p)
    assert np.array_equal(got, want)
    for f, v in [(0, 3), (1, 0), (2, 11)]:
        m = np.uint64(sum(1 << p for p in of.probe_positions(f, v, bits, 3, 7)))
        assert np.array_equal((got & m) == m, of.term_mask(words, offs, n, f, v, 3, 7))


def test_cpu_baseline_hamming_topk_equals_oracle():
    """The bench's CPU baseline for the 1-bit scan (XOR + bitwise_count over item chunks, a
    lexsort merge per chunk) against the oracle's full-scan top-k: few distinct rows, so every
    boundary is a tie broken by the lower id, with and without a filter."""
    from oracle import baseline

    g = rng(71)
    base = g.integers(-(2**63), 2**63 - 1, (37, 8), dtype=np.int64)
    items = base[g.integers(0, 37, 5000)]
    q = g.integers(-(2**63), 2**63 - 1, (5, 8), dtype=np.int64)
    valid = g.random((5, 5000)) < 0.3
    for v in (None, valid):
        s, i = baseline.hamming_topk_cpu(q, items, 50, v, chunk=700)
        want_i, want_s = osc.hamming_topk(q, items, 50, v)
        assert np.array_equal(i, want_i) and np.array_equal(s, want_s)


def test_candidate_topk_brute_force():
    """``candidate_topk`` against a brute-force full sort over each row's first ``counts[b]``
    candidates (tie-heavy scores, duplicates, short rows) and against ``candidate_int8_topk``."""
    g = rng(91)
    b, p, k = 6, 40, 7
    cand = g.integers(0, 25, (b, p))
    counts = np.array([40, 3, 0, 39, 7, 12])
    table = g.integers(-2, 3, 25)  # few distinct scores: ties everywhere
    ids, sc = osc.candidate_topk(lambda r, c: table[c], cand, counts, k, pad_to_k=True,
                                 empty_score=np.iinfo(np.int64).min)
    for r in range(b):
        c = cand[r, : counts[r]]
        pairs = sorted(((-int(table[i]), int(i)) for i in c))[:k]
        want = [i for _, i in pairs] + [-1] * (k - len(pairs))
        assert ids[r].tolist() == want
    codes = g.integers(-128, 128, (25, 64), dtype=np.int8)
    q = g.integers(-128, 128, (b, 64), dtype=np.int8)
    full = np.full(b, p)
    ids2, sc2 = osc.candidate_topk(lambda r, c: osc.int8_scores(q[r:r + 1], codes[c])[0], cand,
                                   full, 9, pad_to_k=False, empty_score=np.iinfo(np.int32).min)
    want_ids, want_sc = osc.candidate_int8_topk(q, codes, cand, 9)
    assert np.array_equal(ids2, want_ids) and np.array_equal(sc2.astype(np.int32), want_sc)


def test_gemv_oracle_equals_fma_order():
    """The float32 oracle of the in-order fp16 GEMV against exact rational arithmetic per step:
    every step is round-to-nearest of (acc + q_k * e_k) with the product exact."""
    from fractions import Fraction

    g = rng(95)
    q = g.standard_normal(40).astype(np.float16)
    e = g.standard_normal((40, 5)).astype(np.float16)
    got = osc.gemv_scores(q, e)
    for n in range(5):
        acc = np.float32(0)
        for k in range(40):
            exact = Fraction(float(acc)) + Fraction(float(q[k])) * Fraction(float(e[k, n]))
            acc = np.float32(float(exact))  # one rounding (float(exact) is exact-enough here)
        assert got[n] == acc


def test_search_oracle_one_list_is_the_full_scan():
    """One list of every item, identity permutation: the search oracle is the int8 full-scan
    top-k of the quantized rows (pinned by the int8 KAT), scored (dot * scale) * global_scale."""
    from oracle import quantize as oq
    from oracle import silvertorch as ost

    g = rng(96)
    n, d, b, k = 3000, 64, 5, 20
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    q = g.standard_normal((b, d)).astype(np.float32)
    ids, sc = ost.search(q, np.zeros((b, 1), np.int64), [0], [n], items, np.arange(n), [0.5], k,
                         n)
    codes, scales = oq.quantize_int8(q)
    want_ids, want_dots = osc.int8_topk(codes, items, k)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(sc, (want_dots.astype(np.float32) * scales[:, None]) * np.float32(0.5))


def test_search_oracle_slot_order_by_hand():
    """Two clusters probed in the order [1, 0]: slots are cluster 1's items, then cluster 0's;
    equal rows tie, so the lowest slots win; ``width`` truncates; ``sort_perm`` maps ids."""
    from oracle import silvertorch as ost

    items = np.ones((6, 16), np.int8)  # every dot equal
    perm = np.array([10, 11, 12, 13, 14, 15])
    q = np.ones((1, 16), np.float32)
    ids, _ = ost.search(q, np.array([[1, 0]]), [0, 4], [4, 2], items, perm, [1.0], 3, 64)
    assert ids.tolist() == [[14, 15, 10]]
    ids, _ = ost.search(q, np.array([[1, 0]]), [0, 4], [4, 2], items, perm, [1.0], 8, 5)
    # width 5 -> 32 slots after rounding: all 6 items, then -1 pads
    assert ids.tolist() == [[14, 15, 10, 11, 12, 13, -1, -1]]


def test_search_oracle_warps_then_remainders_by_hand():
    """The GPU scorer's write order (``fork_search_cuda.cu:989-991`` full warps, ``:1051-1053``
    remainders): clusters of 40, 50 and 7 docs at positions 0, 40 and 90, probed [1, 0, 2].
    Slots 0-31: cluster 1's first warp (40-71); 32-63: cluster 0's (0-31); cluster 2 has no full
    warp; then the remainders in probe order: 64-81 cluster 1 (72-89), 82-89 cluster 0 (32-39),
    90-96 cluster 2 (90-96). Every dot is equal, so the top-k is the lowest slots."""
    from oracle import silvertorch as ost

    offs, sizes = [0, 40, 90], [40, 50, 7]
    want = (list(range(40, 72)) + list(range(0, 32)) + list(range(72, 90)) + list(range(32, 40))
            + list(range(90, 97)))
    assert ost.row_slots([1, 0, 2], offs, sizes, 97, 128).tolist() == want
    assert ost.row_slots([1, 0, 2], offs, sizes, 97, 70).tolist() == want[:70]
    items = np.ones((97, 16), np.int8)
    perm = np.arange(97) + 1000
    q = np.ones((2, 16), np.float32)
    ids, _ = ost.search(q, np.array([[1, 0, 2], [2, 1, 0]]), offs, sizes, items, perm, [1.0],
                        97, 97)
    assert ids[0].tolist() == [1000 + p for p in want]
    want1 = (list(range(40, 72)) + list(range(0, 32)) + list(range(90, 97)) + list(range(72, 90))
             + list(range(32, 40)))
    assert ids[1].tolist() == [1000 + p for p in want1]


def test_fused_kmean_ann_per_doc_scale_rounds_twice():
    """The per-doc fp16 scale branch restates ``c10::Half(dot) / scale``
    (``index_mm_helpers.cuh:51-53``): fp16(fp32(fp16(dot)) / scale). Hand-computed from IEEE
    half arithmetic: 2051 lies halfway between the fp16 values 2050 and 2052 (spacing 2 on
    [2048, 4096)), so it rounds to the even significand, 2052, and 2052 / 1.5 = 1368 exactly;
    2053 rounds to 2052 too, and 2052 / 0.75 = 2736. One rounding (fp16(2051 / 1.5) = 1367,
    fp16(2053 / 0.75) = 2738, Meta's CPU twin ``fused_kmean_ann.cpp:200-202``) differs, so the
    test tells the two apart."""
    from oracle import silvertorch as ost

    d = 64
    q = np.ones((1, d), np.int8)
    emb = np.zeros((2, d), np.int8)
    emb[:, :16] = 127
    emb[:, 16] = [19, 21]
    assert (emb.astype(np.int64) @ q[0].astype(np.int64)).tolist() == [2051, 2053]
    sc, ix = ost.fused_kmean_ann([0, 2], np.zeros((1, 1), np.int64), np.array([[2]]), emb, q, 2,
                                 scale=np.array([1.5, 0.75], np.float16))
    assert sc.dtype == np.float16
    assert sc[0, :2].astype(np.float64).tolist() == [1368.0, 2736.0]
    assert ix[0, :2].tolist() == [0, 1]
    once = [float(np.float16(2051 / 1.5)), float(np.float16(2053 / 0.75))]
    assert once == [1367.0, 2738.0]


@pytest.mark.parametrize("k", [1, 7, 100, 1000, 3500])
@pytest.mark.parametrize("kind", ["int", "float"])
@pytest.mark.parametrize("n_base", [60, 700])
def test_repeated_rows_topk_equals_topk_rows(k, kind, n_base):
    """``RepeatedRows.topk`` (the GPU tests' oracle over tables of repeated base rows) equals
    ``topk_rows`` over the expanded ``[B, N]`` scores: few distinct scores (ties across base rows
    and, by construction, within every base row), masks with empty rows, k above N; 700 base
    rows take the partial-selection path (more than its first 64 candidates, grown 4x)."""
    g = rng(1200 + k + n_base)
    n, b = 3000, 12
    row_of = g.integers(0, n_base, n)
    if kind == "int":
        base = g.integers(-5, 5, (b, n_base)).astype(np.int32)
    else:
        base = (g.integers(-5, 5, (b, n_base)) * 0.25).astype(np.float32)
    valid = g.random((b, n)) < 0.5
    valid[3] = False
    rep = osel.RepeatedRows(row_of, n_base)
    for v in (None, valid):
        want_i, want_s = osel.topk_rows(base[:, row_of], k, v)
        for r in range(b):
            got_i, got_s = rep.topk(base[r], k, None if v is None else v[r])
            assert np.array_equal(got_i, want_i[r]) and np.array_equal(got_s, want_s[r])
