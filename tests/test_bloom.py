"""Bloom index on the GPU against the oracle (``oracle.filters``): the build's words bit for bit
(fixed and upstream widths), the plan search's masks for random expressions (uniform widths take
the resolved-position path, mixed widths the per-lane one), the reference's README KAT, and the
exact recheck invariant bloom AND exact == exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import retrieve_amd.st as st
from oracle import filters as of
from oracle import scan as osc
from retrieve_amd import bloom as bl
from tests.conftest import rng
from tests.test_bloom_host import _random_expr
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _attrs(g, n, c, a, vocab, pad):
    x = g.integers(0, vocab, (n, c, a), dtype=np.int64)
    x[g.random((n, c, a)) < pad] = -1
    return x


def _build(dev, attrs, k, *, bits=None, mult=None):
    print(f"bloom build N={attrs.shape[0]} C={attrs.shape[1]} A={attrs.shape[2]} k={k} "
          f"bits={bits} mult={mult}", flush=True)
    fid, fo, fv = st.attrs_to_features(torch.from_numpy(attrs).to(dev))
    if bits is not None:
        words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, bits, k)
    else:
        words, offs = torch.ops.st.bloom_index_build(fid, fo, fv, mult, k)
    torch.cuda.synchronize()
    return words, offs


@pytest.mark.parametrize("n,c,a,bits,k", [(1, 1, 1, 64, 3), (5000, 3, 2, 64, 3),
                                          (4097, 2, 3, 128, 5), (3000, 4, 1, 200, 2)])
def test_build_fixed_matches_oracle(dev, n, c, a, bits, k):
    g = rng(n + c + a + bits + k)
    attrs = _attrs(g, n, c, a, 50, 0.3)
    words, offs = _build(dev, attrs, k, bits=bits)
    want_w, want_o = of.bloom_build(attrs, k, bits_per_doc=bits)
    assert offs.cpu().numpy().tolist() == want_o.tolist()
    assert np.array_equal(words.cpu().numpy(), want_w)


def test_build_upstream_matches_oracle(dev):
    g = rng(81)
    attrs = _attrs(g, 6500, 3, 2, 40, 0.5)  # bundles of different widths
    attrs[4096:6144] = -1  # an empty bundle: width 0
    words, offs = _build(dev, attrs, 3, mult=2.5)
    want_w, want_o = of.bloom_build(attrs, 3, b_multiplier=2.5)
    assert offs.cpu().numpy().tolist() == want_o.tolist()
    assert np.array_equal(words.cpu().numpy(), want_w)


def _search(dev, words, offs, exprs, k, hash_k, prepared=True, as_bool=False):
    if prepared:
        blob, count, max_stack = st.prepare_plans(exprs, hash_k, dev)
        out = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, max_stack,
                                                             k, hash_k, as_bool)
    else:
        _, (data, po) = torch.ops.st.parse_expression_query_batch(
            exprs, torch.ones(len(exprs), dtype=torch.int64), hash_k)
        out = torch.ops.st.bloom_index_search_batch(words, offs, data, po, k, hash_k, as_bool)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _unpack(words: np.ndarray, n: int) -> np.ndarray:
    """[B, W] mask words → [B, n] bool (item d at bit 63 - d % 64 of word d / 64)."""
    bits = np.unpackbits(words.view(np.uint64).astype(">u8").view(np.uint8), axis=1)
    return bits[:, :n].astype(bool)


def test_readme_kat(dev, kat):
    """README corpus, upstream width (b_multiplier 5, build k 3), hash_k 7
    (``test_official.py:229-245, 353-366``)."""
    a, meta = kat
    attrs = a["readme_attrs"]
    words, offs = _build(dev, attrs, meta["readme_build_k"], mult=meta["readme_b_multiplier"])
    for prepared in (True, False):
        for as_bool in (False, True):
            m = _search(dev, words, offs, meta["readme_queries"], meta["readme_build_k"],
                        meta["readme_hash_k"], prepared, as_bool)
            m = m[:, :4] if as_bool else _unpack(m, 4)
            assert [np.flatnonzero(r).tolist() for r in m] == meta["readme_hits"]


@pytest.mark.parametrize("mode", ["fixed", "upstream"])
def test_search_matches_oracle(dev, mode):
    g = rng(82 if mode == "fixed" else 83)
    n = 4500
    attrs = _attrs(g, n, 4, 1, 6, 0.2)
    k, hash_k = 3, 7
    if mode == "fixed":
        words, offs = _build(dev, attrs, k, bits=64)
        ow, oo = of.bloom_build(attrs, k, bits_per_doc=64)
    else:
        attrs[2048:2300, :, :] = -1
        attrs[3000:, 1:, :] = -1  # bundles of different widths
        words, offs = _build(dev, attrs, k, mult=3.0)
        ow, oo = of.bloom_build(attrs, k, b_multiplier=3.0)
    exprs = [_random_expr(g) for _ in range(12)] + ["", "NOT 0:1", "0:1 OR 1:2 OR 2:3"]
    got = _unpack(_search(dev, words, offs, exprs, k, hash_k), n)
    for e, row in zip(exprs, got):
        want = of.bloom_expression_mask(ow, oo, n, e, k, hash_k)
        assert np.array_equal(row, want), e


def test_bloom_and_exact_is_exact(dev):
    """No false negatives: the Bloom mask AND the exact value-set clauses equals the exact
    clauses alone, and gates the int8 scan like the exact mask."""
    g = rng(84)
    n, c = 30_000, 3
    attrs = _attrs(g, n, c, 1, 12, 0.0)
    words, offs = _build(dev, attrs, 3, bits=64)
    sets = g.integers(0, 12, (7, c, 3), dtype=np.int64)
    sets[g.random(sets.shape) < 0.5] = -1
    exprs = bl.sets_to_expressions(sets)
    blob, count, max_stack = st.prepare_plans(exprs, 7, dev)
    bmask = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, max_stack,
                                                           3, 7)
    exact = of.clause_match_sets(attrs, sets)
    assert (_unpack(bmask.cpu().numpy(), n) | ~exact).all()  # no false negatives
    rev = torch.zeros(c, dtype=torch.bool, device=dev)
    ta = torch.from_numpy(attrs).to(dev)
    both = torch.ops.retrieve_amd.clause_bits(ta, rev, torch.from_numpy(sets).to(dev), bmask)
    assert np.array_equal(both.cpu().numpy(), _pack(exact))
    codes = g.integers(-128, 128, (n, 64), dtype=np.int8)
    qc = g.integers(-128, 128, (7, 64), dtype=np.int8)
    ids, sc = torch.ops.retrieve_amd.int8_scan_topk(torch.from_numpy(qc).to(dev),
                                               torch.from_numpy(codes).to(dev), 20, both)
    want_ids, want_sc = osc.int8_topk(qc, codes, 20, exact)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(sc.cpu().numpy(), want_sc)


def test_malformed_plan_matches_nothing(dev):
    g = rng(85)
    attrs = _attrs(g, 3000, 2, 1, 5, 0.0)
    words, offs = _build(dev, attrs, 3, bits=64)
    blob, count, max_stack = st.prepare_plans(["0:1 AND 1:2", "0:3"], 7, dev)
    bad = blob.clone()
    bad[1] = 10**9  # ops end past the data
    m = torch.ops.st.bloom_index_search_batch_prepared(words, offs, bad, count, max_stack, 3, 7)
    assert (m[0] == 0).all()
    good = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, max_stack,
                                                          3, 7)
    assert torch.equal(m[1], good[1])


def test_errors(dev):
    fid = torch.zeros(1, dtype=torch.int32, device=dev)
    fo = torch.zeros(3, dtype=torch.int64, device=dev)
    fv = torch.zeros(0, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 2, 3)  # bits < k
    with pytest.raises(RuntimeError):
        torch.ops.st.bloom_index_build(fid, fo, fv, 1.0, 3)
    with pytest.raises(ValueError):
        torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 64, 11)


def _nested(depth: int) -> str:
    """AND / OR alternating ``depth`` levels deep, each level with a term beside the subtree."""
    e = "0:1"
    for d in range(depth):
        e = f"({e} {'AND' if d % 2 else 'OR'} {d % 4}:{d % 5})"
    return e


@pytest.mark.parametrize("bits,k,hash_k,n", [(64, 3, 7, 4500), (64, 5, 7, 1000),
                                             (128, 3, 7, 1000), (64, 2, 2, 70)])
def test_search_paths(dev, bits, k, hash_k, n):
    """Programs over LDS-staged bundles (64 bits, k <= 4) and the stack evaluation (deep plans,
    k > 4, wider bundles) in one batch; many plans over few bundles split across workgroups."""
    g = rng(86 + bits + k + n)
    attrs = _attrs(g, n, 4, 1, 6, 0.2)
    words, offs = _build(dev, attrs, k, bits=bits)
    ow, oo = of.bloom_build(attrs, k, bits_per_doc=bits)
    exprs = [_random_expr(g) for _ in range(16)]
    exprs += [_nested(d) for d in (3, 4, 5, 6, 9)]
    exprs += ["NOT (NOT (NOT (NOT (NOT (0:1 OR 1:1)))))", "0:0 OR 0:1 OR 0:2 OR 0:3 OR 0:4"]
    got = _unpack(_search(dev, words, offs, exprs, k, hash_k), n)
    for e, row in zip(exprs, got):
        want = of.bloom_expression_mask(ow, oo, n, e, k, hash_k)
        assert np.array_equal(row, want), e


@pytest.mark.parametrize("plans", [16, 300])
def test_search_transposed_words(dev, plans):
    """``st.bloom_search_t``: the same words as the prepared search (stack-evaluated plans
    included), stored transposed with the plan count rounded up to 256 as the row stride."""
    g = rng(93 + plans)
    n = 5000
    attrs = _attrs(g, n, 4, 1, 6, 0.2)
    words, offs = _build(dev, attrs, 3, bits=64)
    exprs = [_random_expr(g) for _ in range(plans - 3)]
    exprs += [_nested(9), "NOT (0:1 OR 1:1)", "0:0 OR 0:1 OR 0:2"]
    blob, count, max_stack = st.prepare_plans(exprs, 7, dev)
    want = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, max_stack, 3, 7)
    got = st.bloom_search_t(words, offs, blob, count, max_stack, 3, 7)
    assert got.shape == want.shape and got.stride() == (1, -(-plans // 256) * 256)
    assert torch.equal(got, want)


def test_long_plans(dev):
    """Value sets of hundreds of terms (plans of 500 - 2000 ops, the program's capacity) and one
    past it (the stack evaluation), against the oracle."""
    g = rng(91)
    n = 3000
    attrs = _attrs(g, n, 3, 1, 400, 0.1)
    words, offs = _build(dev, attrs, 3, bits=64)
    ow, oo = of.bloom_build(attrs, 3, bits_per_doc=64)

    def ors(c, vals):
        return "(" + " OR ".join(f"{c}:{v}" for v in vals) + ")"

    exprs = [ors(0, range(300)),
             ors(0, range(0, 400, 2)) + " AND " + ors(1, range(250)),
             ors(0, range(200)) + " AND " + ors(1, range(200)) + " AND " + ors(2, range(300)),
             "NOT " + ors(2, range(350)),
             ors(0, range(400)) + " AND " + ors(1, range(400)) + " AND " + ors(2, range(400))]
    got = _unpack(_search(dev, words, offs, exprs, 3, 7), n)
    for e, row in zip(exprs, got):
        want = of.bloom_expression_mask(ow, oo, n, e, 3, 7)
        assert np.array_equal(row, want), e[:60]


@pytest.mark.parametrize("mode", ["fixed", "upstream"])
@pytest.mark.parametrize("n_sets", [25, 150])
def test_compiled_plans_and_clauses(dev, mode, n_sets):
    """The prepared search compiles a blob's programs once. With 25 value sets behind 60 plans
    (clauses repeat across plans) the ANDs of clauses read the batch's distinct clauses,
    evaluated once per column, while the plans of other shapes (nested, NOT of an AND, a
    random mix) run their programs in the same search; with 150 value sets there are more
    distinct clauses than the table holds and every plan runs its program. Either way the words
    equal the search that compiles in its workspace (uniform widths; mixed widths, whose
    unstaged bundles evaluate the clauses' terms from their hashes) and the oracle; a blob
    changed in place is compiled again."""
    g = rng(97 + n_sets + (mode == "upstream"))
    n = 9000
    attrs = _attrs(g, n, 3, 1, 200, 0.1)
    if mode == "fixed":
        words, offs = _build(dev, attrs, 3, bits=64)
        ow, oo = of.bloom_build(attrs, 3, bits_per_doc=64)
    else:
        attrs[5000:, 1:, :] = -1  # bundles of different widths
        words, offs = _build(dev, attrs, 3, mult=3.0)
        ow, oo = of.bloom_build(attrs, 3, b_multiplier=3.0)
    sets = [(int(g.integers(0, 3)), np.sort(g.choice(200, int(g.integers(1, 40)), replace=False)))
            for _ in range(n_sets)]

    def exprs_of(shift):
        out = []
        for r in range(max(60, n_sets)):
            c1, v1 = sets[r % n_sets]
            c2, v2 = sets[(7 * r + 3) % n_sets]
            e = "(" + " OR ".join(f"{c1}:{(v + shift) % 200}" for v in v1) + ")"
            if r % 3:
                e += " AND " + ("NOT " if r % 5 == 0 else "") + \
                    "(" + " OR ".join(f"{c2}:{(v + shift) % 200}" for v in v2) + ")"
            out.append(e)
        return out + [_nested(5), "NOT (0:1 AND 1:2)", "", _random_expr(g), _random_expr(g)]

    exprs = exprs_of(0)
    blob, count, depth = st.prepare_plans(exprs, 7, dev)
    print(f"compiled plans {mode}, {n_sets} value sets: {count} plans", flush=True)
    got = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, depth, 3, 7)
    hits = [v for key, v in st._COMPILED.items() if key[0] == st._tkey(blob)]
    assert len(hits) == 1
    if n_sets == 25:
        assert 0 < hits[0][2] <= st.MAX_CLAUSES  # the clause plans read the table
    else:
        assert hits[0][2] == 0  # more distinct clauses than the table holds
    data = blob[8 * count:]
    ref = st._bloom_search(words, offs, blob, data, data.numel() * 8, count, depth, 3, 7, False)
    assert torch.equal(got, ref)
    assert torch.equal(st.bloom_search_t(words, offs, blob, count, depth, 3, 7), got)
    rows = _unpack(got.cpu().numpy(), n)
    for e, row in list(zip(exprs, rows))[::7] + list(zip(exprs, rows))[-5:]:
        assert np.array_equal(row, of.bloom_expression_mask(ow, oo, n, e, 3, 7)), e[:40]
    # the same blob rewritten in place (same sizes, other values): compiled again
    exprs2 = exprs_of(7)
    exprs2[-2:] = exprs[-2:]
    blob2, count2, depth2 = st.prepare_plans(exprs2, 7, dev)
    assert blob2.shape == blob.shape and (count2, depth2) == (count, depth)
    blob.copy_(blob2)
    got2 = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, depth, 3, 7)
    rows2 = _unpack(got2.cpu().numpy(), n)
    for e, row in list(zip(exprs2, rows2))[::7]:
        assert np.array_equal(row, of.bloom_expression_mask(ow, oo, n, e, 3, 7)), e[:40]


@pytest.mark.parametrize("n,n_plans", [(9000, 100), (8_500_000, 150)])
def test_clause_plans_transposed_words(dev, n, n_plans):
    """Every plan a clause plan: the transposed words are gathered 64 plans at a time in the
    column kernel's LDS and leave in contiguous runs. 8.5M documents (one workgroup takes every
    plan: two full chunks and a partial one) and 9000 (plans split over workgroups, a partial
    chunk each); the words equal the prepared search of the same plans without the clause
    table (row-major, programs), and the oracle on the small table."""
    import bench

    g = rng(99 + n_plans)
    print(f"clause plans, transposed words: N={n} plans={n_plans}", flush=True)
    if n > 100_000:
        attrs = bench.attr_table(n, 4321, dev).long()
    else:
        attrs = torch.from_numpy(_attrs(g, n, 8, 1, 40, 0.0)).to(dev)
    fid, fo, fv = st.attrs_to_features(attrs)
    words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 64, 3)
    del fid, fo, fv
    pool = [(int(g.integers(0, 8)), np.sort(g.choice(16, int(g.integers(1, 6)), replace=False)))
            for _ in range(12)]
    exprs = []
    for r in range(n_plans):
        parts = [pool[(r * j + 5) % 12] for j in range(1, 2 + r % 3)]
        exprs.append(" AND ".join("(" + " OR ".join(f"{c}:{v}" for v in vs) + ")"
                                  for c, vs in parts))
    blob, count, depth = st.prepare_plans(exprs, 7, dev)
    got = st.bloom_search_t(words, offs, blob, count, depth, 3, 7)
    hits = [v for key, v in st._COMPILED.items() if key[0] == st._tkey(blob)]
    assert len(hits) == 1 and hits[0][2] > 0 and hits[0][1][2]  # every plan a clause plan
    data = blob[8 * count:]
    ref = st._bloom_search(words, offs, blob, data, data.numel() * 8, count, depth, 3, 7, False)
    assert torch.equal(got, ref)
    if n < 100_000:
        ow, oo = of.bloom_build(attrs.cpu().numpy(), 3, bits_per_doc=64)
        rows = _unpack(got.contiguous().cpu().numpy(), n)
        for e, row in list(zip(exprs, rows))[::9]:
            assert np.array_equal(row, of.bloom_expression_mask(ow, oo, n, e, 3, 7)), e


def test_stack_limit_matches_nothing(dev):
    """A plan that needs more stack than max_stack_size matches nothing; the others evaluate."""
    g = rng(90)
    attrs = _attrs(g, 3000, 2, 1, 5, 0.0)
    words, offs = _build(dev, attrs, 3, bits=64)
    blob, count, _ = st.prepare_plans(["0:1 OR 1:2 OR 0:3", "0:1", "NOT 1:2"], 7, dev)
    m = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, 2, 3, 7)
    assert (m[0] == 0).all()
    full = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, 3, 3, 7)
    assert (full[0] != 0).any()
    assert torch.equal(m[1:], full[1:])
