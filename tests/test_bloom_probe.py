"""The Bloom pre-filter probed per candidate inside the scan: the index's row view
(``retrieve_amd::bloom_doc_bits``) against the oracle, every compiled plan evaluated on it
(``rt_bloom_probe_search``) against the column search's words, and
``retrieve_amd::scan_topk_bloom_clauses`` bit for bit against the unfused pair (the prepared
search's words, then ``int8_scan_topk_clauses`` / ``dense_scan_topk_clauses``) and against the
oracle. The plans are either the Bloom form of the query's value sets (the benchmark's filter) or
random ANDs of value-set clauses unrelated to them (NOT, EMPTY), so the probe's Bloom verdict
itself, not only the clauses behind it, decides the results. The cases the probe does not take
(blocked batches, fp32, plans of another form, bundles of mixed widths) fall back to the unfused
pair and must give its results too."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import retrieve_amd.st as st
from oracle import filters as of
from oracle import scan as osc
from retrieve_amd import _native as nat
from retrieve_amd import bloom as bl
from tests.conftest import rng
from tests.test_bloom import _build, _nested
from tests.test_scan_clauses import _sets

pytestmark = pytest.mark.gpu

BLOOM_K, HASH_K = 3, 7


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _unpack(words: np.ndarray, n: int) -> np.ndarray:
    be = np.ascontiguousarray(words).view(np.uint64).astype(">u8")
    return np.unpackbits(be.view(np.uint8), axis=1)[:, :n].astype(bool)


@pytest.mark.parametrize("n,bits", [(1, 64), (5000, 64), (4500, 40), (70_000, 64)])
def test_doc_bits_match_oracle(dev, n, bits):
    g = rng(n + bits)
    attrs = g.integers(-1, 9, (n, 4, 2))
    words, offs = _build(dev, attrs, BLOOM_K, bits=bits)
    got = torch.ops.retrieve_amd.bloom_doc_bits(words, offs, n)
    torch.cuda.synchronize()
    want = of.bloom_doc_bits(words.cpu().numpy(), offs.cpu().numpy(), n)
    assert np.array_equal(got.cpu().numpy(), want)


def test_doc_bits_rejects_mixed_widths(dev):
    g = rng(82)
    attrs = g.integers(0, 40, (6500, 3, 2))
    attrs[g.random(attrs.shape) < 0.5] = -1
    attrs[4096:6144] = -1  # an empty bundle: width 0
    words, offs = _build(dev, attrs, BLOOM_K, mult=2.5)
    assert len(set(np.diff(offs.cpu().numpy()).tolist())) > 1
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.bloom_doc_bits(words, offs, 6500)


def _plans(dev, exprs):
    blob, count, max_stack = st.prepare_plans(exprs, HASH_K, dev)
    return blob, count, max_stack


def _clause_expr(g, c=4, vocab=6, max_clauses=3, max_values=4):
    """A random AND of value-set clauses, some negated ("" is EMPTY): the form the probe takes
    (unrelated to any query's exact clauses)."""
    parts = []
    for _ in range(int(g.integers(0, max_clauses + 1))):
        attr = int(g.integers(0, c))
        vals = g.choice(np.arange(-1, vocab + 2), int(g.integers(1, max_values + 1)),
                        replace=False)
        clause = " OR ".join(f"{attr}:{int(v)}" for v in vals)
        clause = f"({clause})" if len(vals) > 1 else clause
        parts.append(("NOT " + clause) if g.random() < 0.25 else clause)
    return " AND ".join(parts)


def _tables(dev, words, offs, exprs):
    blob, count, max_stack = _plans(dev, exprs)
    depth = max(1, min(max_stack, st.MAX_STACK))
    return st._probe_tables(offs, blob, count, depth, BLOOM_K, HASH_K), blob, count, max_stack


def test_probe_search_equals_column_search(dev):
    """Every plan through the per-document probe (its clause table) equals the column search's
    word bits for the documents below N: random ANDs of value-set clauses with NOTs, EMPTY, a
    term, a NOT term, and plans of 64 and 131 terms (one and three chunks); a batch holding a
    plan of another form (or of 65 clauses) has no tables."""
    g = rng(97)
    n = 4500
    attrs = g.integers(-1, 6, (n, 4, 1))
    words, offs = _build(dev, attrs, BLOOM_K, bits=64)
    exprs = [_clause_expr(g) for _ in range(60)]
    wide = " AND ".join("(" + " OR ".join(f"{a}:{v}" for v in range(16)) + ")" for a in range(4))
    long = " AND ".join("(" + " OR ".join(f"{a}:{v}" for v in range(-8, 35)) + ")"
                        for a in (0, 2, 3)) + " AND NOT (1:2 OR 1:4)"
    exprs += ["", "1:3", "NOT 2:2", "NOT (0:1 OR 0:2) AND 3:4", wide, long]
    tables, blob, count, max_stack = _tables(dev, words, offs, exprs)
    assert tables is not False
    want = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, max_stack,
                                                          BLOOM_K, HASH_K)
    bits = torch.ops.retrieve_amd.bloom_doc_bits(words, offs, n)
    out = torch.empty((count, -(-n // 64)), dtype=torch.int64, device=dev)
    lib = nat.lib()
    nat.check(lib.rt_bloom_probe_search(nat.ptr(bits), n, nat.ptr(tables), count, nat.ptr(out),
                                        nat.stream(dev)))
    torch.cuda.synchronize()
    got, ref = _unpack(out.cpu().numpy(), n), _unpack(want.cpu().numpy(), n)
    for r, e in enumerate(exprs):
        assert np.array_equal(got[r], ref[r]), e
    assert 0 < ref.sum() < ref.size
    many = " AND ".join(f"({a}:{v} OR {a}:{v + 1})" for a in range(4) for v in range(17))
    for other in (_nested(4), many):
        assert _tables(dev, words, offs, exprs[:3] + [other])[0] is False, other


def _case(dev, g, b, n, d, dtype, plans_from_sets=True, bits=64, vocab=6, c=4):
    print(f"probe scan B={b} N={n} D={d} {dtype} sets={plans_from_sets} bits={bits}", flush=True)
    attrs = g.integers(0, vocab, (n, c, 1))
    attrs[g.random(attrs.shape) < 0.1] = -1
    sets = _sets(g, b, c, 3, vocab, 0.6)
    exprs = bl.sets_to_expressions(sets) if plans_from_sets else \
        [_clause_expr(g) for _ in range(b)]
    words, offs = _build(dev, attrs, BLOOM_K, bits=bits)
    blob, count, max_stack = _plans(dev, exprs)
    if dtype == torch.int8:
        q = _t(dev, g.integers(-128, 128, (b, d), dtype=np.int8))
        items = _t(dev, g.integers(-128, 128, (n, d), dtype=np.int8))
    else:
        q = _t(dev, g.standard_normal((b, d)).astype(np.float32)).to(dtype)
        items = _t(dev, g.standard_normal((n, d)).astype(np.float32)).to(dtype)
    return dict(q=q, items=items, attrs=_t(dev, attrs.astype(np.int16)),
                rev=torch.zeros(c, dtype=torch.bool, device=dev), sets=_t(dev, sets),
                words=words, offs=offs, blob=blob, count=count, max_stack=max_stack,
                attrs_np=attrs, sets_np=sets)


def _fused(x, k, doc_bits):
    return torch.ops.retrieve_amd.scan_topk_bloom_clauses(
        x["q"], x["items"], k, x["attrs"], x["rev"], x["sets"], doc_bits, x["words"], x["offs"],
        x["blob"], x["count"], x["max_stack"], BLOOM_K, HASH_K)


def _unfused(x, k):
    mask = torch.ops.st.bloom_index_search_batch_prepared(x["words"], x["offs"], x["blob"],
                                                          x["count"], x["max_stack"], BLOOM_K,
                                                          HASH_K)
    op = torch.ops.retrieve_amd.int8_scan_topk_clauses if x["q"].dtype == torch.int8 else \
        torch.ops.retrieve_amd.dense_scan_topk_clauses
    return op(x["q"], x["items"], k, x["attrs"], x["rev"], x["sets"], mask), mask


@pytest.mark.parametrize("b,n,d,k,from_sets", [
    (1, 40_000, 128, 10, True), (16, 60_000, 512, 100, True), (31, 50_000, 128, 64, False),
    (16, 2_200_000, 128, 100, True), (7, 2_200_000, 64, 1000, False)])
def test_int8_probe_scan(dev, b, n, d, k, from_sets):
    """Bit for bit with the unfused pair, and with the oracle's top-k over Bloom AND exact
    (Bloom from the unfused search's words, whose parity the search tests hold) where N is
    small. 2.2M rows take the seeded path, whose bound comes from the clauses alone: with plans
    unrelated to the clauses (from_sets False) a query can end short behind it, and the fallback
    pass must restore the exact results."""
    g = rng(b * 13 + n + d + k)
    x = _case(dev, g, b, n, d, torch.int8, from_sets)
    depth = max(1, min(x["max_stack"], st.MAX_STACK))
    assert st._probe_tables(x["offs"], x["blob"], x["count"], depth, BLOOM_K, HASH_K) is not False
    doc_bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], n)
    ids, sc = _fused(x, k, doc_bits)
    (want_ids, want_sc), mask = _unfused(x, k)
    torch.cuda.synchronize()
    assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)
    if n <= 100_000:
        valid = of.clause_match_sets(x["attrs_np"], x["sets_np"], np.zeros(4, bool))
        valid &= _unpack(mask.cpu().numpy(), n)
        q, items = x["q"].cpu().numpy(), x["items"].cpu().numpy()
        oi, os_ = osc.int8_topk(q, items, k, valid)
        assert np.array_equal(ids.cpu().numpy(), oi) and np.array_equal(sc.cpu().numpy(), os_)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_probe_scan(dev, dtype):
    g = rng(311 if dtype == torch.bfloat16 else 312)
    x = _case(dev, g, 16, 30_000, 64, dtype, False)
    doc_bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], 30_000)
    ids, sc = _fused(x, 50, doc_bits)
    (want_ids, want_sc), _ = _unfused(x, 50)
    torch.cuda.synchronize()
    assert torch.equal(ids, want_ids) and torch.equal(sc, want_sc)


def test_probe_scan_fallbacks(dev):
    """The unfused pair's results where the probe does not apply: a blocked batch, fp32, a plan
    of another form in the batch (here also one of the stack evaluation), and an index of mixed
    bundle widths (whose row bits cannot be built: any [N] tensor is accepted and unused)."""
    g = rng(401)
    x = _case(dev, g, 64, 20_000, 128, torch.int8, True)
    bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], 20_000)
    got, (want, _) = _fused(x, 30, bits), _unfused(x, 30)
    assert all(torch.equal(a, b) for a, b in zip(got, want)), "blocked batch"

    x = _case(dev, g, 8, 20_000, 64, torch.float32, True)
    bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], 20_000)
    got, (want, _) = _fused(x, 30, bits), _unfused(x, 30)
    assert all(torch.equal(a, b) for a, b in zip(got, want)), "fp32"

    x = _case(dev, g, 8, 20_000, 128, torch.int8, False)
    exprs = [_clause_expr(g) for _ in range(7)] + [_nested(9)]
    x["blob"], x["count"], x["max_stack"] = _plans(dev, exprs)
    bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], 20_000)
    got, (want, _) = _fused(x, 30, bits), _unfused(x, 30)
    assert all(torch.equal(a, b) for a, b in zip(got, want)), "a stack plan"

    n = 6500
    attrs = g.integers(0, 6, (n, 4, 1))
    attrs[4096:6144] = -1  # bundles of different widths
    words, offs = _build(dev, attrs, BLOOM_K, mult=2.5)
    x = _case(dev, g, 8, n, 128, torch.int8, True)
    x.update(words=words, offs=offs, attrs=_t(dev, attrs.astype(np.int16)))
    zeros = torch.zeros(n, dtype=torch.int64, device=dev)
    got, (want, _) = _fused(x, 30, zeros), _unfused(x, 30)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got, want)), "mixed widths"


def test_probe_scan_errors(dev):
    g = rng(402)
    x = _case(dev, g, 4, 5000, 64, torch.int8, True)
    bits = torch.ops.retrieve_amd.bloom_doc_bits(x["words"], x["offs"], 5000)
    with pytest.raises(ValueError):
        _fused(x, 10, bits[:-1])
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.scan_topk_bloom_clauses(
            x["q"][:3], x["items"], 10, x["attrs"], x["rev"], x["sets"][:3], bits, x["words"],
            x["offs"], x["blob"], x["count"], x["max_stack"], BLOOM_K, HASH_K)
