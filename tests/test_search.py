"""``torch.ops.st.search`` / ``st.probe_prep`` on the GPU against the CPU restatement
(``oracle.silvertorch``): quantization bit for bit, one-list full scans and IVF probes (int32
and fp16 key paths), ties to the lower slot, ``sort_perm`` ids and dequantized scores, and the
filters (full-N mask, Bloom plans with the exact recheck, exact clauses in the slot layout)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import retrieve_amd.st as st
from oracle import filters as of
from oracle import quantize as oq
from oracle import silvertorch as ost
from retrieve_amd import bloom as bl
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _ivf(g, n, d, n_lists):
    """Items sorted by cluster: offsets / sizes of n_lists contiguous clusters, a random
    sort_perm (sorted position -> original id)."""
    cuts = np.sort(g.choice(np.arange(1, n), n_lists - 1, replace=False))
    offsets = np.concatenate([[0], cuts]).astype(np.int64)
    sizes = np.diff(np.concatenate([offsets, [n]])).astype(np.int64)
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    perm = g.permutation(n).astype(np.int64)
    return items, offsets, sizes, perm


def _run(dev, q, probes, offsets, sizes, items, perm, gs, k, width, divisor=-1, **kw):
    print(f"search B={q.shape[0]} N={items.shape[0]} D={q.shape[1]} n_lists={len(offsets)} "
          f"n_probe={probes.shape[1]} k={k} width={width} divisor={divisor} "
          f"filters={sorted(kw)}", flush=True)
    ids, sc = torch.ops.st.search(
        _t(dev, q), _t(dev, probes), _t(dev, offsets), _t(dev, sizes), _t(dev, items),
        _t(dev, perm), _t(dev, np.array([gs], np.float32)), k, width, divisor, **kw)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), sc.cpu().numpy()


def test_probe_prep(dev):
    g = rng(101)
    q = (g.standard_normal((9, 200)) * np.exp(g.standard_normal((9, 1)))).astype(np.float32)
    q[3] = 0.0  # abs_max clamps to 1e-8
    q[4, :7] = [127 * 0.01 / 2.54, -2.54, 0.5, 1.5, -0.5, 2.5, 0.0]  # exact .5 quotients
    sizes = g.integers(0, 100, 12).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    probes = g.integers(0, 12, (9, 5)).astype(np.int64)
    out = torch.ops.st.probe_prep(_t(dev, q), _t(dev, probes), _t(dev, offsets), _t(dev, sizes))
    codes, scales = oq.quantize_int8(q)
    assert np.array_equal(out[0].cpu().numpy(), codes)
    assert np.array_equal(out[1].cpu().numpy(), scales)
    lens = sizes[probes]
    assert np.array_equal(out[3].cpu().numpy(), lens)
    assert np.array_equal(out[4].cpu().numpy(), offsets[probes])
    assert np.array_equal(out[6].cpu().numpy(), np.cumsum((lens // 32) * 32, axis=1))
    assert np.array_equal(out[7].cpu().numpy(), np.cumsum((lens % 32).reshape(-1)))
    assert np.array_equal(out[8].cpu().numpy(), np.cumsum((lens // 32).reshape(-1)))


@pytest.mark.parametrize("divisor", [-1, 64])
def test_one_list_full_scan(dev, divisor):
    g = rng(102)
    n, d, b, k = 60_000, 128, 6, 100
    items, _, _, perm = _ivf(g, n, d, 2)
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.zeros((b, 1), np.int64)
    ids, sc = _run(dev, q, probes, [0], [n], items, perm, 0.25, k, n, divisor)
    want_ids, want_sc = ost.search(q, probes, [0], [n], items, perm, [0.25], k, n, divisor)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(sc, want_sc)


@pytest.mark.parametrize("divisor", [-1, 128])
@pytest.mark.parametrize("n_lists,n_probe,width_frac", [(50, 8, 1.0), (7, 7, 0.5), (300, 40, 1.0)])
def test_ivf_probes(dev, divisor, n_lists, n_probe, width_frac):
    g = rng(103 + n_lists + n_probe)
    n, d, b, k = 40_000, 256, 5, 100
    items, offsets, sizes, perm = _ivf(g, n, d, n_lists)
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.stack([g.permutation(n_lists)[:n_probe] for _ in range(b)]).astype(np.int64)
    probes[0, 1] = 10**6  # an invalid cluster id probes nothing
    width = int(max(sizes[probes[r][probes[r] < n_lists]].sum() for r in range(b)) * width_frac)
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 1.5, k, width, divisor)
    want_ids, want_sc = ost.search(q, probes, offsets, sizes, items, perm, [1.5], k, width,
                                   divisor)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(sc, want_sc)


@pytest.mark.parametrize("divisor", [-1, 96])
def test_k_above_1024(dev, divisor):
    """Above the radix select's 1024 the search selects from the raw scorer's buffer (the
    reference's ``at::topk`` path, fork_search_cuda.cu:843-915): IVF probes with a full-N mask,
    and the one-list table."""
    g = rng(140)
    n, d, b, k = 30_000, 128, 4, 1500
    items, offsets, sizes, perm = _ivf(g, n, d, 40)
    items = (items // 32).astype(np.int8)  # narrow codes: tied keys across slots
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.stack([g.permutation(40)[:12] for _ in range(b)]).astype(np.int64)
    probes[1, 0] = 10**6
    width = int(max(sizes[probes[r][probes[r] < 40]].sum() for r in range(b)))
    valid = g.random((b, n)) < 0.7
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 0.5, k, width, divisor,
                   filtering_bit_mask=_t(dev, _pack(valid)))
    want_ids, want_sc = ost.search(q, probes, offsets, sizes, items, perm, [0.5], k, width,
                                   divisor, valid)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(sc, want_sc)
    one = np.array([0], np.int64), np.array([n], np.int64)
    probes1 = np.zeros((b, 1), np.int64)
    ids, sc = _run(dev, q, probes1, *one, items, perm, 0.5, 2000, n, divisor)
    want_ids, want_sc = ost.search(q, probes1, *one, items, perm, [0.5], 2000, n, divisor)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(sc, want_sc)


def test_ties_go_to_the_lower_slot(dev):
    g = rng(104)
    n, d = 5000, 64
    items, offsets, sizes, perm = _ivf(g, n, d, 10)
    items[:] = items[0]  # every dot equal
    q = g.standard_normal((3, d)).astype(np.float32)
    probes = np.array([[9, 2, 5], [0, 1, 2], [4, 4, 3]], np.int64)  # a repeated probe too
    ids, _ = _run(dev, q, probes, offsets, sizes, items, perm, 1.0, 50, n)
    want_ids, _ = ost.search(q, probes, offsets, sizes, items, perm, [1.0], 50, n)
    assert np.array_equal(ids, want_ids)


def test_slot_order_warps_then_remainders(dev):
    """The reference GPU scorer's slot order, written out by hand: clusters of 40, 50 and 7
    equal rows at positions 0, 40 and 90 probed [1, 0, 2] fill slots with cluster 1's full warp
    (40-71), cluster 0's (0-31), then the remainders in probe order: 72-89, 32-39, 90-96
    (``fork_search_cuda.cu:989-991``, ``:1051-1053``). Every dot ties, so the top-k is the
    lowest slots; under a mask a filtered-out doc keeps its slot."""
    d = 64
    items = np.full((97, d), 3, np.int8)
    perm = np.arange(97, dtype=np.int64) + 1000
    q = np.ones((2, d), np.float32)
    offs, sizes = np.array([0, 40, 90], np.int64), np.array([40, 50, 7], np.int64)
    probes = np.array([[1, 0, 2], [1, 0, 2]], np.int64)
    order = (list(range(40, 72)) + list(range(0, 32)) + list(range(72, 90)) + list(range(32, 40))
             + list(range(90, 97)))
    ids, _ = _run(dev, q, probes, offs, sizes, items, perm, 1.0, 97, 97)
    assert ids[0].tolist() == [1000 + p for p in order]
    ids, _ = _run(dev, q, probes, offs, sizes, items, perm, 1.0, 70, 97)
    assert ids[1].tolist() == [1000 + p for p in order[:70]]
    valid = np.ones((2, 97), bool)
    valid[:, 40:72:2] = False  # every other doc of cluster 1's warp
    ids, _ = _run(dev, q, probes, offs, sizes, items, perm, 1.0, 40, 97,
                  filtering_bit_mask=_t(dev, _pack(valid)))
    kept = [p for p in order if valid[0, p]]
    assert ids[0].tolist() == [1000 + p for p in kept[:40]]


@pytest.mark.parametrize("d", [192, 384, 1280])
def test_one_list_widths_without_a_full_scan_kernel(dev, d):
    """Row widths the full-scan kernels lack (the reference's DIM switch holds them,
    ``fused_kmean_ann_cuda.cu:1566-1577``) take the IVF kernel on one list, with the same
    results; a row probing a list that does not exist ends as pads."""
    g = rng(106 + d)
    n, b, k = 5000, 4, 50
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    perm = g.permutation(n).astype(np.int64)
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.zeros((b, 1), np.int64)
    probes[3, 0] = 1  # no list 1
    ids, sc = _run(dev, q, probes, [0], [n], items, perm, 0.5, k, n)
    want_ids, want_sc = ost.search(q, probes, [0], [n], items, perm, [0.5], k, n)
    assert np.array_equal(ids, want_ids) and np.array_equal(sc, want_sc)
    assert (ids[3] == -1).all()


def test_one_list_full_scan_invalid_probe(dev):
    """The full-scan path of one list: a row whose probe is not list 0 has no slot."""
    g = rng(107)
    n, d, b, k = 20_000, 128, 3, 30
    items = g.integers(-128, 128, (n, d), dtype=np.int8)
    perm = g.permutation(n).astype(np.int64)
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.array([[0], [5], [0]], np.int64)
    ids, sc = _run(dev, q, probes, [0], [n], items, perm, 2.0, k, n)
    want_ids, want_sc = ost.search(q, probes, [0], [n], items, perm, [2.0], k, n)
    assert np.array_equal(ids, want_ids) and np.array_equal(sc, want_sc)
    assert (ids[1] == -1).all() and np.isneginf(sc[1]).all()


def test_filters(dev):
    g = rng(105)
    n, d, b, k, c = 30_000, 64, 6, 50, 3
    items, offsets, sizes, perm = _ivf(g, n, d, 20)
    q = g.standard_normal((b, d)).astype(np.float32)
    probes = np.stack([g.permutation(20)[:6] for _ in range(b)]).astype(np.int64)
    width = n
    # full-N mask
    valid = g.random((b, n)) < 0.3
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 1.0, k, width,
                   filtering_bit_mask=_t(dev, _pack(valid)))
    want = ost.search(q, probes, offsets, sizes, items, perm, [1.0], k, width, valid=valid)
    assert np.array_equal(ids, want[0]) and np.array_equal(sc, want[1])
    # exact clauses in the slot layout (one value per doc and clause, -1 for none)
    attrs = g.integers(0, 8, (n, c, 1)).astype(np.int64)
    attrs[g.random((n, c, 1)) < 0.2] = -1
    qa = g.integers(0, 8, (b, c)).astype(np.int64)
    qa[g.random((b, c)) < 0.3] = -1
    rev = np.array([0, 1, 0], bool)
    exact = of.clause_match(attrs, rev, qa)
    slots = attrs[:, :, 0].T.astype(np.int32)  # [R = C, N]: one slot row per clause
    cs = np.arange(c + 1, dtype=np.int64)
    kw = dict(item_clause_attrs=_t(dev, slots), clause_slots=_t(dev, cs),
              clause_is_reverse=_t(dev, rev), query_clause_attrs=_t(dev, qa))
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 1.0, k, width, **kw)
    want = ost.search(q, probes, offsets, sizes, items, perm, [1.0], k, width, valid=exact)
    assert np.array_equal(ids, want[0]) and np.array_equal(sc, want[1])
    # Bloom plans + the exact recheck: bloom AND exact == exact
    fid, fo, fv = st.attrs_to_features(_t(dev, attrs))
    words, boffs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 64, 3)
    exprs = bl.queries_to_expressions(qa, rev)
    blob, count, max_stack = st.prepare_plans(exprs, 7, dev)
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 1.0, k, width,
                   bloom_index=words, bloom_bundle_b_offsets=boffs, plans=blob,
                   plan_count=count, max_stack_size=max_stack, bloom_k=3, hash_k=7, **kw)
    assert np.array_equal(ids, want[0]) and np.array_equal(sc, want[1])
    # Bloom plans alone, evaluated on the probed payloads' columns only: the Bloom mask's result
    # (false positives included), with the plans in another order than the rows
    wn, bn = words.cpu().numpy(), boffs.cpu().numpy()
    bloom = np.stack([of.bloom_expression_mask(wn, bn, n, e, 3, 7) for e in exprs])
    order = g.permutation(b)
    blob2, count2, stack2 = st.prepare_plans([exprs[i] for i in order], 7, dev)
    qpi = np.argsort(order).astype(np.int64)  # row r's plan: where exprs[r] went
    ids, sc = _run(dev, q, probes, offsets, sizes, items, perm, 1.0, k, width,
                   bloom_index=words, bloom_bundle_b_offsets=boffs, plans=blob2,
                   plan_count=count2, max_stack_size=stack2, bloom_k=3, hash_k=7,
                   query_plan_index=_t(dev, qpi))
    want = ost.search(q, probes, offsets, sizes, items, perm, [1.0], k, width, valid=bloom)
    assert np.array_equal(ids, want[0]) and np.array_equal(sc, want[1])


def test_errors(dev):
    q = torch.zeros((2, 64), device=dev)
    items = torch.zeros((10, 64), dtype=torch.int8, device=dev)
    probes = torch.zeros((2, 1), dtype=torch.int64, device=dev)
    o = torch.zeros(1, dtype=torch.int64, device=dev)
    s = torch.full((1,), 10, dtype=torch.int64, device=dev)
    perm = torch.arange(10, device=dev)
    gs = torch.ones(1, device=dev)
    with pytest.raises(RuntimeError):
        torch.ops.st.search(q, probes, o, s, items.float(), perm, gs, 5, 10)
    with pytest.raises(RuntimeError):
        torch.ops.st.search(q, probes, o, s, items, perm, gs, 5, 10,
                            filtering_bit_mask=torch.zeros((2, 1), dtype=torch.int64, device=dev),
                            query_clause_attrs=torch.zeros((2, 1), dtype=torch.int64, device=dev))
