"""The module layer (``retrieve_amd.modules``) on the GPU against oracle compositions: the exact
filter's mask / words / compaction / subset, the dense and candidate KNNs, the 1-bit KNNs (codes
bit for bit, Hamming top-k exact), LiNR V1-V3 with the filter, and SilverTorch's IVF search
(none / exact / bloom with recheck, int32 and fp16 keys) and candidate re-rank; plus the small
ops the modules add (``pack_mask``, ``pack_signs``, ``quantize_int8``, ``int8_rerank_topk``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import filters as of
from oracle import quantize as oq
from oracle import scan as osc
from oracle import silvertorch as ost
from tests.conftest import rng

pytestmark = pytest.mark.gpu


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(t):
    return t.detach().cpu().numpy()


def _attrs(g, n, c=4, a=2, card=6):
    attrs = g.integers(0, card, (n, c, a)).astype(np.int64)
    attrs[g.random((n, c, a)) < 0.3] = -1
    return attrs


def _queries(g, b, c=4, card=6):
    q = g.integers(0, card, (b, c)).astype(np.int64)
    q[g.random((b, c)) < 0.5] = -1
    return q


# --- small ops ---------------------------------------------------------------------------


def test_pack_mask_and_signs(dev):
    import retrieve_amd.hip  # noqa: F401

    g = rng(1)
    valid = g.random((5, 1000)) < 0.4
    words = _np(torch.ops.retrieve_amd.pack_mask(_t(dev, valid)))
    bits = ((words.view(np.uint64)[:, :, None] >> np.arange(63, -1, -1, dtype=np.uint64)) & 1)
    assert np.array_equal(bits.reshape(5, -1)[:, :1000].astype(bool), valid)
    assert (bits.reshape(5, -1)[:, 1000:] == 0).all()

    x = g.standard_normal((37, 256)).astype(np.float32)
    x[0, :4] = [0.0, -0.0, np.nan, 1e-45]
    x[1] = 0.0
    got = _np(torch.ops.retrieve_amd.pack_signs(_t(dev, x)))
    assert np.array_equal(got, oq.pack_signs(x))
    h = torch.from_numpy(x).to(dev).to(torch.float16)
    assert np.array_equal(_np(torch.ops.retrieve_amd.pack_signs(h)),
                          oq.pack_signs(h.float().cpu().numpy()))


def test_quantize_int8_op(dev):
    import retrieve_amd.hip  # noqa: F401

    g = rng(2)
    x = (g.standard_normal((50, 96)) * np.exp(2 * g.standard_normal((50, 1)))).astype(np.float32)
    x[3] = 0.0
    codes, scales = torch.ops.retrieve_amd.quantize_int8(_t(dev, x))
    want_c, want_s = oq.quantize_int8(x, divide=True)
    assert np.array_equal(_np(codes), want_c)
    assert np.array_equal(_np(scales), want_s)


@pytest.mark.parametrize("n,d,offset", [(5000, 96, 0), (333, 7, 1), (0, 16, 0)])
def test_quantize_int8_global_op(dev, n, d, offset):
    """The HIP global quantizer (16-byte and scalar loads: a table offset by one float) against
    the oracle, with and without a row permutation."""
    import retrieve_amd.hip  # noqa: F401
    from retrieve_amd import modules as mods

    g = rng(5)
    flat = (g.standard_normal(n * d + offset) * 2).astype(np.float32)
    if n:
        flat[offset + (n * d) // 2] = 9.5  # a positive extreme
        flat[offset + 1 :: 97] = np.round(flat[offset + 1 :: 97] * 4) / 4  # quarter values
    xt = _t(dev, flat)[offset:].view(n, d)
    x = flat[offset:].reshape(n, d)
    perm = g.permutation(n)
    for rows in (None, perm):
        codes, abs_max = torch.ops.retrieve_amd.quantize_int8_global(
            xt, None if rows is None else _t(dev, rows))
        want_c, want_m = oq.quantize_int8_global(x, rows)
        assert np.array_equal(_np(codes), want_c)
        assert _np(abs_max)[0] == want_m
    if n:
        codes, scale = mods.quantize_int8_global(xt, rows=_t(dev, perm))
        assert np.array_equal(_np(codes), oq.quantize_int8_global(x, perm)[0])
        assert scale == float(np.float32(oq.quantize_int8_global(x)[1] / np.float32(127)))


def _rerank_oracle(q_codes, q_scales, codes_sorted, inv_perm, gs, cand, k):
    b, p = cand.shape
    kk = min(k, p)
    ids = np.full((b, kk), -1, np.int64)
    sc = np.full((b, kk), -np.inf, np.float32)
    for r in range(b):
        c = cand[r][cand[r] >= 0]
        dots = codes_sorted[inv_perm[c]].astype(np.int64) @ q_codes[r].astype(np.int64)
        s = (dots.astype(np.float32) * q_scales[r]).astype(np.float32) * np.float32(gs)
        order = np.lexsort((c, -s.astype(np.float64)))[:kk]
        ids[r, : order.size] = c[order]
        sc[r, : order.size] = s[order]
    return ids, sc


def test_int8_rerank_topk(dev):
    import retrieve_amd.hip  # noqa: F401

    g = rng(3)
    n, d, b, p, k = 3000, 128, 6, 300, 40
    codes = g.integers(-128, 128, (n, d), dtype=np.int8)
    codes[7] = codes[11]  # equal rows: ties go to the lower original id
    perm = g.permutation(n).astype(np.int64)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(n)
    q = g.standard_normal((b, d)).astype(np.float32)
    q_codes, q_scales = oq.quantize_int8(q, divide=True)
    cand = g.integers(0, n, (b, p)).astype(np.int64)
    cand[:, :2] = [perm[7], perm[11]]
    cand[1, 100:] = -1
    cand[2, :] = -1
    gs = np.float32(0.0123)
    ids, sc = torch.ops.retrieve_amd.int8_rerank_topk(
        _t(dev, q_codes), _t(dev, q_scales), _t(dev, codes), _t(dev, inv),
        _t(dev, np.array([gs], np.float32)), _t(dev, cand), k)
    want_ids, want_sc = _rerank_oracle(q_codes, q_scales, codes, inv, gs, cand, k)
    assert np.array_equal(_np(ids), want_ids)
    assert np.array_equal(_np(sc), want_sc)


# --- LiNR --------------------------------------------------------------------------------


def _filter(dev, attrs, rev=None):
    from retrieve_amd.modules import ExactAttributeFilter

    f = ExactAttributeFilter()
    f.register_index(_t(dev, attrs), clause_is_reverse=None if rev is None else _t(dev, rev))
    return f


def test_exact_attribute_filter(dev):
    g = rng(10)
    n, b = 5000, 7
    attrs = _attrs(g, n)
    rev = np.array([False, True, False, False])
    q = _queries(g, b)
    f = _filter(dev, attrs, rev)
    qp = f.prepare_queries(_t(dev, q))
    want = of.clause_match(attrs, rev, q)
    assert np.array_equal(_np(f.evaluate_mask(qp)), want)
    assert np.array_equal(_np(f(qp)), want)
    assert np.array_equal(_np(f.evaluate_mask(qp, 100, 1333)), want[:, 100:1333])
    words = _np(f.mask_bits(qp))
    assert np.array_equal(words, _np(torch.ops.retrieve_amd.pack_mask(_t(dev, want))))
    ids, counts = f.evaluate_indices(qp)
    ids, counts = _np(ids), _np(counts)
    for r in range(b):
        nz = np.flatnonzero(want[r])
        assert counts[r] == nz.size and np.array_equal(ids[r, : nz.size], nz)
    cand = g.integers(0, n, (b, 50)).astype(np.int64)
    sub = _np(f.evaluate_subset(qp, _t(dev, cand)))
    assert np.array_equal(sub, np.take_along_axis(want, cand, axis=1))
    scores = g.standard_normal((b, n)).astype(np.float32)
    ms = _np(f.mask_scores(_t(dev, scores), qp))
    assert np.array_equal(ms, np.where(want, scores, -np.inf).astype(np.float32))


def _dense_check(ids, sc, q16, items16, k, valid=None, rtol=1e-3):
    """ids/scores against the float64 dot of the fp16 values: scores within ``rtol``; the ids
    the exact top-k except near-ties of the boundary."""
    exact = osc.dense_scores(q16, items16)
    want_ids, want_sc = osc.dense_topk(q16, items16, k, valid)
    for r in range(ids.shape[0]):
        m = int((want_ids[r] >= 0).sum())
        assert (ids[r, m:] == -1).all()
        got = ids[r, :m]
        assert len(set(got.tolist())) == m and (got >= 0).all()
        if valid is not None:
            assert valid[r, got].all()
        e = exact[r, got]
        assert (np.abs(sc[r, :m] - e) <= rtol * np.maximum(np.abs(e), 1e-3)).all()
        if m:
            band = 2 * rtol * max(abs(want_sc[r, m - 1]), 1e-3)
            assert (e >= want_sc[r, m - 1] - band).all()


def test_postfilter_knn(dev):
    from retrieve_amd.modules import PostfilterKNN

    g = rng(11)
    n, d, b, k = 6000, 128, 5, 50
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    m = PostfilterKNN(k)
    m.register_index(_t(dev, items))
    valid = g.random((b, n)) < 0.2
    valid[4] = False
    valid[4, :10] = True  # fewer than k pass: -1 / -inf tail
    q16 = q.astype(np.float16).astype(np.float32)
    i16 = items.astype(np.float16).astype(np.float32)
    ids, sc = m(_t(dev, q), _t(dev, valid))
    _dense_check(_np(ids), _np(sc), q16, i16, k, valid)
    assert np.isneginf(_np(sc)[4, 10:]).all()
    ids, sc = m(_t(dev, q))
    _dense_check(_np(ids), _np(sc), q16, i16, k)
    full = _np(m.score(_t(dev, q)))
    assert np.allclose(full, osc.dense_scores(q16, i16), rtol=1e-3, atol=1e-3)


def test_prefilter_knn(dev):
    from retrieve_amd.modules import PrefilterKNN

    g = rng(12)
    n, d, b, k = 4000, 64, 4, 20
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    m = PrefilterKNN(k)
    m.register_index(_t(dev, items))
    q16 = q.astype(np.float16).astype(np.float32)
    i16 = items.astype(np.float16).astype(np.float32)
    cand = np.stack([g.choice(n, 300, replace=False) for _ in range(b)]).astype(np.int64)
    counts = np.array([300, 5, 0, 150], np.int64)
    ids, sc = m(_t(dev, q), _t(dev, cand), _t(dev, counts))
    exact = osc.dense_scores(q16, i16)
    want_ids, _ = osc.candidate_topk(lambda r, c: exact[r, c], cand, counts, k, pad_to_k=True,
                                     empty_score=-np.inf)
    ids, sc = _np(ids), _np(sc)
    for r in range(b):
        mm = int((want_ids[r] >= 0).sum())
        assert (ids[r, mm:] == -1).all()
        assert set(ids[r, :mm].tolist()) <= set(cand[r, : counts[r]].tolist())
        assert np.allclose(sc[r, :mm], exact[r, ids[r, :mm]], rtol=1e-3, atol=1e-4)
    # P < k pads the candidates; no candidates: the full scan
    ids, _ = m(_t(dev, q), _t(dev, cand[:, :7]))
    assert (_np(ids)[:, 7:] == -1).all()
    ids, sc = m(_t(dev, q))
    _dense_check(_np(ids), _np(sc), q16, i16, k)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b", [3, 40])
def test_full_scan_knn(dev, dtype, b):
    """``FullScanKNN`` (``modules/knn.py:125-170``): the exact top k in the items' dtype; with a
    mask the same ids with the failing hits tombstoned to -1 and every score kept (post-filter:
    a failing hit is not replaced); candidates with -1 padding anywhere re-ranked to min(k, P)
    columns. Scores are rounded once from fp32, so they sit within that dtype's rounding of the
    float64 dot."""
    from retrieve_amd.modules import FullScanKNN

    print(f"FullScanKNN {dtype} B={b}", flush=True)
    g = rng(13 + b)
    n, d, k = 5000, 64, 30
    rtol = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 8e-3}[dtype]
    m = FullScanKNN(k)
    m.register_index(torch.from_numpy(g.standard_normal((n, d)).astype(np.float32)).to(dev)
                     .to(dtype))
    qt = torch.from_numpy(g.standard_normal((b, d)).astype(np.float32)).to(dev).to(dtype)
    qv, iv = _np(qt.float()), _np(m.item_embs.float())
    ids, sc = m(qt)
    assert ids.shape == (b, k) and sc.dtype == dtype
    _dense_check(_np(ids), _np(sc.float()), qv, iv, k, rtol=rtol)

    valid = g.random((b, n)) < 0.5
    ids_pf, sc_pf = m(qt, _t(dev, valid))
    assert torch.equal(sc_pf, sc)
    want = np.where(np.take_along_axis(valid, _np(ids), 1), _np(ids), -1)
    assert np.array_equal(_np(ids_pf), want)

    cand = np.stack([g.choice(n, 60, replace=False) for _ in range(b)]).astype(np.int64)
    cand[g.random(cand.shape) < 0.3] = -1
    cand[1] = -1  # a row with no candidates at all
    exact = osc.dense_scores(qv, iv)
    for p in (60, 7):
        ids_c, sc_c = m(qt, candidate_ids=_t(dev, cand[:, :p]))
        kk = min(k, p)
        assert ids_c.shape == (b, kk) and sc_c.dtype == dtype
        ids_c, sc_c = _np(ids_c), _np(sc_c.float())
        for r in range(b):
            c = cand[r, :p][cand[r, :p] >= 0]
            mm = min(kk, c.size)
            assert (ids_c[r, mm:] == -1).all() and np.isneginf(sc_c[r, mm:]).all()
            got = ids_c[r, :mm]
            assert len(set(got.tolist())) == mm and set(got.tolist()) <= set(c.tolist())
            e = exact[r, got]
            assert (np.abs(sc_c[r, :mm] - e) <= rtol * np.maximum(np.abs(e), 1e-3)).all()
            if mm:
                kth = np.sort(exact[r, c])[::-1][mm - 1]
                assert (e >= kth - 2 * rtol * max(abs(kth), 1e-3)).all()

    with pytest.raises(RuntimeError, match="same dtype"):
        m(qt.to(torch.float64))
    with pytest.raises(RuntimeError, match="out of range"):
        big = FullScanKNN(n + 1)
        big.register_index(m.item_embs)
        big(qt)


def _hamming_oracle(qbits, item_bits, k, valid=None):
    ids, sc = osc.hamming_topk(qbits, item_bits, k, valid)
    return ids, sc


def test_one_bit_knn(dev):
    from retrieve_amd.modules import OneBitKNN

    g = rng(13)
    n, d, b, k = 5000, 128, 6, 64
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    for k_bits in (0, 64):
        m = OneBitKNN(k, seed=3, k_bits=k_bits)
        m.register_index(_t(dev, items))
        # the codes are the packed signs of the module's own sketch
        from retrieve_amd.modules import _oporp_sketch

        sk = _np(_oporp_sketch(_t(dev, items), m.oporp_signs, m.oporp_perm, m.k_bits))
        assert np.array_equal(_np(m.item_bits), oq.pack_signs(sk))
        qbits = _np(m._project_query(_t(dev, q)))
        ids, sc = m(_t(dev, q))
        want_ids, want_sc = osc.hamming_topk(qbits, _np(m.item_bits), k)
        assert np.array_equal(_np(ids), want_ids)
        assert np.array_equal(_np(sc), want_sc.astype(np.float32))
        cand = np.stack([g.choice(n, 200, replace=False) for _ in range(b)]).astype(np.int64)
        counts = np.full(b, 200, np.int64)
        counts[0] = 30
        ids, sc = m(_t(dev, q), _t(dev, cand), _t(dev, counts))
        hs = osc.hamming_scores(qbits, _np(m.item_bits))
        want_ids, want_sc = osc.candidate_topk(lambda r, c: hs[r, c], cand, counts, k,
                                               pad_to_k=False, empty_score=-np.inf)
        assert np.array_equal(_np(ids), want_ids)


def test_simhash_knn(dev):
    from retrieve_amd.modules import SimHashKNN

    g = rng(14)
    n, d, b, k = 4000, 96, 5, 33
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    m = SimHashKNN(k, k_bits=192, seed=1)
    m.register_index(_t(dev, items))
    proj = _np(_t(dev, items) @ m.simhash_R.t())
    assert np.array_equal(_np(m.item_bits), oq.pack_signs(proj))
    qbits = _np(m._project_query(_t(dev, q)))
    ids, sc = m(_t(dev, q))
    want_ids, want_sc = osc.hamming_topk(qbits, _np(m.item_bits), k)
    assert np.array_equal(_np(ids), want_ids)
    assert np.array_equal(_np(sc), want_sc.astype(np.float32))


def test_linr_variants(dev):
    from retrieve_amd.modules import ExactAttributeFilter, LiNRBuilder, LiNRV1, LiNRV2, LiNRV3

    g = rng(15)
    n, d, b, k = 6000, 128, 5, 30
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    attrs = _attrs(g, n, card=3)
    qa = _queries(g, b, card=3)
    valid = of.clause_match(attrs, np.zeros(4, bool), qa)
    q16 = q.astype(np.float16).astype(np.float32)
    i16 = items.astype(np.float16).astype(np.float32)
    exact = osc.dense_scores(q16, i16)

    v1 = LiNRV1(k, filter=ExactAttributeFilter())
    v1.register_index(_t(dev, items), _t(dev, attrs))
    ids, sc = v1(_t(dev, q), v1.prepare_queries(_t(dev, qa)))
    _dense_check(_np(ids), _np(sc), q16, i16, k, valid)
    ids, sc = v1(_t(dev, q))
    _dense_check(_np(ids), _np(sc), q16, i16, k)

    v2 = LiNRV2(k, filter=ExactAttributeFilter())
    v2.register_index(_t(dev, items), _t(dev, attrs))
    ids, sc = v2(_t(dev, q), v2.prepare_queries(_t(dev, qa)))
    _dense_check(_np(ids), _np(sc), q16, i16, k, valid)

    v3 = LiNRV3(k, candidate_pool=400, seed=2, filter=ExactAttributeFilter())
    v3.register_index(_t(dev, items), _t(dev, attrs))
    qbits = _np(v3.stage1._project_query(_t(dev, q)))
    item_bits = _np(v3.stage1.item_bits)
    for prepared, vmask in ((None, None), (v3.prepare_queries(_t(dev, qa)), valid)):
        ids, sc = v3(_t(dev, q), prepared)
        short, _ = osc.hamming_topk(qbits, item_bits, 400, vmask)  # stage 1, exact
        counts = (short >= 0).sum(axis=1)
        want_ids, _ = osc.candidate_topk(lambda r, c: exact[r, c], short, counts, k,
                                         pad_to_k=True, empty_score=-np.inf)
        ids, sc = _np(ids), _np(sc)
        for r in range(b):
            mm = int((want_ids[r] >= 0).sum())
            assert (ids[r, mm:] == -1).all()
            assert set(ids[r, :mm].tolist()) <= set(short[r, : counts[r]].tolist())
            assert np.allclose(sc[r, :mm], exact[r, ids[r, :mm]], rtol=1e-3, atol=1e-4)
            kth = exact[r, want_ids[r, mm - 1]] if mm else 0.0
            assert (exact[r, ids[r, :mm]] >= kth - 2e-3 * max(abs(kth), 1e-3)).all()
    # the reference's default pool of 5000 (selected by counting Hamming scores): over these
    # 5000 items the shortlist holds every passing item, so the result is the exact filtered top-k
    v3d = LiNRV3(k, seed=2, filter=ExactAttributeFilter())
    v3d.register_index(_t(dev, items), _t(dev, attrs))
    ids, sc = v3d(_t(dev, q), v3d.prepare_queries(_t(dev, qa)))
    _dense_check(_np(ids), _np(sc), q16, i16, k, valid)
    with pytest.raises(ValueError):
        LiNRV3(k, candidate_pool=9000)
    built = (LiNRBuilder("v2", k=k).set_filter(ExactAttributeFilter(), _t(dev, attrs))
             .set_item_embeddings(_t(dev, items)).build())
    ids2, _ = built(_t(dev, q), built.prepare_queries(_t(dev, qa)))
    ids1, _ = v2(_t(dev, q), v2.prepare_queries(_t(dev, qa)))
    assert torch.equal(ids1, ids2)


# --- SilverTorch -------------------------------------------------------------------------


def _st_oracle(m, q, k, valid_sorted=None, divisor=-1):
    n_probe = m.n_probe
    qt = torch.from_numpy(q).to(m.item_codes.device)
    probes = _np(torch.topk(qt @ m.centroids.t(), n_probe, dim=1).indices) \
        if m.n_lists > 1 else np.zeros((q.shape[0], 1), np.int64)
    return ost.search(q, probes, _np(m.cluster_offsets), _np(m.cluster_sizes),
                      _np(m.item_codes), _np(m.sort_perm), _np(m.global_scale), k,
                      m._probe_width, divisor, valid_sorted)


@pytest.mark.parametrize("score_path", ["int32", "fp16"])
def test_silvertorch_ivf(dev, score_path):
    from retrieve_amd.modules import OfficialConfig, SilverTorch

    g = rng(16)
    n, d, b, k = 8000, 128, 6, 25
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    cfg = OfficialConfig(score_path=score_path)
    m = SilverTorch(k, n_lists=16, n_probe=4, seed=5, official=cfg)
    m.register_index(_t(dev, items))
    sizes = _np(m.cluster_sizes)
    assert sizes.sum() == n and m._probe_width == np.sort(sizes)[-4:].sum()
    ids, sc = m(_t(dev, q))
    div = cfg.divisor_for(d)
    want_ids, want_sc = _st_oracle(m, q, k, None, div)
    assert np.array_equal(_np(ids), want_ids)
    assert np.array_equal(_np(sc), want_sc)


def test_silvertorch_filters(dev):
    from retrieve_amd.modules import OfficialConfig, SilverTorch, SilverTorchBuilder

    g = rng(17)
    n, d, b, k = 6000, 64, 5, 20
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    attrs = _attrs(g, n, c=3, a=1, card=4)
    qa = _queries(g, b, c=3, card=4)
    cfg = OfficialConfig(score_path="int32")
    for mode, kw in (("exact", {}), ("bloom", dict(m_bits=64, k_hash=3))):
        m = SilverTorch(k, n_lists=8, n_probe=3, filter_mode=mode, seed=1, official=cfg, **kw)
        m.register_index(_t(dev, items), _t(dev, attrs))
        perm = _np(m.sort_perm)
        # the filter over sorted positions; bloom with the recheck equals the exact filter
        valid = of.clause_match(attrs[perm], np.zeros(3, bool), qa)
        ids, sc = m(_t(dev, q), m.prepare_queries(_t(dev, qa)))
        want_ids, want_sc = _st_oracle(m, q, k, valid)
        assert np.array_equal(_np(ids), want_ids), mode
        assert np.array_equal(_np(sc), want_sc), mode
    # the builder and a state-dict round trip give the same module
    sd = {kk: v.clone() for kk, v in m.state_dict().items()}
    m2 = (SilverTorchBuilder(k=k, n_lists=8, n_probe=3, filter_mode="bloom", m_bits=64,
                             k_hash=3, official=cfg).set_state_dict(sd).build())
    ids2, sc2 = m2(_t(dev, q), m2.prepare_queries(_t(dev, qa)))
    assert torch.equal(ids2, torch.from_numpy(want_ids).to(dev))
    assert torch.equal(sc2, torch.from_numpy(want_sc).to(dev))


def test_silvertorch_candidates(dev):
    from retrieve_amd.modules import OfficialConfig, SilverTorch

    g = rng(18)
    n, d, b, k = 3000, 128, 4, 15
    items = g.standard_normal((n, d)).astype(np.float32)
    q = g.standard_normal((b, d)).astype(np.float32)
    m = SilverTorch(k, n_lists=4, n_probe=2, official=OfficialConfig(score_path="int32"))
    m.register_index(_t(dev, items))
    cand = g.integers(0, n, (b, 200)).astype(np.int64)
    cand[0, 50:] = -1
    cand[3, :] = -1
    ids, sc = m(_t(dev, q), candidate_ids=_t(dev, cand))
    q_codes, q_scales = oq.quantize_int8(q, divide=True)
    want_ids, want_sc = _rerank_oracle(q_codes, q_scales, _np(m.item_codes), _np(m.inv_perm),
                                       _np(m.global_scale), cand, k)
    assert np.array_equal(_np(ids), want_ids)
    assert np.array_equal(_np(sc), want_sc)
    ids, _ = m(_t(dev, q), candidate_ids=_t(dev, cand[:, :6]))
    assert ids.shape == (b, 6)
