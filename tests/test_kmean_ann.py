"""``st::fused_kmean_ann`` / ``_with_partial_masks`` and
``st::bloom_index_search_batch_return_partial_response[_prepared]`` on the GPU against the CPU
restatements (``oracle.silvertorch.fused_kmean_ann``, ``oracle.filters.bloom_partial_response``):
the raw slot buffer (full warps per probe, then remainders) bit for bit for int8 rows (int32,
the fp16 divisor path and the per-doc fp16 scales), within the row type's rounding for
bf16 / fp16 / fp32 rows; full-N masks with and without ``filtering_bit_index``; the probed-column
Bloom words and their use as partial masks."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import retrieve_amd.st as st
from oracle import filters as ofl
from oracle import silvertorch as ost
from retrieve_amd import bloom as bl
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _clusters(g, n, n_lists):
    cuts = np.sort(g.choice(np.arange(1, n), n_lists - 1, replace=False))
    starts = np.concatenate([[0], cuts]).astype(np.int64)
    sizes = np.diff(np.concatenate([starts, [n]])).astype(np.int64)
    offsets = np.concatenate([starts, [n]]).astype(np.int64)  # CSR, n_lists + 1 entries
    return offsets, sizes


def _probes(g, b, p, n_lists, sizes):
    ids = np.stack([g.permutation(n_lists)[:p] for _ in range(b)]).astype(np.int64)
    lens = sizes[np.clip(ids, 0, n_lists - 1)].copy()
    return ids, lens


def _check_int8(dev, offsets, ids, lens, emb, q, width, **kw):
    print(f"fused_kmean_ann int8 B={q.shape[0]} N={emb.shape[0]} P={ids.shape[1]} "
          f"width={width} {sorted(kw)}", flush=True)
    gpu_kw = {}
    for key, val in kw.items():
        if key == "valid":
            gpu_kw["filtering_bit_mask"] = _t(dev, _pack(val))
        elif key == "valid_index":
            gpu_kw["filtering_bit_index"] = _t(dev, val)
        elif key == "scale":
            gpu_kw["per_embedding_scale"] = _t(dev, val)
        elif key == "divisor":
            gpu_kw["divisor_for_int8"] = val
        elif key == "invalid":
            gpu_kw["invalid_index_value"] = val
    sc, ix = torch.ops.st.fused_kmean_ann(_t(dev, offsets), _t(dev, ids), _t(dev, lens),
                                          _t(dev, emb), _t(dev, q), width, **gpu_kw)
    want_sc, want_ix = ost.fused_kmean_ann(offsets, ids, lens, emb, q, width, **kw)
    assert np.array_equal(ix.cpu().numpy(), want_ix)
    got = sc.cpu().numpy()
    assert got.dtype == want_sc.dtype
    assert np.array_equal(got.view(np.uint8), want_sc.view(np.uint8))


def test_int8_raw_scores(dev):
    g = rng(800)
    n, d, b, p, n_lists = 6000, 128, 5, 6, 17
    _, sizes = _clusters(g, n, n_lists)
    sizes[3] = 64  # whole warps only
    sizes[5] = 7   # a remainder only
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    n = int(offsets[-1])
    emb = g.integers(-128, 128, (n, d), dtype=np.int8)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    ids, lens = _probes(g, b, p, n_lists, sizes)
    ids[0, :3] = [3, 5, 0]
    lens[0, :3] = sizes[[3, 5, 0]]
    ids[1, 2] = 10**6  # an invalid cluster probes nothing
    width = int(lens.sum(1).max())
    _check_int8(dev, offsets, ids, lens, emb, q, width)
    _check_int8(dev, offsets, ids, lens, emb, q, width + 70, invalid=-7)
    _check_int8(dev, offsets, ids, lens, emb, q, width // 2)  # rows cut at the width
    valid = g.random((b, n)) < 0.4
    valid[2] = False
    _check_int8(dev, offsets, ids, lens, emb, q, width, valid=valid)
    vrows = g.random((2, n)) < 0.5
    _check_int8(dev, offsets, ids, lens, emb, q, width, valid=vrows,
                valid_index=np.array([1, 0, 1, 1, 0], np.int64))
    _check_int8(dev, offsets, ids, lens, emb, q, width, divisor=64)
    _check_int8(dev, offsets, ids, lens, emb, q, width, divisor=3, valid=valid)
    scale = (g.random(n) * 8 + 0.25).astype(np.float16)
    _check_int8(dev, offsets, ids, lens, emb, q, width, scale=scale)


def test_fp16_divisor_ties(dev):
    """The fp16 keys of the serving path land on fp16 rounding ties: dot / 2 = 1024.5 rounds to
    1024 (even), 1025.5 to 1026, and dots 2048 / 2049 merge into one key, 2052 / 2053 too."""
    d = 64
    q = np.zeros((1, d), np.int8)
    q[0, :2] = [127, 1]
    emb = np.zeros((4, d), np.int8)
    emb[:, 0] = 16
    emb[:, 1] = [16, 17, 20, 21]  # dots 2048, 2049, 2052, 2053
    offsets = np.array([0, 4], np.int64)
    sc, ix = torch.ops.st.fused_kmean_ann(_t(dev, offsets), _t(dev, np.zeros((1, 1), np.int64)),
                                          _t(dev, np.array([[4]], np.int64)), _t(dev, emb),
                                          _t(dev, q), 4, divisor_for_int8=2)
    assert sc.dtype == torch.float16
    assert sc[0, :4].float().cpu().tolist() == [1024.0, 1024.0, 1026.0, 1026.0]
    assert ix[0, :4].cpu().tolist() == [0, 1, 2, 3]


def test_per_doc_scale_rounds_twice(dev):
    """The per-doc fp16 scale branch is ``c10::Half(dot) / scale`` (``index_mm_helpers.cuh:
    51-53``): the dot is rounded to fp16 before the division and the quotient again. Known
    answers from IEEE half arithmetic: dot 2051 → fp16 2052 (a tie at spacing 2, to even), / 1.5
    = 1368; dot 2053 → 2052, / 0.75 = 2736. Rounding once (Meta's CPU twin,
    ``fused_kmean_ann.cpp:200-202``) gives 1367 and 2738 instead; this build follows the CUDA
    op."""
    d = 64
    q = np.ones((1, d), np.int8)
    emb = np.zeros((2, d), np.int8)
    emb[:, :16] = 127  # 2032
    emb[:, 16] = [19, 21]  # dots 2051, 2053
    scale = np.array([1.5, 0.75], np.float16)
    offsets = np.array([0, 2], np.int64)
    sc, ix = torch.ops.st.fused_kmean_ann(_t(dev, offsets), _t(dev, np.zeros((1, 1), np.int64)),
                                          _t(dev, np.array([[2]], np.int64)), _t(dev, emb),
                                          _t(dev, q), 2, per_embedding_scale=_t(dev, scale))
    assert sc.dtype == torch.float16
    assert sc[0, :2].float().cpu().tolist() == [1368.0, 2736.0]
    assert ix[0, :2].cpu().tolist() == [0, 1]


@pytest.mark.parametrize("dtype,rtol", [(torch.bfloat16, 2.0**-7), (torch.float16, 2.0**-10),
                                        (torch.float32, 1e-5)])
def test_float_raw_scores(dev, dtype, rtol):
    """Float rows: indices exact, scores within the row type's rounding of the float64 dot,
    relative to the sum of the products' magnitudes (the scale of any accumulation's error; the
    reference accumulates fp16 / bf16 in the row type, so no bit-for-bit claim is made)."""
    g = rng(801)
    n, d, b, p, n_lists = 4000, 96, 3, 4, 9
    offsets, sizes = _clusters(g, n, n_lists)
    emb32 = g.standard_normal((n, d)).astype(np.float32)
    q32 = g.standard_normal((b, d)).astype(np.float32)
    emb_t = torch.from_numpy(emb32).to(dtype)
    q_t = torch.from_numpy(q32).to(dtype)
    ids, lens = _probes(g, b, p, n_lists, sizes)
    width = int(lens.sum(1).max())
    valid = g.random((b, n)) < 0.7
    sc, ix = torch.ops.st.fused_kmean_ann(_t(dev, offsets), _t(dev, ids), _t(dev, lens),
                                          emb_t.to(dev), q_t.to(dev), width,
                                          filtering_bit_mask=_t(dev, _pack(valid)))
    assert sc.dtype == dtype
    want_sc, want_ix = ost.fused_kmean_ann(offsets, ids, lens, emb_t.float().numpy(),
                                           q_t.float().numpy(), width, valid=valid)
    assert np.array_equal(ix.cpu().numpy(), want_ix)
    got = sc.float().cpu().numpy()
    written = want_ix >= 0
    ev = emb_t.double().numpy()
    qv = q_t.double().numpy()
    safe = np.maximum(want_ix, 0)
    e = np.einsum("rwd,rd->rw", ev[safe], qv)
    mag = np.einsum("rwd,rd->rw", np.abs(ev[safe]), np.abs(qv))
    assert (np.abs(got[written] - e[written]) <= rtol * mag[written]).all()
    lowest = {torch.bfloat16: -3.3895313892515355e38, torch.float16: -65504.0,
              torch.float32: -3.4028234663852886e38}[dtype]
    assert (got[~written] == np.float32(lowest)).all()


# --- probed-column Bloom search and partial masks ---------------------------------------------


@pytest.fixture(scope="module")
def bloom_case():
    """A 6000-doc index over 3 attributes, 64 bits a doc (the fixed-width build), its plans, and
    each plan's column words over the whole index from the oracle's expression evaluation: every
    doc of the index's bundles, the padding past doc 6000 included (a plan is evaluated on whole
    column words, so EMPTY and NOT set padding bits there, bloom_index_search.cpp:255-277)."""
    g = rng(810)
    n, c = 6000, 3
    attrs = g.integers(0, 12, (n, c, 1)).astype(np.int64)
    words, boffs = ofl.bloom_build(attrs, 3, bits_per_doc=64)
    exprs = ["0:1 OR 0:2", "1:3 AND NOT 2:4", "", "(0:5 OR 1:6) AND 2:7", "2:0"]
    ncol = (len(boffs) - 1) * 32
    cols = np.zeros((len(exprs), ncol), np.int64)
    for i, e in enumerate(exprs):
        m = ofl.bloom_expression_mask(words, boffs, ncol * 64, e, 3, 7)
        cols[i] = _pack(m[None, :])[0]
    return g, n, attrs, words, boffs, exprs, cols


def _probed(g, n, b, p):
    offsets, sizes = _clusters(g, n, 23)
    ids = np.stack([g.permutation(23)[:p] for _ in range(b)]).astype(np.int64)
    lens = sizes[ids].copy()
    lens[0, 0] = 0  # an empty probe spans no column
    return offsets, ids, offsets[ids], lens


def test_partial_response(dev, bloom_case):
    g, n, _, words, boffs, exprs, cols = bloom_case
    b, p = len(exprs), 4
    offsets, ids, starts, lens = _probed(g, n, b, p)
    _, data, poffs = bl.parse_batch(exprs, 7, 5)
    out = torch.ops.st.bloom_index_search_batch_return_partial_response(
        _t(dev, words), _t(dev, boffs), torch.from_numpy(data.view(np.int8)),
        torch.from_numpy(poffs), _t(dev, starts), _t(dev, lens), 3, 7)
    want = ofl.bloom_partial_response(cols, starts, lens)
    for got, w in zip(out, want):
        assert got.dtype == torch.from_numpy(w).dtype
        assert np.array_equal(got.cpu().numpy(), w)
    # prepared plans: a static capacity past the total (zeros) and a row -> plan index
    blob, count, stack = st.prepare_plans(exprs, 7, dev)
    qpi = np.array([4, 4, 0, 2, 1], np.int64)
    total = int(want[0][-1])
    out = torch.ops.st.bloom_index_search_batch_return_partial_response_prepared(
        _t(dev, words), _t(dev, boffs), blob, count, stack, _t(dev, starts), _t(dev, lens), 3, 7,
        _t(dev, qpi), total + 100)
    want = ofl.bloom_partial_response(cols, starts, lens, qpi)
    assert np.array_equal(out[0].cpu().numpy(), want[0])
    assert np.array_equal(out[1].cpu().numpy(), want[1])
    got = out[2].cpu().numpy()
    assert np.array_equal(got[: want[2].size], want[2]) and (got[want[2].size :] == 0).all()


def test_fused_kmean_ann_with_partial_masks(dev, bloom_case):
    """The scorer filtered by the probed-column Bloom words: a doc is scored iff its bit in its
    probe's words is set."""
    g, n, _, words, boffs, exprs, cols = bloom_case
    b, p, d = len(exprs), 4, 64
    offsets, ids, starts, lens = _probed(g, n, b, p)
    emb = g.integers(-128, 128, (n, d), dtype=np.int8)
    q = g.integers(-128, 128, (b, d), dtype=np.int8)
    blob, count, stack = st.prepare_plans(exprs, 7, dev)
    cap = b * (int(lens.sum(1).max()) // 64 + 2 * p)
    partial = torch.ops.st.bloom_index_search_batch_return_partial_response_prepared(
        _t(dev, words), _t(dev, boffs), blob, count, stack, _t(dev, starts), _t(dev, lens), 3, 7,
        None, cap)
    width = int(lens.sum(1).max())
    for div in (-1, 16):
        sc, ix = torch.ops.st.fused_kmean_ann_with_partial_masks(
            _t(dev, offsets), _t(dev, ids), _t(dev, lens), _t(dev, emb), _t(dev, q), width,
            *partial, divisor_for_int8=div)
        want_partial = ofl.bloom_partial_response(cols, starts, lens)
        want_sc, want_ix = ost.fused_kmean_ann(offsets, ids, lens, emb, q, width, divisor=div,
                                               partial=want_partial)
        assert np.array_equal(ix.cpu().numpy(), want_ix)
        assert np.array_equal(sc.cpu().numpy().view(np.uint8), want_sc.view(np.uint8))
    # every scored doc passes its row's plan over the whole index
    for r in range(b):
        m = np.unpackbits(cols[r].view(np.uint64).astype(">u8").view(np.uint8)).astype(bool)
        assert m[want_ix[r][want_ix[r] >= 0]].all()


def test_opcheck_st_ops(dev, bloom_case):
    """``torch.library.opcheck`` (schema, fake tensor, autograd registration, AOT dispatch) over
    the forward's ops, as the reference's compile gate runs it."""
    g, n, attrs, words, boffs, exprs, cols = bloom_case
    b, p, d = len(exprs), 4, 64
    offsets, ids, starts, lens = _probed(g, n, b, p)
    emb = _t(dev, g.integers(-128, 128, (n, d), dtype=np.int8))
    q8 = _t(dev, g.integers(-128, 128, (b, d), dtype=np.int8))
    qf = _t(dev, g.standard_normal((b, d)).astype(np.float32))
    blob, count, stack = st.prepare_plans(exprs, 7, dev)
    cap = b * (int(lens.sum(1).max()) // 64 + 2 * p)
    width = int(lens.sum(1).max())
    tw, tb, ts, tl, to, ti = (_t(dev, x) for x in (words, boffs, starts, lens, offsets, ids))
    partial = torch.ops.st.bloom_index_search_batch_return_partial_response_prepared(
        tw, tb, blob, count, stack, ts, tl, 3, 7, None, cap)
    perm = _t(dev, np.arange(n, dtype=np.int64))
    gs = _t(dev, np.array([0.5], np.float32))
    cases = [
        (torch.ops.st.fused_kmean_ann.default, (to, ti, tl, emb, q8, width), {}),
        (torch.ops.st.fused_kmean_ann.default, (to, ti, tl, emb, q8, width),
         {"divisor_for_int8": 8}),
        (torch.ops.st.fused_kmean_ann_with_partial_masks.default,
         (to, ti, tl, emb, q8, width, *partial), {}),
        (torch.ops.st.bloom_index_search_batch_return_partial_response_prepared.default,
         (tw, tb, blob, count, stack, ts, tl, 3, 7, None, cap), {}),
        (torch.ops.st.bloom_index_search_batch_prepared.default, (tw, tb, blob, count, stack, 3,
                                                                   7), {}),
        (torch.ops.st.search.default, (qf, ti, to[:-1], tl[0].new_tensor(np.diff(offsets)),
                                       emb, perm, gs, 20, width), {}),
        (torch.ops.st.probe_prep.default, (qf, ti, to[:-1], _t(dev, np.diff(offsets))), {}),
    ]
    for op, args, kwargs in cases:
        print(f"opcheck {op}", flush=True)
        torch.library.opcheck(op, args, kwargs)
