"""The oracle, the host-side parser and the HIP ops against the reference's own CPU ops: fixtures
written by ``tests/golden/make_ref_fixtures.py`` from Meta's SilverTorch C++ built from source
(``oracle/build_ref.py``). They pin bit for bit what no closed form does: the parser's plan bytes,
the Bloom index words at the upstream width, the Bloom search's column words and partial
response, and the scorer's int32 / fp16-divisor raw buffers."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import filters as ofl
from oracle import silvertorch as ost
from tests.conftest import GOLDEN
from tests.test_int8_scan import _pack


@pytest.fixture(scope="module")
def ref():
    arrays = dict(np.load(os.path.join(GOLDEN, "ref_cpu.npz")))
    with open(os.path.join(GOLDEN, "ref_cpu.json")) as f:
        meta = json.load(f)
    return arrays, meta


def _features(attrs):
    n, c, _ = attrs.shape
    valid = attrs != -1
    offsets = np.zeros(n * c + 1, np.int64)
    offsets[1:] = np.cumsum(valid.sum(-1).reshape(-1))
    return (np.arange(c, dtype=np.int32), offsets,
            attrs.reshape(-1)[valid.reshape(-1)].astype(np.int64))


# --- CPU: the oracle and the host parser ------------------------------------------------------


def test_parser_plan_bytes(ref):
    """``retrieve_amd.bloom.parse_batch`` writes Meta's plan bytes and max stack depth, including
    the fan-out batching at small ``max_sub_queries`` (chains ending on a batch carry a one-child
    node)."""
    from retrieve_amd import bloom as bl

    a, meta = ref
    for i, (hk, msq) in enumerate(meta["parse_settings"]):
        stack, data, offs = bl.parse_batch(meta["expressions"], hk, msq)
        assert stack == meta["parse_max_stack"][i], (hk, msq)
        assert np.array_equal(offs, a[f"parse{i}_offsets"]), (hk, msq)
        assert np.array_equal(data.view(np.int8), a[f"parse{i}_data"]), (hk, msq)


@pytest.mark.parametrize("name", ["b5k3", "b2k2"])
def test_oracle_bloom_build_upstream_width(ref, name):
    a, meta = ref
    bm, k = meta["bloom_builds"][name]
    words, offs = ofl.bloom_build(a["bloom_attrs"].astype(np.int64), k, b_multiplier=bm)
    assert np.array_equal(offs, a[f"bloom_{name}_offsets"])
    assert np.array_equal(words, a[f"bloom_{name}_words"])


def _oracle_columns(a, meta):
    words, offs = a["bloom_b5k3_words"], a["bloom_b5k3_offsets"]
    ncol = (len(offs) - 1) * 32
    cols = np.zeros((len(meta["expressions"]), ncol), np.int64)
    for i, e in enumerate(meta["expressions"]):
        cols[i] = _pack(ofl.bloom_expression_mask(words, offs, ncol * 64, e, 3, 7)[None])[0]
    return cols


def test_oracle_bloom_search(ref):
    """Every plan over every column word, padding docs of the last bundle included."""
    a, meta = ref
    assert np.array_equal(_oracle_columns(a, meta), a["search_words"])


@pytest.mark.parametrize("tag", ["", "_qpi"])
def test_oracle_partial_response(ref, tag):
    a, _ = ref
    qpi = a["partial_plan_index"] if tag else None
    cum, first, words = ofl.bloom_partial_response(a["search_words"], a["partial_starts"],
                                                   a["partial_lengths"], qpi)
    assert np.array_equal(cum, a[f"partial{tag}_cumsum"])
    assert np.array_equal(first, a[f"partial{tag}_first"])
    assert np.array_equal(words, a[f"partial{tag}_words"])


@pytest.mark.parametrize("layout", ["warps", "short"])
@pytest.mark.parametrize("div", [-1, 64, 3])
def test_oracle_scorer(ref, layout, div):
    """int32 dots and fp16(fp32(dot) / divisor) keys, bit for bit, in the layouts where the CPU
    op's slot order (probe, then doc) is the CUDA op's (whole warps; short clusters)."""
    a, meta = ref
    sc, ix = ost.fused_kmean_ann(a[f"scorer_{layout}_offsets"], a[f"scorer_{layout}_ids"],
                                 a[f"scorer_{layout}_lengths"], a["scorer_emb"],
                                 a["scorer_queries"], meta[f"scorer_{layout}_width"], divisor=div)
    want_sc = a[f"scorer_{layout}_div{div}_scores"]
    assert sc.dtype == want_sc.dtype
    assert np.array_equal(ix, a[f"scorer_{layout}_div{div}_indices"])
    assert np.array_equal(sc.view(np.uint8), want_sc.view(np.uint8))


# --- GPU: the HIP ops ---------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["b5k3", "b2k2"])
def test_gpu_bloom_build_upstream_width(dev, ref, name):
    import torch

    import retrieve_amd.st  # noqa: F401

    a, meta = ref
    bm, k = meta["bloom_builds"][name]
    fid, fo, fv = (torch.from_numpy(x).to(dev) for x in
                   _features(a["bloom_attrs"].astype(np.int64)))
    words, offs = torch.ops.st.bloom_index_build(fid, fo, fv, bm, k)
    assert np.array_equal(offs.cpu().numpy(), a[f"bloom_{name}_offsets"])
    assert np.array_equal(words.cpu().numpy(), a[f"bloom_{name}_words"])


@pytest.mark.gpu
def test_gpu_bloom_search_and_partial_response(dev, ref):
    import torch

    import retrieve_amd.st  # noqa: F401

    a, _ = ref
    words = torch.from_numpy(a["bloom_b5k3_words"]).to(dev)
    offs = torch.from_numpy(a["bloom_b5k3_offsets"]).to(dev)
    data = torch.from_numpy(a["parse0_data"])
    poffs = torch.from_numpy(a["parse0_offsets"])
    got = torch.ops.st.bloom_index_search_batch(words, offs, data, poffs, 3, 7, False)
    assert np.array_equal(got.cpu().numpy(), a["search_words"])
    # the same expressions parsed with more fan-out batching (one-child AND / OR nodes, deeper
    # chains) evaluate to the same words
    for i, (hk, msq) in enumerate(ref[1]["parse_settings"]):
        if hk != 7:
            continue
        got = torch.ops.st.bloom_index_search_batch(
            words, offs, torch.from_numpy(a[f"parse{i}_data"]),
            torch.from_numpy(a[f"parse{i}_offsets"]), 3, 7, False)
        assert np.array_equal(got.cpu().numpy(), a["search_words"]), msq
    bools = torch.ops.st.bloom_index_search_batch(words, offs, data, poffs, 3, 7, True)
    unpacked = np.unpackbits(a["search_words"].view(np.uint64).astype(">u8").view(np.uint8),
                             axis=1).astype(bool)
    assert np.array_equal(bools.cpu().numpy(), unpacked)
    starts = torch.from_numpy(a["partial_starts"]).to(dev)
    lens = torch.from_numpy(a["partial_lengths"]).to(dev)
    for tag in ("", "_qpi"):
        qpi = torch.from_numpy(a["partial_plan_index"]).to(dev) if tag else None
        out = torch.ops.st.bloom_index_search_batch_return_partial_response(
            words, offs, data, poffs, starts, lens, 3, 7, qpi)
        for got, key in zip(out, ("cumsum", "first", "words")):
            assert np.array_equal(got.cpu().numpy(), a[f"partial{tag}_{key}"]), (tag, key)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["warps", "short"])
def test_gpu_scorer(dev, ref, layout):
    import torch

    import retrieve_amd.st  # noqa: F401

    a, meta = ref
    args = [torch.from_numpy(a[f"scorer_{layout}_{k}"]).to(dev)
            for k in ("offsets", "ids", "lengths")]
    emb = torch.from_numpy(a["scorer_emb"]).to(dev)
    q = torch.from_numpy(a["scorer_queries"]).to(dev)
    for div in (-1, 64, 3):
        sc, ix = torch.ops.st.fused_kmean_ann(*args, emb, q, meta[f"scorer_{layout}_width"],
                                              divisor_for_int8=div)
        want = a[f"scorer_{layout}_div{div}_scores"]
        assert np.array_equal(ix.cpu().numpy(), a[f"scorer_{layout}_div{div}_indices"])
        assert np.array_equal(sc.cpu().numpy().view(np.uint8), want.view(np.uint8)), div
