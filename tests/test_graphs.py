"""The hot paths captured in a HIP graph (``torch.cuda.graph``): the ops enqueue kernels only
on torch's current stream, with no host sync and no memset in the captured region, so one
capture replays the whole forward. Each test replays several times with eager calls and
synchronizations in between and checks every replay against the eager result (the reference
times its headline ``graph`` mode this way, ``evaluation/bench/measure.py:348-373``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import retrieve_amd.st as st
from retrieve_amd import bloom as bl
from tests.conftest import rng
from tests.test_configs import _query_sets, _zipf_attrs
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _replays_match(fn, replays=3):
    eager = [t.clone() for t in fn()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on a side stream, as torch.cuda.graph recommends
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = fn()
    for i in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(captured, eager):
            assert torch.equal(got, want), f"replay {i}"
        again = fn()  # eager work between replays
        torch.cuda.synchronize()
        for got, want in zip(again, eager):
            assert torch.equal(got, want)
    return captured


def test_filtered_int8_step(dev):
    """The headline step: prepared Bloom search, the exact clause post-check AND-ed with it, and
    the int8 scan with the fused top-100 (seeded: N above 2**21 rows)."""
    g = rng(900)
    n, d, b = 2_200_000, 512, 16
    items = torch.from_numpy(g.integers(-128, 128, (n, d), dtype=np.int8)).to(dev)
    q = torch.from_numpy(g.integers(-128, 128, (b, d), dtype=np.int8)).to(dev)
    attrs = _zipf_attrs(g, n)
    sets = _query_sets(g, attrs, b, 0.1)
    at = torch.from_numpy(attrs).to(dev)
    fid, fo, fv = st.attrs_to_features(at)
    words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 64, 3)
    blob, count, stack = st.prepare_plans(bl.sets_to_expressions(sets), 7, dev)
    a16 = at.to(torch.int16)
    rev = torch.zeros(8, dtype=torch.bool, device=dev)
    qs = torch.from_numpy(sets).to(dev)

    def step():
        pre = torch.ops.st.bloom_index_search_batch_prepared(words, offs, blob, count, stack, 3, 7)
        mask = torch.ops.retrieve_amd.clause_bits(a16, rev, qs, pre)
        return torch.ops.retrieve_amd.int8_scan_topk(q, items, 100, mask)

    print("graph: filtered int8 step B=16 N=2.2M", flush=True)
    _replays_match(step)


def test_search_one_list(dev):
    """st::search over one list (the full-scan path, kept from the warm-up's one check of the
    list) and over IVF probes with the Bloom recheck."""
    g = rng(901)
    n, d, b = 300_000, 256, 8
    items = torch.from_numpy(g.integers(-128, 128, (n, d), dtype=np.int8)).to(dev)
    query = torch.from_numpy(g.standard_normal((b, d)).astype(np.float32)).to(dev)
    perm = torch.from_numpy(g.permutation(n).astype(np.int64)).to(dev)
    gs = torch.tensor([0.25], device=dev)
    offs = torch.zeros(1, dtype=torch.int64, device=dev)
    sizes = torch.full((1,), n, dtype=torch.int64, device=dev)
    probes = torch.zeros((b, 1), dtype=torch.int64, device=dev)

    def one_list():
        return torch.ops.st.search(query, probes, offs, sizes, items, perm, gs, 100, n)

    print("graph: st::search one list", flush=True)
    _replays_match(one_list)

    n_lists = 40
    cuts = np.sort(g.choice(np.arange(1, n), n_lists - 1, replace=False))
    starts = np.concatenate([[0], cuts]).astype(np.int64)
    csz = np.diff(np.concatenate([starts, [n]])).astype(np.int64)
    pr = torch.from_numpy(np.stack([g.permutation(n_lists)[:6] for _ in range(b)])).to(dev)
    so, ss = torch.from_numpy(starts).to(dev), torch.from_numpy(csz).to(dev)
    valid = torch.from_numpy(_pack(g.random((b, n)) < 0.3)).to(dev)

    def ivf():
        return torch.ops.st.search(query, pr, so, ss, items, perm, gs, 64, int(n), 64,
                                   filtering_bit_mask=valid)

    print("graph: st::search IVF fp16 keys, masked", flush=True)
    _replays_match(ivf)

    # Bloom plans over the probed payloads only, with the exact recheck (the column bound comes
    # from the eager calls before the capture)
    attrs = _zipf_attrs(g, n)
    sets = _query_sets(g, attrs, b, 0.1)
    at = torch.from_numpy(attrs).to(dev)
    fid, fo, fv = st.attrs_to_features(at)
    words, boffs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, 64, 3)
    blob, count, stack = st.prepare_plans(bl.sets_to_expressions(sets), 7, dev)
    slots = at[:, :, 0].t().contiguous().to(torch.int32)
    cs = torch.arange(attrs.shape[1] + 1, dtype=torch.int64, device=dev)
    rev = torch.zeros(attrs.shape[1], dtype=torch.bool, device=dev)
    qa = torch.full((b, attrs.shape[1]), -1, dtype=torch.int64, device=dev)
    qa[:, 0] = at[:b, 0, 0]  # one active clause: the value of a doc each row can match

    def payload():
        return torch.ops.st.search(query, pr, so, ss, items, perm, gs, 50, int(n),
                                   bloom_index=words, bloom_bundle_b_offsets=boffs, plans=blob,
                                   plan_count=count, max_stack_size=stack, bloom_k=3, hash_k=7,
                                   item_clause_attrs=slots, clause_slots=cs,
                                   clause_is_reverse=rev, query_clause_attrs=qa)

    print("graph: st::search IVF, payload Bloom + exact recheck", flush=True)
    _replays_match(payload)


def test_dense_and_hamming_masked(dev):
    """Configuration 3's masked register-blocked bf16 scan (B = 256, the mask transposed in the
    workspace) and configuration 5's masked 512-bit Hamming scan at k = 1000."""
    g = rng(902)
    n = 300_000
    q = torch.from_numpy(g.standard_normal((256, 128)).astype(np.float32)).to(dev).bfloat16()
    it = torch.from_numpy(g.standard_normal((n, 128)).astype(np.float32)).to(dev).bfloat16()
    mask = torch.from_numpy(_pack(g.random((256, n)) < 0.1)).to(dev)
    print("graph: masked bf16 B=256", flush=True)
    _replays_match(lambda: torch.ops.retrieve_amd.dense_scan_topk(q, it, 100, mask))
    qb = torch.from_numpy(g.integers(-(2**63), 2**63 - 1, (256, 8), dtype=np.int64)).to(dev)
    ib = torch.from_numpy(g.integers(-(2**63), 2**63 - 1, (n, 8), dtype=np.int64)).to(dev)
    print("graph: masked hamming B=256 k=1000", flush=True)
    _replays_match(lambda: torch.ops.retrieve_amd.hamming_scan_topk(qb, ib, 1000, mask))
