"""The reference harness's ``graph`` mode gate (``evaluation/bench/measure.py:348-373``, restated
as ``bench.graph_callable``): ``torch.compile(..., mode="reduce-overhead", dynamic=False,
fullgraph=True)`` warmed on the example arguments must cause no cudagraph skip, and one call must
be exactly one graph launch. Covered: LiNR V1 at B = 64 with the exact filter, LiNR V3 with the
filter, SilverTorch over one list and over IVF probes with the Bloom filter and its exact recheck,
and the headline step as ``bench.py --mode graph`` compiles it. Every compiled call (with eager
calls in between) equals the eager result, and the headline step's compiled code launches this
library's kernels only: the compiler generates no kernel of its own for it."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from tests.conftest import rng

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(400)]


@pytest.fixture(autouse=True)
def _fresh_dynamo():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _t(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _gate(fn, *args, calls=3):
    with torch.inference_mode():
        eager = [t.clone() for t in fn(*args)]
    compiled = bench.graph_callable(fn, *args)
    for i in range(calls):
        with torch.inference_mode():
            got = [t.clone() for t in compiled(*args)]
            again = fn(*args)  # eager work between the compiled calls
        torch.cuda.synchronize()
        for a, b in zip(got, eager):
            assert torch.equal(a, b), f"compiled call {i}"
        for a, b in zip(again, eager):
            assert torch.equal(a, b)


def _attrs(g, n, c=4, a=2, card=6):
    attrs = g.integers(0, card, (n, c, a)).astype(np.int64)
    attrs[g.random((n, c, a)) < 0.3] = -1
    return attrs


def _query_attrs(g, b, c=4, card=6):
    q = g.integers(0, card, (b, c)).astype(np.int64)
    q[g.random((b, c)) < 0.5] = -1
    return q


def test_linr_v1_b64(dev):
    from retrieve_amd.modules import ExactAttributeFilter, LiNRV1

    print("compile gate: LiNRV1 B=64", flush=True)
    g = rng(1400)
    n, d, b, k = 200_000, 128, 64, 100
    m = LiNRV1(k, filter=ExactAttributeFilter())
    m.register_index(_t(dev, g.standard_normal((n, d)).astype(np.float32)),
                     _t(dev, _attrs(g, n)))
    q = _t(dev, g.standard_normal((b, d)).astype(np.float32)).half()
    prepared = m.prepare_queries(_t(dev, _query_attrs(g, b)))
    _gate(m, q, prepared)
    _gate(m, q)


def test_linr_v3_filtered(dev):
    from retrieve_amd.modules import ExactAttributeFilter, LiNRV3

    print("compile gate: LiNRV3 B=16, pool 1000, exact filter", flush=True)
    g = rng(1401)
    n, d, b, k = 100_000, 128, 16, 50
    m = LiNRV3(k, candidate_pool=1000, seed=3, filter=ExactAttributeFilter())
    m.register_index(_t(dev, g.standard_normal((n, d)).astype(np.float32)),
                     _t(dev, _attrs(g, n, card=3)))
    q = _t(dev, g.standard_normal((b, d)).astype(np.float32))
    _gate(m, q, m.prepare_queries(_t(dev, _query_attrs(g, b, card=3))))


def test_silvertorch_one_list_and_ivf_bloom(dev):
    from retrieve_amd.modules import OfficialConfig, SilverTorch

    g = rng(1402)
    n, d, b = 60_000, 128, 8
    items = _t(dev, g.standard_normal((n, d)).astype(np.float32))
    q = _t(dev, g.standard_normal((b, d)).astype(np.float32))
    print("compile gate: SilverTorch one list", flush=True)
    one = SilverTorch(100, n_lists=1, n_probe=1, seed=1)
    one.register_index(items)
    _gate(one, q)

    print("compile gate: SilverTorch IVF, Bloom filter + exact recheck", flush=True)
    attrs = _attrs(g, n, c=3, a=1, card=4)
    ivf = SilverTorch(50, n_lists=16, n_probe=4, filter_mode="bloom", m_bits=64, k_hash=3,
                      seed=2, official=OfficialConfig(score_path="int32"))
    ivf.register_index(items, _t(dev, attrs))
    _gate(ivf, q, ivf.prepare_queries(_t(dev, _query_attrs(g, b, c=3, card=4))))


@pytest.mark.parametrize("bloom", ["probe", "search"])
def test_headline_step_as_bench_compiles_it(dev, bloom):
    """bench.py's default step (the Bloom plans probed inside the scan) and its --bloom-search
    form (the search's mask, then the clause scan)."""
    from torch._inductor.utils import run_and_get_code

    n, b, d = 2_300_000, 16, 512
    print(f"compile gate: headline step B={b} N={n} D={d}, Bloom {bloom}", flush=True)
    items = bench.int8_table(n, d, 1234, dev)
    queries = bench.int8_table(b, d, 99, dev)
    flt = bench.Filter(n, b, 0.1, dev)

    def step():
        if bloom == "probe":
            return flt.scan(queries, items, 100)
        return torch.ops.retrieve_amd.int8_scan_topk_clauses(queries, items, 100, flt.attrs,
                                                             flt.rev, flt.sets, flt.bloom())

    _gate(step)
    torch._dynamo.reset()
    with torch.inference_mode():
        _, codes = run_and_get_code(torch.compile(step, mode="reduce-overhead", dynamic=False,
                                                  fullgraph=True))
    src = "\n".join(codes)
    if bloom == "probe":
        assert "scan_topk_bloom_clauses" in src
    else:
        assert "bloom_index_search_batch_prepared" in src and "int8_scan_topk_clauses" in src
    assert "async_compile.triton(" not in src, "the compiler generated a kernel of its own"
