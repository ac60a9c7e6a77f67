"""The allocation-free int8 scan, ``rt_int8_scan_topk_noalloc``, through the C ABI: bit-exact
against ``rt_int8_scan_topk`` (the same kernels with a caller workspace) on two calls in a row,
the second smaller than the first (the fixed scratch keeps the first call's contents), and the
over-size rejection before any launch. Named to run last: it shares the process's scratch
array with nothing else, and must pass alone or after every other test."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from retrieve_amd import _native as nat
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu


def _outputs(b, k, dev):
    return (torch.full((b, k), -7, dtype=torch.int64, device=dev),
            torch.full((b, k), -7, dtype=torch.int32, device=dev))


def _with_workspace(lib, q, it, k, mask):
    b, d = q.shape
    n = it.shape[0]
    ids, sc = _outputs(b, k, q.device)
    ws = nat.workspace(lib.rt_int8_scan_topk_workspace(b, n, d, k), q.device)
    nat.check(lib.rt_int8_scan_topk(
        nat.ptr(q), b, nat.ptr(it), n, d, k, nat.ptr(mask),
        0 if mask is None else mask.shape[1], nat.ptr(ids), nat.ptr(sc), nat.ptr(ws),
        ws.numel(), nat.stream(q.device)))
    return ids, sc


def _no_alloc(lib, q, it, k, mask):
    b, d = q.shape
    n = it.shape[0]
    ids, sc = _outputs(b, k, q.device)
    nat.check(lib.rt_int8_scan_topk_noalloc(
        nat.ptr(q), b, nat.ptr(it), n, d, k, nat.ptr(mask),
        0 if mask is None else mask.shape[1], nat.ptr(ids), nat.ptr(sc),
        nat.stream(q.device)))
    return ids, sc


def test_no_alloc_matches_workspace_entry_point(dev):
    lib = nat.lib()
    g = rng(700)
    # call 1: two 16-query groups, the seeded path (N above 8 x 2**18 rows), a mask
    b1, n1, d1, k1 = 32, 2_500_000, 512, 100
    q1 = torch.from_numpy(g.integers(-128, 128, (b1, d1), dtype=np.int8)).to(dev)
    it1 = torch.from_numpy(g.integers(-128, 128, (n1, d1), dtype=np.int8)).to(dev)
    m1 = g.random((b1, n1)) < 0.3
    m1[3] = False
    mask1 = torch.from_numpy(_pack(m1)).to(dev)
    print(f"no-alloc call 1: B={b1} N={n1} D={d1} k={k1} masked", flush=True)
    got1 = _no_alloc(lib, q1, it1, k1, mask1)
    want1 = _with_workspace(lib, q1, it1, k1, mask1)
    torch.cuda.synchronize()
    assert torch.equal(got1[0], want1[0]) and torch.equal(got1[1], want1[1])
    assert (got1[0][3] == -1).all()
    del it1, mask1
    # call 2: smaller (one group, unseeded, no mask) over the scratch call 1 left behind
    b2, n2, d2, k2 = 5, 70_000, 256, 10
    q2 = g.integers(-128, 128, (b2, d2), dtype=np.int8)
    it2 = g.integers(-128, 128, (n2, d2), dtype=np.int8)
    print(f"no-alloc call 2: B={b2} N={n2} D={d2} k={k2}", flush=True)
    qt, itt = torch.from_numpy(q2).to(dev), torch.from_numpy(it2).to(dev)
    got2 = _no_alloc(lib, qt, itt, k2, None)
    want2 = _with_workspace(lib, qt, itt, k2, None)
    torch.cuda.synchronize()
    assert torch.equal(got2[0], want2[0]) and torch.equal(got2[1], want2[1])
    want_ids, want_sc = osc.int8_topk(q2, it2, k2)
    assert np.array_equal(got2[0].cpu().numpy(), want_ids)
    assert np.array_equal(got2[1].cpu().numpy(), want_sc)


def test_no_alloc_rejects_plans_above_its_scratch(dev):
    """k = 1000 over 6000 queries: 375 groups of candidate lists at one workgroup each (the
    1024-row table gives one workgroup whatever the CU count) need 375 MiB, above the fixed
    160 MiB. Every buffer is real and sized for the call, so nothing is read out of bounds
    whatever the outcome; the call returns 1 before any launch and leaves the outputs alone."""
    lib = nat.lib()
    g = rng(701)
    b, n, d, k = 6000, 1024, 64, 1000
    q = torch.from_numpy(g.integers(-128, 128, (b, d), dtype=np.int8)).to(dev)
    it = torch.from_numpy(g.integers(-128, 128, (n, d), dtype=np.int8)).to(dev)
    ids, sc = _outputs(b, k, dev)
    st = lib.rt_int8_scan_topk_noalloc(nat.ptr(q), b, nat.ptr(it), n, d, k, None, 0,
                                       nat.ptr(ids), nat.ptr(sc), nat.stream(dev))
    msg = lib.rt_last_error().decode()
    assert st == 1, msg
    assert "scratch" in msg and "rt_int8_scan_topk" in msg
    with pytest.raises(ValueError, match="scratch"):
        nat.check(st)
    torch.cuda.synchronize()
    assert (ids == -7).all() and (sc == -7).all()
