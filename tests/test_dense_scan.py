"""bf16 / fp16 dense full scan + top-k on the GPU against the float64 oracle: returned scores
within 1e-3 relative of the float64 dot of the returned ids; ids equal to the exact top-k
except inside a tolerance band around the k-th score (near-ties may swap); recall@k against
exact scoring 1.0 on clustered data (``torch.ops.retrieve_amd.dense_scan_topk``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from tests.conftest import rng
from tests.test_int8_scan import _pack

pytestmark = pytest.mark.gpu

RTOL = 1e-3


def _clustered(g, n, d, centres, sigma=0.3):
    """BASELINE configs[1] generator: centre + sigma * N(0,1), L2-normalised."""
    x = centres[g.integers(0, centres.shape[0], n)] + sigma * g.standard_normal((n, d))
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def _check(dev, q32, it32, k, dtype=torch.bfloat16, mask=None):
    print(f"dense scan {dtype} B={q32.shape[0]} N={it32.shape[0]} D={q32.shape[1]} k={k} "
          f"mask={mask is not None}", flush=True)
    qt = torch.from_numpy(q32).to(dev).to(dtype)
    it = torch.from_numpy(it32).to(dev).to(dtype)
    mt = None if mask is None else torch.from_numpy(_pack(mask)).to(dev)
    ids, sc = torch.ops.retrieve_amd.dense_scan_topk(qt, it, k, mt)
    torch.cuda.synchronize()
    ids, sc = ids.cpu().numpy(), sc.cpu().numpy()
    # exact scores of the values the kernel saw (the 16-bit roundings), in float64
    qv = qt.float().cpu().numpy()
    iv = it.float().cpu().numpy()
    want_ids, want_sc = osc.dense_topk(qv, iv, k, mask)
    exact = osc.dense_scores(qv, iv)
    for r in range(q32.shape[0]):
        m = int((want_ids[r] >= 0).sum())
        assert (ids[r, m:] == -1).all() and np.isneginf(sc[r, m:]).all()
        got = ids[r, :m]
        assert (got >= 0).all() and len(set(got.tolist())) == m
        if mask is not None:
            assert mask[r, got].all()
        e = exact[r, got]
        scale = np.maximum(np.abs(e), 1e-3)
        assert (np.abs(sc[r, :m] - e) <= RTOL * scale).all()
        if m:
            assert (sc[r, :m - 1] >= sc[r, 1:m]).all()
            kth = want_sc[r, m - 1]
            band = RTOL * max(abs(kth), 1e-3) * 2
            assert (e >= kth - band).all()  # nothing far below the exact k-th is returned
            missing = set(want_ids[r, :m].tolist()) - set(got.tolist())
            for i in missing:  # anything missed is a near-tie of the boundary
                assert exact[r, i] <= sc[r, m - 1] + band
    return ids


@pytest.mark.parametrize(
    "b,n,d,k", [(1, 1, 64, 1), (3, 1000, 128, 10), (16, 20000, 128, 100), (17, 5000, 256, 100),
                (64, 12345, 64, 100), (5, 3000, 512, 1000), (2, 4096, 32, 7)],
)
def test_random_parity(dev, b, n, d, k):
    g = rng(b + n + d + k)
    q = g.standard_normal((b, d)).astype(np.float32)
    it = g.standard_normal((n, d)).astype(np.float32)
    _check(dev, q, it, k)


@pytest.mark.parametrize("b,n,d,k", [(128, 20000, 128, 100), (1024, 5000, 64, 10),
                                     (300, 3000, 256, 1000), (40, 9000, 128, 100),
                                     (64, 20000, 128, 700), (96, 9000, 64, 1000)])
def test_large_batch_parity(dev, b, n, d, k):
    """B >= 32 (rows of 128, 256 or 512 bytes) runs the register-blocked kernel; B <= 128 below
    512-byte rows the row-quarter layout, two stages beside the lists of k = 700 and 1000."""
    g = rng(b + n + d + k + 5)
    q = g.standard_normal((b, d)).astype(np.float32)
    it = g.standard_normal((n, d)).astype(np.float32)
    _check(dev, q, it, k)
    _check(dev, q, it, k, torch.float16)


def test_fp16(dev):
    g = rng(41)
    q = g.standard_normal((9, 128)).astype(np.float32)
    it = g.standard_normal((30000, 128)).astype(np.float32)
    _check(dev, q, it, 100, torch.float16)


def test_clustered_recall_seeded(dev):
    """configs[1]'s generator (1024 Gaussian clusters, sigma 0.3, L2-normalised) above the seed
    threshold: recall@100 against exact scoring of the same bf16 values is 1."""
    g = rng(42)
    centres = g.standard_normal((1024, 128))
    it = _clustered(g, 2_300_000, 128, centres)
    q = _clustered(g, 16, 128, centres)
    ids = _check(dev, q, it, 100)
    qv = torch.from_numpy(q).bfloat16().float().numpy()
    iv = torch.from_numpy(it).bfloat16().float().numpy()
    want, _ = osc.dense_topk(qv, iv, 100)
    recall = np.mean([len(set(a) & set(b)) / 100 for a, b in zip(ids.tolist(), want.tolist())])
    assert recall >= 0.99


def test_masked(dev):
    g = rng(43)
    q = g.standard_normal((6, 128)).astype(np.float32)
    it = g.standard_normal((30000, 128)).astype(np.float32)
    mask = g.random((6, 30000)) < 0.1
    mask[2] = g.random(30000) < 0.001
    mask[4] = False
    _check(dev, q, it, 100, mask=mask)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k_above_1024(dev, dtype):
    g = rng(44)
    q = g.standard_normal((3, 128)).astype(np.float32)
    it = g.standard_normal((12000, 128)).astype(np.float32)
    mask = g.random((3, 12000)) < 0.6
    mask[2] = g.random(12000) < 0.05  # ~600 survivors < k
    _check(dev, q, it, 1500, dtype=dtype, mask=mask)


@pytest.mark.parametrize("b,n,d,masked", [(8, 5000, 128, False), (64, 20000, 128, True),
                                            (256, 30000, 128, False), (300, 20000, 64, True),
                                            (128, 9000, 32, False)])
def test_fp32(dev, b, n, d, masked):
    """fp32 rows: the blocked scan on the fp32 matrix cores from B = 32 (wide and narrow layouts,
    D 32 / 64 / 128), the raw scorer and key select below."""
    g = rng(45 + b + d)
    q = g.standard_normal((b, d)).astype(np.float32)
    it = g.standard_normal((n, d)).astype(np.float32)
    mask = (g.random((b, n)) < 0.3) if masked else None
    _check(dev, q, it, 100, dtype=torch.float32, mask=mask)


def test_errors(dev):
    q = torch.zeros((2, 64), dtype=torch.bfloat16, device=dev)
    it = torch.zeros((10, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(TypeError):
        torch.ops.retrieve_amd.dense_scan_topk(q.float(), it, 3)
    with pytest.raises(TypeError):
        torch.ops.retrieve_amd.dense_scan_topk(q, it.half(), 3)
    with pytest.raises(ValueError):
        torch.ops.retrieve_amd.dense_scan_topk(q[:, :32], it, 3)


def test_large_batch_seeded_path(dev):
    """bf16 at B = 256 over 2.2M clustered rows: the blocked kernel's seeded path, the main pass
    behind the seed sample's rank-th best."""
    g = rng(18)
    centres = g.standard_normal((64, 128))
    it = _clustered(g, 2_200_000, 128, centres)
    q = _clustered(g, 256, 128, centres)
    _check(dev, q, it, 100)
