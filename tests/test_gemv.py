"""``torch.ops.retrieve.gemv_scores`` on the GPU: bit-exact against the in-order float32
accumulation (``oracle.scan.gemv_scores``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scan as osc
from tests.conftest import rng

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,n", [(1, 1), (128, 100_000), (256, 4099), (7, 31), (512, 65536)])
def test_gemv_bit_exact(dev, d, n):
    g = rng(d + n)
    print(f"gemv D={d} N={n}", flush=True)
    q = g.standard_normal((1, d)).astype(np.float16)
    e = g.standard_normal((d, n)).astype(np.float16)
    out = torch.ops.retrieve.gemv_scores(torch.from_numpy(q).to(dev), torch.from_numpy(e).to(dev))
    assert out.shape == (1, n) and out.dtype == torch.float32
    assert np.array_equal(out.cpu().numpy()[0], osc.gemv_scores(q[0], e))


def test_gemv_errors(dev):
    q = torch.zeros((2, 8), dtype=torch.float16, device=dev)
    e = torch.zeros((8, 16), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):
        torch.ops.retrieve.gemv_scores(q, e)
    with pytest.raises(ValueError):
        torch.ops.retrieve.gemv_scores(q[:1].float(), e)
    with pytest.raises(ValueError):
        torch.ops.retrieve.gemv_scores(q[:1], e.t().contiguous().t())
