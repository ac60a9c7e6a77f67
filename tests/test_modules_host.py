"""Host-side logic of the module layer, on the CPU: k-means (reproducible, Lloyd's fixed point
under inner product), the IVF CSR layout, the global int8 codes, the clause slot layout, the
fp16 divisor, config validation and loading a reference-layout state dict."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import rng


@pytest.fixture(scope="module")
def mods():
    from retrieve_amd import modules

    return modules


def test_kmeans_reproducible_and_lloyd_fixed_point(mods):
    g = rng(1)
    x = torch.from_numpy(g.standard_normal((700, 16)).astype(np.float32))
    for init in ("random", "kmeans++"):
        c1, a1 = mods.KMeans(9, n_iter=6, seed=4, init=init).fit(x)
        c2, a2 = mods.KMeans(9, n_iter=6, seed=4, init=init).fit(x)
        assert torch.equal(c1, c2) and torch.equal(a1, a2)
        # every row sits at its largest inner product, first index on ties
        assert torch.equal(a1, (x @ c1.t()).argmax(dim=1))
    # one more Lloyd step from the returned centroids: the means of the returned clusters
    c, a = mods.KMeans(5, n_iter=30, seed=0).fit(x)
    for j in range(5):
        rows = x[a == j]
        if rows.shape[0]:
            assert torch.allclose(rows.double().mean(0).float(), c[j], atol=1e-5)


def test_csr_layout_and_probe_width(mods):
    g = rng(2)
    a = torch.from_numpy(g.integers(0, 7, 500)).long()
    a[a == 3] = 4  # an empty list
    perm, inv, offsets, sizes = mods.csr_layout(a, 7)
    assert torch.equal(inv[perm], torch.arange(500))
    assert sizes[3] == 0 and int(offsets[-1]) == 500
    for j in range(7):
        seg = perm[offsets[j]:offsets[j + 1]]
        assert (a[seg] == j).all() and (seg[1:] > seg[:-1]).all()  # ascending ids inside
    assert mods.probe_width(sizes, 2) == int(sizes.sort().values[-2:].sum())


def test_quantize_int8_global(mods):
    g = rng(3)
    x = torch.from_numpy(g.standard_normal((300, 32)).astype(np.float32))
    perm = torch.from_numpy(g.permutation(300)).long()
    codes, scale = mods.quantize_int8_global(x, rows=perm)
    m = float(max(x.max(), -x.min()))
    assert scale == pytest.approx(m / 127, rel=1e-6)
    assert codes.abs().max() == 127
    assert (codes.float() * scale - x[perm]).abs().max() <= scale / 2 + 1e-6


def test_fork_clause_attrs(mods):
    g = rng(4)
    attrs = torch.from_numpy(g.integers(-1, 5, (40, 3, 3))).long()
    attrs[:, 2] = -1  # a clause nobody holds: zero width
    slots, cs = mods.fork_clause_attrs(attrs)
    assert cs.tolist()[0] == 0 and cs[3] == cs[2]
    assert slots.shape == (int(cs[-1]), 40) and slots.dtype == torch.int32
    for c in range(3):
        block = slots[cs[c]:cs[c + 1]]  # [width, N], each doc's values descending
        for d in range(40):
            vals = sorted((v for v in attrs[d, c].tolist() if v != -1), reverse=True)
            col = block[:, d].tolist()
            assert col[: len(vals)] == vals and all(v == -1 for v in col[len(vals):])
    q = mods.fork_query_attrs(torch.tensor([[-1, 3, 2**40], [-7, 0, 2**31 - 1]]))
    assert q.tolist() == [[-1, 3, -(2**31)], [-(2**31), 0, 2**31 - 1]]


def test_default_divisor_and_config(mods):
    for d in (1, 64, 128, 512, 1024, 4096):
        v = mods.default_divisor(d)
        assert v & (v - 1) == 0 and 127 * 127 * d / v <= 65504
        assert v == 1 or 127 * 127 * d / (v // 2) > 65504
    assert mods.OfficialConfig(score_path="int32").divisor_for(512) == -1
    assert mods.OfficialConfig(divisor=8).divisor_for(512) == 8
    for bad in (dict(score_path="x"), dict(divisor=3), dict(b_multiplier=1.0),
                dict(n_stored_hashes=0), dict(build_k=11), dict(bloom_width="y")):
        with pytest.raises(ValueError):
            mods.OfficialConfig(**bad)


def test_module_argument_checks(mods):
    with pytest.raises(ValueError):
        mods.PostfilterKNN(10, backend="triton")
    with pytest.raises(ValueError):
        mods.SilverTorch(10, 4, 2, filter_mode="bloom")  # needs m_bits and k_hash
    with pytest.raises(ValueError):
        mods.SilverTorch(10, 4, 2, filter_mode="bloom", m_bits=96, k_hash=3)
    with pytest.raises(ValueError):
        mods.SilverTorch(10, 4, 2, m_bits=64)
    with pytest.raises(ValueError):
        mods.LiNRV3(100, candidate_pool=9000)  # above the 1-bit scan's 8192
    with pytest.raises(ValueError):
        mods.LiNRV3(100, candidate_pool=50)
    with pytest.raises(ValueError):
        mods.LiNRV2(10, filter=None)


def test_postfilter_loads_reference_state_dict(mods):
    """The reference keeps ``item_embs_t [D, N]`` fp16; loading it transposes once."""
    g = rng(5)
    e = torch.from_numpy(g.standard_normal((50, 8)).astype(np.float32)).half()
    sd = {"idx.item_embs_t": e.t().contiguous()}
    v1 = mods.LiNRBuilder("v1", k=5).set_state_dict(sd).build()
    assert torch.equal(v1.idx.item_embs, e) and "item_embs_t" not in dict(v1.idx.named_buffers())
    own = mods.PostfilterKNN(5)
    own.register_index(e.float())
    again = mods.LiNRBuilder("v1", k=5).set_state_dict(
        {"idx." + k: v for k, v in own.state_dict().items()}).build()
    assert torch.equal(again.idx.item_embs, e)


def test_blocked_gate_mirrors_the_kernel_plan():
    """The Python gate's LDS estimate follows the kernel's (tile rows and list capacity per
    layout): lists of k + 128 entries at the wide layout's 128-row tiles."""
    from retrieve_amd import hip

    assert hip._use_blocked(64, 256, 384) and not hip._use_blocked(64, 256, 900)
    assert hip._use_blocked(64, 256, 700)  # two 32 KiB stages beside 1024-entry lists
    assert not hip._use_blocked(31, 256, 100)  # below the blocked batch
    assert hip._use_blocked(300, 512, 990)  # narrow 32-row tiles: lists of 1024
