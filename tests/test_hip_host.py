"""Host-side checks of ``retrieve_amd.hip`` that need no GPU: which strided masks the blocked
scans may read in place (the transposed Bloom words of ``st.bloom_search_t``)."""

from __future__ import annotations

import torch


def _hip():
    import retrieve_amd.hip as hip

    return hip


def _transposed(cols: int, stride: int, b: int) -> torch.Tensor:
    """``st.bloom_search_t``'s layout on the host: ``[cols, stride]`` words viewed ``[b, cols]``."""
    return torch.zeros((cols, stride), dtype=torch.int64).t()[:b]


def test_transposed_stride_accepts_the_search_layout():
    hip = _hip()
    assert hip._transposed_stride(_transposed(40, 256, 200), 200) == 256
    assert hip._transposed_stride(_transposed(40, 512, 300), 300) == 512
    # fewer rows than the stride was sized for: the staged block still ends inside the buffer
    assert hip._transposed_stride(_transposed(40, 512, 100), 100) == 512


def test_transposed_stride_rejects_views_that_would_overrun():
    """A row-sliced view starts one word in, so its last word row's staged block (all
    ``roundup(B, 256)`` entries) would end past the allocation: it must take the copy."""
    hip = _hip()
    m = _transposed(40, 256, 200)
    assert hip._transposed_stride(m[1:], 199) == 0
    assert hip._transposed_stride(_transposed(40, 512, 300)[1:], 299) == 0
    # the second half of a [cols, 512] buffer, viewed transposed: exactly fits
    buf = torch.zeros((40, 512), dtype=torch.int64)
    half = buf[:, 256:].t()
    assert half.storage_offset() == 256
    assert hip._transposed_stride(half, 256) == 512
    # ... but one word further in does not
    assert hip._transposed_stride(buf[:, 257:].t(), 255) == 0


def test_transposed_stride_ignores_other_layouts():
    hip = _hip()
    assert hip._transposed_stride(torch.zeros((16, 40), dtype=torch.int64), 16) == 0
    assert hip._transposed_stride(torch.zeros((16, 1), dtype=torch.int64), 16) == 0
    assert hip._transposed_stride(torch.zeros((40, 200), dtype=torch.int64).t(), 200) == 0
    assert hip._transposed_stride(None, 16) == 0
