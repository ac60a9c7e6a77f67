"""Code formats the scans consume (test infrastructure; see ``oracle/__init__``).

Pinned by: the reference's edge-value tests restated in ``tests/test_oracle.py`` (±abs_max →
±127, an all-zero row, a 1e-30 row, exact ``.5`` quotients that round half to even), and the
closed form below evaluated in fp64 element by element on small inputs. ``quantize_int8_global``
is pinned against torch's own CPU eager ops on the same inputs (the reference's function is
those ops) and by its closed-form properties (the extreme element → ±127, the reconstruction
error bound, the row permutation).
"""

from __future__ import annotations

import numpy as np

INV127 = np.float32(1.0) / np.float32(127.0)
ABS_MAX_FLOOR = np.float32(1e-8)


def quantize_int8(x: np.ndarray, divide: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8: ``retrieve/src/retrieve/indexing/quantize.py:9-18`` as the GPU
    computes it (``silvertorch/.../fork_search_cuda.cu:680-699``): ``abs_max = max(max|x|,
    fp32(1e-8))``; ``scale = abs_max * fp32(1/127)`` (``divide``: ``fp32(abs_max / 127)``, the
    Python function's ``abs_max / 127.0``); ``code = clamp(rint(fp32(fp64(x) /
    fp64(abs_max)) * 127), -128, 127)`` with round-half-to-even.

    ``x`` is ``[R, D]`` float32. Returns ``(codes int8 [R, D], scales float32 [R])``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    abs_max = np.maximum(np.abs(x).max(axis=1), ABS_MAX_FLOOR).astype(np.float32)
    if divide:
        scales = (abs_max / np.float32(127.0)).astype(np.float32)
    else:
        scales = (abs_max * INV127).astype(np.float32)
    q = (x.astype(np.float64) / abs_max.astype(np.float64)[:, None]).astype(np.float32)
    v = np.rint(q * np.float32(127.0))
    codes = np.clip(v, -128, 127).astype(np.int8)
    return codes, scales


def quantize_int8_global(x: np.ndarray, rows: np.ndarray | None = None
                         ) -> tuple[np.ndarray, np.float32]:
    """One scale for the table (``retrieve/src/retrieve/indexing/quantize.py:25-52``): ``abs_max
    = max(max x, -min x)`` floored at fp32(1e-8); ``code = clamp(rint(fp32(fp32(x / abs_max) *
    127)), -128, 127)`` (fp32 throughout); row ``i`` of the codes from row ``rows[i]``. Returns
    ``(codes int8 [N, D], abs_max float32)``; the scale is ``fp32(abs_max / 127)``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size:
        abs_max = np.float32(max(np.float32(x.max()), -np.float32(x.min())))
    else:
        abs_max = np.float32(0.0)
    abs_max = np.maximum(abs_max, ABS_MAX_FLOOR).astype(np.float32)
    src = x if rows is None else x[rows]
    q = (src / abs_max).astype(np.float32) * np.float32(127.0)
    codes = np.clip(np.rint(q), -128, 127).astype(np.int8)
    return codes, np.float32(abs_max)


def pack_signs(values: np.ndarray) -> np.ndarray:
    """``[R, D]`` floats → ``[R, D // 64]`` int64 words, bit ``b`` of word ``w`` set iff
    ``values[:, 64 w + b] > 0`` (LSB-first): ``indexing/quantize.py:63-72``."""
    r, d = values.shape
    if d % 64:
        raise ValueError(f"D must be a multiple of 64, got {d}")
    bits = (values > 0).reshape(r, d // 64, 64).astype(np.uint64)
    shifts = np.arange(64, dtype=np.uint64)
    words = np.bitwise_or.reduce(bits << shifts, axis=2)
    return words.view(np.int64)


def simhash_bits(x: np.ndarray, r: np.ndarray) -> np.ndarray:
    """SimHash codes ``pack_signs(x @ r.T)`` (``indexing/quantize.py:148-173``). The sign of a
    near-zero projection depends on the BLAS summation order, so parity tests feed the same
    codes to both sides rather than regenerating them."""
    return pack_signs(np.asarray(x, np.float32) @ np.asarray(r, np.float32).T)
