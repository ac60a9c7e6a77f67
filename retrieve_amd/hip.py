"""The ``"hip"`` op namespace: the reference's ``retrieve.ops.triton`` surface, re-implemented as
HIP kernels behind the C ABI and registered as ``torch.ops.retrieve.*``.

``torch.ops.retrieve`` holds exactly the reference's seven ops (``clause_mask``,
``clause_mask_scores``, ``clause_compact``, ``fused_masked_knn_topk``, ``gemv_scores``,
``oporp_1bit_match_topk_full``, ``oporp_1bit_match_topk_indirect``) with the reference's
schemas, as its export gate requires (``retrieve/tests/compile/test_export_kernel_ref.py:115-143``).
The ops this build adds (the fused full scans with and without clauses, ``clause_bits``,
``mask_compact``, the re-ranks, the quantize and pack kernels) register under
``torch.ops.retrieve_amd.*`` instead, so they never enter the reference's namespace.

Importing this module registers the ops (the one side-effecting import, as the reference's
``retrieve.ops.triton``; ``import retrieve_amd`` registers nothing). Every op validates its
inputs here (``ValueError`` on shapes / contiguity, ``TypeError`` on dtypes, as
``retrieve/src/retrieve/ops/triton/_host.py:25-31`` and the preps do), allocates its outputs
and scratch from torch's caching allocator, and enqueues on torch's current stream.
"""

from __future__ import annotations

import torch
from torch import Tensor

from retrieve_amd import _native as nat


def _check_items(**tables: Tensor) -> None:
    """Item-side tables must arrive contiguous (``ops/triton/_host.py:25-31``)."""
    for name, t in tables.items():
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (copy it once at index build)")


# --- large-batch dispatch ---------------------------------------------------------------------

# From this batch on the dense scans run the register-blocked kernel (256 queries per
# workgroup, item tiles read once per 256 queries) instead of 16 queries per wave.
BLOCKED_MIN_BATCH = 32
# The fused scans' list bound; above it int8_scan_topk and dense_scan_topk select from the raw
# scorer's buffer (retrieve_amd.large_k).
MAX_FUSED_K = 1024
_BLOCKED_ROW_BYTES = (128, 256, 512)


def _use_blocked(b: int, row_bytes: int, k: int) -> bool:
    """Mirrors the kernel's LDS plan (``blk_rows``, ``blk_capw``, ``blk_lds``, ``blk_stages`` in
    ``csrc/scan_blocked.h``): the blocked scan only where its lists and fewest stages fit."""
    wide = b <= 128  # the kernel's wide / narrow layout
    if wide:
        rows = 128 if row_bytes < 512 else 64
    else:
        rows = 32 if row_bytes >= 512 else 64
    capw = 1 << (k + rows - 1).bit_length()  # the next power of two >= k + rows
    stage = rows * row_bytes + 256 * (rows // 32) * 4  # a tile and its mask words
    # the fewest stages the kernel is built with: 2 for the wide layout's 32 KiB tiles, else 3
    lds = (2 if wide and row_bytes < 512 else 3) * stage + (8 if wide else 4) * (capw * 8 + 64 * 4)
    return b >= BLOCKED_MIN_BATCH and row_bytes in _BLOCKED_ROW_BYTES and lds <= 160 * 1024


def _blocked(q: Tensor, items: Tensor, k: int, dtype: int, mask: Tensor | None,
             ids: Tensor, scores: Tensor) -> None:
    b, d = q.shape
    n = items.shape[0]
    lib = nat.lib()
    dev = q.device
    ws = nat.workspace(lib.rt_blocked_scan_topk_workspace(b, n, d * q.element_size(), k,
                                                          int(mask is not None)), dev)
    with torch.cuda.device(dev):
        st = lib.rt_blocked_scan_topk(
            nat.ptr(q), b, nat.ptr(items), n, d, k, dtype, nat.ptr(mask),
            0 if mask is None else mask.shape[1], nat.ptr(ids), nat.ptr(scores), nat.ptr(ws),
            ws.numel(), nat.stream(dev),
        )
    nat.check(st)


# --- int8 full scan + top-k ---------------------------------------------------------------


def _int8_scan_prep(query_codes: Tensor, item_codes: Tensor, k: int, mask: Tensor | None):
    if query_codes.dim() != 2 or item_codes.dim() != 2:
        raise ValueError("query_codes must be [B, D] and item_codes [N, D]")
    if query_codes.dtype != torch.int8 or item_codes.dtype != torch.int8:
        raise TypeError("query_codes and item_codes must be int8")
    if query_codes.shape[1] != item_codes.shape[1]:
        raise ValueError(
            f"D mismatch: query D={query_codes.shape[1]} vs item D={item_codes.shape[1]}"
        )
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    _check_items(item_codes=item_codes)
    b, n = query_codes.shape[0], item_codes.shape[0]
    if mask is not None:
        if mask.dtype != torch.int64:
            raise TypeError("mask must be int64 words")
        if mask.dim() != 2 or mask.shape[0] != b or mask.shape[1] < (n + 63) // 64:
            raise ValueError(f"mask must be [B, ceil(N/64)] = [{b}, {(n + 63) // 64}]")
        mask = mask.contiguous()
    return query_codes.contiguous(), mask


@torch.library.custom_op("retrieve_amd::int8_scan_topk", mutates_args=(), device_types="cuda")
def int8_scan_topk(
    query_codes: Tensor, item_codes: Tensor, k: int, mask: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """Exact int8 full-scan top-k: ``query_codes [B, D]`` int8 against ``item_codes [N, D]`` int8,
    int32 dot products, top ``k`` by (score desc, item index asc) → ``(ids int64 [B, k], scores
    int32 [B, k])``, ``-1`` / ``INT32_MIN`` where fewer than ``k`` items pass ``mask``
    (``[B, ceil(N/64)]`` int64 words, item ``d`` at bit ``63 - d % 64``). The int8 scorer and
    radix select of ``st::search`` on a single cluster
    (``silvertorch/.../fork_search_cuda.cu:1256-1524``)."""
    q, mask = _int8_scan_prep(query_codes, item_codes, k, mask)
    dev = nat.require_device(q, item_codes)
    if k > MAX_FUSED_K:
        from retrieve_amd import large_k

        return large_k.full_scan_topk(q, item_codes, k, mask, -(2**31))
    b, d = q.shape
    n = item_codes.shape[0]
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.int32, device=dev)
    if _use_blocked(b, d, k):
        _blocked(q, item_codes, k, 0, mask, ids, scores)
        return ids, scores
    lib = nat.lib()
    ws_bytes = lib.rt_int8_scan_topk_workspace(b, n, d, k)
    ws = nat.workspace(ws_bytes, dev)
    with torch.cuda.device(dev):
        st = lib.rt_int8_scan_topk(
            nat.ptr(q), b, nat.ptr(item_codes), n, d, k, nat.ptr(mask),
            0 if mask is None else mask.shape[1],
            nat.ptr(ids), nat.ptr(scores), nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@int8_scan_topk.register_fake
def _(query_codes, item_codes, k, mask=None):
    b = query_codes.shape[0]
    return (
        query_codes.new_empty((b, k), dtype=torch.int64),
        query_codes.new_empty((b, k), dtype=torch.int32),
    )


# --- bf16 / fp16 dense full scan + top-k -----------------------------------------------------

_DENSE_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


@torch.library.custom_op("retrieve_amd::dense_scan_topk", mutates_args=(), device_types="cuda")
def dense_scan_topk(
    query: Tensor, item_embs: Tensor, k: int, mask: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """Dense full-scan top-k: ``query [B, D]`` against ``item_embs [N, D]`` (both bf16, both
    fp16 or both fp32: the fused scan for the 16-bit types up to k 1024, the raw scorer and a
    key select otherwise), fp32 accumulation, top ``k`` by (score desc, index asc) →
    ``(ids int64 [B, k], scores fp32 [B, k])``, ``-1`` / ``-inf`` where fewer than ``k`` items
    pass ``mask``. LiNR V1's ``torch.mm`` + ``masked_topk`` (``modules/knn.py:62-76``); the
    fused scan has no ``[B, N]`` score matrix."""
    if query.dim() != 2 or item_embs.dim() != 2:
        raise ValueError("query must be [B, D] and item_embs [N, D]")
    if query.dtype not in (*_DENSE_DTYPES, torch.float32) or item_embs.dtype != query.dtype:
        raise TypeError("query and item_embs must both be bfloat16, float16 or float32")
    if query.shape[1] != item_embs.shape[1]:
        raise ValueError(f"D mismatch: query D={query.shape[1]} vs item D={item_embs.shape[1]}")
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    _check_items(item_embs=item_embs)
    b, d = query.shape
    n = item_embs.shape[0]
    if mask is not None:
        if mask.dtype != torch.int64:
            raise TypeError("mask must be int64 words")
        if mask.dim() != 2 or mask.shape[0] != b or mask.shape[1] < (n + 63) // 64:
            raise ValueError(f"mask must be [B, ceil(N/64)] = [{b}, {(n + 63) // 64}]")
        mask = mask.contiguous()
    q = query.contiguous()
    dev = nat.require_device(q, item_embs)
    fp32 = q.dtype == torch.float32
    if k > MAX_FUSED_K or (fp32 and not _use_blocked(b, 4 * d, k)):
        # every score kept in fp32, then the select (fp32 rows below the blocked scan's batch)
        from retrieve_amd import large_k

        return large_k.full_scan_topk(q, item_embs, k, mask, float("-inf"))
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.float32, device=dev)
    if fp32:
        _blocked(q, item_embs, k, 3, mask, ids, scores)
        return ids, scores
    if _use_blocked(b, 2 * d, k):
        _blocked(q, item_embs, k, 1 + _DENSE_DTYPES[q.dtype], mask, ids, scores)
        return ids, scores
    lib = nat.lib()
    ws = nat.workspace(lib.rt_dense_scan_topk_workspace(b, n, d, k), dev)
    with torch.cuda.device(dev):
        st = lib.rt_dense_scan_topk(
            nat.ptr(q), b, nat.ptr(item_embs), n, d, k, _DENSE_DTYPES[q.dtype], nat.ptr(mask),
            0 if mask is None else mask.shape[1], nat.ptr(ids), nat.ptr(scores), nat.ptr(ws),
            ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@dense_scan_topk.register_fake
def _(query, item_embs, k, mask=None):
    b = query.shape[0]
    return (query.new_empty((b, k), dtype=torch.int64),
            query.new_empty((b, k), dtype=torch.float32))


# --- 1-bit Hamming full scan + top-k --------------------------------------------------------


# The full 1-bit scan selects up to this many items (above 1024 by counting its 64 W + 1 scores);
# the other scans up to 1024.
HAMMING_MAX_K = 8192


def _hamming_prep(query_bits: Tensor, item_bits: Tensor, k: int, mask: Tensor | None,
                  keep_transposed: bool = False):
    """``_oporp_prep``'s checks (``ops/triton/oporp_1bit_match_topk.py:148-165``); with
    ``keep_transposed`` a mask stored transposed (``_transposed_stride``) stays as it is."""
    if query_bits.dim() != 2 or item_bits.dim() != 2:
        raise ValueError("query_bits must be [B, W] and item_bits [N, W]")
    if query_bits.dtype != torch.int64 or item_bits.dtype != torch.int64:
        raise TypeError("query_bits and item_bits must be int64")
    if query_bits.shape[1] != item_bits.shape[1]:
        raise ValueError(
            f"W mismatch: query_bits W={query_bits.shape[1]} vs item_bits W={item_bits.shape[1]}"
        )
    if not 1 <= k <= HAMMING_MAX_K:
        raise ValueError(f"k must be in [1, {HAMMING_MAX_K}], got {k}")
    _check_items(item_bits=item_bits)
    b, n = query_bits.shape[0], item_bits.shape[0]
    if mask is not None:
        if mask.dtype != torch.int64:
            raise TypeError("mask must be int64 words")
        if mask.dim() != 2 or mask.shape[0] != b or mask.shape[1] < (n + 63) // 64:
            raise ValueError(f"mask must be [B, ceil(N/64)] = [{b}, {(n + 63) // 64}]")
        if not (keep_transposed and _transposed_stride(mask, b)):
            mask = mask.contiguous()
    return query_bits.contiguous(), mask


def _hamming_call(query_bits, item_bits, k, mask, score_dtype):
    q, mask = _hamming_prep(query_bits, item_bits, k, mask)
    dev = nat.require_device(q, item_bits)
    b, w = q.shape
    n = item_bits.shape[0]
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=score_dtype, device=dev)
    lib = nat.lib()
    ws = nat.workspace(lib.rt_hamming_scan_topk_workspace(b, n, w, k, int(mask is not None)),
                       dev)
    with torch.cuda.device(dev):
        st = lib.rt_hamming_scan_topk(
            nat.ptr(q), b, nat.ptr(item_bits), n, w, k, nat.ptr(mask),
            0 if mask is None else mask.shape[1], nat.ptr(ids), nat.ptr(scores),
            int(score_dtype == torch.float32), nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@torch.library.custom_op("retrieve_amd::hamming_scan_topk", mutates_args=(), device_types="cuda")
def hamming_scan_topk(
    query_bits: Tensor, item_bits: Tensor, k: int, mask: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """Exact 1-bit Hamming full-scan top-k on the integer score ``64 W - 2 popcount(q ^ item)``:
    ``(ids int64 [B, k], scores int32 [B, k])``, ties to the lower index, ``-1`` /
    ``INT32_MIN`` where fewer than ``k`` items pass ``mask``."""
    return _hamming_call(query_bits, item_bits, k, mask, torch.int32)


@hamming_scan_topk.register_fake
def _(query_bits, item_bits, k, mask=None):
    b = query_bits.shape[0]
    return (query_bits.new_empty((b, k)), query_bits.new_empty((b, k), dtype=torch.int32))


@torch.library.custom_op(
    "retrieve::oporp_1bit_match_topk_full", mutates_args=(), device_types="cuda"
)
def oporp_1bit_match_topk_full(
    query_bits: Tensor, item_bits: Tensor, k: int
) -> tuple[Tensor, Tensor]:
    """Full-scan Sign-OPORP 1-bit Hamming top-K (``ops/triton/oporp_1bit_match_topk.py:261-273``):
    ``64·W − 2·popcount(q ^ item)`` over every row of ``item_bits`` → ``(ids [B, k] int64,
    scores [B, k] fp32)``; ties go to the lower index (the reference's ``torch.topk`` leaves
    them unspecified). ``k > N`` pads ``-1`` / ``-inf`` (the reference's layer asserts
    ``k <= N``)."""
    return _hamming_call(query_bits, item_bits, k, None, torch.float32)


@oporp_1bit_match_topk_full.register_fake
def _(query_bits, item_bits, k):
    b = query_bits.shape[0]
    return (query_bits.new_empty((b, k)), query_bits.new_empty((b, k), dtype=torch.float32))


__all__ = [
    "dense_scan_topk",
    "hamming_scan_topk",
    "int8_scan_topk",
    "oporp_1bit_match_topk_full",
]


# --- exact clause filter (functional.py:173-185) --------------------------------------------

_CLAUSE_BITS, _CLAUSE_BOOL, _CLAUSE_SCORES = 0, 1, 2


_ATTR_DTYPES = (torch.int16, torch.int32, torch.int64)


def _clause_prep(item_clause_attrs: Tensor, clause_is_reverse: Tensor, query_values: Tensor,
                 *, sets: bool = False):
    """The checks of ``ops/triton/clause_mask.py:158-181``: ``[N, C, A_max]`` items (contiguous),
    ``[B, C]`` query values (``[B, C, V]`` value sets where ``sets``), ``[C]`` reverse flags."""
    if item_clause_attrs.dim() != 3:
        raise ValueError("item_clause_attrs must be [N, C, A_max]")
    if query_values.dim() != 2 and not (sets and query_values.dim() == 3):
        raise ValueError("query_clause_attrs must be [B, C]" + (" or [B, C, V]" if sets else ""))
    n, c, _ = item_clause_attrs.shape
    if query_values.shape[1] != c:
        raise ValueError(f"clause-count mismatch: items C={c}, query C={query_values.shape[1]}")
    # the reference ops take int64 tables; the packed-bits form also takes int16 / int32 ones
    attr_ok = item_clause_attrs.dtype in _ATTR_DTYPES if sets else \
        item_clause_attrs.dtype == torch.int64
    if not attr_ok or query_values.dtype != torch.int64:
        raise TypeError("item_clause_attrs must be int64 (int16 / int32 also for clause_bits) "
                        "and query values int64")
    if clause_is_reverse.shape != (c,):
        raise ValueError(f"clause_is_reverse must be [C] = [{c}]")
    if c > 32:
        raise ValueError(f"at most 32 clauses, got C={c}")
    _check_items(item_clause_attrs=item_clause_attrs)
    rev = clause_is_reverse.contiguous()
    # (a bool flag is its 0 / 1 byte: a view, not a copy kernel a call)
    rev = rev.view(torch.int8) if rev.dtype == torch.bool else rev.to(torch.int8)
    q = query_values.contiguous()
    if q.dim() == 2:
        q = q.unsqueeze(2)
    return rev, q


def _clause_filter(item_clause_attrs: Tensor, rev: Tensor, q: Tensor, mode: int, out: Tensor,
                   scores: Tensor | None = None, and_mask: Tensor | None = None) -> None:
    n, c, a = item_clause_attrs.shape
    b, _, v = q.shape
    if b == 0 or n == 0:
        return
    dev = nat.require_device(item_clause_attrs, q, rev, out)
    lib = nat.lib()
    ws = nat.workspace(lib.rt_clause_filter_workspace(b, c, v), dev)
    with torch.cuda.device(dev):
        st = lib.rt_clause_filter(
            nat.ptr(item_clause_attrs), item_clause_attrs.element_size(), n, c, a, nat.ptr(rev),
            nat.ptr(q), b, v, mode,
            nat.ptr(scores), nat.ptr(and_mask), 0 if and_mask is None else and_mask.shape[1],
            nat.ptr(out), nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)


@torch.library.custom_op("retrieve::clause_mask", mutates_args=(), device_types="cuda")
def clause_mask(
    item_clause_attrs: Tensor, clause_is_reverse: Tensor, query_clause_attrs: Tensor
) -> Tensor:
    """Exact clause evaluation → ``[B, N]`` bool (``ops/triton/clause_mask.py:270-281``): clause
    ``c`` matches iff some item value equals the query value, XOR ``clause_is_reverse[c]``; a
    query value ``-1`` is an inactive clause; AND over clauses."""
    rev, q = _clause_prep(item_clause_attrs, clause_is_reverse, query_clause_attrs)
    out = torch.empty((q.shape[0], item_clause_attrs.shape[0]), dtype=torch.bool,
                      device=query_clause_attrs.device)
    _clause_filter(item_clause_attrs, rev, q, _CLAUSE_BOOL, out)
    return out


@clause_mask.register_fake
def _(item_clause_attrs, clause_is_reverse, query_clause_attrs):
    return query_clause_attrs.new_empty(
        (query_clause_attrs.shape[0], item_clause_attrs.shape[0]), dtype=torch.bool
    )


@torch.library.custom_op("retrieve::clause_mask_scores", mutates_args=(), device_types="cuda")
def clause_mask_scores(
    scores: Tensor, item_clause_attrs: Tensor, clause_is_reverse: Tensor,
    query_clause_attrs: Tensor,
) -> Tensor:
    """``where(clause_mask(...), scores, -inf)`` in one pass
    (``ops/triton/clause_mask.py:284-303``);
    ``scores`` must be ``[B, N]`` float32."""
    rev, q = _clause_prep(item_clause_attrs, clause_is_reverse, query_clause_attrs)
    b, n = q.shape[0], item_clause_attrs.shape[0]
    if scores.shape != (b, n) or scores.dtype != torch.float32:
        raise ValueError(
            f"scores must be [B, N] = {[b, n]} float32, got {list(scores.shape)} {scores.dtype}"
        )
    s = scores.contiguous()
    out = torch.empty((b, n), dtype=torch.float32, device=scores.device)
    _clause_filter(item_clause_attrs, rev, q, _CLAUSE_SCORES, out, scores=s)
    return out


@clause_mask_scores.register_fake
def _(scores, item_clause_attrs, clause_is_reverse, query_clause_attrs):
    return torch.empty_like(scores)


@torch.library.custom_op("retrieve_amd::clause_bits", mutates_args=(), device_types="cuda")
def clause_bits(
    item_clause_attrs: Tensor, clause_is_reverse: Tensor, query_values: Tensor,
    and_mask: Tensor | None = None,
) -> Tensor:
    """The clause filter as the scans' packed mask: ``[B, ceil(N/64)]`` int64 words, item ``d``
    at bit ``63 - d % 64`` (the order of ``silvertorch/.../ops/official/__init__.py:33-35``).
    ``query_values`` is ``[B, C]`` (the reference predicate) or ``[B, C, V]`` value sets, ``-1``
    pads: clause ``c`` is active iff a value is not ``-1`` and matches iff an item value is in
    the set. ``item_clause_attrs`` may be int16 / int32 (a compact copy of the table).
    ``and_mask`` (``[B, >= ceil(N/64)]`` words, same bit layout) is AND-ed in, e.g. a Bloom
    search's ``[B, n_bundles * 32]`` pre-filter."""
    rev, q = _clause_prep(item_clause_attrs, clause_is_reverse, query_values, sets=True)
    b, n = q.shape[0], item_clause_attrs.shape[0]
    w = (n + 63) // 64
    if and_mask is not None:
        if and_mask.dtype != torch.int64 or and_mask.dim() != 2 or and_mask.shape[0] != b \
                or and_mask.shape[1] < w:
            raise ValueError(f"and_mask must be [B, >= ceil(N/64)] = [{b}, >= {w}] int64")
        and_mask = and_mask.contiguous()
    out = torch.empty((b, w), dtype=torch.int64, device=query_values.device)
    _clause_filter(item_clause_attrs, rev, q, _CLAUSE_BITS, out, and_mask=and_mask)
    return out


@clause_bits.register_fake
def _(item_clause_attrs, clause_is_reverse, query_values, and_mask=None):
    n = item_clause_attrs.shape[0]
    return query_values.new_empty((query_values.shape[0], (n + 63) // 64), dtype=torch.int64)


# --- full scans with the exact clause filter tested per candidate ----------------------------


def _transposed_stride(mask: Tensor | None, b: int) -> int:
    """The row stride S of a ``[B, W]`` mask whose words are stored transposed, ``[W, S]`` with
    S >= B rounded up to 256 (``st.bloom_search_t``'s layout, viewed as ``[B, W]``), else 0. The
    blocked scans read such a mask as it is; every other path takes ``mask.contiguous()``.

    The scans stage all ``roundup(B, 256)`` entries of a word row from the view's first element,
    so a view qualifies only where the last row's block ends inside its storage: a row-sliced or
    offset view of the transposed buffer (``m[1:]``) would read past the allocation's end and is
    copied instead."""
    if mask is None or mask.dim() != 2 or b == 0:
        return 0
    s0, s1 = mask.stride()
    pad = -(-b // 256) * 256
    if not (s0 == 1 and s1 >= pad and s1 % 256 == 0):
        return 0
    words = mask.shape[1]
    end = mask.storage_offset() + (words - 1) * s1 + pad
    return int(s1) if end <= mask.untyped_storage().nbytes() // mask.element_size() else 0


def _scan_clauses(q: Tensor, items: Tensor, k: int, dtype: int, item_clause_attrs: Tensor,
                  clause_is_reverse: Tensor, query_values: Tensor, mask: Tensor | None,
                  scores: Tensor, ids: Tensor) -> bool:
    """The fused scan into ``ids`` / ``scores`` (dtype 0 int8, 1 bf16, 2 fp16, 3 fp32): below
    the blocked batch ``rt_scan_topk_clauses`` (not fp32), from it ``rt_blocked_scan_topk_clauses``
    (with a mask only: its sampled bound is taken over the mask); False where neither applies
    (k above the fused lists' bound too), and the caller then scans over ``clause_bits``."""
    rev, qs = _clause_prep(item_clause_attrs, clause_is_reverse, query_values, sets=True)
    b, d = q.shape
    n = items.shape[0]
    if item_clause_attrs.shape[0] != n:
        raise ValueError(f"item_clause_attrs has {item_clause_attrs.shape[0]} rows, the items {n}")
    if qs.shape[0] != b:
        raise ValueError(f"query_values has {qs.shape[0]} rows, the queries {b}")
    if k > MAX_FUSED_K:
        return False
    blocked = _use_blocked(b, d * q.element_size(), k)
    if (blocked and mask is None) or (not blocked and dtype == 3):
        return False
    dev = nat.require_device(q, items, item_clause_attrs, qs)
    _, c, a = item_clause_attrs.shape
    v = qs.shape[2]
    lib = nat.lib()
    ts = _transposed_stride(mask, b) if blocked else 0
    if mask is not None and not ts:
        mask = mask.contiguous()
    words = 0 if mask is None else mask.shape[1]
    tail = (nat.ptr(item_clause_attrs), item_clause_attrs.element_size(), c, a, nat.ptr(rev),
            nat.ptr(qs), v, nat.ptr(ids), nat.ptr(scores))
    with torch.cuda.device(dev):
        if blocked:
            ws = nat.workspace(lib.rt_blocked_scan_topk_clauses_workspace(
                b, n, d * q.element_size(), k, c, v), dev)
            st = lib.rt_blocked_scan_topk_clauses(
                nat.ptr(q), b, nat.ptr(items), n, d, k, dtype, nat.ptr(mask), words, ts, *tail,
                nat.ptr(ws), ws.numel(), nat.stream(dev))
        else:
            ws = nat.workspace(lib.rt_scan_topk_clauses_workspace(b, n, d, k, c, v), dev)
            st = lib.rt_scan_topk_clauses(
                nat.ptr(q), b, nat.ptr(items), n, d, k, dtype, nat.ptr(mask), words, *tail,
                nat.ptr(ws), ws.numel(), nat.stream(dev))
    nat.check(st)
    return True


@torch.library.custom_op("retrieve_amd::int8_scan_topk_clauses", mutates_args=(),
                         device_types="cuda")
def int8_scan_topk_clauses(
    query_codes: Tensor, item_codes: Tensor, k: int, item_clause_attrs: Tensor,
    clause_is_reverse: Tensor, query_values: Tensor, mask: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """``int8_scan_topk`` over the items that pass ``mask`` and the exact clauses
    (``clause_bits``' arguments and predicate): the same results as
    ``int8_scan_topk(q, items, k, clause_bits(attrs, rev, values, mask))``. Up to the blocked
    scan's batch the clauses are tested inside the scan, only for the items whose score beats
    their query's running bound, so no ``[B, N]`` clause mask is written or read (the exact
    post-check inside the scorer, as ``silvertorch/.../fork_filters.cuh:15-41`` runs in
    ``fork_search_cuda.cu:918-1130``)."""
    q, mask = _int8_scan_prep(query_codes, item_codes, k, mask)
    b = q.shape[0]
    ids = torch.empty((b, k), dtype=torch.int64, device=q.device)
    scores = torch.empty((b, k), dtype=torch.int32, device=q.device)
    if _scan_clauses(q, item_codes, k, 0, item_clause_attrs, clause_is_reverse, query_values,
                     mask, scores, ids):
        return ids, scores
    bits = clause_bits(item_clause_attrs, clause_is_reverse, query_values, mask)
    return int8_scan_topk(q, item_codes, k, bits)


@int8_scan_topk_clauses.register_fake
def _(query_codes, item_codes, k, item_clause_attrs, clause_is_reverse, query_values, mask=None):
    b = query_codes.shape[0]
    return (query_codes.new_empty((b, k), dtype=torch.int64),
            query_codes.new_empty((b, k), dtype=torch.int32))


@torch.library.custom_op("retrieve_amd::dense_scan_topk_clauses", mutates_args=(),
                         device_types="cuda")
def dense_scan_topk_clauses(
    query: Tensor, item_embs: Tensor, k: int, item_clause_attrs: Tensor,
    clause_is_reverse: Tensor, query_values: Tensor, mask: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """``dense_scan_topk`` over the items that pass ``mask`` and the exact clauses: the same
    results as ``dense_scan_topk(q, items, k, clause_bits(attrs, rev, values, mask))``, the
    clauses tested inside the bf16 / fp16 scan up to the blocked scan's batch (as
    ``int8_scan_topk_clauses``). LiNR V1's ``ExactAttributeFilter.mask_scores`` +
    ``masked_topk`` (``retrieve/src/retrieve/modules/filters.py:48-52``,
    ``functional.py:57-85``) without the ``[B, N]`` scores."""
    if query.dim() != 2 or item_embs.dim() != 2 or query.dtype != item_embs.dtype:
        raise ValueError("query [B, D] and item_embs [N, D] of one dtype")
    dtype = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}.get(query.dtype)
    if dtype is None:
        raise TypeError("query and item_embs must both be bfloat16, float16 or float32")
    if query.shape[1] != item_embs.shape[1]:
        raise ValueError(f"D mismatch: query D={query.shape[1]} vs item D={item_embs.shape[1]}")
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    _check_items(item_embs=item_embs)
    b, n = query.shape[0], item_embs.shape[0]
    if mask is not None:
        if mask.dtype != torch.int64:
            raise TypeError("mask must be int64 words")
        if mask.dim() != 2 or mask.shape[0] != b or mask.shape[1] < (n + 63) // 64:
            raise ValueError(f"mask must be [B, ceil(N/64)] = [{b}, {(n + 63) // 64}]")
    q = query.contiguous()
    ids = torch.empty((b, k), dtype=torch.int64, device=q.device)
    scores = torch.empty((b, k), dtype=torch.float32, device=q.device)
    # (a mask stored transposed reaches the blocked scan as it is)
    if _scan_clauses(q, item_embs, k, dtype, item_clause_attrs, clause_is_reverse, query_values,
                     mask, scores, ids):
        return ids, scores
    bits = clause_bits(item_clause_attrs, clause_is_reverse, query_values,
                       None if mask is None else mask.contiguous())
    return dense_scan_topk(q, item_embs, k, bits)


@dense_scan_topk_clauses.register_fake
def _(query, item_embs, k, item_clause_attrs, clause_is_reverse, query_values, mask=None):
    b = query.shape[0]
    return (query.new_empty((b, k), dtype=torch.int64),
            query.new_empty((b, k), dtype=torch.float32))


@torch.library.custom_op("retrieve_amd::hamming_scan_topk_clauses", mutates_args=(),
                         device_types="cuda")
def hamming_scan_topk_clauses(
    query_bits: Tensor, item_bits: Tensor, k: int, item_clause_attrs: Tensor,
    clause_is_reverse: Tensor, query_values: Tensor, mask: Tensor | None = None,
    fused: bool = True,
) -> tuple[Tensor, Tensor]:
    """``hamming_scan_topk`` over the items that pass ``mask`` and the exact clauses: the same
    results as ``hamming_scan_topk(q, items, k, clause_bits(attrs, rev, values, mask))``.
    ``fused`` (default): where the matrix-core scan takes the batch and a mask is given (e.g. a
    Bloom search's words), the clauses are tested inside the scan, for the candidates that pass
    the mask (no ``[B, ceil(N/64)]`` clause mask in memory); elsewhere, or with ``fused=False``,
    the clause mask is written first, as above. LiNR V3's filtered shortlist
    (``modules/linr.py:155-162``)."""
    q, mask = _hamming_prep(query_bits, item_bits, k, mask, keep_transposed=True)
    rev, qs = _clause_prep(item_clause_attrs, clause_is_reverse, query_values, sets=True)
    b, w = q.shape
    n = item_bits.shape[0]
    if item_clause_attrs.shape[0] != n:
        raise ValueError(f"item_clause_attrs has {item_clause_attrs.shape[0]} rows, the items {n}")
    if qs.shape[0] != b:
        raise ValueError(f"query_values has {qs.shape[0]} rows, the queries {b}")
    lib = nat.lib()
    if not fused or mask is None or not lib.rt_hamming_scan_topk_clauses_fused(b, w, k):
        bits = clause_bits(item_clause_attrs, clause_is_reverse, query_values,
                           None if mask is None else mask.contiguous())
        return hamming_scan_topk(q, item_bits, k, bits)
    ts = _transposed_stride(mask, b)  # (the blocked scan reads a transposed mask as it is)
    dev = nat.require_device(q, item_bits, item_clause_attrs, qs)
    _, c, a = item_clause_attrs.shape
    v = qs.shape[2]
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.int32, device=dev)
    ws = nat.workspace(lib.rt_hamming_scan_topk_clauses_workspace(b, n, w, k, c, v), dev)
    with torch.cuda.device(dev):
        st = lib.rt_hamming_scan_topk_clauses(
            nat.ptr(q), b, nat.ptr(item_bits), n, w, k, nat.ptr(mask), mask.shape[1], ts,
            nat.ptr(item_clause_attrs), item_clause_attrs.element_size(), c, a, nat.ptr(rev),
            nat.ptr(qs), v, nat.ptr(ids), nat.ptr(scores), 0, nat.ptr(ws), ws.numel(),
            nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@hamming_scan_topk_clauses.register_fake
def _(query_bits, item_bits, k, item_clause_attrs, clause_is_reverse, query_values, mask=None,
      fused=True):
    b = query_bits.shape[0]
    return (query_bits.new_empty((b, k)), query_bits.new_empty((b, k), dtype=torch.int32))


def _mask_compact(mask: Tensor, n: int) -> tuple[Tensor, Tensor]:
    b = mask.shape[0]
    dev = mask.device
    ids = torch.empty((b, n), dtype=torch.int64, device=dev)
    counts = torch.empty((b,), dtype=torch.int64, device=dev)
    if b == 0:
        return ids, counts
    nat.require_device(mask)
    lib = nat.lib()
    ws = nat.workspace(lib.rt_mask_compact_workspace(b, n), dev)
    with torch.cuda.device(dev):
        st = lib.rt_mask_compact(nat.ptr(mask), b, n, nat.ptr(ids), nat.ptr(counts),
                                 nat.ptr(ws), ws.numel(), nat.stream(dev))
    nat.check(st)
    return ids, counts


@torch.library.custom_op("retrieve_amd::mask_compact", mutates_args=(), device_types="cuda")
def mask_compact(mask: Tensor, n: int) -> tuple[Tensor, Tensor]:
    """Packed mask ``[B, ceil(n/64)]`` int64 → ``(ids [B, n] int64, counts [B] int64)``: row
    ``b``'s set items in ascending order on ``[0, counts[b])``; the tail is not written."""
    if mask.dtype != torch.int64 or mask.dim() != 2 or mask.shape[1] != (n + 63) // 64:
        raise ValueError(f"mask must be [B, ceil(n/64)] int64 for n={n}")
    return _mask_compact(mask.contiguous(), n)


@mask_compact.register_fake
def _(mask, n):
    b = mask.shape[0]
    return mask.new_empty((b, n), dtype=torch.int64), mask.new_empty((b,), dtype=torch.int64)


@torch.library.custom_op("retrieve::clause_compact", mutates_args=(), device_types="cuda")
def clause_compact(
    item_clause_attrs: Tensor, clause_is_reverse: Tensor, query_clause_attrs: Tensor
) -> tuple[Tensor, Tensor]:
    """Clause evaluation + compaction → ``(positive_indices [B, N] int64, counts [B] int64)``
    (``ops/triton/clause_compact.py:174-187``): row ``b``'s passing items in ascending order on
    ``[0, counts[b])``; the tail is not written."""
    rev, q = _clause_prep(item_clause_attrs, clause_is_reverse, query_clause_attrs)
    b, n = q.shape[0], item_clause_attrs.shape[0]
    bits = torch.empty((b, (n + 63) // 64), dtype=torch.int64, device=query_clause_attrs.device)
    _clause_filter(item_clause_attrs, rev, q, _CLAUSE_BITS, bits)
    return _mask_compact(bits, n)


@clause_compact.register_fake
def _(item_clause_attrs, clause_is_reverse, query_clause_attrs):
    b, n = query_clause_attrs.shape[0], item_clause_attrs.shape[0]
    return (
        query_clause_attrs.new_empty((b, n), dtype=torch.int64),
        query_clause_attrs.new_empty((b,), dtype=torch.int64),
    )


# --- candidate lists: gather + score + top-k ----------------------------------------------------

_CAND_KIND = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _cand_check(positive_indices: Tensor, counts: Tensor, b: int) -> Tensor:
    if positive_indices.dim() != 2 or positive_indices.shape[0] != b:
        raise ValueError(f"positive_indices must be [B, P] with B={b}")
    if counts.dim() != 1 or counts.shape[0] != b:
        raise ValueError(f"counts must be [B] with B={b}")
    if positive_indices.dtype != torch.int64:
        raise TypeError("positive_indices must be int64")
    _check_items(positive_indices=positive_indices)
    return counts.to(torch.int64).contiguous()


def _cand_topk(q: Tensor, items: Tensor, d: int, kind: int, positive_indices: Tensor,
               counts: Tensor, k: int, score_dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    b, p = positive_indices.shape
    dev = nat.require_device(q, items, positive_indices, counts)
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=score_dtype, device=dev)
    if b == 0:
        return ids, scores
    lib = nat.lib()
    ws = nat.workspace(lib.rt_cand_topk_workspace(b, p, k), dev)
    with torch.cuda.device(dev):
        st = lib.rt_cand_topk(
            nat.ptr(q), b, nat.ptr(items), items.shape[0], d, kind, nat.ptr(positive_indices), p,
            nat.ptr(counts), k, nat.ptr(ids), nat.ptr(scores), nat.ptr(ws), ws.numel(),
            nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@torch.library.custom_op("retrieve::fused_masked_knn_topk", mutates_args=(), device_types="cuda")
def fused_masked_knn_topk(
    query: Tensor, item_embs: Tensor, positive_indices: Tensor, counts: Tensor, k: int
) -> tuple[Tensor, Tensor]:
    """Top-``k`` of the fp32 dot of ``query [B, D]`` with ``item_embs[positive_indices[b,
    :counts[b]]]`` → ``(ids int64 [B, k], scores fp32 [B, k])``, ties to the lower item id, ``-1``
    where no candidate is left or the score is not finite
    (``ops/triton/fused_masked_knn_topk.py:289-310``). ``P < k`` raises ``ValueError``."""
    if query.dim() != 2 or item_embs.dim() != 2:
        raise ValueError("query must be [B, D] and item_embs [N, D]")
    if query.dtype not in _CAND_KIND or item_embs.dtype not in _CAND_KIND:
        raise TypeError("query and item_embs must be float16, bfloat16 or float32, "
                        f"got {query.dtype} and {item_embs.dtype}")
    if query.shape[1] != item_embs.shape[1]:
        raise ValueError(f"D mismatch: query D={query.shape[1]} vs item D={item_embs.shape[1]}")
    if positive_indices.dim() == 2 and positive_indices.shape[1] < k:
        raise ValueError(
            f"positive_indices has {positive_indices.shape[1]} columns, fewer than k={k}")
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    _check_items(item_embs=item_embs)
    counts = _cand_check(positive_indices, counts, query.shape[0])
    q = query.to(torch.float32).contiguous()
    return _cand_topk(q, item_embs, query.shape[1], _CAND_KIND[item_embs.dtype],
                      positive_indices, counts, k, torch.float32)


@fused_masked_knn_topk.register_fake
def _(query, item_embs, positive_indices, counts, k):
    b = query.shape[0]
    return (query.new_empty((b, k), dtype=torch.int64),
            query.new_empty((b, k), dtype=torch.float32))


@torch.library.custom_op(
    "retrieve::oporp_1bit_match_topk_indirect", mutates_args=(), device_types="cuda"
)
def oporp_1bit_match_topk_indirect(
    query_bits: Tensor, item_bits: Tensor, k: int, positive_indices: Tensor, counts: Tensor
) -> tuple[Tensor, Tensor]:
    """Hamming top-``k`` over ``positive_indices[b, :counts[b]]`` only
    (``ops/triton/oporp_1bit_match_topk.py:274-292``): score ``64 W - 2 popcount`` as fp32,
    ``min(k, P)`` columns (no pad tail), ties to the lower item id."""
    if query_bits.dim() != 2 or item_bits.dim() != 2:
        raise ValueError("query_bits must be [B, W] and item_bits [N, W]")
    if query_bits.dtype != torch.int64 or item_bits.dtype != torch.int64:
        raise TypeError("query_bits and item_bits must be int64")
    if query_bits.shape[1] != item_bits.shape[1]:
        raise ValueError(f"W mismatch: query_bits W={query_bits.shape[1]} vs item_bits "
                         f"W={item_bits.shape[1]}")
    _check_items(item_bits=item_bits)
    counts = _cand_check(positive_indices, counts, query_bits.shape[0])
    kk = min(k, positive_indices.shape[1])
    if k < 1 or kk > 1024:
        raise ValueError(f"k must be >= 1 and min(k, P) <= 1024, got k={k}")
    b = query_bits.shape[0]
    if kk == 0:
        return (query_bits.new_empty((b, 0), dtype=torch.int64),
                query_bits.new_empty((b, 0), dtype=torch.float32))
    return _cand_topk(query_bits.contiguous(), item_bits, query_bits.shape[1], 4,
                      positive_indices, counts, kk, torch.float32)


@oporp_1bit_match_topk_indirect.register_fake
def _(query_bits, item_bits, k, positive_indices, counts):
    kk = min(k, positive_indices.shape[1])
    b = query_bits.shape[0]
    return (query_bits.new_empty((b, kk), dtype=torch.int64),
            query_bits.new_empty((b, kk), dtype=torch.float32))


@torch.library.custom_op("retrieve_amd::int8_candidates_topk", mutates_args=(), device_types="cuda")
def int8_candidates_topk(
    query_codes: Tensor, item_codes: Tensor, positive_indices: Tensor, counts: Tensor, k: int
) -> tuple[Tensor, Tensor]:
    """Exact int8 re-rank of given ids: int32 dots of ``query_codes [B, D]`` with
    ``item_codes[positive_indices[b, :counts[b]]]``, top ``min(k, P)`` by (score desc, item id
    asc) → ``(ids int64, scores int32)``, ``-1`` / ``INT32_MIN`` past a row's candidates (the
    selection of ``modules/silvertorch.py:363-379``, before its fp32 scaling)."""
    if query_codes.dim() != 2 or item_codes.dim() != 2:
        raise ValueError("query_codes must be [B, D] and item_codes [N, D]")
    if query_codes.dtype != torch.int8 or item_codes.dtype != torch.int8:
        raise TypeError("query_codes and item_codes must be int8")
    if query_codes.shape[1] != item_codes.shape[1]:
        raise ValueError("D mismatch between query_codes and item_codes")
    _check_items(item_codes=item_codes)
    counts = _cand_check(positive_indices, counts, query_codes.shape[0])
    kk = min(k, positive_indices.shape[1])
    if k < 1 or kk > 1024:
        raise ValueError(f"k must be >= 1 and min(k, P) <= 1024, got k={k}")
    b = query_codes.shape[0]
    if kk == 0:
        return (query_codes.new_empty((b, 0), dtype=torch.int64),
                query_codes.new_empty((b, 0), dtype=torch.int32))
    return _cand_topk(query_codes.contiguous(), item_codes, query_codes.shape[1], 3,
                      positive_indices, counts, kk, torch.int32)


@int8_candidates_topk.register_fake
def _(query_codes, item_codes, positive_indices, counts, k):
    kk = min(k, positive_indices.shape[1])
    b = query_codes.shape[0]
    return (query_codes.new_empty((b, kk), dtype=torch.int64),
            query_codes.new_empty((b, kk), dtype=torch.int32))


# --- B = 1 dense scores in cuBLAS gemv2N order ---------------------------------------------------


@torch.library.custom_op("retrieve::gemv_scores", mutates_args=(), device_types="cuda")
def gemv_scores(query: Tensor, item_embs_t: Tensor) -> Tensor:
    """``query [1, D]`` fp16 against ``item_embs_t [D, N]`` fp16 (contiguous) → ``[1, N]`` fp32,
    one fp32 FMA per k in order (``ops/triton/gemv_scores.py:31-43``)."""
    if query.dim() != 2 or query.shape[0] != 1 or query.dtype != torch.float16 or \
            item_embs_t.dtype != torch.float16 or item_embs_t.dim() != 2 or \
            item_embs_t.shape[0] != query.shape[1]:
        raise ValueError("gemv_scores takes one fp16 query row and an fp16 [D, N] table")
    _check_items(item_embs_t=item_embs_t)
    d, n = item_embs_t.shape
    q = query.contiguous()
    dev = nat.require_device(q, item_embs_t)
    out = torch.empty((1, n), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        st = nat.lib().rt_gemv_scores(nat.ptr(q), nat.ptr(item_embs_t), d, n, nat.ptr(out),
                                      nat.stream(dev))
    nat.check(st)
    return out


@gemv_scores.register_fake
def _(query, item_embs_t):
    return query.new_empty((1, item_embs_t.shape[1]), dtype=torch.float32)


# --- the reference's per-row quantization and bool masks for the scans ---------------------------


@torch.library.custom_op("retrieve_amd::quantize_int8", mutates_args=(), device_types="cuda")
def quantize_int8(embs: Tensor) -> tuple[Tensor, Tensor]:
    """Per-row symmetric int8 codes and scales (``retrieve/src/retrieve/indexing/quantize.py:
    9-18``): ``abs_max = clamp(max |x|, 1e-8)``, ``scale = abs_max / 127``,
    ``code = clamp(round(fp32(fp64(x) / fp64(abs_max)) * 127), -128, 127)``."""
    if embs.dim() != 2:
        raise ValueError(f"embs must be [N, D], got {tuple(embs.shape)}")
    from retrieve_amd import st

    return st.quantize_rows(embs, scale_div=True)


@quantize_int8.register_fake
def _(embs):
    return (embs.new_empty(embs.shape, dtype=torch.int8),
            embs.new_empty(embs.shape[:1], dtype=torch.float32))


@torch.library.custom_op("retrieve_amd::pack_mask", mutates_args=(), device_types="cuda")
def pack_mask(valid: Tensor) -> Tensor:
    """``[B, N]`` bool → ``[B, ceil(N/64)]`` int64 words, item ``d`` at bit ``63 - d % 64``: the
    mask form of the fused scans (``int8_scan_topk``, ``dense_scan_topk``,
    ``hamming_scan_topk``)."""
    if valid.dim() != 2 or valid.dtype != torch.bool:
        raise ValueError("valid must be a [B, N] bool tensor")
    v = valid.contiguous()
    dev = nat.require_device(v)
    b, n = v.shape
    out = torch.empty((b, (n + 63) // 64), dtype=torch.int64, device=dev)
    if b and n:
        with torch.cuda.device(dev):
            st = nat.lib().rt_pack_mask(nat.ptr(v), b, n, nat.ptr(out), nat.stream(dev))
        nat.check(st)
    return out


@pack_mask.register_fake
def _(valid):
    return valid.new_empty((valid.shape[0], (valid.shape[1] + 63) // 64), dtype=torch.int64)


@torch.library.custom_op("retrieve_amd::pack_signs", mutates_args=(), device_types="cuda")
def pack_signs(values: Tensor) -> Tensor:
    """``[R, D]`` floats → ``[R, D // 64]`` int64, bit ``b`` of word ``w`` set iff ``values[:,
    64 w + b] > 0`` (``_pack_signs_to_int64``, ``retrieve/src/retrieve/indexing/quantize.py:
    63-72``). fp16 / bf16 inputs are widened to fp32 first (exact, so the signs are kept)."""
    if values.dim() != 2:
        raise ValueError(f"values must be [R, D], got {tuple(values.shape)}")
    if not values.is_floating_point():
        raise TypeError(f"values must be floating point, got {values.dtype}")
    r, d = values.shape
    if d % 64:
        raise ValueError(f"D must be a multiple of 64, got {d}")
    v = values.to(torch.float32).contiguous()
    dev = nat.require_device(v)
    out = torch.empty((r, d // 64), dtype=torch.int64, device=dev)
    if out.numel():
        with torch.cuda.device(dev):
            st = nat.lib().rt_pack_signs(nat.ptr(v), r, d, nat.ptr(out), nat.stream(dev))
        nat.check(st)
    return out


@pack_signs.register_fake
def _(values):
    return values.new_empty((values.shape[0], values.shape[1] // 64), dtype=torch.int64)


@torch.library.custom_op("retrieve_amd::quantize_int8_global", mutates_args=(), device_types="cuda")
def quantize_int8_global(embs: Tensor, rows: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """One global int8 scale (``quantize_int8_global``, ``retrieve/src/retrieve/indexing/
    quantize.py:25-52``): ``abs_max = max(max |x|, 1e-8)``, codes ``clamp(round(x / abs_max *
    127), -128, 127)`` in fp32, row ``i`` from row ``rows[i]`` when given → ``(codes int8
    [N, D], abs_max float32 [1])``; the scale is ``abs_max / 127``."""
    if embs.dim() != 2 or embs.dtype != torch.float32:
        raise ValueError("embs must be a float32 [N, D] tensor")
    x = embs.contiguous()
    dev = nat.require_device(x)
    n, d = x.shape
    perm = None
    if rows is not None:
        if rows.dtype != torch.int64 or rows.shape != (n,):
            raise ValueError("rows must be an int64 [N] permutation")
        perm = rows.to(dev).contiguous()
        # (a build-time op: one host check keeps every row the kernel reads inside the table)
        if n and (int(perm.min()) < 0 or int(perm.max()) >= n):
            raise IndexError(f"rows must lie in [0, {n})")
    codes = torch.empty((n, d), dtype=torch.int8, device=dev)
    abs_max = torch.empty((1,), dtype=torch.float32, device=dev)
    scratch = torch.empty((1,), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        st = nat.lib().rt_quantize_int8_global(
            nat.ptr(x), n, max(d, 1), nat.ptr(perm) if perm is not None else None,
            nat.ptr(codes), nat.ptr(abs_max), nat.ptr(scratch), nat.stream(dev))
    nat.check(st)
    return codes, abs_max


@quantize_int8_global.register_fake
def _(embs, rows=None):
    return embs.new_empty(embs.shape, dtype=torch.int8), embs.new_empty((1,))


@torch.library.custom_op("retrieve_amd::int8_rerank_topk", mutates_args=(), device_types="cuda")
def int8_rerank_topk(
    query_codes: Tensor, query_scales: Tensor, item_codes: Tensor, item_rows: Tensor,
    global_scale: Tensor, candidate_ids: Tensor, k: int
) -> tuple[Tensor, Tensor]:
    """SilverTorch's re-rank of original ids (``modules/silvertorch.py:363-379``): candidate
    ``c`` (``-1`` = padding, never read or returned) is ``item_codes[item_rows[c]]``, scored as
    ``(float(dot) * query_scales[b]) * global_scale``; the top ``min(k, P)`` by (score desc, id
    asc) → ``(ids int64, scores fp32)``, ``-1`` / ``-inf`` past a row's candidates."""
    if query_codes.dim() != 2 or item_codes.dim() != 2 or candidate_ids.dim() != 2:
        raise ValueError("query_codes [B, D], item_codes [N, D], candidate_ids [B, P] expected")
    if query_codes.dtype != torch.int8 or item_codes.dtype != torch.int8:
        raise TypeError("query_codes and item_codes must be int8")
    if candidate_ids.dtype != torch.int64 or item_rows.dtype != torch.int64:
        raise TypeError("candidate_ids and item_rows must be int64")
    b, d = query_codes.shape
    n = item_codes.shape[0]
    if item_codes.shape[1] != d or candidate_ids.shape[0] != b or query_scales.shape != (b,) \
            or item_rows.shape != (n,) or global_scale.numel() != 1:
        raise ValueError("shape mismatch among query_codes, query_scales, item_codes, "
                         "item_rows, global_scale and candidate_ids")
    _check_items(item_codes=item_codes, item_rows=item_rows)
    p = candidate_ids.shape[1]
    kk = min(k, p)
    if k < 1 or kk > 1024:
        raise ValueError(f"k must be >= 1 and min(k, P) <= 1024, got k={k}")
    q = query_codes.contiguous()
    dev = nat.require_device(q, item_codes, item_rows, candidate_ids)
    ids = torch.empty((b, kk), dtype=torch.int64, device=dev)
    scores = torch.empty((b, kk), dtype=torch.float32, device=dev)
    if b == 0 or kk == 0:
        return ids, scores
    cand = candidate_ids.contiguous()
    qs = query_scales.to(torch.float32).contiguous()
    gs = global_scale.to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    counts = torch.full((b,), p, dtype=torch.int64, device=dev)
    lib = nat.lib()
    ws = nat.workspace(lib.rt_cand_topk_workspace(b, p, kk), dev)
    with torch.cuda.device(dev):
        st = lib.rt_int8_rerank_topk(
            nat.ptr(q), nat.ptr(qs), b, nat.ptr(item_codes), n, d, nat.ptr(item_rows), nat.ptr(gs),
            nat.ptr(cand), p, nat.ptr(counts), kk, nat.ptr(ids), nat.ptr(scores), nat.ptr(ws),
            ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return ids, scores


@int8_rerank_topk.register_fake
def _(query_codes, query_scales, item_codes, item_rows, global_scale, candidate_ids, k):
    kk = min(k, candidate_ids.shape[1])
    b = query_codes.shape[0]
    return (query_codes.new_empty((b, kk), dtype=torch.int64),
            query_codes.new_empty((b, kk), dtype=torch.float32))
