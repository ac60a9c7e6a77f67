"""The reference's retrieval modules (``retrieve/src/retrieve/modules/*.py``) composed from the
fused HIP ops: the same classes, constructors, ``register_index`` / ``prepare_queries`` /
``forward`` signatures, buffer names and outputs, with each score-then-select pair replaced by
one fused scan or candidate kernel, so no ``[B, N]`` score matrix is written.

- LiNR: ``ExactAttributeFilter``, ``PostfilterKNN``, ``PrefilterKNN``, ``FullScanKNN``, ``OneBitKNN``,
  ``SimHashKNN``, ``LiNRV1`` / ``LiNRV2`` / ``LiNRV3``, ``LiNRBuilder``.
- SilverTorch: ``SilverTorch`` (IVF + int8 with a none / bloom / exact filter),
  ``SilverTorchBuilder``, ``OfficialConfig``, ``PreparedFilter``.

Every forward runs on the HIP library; constructing a module loads it and raises if it is
missing. Build-time work (k-means, the global int8 codes, the 1-bit projections' matrix
products, the IVF layout) is torch on the same device, as the reference's is. Ties go to the
lower item id everywhere (the reference's ``torch.topk`` leaves their order unspecified).
"""

from __future__ import annotations

import abc
import math
import time
from dataclasses import dataclass
from typing import NamedTuple

import torch
from torch import Tensor, nn

from retrieve_amd import _native as nat
from retrieve_amd import bloom as _bloom
from retrieve_amd import hip as _hip  # registers torch.ops.retrieve.* / retrieve_amd.*
from retrieve_amd import st as _st  # registers torch.ops.st.*

ops = torch.ops.retrieve  # the reference's seven ops
xops = torch.ops.retrieve_amd  # the fused scans, masks, re-ranks and packing this build adds

__all__ = [
    "ExactAttributeFilter",
    "FilterModule",
    "FullScanKNN",
    "KMeans",
    "LiNRBuilder",
    "LiNRV1",
    "LiNRV2",
    "LiNRV3",
    "OfficialConfig",
    "OneBitKNN",
    "PostfilterKNN",
    "PrefilterKNN",
    "PreparedFilter",
    "RetrievalModule",
    "SilverTorch",
    "SilverTorchBuilder",
    "SimHashKNN",
]

_BACKENDS = ("hip",)
_CODE_CHUNK_ROWS = 1 << 16  # build-time chunk of rows (quantization, projections)


def _check_backend(backend: str, allowed=_BACKENDS) -> None:
    if backend not in allowed:
        raise ValueError(f"unknown backend {backend!r}; expected one of "
                         f"{', '.join(map(repr, allowed))}")
    nat.lib()  # the HIP library, or an error naming why it is missing


def load_prebuilt(module: nn.Module, state_dict: dict[str, Tensor]) -> None:
    """A freshly constructed module takes a saved one's buffers: one buffer per key, shaped and
    placed like the saved tensor, then ``load_state_dict`` so the load hooks re-derive the cached
    scalars (``retrieve/src/retrieve/interfaces.py:58-68``)."""
    for name, t in state_dict.items():
        owner, _, leaf = name.rpartition(".")
        module.get_submodule(owner).register_buffer(leaf, torch.empty_like(t))
    module.load_state_dict(state_dict)


class RetrievalModule(nn.Module, abc.ABC):
    """``construct(k, ...)`` → ``register_index(item_embs, ...)`` → ``forward(query, ...)`` →
    ``(ids int64 [B, k], scores [B, k])`` with ``-1`` / ``-inf`` for "no item"
    (``retrieve/src/retrieve/interfaces.py:71-80``)."""

    k: int

    @abc.abstractmethod
    def register_index(self, item_embs: Tensor, **kwargs) -> None: ...


class FilterModule(nn.Module, abc.ABC):
    """A predicate over the registered items (``interfaces.py:83-122``): ``prepare_queries``
    encodes a batch once; ``evaluate_mask`` / ``evaluate_indices`` / ``evaluate_subset`` /
    ``mask_scores`` evaluate it, and ``mask_bits`` gives the packed ``[B, ceil(N/64)]`` words
    the fused scans take (item ``d`` at bit ``63 - d % 64`` of word ``d // 64``)."""

    @abc.abstractmethod
    def register_index(self, item_clause_attrs: Tensor, *,
                       clause_is_reverse: Tensor | None = None) -> None: ...

    def prepare_queries(self, query_clause_attrs: Tensor) -> Tensor:
        return query_clause_attrs.long().contiguous()

    @abc.abstractmethod
    def evaluate_mask(self, q: Tensor, start: int = 0, end: int | None = None) -> Tensor: ...

    def mask_bits(self, q: Tensor) -> Tensor:
        return xops.pack_mask(self.evaluate_mask(q))

    def evaluate_indices(self, q: Tensor) -> tuple[Tensor, Tensor]:
        bits = self.mask_bits(q)
        return xops.mask_compact(bits, self._n_items())

    def evaluate_subset(self, q: Tensor, candidate_ids: Tensor) -> Tensor:
        return self.evaluate_mask(q).gather(1, candidate_ids)

    def mask_scores(self, scores: Tensor, q: Tensor) -> Tensor:
        return torch.where(self.evaluate_mask(q), scores, float("-inf"))

    def forward(self, q: Tensor) -> Tensor:
        return self.evaluate_mask(q)

    def _n_items(self) -> int:
        raise NotImplementedError


# --- LiNR primitives --------------------------------------------------------------------------


class ExactAttributeFilter(FilterModule):
    """The exact clause filter (``retrieve/src/retrieve/modules/filters.py:14-65``): item ``n``
    passes query ``b`` iff every active clause ``c`` (``q[b, c] != -1``) holds ``q[b, c]`` among
    ``item_clause_attrs[n, c, :]``, XOR ``clause_is_reverse[c]``. Dense masks, packed words,
    masked scores and ascending compactions are one clause kernel each."""

    item_clause_attrs: Tensor  # [N, C, A_max] int64
    clause_is_reverse: Tensor  # [C] bool

    def __init__(self, backend: str = "hip") -> None:
        super().__init__()
        _check_backend(backend)
        self.backend = backend

    def register_index(self, item_clause_attrs: Tensor, *,
                       clause_is_reverse: Tensor | None = None) -> None:
        if item_clause_attrs.dim() != 3:
            raise ValueError("item_clause_attrs must be [N, C, A_max]")
        c = item_clause_attrs.shape[1]
        self.register_buffer("item_clause_attrs", item_clause_attrs.long().contiguous())
        if clause_is_reverse is None:
            clause_is_reverse = torch.zeros(c, dtype=torch.bool, device=item_clause_attrs.device)
        self.register_buffer("clause_is_reverse", clause_is_reverse)

    def _n_items(self) -> int:
        return self.item_clause_attrs.shape[0]

    def evaluate_mask(self, q: Tensor, start: int = 0, end: int | None = None) -> Tensor:
        """``[B, end - start]`` bool over items ``[start, end)`` (a row slice of the table)."""
        return ops.clause_mask(self.item_clause_attrs[start:end], self.clause_is_reverse, q)

    def mask_bits(self, q: Tensor, and_mask: Tensor | None = None) -> Tensor:
        """The packed ``[B, ceil(N/64)]`` words, optionally AND-ed with ``and_mask``."""
        return xops.clause_bits(self.item_clause_attrs, self.clause_is_reverse, q, and_mask)

    def mask_scores(self, scores: Tensor, q: Tensor) -> Tensor:
        return ops.clause_mask_scores(scores, self.item_clause_attrs, self.clause_is_reverse, q)

    def evaluate_indices(self, q: Tensor) -> tuple[Tensor, Tensor]:
        """``(positive_indices [B, N], counts [B])``, ids ascending; the tail past
        ``counts[b]`` is not written."""
        return ops.clause_compact(self.item_clause_attrs, self.clause_is_reverse, q)

    def evaluate_subset(self, q: Tensor, candidate_ids: Tensor) -> Tensor:
        """The predicate over ``candidate_ids [B, P]`` only: the candidates' attrs gathered and
        compared (``functional.py:173-185``), no full-N pass."""
        gathered = self.item_clause_attrs[candidate_ids]  # [B, P, C, A]
        qq = q.long().unsqueeze(1).unsqueeze(-1)
        match = (gathered == qq).any(dim=-1)
        match = match ^ self.clause_is_reverse.view(1, 1, -1)
        return (match | (q.long() == -1).unsqueeze(1)).all(dim=-1)


class PostfilterKNN(RetrievalModule):
    """Dense fp16 scan + optional ``[B, N]`` bool mask + top-k
    (``retrieve/src/retrieve/modules/knn.py:22-76``): one fused ``dense_scan_topk`` launch
    chain, fp32 accumulation, no score matrix. Items live as ``item_embs [N, D]`` fp16; a state
    dict holding the reference's ``item_embs_t [D, N]`` loads by transposing it once."""

    item_embs: Tensor

    def __init__(self, k: int, backend: str = "hip") -> None:
        super().__init__()
        _check_backend(backend)
        self.k = k
        self.backend = backend

    def register_index(self, item_embs: Tensor) -> None:
        self.register_buffer("item_embs", item_embs.to(torch.float16).contiguous())

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        key_t = prefix + "item_embs_t"
        if key_t in state_dict and prefix + "item_embs" not in state_dict:
            state_dict[prefix + "item_embs"] = state_dict.pop(key_t).t().contiguous()
            if "item_embs" not in self._buffers or self.item_embs.shape != \
                    state_dict[prefix + "item_embs"].shape:
                self.register_buffer("item_embs",
                                     torch.empty_like(state_dict[prefix + "item_embs"]))
            self._buffers.pop("item_embs_t", None)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    def score(self, query: Tensor) -> Tensor:
        """``[B, N]`` fp32 scores of every item (a library GEMM; the fused paths never write
        this matrix)."""
        return torch.mm(query.to(torch.float16), self.item_embs.t(), out_dtype=torch.float32)

    def forward_bits(self, query: Tensor, bits: Tensor | None) -> tuple[Tensor, Tensor]:
        """Top-k over the items whose bit is set in the packed ``bits`` (all items if None)."""
        return xops.dense_scan_topk(query.to(torch.float16), self.item_embs, self.k, bits)

    def forward(self, query: Tensor, mask: Tensor | None = None) -> tuple[Tensor, Tensor]:
        bits = None if mask is None else xops.pack_mask(mask)
        return self.forward_bits(query, bits)


class PrefilterKNN(RetrievalModule):
    """Exact rescoring of given candidates (``modules/knn.py:79-122``): ``candidate_ids [B, P]``
    (+ ``counts [B]``) through ``fused_masked_knn_topk``; without candidates, the full fp16
    scan. fp16 items, fp32 scores."""

    item_embs: Tensor

    def __init__(self, k: int, backend: str = "hip") -> None:
        super().__init__()
        _check_backend(backend)
        self.k = k
        self.backend = backend

    def register_index(self, item_embs: Tensor) -> None:
        self.register_buffer("item_embs", item_embs.to(torch.float16).contiguous())

    def forward(self, query: Tensor, candidate_ids: Tensor | None = None,
                counts: Tensor | None = None) -> tuple[Tensor, Tensor]:
        query = query.to(torch.float16)
        if candidate_ids is None:
            return xops.dense_scan_topk(query, self.item_embs, self.k)
        b, p = candidate_ids.shape
        if counts is None:
            counts = torch.full((b,), p, dtype=torch.int64, device=query.device)
        if p < self.k:  # the op needs >= k columns; lanes past counts are never read
            candidate_ids = torch.nn.functional.pad(candidate_ids, (0, self.k - p), value=-1)
        return ops.fused_masked_knn_topk(query, self.item_embs, candidate_ids, counts, self.k)


class FullScanKNN(RetrievalModule):
    """Exhaustive scan + top-k with POST-filter semantics (``modules/knn.py:125-170``).

    - ``mask [B, N]`` bool: the top k over every item first, then the hits that fail the mask
      tombstoned to id ``-1`` with their scores kept (``post_filter_topk``,
      ``functional.py:146-155``): a masked hit is not replaced by the next passing item.
    - ``candidate_ids [B, P]``: re-rank the given ids only; ``-1`` entries are padding, never
      scored or returned; ``min(k, P)`` columns, short rows ending in ``-1`` / ``-inf``.

    Items keep their dtype (fp32, fp16 or bf16) and scores come back in it, as the reference's
    ``query @ item_embs.T`` does; here they are accumulated in fp32 by the fused scan
    (``dense_scan_topk``) or the candidate kernel (``fused_masked_knn_topk``) and rounded once.
    Ties go to the lower item id."""

    item_embs: Tensor

    def __init__(self, k: int) -> None:
        super().__init__()
        self.k = k
        nat.lib()

    def register_index(self, item_embs: Tensor) -> None:
        self.register_buffer("item_embs", item_embs.contiguous())

    def forward(self, query: Tensor, mask: Tensor | None = None,
                candidate_ids: Tensor | None = None) -> tuple[Tensor, Tensor]:
        if query.dtype != self.item_embs.dtype:
            raise RuntimeError(f"expected query and item_embs to have the same dtype, got "
                               f"{query.dtype} and {self.item_embs.dtype}")
        if candidate_ids is not None:
            return self._rerank(query, candidate_ids)
        n = self.item_embs.shape[0]
        if self.k > n:  # torch.topk's own check on the [B, N] scores
            raise RuntimeError(f"selected index k out of range: k={self.k}, N={n}")
        ids, scores = xops.dense_scan_topk(query, self.item_embs, self.k)
        if mask is not None:
            ids = ids.masked_fill(~mask.gather(1, ids), -1)
        return ids, scores.to(query.dtype)

    def _rerank(self, query: Tensor, candidate_ids: Tensor) -> tuple[Tensor, Tensor]:
        b, p = candidate_ids.shape
        valid = candidate_ids >= 0
        # the real ids first, in their order: the candidate kernel reads a prefix of counts[b]
        order = torch.argsort((~valid).to(torch.int8), dim=1, stable=True)
        cand = candidate_ids.gather(1, order)
        if p < self.k:
            cand = torch.nn.functional.pad(cand, (0, self.k - p), value=-1)
        ids, scores = ops.fused_masked_knn_topk(query, self.item_embs, cand, valid.sum(1),
                                                self.k)
        kk = min(self.k, p)
        return ids[:, :kk], scores[:, :kk].to(query.dtype)


# --- 1-bit codes ---------------------------------------------------------------------------


def _pack_rows(x: Tensor, words: int, project) -> Tensor:
    """``project`` ([R, D] → [R, 64 * words] floats) and the sign packing, chunk by chunk."""
    out = torch.empty((x.shape[0], words), dtype=torch.int64, device=x.device)
    for s in range(0, x.shape[0], _CODE_CHUNK_ROWS):
        out[s:s + _CODE_CHUNK_ROWS] = xops.pack_signs(project(x[s:s + _CODE_CHUNK_ROWS]))
    return out


def _oporp_k_bits(d: int, k_bits: int) -> int:
    """``k_bits = 0`` means ``D``; it must divide ``D`` and be a multiple of 64
    (``indexing/quantize.py:86-94``)."""
    k_bits = d if k_bits == 0 else k_bits
    if d % k_bits:
        raise ValueError(f"k_bits must divide D; got k_bits={k_bits}, D={d}")
    if k_bits % 64:
        raise ValueError(f"k_bits (D when 0) must be a multiple of 64, got {k_bits}")
    return k_bits


def _oporp_sketch(x: Tensor, signs: Tensor, perm: Tensor, k_bits: int) -> Tensor:
    """Sign flip, permutation, ``k_bits`` bins summed, L2-normalised
    (``indexing/quantize.py:97-106``): the floats whose signs are the code."""
    r, d = x.shape
    proj = (x * signs.to(x.dtype)).index_select(1, perm)
    binned = proj.view(r, k_bits, d // k_bits).sum(dim=-1)
    return binned / binned.norm(dim=-1, keepdim=True).clamp_min(1e-8)


class _PackedBitsKNN(RetrievalModule):
    """Hamming KNN over packed sign bits, score ``64 W - 2 popcount(q ^ item)``
    (``modules/bit_knn.py:21-81``): the full scan is ``oporp_1bit_match_topk_full``, the
    candidate form ``oporp_1bit_match_topk_indirect``; subclasses produce the bits."""

    item_bits: Tensor

    def __init__(self, k: int, backend: str = "hip") -> None:
        super().__init__()
        _check_backend(backend)
        self.k = k
        self.backend = backend

    @abc.abstractmethod
    def _quantize_index(self, item_embs: Tensor) -> None: ...

    @abc.abstractmethod
    def _project_query(self, query: Tensor) -> Tensor: ...

    def register_index(self, item_embs: Tensor) -> None:
        n = item_embs.shape[0]
        if self.k > n:
            raise ValueError(f"k={self.k} exceeds corpus size N={n}")
        self._quantize_index(item_embs)

    @property
    def d_total(self) -> int:
        return 64 * self.item_bits.shape[1]

    def forward_bits(self, query: Tensor, bits: Tensor | None) -> tuple[Tensor, Tensor]:
        """Full scan restricted to the items set in packed ``bits``: ``(ids, fp32 scores)``,
        ``-1`` / ``-inf`` past the passing items."""
        ids, s = xops.hamming_scan_topk(self._project_query(query), self.item_bits, self.k, bits)
        return ids, torch.where(ids >= 0, s.to(torch.float32), float("-inf"))

    def forward(self, query: Tensor, candidate_ids: Tensor | None = None,
                counts: Tensor | None = None) -> tuple[Tensor, Tensor]:
        qbits = self._project_query(query)
        if candidate_ids is None:
            return ops.oporp_1bit_match_topk_full(qbits, self.item_bits, self.k)
        if counts is None:
            counts = torch.full((candidate_ids.shape[0],), candidate_ids.shape[1],
                                dtype=torch.int64, device=query.device)
        return ops.oporp_1bit_match_topk_indirect(qbits, self.item_bits, self.k, candidate_ids,
                                                  counts)


class OneBitKNN(_PackedBitsKNN):
    """Sign-OPORP 1-bit codes (``modules/bit_knn.py:84-125``, ``indexing/quantize.py:
    109-140``): seeded ±1 signs and a permutation of the ``D`` dimensions, ``k_bits`` bins
    (``0`` = ``D``)."""

    item_bits: Tensor
    oporp_signs: Tensor
    oporp_perm: Tensor

    def __init__(self, k: int, seed: int = 0, backend: str = "hip", k_bits: int = 0) -> None:
        super().__init__(k, backend)
        self.seed = seed
        self.k_bits = k_bits
        self._k_bits_arg = k_bits
        self.register_load_state_dict_post_hook(_rederive_k_bits)

    def _quantize_index(self, item_embs: Tensor) -> None:
        d = item_embs.shape[1]
        self.k_bits = _oporp_k_bits(d, self._k_bits_arg)
        g = torch.Generator(device=item_embs.device)
        g.manual_seed(int(self.seed))
        signs = torch.randint(0, 2, (d,), generator=g, device=item_embs.device,
                              dtype=torch.int8) * 2 - 1
        perm = torch.randperm(d, generator=g, device=item_embs.device)
        bits = _pack_rows(item_embs, self.k_bits // 64,
                          lambda x: _oporp_sketch(x, signs, perm, self.k_bits))
        self.register_buffer("item_bits", bits)
        self.register_buffer("oporp_signs", signs)
        self.register_buffer("oporp_perm", perm)

    def _project_query(self, query: Tensor) -> Tensor:
        if query.dim() != 2:
            raise ValueError(f"expected 2-D [B, D] query, got shape {tuple(query.shape)}")
        k_bits = _oporp_k_bits(query.shape[1], self.k_bits)
        return xops.pack_signs(_oporp_sketch(query, self.oporp_signs, self.oporp_perm, k_bits))


def _rederive_k_bits(module: OneBitKNN, incompatible_keys) -> None:
    if module._k_bits_arg == 0 and hasattr(module, "oporp_signs"):
        module.k_bits = int(module.oporp_signs.shape[0])


class SimHashKNN(_PackedBitsKNN):
    """SimHash codes (``modules/bit_knn.py:132-155``, ``indexing/quantize.py:143-173``):
    ``R [k_bits, D]`` ~ N(0, 1) from a seeded generator, bits = signs of ``x @ R^T``."""

    item_bits: Tensor
    simhash_R: Tensor

    def __init__(self, k: int, k_bits: int, seed: int = 0, backend: str = "hip") -> None:
        super().__init__(k, backend)
        self.k_bits = k_bits
        self.seed = seed

    def _quantize_index(self, item_embs: Tensor) -> None:
        if self.k_bits % 64:
            raise ValueError(f"k_bits must be a multiple of 64, got {self.k_bits}")
        g = torch.Generator(device=item_embs.device).manual_seed(int(self.seed))
        r = torch.randn(self.k_bits, item_embs.shape[1], generator=g, device=item_embs.device)
        self.register_buffer("item_bits", _pack_rows(item_embs, self.k_bits // 64,
                                                     lambda x: x @ r.t()))
        self.register_buffer("simhash_R", r)

    def _project_query(self, query: Tensor) -> Tensor:
        if query.dim() != 2:
            raise ValueError(f"expected 2-D [B, D] query, got shape {tuple(query.shape)}")
        return xops.pack_signs(query @ self.simhash_R.t())


# --- LiNR variants ---------------------------------------------------------------------------


def _k_of(attr: str) -> property:
    return property(lambda self: getattr(self, attr).k,
                    lambda self, k: setattr(getattr(self, attr), "k", int(k)))


def _filter(filter_mod: FilterModule | None) -> FilterModule:
    if filter_mod is None:
        raise ValueError("query or item clause attrs given, but the module has no filter")
    return filter_mod


def _prepare(self, query_clause_attrs: Tensor) -> Tensor:
    return _filter(self.filter).prepare_queries(query_clause_attrs)


def _register_filter(filter_mod, item_clause_attrs, clause_is_reverse) -> None:
    if item_clause_attrs is not None:
        _filter(filter_mod).register_index(item_clause_attrs, clause_is_reverse=clause_is_reverse)


class LiNRV1(RetrievalModule):
    """LiNR V1 (``modules/linr.py:51-79``): dense fp16 scoring with the filter folded in. The
    reference writes ``[B, N]`` scores, masks them and takes ``masked_topk``; here the filter's
    packed words go straight into the fused scan, so failing items are never scored into
    memory."""

    capturable = True
    k = _k_of("idx")

    def __init__(self, k: int, *, filter: FilterModule | None = None,
                 backend: str = "hip") -> None:
        super().__init__()
        self.idx = PostfilterKNN(k=k, backend=backend)
        self.filter = filter
        self.backend = backend

    def register_index(self, item_embs: Tensor, item_clause_attrs: Tensor | None = None,
                       clause_is_reverse: Tensor | None = None) -> None:
        self.idx.register_index(item_embs)
        _register_filter(self.filter, item_clause_attrs, clause_is_reverse)

    prepare_queries = _prepare

    def forward(self, query: Tensor, prepared: Tensor | None = None):
        if prepared is None:
            return self.idx(query)
        return self.idx.forward_bits(query, _filter(self.filter).mask_bits(prepared))


class LiNRV2(RetrievalModule):
    """LiNR V2 (``modules/linr.py:82-109``): the filter's ascending compaction rescored exactly
    by ``PrefilterKNN``."""

    capturable = True
    k = _k_of("idx")

    def __init__(self, k: int, *, filter: FilterModule, backend: str = "hip") -> None:
        super().__init__()
        _filter(filter)
        self.idx = PrefilterKNN(k=k, backend=backend)
        self.filter = filter
        self.backend = backend

    def register_index(self, item_embs: Tensor, item_clause_attrs: Tensor | None = None,
                       clause_is_reverse: Tensor | None = None) -> None:
        self.idx.register_index(item_embs)
        _register_filter(self.filter, item_clause_attrs, clause_is_reverse)

    prepare_queries = _prepare

    def forward(self, query: Tensor, prepared: Tensor):
        cand, counts = self.filter.evaluate_indices(prepared)
        return self.idx(query, candidate_ids=cand, counts=counts)


class LiNRV3(RetrievalModule):
    """LiNR V3 (``modules/linr.py:112-162``): a 1-bit OPORP shortlist of ``candidate_pool``
    items, then exact fp16 rescoring to ``k``. With a filter, the shortlist is the Hamming
    full scan under the filter's packed words: the same items as the reference's compaction
    followed by the indirect Hamming top-k (both keep the best ``candidate_pool`` passing items,
    ties to the lower id), without the ``[B, N]`` id list. Pools above 1024 (the reference's
    default is 5000) are selected by counting the Hamming scores; above 8192 they raise
    ``ValueError``."""

    capturable = True
    k = _k_of("stage2")

    def __init__(self, k: int, *, candidate_pool: int = 5000, seed: int = 0,
                 filter: FilterModule | None = None, backend: str = "hip") -> None:
        super().__init__()
        if k > candidate_pool:
            raise ValueError(f"k={k} exceeds candidate_pool={candidate_pool}")
        _check_pool(candidate_pool)
        self.stage1 = OneBitKNN(k=candidate_pool, seed=seed, backend=backend)
        self.stage2 = PrefilterKNN(k=k, backend=backend)
        self.filter = filter
        self.backend = backend

    def register_index(self, item_embs: Tensor, item_clause_attrs: Tensor | None = None,
                       clause_is_reverse: Tensor | None = None) -> None:
        self.stage1.register_index(item_embs)
        self.stage2.register_index(item_embs)
        _register_filter(self.filter, item_clause_attrs, clause_is_reverse)

    def set_query_params(self, *, candidate_pool: int) -> None:
        if candidate_pool > self.stage1.item_bits.shape[0]:
            raise ValueError(f"candidate_pool={candidate_pool} exceeds N")
        if candidate_pool < self.k:
            raise ValueError(f"candidate_pool={candidate_pool} is below k={self.k}")
        _check_pool(candidate_pool)
        self.stage1.k = int(candidate_pool)

    prepare_queries = _prepare

    def forward(self, query: Tensor, prepared: Tensor | None = None):
        if prepared is None:
            cand, _ = self.stage1(query)
            return self.stage2(query, candidate_ids=cand)
        cand, _ = self.stage1.forward_bits(query, _filter(self.filter).mask_bits(prepared))
        return self.stage2(query, candidate_ids=cand, counts=(cand >= 0).sum(dim=1))


def _check_pool(candidate_pool: int) -> None:
    if candidate_pool > _hip.HAMMING_MAX_K:
        raise ValueError(f"candidate_pool={candidate_pool} exceeds the 1-bit scan's top-k "
                         f"limit of {_hip.HAMMING_MAX_K}")


VARIANTS = {"v1": LiNRV1, "v2": LiNRV2, "v3": LiNRV3}


class LiNRBuilder:
    """``LiNRBuilder("v3", k=100, candidate_pool=800)`` → ``set_item_embeddings`` (+
    ``set_filter``) or ``set_state_dict`` → ``build()`` (``modules/linr.py:168-219``)."""

    def __init__(self, variant: str, **kwargs) -> None:
        self._cls = VARIANTS[variant]
        self._kwargs = kwargs
        self._embs = self._attrs = self._reverse = self._state_dict = self._device = None

    def set_item_embeddings(self, item_embs: Tensor) -> LiNRBuilder:
        self._embs = item_embs
        return self

    def set_filter(self, filter: FilterModule, item_clause_attrs: Tensor | None = None,
                   clause_is_reverse: Tensor | None = None) -> LiNRBuilder:
        self._kwargs["filter"] = filter
        self._attrs, self._reverse = item_clause_attrs, clause_is_reverse
        return self

    def set_backend(self, backend: str) -> LiNRBuilder:
        self._kwargs["backend"] = backend
        return self

    def set_device(self, device) -> LiNRBuilder:
        self._device = device
        return self

    def set_state_dict(self, state_dict: dict[str, Tensor]) -> LiNRBuilder:
        self._state_dict = state_dict
        return self

    def build(self) -> RetrievalModule:
        if (self._embs is None) == (self._state_dict is None):
            raise ValueError("set exactly one of set_item_embeddings / set_state_dict")
        module = self._cls(**self._kwargs)
        if self._state_dict is not None:
            load_prebuilt(module, self._state_dict)
        else:
            module.register_index(self._embs, self._attrs, self._reverse)
        return module if self._device is None else module.to(self._device)


# --- SilverTorch -----------------------------------------------------------------------------

MAX_SEARCH_K = 10  # hash positions per term the Bloom search supports (MAX_K_V2)
FP16_MAX = 65504.0


def default_divisor(d: int) -> int:
    """The smallest power of two ``v`` with ``127^2 * d / v <= 65504``: the fp16 score path's
    divisor (``retrieve/src/retrieve/ops/official/adapter.py:30-35``)."""
    need = (127 * 127 * d) / FP16_MAX
    return 1 << max(0, math.ceil(math.log2(need)))


@dataclass(frozen=True)
class OfficialConfig:
    """SilverTorch's search knobs (``retrieve/src/retrieve/ops/official/__init__.py:72-131``):
    ``score_path`` ``"int32"`` (raw dots, the parity path) or ``"fp16"`` (``fp16(dot /
    divisor)`` keys); the Bloom build (``b_multiplier``, ``build_k``, ``fast_build``,
    ``bloom_width``), the query parse (``n_stored_hashes``, ``max_sub_queries``) and the exact
    ``recheck`` of the Bloom's survivors."""

    score_path: str = "fp16"
    divisor: int | None = None
    b_multiplier: float = 10.0
    build_k: int | None = None
    max_sub_queries: int = 5
    fast_build: bool = False
    n_stored_hashes: int = 7
    bloom_width: str = "configured"
    recheck: bool = True

    def __post_init__(self) -> None:
        if self.score_path not in ("int32", "fp16"):
            raise ValueError(f"score_path must be 'int32' or 'fp16', got {self.score_path!r}")
        if self.divisor is not None and (self.divisor <= 0 or
                                         self.divisor & (self.divisor - 1)):
            raise ValueError(f"divisor must be a positive power of two, got {self.divisor}")
        if not self.b_multiplier > 1.0:
            raise ValueError(f"b_multiplier must be > 1.0, got {self.b_multiplier}")
        if self.n_stored_hashes <= 0:
            raise ValueError(f"n_stored_hashes must be positive, got {self.n_stored_hashes}")
        if self.build_k is not None and not 0 < self.build_k <= MAX_SEARCH_K:
            raise ValueError(f"build_k must be in [1, {MAX_SEARCH_K}], got {self.build_k}")
        if self.max_sub_queries <= 0:
            raise ValueError(f"max_sub_queries must be positive, got {self.max_sub_queries}")
        if self.bloom_width not in ("configured", "upstream"):
            raise ValueError(f"bloom_width must be 'configured' or 'upstream', "
                             f"got {self.bloom_width!r}")

    def divisor_for(self, d: int) -> int:
        if self.score_path == "int32":
            return -1
        return default_divisor(d) if self.divisor is None else int(self.divisor)


DEFAULT_CONFIG = OfficialConfig()


class PreparedFilter(NamedTuple):
    """One batch's filter (``modules/silvertorch.py:21-33``): the int32 ``query_attrs`` of the
    exact filter (the Bloom recheck's), and the Bloom's device plans with the row → plan
    index."""

    query_attrs: Tensor | None = None
    plan_index: Tensor | None = None
    plan_blob: Tensor | None = None
    plan_slots: int = 0
    plan_stack: int = 0


class KMeans:
    """Lloyd's k-means under inner product (``retrieve/src/retrieve/indexing/kmeans.py:16-122``):
    a row joins the centroid of largest ``x . c`` (first on ties); a centroid is its cluster's
    mean (an empty cluster keeps its centroid). Initial centroids: ``n_lists`` distinct rows
    drawn by a CPU generator seeded with ``seed`` ("random"), or D^2 sampling ("kmeans++").
    Cluster sums are float64 one-hot products, so a fit is the same run to run."""

    def __init__(self, n_lists: int, n_iter: int = 10, seed: int = 0,
                 init: str = "random") -> None:
        if init not in ("random", "kmeans++"):
            raise ValueError(f"init must be 'random' or 'kmeans++', got {init!r}")
        self.n_lists, self.n_iter, self.seed, self.init = n_lists, n_iter, seed, init

    def fit(self, embs: Tensor) -> tuple[Tensor, Tensor]:
        g = torch.Generator(device="cpu")
        g.manual_seed(self.seed)
        if self.init == "kmeans++":
            cent = self._plusplus(embs, g)
        else:
            rows = torch.randperm(embs.shape[0], generator=g)[: self.n_lists]
            cent = embs[rows.to(embs.device)].float().clone()
        for _ in range(self.n_iter):
            a = self.assign(embs, cent)
            sums, counts = self._sums(embs, a)
            cent = torch.where((counts > 0).unsqueeze(1),
                               sums / counts.clamp(min=1).unsqueeze(1), cent)
        return cent, self.assign(embs, cent)

    def _plusplus(self, embs: Tensor, g: torch.Generator) -> Tensor:
        x = embs.float()
        n = x.shape[0]
        sq = (x * x).sum(dim=1)
        cent = torch.empty(self.n_lists, x.shape[1], dtype=torch.float32, device=x.device)
        cent[0] = x[int(torch.randint(n, (1,), generator=g)[0])]
        d2 = (sq - 2 * torch.mv(x, cent[0]) + cent[0].dot(cent[0])).clamp_min(0)
        for j in range(1, self.n_lists):
            cum = torch.cumsum(d2, dim=0)
            target = torch.rand((), generator=g).to(x.device) * cum[-1:]
            i = torch.searchsorted(cum, target, right=True).clamp_max(n - 1)[0]
            cent[j] = x[i]
            d2 = torch.minimum(d2, (sq - 2 * torch.mv(x, cent[j]) + cent[j].dot(cent[j]))
                               .clamp_min(0))
        return cent

    def _sums(self, embs: Tensor, a: Tensor) -> tuple[Tensor, Tensor]:
        n, d = embs.shape
        counts = torch.bincount(a, minlength=self.n_lists).to(torch.float32)
        sums = torch.zeros(self.n_lists, d, dtype=torch.float64, device=embs.device)
        width = max(1, min(1 << 14, (1 << 23) // max(1, self.n_lists)))
        for s in range(0, n, width):
            e = min(s + width, n)
            onehot = torch.zeros(self.n_lists, e - s, dtype=torch.float64, device=embs.device)
            onehot.scatter_(0, a[s:e].unsqueeze(0), 1.0)
            sums.addmm_(onehot, embs[s:e].double())
        return sums.float(), counts

    @staticmethod
    def assign(embs: Tensor, cent: Tensor) -> Tensor:
        out = torch.empty(embs.shape[0], dtype=torch.int64, device=embs.device)
        for s in range(0, embs.shape[0], 1 << 14):
            out[s:s + (1 << 14)] = (embs[s:s + (1 << 14)].float() @ cent.t()).argmax(dim=1)
        return out


def csr_layout(assignments: Tensor, n_lists: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Cluster-sorted CSR (``retrieve/src/retrieve/indexing/ivf.py:15-27``): a stable sort, so
    items keep ascending ids inside a cluster → ``(sort_perm, inv_perm, cluster_offsets
    [n_lists + 1], cluster_sizes)``."""
    sizes = torch.bincount(assignments, minlength=n_lists)
    perm = torch.argsort(assignments, stable=True)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), device=perm.device)
    offsets = torch.zeros(n_lists + 1, dtype=torch.int64, device=assignments.device)
    offsets[1:] = sizes.cumsum(0)
    return perm, inv, offsets, sizes


def probe_width(cluster_sizes: Tensor, n_probe: int) -> int:
    """The sum of the ``n_probe`` largest clusters (``indexing/ivf.py:30-35``)."""
    return int(cluster_sizes.topk(n_probe).values.sum().item())


def quantize_int8_global(embs: Tensor, rows: Tensor | None = None) -> tuple[Tensor, float]:
    """One global scale (``retrieve/src/retrieve/indexing/quantize.py:34-52``): ``abs_max =
    max(max x, -min x)`` floored at 1e-8, codes ``clamp(round(x / abs_max * 127))`` in fp32,
    rows written in ``rows`` order when given; returns ``(codes [N, D] int8, abs_max / 127)``.
    GPU tables go through the HIP kernels (``torch.ops.retrieve_amd.quantize_int8_global``); a
    table held on the host (an index built on the CPU) is quantized there with the same
    arithmetic."""
    if embs.is_cuda:
        codes, abs_max = torch.ops.retrieve_amd.quantize_int8_global(
            embs.to(torch.float32), None if rows is None else rows.to(embs.device))
        return codes, float((abs_max / 127.0).item())
    abs_max = torch.maximum(embs.amax(), -embs.amin()).clamp(min=1e-8)
    codes = torch.empty(embs.shape, dtype=torch.int8, device=embs.device)
    for s in range(0, embs.shape[0], _CODE_CHUNK_ROWS):
        chunk = embs[s:s + _CODE_CHUNK_ROWS] if rows is None else \
            embs[rows[s:s + _CODE_CHUNK_ROWS]]
        codes[s:s + _CODE_CHUNK_ROWS] = (chunk / abs_max * 127.0).round().clamp(-128, 127) \
            .to(torch.int8)
    return codes, float((abs_max / 127.0).item())


def fork_clause_attrs(attrs: Tensor) -> tuple[Tensor, Tensor]:
    """``[N, C, A]`` attrs (values in ``[-1, 2^31 - 1]``) → the search's clause-major int32 slot
    table ``[R, N]`` (each doc's values of clause ``c`` descending in rows ``clause_slots[c] ..
    clause_slots[c + 1]``, ``-1`` pads last) and ``clause_slots [C + 1]``
    (``retrieve/src/retrieve/ops/official/adapter.py:68-81``)."""
    if attrs.numel() and (int(attrs.min()) < -1 or int(attrs.max()) > 2**31 - 1):
        raise ValueError("the exact filter takes attr values in [-1, 2**31 - 1]")
    attrs = attrs.sort(dim=2, descending=True).values
    widths = (attrs != -1).sum(dim=2).amax(dim=0)
    slots = torch.cat([attrs[:, c, :w].T for c, w in enumerate(widths.tolist())])
    clause_slots = torch.zeros(attrs.shape[1] + 1, dtype=torch.int64, device=attrs.device)
    clause_slots[1:] = widths.cumsum(0)
    return slots.to(torch.int32).contiguous(), clause_slots


def fork_query_attrs(query_clause_attrs: Tensor) -> Tensor:
    """``[B, C]`` → int32; values outside ``[-1, 2^31 - 1]`` become ``INT32_MIN``, which no doc
    holds (``adapter.py:84-89``)."""
    q = query_clause_attrs.long()
    return torch.where((q >= -1) & (q <= 2**31 - 1), q, -(2**31)).to(torch.int32).contiguous()


class SilverTorch(RetrievalModule):
    """IVF + int8 retrieval with an optional attribute filter
    (``retrieve/src/retrieve/modules/silvertorch.py:36-380``): k-means lists, the items' int8
    codes under one global scale in cluster-sorted order, per-row int8 queries and int32 dots;
    phases 2 and 3 (filter, scoring of the probed lists, top-k, epilogue) are one
    ``torch.ops.st.search`` call. ``filter_mode`` is ``"none"``, ``"bloom"`` (with the exact
    recheck unless ``OfficialConfig.recheck`` is off) or ``"exact"``."""

    capturable = True

    def __init__(self, k: int, n_lists: int, n_probe: int, filter_mode: str = "none",
                 m_bits: int | None = None, k_hash: int | None = None, n_iter: int = 10,
                 seed: int = 0, kmeans_init: str = "random", backend: str = "cuda",
                 official: OfficialConfig | None = None) -> None:
        super().__init__()
        if filter_mode not in ("none", "bloom", "exact"):
            raise ValueError(f"filter_mode must be 'none', 'bloom', or 'exact', "
                             f"got {filter_mode!r}")
        _check_backend(backend, ("cuda", "hip"))
        self.official = official if official is not None else DEFAULT_CONFIG
        if filter_mode == "bloom":
            configured = self.official.bloom_width == "configured"
            if k_hash is None or (m_bits is None and configured):
                raise ValueError("filter_mode='bloom' requires both m_bits and k_hash (m_bits "
                                 "is optional with OfficialConfig(bloom_width='upstream'))")
            if m_bits is not None and (m_bits <= 0 or m_bits & (m_bits - 1) or m_bits % 64):
                raise ValueError(f"m_bits must be a positive power of 2 and a multiple of 64, "
                                 f"got {m_bits}")
            if not 0 < k_hash <= MAX_SEARCH_K:
                raise ValueError(f"k_hash must be in [1, {MAX_SEARCH_K}], got {k_hash}")
            self.m_bits, self.k_hash = (m_bits or 0), k_hash
        else:
            if m_bits is not None or k_hash is not None:
                raise ValueError(f"m_bits/k_hash only apply to filter_mode='bloom', got "
                                 f"filter_mode={filter_mode!r}")
            self.m_bits = self.k_hash = 0
        self.filter_mode = filter_mode
        self.k, self.n_lists, self.n_probe = k, n_lists, n_probe
        self.n_iter, self.seed, self.kmeans_init, self.backend = n_iter, seed, kmeans_init, backend
        self.build_timings: dict[str, float] = {}
        self.register_load_state_dict_post_hook(_rederive_cached_scalars)

    # -- build ---------------------------------------------------------------------------

    def register_index(self, item_embs: Tensor, item_clause_attrs: Tensor | None = None,
                       clause_is_reverse: Tensor | None = None) -> None:
        self._validate(item_embs, item_clause_attrs, clause_is_reverse)
        clock = _clock(item_embs)
        t0 = clock()
        cent, assignments = KMeans(self.n_lists, self.n_iter, self.seed,
                                   self.kmeans_init).fit(item_embs)
        self.register_buffer("centroids", cent)
        t1 = clock()
        perm, inv, offsets, sizes = csr_layout(assignments, self.n_lists)
        self._probe_width = probe_width(sizes, self.n_probe)
        self._check_pool(self.n_probe, self._probe_width)
        t2 = clock()
        codes, gs = quantize_int8_global(item_embs, rows=perm)
        self.register_buffer("item_codes", codes)
        self.register_buffer("global_scale",
                             torch.tensor(gs, dtype=torch.float32, device=item_embs.device))
        self._global_scale_f = gs
        t3 = clock()
        for name, buf in (("cluster_offsets", offsets), ("cluster_sizes", sizes),
                          ("sort_perm", perm), ("inv_perm", inv)):
            self.register_buffer(name, buf)
        self._register_filter(item_clause_attrs, clause_is_reverse, perm)
        t4 = clock()
        self.build_timings = {"kmeans_s": t1 - t0, "assemble_s": t2 - t1,
                              "quantize_s": t3 - t2, "filter_s": t4 - t3}

    def _validate(self, item_embs, item_clause_attrs, clause_is_reverse) -> None:
        if self.filter_mode == "none" and item_clause_attrs is not None:
            raise ValueError("item_clause_attrs requires filter_mode='bloom' or "
                             "filter_mode='exact'")
        if self.filter_mode == "none" and clause_is_reverse is not None:
            raise ValueError("clause_is_reverse requires filter_mode='exact'")
        if self.filter_mode == "exact" and item_clause_attrs is None:
            raise ValueError("filter_mode='exact' requires item_clause_attrs at register_index")
        if self.filter_mode == "bloom" and clause_is_reverse is not None:
            raise ValueError("clause_is_reverse is only used with filter_mode='exact'")
        n = item_embs.shape[0]
        if self.n_lists > n:
            raise ValueError(f"n_lists ({self.n_lists}) cannot exceed N ({n}).")
        if self.n_probe > self.n_lists:
            raise ValueError(f"n_probe ({self.n_probe}) cannot exceed n_lists ({self.n_lists}).")

    def _check_pool(self, n_probe: int, width: int) -> None:
        if width < self.k:
            raise ValueError(f"k={self.k} exceeds the probe pool: the {n_probe} largest "
                             f"clusters hold {width}")

    def set_query_params(self, *, n_probe: int) -> None:
        if n_probe > self.n_lists:
            raise ValueError(f"n_probe ({n_probe}) cannot exceed n_lists ({self.n_lists}).")
        width = probe_width(self.cluster_sizes, n_probe)
        self._check_pool(n_probe, width)
        self.n_probe, self._probe_width = n_probe, width

    def _register_filter(self, item_clause_attrs, clause_is_reverse, perm) -> None:
        device = self.item_codes.device
        attrs = None if item_clause_attrs is None else \
            item_clause_attrs.long()[perm].contiguous()
        if self.filter_mode == "bloom":
            cfg = self.official
            if attrs is None:
                index = torch.empty(0, dtype=torch.int64, device=device)
                offsets = torch.zeros(1, dtype=torch.int64, device=device)
            else:
                fid, fo, fv = _st.attrs_to_features(attrs)
                build_k = cfg.build_k if cfg.build_k is not None else self.k_hash
                if cfg.bloom_width == "configured":
                    index, offsets = torch.ops.st.bloom_index_build_fixed(
                        fid, fo, fv, int(self.m_bits), int(build_k), cfg.fast_build)
                else:
                    index, offsets = torch.ops.st.bloom_index_build(
                        fid, fo, fv, float(cfg.b_multiplier), int(build_k), cfg.fast_build)
            self.register_buffer("bloom_index", index.contiguous())
            self.register_buffer("bundle_b_offsets", offsets.contiguous())
            if attrs is not None and cfg.recheck:
                self._register_exact(attrs, torch.zeros(attrs.shape[1], dtype=torch.bool,
                                                        device=device))
        elif self.filter_mode == "exact":
            if clause_is_reverse is None:
                clause_is_reverse = torch.zeros(attrs.shape[1], dtype=torch.bool, device=device)
            self._register_exact(attrs, clause_is_reverse)

    def _register_exact(self, attrs: Tensor, clause_is_reverse: Tensor) -> None:
        slots, clause_slots = fork_clause_attrs(attrs)
        self.register_buffer("clause_slots", clause_slots)
        self.register_buffer("item_clause_attrs", slots)
        self.register_buffer("clause_is_reverse", clause_is_reverse)

    # -- query ---------------------------------------------------------------------------

    def prepare_queries(self, query_clause_attrs: Tensor) -> PreparedFilter:
        """The batch's filter, once, outside ``forward``: int32 attrs (exact), or the parsed
        Bloom plans uploaded in one copy, one plan per distinct expression."""
        if self.filter_mode == "none":
            raise ValueError("prepare_queries needs filter_mode='bloom' or filter_mode='exact'")
        if self.filter_mode == "exact":
            return PreparedFilter(query_attrs=fork_query_attrs(query_clause_attrs))
        if self.bloom_index.numel() == 0:
            raise RuntimeError("this bloom index was registered without item_clause_attrs, so "
                               "there is nothing to search")
        cfg = self.official
        attrs = query_clause_attrs.long().cpu().numpy()
        if (attrs < -1).any():
            raise ValueError("attribute values must be >= 0 (or -1 inactive)")
        expressions = _bloom.queries_to_expressions(attrs)
        unique = list(dict.fromkeys(expressions))
        at = {e: i for i, e in enumerate(unique)}
        index = torch.tensor([at[e] for e in expressions], dtype=torch.int64)
        blob, slots, stack = _st.prepare_plans(unique, cfg.n_stored_hashes,
                                               query_clause_attrs.device, cfg.max_sub_queries)
        return PreparedFilter(
            query_attrs=fork_query_attrs(query_clause_attrs) if cfg.recheck else None,
            plan_index=index.to(query_clause_attrs.device), plan_blob=blob, plan_slots=slots,
            plan_stack=stack)

    def forward(self, query: Tensor, prepared: PreparedFilter | None = None,
                candidate_ids: Tensor | None = None) -> tuple[Tensor, Tensor]:
        if candidate_ids is not None:
            if prepared is not None:
                raise ValueError("candidate_ids path scores the given candidates without the "
                                 "fused attribute filter; pass prepared OR candidate_ids")
            return self._forward_candidates(query, candidate_ids)
        if self.filter_mode == "none" and prepared is not None:
            raise ValueError("a prepared filter requires filter_mode='bloom' or 'exact'")
        return self._search(query, prepared)

    def _phase1_probe_ids(self, query: Tensor) -> Tensor:
        if self.n_probe == self.n_lists == 1:
            return torch.zeros((query.shape[0], 1), dtype=torch.int64, device=query.device)
        return torch.topk(query @ self.centroids.t(), self.n_probe, dim=1).indices

    def _search(self, query: Tensor, prepared: PreparedFilter | None):
        probe_ids = self._phase1_probe_ids(query)
        kw = {}
        if prepared is not None and self.filter_mode == "bloom":
            kw.update(bloom_index=self.bloom_index, bloom_bundle_b_offsets=self.bundle_b_offsets,
                      plans=prepared.plan_blob, plan_count=prepared.plan_slots,
                      max_stack_size=prepared.plan_stack, query_plan_index=prepared.plan_index,
                      bloom_k=self.k_hash, hash_k=self.official.n_stored_hashes)
        if prepared is not None and prepared.query_attrs is not None:
            kw.update(item_clause_attrs=self.item_clause_attrs, clause_slots=self.clause_slots,
                      clause_is_reverse=self.clause_is_reverse,
                      query_clause_attrs=prepared.query_attrs)
        return torch.ops.st.search(
            query, probe_ids, self.cluster_offsets, self.cluster_sizes, self.item_codes,
            self.sort_perm, self.global_scale, self.k, self._probe_width,
            self.official.divisor_for(self.item_codes.shape[1]), **kw)

    def _forward_candidates(self, query: Tensor, candidate_ids: Tensor):
        """Re-rank original ids (``-1`` = padding): ``min(k, P)`` columns, ``-1`` / ``-inf``
        past a row's candidates (``modules/silvertorch.py:363-379``)."""
        q_codes, q_scales = xops.quantize_int8(query.to(torch.float32))
        return xops.int8_rerank_topk(q_codes, q_scales, self.item_codes, self.inv_perm,
                                    self.global_scale, candidate_ids.to(torch.int64), self.k)


def _rederive_cached_scalars(module: SilverTorch, incompatible_keys) -> None:
    module._global_scale_f = float(module.global_scale.item())
    module._probe_width = probe_width(module.cluster_sizes, module.n_probe)


def _clock(t: Tensor):
    def now() -> float:
        if t.device.type == "cuda":
            torch.cuda.synchronize(t.device)
        return time.perf_counter()
    return now


class SilverTorchBuilder:
    """``SilverTorch``'s keywords → ``set_item_embeddings`` (+ ``set_item_attributes``) or
    ``set_state_dict`` → ``build()`` (``modules/silvertorch.py:413-469``)."""

    def __init__(self, **kwargs) -> None:
        self._kwargs = kwargs
        self._embs = self._attrs = self._reverse = self._state_dict = self._device = None

    def set_item_embeddings(self, item_embs: Tensor) -> SilverTorchBuilder:
        self._embs = item_embs
        return self

    def set_item_attributes(self, item_clause_attrs: Tensor,
                            clause_is_reverse: Tensor | None = None) -> SilverTorchBuilder:
        self._attrs, self._reverse = item_clause_attrs, clause_is_reverse
        return self

    def set_backend(self, backend: str, official: OfficialConfig | None = None):
        self._kwargs.update(backend=backend, official=official)
        return self

    def set_device(self, device) -> SilverTorchBuilder:
        self._device = device
        return self

    def set_state_dict(self, state_dict: dict[str, Tensor]) -> SilverTorchBuilder:
        self._state_dict = state_dict
        return self

    def build(self) -> SilverTorch:
        if (self._embs is None) == (self._state_dict is None):
            raise ValueError("set exactly one of set_item_embeddings / set_state_dict")
        module = SilverTorch(**self._kwargs)
        if self._state_dict is not None:
            load_prebuilt(module, self._state_dict)
        else:
            module.register_index(self._embs, self._attrs, self._reverse)
        return module if self._device is None else module.to(self._device)
