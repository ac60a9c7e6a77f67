"""The ``torch.ops.st.*`` surface (SilverTorch's op namespace) on the HIP library, with the
reference's schemas: the raw scorer ``fused_kmean_ann`` (``+ _with_partial_masks``,
``silvertorch/.../ops/csrc/fused_kmean_ann.cpp:420-460``), the Bloom index build, the expression
parser, the Bloom plan search over every column or over the probed clusters' columns only
(``bloom_indexer.cpp:117-136``, ``expression_query_parser.cpp:457-465``,
``bloom_index_search.cpp:551-601``), ``search`` and ``probe_prep`` (``fork_search.cpp:13-49``).
Every op has a fake (``silvertorch/silvertorch/ops/_fake.py:26-219``), so forwards trace whole
under ``torch.compile``. Importing this module registers them (as loading the reference's
extension does); ``import retrieve_amd`` registers nothing. The reference's loader
(``retrieve/src/retrieve/ops/official/__init__.py:46-54, 161-167``) accepts the namespace: it
holds every one of its ``REQUIRED_OPS``.

The parser's plan bytes are this library's own encoding (``retrieve_amd.bloom``), read only by
the searches here; the index words follow the reference's bundle layout bit for bit.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from retrieve_amd import _native as nat
from retrieve_amd import bloom as bl

DOCS_PER_BUNDLE = 2048
WORDS_PER_BUNDLE = 32
MAX_K = 10  # MAX_K_V2: positions per term
MAX_BUILD_WIDTH = 256  # bits per doc the HIP build supports
MAX_STACK = 64

_LIB = torch.library.Library("st", "FRAGMENT")
_LIB.define(
    "parse_expression_query_batch(str[] expressions, Tensor silvertorch_ks, int bloom_hash_k, "
    "bool return_query_plan=True, int max_sub_queries=5) -> (int, Tensor[])"
)
_LIB.define(
    "bloom_index_build(Tensor feature_ids, Tensor feature_offsets, Tensor feature_values, "
    "float b_multiplier, int k, bool fast_build=False) -> (Tensor, Tensor)"
)
_LIB.define(
    "bloom_index_build_fixed(Tensor feature_ids, Tensor feature_offsets, Tensor feature_values, "
    "int bits_per_doc, int k, bool fast_build=False) -> (Tensor, Tensor)"
)
_LIB.define(
    "bloom_index_search_batch(Tensor bloom_index, Tensor bloom_bundle_b_offsets, "
    "Tensor bloom_query_plans_data, Tensor bloom_query_plans_offsets, int k, int hash_k, "
    "bool return_bool_mask=True) -> Tensor"
)
_LIB.define(
    "bloom_index_search_batch_prepared(Tensor bloom_index, Tensor bloom_bundle_b_offsets, "
    "Tensor plans, int plan_count, int max_stack_size, int k, int hash_k, "
    "bool return_bool_mask=False) -> Tensor"
)


# --- parser ---------------------------------------------------------------------------------


def _parse(expressions, silvertorch_ks, bloom_hash_k, return_query_plan=True, max_sub_queries=5):
    """``(max_stack_size, [plans_data int8, plans_offsets int64 [8 * B]])`` on the CPU;
    ``silvertorch_ks`` is accepted and unused, as upstream (``expression_query_parser.cpp:395``)."""
    max_stack, data, offsets = bl.parse_batch(list(expressions), int(bloom_hash_k),
                                              int(max_sub_queries))
    if not return_query_plan:
        return max_stack, []
    return max_stack, [torch.from_numpy(data.view(np.int8)), torch.from_numpy(offsets)]


_LIB.impl("parse_expression_query_batch", _parse, "CompositeExplicitAutograd")


@torch.library.register_fake("st::parse_expression_query_batch")
def _(expressions, silvertorch_ks, bloom_hash_k, return_query_plan=True, max_sub_queries=5):
    # the parse depends on the strings and ints only: its shapes are the real parse's
    from torch._subclasses.fake_tensor import unset_fake_temporarily

    with unset_fake_temporarily():
        stack, tensors = _parse(expressions, None, bloom_hash_k, return_query_plan,
                                max_sub_queries)
    return stack, [silvertorch_ks.new_empty(t.shape, dtype=t.dtype) for t in tensors]


# --- build ----------------------------------------------------------------------------------


def _features(feature_ids: Tensor, feature_offsets: Tensor, feature_values: Tensor):
    if feature_ids.dim() != 1 or feature_offsets.dim() != 1 or feature_values.dim() != 1:
        raise ValueError("feature_ids, feature_offsets and feature_values must be 1-D")
    c = feature_ids.numel()
    if c == 0 or (feature_offsets.numel() - 1) % c != 0:
        raise ValueError("feature_offsets must hold N * C + 1 entries")
    dev = nat.require_device(feature_ids, feature_offsets, feature_values)
    fid = feature_ids.to(torch.int32).contiguous()
    fo = feature_offsets.to(torch.int64).contiguous()
    fv = feature_values.to(torch.int64).contiguous()
    # the kernels read feature_values[fo[i] : fo[i + 1]]: the ranges must stay inside it
    if int(fo[0].item()) != 0 or int(fo[-1].item()) != fv.numel() or \
            bool((fo[1:] < fo[:-1]).any().item()):
        raise ValueError("feature_offsets must rise from 0 to len(feature_values)")
    return dev, fid, fo, fv, c, (feature_offsets.numel() - 1) // c


def _build(dev, fid, fo, fv, c, n, offsets: Tensor, max_width: int, k: int) -> Tensor:
    total = int(offsets[-1].item()) if offsets.numel() > 1 else 0
    words = torch.empty(total * WORDS_PER_BUNDLE, dtype=torch.int64, device=dev)
    if total == 0:
        return words
    with torch.cuda.device(dev):
        st = nat.lib().rt_bloom_build(
            nat.ptr(fid), c, nat.ptr(fo), nat.ptr(fv), n, nat.ptr(offsets), max_width, k,
            nat.ptr(words), nat.stream(dev),
        )
    nat.check(st)
    return words


def _build_fixed(feature_ids, feature_offsets, feature_values, bits_per_doc, k, fast_build=False):
    """Every bundle ``bits_per_doc`` bits per doc (``bloom_indexer_cuda.cu:942-961``)."""
    dev, fid, fo, fv, c, n = _features(feature_ids, feature_offsets, feature_values)
    if not 1 <= k <= MAX_K:
        raise ValueError(f"k must be in [1, {MAX_K}], got {k}")
    if not k <= bits_per_doc <= MAX_BUILD_WIDTH:
        raise ValueError(f"bits_per_doc must be in [k, {MAX_BUILD_WIDTH}], got {bits_per_doc}")
    nb = -(-n // DOCS_PER_BUNDLE)
    offsets = torch.arange(nb + 1, dtype=torch.int64, device=dev) * int(bits_per_doc)
    return _build(dev, fid, fo, fv, c, n, offsets, int(bits_per_doc), int(k)), offsets


def _build_upstream(feature_ids, feature_offsets, feature_values, b_multiplier, k,
                    fast_build=False):
    """Bundle width ``(int64)((double)(max_terms * k) * b_multiplier)``
    (``bloom_indexer.cpp:52-70``)."""
    if not b_multiplier > 1.0:
        raise RuntimeError("b_multiplier must be greater than 1.0")
    dev, fid, fo, fv, c, n = _features(feature_ids, feature_offsets, feature_values)
    if not 1 <= k <= MAX_K:
        raise ValueError(f"k must be in [1, {MAX_K}], got {k}")
    nb = -(-n // DOCS_PER_BUNDLE)
    max_terms = torch.empty(nb, dtype=torch.int64, device=dev)
    if nb:
        with torch.cuda.device(dev):
            st = nat.lib().rt_bloom_bundle_terms(nat.ptr(fo), n, c, nat.ptr(max_terms),
                                                 nat.stream(dev))
        nat.check(st)
    widths = ((max_terms * int(k)).double() * float(b_multiplier)).to(torch.int64)
    offsets = torch.zeros(nb + 1, dtype=torch.int64, device=dev)
    offsets[1:] = widths.cumsum(0)
    max_width = int(widths.max().item()) if nb else 0
    if max_width > MAX_BUILD_WIDTH:
        raise ValueError(f"a bundle needs {max_width} bits per doc; the build supports "
                         f"{MAX_BUILD_WIDTH}")
    return _build(dev, fid, fo, fv, c, n, offsets, max_width, int(k)), offsets


_LIB.impl("bloom_index_build_fixed", _build_fixed, "CUDA")
_LIB.impl("bloom_index_build", _build_upstream, "CUDA")


@torch.library.register_fake("st::bloom_index_build")
def _(feature_ids, feature_offsets, feature_values, b_multiplier, k, fast_build=False):
    # the words depend on the bundles' term counts: a size known only after the build
    n = (feature_offsets.shape[0] - 1) // feature_ids.shape[0]
    words = torch.library.get_ctx().new_dynamic_size()
    return (feature_values.new_empty((words,), dtype=torch.int64),
            feature_values.new_empty((-(-n // DOCS_PER_BUNDLE) + 1,), dtype=torch.int64))


@torch.library.register_fake("st::bloom_index_build_fixed")
def _(feature_ids, feature_offsets, feature_values, bits_per_doc, k, fast_build=False):
    n = (feature_offsets.shape[0] - 1) // feature_ids.shape[0]
    nb = -(-n // DOCS_PER_BUNDLE)
    return (feature_values.new_empty((nb * bits_per_doc * WORDS_PER_BUNDLE,)),
            feature_values.new_empty((nb + 1,)))


# --- search ---------------------------------------------------------------------------------


def _max_stack(data: np.ndarray, offsets: np.ndarray) -> int:
    """The evaluation stack depth of host-side encoded plans (ops segment walk)."""
    deepest = 1
    for i in range(offsets.size // 8):
        o = offsets[8 * i : 8 * i + 8]
        ops = data[o[0] : o[1]].view(np.uint8)
        ends = data[o[2] : o[3]].view(np.int32)
        depth = 0
        for j, op in enumerate(ops.tolist()):
            if op in (bl.AND, bl.OR):
                depth -= int(ends[j + 1] - ends[j]) - 1
            elif op in (bl.TERM, bl.EMPTY):
                depth += 1
            deepest = max(deepest, depth)
    return deepest


def _bloom_search(bloom_index: Tensor, offsets: Tensor, plan_offsets: Tensor, data: Tensor,
            data_bytes: int, plan_count: int, max_stack: int, k: int, hash_k: int,
            return_bool: bool) -> Tensor:
    dev = nat.require_device(bloom_index, offsets, plan_offsets, data)
    if bloom_index.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("bloom_index and bloom_bundle_b_offsets must be int64")
    nb = offsets.numel() - 1
    cols = nb * WORDS_PER_BUNDLE
    if return_bool:
        out = torch.empty((plan_count, cols * 64), dtype=torch.bool, device=dev)
    else:
        out = torch.empty((plan_count, cols), dtype=torch.int64, device=dev)
    if plan_count == 0 or nb <= 0:
        return out
    lib = nat.lib()
    ws = nat.workspace(lib.rt_bloom_search_workspace(data_bytes, plan_count), dev)
    with torch.cuda.device(dev):
        st = lib.rt_bloom_search(
            nat.ptr(bloom_index), nat.ptr(offsets), nb, nat.ptr(plan_offsets), nat.ptr(data),
            data_bytes, plan_count, max(1, min(int(max_stack), MAX_STACK)), k, hash_k,
            None if return_bool else nat.ptr(out), nat.ptr(out) if return_bool else None,
            nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return out


# A batch's plans are compiled once into the column kernel's programs (the prep pass), and the
# plans that are ANDs of clauses are rewritten over the batch's distinct clauses (the clause
# pass): keyed by the plan blob and the bundle offsets (id and version: an in-place change
# recompiles) and the search parameters, kept until either tensor is freed. Under graph capture
# with nothing kept, the search compiles in its workspace instead.
_COMPILED: dict = {}
MAX_CLAUSES = 128  # the column kernel's LDS beside its two staged bundles
_PROG_MAX_OPS = 2048  # program words per plan (kProgMaxOps)
_AND, _OR, _NOT, _TERM, _EMPTY = bl.AND, bl.OR, bl.NOT, bl.TERM, bl.EMPTY


def _plan_clauses(words: np.ndarray, plan_count: int, b: int, hdr: np.ndarray,
                  prog: np.ndarray):
    """Program plan ``b``'s tree as ``[(terms, negated)]`` (AND of clauses; ``terms`` the
    ordinals of its TERM ops, which number the program's TERM words) or None when it is not of
    that form, and the TERM program words (kind TERM, place push; positions only)."""
    offs = words[: 8 * plan_count].reshape(plan_count, 8)
    data = words[8 * plan_count :].view(np.uint8)
    o = offs[b]
    ops = data[o[0] : o[1]]
    ends = data[o[2] : o[3]].view(np.int32)
    params = data[o[4] : o[5]].view(np.int32)
    pw = prog[b, : hdr[b, 1]]
    is_term = (pw[:, 0] & 3) == 0
    tw0 = pw[is_term, 0] & np.uint32(0xFFFFFFF0)  # kind TERM, place push
    tw1 = pw[is_term, 1]
    ordinal = np.cumsum(ops == _TERM) - 1

    def children(i):
        return params[ends[i] : ends[i + 1]].tolist()

    def or_terms(i):
        if ops[i] == _TERM:
            return [int(ordinal[i])]
        if ops[i] != _OR:
            return None
        out = []
        for ch in children(i):
            got = or_terms(ch)
            if got is None:
                return None
            out += got
        return out

    def clauses(i):
        if ops[i] == _AND:
            out = []
            for ch in children(i):
                got = clauses(ch)
                if got is None:
                    return None
                out += got
            return out
        if ops[i] == _EMPTY:
            return []
        neg = ops[i] == _NOT
        got = or_terms(children(i)[0] if neg else i)
        return None if got is None else [(got, neg)]

    return clauses(ops.size - 1), tw0, tw1


def _term_bits(w0: int, w1: int) -> int:
    """A TERM's positions (program words: byte offsets p * 256) as a mask over a doc's bits."""
    offs = ((w0 >> 4) & 0x3FFF, w0 >> 18, w1 & 0x3FFF, (w1 >> 16) & 0x3FFF)
    return sum({1 << (x // 256) for x in offs})


def probe_tables(blob: np.ndarray, plan_count: int, hdr: np.ndarray, prog: np.ndarray):
    """The clause tables of the scans' per-candidate Bloom probe (``rt_scan_topk_bloom_clauses``;
    layout in ``csrc/bloom_prog.h``) as one int64 array: each plan's table offset, then per plan
    a header (matches nothing, chunk count; the clauses in use; the negated ones) and per chunk
    of 64 terms the terms' position bits and, per clause, the chunk's lanes holding its terms.
    None when a plan takes the stack evaluation or is not an AND of at most 64 clauses (an OR of
    terms, a term, or the NOT of either): the probe cannot hold it."""
    words = np.asarray(blob).view(np.int64)
    ones = (1 << 64) - 1
    tables: list = []
    for b in range(plan_count):
        if hdr[b, 0] == 1:  # malformed: matches nothing
            tables.append([1, 0, 0, 0])
            continue
        if hdr[b, 0] != 0:
            return None
        found, tw0, tw1 = _plan_clauses(words, plan_count, b, hdr, prog)
        if found is None or len(found) > 64:
            return None
        terms = [(_term_bits(int(tw0[t]), int(tw1[t])), j)
                 for j, (ts, _) in enumerate(found) for t in ts]
        chunks = -(-len(terms) // 64)
        neg = sum(1 << j for j, (_, n) in enumerate(found) if n)
        table = [chunks << 1, (1 << len(found)) - 1, neg, 0]
        for c in range(chunks):
            tm, cl = [ones] * 64, [0] * 64
            for lane, (bits, j) in enumerate(terms[64 * c : 64 * c + 64]):
                tm[lane] = bits
                cl[j] |= 1 << lane
            table += tm + cl
        tables.append(table)
    head = plan_count + 1
    offs = np.cumsum([head] + [len(t) for t in tables])
    flat = [int(x) for x in offs] + [w for t in tables for w in t]
    return np.array(flat, np.uint64).view(np.int64)


def clause_plans(blob: np.ndarray, plan_count: int, hash_k: int, hdr: np.ndarray,
                 prog: np.ndarray, cap: int = MAX_CLAUSES, min_share: float = 2.0):
    """The clause pass over a batch's compiled plans (``blob`` the prepared int64 words: 8
    offsets a plan, then the data; ``hdr`` int32 ``[P, 4]`` and ``prog`` uint32 ``[P, ops, 2]``
    from ``rt_bloom_compile``). A program plan whose tree is an AND (nested ANDs flattened) of
    clauses -- an OR of terms (nested ORs flattened), a term, or the NOT of either; an EMPTY
    child passes everything -- is rewritten as references to the batch's distinct clauses: the
    same set of stored hash lists, so the same word in every column of any bundle width.
    Returns ``(clause_ptr [C + 1], clause_terms [T, 4], plan_desc [P], plan_refs [R])`` as
    uint32 (the layouts of ``rt_bloom_search_compiled``), or None when no plan has that form,
    the batch has more than ``cap`` distinct clauses, or its clause plans reference fewer than
    ``min_share`` times the distinct clauses' terms. A term's entry is its program word pair
    and the index of its stored hashes in the data (uint64 words): term t of a plan is its t-th
    TERM op, as the compiled program numbers them."""
    words = np.asarray(blob).view(np.int64)
    h64 = words[8 * plan_count :].view(np.uint64)
    slots: dict = {}
    clause_terms: list = []
    desc = np.zeros(plan_count, np.uint32)
    refs: list[int] = []
    for b in range(plan_count):
        if hdr[b, 0] != 0:  # not a program plan (stack path, or no match)
            continue
        found, tw0, tw1 = _plan_clauses(words, plan_count, b, hdr, prog)
        h0 = int(np.uint32(hdr[b, 2])) | (int(hdr[b, 3]) << 32)
        if found is None or len(found) > 0xFFF or len(refs) + len(found) > (1 << 19):
            continue
        first = len(refs)
        for terms, neg in found:
            key = frozenset(tuple(h64[h0 + t * hash_k : h0 + (t + 1) * hash_k].tolist())
                            for t in terms)
            slot = slots.get(key)
            if slot is None:
                slot = slots[key] = len(slots)
                clause_terms.append([(int(tw0[t]), int(tw1[t]), h0 + t * hash_k)
                                     for t in terms])
            refs.append(slot | (0x8000 if neg else 0))
        desc[b] = np.uint32((1 << 31) | (first << 12) | len(found))
    if not slots or len(slots) > cap:
        return None
    # the clause table costs LDS (occupancy) and a barrier: it pays where the clause plans
    # reference each distinct clause's terms min_share times over (a batch of plans that share
    # little runs its programs)
    refs_terms = sum(len(clause_terms[r & 0x7FFF]) for r in refs)
    if refs_terms < min_share * sum(len(c) for c in clause_terms):
        return None
    ptr = np.zeros(len(slots) + 1, np.uint32)
    ptr[1:] = np.cumsum([len(c) for c in clause_terms])
    flat = [t for c in clause_terms for t in c]
    terms = np.array([(w0, w1, h & 0xFFFFFFFF, h >> 32) for w0, w1, h in flat], np.uint64)
    return ptr, terms.astype(np.uint32).reshape(-1, 4), desc, np.array(refs, np.uint32)


def _compiled_plans(offsets: Tensor, plans: Tensor, data: Tensor, plan_count: int,
                    max_stack: int, k: int, hash_k: int):
    """``(programs uint8, the clause tables (one int32 tensor, the tables' offsets, whether
    every plan is a clause plan) or None, n_clauses, whether no plan takes the stack path)``
    for these plans, compiled once (``rt_bloom_compile`` + ``clause_plans``); None
    under graph capture with nothing kept."""
    import weakref

    key = (_tkey(plans), _tkey(offsets), plan_count, max_stack, k, hash_k)
    hit = _COMPILED.get(key)
    if hit is not None or _capturing():
        return hit
    dev = nat.require_device(offsets, plans)
    lib = nat.lib()
    nbytes = lib.rt_bloom_compiled_bytes(plan_count)
    programs = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        nat.check(lib.rt_bloom_compile(
            nat.ptr(offsets), offsets.numel() - 1, nat.ptr(plans), nat.ptr(data),
            data.numel() * 8, plan_count, max_stack, k, hash_k, nat.ptr(programs), nbytes,
            nat.stream(dev)))
    tables, n_clauses, no_stack = None, 0, False
    if min(k, hash_k) <= 4:  # (above, every plan takes the stack path)
        host = programs.cpu().numpy()
        start = -(-plan_count * 16 // 256) * 256
        hdr = host[: plan_count * 16].view(np.int32).reshape(plan_count, 4)
        prog = host[start : start + plan_count * _PROG_MAX_OPS * 8].view(np.uint32)
        found = clause_plans(plans.cpu().numpy(), plan_count, hash_k, hdr,
                             prog.reshape(plan_count, _PROG_MAX_OPS, 2))
        if found is not None:
            n_clauses = int(found[0].size - 1)
            # one int32 tensor: clause_ptr, plan_desc, plan_refs, clause_terms
            parts = [found[0], found[2], found[3], found[1].reshape(-1)]
            at = np.cumsum([0] + [p.size for p in parts])
            tables = (torch.from_numpy(np.concatenate(parts).view(np.int32)).to(dev),
                      tuple(int(x) for x in at[:4]), bool((found[2] >> 31).all()))
        no_stack = bool((hdr[:, 0] != 2).all())  # (status 2: the stack evaluation)
    hit = (programs, tables, n_clauses, no_stack)
    _COMPILED[key] = hit
    for t in (plans, offsets):
        weakref.finalize(t, _COMPILED.pop, key, None)
    return hit


_PROBES: dict = {}


def _probe_tables(offsets: Tensor, plans: Tensor, plan_count: int, max_stack: int, k: int,
                  hash_k: int):
    """``probe_tables`` of these plans on the device, built once (False when the probe cannot
    hold them); None under graph capture with nothing kept."""
    import weakref

    key = (_tkey(plans), _tkey(offsets), plan_count, max_stack, k, hash_k)
    hit = _PROBES.get(key)
    if hit is not None or _capturing():
        return hit
    compiled = _compiled_plans(offsets, plans, plans[8 * plan_count:], plan_count, max_stack, k,
                               hash_k)
    tables = False
    if min(k, hash_k) <= 4:
        host = compiled[0].cpu().numpy()
        start = -(-plan_count * 16 // 256) * 256
        hdr = host[: plan_count * 16].view(np.int32).reshape(plan_count, 4)
        prog = host[start : start + plan_count * _PROG_MAX_OPS * 8].view(np.uint32)
        found = probe_tables(plans.cpu().numpy(), plan_count, hdr,
                             prog.reshape(plan_count, _PROG_MAX_OPS, 2))
        if found is not None:
            tables = torch.from_numpy(found).to(offsets.device)
    _PROBES[key] = tables
    for t in (plans, offsets):
        weakref.finalize(t, _PROBES.pop, key, None)
    return tables


def _search_compiled(bloom_index: Tensor, offsets: Tensor, plans: Tensor, data: Tensor,
                     plan_count: int, max_stack: int, k: int, hash_k: int, compiled,
                     out: Tensor, transposed: bool) -> None:
    programs, tables, n_clauses, no_stack = compiled
    dev = bloom_index.device
    lib = nat.lib()
    ptrs, flags = [None] * 4, 2 if no_stack else 0
    if tables is not None:
        base, at = nat.ptr(tables[0]), tables[1]
        ptrs = [base + 4 * a for a in at]  # clause_ptr, plan_desc, plan_refs, clause_terms
        flags |= 1 if tables[2] else 0
    with torch.cuda.device(dev):
        nat.check(lib.rt_bloom_search_compiled(
            nat.ptr(bloom_index), nat.ptr(offsets), offsets.numel() - 1, nat.ptr(plans),
            nat.ptr(data), data.numel() * 8, plan_count, max_stack, k, hash_k,
            nat.ptr(programs), programs.numel(), ptrs[0], ptrs[3], ptrs[1], ptrs[2], n_clauses,
            flags, None if transposed else nat.ptr(out), nat.ptr(out) if transposed else None,
            out.shape[1] if transposed else 0, nat.stream(dev)))


def _search_prepared(bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size, k,
                     hash_k, return_bool_mask=False):
    """Plans prepared once on the device: ``plans`` int64 ``[8 * plan_count + data words]``,
    the offsets then the parser's data (``bloom_index_search_cuda.cu:103-137``). The words
    come from the plans' compiled programs (compiled on the first search of a blob)."""
    if plans.dtype != torch.int64 or plans.dim() != 1 or plans.numel() < 8 * plan_count:
        raise ValueError("plans must be int64 [8 * plan_count + data words]")
    if max_stack_size > MAX_STACK:
        raise ValueError(f"max_stack_size must be <= {MAX_STACK}")
    plans = plans.contiguous()
    data = plans[8 * plan_count :]
    index, offsets = bloom_index.contiguous(), bloom_bundle_b_offsets.contiguous()
    plan_count, max_stack_size, k, hash_k = (int(plan_count), int(max_stack_size), int(k),
                                             int(hash_k))
    nb = offsets.numel() - 1
    if not return_bool_mask and plan_count > 0 and nb > 0:
        nat.require_device(index, offsets, plans)
        if index.dtype != torch.int64 or offsets.dtype != torch.int64:
            raise TypeError("bloom_index and bloom_bundle_b_offsets must be int64")
        compiled = _compiled_plans(offsets, plans, data, plan_count,
                                   max(1, min(max_stack_size, MAX_STACK)), k, hash_k)
        if compiled is not None:
            out = torch.empty((plan_count, nb * WORDS_PER_BUNDLE), dtype=torch.int64,
                              device=index.device)
            _search_compiled(index, offsets, plans, data, plan_count,
                             max(1, min(max_stack_size, MAX_STACK)), k, hash_k, compiled, out,
                             False)
            return out
    return _bloom_search(index, offsets, plans, data, data.numel() * 8, plan_count,
                         max_stack_size, k, hash_k, bool(return_bool_mask))


def _transposed_shape(offsets: Tensor, plan_count: int) -> tuple[int, int]:
    """``(nb * 32 columns, S)``: S = plan_count rounded up to 256 (at least 256)."""
    cols = max(offsets.shape[0] - 1, 0) * WORDS_PER_BUNDLE
    return cols, max(-(-plan_count // 256) * 256, 256)


@torch.library.custom_op("retrieve_amd::bloom_search_cols", mutates_args=(),
                         device_types="cuda")
def bloom_search_cols(bloom_index: Tensor, bloom_bundle_b_offsets: Tensor, plans: Tensor,
                      plan_count: int, max_stack_size: int, k: int, hash_k: int) -> Tensor:
    """The Bloom search's words column-major: ``[nb * 32, S]`` int64, column ``c`` of plan ``b``
    at ``[c, b]`` (``rt_bloom_search_t``); entries ``[:, plan_count:]`` are not written. Use
    ``bloom_search_t`` for the ``[plan_count, nb * 32]`` view."""
    if plans.dtype != torch.int64 or plans.dim() != 1 or plans.numel() < 8 * plan_count:
        raise ValueError("plans must be int64 [8 * plan_count + data words]")
    if max_stack_size > MAX_STACK:
        raise ValueError(f"max_stack_size must be <= {MAX_STACK}")
    bloom_index = bloom_index.contiguous()
    offsets = bloom_bundle_b_offsets.contiguous()
    plans = plans.contiguous()
    dev = nat.require_device(bloom_index, offsets, plans)
    if bloom_index.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("bloom_index and bloom_bundle_b_offsets must be int64")
    data = plans[8 * plan_count :]
    nb = offsets.numel() - 1
    cols, stride = _transposed_shape(offsets, plan_count)
    out = torch.empty((cols, stride), dtype=torch.int64, device=dev)
    if plan_count == 0 or nb <= 0:
        return out
    depth = max(1, min(int(max_stack_size), MAX_STACK))
    compiled = _compiled_plans(offsets, plans, data, int(plan_count), depth, int(k), int(hash_k))
    if compiled is not None:
        _search_compiled(bloom_index, offsets, plans, data, int(plan_count), depth, int(k),
                         int(hash_k), compiled, out, True)
        return out
    lib = nat.lib()
    ws = nat.workspace(lib.rt_bloom_search_workspace(data.numel() * 8, plan_count), dev)
    with torch.cuda.device(dev):
        st = lib.rt_bloom_search_t(
            nat.ptr(bloom_index), nat.ptr(offsets), nb, nat.ptr(plans), nat.ptr(data),
            data.numel() * 8, plan_count, max(1, min(int(max_stack_size), MAX_STACK)), k, hash_k,
            nat.ptr(out), stride, nat.ptr(ws), ws.numel(), nat.stream(dev),
        )
    nat.check(st)
    return out


@bloom_search_cols.register_fake
def _(bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size, k, hash_k):
    return bloom_index.new_empty(_transposed_shape(bloom_bundle_b_offsets, plan_count))


def bloom_search_t(bloom_index: Tensor, bloom_bundle_b_offsets: Tensor, plans: Tensor,
                   plan_count: int, max_stack_size: int, k: int, hash_k: int) -> Tensor:
    """``bloom_index_search_batch_prepared``'s words (``return_bool_mask=False``) stored
    transposed: a ``[plan_count, nb * 32]`` view with strides ``(1, S)`` over ``[nb * 32, S]``
    words, S = plan_count rounded up to 256 (``bloom_search_cols``). The values are the same;
    the blocked scans (``dense_scan_topk_clauses``, ``hamming_scan_topk_clauses`` at their
    blocked batches) read this layout directly instead of transposing the mask per call, and
    any other consumer sees an ordinary strided tensor. (A view of the op's output, so it
    traces under ``torch.compile``.) No counterpart in the reference."""
    return bloom_search_cols(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                             max_stack_size, k, hash_k).t()[:plan_count]


# --- the Bloom pre-filter probed inside the scans -------------------------------------------

_WIDTHS: dict = {}


def _uniform_width(offsets: Tensor) -> int | None:
    """The index's bits per document when every bundle has the same width of 1 to 64, else 0;
    read back once per offsets tensor (None under graph capture with nothing kept)."""
    import weakref

    key = _tkey(offsets)
    hit = _WIDTHS.get(key)
    if hit is not None or _capturing():
        return hit
    width = 0
    if offsets.numel() > 1:
        d = torch.diff(offsets)
        lo, hi = (int(x) for x in torch.stack([d.min(), d.max()]).cpu())
        width = lo if lo == hi and 1 <= lo <= 64 else 0
    _WIDTHS[key] = width
    weakref.finalize(offsets, _WIDTHS.pop, key, None)
    return width


@torch.library.custom_op("retrieve_amd::bloom_doc_bits", mutates_args=(), device_types="cuda")
def bloom_doc_bits(bloom_index: Tensor, bloom_bundle_b_offsets: Tensor, n_docs: int) -> Tensor:
    """Each document's Bloom bits in one int64 word, position ``p`` at bit ``p``
    (``rt_bloom_doc_bits``): the row view of the bit-sliced index, which the scans' per-candidate
    Bloom probe reads (``scan_topk_bloom_clauses``). Every bundle must hold the same 1 to 64
    bits per document (``bloom_index_build_fixed``'s index). Built once per index, beside it; no
    counterpart in the reference."""
    if bloom_index.dtype != torch.int64 or bloom_bundle_b_offsets.dtype != torch.int64:
        raise TypeError("bloom_index and bloom_bundle_b_offsets must be int64")
    index = bloom_index.contiguous()
    offsets = bloom_bundle_b_offsets.contiguous()
    dev = nat.require_device(index, offsets)
    nb = offsets.numel() - 1
    if n_docs < 0 or n_docs > max(nb, 0) * DOCS_PER_BUNDLE:
        raise ValueError(f"n_docs must be in [0, {max(nb, 0) * DOCS_PER_BUNDLE}], got {n_docs}")
    out = torch.empty(n_docs, dtype=torch.int64, device=dev)
    if n_docs == 0:
        return out
    width = _uniform_width(offsets)
    if width is None:
        raise RuntimeError("bloom_doc_bits reads the bundle widths back: build the row bits "
                           "outside graph capture")
    if not width:
        raise ValueError("every bundle must hold the same 1 to 64 bits per document")
    lib = nat.lib()
    with torch.cuda.device(dev):
        nat.check(lib.rt_bloom_doc_bits(nat.ptr(index), nat.ptr(offsets), nb, n_docs, width,
                                        nat.ptr(out), nat.stream(dev)))
    return out


@bloom_doc_bits.register_fake
def _(bloom_index, bloom_bundle_b_offsets, n_docs):
    return bloom_index.new_empty((n_docs,), dtype=torch.int64)


@torch.library.custom_op("retrieve_amd::scan_topk_bloom_clauses", mutates_args=(),
                         device_types="cuda")
def scan_topk_bloom_clauses(
    queries: Tensor, items: Tensor, k: int, item_clause_attrs: Tensor, clause_is_reverse: Tensor,
    query_values: Tensor, bloom_doc_bits: Tensor, bloom_index: Tensor,
    bloom_bundle_b_offsets: Tensor, plans: Tensor, plan_count: int, max_stack_size: int,
    bloom_k: int, hash_k: int,
) -> tuple[Tensor, Tensor]:
    """The filtered top-k under a Bloom pre-filter and the exact clause post-check, the Bloom
    plans probed inside the scan: the same results as ``int8_scan_topk_clauses`` (int8 queries
    and items, int32 scores) or ``dense_scan_topk_clauses`` (bf16 / fp16 / fp32, float scores)
    with ``mask = bloom_index_search_batch_prepared(bloom_index, offsets, plans, plan_count,
    max_stack_size, bloom_k, hash_k)``, plan ``b`` for query ``b``.

    Below the blocked scan's batch, a candidate (an item whose score beats its query's running
    bound) is tested against the clauses, then against its query's plan on the item's row bits
    (``bloom_doc_bits``; the plan's clause table ``probe_tables``, all 64 lanes of a wave
    testing its terms at once): no Bloom mask is written or read, and the index words are not
    read at all (``bloom_index_search_cuda.cu:471-534`` evaluates the same plans column by
    column). Where that does not apply (the blocked batches, fp32, plans that are not an AND of
    at most 64 value-set clauses, bundles of mixed widths, a graph capture before the plans were
    first seen) the op searches the index and scans under its words, as the unfused pair
    does."""
    from retrieve_amd import hip as _hip

    if queries.dim() != 2 or items.dim() != 2 or queries.dtype != items.dtype:
        raise ValueError("queries [B, D] and items [N, D] of one dtype")
    dtype = {torch.int8: 0, torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}.get(
        queries.dtype)
    if dtype is None:
        raise TypeError("queries and items must be int8, bfloat16, float16 or float32")
    if queries.shape[1] != items.shape[1]:
        raise ValueError(f"D mismatch: query D={queries.shape[1]} vs item D={items.shape[1]}")
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    if plans.dtype != torch.int64 or plans.dim() != 1 or plans.numel() < 8 * plan_count:
        raise ValueError("plans must be int64 [8 * plan_count + data words]")
    b, d = queries.shape
    n = items.shape[0]
    if plan_count != b:
        raise ValueError(f"one Bloom plan per query: plan_count {plan_count} != B {b}")
    if bloom_doc_bits.dtype != torch.int64 or bloom_doc_bits.shape != (n,):
        raise ValueError(f"bloom_doc_bits must be int64 [N] = [{n}]")
    _hip._check_items(items=items, bloom_doc_bits=bloom_doc_bits)
    fused = (dtype != 3 and 0 < b and 0 < n and k <= _hip.MAX_FUSED_K
             and not _hip._use_blocked(b, d * queries.element_size(), k))
    tables = None
    if fused:
        offsets = bloom_bundle_b_offsets.contiguous()
        plans = plans.contiguous()
        depth = max(1, min(int(max_stack_size), MAX_STACK))
        tables = _probe_tables(offsets, plans, int(plan_count), depth, int(bloom_k), int(hash_k))
        fused = tables is not None and tables is not False and bool(_uniform_width(offsets))
    if not fused:
        if _hip._use_blocked(b, d * queries.element_size(), k):
            mask = bloom_search_t(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                                  max_stack_size, bloom_k, hash_k)
        else:
            mask = torch.ops.st.bloom_index_search_batch_prepared(
                bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size, bloom_k,
                hash_k)
        op = torch.ops.retrieve_amd.int8_scan_topk_clauses if dtype == 0 else \
            torch.ops.retrieve_amd.dense_scan_topk_clauses
        return op(queries, items, k, item_clause_attrs, clause_is_reverse, query_values, mask)
    rev, qs = _hip._clause_prep(item_clause_attrs, clause_is_reverse, query_values, sets=True)
    if item_clause_attrs.shape[0] != n:
        raise ValueError(f"item_clause_attrs has {item_clause_attrs.shape[0]} rows, the items {n}")
    if qs.shape[0] != b:
        raise ValueError(f"query_values has {qs.shape[0]} rows, the queries {b}")
    q = queries.contiguous()
    dev = nat.require_device(q, items, item_clause_attrs, qs, bloom_doc_bits)
    _, c, a = item_clause_attrs.shape
    v = qs.shape[2]
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.int32 if dtype == 0 else torch.float32, device=dev)
    lib = nat.lib()
    with torch.cuda.device(dev):
        ws = nat.workspace(lib.rt_scan_topk_clauses_workspace(b, n, d, k, c, v), dev)
        nat.check(lib.rt_scan_topk_bloom_clauses(
            nat.ptr(q), b, nat.ptr(items), n, d, k, dtype, nat.ptr(bloom_doc_bits),
            nat.ptr(tables), plan_count, nat.ptr(item_clause_attrs),
            item_clause_attrs.element_size(), c, a, nat.ptr(rev), nat.ptr(qs), v, nat.ptr(ids),
            nat.ptr(scores), nat.ptr(ws), ws.numel(), nat.stream(dev)))
    return ids, scores


@scan_topk_bloom_clauses.register_fake
def _(queries, items, k, item_clause_attrs, clause_is_reverse, query_values, bloom_doc_bits,
      bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size, bloom_k, hash_k):
    b = queries.shape[0]
    return (queries.new_empty((b, k), dtype=torch.int64),
            queries.new_empty((b, k), dtype=torch.int32 if queries.dtype == torch.int8
                              else torch.float32))


def _search_batch(bloom_index, bloom_bundle_b_offsets, bloom_query_plans_data,
                  bloom_query_plans_offsets, k, hash_k, return_bool_mask=True):
    """Plans as the parser returns them (host tensors are copied to the index's device)."""
    dev = bloom_index.device
    data = bloom_query_plans_data.contiguous()
    offs = bloom_query_plans_offsets.to(torch.int64).contiguous()
    if offs.numel() % 8:
        raise ValueError("bloom_query_plans_offsets must hold 8 offsets per plan")
    max_stack = MAX_STACK
    if data.device.type == "cpu" and offs.device.type == "cpu":
        max_stack = _max_stack(data.numpy().view(np.uint8), offs.numpy())
        if max_stack > MAX_STACK:
            raise ValueError(f"plans need a stack of {max_stack} (> {MAX_STACK})")
    nbytes = data.numel()
    # 8-aligned device copy of the data
    dev_data = torch.zeros((nbytes + 7) // 8, dtype=torch.int64, device=dev)
    if nbytes:
        dev_data.view(torch.uint8)[:nbytes].copy_(data.view(torch.uint8).to(dev))
    return _bloom_search(bloom_index.contiguous(), bloom_bundle_b_offsets.contiguous(),
                         offs.to(dev), dev_data, nbytes, offs.numel() // 8, max_stack, int(k),
                         int(hash_k), bool(return_bool_mask))


_LIB.impl("bloom_index_search_batch_prepared", _search_prepared, "CUDA")
_LIB.impl("bloom_index_search_batch", _search_batch, "CUDA")


@torch.library.register_fake("st::bloom_index_search_batch")
def _(bloom_index, bloom_bundle_b_offsets, bloom_query_plans_data, bloom_query_plans_offsets, k,
      hash_k, return_bool_mask=True):
    plans = bloom_query_plans_offsets.shape[0] // 8
    cols = (bloom_bundle_b_offsets.shape[0] - 1) * WORDS_PER_BUNDLE
    if return_bool_mask:
        return bloom_index.new_empty((plans, cols * 64), dtype=torch.bool)
    return bloom_index.new_empty((plans, cols), dtype=torch.int64)


# --- Bloom plans over the probed clusters' columns (bloom_index_search.cpp:219-345, 561-601) ---

_LIB.define(
    "bloom_index_search_batch_return_partial_response(Tensor bloom_index, "
    "Tensor bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
    "Tensor bloom_query_plans_offsets, Tensor selected_cluster_offsets, "
    "Tensor selected_cluster_lengths, int k, int hash_k, Tensor? query_plan_index=None) "
    "-> (Tensor, Tensor, Tensor)"
)
_LIB.define(
    "bloom_index_search_batch_return_partial_response_prepared(Tensor bloom_index, "
    "Tensor bloom_bundle_b_offsets, Tensor plans, int plan_count, int max_stack_size, "
    "Tensor selected_cluster_offsets, Tensor selected_cluster_lengths, int k, int hash_k, "
    "Tensor? query_plan_index, int max_columns) -> (Tensor, Tensor, Tensor)"
)


def _column_info(starts: Tensor, lengths: Tensor, plan_count: int,
                 query_plan_index: Tensor | None) -> tuple[Tensor, Tensor, Tensor]:
    """``(column_counts_cumsum int32 [B·P], first_item_offsets int8 [B·P], starts int64)`` of the
    probed clusters (``generate_column_info_for_clusters``, ``bloom_index_search.cpp:447-490``):
    cluster (q, c) starting ``start % 64`` docs into its first 64-doc column spans
    ``ceil((len + start % 64) / 64)`` columns, none when it is empty."""
    if starts.dim() != 2 or lengths.dim() != 2:
        raise RuntimeError("selected_cluster_offsets and selected_cluster_lengths must be 2-D")
    if starts.dtype != torch.int64 or lengths.dtype != torch.int64:
        raise RuntimeError("selected_cluster_offsets and selected_cluster_lengths must be int64")
    if starts.shape != lengths.shape:
        raise RuntimeError("selected_cluster_offsets must have the shape of "
                           "selected_cluster_lengths")
    if query_plan_index is not None:
        if query_plan_index.dim() != 1 or query_plan_index.shape[0] != starts.shape[0]:
            raise RuntimeError("query_plan_index must be [B]")
    elif plan_count != starts.shape[0]:
        raise RuntimeError("without query_plan_index there must be one plan per row")
    starts = starts.contiguous()
    off = torch.remainder(starts, 64)
    counts = torch.where(lengths > 0, torch.div(lengths + off + 63, 64, rounding_mode="floor"),
                         torch.zeros_like(lengths))
    return (counts.reshape(-1).cumsum(0).to(torch.int32), off.reshape(-1).to(torch.int8),
            starts.reshape(-1))


def _columns(bloom_index, offsets, plan_offsets, data, data_bytes, plan_count, max_stack, k,
             hash_k, starts, cumsum, per_row, query_plan_index, max_columns) -> Tensor:
    dev = nat.require_device(bloom_index, offsets, plan_offsets, data, starts)
    if bloom_index.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("bloom_index and bloom_bundle_b_offsets must be int64")
    out = torch.empty((max_columns,), dtype=torch.int64, device=dev)
    if max_columns == 0:
        return out
    qpi = None if query_plan_index is None else query_plan_index.to(torch.int64).contiguous()
    with torch.cuda.device(dev):
        st = nat.lib().rt_bloom_search_columns(
            nat.ptr(bloom_index), nat.ptr(offsets), offsets.numel() - 1, nat.ptr(plan_offsets),
            nat.ptr(data), data_bytes, plan_count, max(1, min(int(max_stack), MAX_STACK)), k,
            hash_k, nat.ptr(starts), nat.ptr(cumsum), starts.numel(), max(1, per_row),
            nat.ptr(qpi), max_columns, nat.ptr(out), nat.stream(dev))
    nat.check(st)
    return out


def _partial_response(bloom_index, bloom_bundle_b_offsets, bloom_query_plans_data,
                      bloom_query_plans_offsets, selected_cluster_offsets,
                      selected_cluster_lengths, k, hash_k, query_plan_index=None):
    """Plans as the parser returns them; the output's length is the probed columns' total, so
    this form reads it back (as the reference's ``repeat_interleave`` does,
    ``bloom_index_search_cuda.cu:1755-1760``); the ``_prepared`` form does not."""
    dev = bloom_index.device
    offs = bloom_query_plans_offsets.to(torch.int64).contiguous()
    if offs.numel() % 8:
        raise ValueError("bloom_query_plans_offsets must hold 8 offsets per plan")
    data = bloom_query_plans_data.contiguous()
    max_stack = MAX_STACK
    if data.device.type == "cpu" and offs.device.type == "cpu":
        max_stack = _max_stack(data.numpy().view(np.uint8), offs.numpy())
        if max_stack > MAX_STACK:
            raise ValueError(f"plans need a stack of {max_stack} (> {MAX_STACK})")
    plan_count = offs.numel() // 8
    cumsum, first, starts = _column_info(selected_cluster_offsets.to(dev),
                                         selected_cluster_lengths.to(dev), plan_count,
                                         query_plan_index)
    total = int(cumsum[-1].item()) if cumsum.numel() else 0
    nbytes = data.numel()
    dev_data = torch.zeros((nbytes + 7) // 8, dtype=torch.int64, device=dev)
    if nbytes:
        dev_data.view(torch.uint8)[:nbytes].copy_(data.view(torch.uint8).to(dev))
    words = _columns(bloom_index.contiguous(), bloom_bundle_b_offsets.contiguous(), offs.to(dev),
                     dev_data, nbytes, plan_count, max_stack, int(k), int(hash_k), starts, cumsum,
                     selected_cluster_lengths.shape[1], query_plan_index, total)
    return cumsum, first, words


def _partial_response_prepared(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                               max_stack_size, selected_cluster_offsets, selected_cluster_lengths,
                               k, hash_k, query_plan_index, max_columns):
    """Prepared plans, no host sync: ``column_mask_response`` has the caller's static capacity
    ``max_columns``; its words past the probed columns' total are 0
    (``bloom_index_search_cuda.cu:1857-1940``)."""
    if plans.dtype != torch.int64 or plans.dim() != 1 or plans.numel() < 8 * plan_count:
        raise ValueError("plans must be int64 [8 * plan_count + data words]")
    if max_stack_size > MAX_STACK:
        raise ValueError(f"max_stack_size must be <= {MAX_STACK}")
    if max_columns < 0:
        raise ValueError("max_columns must be >= 0")
    plans = plans.contiguous()
    data = plans[8 * plan_count :]
    cumsum, first, starts = _column_info(selected_cluster_offsets, selected_cluster_lengths,
                                         int(plan_count), query_plan_index)
    words = _columns(bloom_index.contiguous(), bloom_bundle_b_offsets.contiguous(), plans, data,
                     data.numel() * 8, int(plan_count), int(max_stack_size), int(k), int(hash_k),
                     starts, cumsum, selected_cluster_lengths.shape[1], query_plan_index,
                     int(max_columns))
    return cumsum, first, words


_LIB.impl("bloom_index_search_batch_return_partial_response", _partial_response, "CUDA")
_LIB.impl("bloom_index_search_batch_return_partial_response_prepared",
          _partial_response_prepared, "CUDA")


@torch.library.register_fake("st::bloom_index_search_batch_return_partial_response")
def _(bloom_index, bloom_bundle_b_offsets, bloom_query_plans_data, bloom_query_plans_offsets,
      selected_cluster_offsets, selected_cluster_lengths, k, hash_k, query_plan_index=None):
    clusters = selected_cluster_lengths.numel()
    columns = torch.library.get_ctx().new_dynamic_size()
    return (bloom_index.new_empty((clusters,), dtype=torch.int32),
            bloom_index.new_empty((clusters,), dtype=torch.int8),
            bloom_index.new_empty((columns,), dtype=torch.int64))


@torch.library.register_fake("st::bloom_index_search_batch_return_partial_response_prepared")
def _(bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size,
      selected_cluster_offsets, selected_cluster_lengths, k, hash_k, query_plan_index,
      max_columns):
    clusters = selected_cluster_lengths.numel()
    return (bloom_index.new_empty((clusters,), dtype=torch.int32),
            bloom_index.new_empty((clusters,), dtype=torch.int8),
            bloom_index.new_empty((max_columns,), dtype=torch.int64))


# --- the raw scorer (fused_kmean_ann.cpp:420-460; fused_kmean_ann_cuda.cu:2126-2501) ---------

_LIB.define(
    "fused_kmean_ann(Tensor cluster_offsets, Tensor cluster_ids, Tensor cluster_length, "
    "Tensor embeddings, Tensor queries, int max_tensor_size_per_row, "
    "Tensor? filtering_bit_mask=None, int invalid_index_value=-1, int divisor_for_int8=-1, "
    "Tensor? filtering_bit_index=None, Tensor? per_embedding_scale=None) -> (Tensor, Tensor)"
)
_LIB.define(
    "fused_kmean_ann_with_partial_masks(Tensor cluster_offsets, Tensor cluster_ids, "
    "Tensor cluster_length, Tensor embeddings, Tensor queries, int max_tensor_size_per_row, "
    "Tensor partial_mask_column_counts_cumsum, Tensor partial_mask_first_item_offset_in_column, "
    "Tensor partial_mask_column_results, int invalid_index_value=-1, int divisor_for_int8=-1, "
    "Tensor? filtering_bit_index=None, Tensor? per_embedding_scale=None, "
    "Tensor? cluster_warp_size=None, Tensor? cluster_warp_rounded_length_cumsum=None, "
    "Tensor? cluster_remaining_length_cumsum=None, Tensor? cluster_warp_size_cumsum=None, "
    "int total_cluster_rounded_warps=0, int total_cluster_remaining_warps=0) -> (Tensor, Tensor)"
)

_ELEM = {torch.int8: 0, torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}


def _score_dtype(emb_dtype, divisor_for_int8, has_scale):
    """int8 rows: int32, or fp16 with a divisor or per-doc scales; else the rows' dtype
    (``fused_kmean_ann.cpp:30-41``)."""
    if emb_dtype != torch.int8:
        return emb_dtype
    return torch.float16 if (divisor_for_int8 != -1 or has_scale) else torch.int32


def _kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
               max_tensor_size_per_row, invalid_index_value, divisor_for_int8,
               filtering_bit_index, per_embedding_scale, mask=None, partial=None,
               f32_scores=False):
    for name, t, dim in (("cluster_offsets", cluster_offsets, 1), ("cluster_ids", cluster_ids, 2),
                         ("cluster_length", cluster_length, 2), ("embeddings", embeddings, 2),
                         ("queries", queries, 2)):
        if t.dim() != dim:
            raise RuntimeError(f"{name} must be {dim}-D")
    if cluster_ids.shape != cluster_length.shape or cluster_ids.shape[0] != queries.shape[0]:
        raise RuntimeError("cluster_ids and cluster_length must be [B, n_probe] with B query rows")
    if embeddings.shape[1] != queries.shape[1]:
        raise RuntimeError("embeddings and queries must have the same D")
    if embeddings.dtype not in _ELEM or queries.dtype != embeddings.dtype:
        raise RuntimeError("embeddings and queries must be int8, bfloat16, float16 or float32 "
                           "of one dtype")
    if not embeddings.is_contiguous():
        raise RuntimeError("embeddings must be contiguous")
    b, p = cluster_ids.shape
    n, d = embeddings.shape
    dev = nat.require_device(cluster_offsets, cluster_ids, cluster_length, embeddings, queries)
    scale = None
    if per_embedding_scale is not None:
        if per_embedding_scale.dim() != 1 or per_embedding_scale.shape[0] != n or \
                per_embedding_scale.dtype != torch.float16:
            raise RuntimeError("per_embedding_scale must be float16 [N]")
        scale = per_embedding_scale.contiguous()
    index = None
    if filtering_bit_index is not None:
        if filtering_bit_index.dim() != 1 or filtering_bit_index.shape[0] != b:
            raise RuntimeError("filtering_bit_index must be [B]")
        index = filtering_bit_index.to(torch.int64).contiguous()
    if mask is not None:
        if mask.dtype != torch.int64 or mask.dim() != 2:
            raise RuntimeError("filtering_bit_mask must be int64 [rows, ceil(N/64)]")
        if index is None and mask.shape[0] != b:
            raise RuntimeError("filtering_bit_mask must have B rows without filtering_bit_index")
        if mask.shape[1] < (n + 63) // 64:
            raise RuntimeError("filtering_bit_mask must cover every doc (ceil(N/64) words)")
        mask = mask.contiguous()
    width = (int(max_tensor_size_per_row) + 31) // 32 * 32
    dtype = _score_dtype(embeddings.dtype, divisor_for_int8, scale is not None)
    elem = _ELEM[embeddings.dtype]
    if f32_scores and embeddings.dtype != torch.int8:
        dtype = torch.float32
        elem += 16
    scores = torch.empty((b, width), dtype=dtype, device=dev)
    idx = torch.empty((b, width), dtype=torch.int32, device=dev)
    cum = first = words = None
    if partial is not None:
        cum, first, words = partial
        if cum.dim() != 1 or first.dim() != 1 or words.dim() != 1 or \
                cum.shape[0] != first.shape[0]:
            raise RuntimeError("the partial masks must be 1-D, the counts and offsets of one "
                               "length")
        if words.dtype != torch.int64 or cum.dtype != torch.int32 or first.dtype != torch.int8:
            raise RuntimeError("partial masks: int32 counts, int8 offsets, int64 words")
        if index is None and first.shape[0] != b * p:
            raise RuntimeError("partial masks must hold one entry per (row, probe)")
        cum, first, words = cum.contiguous(), first.contiguous(), words.contiguous()
    offs = cluster_offsets.to(torch.int64).contiguous()
    ids = cluster_ids.to(torch.int64).contiguous()
    lens = cluster_length.to(torch.int64).contiguous()
    q = queries.contiguous()
    with torch.cuda.device(dev):
        st = nat.lib().rt_fused_kmean_ann(
            nat.ptr(q), nat.ptr(embeddings), elem, b, n, d, nat.ptr(offs),
            offs.numel(), nat.ptr(ids), nat.ptr(lens), p, width, nat.ptr(mask),
            0 if mask is None else mask.shape[0], 0 if mask is None else mask.shape[1],
            nat.ptr(index), nat.ptr(cum), nat.ptr(first), nat.ptr(words),
            0 if first is None else first.numel(), 0 if words is None else words.numel(),
            int(divisor_for_int8), nat.ptr(scale), int(invalid_index_value), nat.ptr(scores),
            nat.ptr(idx), nat.stream(dev))
    nat.check(st)
    return scores, idx


def raw_scores(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
               max_tensor_size_per_row, mask=None, divisor_for_int8=-1):
    """The raw scorer for this package's own callers (the searches' top-k above 1024): every
    probed slot's score (int32 dots, fp16 with a divisor, the fp32 accumulator for float items)
    and its item index (``-1`` for a pad), as ``fused_kmean_ann`` writes them."""
    return _kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                      max_tensor_size_per_row, -1, divisor_for_int8, None, None, mask=mask,
                      f32_scores=True)


def _fused_kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                     max_tensor_size_per_row, filtering_bit_mask=None, invalid_index_value=-1,
                     divisor_for_int8=-1, filtering_bit_index=None, per_embedding_scale=None):
    """``(scores [B, W], indices int32 [B, W])``, ``W`` = ``max_tensor_size_per_row`` rounded up
    to 32: every probed doc scored in its slot (the probes' full 32-doc warps in probe order,
    then their remainders), filtered-out docs and the tail left as pads
    (``fused_kmean_ann_cuda.cu:2126-2262``)."""
    return _kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                      max_tensor_size_per_row, invalid_index_value, divisor_for_int8,
                      filtering_bit_index, per_embedding_scale, mask=filtering_bit_mask)


def _fused_kmean_ann_partial(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                             max_tensor_size_per_row, partial_mask_column_counts_cumsum,
                             partial_mask_first_item_offset_in_column,
                             partial_mask_column_results, invalid_index_value=-1,
                             divisor_for_int8=-1, filtering_bit_index=None,
                             per_embedding_scale=None, cluster_warp_size=None,
                             cluster_warp_rounded_length_cumsum=None,
                             cluster_remaining_length_cumsum=None, cluster_warp_size_cumsum=None,
                             total_cluster_rounded_warps=0, total_cluster_remaining_warps=0):
    """``fused_kmean_ann`` filtered by the probed-column Bloom words of
    ``bloom_index_search_batch_return_partial_response`` (``fused_kmean_ann_cuda.cu:2335-2501``).
    The precomputed warp counts and cumsums are accepted and unused: the kernel derives the slot
    layout from ``cluster_length`` (the totals are ignored upstream too, ``:2459-2460``)."""
    return _kmean_ann(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                      max_tensor_size_per_row, invalid_index_value, divisor_for_int8,
                      filtering_bit_index, per_embedding_scale,
                      partial=(partial_mask_column_counts_cumsum,
                               partial_mask_first_item_offset_in_column,
                               partial_mask_column_results))


_LIB.impl("fused_kmean_ann", _fused_kmean_ann, "CUDA")
_LIB.impl("fused_kmean_ann_with_partial_masks", _fused_kmean_ann_partial, "CUDA")


def _scores_fake(cluster_ids, embeddings, max_tensor_size_per_row, divisor_for_int8, scale):
    width = (max_tensor_size_per_row + 31) // 32 * 32
    rows = cluster_ids.shape[0]
    dtype = _score_dtype(embeddings.dtype, divisor_for_int8, scale is not None)
    return (embeddings.new_empty((rows, width), dtype=dtype),
            embeddings.new_empty((rows, width), dtype=torch.int32))


@torch.library.register_fake("st::fused_kmean_ann")
def _(cluster_offsets, cluster_ids, cluster_length, embeddings, queries, max_tensor_size_per_row,
      filtering_bit_mask=None, invalid_index_value=-1, divisor_for_int8=-1,
      filtering_bit_index=None, per_embedding_scale=None):
    return _scores_fake(cluster_ids, embeddings, max_tensor_size_per_row, divisor_for_int8,
                        per_embedding_scale)


@torch.library.register_fake("st::fused_kmean_ann_with_partial_masks")
def _(cluster_offsets, cluster_ids, cluster_length, embeddings, queries, max_tensor_size_per_row,
      partial_mask_column_counts_cumsum, partial_mask_first_item_offset_in_column,
      partial_mask_column_results, invalid_index_value=-1, divisor_for_int8=-1,
      filtering_bit_index=None, per_embedding_scale=None, cluster_warp_size=None,
      cluster_warp_rounded_length_cumsum=None, cluster_remaining_length_cumsum=None,
      cluster_warp_size_cumsum=None, total_cluster_rounded_warps=0,
      total_cluster_remaining_warps=0):
    return _scores_fake(cluster_ids, embeddings, max_tensor_size_per_row, divisor_for_int8,
                        per_embedding_scale)


@torch.library.register_fake("st::bloom_index_search_batch_prepared")
def _(bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size, k, hash_k,
      return_bool_mask=False):
    cols = (bloom_bundle_b_offsets.shape[0] - 1) * WORDS_PER_BUNDLE
    if return_bool_mask:
        return bloom_index.new_empty((plan_count, cols * 64), dtype=torch.bool)
    return bloom_index.new_empty((plan_count, cols), dtype=torch.int64)


# --- helpers for the filtered scans -----------------------------------------------------------


def attrs_to_features(attrs: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``[N, C, A]`` int64 attrs (``-1`` pads) → ``(feature_ids int32 [C], feature_offsets int64
    [N * C + 1], feature_values int64)``: the clause index is the feature id
    (``ops/official/adapter.py:45-62``)."""
    if attrs.dim() != 3:
        raise ValueError(f"attrs must be [N, C, A_max], got shape {tuple(attrs.shape)}")
    n, c, _ = attrs.shape
    attrs = attrs.long()
    valid = attrs != -1
    offsets = torch.zeros(n * c + 1, dtype=torch.int64, device=attrs.device)
    offsets[1:] = valid.sum(-1).reshape(-1).cumsum(0)
    values = attrs.reshape(-1)[valid.reshape(-1)]
    return (torch.arange(c, dtype=torch.int32, device=attrs.device), offsets.contiguous(),
            values.contiguous())


def prepare_plans(expressions: list[str], hash_k: int, device: torch.device,
                  max_sub_queries: int = 5) -> tuple[Tensor, int, int]:
    """Parse once and upload: ``(blob int64 [8 * B + data words], plan_count, max_stack)``, the
    layout ``bloom_index_search_batch_prepared`` reads (as ``adapter.prepare_plans``)."""
    max_stack, data, offsets = bl.parse_batch(list(expressions), int(hash_k), max_sub_queries)
    b = len(expressions)
    blob = np.zeros(8 * b + (data.size + 7) // 8, np.int64)
    blob[: 8 * b] = offsets
    blob[8 * b :].view(np.uint8)[: data.size] = data
    return torch.from_numpy(blob).to(device), b, max_stack


# --- SilverTorch search (fork_search.cpp:13-49) -------------------------------------------------

_LIB.define(
    "search(Tensor query, Tensor probe_ids, Tensor cluster_offsets, Tensor cluster_sizes, "
    "Tensor item_codes, Tensor sort_perm, Tensor global_scale, int k, "
    "int max_tensor_size_per_row, int divisor_for_int8=-1, Tensor? filtering_bit_mask=None, "
    "Tensor? bloom_index=None, Tensor? bloom_bundle_b_offsets=None, Tensor? plans=None, "
    "int plan_count=0, int max_stack_size=0, Tensor? query_plan_index=None, int bloom_k=0, "
    "int hash_k=0, Tensor? item_clause_attrs=None, Tensor? clause_slots=None, "
    "Tensor? clause_is_reverse=None, Tensor? query_clause_attrs=None) -> (Tensor, Tensor)"
)
_LIB.define(
    "probe_prep(Tensor query, Tensor probe_ids, Tensor cluster_offsets, Tensor cluster_sizes) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"
)

MAX_SEARCH_K = 1024  # kSelectMaxK
MAX_PROBE = 1024


def quantize_rows(query: Tensor, scale_div: bool = False) -> tuple[Tensor, Tensor]:
    """float32 ``[B, D]`` → ``(codes int8 [B, D], scales float32 [B])`` on the GPU (the
    quantization of ``fork_search_cuda.cu:680-699``; ``scale_div``: the scale as
    ``quantize_int8``'s ``abs_max / 127``, ``indexing/quantize.py:9-18``)."""
    q = query.to(torch.float32).contiguous()
    dev = nat.require_device(q)
    b, d = q.shape
    codes = torch.empty((b, d), dtype=torch.int8, device=dev)
    scales = torch.empty((b,), dtype=torch.float32, device=dev)
    if b and d:
        with torch.cuda.device(dev):
            st = nat.lib().rt_quantize_int8_rows(nat.ptr(q), b, d, nat.ptr(codes),
                                                 nat.ptr(scales), int(scale_div),
                                                 nat.stream(dev))
        nat.check(st)
    return codes, scales


def _probe_prep(query, probe_ids, cluster_offsets, cluster_sizes):
    """``(codes, scales, cluster_ids, cluster_length, selected_offsets, warp_size,
    warp_rounded_length_cumsum, remaining_length_cumsum, warp_size_cumsum)``
    (``fork_search_cuda.cu:653-768, 1200-1254``): the quantized rows, the probed clusters'
    ids / lengths / offsets, and the 32-doc warp bookkeeping of the reference's scorer
    (per-row cumulative warp-rounded lengths; cumulative remainders and warp counts over all
    rows)."""
    if query.dim() != 2 or query.dtype != torch.float32:
        raise RuntimeError("query must be float32 [B, D]")
    if probe_ids.dim() != 2 or probe_ids.shape[0] != query.shape[0]:
        raise RuntimeError("probe_ids must be [B, n_probe]")
    if cluster_offsets.dtype != torch.int64 or cluster_sizes.dtype != torch.int64:
        raise RuntimeError("cluster_offsets and cluster_sizes must be int64")
    codes, scales = quantize_rows(query)
    probes = probe_ids.to(torch.int64).contiguous()
    lens = cluster_sizes[probes]
    offs = cluster_offsets[probes]
    warps = lens // 32
    rem = lens % 32
    return (codes, scales, probes.clone(), lens, offs, warps.to(torch.int32).reshape(-1),
            (warps * 32).cumsum(1).to(torch.int32), rem.reshape(-1).cumsum(0).to(torch.int32),
            warps.reshape(-1).cumsum(0).to(torch.int32))


_LIB.impl("probe_prep", _probe_prep, "CUDA")


@torch.library.register_fake("st::probe_prep")
def _(query, probe_ids, cluster_offsets, cluster_sizes):
    rows, n_probe = probe_ids.shape
    i64 = probe_ids.new_empty((rows, n_probe), dtype=torch.int64)
    return (query.new_empty(query.shape, dtype=torch.int8),
            query.new_empty((rows,), dtype=torch.float32), i64, torch.empty_like(i64),
            torch.empty_like(i64), probe_ids.new_empty((rows * n_probe,), dtype=torch.int32),
            probe_ids.new_empty((rows, n_probe), dtype=torch.int32),
            probe_ids.new_empty((rows * n_probe,), dtype=torch.int32),
            probe_ids.new_empty((rows * n_probe,), dtype=torch.int32))


def _capturing() -> bool:
    return torch.cuda.is_current_stream_capturing()


def _tkey(t: Tensor) -> tuple:
    """A cache key for a tensor's contents: its storage address, size and version counter (views
    of one storage share the counter), so another object over the same memory -- as a compiled
    graph may pass -- finds the entry. Entries are dropped with the tensor that made them."""
    return (t.device.index, t.data_ptr(), t.numel(), t.dtype, t._version)


# (id, version) of cluster_sizes -> its largest cluster (the payload columns' static bound)
_MAX_CLUSTER: dict = {}


def _max_cluster(sizes: Tensor) -> int | None:
    """The largest cluster of an index, read back once per index (kept until the tensor is freed
    or modified in place); None under graph capture with nothing kept."""
    import weakref

    key = _tkey(sizes)
    hit = _MAX_CLUSTER.get(key)
    if hit is None:
        if _capturing():
            return None
        hit = int(sizes.max().item()) if sizes.numel() else 0
        _MAX_CLUSTER[key] = hit
        weakref.finalize(sizes, _MAX_CLUSTER.pop, key, None)
    return hit


def _payload_bloom(bloom_index, bloom_bundle_b_offsets, plans, plan_count, max_stack_size,
                   bloom_k, hash_k, query_plan_index, probes, offs, sizes):
    """The Bloom words of every row's probed payloads only (``bloom_index_search_cuda.cu:
    1945-2063``, ``partial_response``'s layout): ``(column_counts_cumsum, first_offsets,
    words)``, entry ``b * n_probe + j`` for probe ``j`` of row ``b``; None when no column bound
    is at hand (a capture before the first eager search on this index)."""
    biggest = _max_cluster(sizes)
    if biggest is None:
        return None
    n_lists = offs.numel()
    valid = (probes >= 0) & (probes < n_lists)
    cluster = torch.where(valid, probes, 0)
    starts = torch.where(valid, offs[cluster], 0).contiguous()
    lengths = torch.where(valid, sizes[cluster], 0).contiguous()
    # a payload of at most `biggest` docs spans at most biggest / 64 + 2 columns
    max_columns = probes.numel() * ((biggest + 63) // 64 + 1)
    qpi = None if query_plan_index is None else query_plan_index.to(torch.int64)
    return _partial_response_prepared(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                                      max_stack_size, starts, lengths, bloom_k, hash_k, qpi,
                                      max_columns)


# Row widths (int8 D) the full-scan kernels take; other widths run the IVF kernel.
_FULL_SCAN_D = (64, 128, 256, 512, 768, 1024)
# (id, version) of cluster_offsets and cluster_sizes, and N -> whether the one list is [0, N).
_ONE_LIST: dict = {}


def _one_list_is_the_table(offsets: Tensor, sizes: Tensor, n: int) -> bool:
    """Whether the single list holds every item in order (offset 0, size N): read back from the
    device once per index and kept until either tensor is freed or modified in place, so a
    steady-state search makes no host sync. Under graph capture with nothing kept, False (the
    IVF kernel takes the call, with the same results)."""
    import weakref

    key = (_tkey(offsets), _tkey(sizes), n)
    hit = _ONE_LIST.get(key)
    if hit is None:
        if _capturing():
            return False
        hit = bool(int(offsets.reshape(-1)[0].item()) == 0 and
                   int(sizes.reshape(-1)[0].item()) == n)
        _ONE_LIST[key] = hit
        for t in (offsets, sizes):
            weakref.finalize(t, _ONE_LIST.pop, key, None)
    return hit


def _st_search(query, probe_ids, cluster_offsets, cluster_sizes, item_codes, sort_perm,
            global_scale, k, max_tensor_size_per_row, divisor_for_int8=-1,
            filtering_bit_mask=None, bloom_index=None, bloom_bundle_b_offsets=None, plans=None,
            plan_count=0, max_stack_size=0, query_plan_index=None, bloom_k=0, hash_k=0,
            item_clause_attrs=None, clause_slots=None, clause_is_reverse=None,
            query_clause_attrs=None):
    """SilverTorch's forward after phase 1 on the HIP kernels: quantize the rows, filter (at most
    one of a full-N mask, Bloom plans -- with the exact recheck when ``query_clause_attrs`` is
    given -- or the exact clauses), score the probed clusters' int8 codes and keep the top ``k``
    by (key desc, slot asc), then ``id = sort_perm[position]`` and the dequantized score
    (``fork_search_cuda.cu:1256-1524``). A one-list int32 search runs as the full scan."""
    if item_codes.dtype != torch.int8 or item_codes.dim() != 2 or \
            item_codes.shape[1] != query.shape[1]:
        raise RuntimeError("item_codes must be int8 [N, D] with the query's D")
    exact = query_clause_attrs is not None
    if filtering_bit_mask is not None and (plans is not None or exact):
        raise RuntimeError("search takes one filter: plans (+ query_clause_attrs to recheck), "
                           "query_clause_attrs or filtering_bit_mask")
    if exact and (item_clause_attrs is None or clause_slots is None or clause_is_reverse is None):
        raise RuntimeError("the exact filter needs item_clause_attrs, clause_slots and "
                           "clause_is_reverse")
    if k < 1:
        raise RuntimeError(f"k must be >= 1, got {k}")
    if probe_ids.dim() != 2 or probe_ids.shape[0] != query.shape[0] or \
            probe_ids.shape[1] > MAX_PROBE:
        raise RuntimeError(f"probe_ids must be [B, n_probe <= {MAX_PROBE}]")
    if not item_codes.is_contiguous():
        raise ValueError("item_codes must be contiguous (copy it once at index build)")
    dev = nat.require_device(query, item_codes, sort_perm, cluster_offsets, cluster_sizes)
    b, d = query.shape
    n = item_codes.shape[0]
    codes, scales = quantize_rows(query)
    width = (int(max_tensor_size_per_row) + 31) // 32 * 32
    ids = torch.empty((b, k), dtype=torch.int64, device=dev)
    scores = torch.empty((b, k), dtype=torch.float32, device=dev)
    if b == 0:
        return ids, scores
    perm = sort_perm.to(torch.int64).contiguous()
    gs = global_scale.to(torch.float32).reshape(-1).contiguous()
    offs = cluster_offsets.to(torch.int64).contiguous()
    sizes = cluster_sizes.to(torch.int64).contiguous()
    probes = probe_ids.to(torch.int64).contiguous()
    lib = nat.lib()
    if plans is not None and (bloom_index is None or bloom_bundle_b_offsets is None):
        raise RuntimeError("plans need bloom_index and bloom_bundle_b_offsets")
    if exact:
        slots = item_clause_attrs.to(torch.int32).contiguous()
        cs = clause_slots.to(torch.int64).contiguous()
        rev = clause_is_reverse.to(torch.int8).contiguous()
        qv = query_clause_attrs.to(torch.int64)
        qv = torch.where((qv >= -1) & (qv <= 2**31 - 1), qv, -(2**31)).to(torch.int32)
        qv = qv.contiguous()
    full = (divisor_for_int8 == -1 and offs.numel() == 1 and probes.shape[1] == 1
            and width >= n and d in _FULL_SCAN_D
            and _one_list_is_the_table(cluster_offsets, cluster_sizes, n))
    if not full and k <= MAX_SEARCH_K and filtering_bit_mask is None and (plans is not None
                                                                          or exact):
        # the IVF kernel with the reference's per-payload filters: Bloom words of the probed
        # columns only, the exact recheck of the probed docs only
        partial = None
        if plans is not None:
            partial = _payload_bloom(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                                     max_stack_size, bloom_k, hash_k, query_plan_index, probes,
                                     offs, sizes)
        if partial is not None or plans is None:
            cum, first, words = partial if partial is not None else (None, None, None)
            ws = nat.workspace(lib.rt_ivf_search_workspace(b, width, k), dev)
            with torch.cuda.device(dev):
                st = lib.rt_ivf_search_payload_filters(
                    nat.ptr(codes), nat.ptr(scales), b, nat.ptr(item_codes), n, d,
                    nat.ptr(probes), probes.shape[1], nat.ptr(offs), nat.ptr(sizes), offs.numel(),
                    width, nat.ptr(cum), nat.ptr(first), nat.ptr(words),
                    0 if first is None else first.numel(), 0 if words is None else words.numel(),
                    nat.ptr(slots) if exact else None,
                    (slots.shape[0] if slots.dim() == 2 else 0) if exact else 0,
                    nat.ptr(cs) if exact else None, cs.numel() - 1 if exact else 0,
                    nat.ptr(rev) if exact else None, nat.ptr(qv) if exact else None,
                    int(divisor_for_int8), nat.ptr(perm), perm.numel(), nat.ptr(gs), k,
                    nat.ptr(ids), nat.ptr(scores), nat.ptr(ws), ws.numel(), nat.stream(dev))
            nat.check(st)
            return ids, scores
    # a full-N mask: the one-list full scan, top-k above 1024, a caller's mask, or a capture
    # with no cached column bound for the per-payload Bloom words
    mask = None
    if filtering_bit_mask is not None:
        mask = filtering_bit_mask.to(torch.int64).contiguous()
    if plans is not None:
        bm = _search_prepared(bloom_index, bloom_bundle_b_offsets, plans, plan_count,
                              max_stack_size, bloom_k, hash_k, False)
        mask = bm[query_plan_index.to(torch.int64)] if query_plan_index is not None else bm[:b]
        mask = mask.contiguous()
    if exact:
        out = torch.empty((b, (n + 63) // 64), dtype=torch.int64, device=dev)
        with torch.cuda.device(dev):
            st = lib.rt_clause_slots_filter(
                nat.ptr(slots), slots.shape[0] if slots.dim() == 2 else 0, n, nat.ptr(cs),
                cs.numel() - 1, nat.ptr(rev), nat.ptr(qv), b, nat.ptr(mask),
                0 if mask is None else mask.shape[1], nat.ptr(out), nat.stream(dev))
        nat.check(st)
        mask = out
    if k > MAX_SEARCH_K:
        return _search_large_k(codes, scales, item_codes, probes, offs, sizes, width, mask,
                               int(divisor_for_int8), perm, gs, k)
    if full:
        # one list holding every item in order: slot = position, the full-scan kernels; a row
        # whose probe is not list 0 has no slot and ends as pads
        from retrieve_amd import hip  # noqa: F401  (registers torch.ops.retrieve.*)
        pos, dots = torch.ops.retrieve_amd.int8_scan_topk(codes, item_codes, k, mask)
        ids.copy_(pos)
        with torch.cuda.device(dev):
            st = lib.rt_search_epilogue(nat.ptr(ids), nat.ptr(dots), nat.ptr(scores), b, k,
                                        nat.ptr(perm), perm.numel(), nat.ptr(scales), nat.ptr(gs),
                                        nat.stream(dev))
        nat.check(st)
        probed = probes[:, :1] == 0
        ids = torch.where(probed, ids, -1)
        scores = torch.where(probed, scores, float("-inf"))
        return ids, scores
    ws = nat.workspace(lib.rt_ivf_search_workspace(b, width, k), dev)
    with torch.cuda.device(dev):
        st = lib.rt_ivf_search(
            nat.ptr(codes), nat.ptr(scales), b, nat.ptr(item_codes), n, d, nat.ptr(probes),
            probes.shape[1], nat.ptr(offs), nat.ptr(sizes), offs.numel(), width, nat.ptr(mask),
            0 if mask is None else mask.shape[1], int(divisor_for_int8), nat.ptr(perm),
            perm.numel(), nat.ptr(gs), k, nat.ptr(ids), nat.ptr(scores), nat.ptr(ws), ws.numel(),
            nat.stream(dev))
    nat.check(st)
    return ids, scores


def _search_large_k(codes, scales, item_codes, probes, offs, sizes, width, mask, divisor, perm,
                    gs, k):
    """``search`` above the radix select's 1024: the raw scorer over every probed slot, the rows'
    top ``k`` by (key desc, slot asc), then the epilogue (``fork_search_cuda.cu:843-915,
    1490-1520``: ``at::topk`` on the raw buffer and ``epilogue_kernel``): ``id =
    sort_perm[position]``; score ``(fp32(dot) * q_scale) * global_scale``, or with a divisor
    ``score16 * ((q_scale * divisor) * global_scale)``; ``-1`` / ``-inf`` pads."""
    from retrieve_amd import large_k

    b = codes.shape[0]
    n_lists = offs.numel()
    dev = codes.device
    valid = (probes >= 0) & (probes < n_lists)
    cluster = torch.where(valid, probes, 0)
    length = torch.where(valid, sizes[cluster], 0)
    ids = torch.full((b, k), -1, dtype=torch.int64, device=dev)
    scores = torch.full((b, k), float("-inf"), dtype=torch.float32, device=dev)
    step = large_k.chunk_rows(width, dev)
    for r0 in range(0, b, step):
        r1 = min(b, r0 + step)
        raw, idx = raw_scores(offs, cluster[r0:r1].contiguous(), length[r0:r1].contiguous(),
                              item_codes, codes[r0:r1].contiguous(), width,
                              mask=None if mask is None else mask[r0:r1], divisor_for_int8=divisor)
        top_raw, slot = large_k.raw_topk(raw, idx, k)
        hit = slot >= 0
        pos = idx.gather(1, slot.clamp(min=0)).to(torch.int64)
        ids[r0:r1] = torch.where(hit, perm[pos.clamp(min=0)], -1)
        q = scales[r0:r1, None]
        if divisor == -1:
            sc = (top_raw.to(torch.float32) * q) * gs
        else:
            sc = top_raw.to(torch.float32) * ((q * float(divisor)) * gs)
        scores[r0:r1] = torch.where(hit, sc, float("-inf"))
    return ids, scores


_LIB.impl("search", _st_search, "CUDA")


@torch.library.register_fake("st::search")
def _(query, probe_ids, cluster_offsets, cluster_sizes, item_codes, sort_perm, global_scale, k,
      max_tensor_size_per_row, divisor_for_int8=-1, filtering_bit_mask=None, bloom_index=None,
      bloom_bundle_b_offsets=None, plans=None, plan_count=0, max_stack_size=0,
      query_plan_index=None, bloom_k=0, hash_k=0, item_clause_attrs=None, clause_slots=None,
      clause_is_reverse=None, query_clause_attrs=None):
    rows = query.shape[0]
    return (query.new_empty((rows, k), dtype=torch.int64),
            query.new_empty((rows, k), dtype=torch.float32))
