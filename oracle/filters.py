"""Attribute filters: the exact clause predicate and the Bloom filter (test infrastructure; see
``oracle/__init__``).

Pinned by:
- exact predicate: the reference's semantics table (reverse XOR, ``-1`` inactive, AND over
  clauses; ``retrieve/src/retrieve/functional.py:173-185``) brute-forced in Python loops on
  small inputs, and the singleton-set reduction of the value-set form.
- ``murmur3_x64_128``: the published SMHasher verification value of MurmurHash3_x64_128
  (``0x6384BA69``). ``murmur_hash3_2x64`` is checked equal to it on the 16-byte key ``x || y``.
- Bloom layout: a hand-computed word/bit position, and the no-false-negative invariant
  (every (doc, token) inserted is found) over random corpora.
- Plans: the reference's README corpus known answer (queries ``0:100``,
  ``0:100 AND NOT 1:201``, ``0:102 OR 1:203`` → hits ``[[0,1,3],[1,3],[2,3]]``,
  ``retrieve/tests/parity/test_official.py:229-245, 353-366``) and the expression mapping
  known answer (``test_official.py:510-514``).
- Bloom words: bit for bit against Meta's CPU builder and search, compiled from the reference's
  sources into ``oracle/_ref`` (fixtures ``tests/golden/ref_cpu.npz``,
  ``tests/test_ref_fixtures.py``), at the upstream widths; the fixed-width build (CUDA-only in
  the reference) by the same position rule, the hand-computed position and the invariants.
- ``bloom_doc_bits`` (the row view of the bundles): against each document's positions computed
  from its tokens directly (``bit_positions``), independent of the word layout, and the term
  test on it against ``term_mask`` (``tests/test_oracle.py``).
"""

from __future__ import annotations

import re

import numpy as np

DOCS_PER_BUNDLE = 2048  # C_BITS_IN_BLOOM_V2_COL_BUNDLE (bloom_index_util.h:42-44)
WORDS_PER_BUNDLE = 32  # C_BLOOM_V2_COL_BUNDLE_SIZE
MAX_K = 10  # MAX_K_V2 (bloom_index_util.h:46)
M64 = (1 << 64) - 1


# --- exact clause predicate ------------------------------------------------------------------


def clause_match(item_attrs: np.ndarray, reverse: np.ndarray, query: np.ndarray) -> np.ndarray:
    """``[N, C, A]`` item attrs (``-1`` pads), ``[C]`` reverse flags, ``[B, C]`` query values →
    ``[B, N]`` bool: clause ``c`` matches iff some item value equals ``query[c]``, XOR
    ``reverse[c]``; ``query[c] == -1`` is inactive (passes); AND over clauses
    (``functional.py:173-185``; ``fork_filters.cuh:15-41``)."""
    q = np.asarray(query)[:, None, :, None]  # [B,1,C,1]
    m = (np.asarray(item_attrs)[None] == q).any(axis=-1)  # [B,N,C]
    m = np.where(np.asarray(reverse, bool)[None, None, :], ~m, m)
    inactive = (np.asarray(query) == -1)[:, None, :]
    return (m | inactive).all(axis=-1)


def clause_match_sets(item_attrs: np.ndarray, query_sets: np.ndarray, reverse=None) -> np.ndarray:
    """Value-set clauses: ``query_sets [B, C, V]`` (``-1`` pads). Clause ``c`` matches iff some
    item value is in the row's set, XOR ``reverse[c]``; a clause whose set is all ``-1`` is
    inactive. With ``V == 1`` this is ``clause_match``."""
    qs = np.asarray(query_sets)
    items = np.asarray(item_attrs)
    b, c, _ = qs.shape
    rev = np.zeros(c, bool) if reverse is None else np.asarray(reverse, bool)
    out = np.ones((b, items.shape[0]), dtype=bool)
    for r in range(b):
        for ci in range(c):
            vals = qs[r, ci][qs[r, ci] != -1]
            if vals.size == 0:
                continue
            hit = (np.isin(items[:, ci, :], vals) & (items[:, ci, :] != -1)).any(axis=1)
            out[r] &= hit ^ rev[ci]
    return out


# --- MurmurHash3 ----------------------------------------------------------------------------


def _rotl(x: int, r: int) -> int:
    return ((x << r) | (x >> (64 - r))) & M64


def _fmix(k: int) -> int:
    k ^= k >> 33
    k = (k * 0xFF51AFD7ED558CCD) & M64
    k ^= k >> 33
    k = (k * 0xC4CEB9FE1A85EC53) & M64
    k ^= k >> 33
    return k


_C1 = 0x87C37B91114253D5
_C2 = 0x4CF5AD432745937F


def murmur3_x64_128(data: bytes, seed: int) -> tuple[int, int]:
    """The published MurmurHash3_x64_128 (Austin Appleby, public domain) over ``data``:
    16-byte blocks, a tail, then the length finalization. Returns ``(h1, h2)``."""
    n = len(data)
    h1 = h2 = seed & M64
    nblocks = n // 16
    for i in range(nblocks):
        k1 = int.from_bytes(data[16 * i : 16 * i + 8], "little")
        k2 = int.from_bytes(data[16 * i + 8 : 16 * i + 16], "little")
        k1 = (k1 * _C1) & M64
        k1 = _rotl(k1, 31)
        k1 = (k1 * _C2) & M64
        h1 ^= k1
        h1 = _rotl(h1, 27)
        h1 = (h1 + h2) & M64
        h1 = (h1 * 5 + 0x52DCE729) & M64
        k2 = (k2 * _C2) & M64
        k2 = _rotl(k2, 33)
        k2 = (k2 * _C1) & M64
        h2 ^= k2
        h2 = _rotl(h2, 31)
        h2 = (h2 + h1) & M64
        h2 = (h2 * 5 + 0x38495AB5) & M64
    tail = data[16 * nblocks :]
    k1 = k2 = 0
    t = len(tail)
    if t > 8:
        k2 = int.from_bytes(tail[8:], "little")
        k2 = (k2 * _C2) & M64
        k2 = _rotl(k2, 33)
        k2 = (k2 * _C1) & M64
        h2 ^= k2
    if t > 0:
        k1 = int.from_bytes(tail[:8], "little")
        k1 = (k1 * _C1) & M64
        k1 = _rotl(k1, 31)
        k1 = (k1 * _C2) & M64
        h1 ^= k1
    h1 ^= n
    h2 ^= n
    h1 = (h1 + h2) & M64
    h2 = (h2 + h1) & M64
    h1 = _fmix(h1)
    h2 = _fmix(h2)
    h1 = (h1 + h2) & M64
    h2 = (h2 + h1) & M64
    return h1, h2


def smhasher_verification() -> int:
    """SMHasher's ``VerificationTest`` for a 128-bit hash: hash ``bytes(range(i))`` with seed
    ``256 - i`` for i in 0..255, hash the concatenated digests with seed 0, first 4 bytes."""
    digests = b""
    for i in range(256):
        h1, h2 = murmur3_x64_128(bytes(range(i)), 256 - i)
        digests += h1.to_bytes(8, "little") + h2.to_bytes(8, "little")
    h1, _ = murmur3_x64_128(digests, 0)
    return h1 & 0xFFFFFFFF


def murmur_hash3_2x64(x: int, y: int, seed: int) -> int:
    """The token hash of ``bloom_index_util.cuh:60-107``: MurmurHash3_x64_128 of the 16-byte
    key ``x || y`` (little-endian 64-bit words) with ``seed``, folded as ``h1 ^ h2``."""
    key = (x & M64).to_bytes(8, "little") + (y & M64).to_bytes(8, "little")
    h1, h2 = murmur3_x64_128(key, seed)
    return h1 ^ h2


def bit_positions(feature: int, value: int, b: int, k: int) -> list[int]:
    """Build side: seeds 0, 1, ... → ``hash % b``, duplicates rejected, until ``k`` distinct
    positions (``bloom_index_util.cuh:185-208``)."""
    out: list[int] = []
    seed = 0
    while len(out) < k:
        p = murmur_hash3_2x64(feature, value, seed) % b
        seed += 1
        if p not in out:
            out.append(p)
    return out


def probe_positions(feature: int, value: int, b: int, k: int, n_stored: int) -> list[int]:
    """Search side: the first ``k`` distinct ``hash % b`` among the ``n_stored`` stored hashes
    (seeds 0..n_stored-1); fewer when they do not hold ``k`` distinct ones
    (``bloom_index_search_cuda.cu:319-349``, ``bloom_index_util.cuh:211-222``)."""
    out: list[int] = []
    for seed in range(n_stored):
        if len(out) == k:
            break
        p = murmur_hash3_2x64(feature, value, seed) % b
        if p not in out:
            out.append(p)
    return out


# --- Bloom index ----------------------------------------------------------------------------


def bloom_build(
    item_attrs: np.ndarray,
    build_k: int,
    *,
    bits_per_doc: int | None = None,
    b_multiplier: float | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Bit-sliced bundles of 2048 docs (``bloom_indexer.cpp:27-114``; fixed width:
    ``bloom_indexer_cuda.cu:291-344``). ``item_attrs [N, C, A]`` (``-1`` pads; the feature id
    of a value is its clause index, ``adapter.py:45-62``). Bundle ``β`` is ``b_β`` bits per
    doc: ``bits_per_doc`` (configured) or ``int(max_terms_in_bundle * k * b_multiplier)``
    (upstream). Bit position ``p`` of doc ``d`` is word ``(offsets[β] + p) * 32 + (d % 2048) //
    64``, bit ``63 - d % 64``. Returns ``(words int64 [offsets[-1] * 32], offsets int64
    [n_bundles + 1])``."""
    attrs = np.asarray(item_attrs, np.int64)
    n, c, _ = attrs.shape
    nb = -(-n // DOCS_PER_BUNDLE)
    offsets = np.zeros(nb + 1, np.int64)
    for beta in range(nb):
        if bits_per_doc is not None:
            width = bits_per_doc
        else:
            chunk = attrs[beta * DOCS_PER_BUNDLE : (beta + 1) * DOCS_PER_BUNDLE]
            terms = int((chunk != -1).sum(axis=(1, 2)).max()) if chunk.size else 0
            width = int(float(terms * build_k) * float(b_multiplier))
        offsets[beta + 1] = offsets[beta] + width
    words = np.zeros(int(offsets[-1]) * WORDS_PER_BUNDLE, np.uint64)
    cache: dict[tuple[int, int, int], list[int]] = {}
    for d in range(n):
        beta = d // DOCS_PER_BUNDLE
        b = int(offsets[beta + 1] - offsets[beta])
        col = (d % DOCS_PER_BUNDLE) // 64
        bit = np.uint64(1) << np.uint64(63 - d % 64)
        for ci in range(c):
            for v in attrs[d, ci]:
                if v == -1:
                    continue
                key = (ci, int(v), b)
                if key not in cache:
                    cache[key] = bit_positions(ci, int(v), b, build_k)
                for p in cache[key]:
                    words[(int(offsets[beta]) + p) * WORDS_PER_BUNDLE + col] |= bit
    return words.view(np.int64), offsets


def term_mask(
    words: np.ndarray, offsets: np.ndarray, n_docs: int, feature: int, value: int, k: int,
    n_stored: int,
) -> np.ndarray:
    """``[n_docs]`` bool: the AND of the term's resolved bit positions, per doc
    (``signature_match<true>``, ``bloom_index_search_cuda.cu:305-349``)."""
    w = np.asarray(words).view(np.uint64)
    out = np.zeros(n_docs, dtype=bool)
    for d in range(n_docs):
        beta = d // DOCS_PER_BUNDLE
        b = int(offsets[beta + 1] - offsets[beta])
        col = (d % DOCS_PER_BUNDLE) // 64
        ok = True
        for p in probe_positions(feature, value, b, k, n_stored):
            word = int(w[(int(offsets[beta]) + p) * WORDS_PER_BUNDLE + col])
            ok &= bool((word >> (63 - d % 64)) & 1)
        out[d] = ok
    return out


def bloom_doc_bits(words: np.ndarray, offsets: np.ndarray, n_docs: int) -> np.ndarray:
    """``[n_docs]`` int64: doc ``d``'s bits in one word, position ``p`` at bit ``p`` -- the row
    view of the bundle layout (``bloom_indexer.cpp:79-110``: position ``p`` of doc ``d`` is word
    ``(offsets[β] + p) * 32 + (d % 2048) // 64``, bit ``63 - d % 64``). Bundles up to 64 bits
    wide; no counterpart in the reference (the fused scans' probe reads it)."""
    w = np.asarray(words).view(np.uint64)
    out = np.zeros(n_docs, np.uint64)
    t = np.arange(DOCS_PER_BUNDLE)
    col, shift = t // 64, (63 - t % 64).astype(np.uint64)
    for beta in range(-(-n_docs // DOCS_PER_BUNDLE)):
        o, b = int(offsets[beta]), int(offsets[beta + 1] - offsets[beta])
        if b > 64:
            raise ValueError("bundles wider than 64 bits have no one-word row view")
        m = min(DOCS_PER_BUNDLE, n_docs - beta * DOCS_PER_BUNDLE)
        f = np.zeros(m, np.uint64)
        for p in range(b):
            row = w[(o + p) * WORDS_PER_BUNDLE : (o + p + 1) * WORDS_PER_BUNDLE]
            f |= ((row[col[:m]] >> shift[:m]) & np.uint64(1)) << np.uint64(p)
        out[beta * DOCS_PER_BUNDLE : beta * DOCS_PER_BUNDLE + m] = f
    return out.view(np.int64)


# --- expressions (the reference DSL: EXPRESSION_SYNTAX.md grammar) ---------------------------

_TOKEN = re.compile(r"\s*(\(|\)|!|&|\||-?\d+(?:\.\d+)?(?::-?\d+(?:\.\d+)?){1,2}|[A-Za-z]+)")


def parse_expression(text: str):
    """``or_expr := and_expr (OR and_expr)*``, ``and_expr := unary (AND unary)*``,
    ``unary := NOT unary | primary``, ``primary := '(' expr ')' | id:value[:weight]``.
    Returns a nested tuple tree; ``""`` → ``("EMPTY",)`` (match all,
    ``expression_query_parser.cpp:400-405``)."""
    toks = [t for t in _TOKEN.findall(text) if t.strip()]
    if not toks:
        return ("EMPTY",)
    pos = 0

    def peek():
        return toks[pos].upper() if pos < len(toks) else None

    def take():
        nonlocal pos
        pos += 1
        return toks[pos - 1]

    def or_expr():
        node = and_expr()
        while peek() in ("OR", "|"):
            take()
            node = ("OR", node, and_expr())
        return node

    def and_expr():
        node = unary()
        while peek() in ("AND", "&"):
            take()
            node = ("AND", node, unary())
        return node

    def unary():
        if peek() in ("NOT", "!"):
            take()
            return ("NOT", unary())
        return primary()

    def primary():
        t = take()
        if t == "(":
            node = or_expr()
            if take() != ")":
                raise ValueError("unbalanced parentheses")
            return node
        parts = t.split(":")
        return ("TERM", int(parts[0]), int(parts[1]))

    tree = or_expr()
    if pos != len(toks):
        raise ValueError(f"trailing tokens in {text!r}")
    return tree


def eval_tree(tree, leaf) -> np.ndarray:
    """Evaluate a parsed tree with ``leaf(feature, value) -> bool [n]``."""
    op = tree[0]
    if op == "TERM":
        return leaf(tree[1], tree[2])
    if op == "NOT":
        return ~eval_tree(tree[1], leaf)
    if op == "AND":
        return eval_tree(tree[1], leaf) & eval_tree(tree[2], leaf)
    if op == "OR":
        return eval_tree(tree[1], leaf) | eval_tree(tree[2], leaf)
    raise ValueError(op)


def bloom_expression_mask(
    words, offsets, n_docs: int, text: str, k: int, n_stored: int
) -> np.ndarray:
    """``[n_docs]`` bool: the expression evaluated over the Bloom terms; ``""`` matches all."""
    tree = parse_expression(text)
    if tree[0] == "EMPTY":
        return np.ones(n_docs, dtype=bool)
    return eval_tree(tree, lambda f, v: term_mask(words, offsets, n_docs, f, v, k, n_stored))


def exact_expression_mask(item_attrs: np.ndarray, text: str) -> np.ndarray:
    """The same expression evaluated exactly: term ``c:v`` ⇔ some value of clause ``c`` is
    ``v``."""
    attrs = np.asarray(item_attrs)
    tree = parse_expression(text)
    if tree[0] == "EMPTY":
        return np.ones(attrs.shape[0], dtype=bool)
    return eval_tree(tree, lambda f, v: ((attrs[:, f, :] == v) & (attrs[:, f, :] != -1)).any(1))


def queries_to_expressions(query_attrs: np.ndarray, reverse=None) -> list[str]:
    """``[B, C]`` query values (``-1`` inactive) → ``"c:v AND ..."``, ``NOT c:v`` for reverse
    clauses, ``""`` when no clause is active (``adapter.py:127-157``)."""
    q = np.asarray(query_attrs).tolist()
    c = len(q[0]) if q else 0
    rev = [False] * c if reverse is None else [bool(x) for x in reverse]
    out = []
    for row in q:
        terms = [(f"NOT {ci}:{v}" if rev[ci] else f"{ci}:{v}") for ci, v in enumerate(row)
                 if v != -1]
        out.append(" AND ".join(terms))
    return out


def sets_to_expression(query_sets_row: np.ndarray) -> str:
    """One row of value-set clauses ``[C, V]`` → ``"(c:v1 OR c:v2) AND ..."``."""
    parts = []
    for ci, vals in enumerate(np.asarray(query_sets_row).tolist()):
        vs = [v for v in vals if v != -1]
        if vs:
            parts.append("(" + " OR ".join(f"{ci}:{v}" for v in vs) + ")")
    return " AND ".join(parts)


def bloom_partial_response(plan_columns: np.ndarray, starts: np.ndarray, lengths: np.ndarray,
                           plan_index=None):
    """The Bloom search over the probed clusters' columns only
    (``bloom_index_search_batch_return_partial_response``, ``bloom_index_search.cpp:219-345``):
    for each (row q, probe c) of ``starts`` / ``lengths [B, P]`` (doc positions), its columns
    ``start // 64 ..`` + ``ceil((len + start % 64) / 64)`` (0 when ``len == 0``) evaluated with
    plan ``plan_index[q]`` (or ``q``). ``plan_columns [plans, n_cols]`` are each plan's column
    words over the whole index (the full search's output). Returns ``(column_counts_cumsum
    int32 [B * P], first_item_offsets int8 [B * P], words int64 [total])``."""
    cols = np.asarray(plan_columns).view(np.uint64)
    st = np.asarray(starts, np.int64)
    ln = np.asarray(lengths, np.int64)
    b, p = st.shape
    counts, firsts, words = [], [], []
    acc = 0
    for q in range(b):
        plan = q if plan_index is None else int(plan_index[q])
        for c in range(p):
            s, n = int(st[q, c]), int(ln[q, c])
            off = s % 64
            cnt = (n + off + 63) // 64 if n > 0 else 0
            acc += cnt
            counts.append(acc)
            firsts.append(off)
            words.extend(cols[plan, s // 64 : s // 64 + cnt].tolist())
    return (np.array(counts, np.int32), np.array(firsts, np.int8),
            np.array(words, np.uint64).view(np.int64))
