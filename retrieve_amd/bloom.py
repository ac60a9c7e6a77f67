"""Bloom query preparation: the expression parser and the plan encoding the HIP search reads.

Grammar (``silvertorch/.../ops/csrc/EXPRESSION_SYNTAX.md``): ``or_expr = and_expr {(OR | "|")
and_expr}``, ``and_expr = unary {(AND | "&") unary}``, ``unary = (NOT | "!") unary | primary``,
``primary = "(" or_expr ")" | id:value[:weight]``; an empty expression matches everything.

Plan encoding (the four segments of ``bloom_index_util.cpp:104-125``, this library's own
bytes): per plan, 8 byte offsets ``[ops, offsets, parameters, hashes] x [begin, end)`` into
the batch's data, every segment 8-aligned:

- ``ops`` uint8, post-order: ``AND=1 OR=2 NOT=3 TERM=4 EMPTY=5`` (``bloom_index_util.h:49-56``);
- ``offsets`` int32 ``[n_ops + 1]``: op ``j``'s parameters are ``parameters[offsets[j]:
  offsets[j+1]]`` -- a term's index, NOT's child op, the children ops of AND / OR (at most
  ``max_sub_queries`` of them: longer chains are folded into nested nodes of the same op);
- ``hashes`` uint64 ``[terms, hash_k]``: the term's ``murmur(id, value, seed)`` for seeds ``0 ..
  hash_k - 1``, terms in post-order.

Evaluating the ops left to right on a stack (AND / OR pop their children count) gives the
expression; the root is the last op.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

AND, OR, NOT, TERM, EMPTY = 1, 2, 3, 4, 5

_U = np.uint64
_C1 = _U(0x87C37B91114253D5)
_C2 = _U(0x4CF5AD432745937F)


def _rotl(x: np.ndarray, r: int) -> np.ndarray:
    return (x << _U(r)) | (x >> _U(64 - r))


def _fmix(k: np.ndarray) -> np.ndarray:
    k = k ^ (k >> _U(33))
    k = k * _U(0xFF51AFD7ED558CCD)
    k = k ^ (k >> _U(33))
    k = k * _U(0xC4CEB9FE1A85EC53)
    return k ^ (k >> _U(33))


def murmur_2x64(x, y, seed) -> np.ndarray:
    """``h1 ^ h2`` of MurmurHash3_x64_128 (Austin Appleby, public domain) over the one 16-byte
    block ``x || y`` (little-endian 64-bit words) with ``seed``; vectorised over numpy arrays
    (the token hash of ``bloom_index_util.cuh:60-107``)."""
    with np.errstate(over="ignore"):
        x = np.asarray(x).astype(np.int64).view(np.uint64)
        y = np.asarray(y).astype(np.int64).view(np.uint64)
        s = np.asarray(seed).astype(np.uint64)
        x, y, s = np.broadcast_arrays(x, y, s)
        h1 = s.copy()
        h2 = s.copy()
        k1 = _rotl(x * _C1, 31) * _C2
        h1 = h1 ^ k1
        h1 = _rotl(h1, 27) + h2
        h1 = h1 * _U(5) + _U(0x52DCE729)
        k2 = _rotl(y * _C2, 33) * _C1
        h2 = h2 ^ k2
        h2 = _rotl(h2, 31) + h1
        h2 = h2 * _U(5) + _U(0x38495AB5)
        h1 = h1 ^ _U(16)
        h2 = h2 ^ _U(16)
        h1 = h1 + h2
        h2 = h2 + h1
        h1 = _fmix(h1)
        h2 = _fmix(h2)
        h1 = h1 + h2
        h2 = h2 + h1
        return h1 ^ h2


# --- parser -----------------------------------------------------------------------------------


def _tokens(text: str) -> list[str]:
    """Operators, parentheses, keywords and ``id:value[:weight]`` terms, in order."""
    out: list[str] = []
    i, n = 0, len(text)
    while i < n:
        ch = text[i]
        if ch.isspace():
            i += 1
        elif ch in "()!&|":
            out.append(ch)
            i += 1
        elif ch.isalpha():
            j = i
            while j < n and text[j].isalpha():
                j += 1
            word = text[i:j].upper()
            if word not in ("AND", "OR", "NOT"):
                raise ValueError(f"unknown keyword {text[i:j]!r} in {text!r}")
            out.append(word)
            i = j
        elif ch == "-" or ch.isdigit():
            j = i
            while j < n and (text[j].isdigit() or text[j] in "-.:"):
                j += 1
            out.append(text[i:j])
            i = j
        else:
            raise ValueError(f"unexpected {ch!r} in {text!r}")
    return out


def _term(tok: str, text: str) -> tuple[int, int]:
    parts = tok.split(":")
    if len(parts) not in (2, 3):
        raise ValueError(f"bad term {tok!r} in {text!r}")
    try:
        fid, val = int(parts[0]), int(parts[1])
        if len(parts) == 3:
            float(parts[2])  # the weight: checked, unused by the Bloom filter
    except ValueError as e:
        raise ValueError(f"bad term {tok!r} in {text!r}") from e
    return fid, val


def parse(text: str):
    """Expression → tree: ``("TERM", id, value)``, ``("NOT", x)``, ``("AND" | "OR", [xs])``
    (operands of one chain at one level), or ``("EMPTY",)`` for an empty expression."""
    toks = _tokens(text)
    if not toks:
        return ("EMPTY",)
    pos = 0

    def at(*want: str) -> bool:
        return pos < len(toks) and toks[pos] in want

    def or_expr():
        nonlocal pos
        xs = [and_expr()]
        while at("OR", "|"):
            pos += 1
            xs.append(and_expr())
        return xs[0] if len(xs) == 1 else ("OR", xs)

    def and_expr():
        nonlocal pos
        xs = [unary()]
        while at("AND", "&"):
            pos += 1
            xs.append(unary())
        return xs[0] if len(xs) == 1 else ("AND", xs)

    def unary():
        nonlocal pos
        if at("NOT", "!"):
            pos += 1
            return ("NOT", unary())
        return primary()

    def primary():
        nonlocal pos
        if pos >= len(toks):
            raise ValueError(f"unexpected end of {text!r}")
        tok = toks[pos]
        pos += 1
        if tok == "(":
            node = or_expr()
            if not at(")"):
                raise ValueError(f"missing ')' in {text!r}")
            pos += 1
            return node
        if tok in (")", "!", "&", "|", "AND", "OR", "NOT"):
            raise ValueError(f"unexpected {tok!r} in {text!r}")
        fid, val = _term(tok, text)
        return ("TERM", fid, val)

    tree = or_expr()
    if pos != len(toks):
        raise ValueError(f"trailing {toks[pos]!r} in {text!r}")
    return tree


@dataclass
class Plan:
    ops: list[int]
    params: list[list[int]]  # per op
    terms: list[tuple[int, int]]
    max_stack: int


def compile_plan(tree, max_sub_queries: int = 5) -> Plan:
    """Post-order ops of the parsed tree, with the reference builder's fan-out rule
    (``expression_query_parser.cpp:207-290``): along an AND / OR chain, each time
    ``max_sub_queries`` operands have gathered they become one node, which then stands as the
    first operand of the rest of the chain; the chain ends in one node over what remains,
    emitted whenever a batch was cut (so a chain whose last operand completes a batch ends in a
    one-child node over it), else only for two operands or more. The plan bytes are then Meta's
    byte for byte (``tests/golden``'s parser fixtures)."""
    m = int(max_sub_queries)
    ops: list[int] = []
    params: list[list[int]] = []
    terms: list[tuple[int, int]] = []
    depth = 0
    max_depth = 0

    def push(op: int, ps: list[int], pops: int) -> int:
        nonlocal depth, max_depth
        ops.append(op)
        params.append(ps)
        depth += 1 - pops
        max_depth = max(max_depth, depth)
        return len(ops) - 1

    def chain(op: int, xs) -> int:
        sub: list[int] = []
        gathered = 0
        batched = False
        for i, x in enumerate(xs):
            sub.append(emit(x))
            gathered += 1
            # (the first operand is batched only when more follow: a chain here has two or more)
            if gathered == m:
                sub = [push(op, sub, len(sub))]
                gathered = 1
                batched = True
        if len(sub) <= 1 and not batched:
            return sub[0]
        return push(op, sub, len(sub))

    def emit(node) -> int:
        kind = node[0]
        if kind == "EMPTY":
            return push(EMPTY, [], 0)
        if kind == "TERM":
            terms.append((node[1], node[2]))
            return push(TERM, [len(terms) - 1], 0)
        if kind == "NOT":
            child = emit(node[1])
            return push(NOT, [child], 1)
        return chain(AND if kind == "AND" else OR, node[1])

    emit(tree)
    return Plan(ops, params, terms, max_depth)


def _pad8(buf: bytearray) -> None:
    buf.extend(b"\0" * (-len(buf) % 8))


def encode(plans: list[Plan], hash_k: int) -> tuple[int, np.ndarray, np.ndarray]:
    """``(max_stack, data uint8 [bytes], offsets int64 [8 * len(plans)])``."""
    all_terms = [t for p in plans for t in p.terms]
    if all_terms:
        ids = np.array([t[0] for t in all_terms], np.int64)[:, None]
        vals = np.array([t[1] for t in all_terms], np.int64)[:, None]
        hashes = murmur_2x64(ids, vals, np.arange(hash_k, dtype=np.uint64)[None, :])
    else:
        hashes = np.zeros((0, hash_k), np.uint64)
    data = bytearray()
    offsets = np.zeros(8 * len(plans), np.int64)
    t0 = 0
    for i, p in enumerate(plans):
        segs = []
        segs.append(np.array(p.ops, np.uint8).tobytes())
        ends = np.zeros(len(p.ops) + 1, np.int32)
        ends[1:] = np.cumsum([len(ps) for ps in p.params])
        segs.append(ends.tobytes())
        segs.append(np.array([x for ps in p.params for x in ps], np.int32).tobytes())
        segs.append(hashes[t0 : t0 + len(p.terms)].tobytes())
        t0 += len(p.terms)
        for s, seg in enumerate(segs):
            offsets[8 * i + 2 * s] = len(data)
            data.extend(seg)
            offsets[8 * i + 2 * s + 1] = len(data)
            _pad8(data)
    max_stack = max((p.max_stack for p in plans), default=1)
    return max_stack, np.frombuffer(bytes(data), np.uint8).copy(), offsets


def parse_batch(expressions: list[str], hash_k: int,
                max_sub_queries: int = 5) -> tuple[int, np.ndarray, np.ndarray]:
    """A batch of expressions → ``(max_stack, data, offsets)`` (the parser op's outputs)."""
    if hash_k < 1:
        raise ValueError(f"hash_k must be >= 1, got {hash_k}")
    return encode([compile_plan(parse(e), max_sub_queries) for e in expressions], hash_k)


def queries_to_expressions(query_attrs, reverse=None) -> list[str]:
    """``[B, C]`` query values (``-1`` inactive) → ``"c:v AND ..."``, ``NOT c:v`` for reverse
    clauses, ``""`` when no clause is active (``ops/official/adapter.py:127-157``)."""
    q = np.asarray(query_attrs).tolist()
    rev = [bool(x) for x in (reverse if reverse is not None else [False] * (len(q[0]) if q else 0))]
    out = []
    for row in q:
        out.append(" AND ".join((f"NOT {c}:{v}" if rev[c] else f"{c}:{v}")
                                for c, v in enumerate(row) if v != -1))
    return out


def sets_to_expressions(query_sets) -> list[str]:
    """``[B, C, V]`` value sets (``-1`` pads) → ``"(c:v1 OR c:v2) AND ..."`` per row: the Bloom
    form of the value-set clause filter."""
    out = []
    for row in np.asarray(query_sets).tolist():
        parts = []
        for c, vals in enumerate(row):
            vs = [v for v in vals if v != -1]
            if vs:
                parts.append("(" + " OR ".join(f"{c}:{v}" for v in vs) + ")")
        out.append(" AND ".join(parts))
    return out
