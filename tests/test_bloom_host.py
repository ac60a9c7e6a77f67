"""Host side of the Bloom path, no GPU: the product's vectorised MurmurHash3 and expression
parser / plan encoding (``retrieve_amd.bloom``) against the oracle's independent restatements
(``oracle.filters``) and the reference's KATs."""

from __future__ import annotations

import numpy as np
import torch

from oracle import filters as of
from retrieve_amd import bloom as bl
from tests.conftest import rng


def test_murmur_matches_oracle():
    g = rng(71)
    x = g.integers(-(2**62), 2**62, 200)
    y = g.integers(-(2**62), 2**62, 200)
    seeds = g.integers(0, 9, 200)
    got = bl.murmur_2x64(x, y, seeds.astype(np.uint64))
    for i in range(200):
        assert int(got[i]) == of.murmur_hash3_2x64(int(x[i]), int(y[i]), int(seeds[i]))


def _random_expr(g, depth=0):
    r = g.random()
    if depth > 3 or r < 0.35:
        return f"{int(g.integers(0, 4))}:{int(g.integers(-3, 6))}"
    if r < 0.5:
        return ("NOT " if g.random() < 0.5 else "!") + _random_expr(g, depth + 1)
    op = g.choice(["AND", "OR", "&", "|"])
    parts = [_random_expr(g, depth + 1) for _ in range(int(g.integers(2, 8)))]
    s = f" {op} ".join(parts)
    return f"({s})" if g.random() < 0.6 else s


def _eval_plan(plan: bl.Plan, leaf) -> np.ndarray:
    """The encoded plan's post-order ops on a stack (AND / OR pop their parameter count)."""
    stack = []
    t = 0
    for op, ps in zip(plan.ops, plan.params):
        if op == bl.TERM:
            stack.append(leaf(*plan.terms[t]))
            t += 1
        elif op == bl.NOT:
            stack.append(~stack.pop())
        elif op == bl.EMPTY:
            stack.append(np.ones(64, bool))
        else:
            xs = [stack.pop() for _ in ps]
            acc = xs[0]
            for x in xs[1:]:
                acc = (acc & x) if op == bl.AND else (acc | x)
            stack.append(acc)
    assert len(stack) == 1
    return stack[0]


def test_plans_evaluate_like_the_oracle_tree():
    g = rng(72)
    table = {}

    def leaf(f, v):
        if (f, v) not in table:
            table[(f, v)] = g.random(64) < 0.5
        return table[(f, v)]

    for i in range(300):
        text = _random_expr(g)
        want = of.eval_tree(of.parse_expression(text), leaf)
        for fan in (2, 3, 5, 64):
            plan = bl.compile_plan(bl.parse(text), fan)
            assert np.array_equal(_eval_plan(plan, leaf), want), text
            assert max(len(p) for p, o in zip(plan.params, plan.ops) if o in (bl.AND, bl.OR)) \
                <= max(fan, 2) if any(o in (bl.AND, bl.OR) for o in plan.ops) else True


def test_precedence_examples():
    """``EXPRESSION_SYNTAX.md``: NOT > AND > OR."""
    a = bl.compile_plan(bl.parse("1:10 OR 2:20 AND NOT 3:30"))
    b = bl.compile_plan(bl.parse("1:10 OR (2:20 AND (NOT 3:30))"))
    assert a.ops == b.ops and a.params == b.params and a.terms == b.terms
    assert bl.compile_plan(bl.parse("")).ops == [bl.EMPTY]
    assert bl.parse("42:100:0.5") == ("TERM", 42, 100)


def test_encoding_segments():
    exprs = ["0:100", "0:100 AND NOT 1:201", "", "(1:2 & 3:4) | !(5:6 & 7:-8:0.5)"]
    max_stack, data, offs = bl.parse_batch(exprs, 7)
    assert offs.shape == (32,) and max_stack == 3
    for i, e in enumerate(exprs):
        o = offs[8 * i : 8 * i + 8]
        assert all(x % 8 == 0 for x in o[0::2])
        plan = bl.compile_plan(bl.parse(e))
        assert data[o[0] : o[1]].tolist() == plan.ops
        ends = data[o[2] : o[3]].view(np.int32)
        assert ends.tolist() == [0] + np.cumsum([len(p) for p in plan.params]).tolist()
        hashes = data[o[6] : o[7]].view(np.uint64).reshape(-1, 7)
        for t, (f, v) in enumerate(plan.terms):
            assert [int(h) for h in hashes[t]] == \
                [of.murmur_hash3_2x64(f, v, s) for s in range(7)]


def test_expression_mapping_kat(kat):
    a, meta = kat
    assert bl.queries_to_expressions(a["expr_kat_in"]) == meta["expr_kat_out"]
    assert bl.queries_to_expressions(a["expr_kat_in"], [False, True]) == \
        meta["expr_kat_out_reverse"]
    sets = np.array([[[1, 2], [-1, -1]], [[-1, -1], [-1, -1]]])
    assert bl.sets_to_expressions(sets) == [of.sets_to_expression(sets[0]), ""]


def test_parse_op_schema():
    import retrieve_amd.st  # noqa: F401  (registers torch.ops.st.*)

    mx, (data, offs) = torch.ops.st.parse_expression_query_batch(
        ["1:100 AND 2:200", "NOT 3:300", "4:400 | 5:500"], torch.ones(3, dtype=torch.int64), 7
    )
    assert mx == 2 and data.dtype == torch.int8 and offs.dtype == torch.int64
    assert offs.shape == (24,)


def _compiled_stand_in(blob: np.ndarray, count: int):
    """What the compile pass gives the clause pass, built on the host: every plan a program
    (status 0) whose t-th TERM op carries the marker t + 1000 * plan in its position bits
    (kind TERM), other ops PASS; the first hash word's index in the header."""
    offs = blob[: 8 * count].reshape(count, 8)
    data = blob[8 * count :].view(np.uint8)
    hdr = np.zeros((count, 4), np.int32)
    prog = np.zeros((count, 64, 2), np.uint32)
    for b in range(count):
        o = offs[b]
        ops = data[o[0] : o[1]]
        hdr[b] = [0, ops.size, o[6] // 8, 0]
        t = 0
        for i, op in enumerate(ops.tolist()):
            if op == bl.TERM:
                prog[b, i] = [(t + 1000 * b) << 4 | (2 << 2), 7]
                t += 1
            else:
                prog[b, i] = [2, 0]
    return hdr, prog


def test_clause_plans_share_clauses():
    """The clause pass: ANDs of clauses (an OR of terms with nested ORs flattened, a term, NOT of
    either, EMPTY) over the batch's distinct clauses (the same set of tokens, in any order);
    other shapes stay programs. Each clause term's entry carries its program words and the
    index of its stored hashes."""
    import retrieve_amd.st as st

    exprs = ["(0:1 OR 0:2) AND 1:5", "(0:2 OR 0:1) AND NOT 2:7", "1:5", "",
             "0:1 OR 0:2", "NOT (0:1 AND 1:5)", "(0:1 AND 1:5) OR 2:3",
             "0:1 OR 0:2 OR 0:3 OR 0:4 OR 0:5 OR 0:6 OR 0:7", "1:5 AND (1:5) AND 2:7"]
    blob, count, _ = st.prepare_plans(exprs, 7, torch.device("cpu"))
    blob = blob.numpy()
    hdr, prog = _compiled_stand_in(blob, count)
    ptr, terms, desc, refs = st.clause_plans(blob, count, 7, hdr, prog, min_share=0)
    h64 = blob[8 * count :].view(np.uint64)

    def clause(slot):
        toks = set()
        for w0, _, lo, hi in terms[ptr[slot] : ptr[slot + 1]].tolist():
            hidx = lo | (hi << 32)
            toks.add(next((f, v) for f in range(3) for v in range(1, 8)
                          if h64[hidx] == of.murmur_hash3_2x64(f, v, 0)))
        return toks

    def plan(b):
        d = int(desc[b])
        if not d >> 31:
            return None
        first, n = (d >> 12) & 0x7FFFF, d & 0xFFF
        return [(frozenset(clause(r & 0x7FFF)), bool(r & 0x8000))
                for r in refs[first : first + n].tolist()]

    a, b5, c7 = frozenset({(0, 1), (0, 2)}), frozenset({(1, 5)}), frozenset({(2, 7)})
    assert plan(0) == [(a, False), (b5, False)]
    assert plan(1) == [(a, False), (c7, True)]
    assert plan(2) == [(b5, False)]
    assert plan(3) == []  # EMPTY: an AND of nothing
    assert plan(4) == [(a, False)]
    assert plan(5) is None and plan(6) is None  # NOT of an AND, OR of an AND
    assert plan(7) == [(frozenset((0, v) for v in range(1, 8)), False)]
    assert plan(8) == [(b5, False), (b5, False), (c7, False)]
    assert ptr.size - 1 == 4  # {0:1, 0:2}, {1:5}, {2:7}, {0:1 .. 0:7}
    # a term's entry carries its program words (the marker of its TERM op, place cleared)
    w0 = terms[ptr[0] : ptr[1], 0]
    assert sorted(((w0 >> 4) % 1000).tolist()) == [0, 1] and (w0 & 0xF == 0).all()
    assert (terms[:, 1] == 7).all()


def test_clause_plans_decline():
    """No tables when no plan has the clause form, there are more distinct clauses than the
    table holds, or the plans share too little of them."""
    import retrieve_amd.st as st

    blob, count, _ = st.prepare_plans(["NOT (0:1 AND 1:2)", "(0:1 AND 1:2) OR 2:3"], 7,
                                      torch.device("cpu"))
    hdr, prog = _compiled_stand_in(blob.numpy(), count)
    assert st.clause_plans(blob.numpy(), count, 7, hdr, prog) is None
    blob, count, _ = st.prepare_plans([f"0:{v} AND 1:{v}" for v in range(5)], 7,
                                      torch.device("cpu"))
    hdr, prog = _compiled_stand_in(blob.numpy(), count)
    assert st.clause_plans(blob.numpy(), count, 7, hdr, prog, cap=9, min_share=0) is None
    assert st.clause_plans(blob.numpy(), count, 7, hdr, prog, cap=10, min_share=0) is not None
    # ten clauses referenced once each: too little sharing for the table
    assert st.clause_plans(blob.numpy(), count, 7, hdr, prog) is None
    blob, count, _ = st.prepare_plans(["0:1 AND 1:2", "0:1 AND 1:3", "(0:1) AND 1:2"], 7,
                                      torch.device("cpu"))
    hdr, prog = _compiled_stand_in(blob.numpy(), count)
    assert st.clause_plans(blob.numpy(), count, 7, hdr, prog) is not None  # 6 refs, 3 terms


def _compiled_positions(blob: np.ndarray, count: int, hash_k: int, k: int, w: int):
    """The compile pass's output with real positions, built on the host: every plan a program
    whose TERM words hold the first k distinct stored hash % w as byte offsets p * 256 (the first
    repeated past them), other ops PASS; op counts and first hash words in the headers."""
    offs = blob[: 8 * count].reshape(count, 8)
    data = blob[8 * count :].view(np.uint8)
    h64 = blob[8 * count :].view(np.uint64)
    hdr = np.zeros((count, 4), np.int32)
    prog = np.zeros((count, 1024, 2), np.uint32)
    for b in range(count):
        o = offs[b]
        ops = data[o[0] : o[1]]
        h0 = int(o[6]) // 8
        hdr[b] = [0, ops.size, h0, 0]
        t = 0
        for i, op in enumerate(ops.tolist()):
            if op == bl.TERM:
                pos: list[int] = []
                for h in h64[h0 + t * hash_k : h0 + (t + 1) * hash_k].tolist():
                    if h % w not in pos and len(pos) < k:
                        pos.append(h % w)
                pos += [pos[0]] * (4 - len(pos))
                prog[b, i] = [(pos[0] * 256) << 4 | (pos[1] * 256) << 18,
                              pos[2] * 256 | (pos[3] * 256) << 16]
                t += 1
            else:
                prog[b, i] = [2, 0]
    return hdr, prog


def _probe(tables: np.ndarray, b: int, f: int) -> bool:
    """One document through plan b's probe table (the wave's ballots, lane by lane)."""
    w = [int(x) for x in tables.view(np.uint64)]
    t = w[w[b] : w[b + 1]]
    chunks, used, neg = t[0] >> 1, t[1], t[2]
    hit = [False] * 64  # clause j holds a hit
    for c in range(chunks):
        tm, cl = t[4 + 128 * c : 68 + 128 * c], t[68 + 128 * c : 132 + 128 * c]
        hits = sum(1 << l for l in range(64) if f & tm[l] == tm[l])
        hit = [hit[j] or bool(hits & cl[j]) for j in range(64)]
    bad = any(hit[j] == bool(neg >> j & 1) for j in range(64) if used >> j & 1)
    return not bad and not t[0] & 1


def test_probe_tables_match_the_search():
    """The scans' per-candidate Bloom probe, on the host: tables from ANDs of value-set clauses
    (NOT, EMPTY, one term, 64 terms, 130 terms over three chunks) evaluated on each document's
    row bits give the oracle's column search verdicts; other plan shapes, 65 clauses, and stack
    plans have no tables; a malformed plan matches nothing."""
    import retrieve_amd.st as st

    g = np.random.default_rng(5)
    n = 700
    attrs = g.integers(-1, 6, (n, 4, 1))
    words, offs = of.bloom_build(attrs, 3, bits_per_doc=64)
    bits = of.bloom_doc_bits(words, offs, n).view(np.uint64)
    wide = " AND ".join("(" + " OR ".join(f"{a}:{v}" for v in range(16)) + ")" for a in range(4))
    long = " AND ".join("(" + " OR ".join(f"{a}:{v}" for v in range(-8, 35)) + ")"
                        for a in (0, 2, 3)) + " AND NOT (1:2 OR 1:4)"
    exprs = ["", "1:3", "NOT 2:2", "(0:1 OR 0:2) AND NOT (3:4 OR 3:5) AND 1:0", wide,
             "NOT 0:0 AND NOT 1:1", "(2:1 OR 2:5 OR 2:-1) AND 0:3", long]
    blob, count, _ = st.prepare_plans(exprs, 7, torch.device("cpu"))
    blob = blob.numpy()
    hdr, prog = _compiled_positions(blob, count, 7, 3, 64)
    tables = st.probe_tables(blob, count, hdr, prog)
    assert int(tables[count]) - int(tables[count - 1]) == 4 + 3 * 128  # 131 terms: 3 chunks
    for b, e in enumerate(exprs):
        want = of.bloom_expression_mask(words, offs, n, e, 3, 7)
        got = np.array([_probe(tables, b, int(f)) for f in bits])
        assert np.array_equal(got, want), e[:60]
    hdr[2, 0] = 1  # malformed: matches nothing
    assert not any(_probe(st.probe_tables(blob, count, hdr, prog), 2, int(f)) for f in bits)
    many = " AND ".join(f"({a}:{v} OR {a}:{v + 1})" for a in range(4) for v in range(17))
    for other in ["NOT (0:1 AND 1:5)", "(0:1 AND 1:5) OR 2:3", many]:
        blob2, count2, _ = st.prepare_plans(exprs[:2] + [other], 7, torch.device("cpu"))
        hdr2, prog2 = _compiled_positions(blob2.numpy(), count2, 7, 3, 64)
        assert st.probe_tables(blob2.numpy(), count2, hdr2, prog2) is None, other
    hdr[1, 0] = 2  # a plan of the stack evaluation
    assert st.probe_tables(blob, count, hdr, prog) is None
