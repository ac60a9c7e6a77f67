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
