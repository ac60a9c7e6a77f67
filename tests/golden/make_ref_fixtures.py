"""Writes ``tests/golden/ref_cpu.npz`` / ``ref_cpu.json``: inputs and outputs of the reference's own
CPU ops (Meta's SilverTorch C++ vendored in rmnigm/retrieve), built from source by
``oracle/build_ref.py`` into ``oracle/_ref/``. Run in the build container only (the GPU box has
no reference checkout); the fixtures are data, committed, and read by ``tests/test_ref_fixtures.py``.

What they pin (and nothing else pins bit for bit):
- the expression parser's plan bytes (``expression_query_parser.cpp:343-425``,
  ``bloom_index_util.cpp:104-125``) for a set of expressions at several ``hash_k`` and
  ``max_sub_queries``;
- the CPU Bloom build's index words at the upstream width (``bloom_indexer.cpp:27-114``);
- the CPU Bloom search's column words (``bloom_index_search.cpp:88-166, 169-217``) and the
  partial response over probed clusters (``:219-345``);
- the CPU scorer's raw buffers (``fused_kmean_ann.cpp:86-228``): int32 dots and the fp16 divisor
  path, in layouts where its probe-then-doc slot order equals the CUDA op's (every probed
  cluster a whole number of 32-doc warps, or every one shorter than 32).

Usage: ``python oracle/build_ref.py && python tests/golden/make_ref_fixtures.py``."""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LIB = os.path.join(ROOT, "oracle", "_ref", "libsilvertorch_cpu_ref.so")

EXPRESSIONS = [
    "0:100", "0:100 AND NOT 1:201", "0:102 OR 1:203", "",
    "(0:1 OR 0:2 OR 0:3) AND 1:5", "NOT 3:7", "0:1 OR (1:2 AND NOT (2:3 OR 3:4))",
    "2:1 AND 2:2 AND 2:3 AND 2:4 AND 2:5 AND 2:6 AND 2:7",
    "0:1 OR 0:2 OR 0:3 OR 0:4 OR 0:5", "(0:1 OR 0:2) AND (1:3 OR 1:4) AND (2:5 OR 2:6)",
    "NOT NOT 1:2", "3:4:0.5 AND 1:2", "0:-3 OR 2:300", "(((0:4)))",
    "1:0 AND 1:1 AND 1:2 AND 1:3 AND 1:4 AND 1:5 AND 1:6 AND 1:7 AND 1:8 AND 1:9 AND 1:10",
]
PARSE_SETTINGS = [(7, 5), (3, 5), (7, 2), (7, 1), (5, 3)]  # (hash_k, max_sub_queries)


def _features(attrs: np.ndarray):
    """[N, C, A] (-1 pads) -> (feature ids = clause index, offsets [N * C + 1], values), the
    adapter's layout (``retrieve/src/retrieve/ops/official/adapter.py:45-62``)."""
    n, c, _ = attrs.shape
    valid = attrs != -1
    offsets = np.zeros(n * c + 1, np.int64)
    offsets[1:] = np.cumsum(valid.sum(-1).reshape(-1))
    values = attrs.reshape(-1)[valid.reshape(-1)].astype(np.int64)
    return np.arange(c, dtype=np.int32), offsets, values


def main() -> None:
    if not os.path.exists(LIB):
        raise SystemExit(f"{LIB} is missing: run python oracle/build_ref.py first")
    torch.ops.load_library(LIB)
    st = torch.ops.st
    g = np.random.Generator(np.random.PCG64(2026))
    arrays: dict[str, np.ndarray] = {}
    meta: dict = {"expressions": EXPRESSIONS, "parse_settings": PARSE_SETTINGS}

    # parser
    ks = torch.ones(len(EXPRESSIONS), dtype=torch.int64)
    stacks = []
    for i, (hk, msq) in enumerate(PARSE_SETTINGS):
        stack, (data, offs) = st.parse_expression_query_batch(EXPRESSIONS, ks, hk, True, msq)
        arrays[f"parse{i}_data"] = data.numpy().copy()
        arrays[f"parse{i}_offsets"] = offs.numpy().copy()
        stacks.append(int(stack))
    meta["parse_max_stack"] = stacks

    # Bloom build at the upstream width: 5000 docs, 4 attributes, up to 2 values each
    n, c = 5000, 4
    attrs = g.integers(0, 9, (n, c, 2)).astype(np.int64)
    attrs[g.random((n, c, 2)) < 0.3] = -1
    attrs[:, :, 1][attrs[:, :, 0] == -1] = -1  # values first, pads last
    arrays["bloom_attrs"] = attrs.astype(np.int16)
    fid, fo, fv = _features(attrs)
    builds = {"b5k3": (5.0, 3), "b2k2": (2.5, 2)}
    meta["bloom_builds"] = {k: list(v) for k, v in builds.items()}
    for name, (bm, k) in builds.items():
        words, boffs = st.bloom_index_build(torch.from_numpy(fid), torch.from_numpy(fo),
                                            torch.from_numpy(fv), bm, k, False)
        arrays[f"bloom_{name}_words"] = words.numpy().copy()
        arrays[f"bloom_{name}_offsets"] = boffs.numpy().copy()

    # Bloom search over the b5k3 index with the (7, 5) plans, k = 3
    words = torch.from_numpy(arrays["bloom_b5k3_words"])
    boffs = torch.from_numpy(arrays["bloom_b5k3_offsets"])
    data = torch.from_numpy(arrays["parse0_data"])
    offs = torch.from_numpy(arrays["parse0_offsets"])
    cols = st.bloom_index_search_batch(words, boffs, data, offs, 3, 7, False)
    arrays["search_words"] = cols.numpy().copy()

    # the partial response over probed clusters (rows = plans, 3 probes each)
    b = len(EXPRESSIONS)
    cuts = np.sort(g.choice(np.arange(1, n), 19, replace=False))
    starts = np.concatenate([[0], cuts]).astype(np.int64)
    sizes = np.diff(np.concatenate([starts, [n]])).astype(np.int64)
    probe = np.stack([g.permutation(20)[:3] for _ in range(b)])
    sel_off, sel_len = starts[probe], sizes[probe]
    sel_len[0, 0] = 0
    qpi = g.integers(0, b, b).astype(np.int64)
    arrays["partial_starts"], arrays["partial_lengths"] = sel_off, sel_len
    arrays["partial_plan_index"] = qpi
    for tag, index in (("", None), ("_qpi", torch.from_numpy(qpi))):
        cum, first, w = st.bloom_index_search_batch_return_partial_response(
            words, boffs, data, offs, torch.from_numpy(sel_off), torch.from_numpy(sel_len), 3, 7,
            index)
        arrays[f"partial{tag}_cumsum"] = cum.numpy().copy()
        arrays[f"partial{tag}_first"] = first.numpy().copy()
        arrays[f"partial{tag}_words"] = w.numpy().copy()

    # the CPU scorer in slot orders equal to the CUDA op's
    d = 128
    emb = g.integers(-128, 128, (384, d), dtype=np.int8)
    q = g.integers(-128, 128, (3, d), dtype=np.int8)
    arrays["scorer_emb"], arrays["scorer_queries"] = emb, q
    layouts = {
        # whole warps: clusters of 64, 96, 32, 128 docs
        "warps": (np.array([0, 64, 160, 192, 320], np.int64),
                  np.array([[1, 3, 0], [2, 1, 3], [0, 2, 1]], np.int64),
                  np.array([64, 96, 32, 128], np.int64)),
        # short clusters only (< 32 docs)
        "short": (np.array([0, 5, 36, 40, 63], np.int64),
                  np.array([[1, 3], [2, 0], [3, 1]], np.int64),
                  np.array([5, 31, 4, 23], np.int64)),
    }
    for name, (coffs, cids, csizes) in layouts.items():
        lens = csizes[cids]
        width = int(lens.sum(1).max())
        arrays[f"scorer_{name}_offsets"] = coffs
        arrays[f"scorer_{name}_ids"] = cids
        arrays[f"scorer_{name}_lengths"] = lens
        for div in (-1, 64, 3):
            sc, ix = st.fused_kmean_ann(torch.from_numpy(coffs), torch.from_numpy(cids),
                                        torch.from_numpy(lens), torch.from_numpy(emb),
                                        torch.from_numpy(q), width, None, -1, div, None, None)
            arrays[f"scorer_{name}_div{div}_scores"] = sc.numpy().copy()
            arrays[f"scorer_{name}_div{div}_indices"] = ix.numpy().copy()
        meta[f"scorer_{name}_width"] = width

    np.savez_compressed(os.path.join(HERE, "ref_cpu.npz"), **arrays)
    with open(os.path.join(HERE, "ref_cpu.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(f"wrote {len(arrays)} arrays", file=sys.stderr)


if __name__ == "__main__":
    main()
