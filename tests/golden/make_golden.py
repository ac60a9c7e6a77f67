"""Writes ``tests/golden/kat.npz`` and ``tests/golden/kat.json``: the known-answer vectors the
reference's own tests hold for this path, as data (inputs + expected outputs). Nothing here
imports or runs the reference; each vector cites the reference test it comes from.

Run: ``python tests/golden/make_golden.py`` (needs torch on CPU for one seeded input, the
same generator call the reference test makes).
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    meta: dict[str, object] = {}

    # silvertorch/silvertorch/ops/csrc/tests/test_fused_kmean_ann.py:353-380:
    # doc0 = [1, 2, 0...], doc1 = [3, 4, 0...], query = [5, 6, 0...] -> 17, 39 (zero-padded)
    items = np.zeros((2, 16), np.int8)
    items[0, :2] = [1, 2]
    items[1, :2] = [3, 4]
    q = np.zeros((1, 16), np.int8)
    q[0, :2] = [5, 6]
    arrays["int8_kat_items"] = items
    arrays["int8_kat_query"] = q
    arrays["int8_kat_scores"] = np.array([17, 39], np.int32)

    # retrieve/tests/correctness/test_quantize.py:195-199
    arrays["popcount_kat_in"] = np.array([0, 1, 2, 3, -1, 0x5555555555555555], np.int64)
    arrays["popcount_kat_out"] = np.array([0, 1, 1, 2, 64, 32], np.int32)

    # evaluation/tests/bench/test_oracle.py:300-324: items 24x8 (torch CPU generator, seed 1),
    # item 13 a copy of item 2, 6 queries (query 0 = item 2), 3 masks > 0.3 with items 2 and 13
    # forced in, query rows use masks qa = [0, 1, 2, 0, 1, 2]; the top-6 of query 5 ends in
    # [2, 13]: the exact tie, the lower id first.
    g = torch.Generator().manual_seed(1)
    item_embs = torch.randn(24, 8, generator=g)
    item_embs[13] = item_embs[2]
    queries = torch.randn(6, 8, generator=g)
    queries[0] = item_embs[2]
    masks = torch.rand(3, 24, generator=g) > 0.3
    masks[:, [2, 13]] = True
    arrays["tie_items"] = item_embs.numpy()
    arrays["tie_queries"] = queries.numpy()
    arrays["tie_masks"] = masks.numpy()
    arrays["tie_qa"] = np.array([0, 1, 2, 0, 1, 2], np.int64)
    meta["tie_k"] = 6
    meta["tie_row5_tail"] = [2, 13]

    # retrieve/tests/correctness/test_quantize.py:102-121: +-abs_max -> +-127
    arrays["quant_extremes_in"] = np.array(
        [[1.0, -1.0, 0.5, -0.25, 1e-8, 0.0, 0.7, -0.7],
         [2.0, -2.0, 1.0, -0.5, 1e-8, 0.0, 1.4, -1.4]], np.float32)
    # retrieve/tests/parity/test_official.py:682-689: 127 * x / 2.54 lands on .5 for
    # x = +-0.01 and +-1.27; torch.round is half-to-even, so the codes are 0, 0, 64, -64.
    row = np.zeros(8, np.float32)
    row[0] = 2.54
    row[1:5] = [0.01, -0.01, 1.27, -1.27]
    arrays["quant_half_in"] = row[None, :]
    arrays["quant_half_codes"] = np.array([[127, 0, 0, 64, -64, 0, 0, 0]], np.int8)

    # retrieve/tests/parity/test_official.py:229-245, 353-366: the README corpus
    arrays["readme_attrs"] = np.array(
        [[[100, -1], [200, 201]], [[100, 101], [200, -1]], [[102, -1], [202, -1]],
         [[100, -1], [200, 203]]], np.int64)
    meta["readme_queries"] = ["0:100", "0:100 AND NOT 1:201", "0:102 OR 1:203"]
    meta["readme_hits"] = [[0, 1, 3], [1, 3], [2, 3]]
    meta["readme_b_multiplier"] = 5.0
    meta["readme_build_k"] = 3
    meta["readme_hash_k"] = 7

    # retrieve/tests/parity/test_official.py:510-514: expression mapping
    arrays["expr_kat_in"] = np.array([[7, -1], [7, 9], [-1, -1]], np.int64)
    meta["expr_kat_out"] = ["0:7", "0:7 AND 1:9", ""]
    meta["expr_kat_out_reverse"] = ["0:7", "0:7 AND NOT 1:9", ""]

    # SMHasher's published verification value of MurmurHash3_x64_128
    meta["murmur3_x64_128_verification"] = 0x6384BA69

    np.savez(os.path.join(HERE, "kat.npz"), **arrays)
    with open(os.path.join(HERE, "kat.json"), "w") as f:
        json.dump(meta, f, indent=1)


if __name__ == "__main__":
    main()
