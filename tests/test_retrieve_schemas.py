"""The ``torch.ops.retrieve`` namespace as the reference's op-registry gate checks it
(``retrieve/tests/compile/test_export_kernel_ref.py:115-143``): after the backend's import it
holds exactly the reference's seven ops, each with the argument names and kinds of its
same-named twin in ``retrieve.ops.reference`` (restated below from
``retrieve/src/retrieve/ops/reference/*.py``), none mutable or aliased. The ops this build adds
live in ``torch.ops.retrieve_amd`` and each has a fake for ``torch.compile``. Registration needs
no GPU."""

from __future__ import annotations

import pytest

# (argument name, kind) per op, as ``inspect.signature`` of the reference twin gives them
# (``ops/reference/clause_mask.py:9-26``, ``clause_compact.py:9-13``,
# ``fused_masked_knn_topk.py:9-15``, ``gemv_scores.py:9``, ``oporp_1bit_match_topk.py:18-35``).
TWINS = {
    "clause_mask": [("item_clause_attrs", "Tensor"), ("clause_is_reverse", "Tensor"),
                    ("query_clause_attrs", "Tensor")],
    "clause_mask_scores": [("scores", "Tensor"), ("item_clause_attrs", "Tensor"),
                           ("clause_is_reverse", "Tensor"), ("query_clause_attrs", "Tensor")],
    "clause_compact": [("item_clause_attrs", "Tensor"), ("clause_is_reverse", "Tensor"),
                       ("query_clause_attrs", "Tensor")],
    "fused_masked_knn_topk": [("query", "Tensor"), ("item_embs", "Tensor"),
                              ("positive_indices", "Tensor"), ("counts", "Tensor"),
                              ("k", "int")],
    "gemv_scores": [("query", "Tensor"), ("item_embs_t", "Tensor")],
    "oporp_1bit_match_topk_full": [("query_bits", "Tensor"), ("item_bits", "Tensor"),
                                   ("k", "int")],
    "oporp_1bit_match_topk_indirect": [("query_bits", "Tensor"), ("item_bits", "Tensor"),
                                       ("k", "int"), ("positive_indices", "Tensor"),
                                       ("counts", "Tensor")],
}

# the gate's schema-type → annotation map (``test_export_kernel_ref.py:80``)
_SCHEMA_KIND = {"Tensor": "Tensor", "float": "float", "SymInt": "int", "int": "int",
                "bool": "bool"}

EXTRAS = (
    "int8_scan_topk", "int8_scan_topk_clauses", "dense_scan_topk", "dense_scan_topk_clauses",
    "hamming_scan_topk", "hamming_scan_topk_clauses", "clause_bits", "mask_compact",
    "int8_candidates_topk", "int8_rerank_topk", "quantize_int8", "quantize_int8_global",
    "pack_mask", "pack_signs", "bloom_search_cols", "bloom_doc_bits", "scan_topk_bloom_clauses",
)


def _schemas(ns: str) -> dict:
    import torch

    import retrieve_amd.hip  # noqa: F401  (registers torch.ops.retrieve / retrieve_amd)
    import retrieve_amd.st  # noqa: F401  (registers torch.ops.st and the transposed search)

    pre = ns + "::"
    return {s.name.removeprefix(pre): s for s in torch._C._jit_get_all_schemas()
            if s.name.startswith(pre)}


def test_retrieve_namespace_is_exactly_the_reference_set():
    assert sorted(_schemas("retrieve")) == sorted(TWINS)


def test_every_op_has_a_same_signature_reference_twin():
    for name, schema in _schemas("retrieve").items():
        got = [(a.name, _SCHEMA_KIND[str(a.type)]) for a in schema.arguments]
        assert got == TWINS[name], f"{name}: op schema {got} vs reference twin {TWINS[name]}"


def test_no_op_declares_a_mutable_argument():
    for ns in ("retrieve", "retrieve_amd"):
        for name, schema in _schemas(ns).items():
            assert schema.is_mutable is False, name
            assert all(a.alias_info is None for a in schema.arguments), name


def test_the_extra_ops_live_in_their_own_namespace():
    assert sorted(_schemas("retrieve_amd")) == sorted(EXTRAS)


@pytest.mark.parametrize("ns,names", [("retrieve", sorted(TWINS)),
                                      ("retrieve_amd", sorted(EXTRAS))])
def test_every_op_has_a_fake(ns, names):
    import torch

    _schemas(ns)
    for name in names:
        op = getattr(getattr(torch.ops, ns), name).default
        entry = torch._library.simple_registry.singleton.find(op.name())
        assert entry.fake_impl.kernel is not None, name
