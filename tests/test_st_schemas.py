"""The ``torch.ops.st`` namespace as the reference's loader checks it: every one of its
``REQUIRED_OPS`` (``retrieve/src/retrieve/ops/official/__init__.py:46-54``) is registered, with
the schema pinned at Meta's 21aa35e plus the adapted ``search``
(``retrieve/tests/parity/test_official.py:68-122``), and the adapted extras with theirs
(``silvertorch/silvertorch/ops/csrc/fork_search.cpp:13-49``, ``bloom_index_search.cpp:576-601``,
``bloom_indexer.cpp:117-136``). Registration needs no GPU."""

from __future__ import annotations

import pytest

REQUIRED_OPS = (
    "fused_kmean_ann",
    "fused_kmean_ann_with_partial_masks",
    "bloom_index_build",
    "parse_expression_query_batch",
    "bloom_index_search_batch",
    "bloom_index_search_batch_return_partial_response",
    "search",
)

PINNED = {
    "fused_kmean_ann": (
        "st::fused_kmean_ann(Tensor cluster_offsets, Tensor cluster_ids, Tensor cluster_length, "
        "Tensor embeddings, Tensor queries, int max_tensor_size_per_row, "
        "Tensor? filtering_bit_mask=None, int invalid_index_value=-1, int divisor_for_int8=-1, "
        "Tensor? filtering_bit_index=None, Tensor? per_embedding_scale=None) -> (Tensor, Tensor)"
    ),
    "fused_kmean_ann_with_partial_masks": (
        "st::fused_kmean_ann_with_partial_masks(Tensor cluster_offsets, Tensor cluster_ids, "
        "Tensor cluster_length, Tensor embeddings, Tensor queries, int max_tensor_size_per_row, "
        "Tensor partial_mask_column_counts_cumsum, "
        "Tensor partial_mask_first_item_offset_in_column, "
        "Tensor partial_mask_column_results, int invalid_index_value=-1, int divisor_for_int8=-1, "
        "Tensor? filtering_bit_index=None, Tensor? per_embedding_scale=None, "
        "Tensor? cluster_warp_size=None, Tensor? cluster_warp_rounded_length_cumsum=None, "
        "Tensor? cluster_remaining_length_cumsum=None, Tensor? cluster_warp_size_cumsum=None, "
        "int total_cluster_rounded_warps=0, int total_cluster_remaining_warps=0) "
        "-> (Tensor, Tensor)"
    ),
    "bloom_index_build": (
        "st::bloom_index_build(Tensor feature_ids, Tensor feature_offsets, Tensor feature_values, "
        "float b_multiplier, int k, bool fast_build=False) -> (Tensor, Tensor)"
    ),
    "parse_expression_query_batch": (
        "st::parse_expression_query_batch(str[] expressions, Tensor silvertorch_ks, "
        "int bloom_hash_k, bool return_query_plan=True, int max_sub_queries=5) -> (int, Tensor[])"
    ),
    "bloom_index_search_batch": (
        "st::bloom_index_search_batch(Tensor bloom_index, Tensor bloom_bundle_b_offsets, "
        "Tensor bloom_query_plans_data, Tensor bloom_query_plans_offsets, int k, int hash_k, "
        "bool return_bool_mask=True) -> Tensor"
    ),
    "bloom_index_search_batch_return_partial_response": (
        "st::bloom_index_search_batch_return_partial_response(Tensor bloom_index, "
        "Tensor bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
        "Tensor bloom_query_plans_offsets, Tensor selected_cluster_offsets, "
        "Tensor selected_cluster_lengths, int k, int hash_k, Tensor? query_plan_index=None) "
        "-> (Tensor, Tensor, Tensor)"
    ),
    "search": (
        "st::search(Tensor query, Tensor probe_ids, Tensor cluster_offsets, Tensor cluster_sizes, "
        "Tensor item_codes, Tensor sort_perm, Tensor global_scale, int k, "
        "int max_tensor_size_per_row, int divisor_for_int8=-1, Tensor? filtering_bit_mask=None, "
        "Tensor? bloom_index=None, Tensor? bloom_bundle_b_offsets=None, Tensor? plans=None, "
        "int plan_count=0, int max_stack_size=0, Tensor? query_plan_index=None, int bloom_k=0, "
        "int hash_k=0, Tensor? item_clause_attrs=None, Tensor? clause_slots=None, "
        "Tensor? clause_is_reverse=None, Tensor? query_clause_attrs=None) -> (Tensor, Tensor)"
    ),
}

EXTRAS = {
    "probe_prep": (
        "st::probe_prep(Tensor query, Tensor probe_ids, Tensor cluster_offsets, "
        "Tensor cluster_sizes) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
        "Tensor, Tensor)"
    ),
    "bloom_index_build_fixed": (
        "st::bloom_index_build_fixed(Tensor feature_ids, Tensor feature_offsets, "
        "Tensor feature_values, int bits_per_doc, int k, bool fast_build=False) "
        "-> (Tensor, Tensor)"
    ),
    "bloom_index_search_batch_prepared": (
        "st::bloom_index_search_batch_prepared(Tensor bloom_index, Tensor bloom_bundle_b_offsets, "
        "Tensor plans, int plan_count, int max_stack_size, int k, int hash_k, "
        "bool return_bool_mask=False) -> Tensor"
    ),
    "bloom_index_search_batch_return_partial_response_prepared": (
        "st::bloom_index_search_batch_return_partial_response_prepared(Tensor bloom_index, "
        "Tensor bloom_bundle_b_offsets, Tensor plans, int plan_count, int max_stack_size, "
        "Tensor selected_cluster_offsets, Tensor selected_cluster_lengths, int k, int hash_k, "
        "Tensor? query_plan_index, int max_columns) -> (Tensor, Tensor, Tensor)"
    ),
}


@pytest.fixture(scope="module")
def st_ops():
    import torch

    import retrieve_amd.st  # noqa: F401  (registers torch.ops.st.*)

    return torch.ops.st


def test_the_reference_loader_finds_every_required_op(st_ops):
    """``_try_load`` returns the namespace only when ``hasattr(ops, name)`` holds for every
    required op (``ops/official/__init__.py:161-167``)."""
    assert sorted(PINNED) == sorted(REQUIRED_OPS)
    missing = [name for name in REQUIRED_OPS if not hasattr(st_ops, name)]
    assert not missing


@pytest.mark.parametrize("name", sorted(PINNED) + sorted(EXTRAS))
def test_schema_is_pinned(st_ops, name):
    want = PINNED.get(name) or EXTRAS[name]
    assert str(getattr(st_ops, name).default._schema) == want


@pytest.mark.parametrize("name", sorted(PINNED) + sorted(EXTRAS))
def test_ops_are_functional(st_ops, name):
    """No mutable argument and no alias in any schema: the ops are functional, as the
    reference's compile gate requires (``retrieve/tests/compile/test_export_kernel_ref.py:
    115-143``)."""
    schema = getattr(st_ops, name).default._schema
    assert not schema.is_mutable
    for arg in list(schema.arguments) + list(schema.returns):
        assert arg.alias_info is None


def test_every_op_has_a_fake(st_ops):
    """``torch.compile`` traces the ops through their fakes (``silvertorch/silvertorch/ops/
    _fake.py:26-219``): each of them has a Meta-capable abstract implementation."""
    import torch

    for name in sorted(PINNED) + sorted(EXTRAS):
        op = getattr(st_ops, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Meta") or \
            torch._library.simple_registry.singleton.find(op.name()).fake_impl.kernel is not None, \
            name
