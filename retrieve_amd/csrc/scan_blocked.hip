// The large-batch dense scans' C entry points; the kernels are in scan_blocked.h, instantiated
// per operand type in scan_blocked_{i8,bf16,f16,bits}.hip.
#include "scan_blocked.h"

using namespace rt;

extern "C" size_t rt_blocked_scan_topk_workspace(int64_t B, int64_t N, int64_t row_bytes,
                                                 int64_t k, int masked) {
  // (the most workgroups any device runs: the workspace covers every CU count)
  return blk_plan(B, N, k, row_bytes, kMaxResidentWorkgroups, false, masked != 0).total;
}

// dtype: 0 int8 (int32 scores), 1 bf16, 2 fp16, 3 fp32 (float scores); D elements per row.
extern "C" int rt_blocked_scan_topk(const void* queries, int64_t B, const void* items, int64_t N,
                                    int64_t D, int64_t k, int dtype, const uint64_t* mask,
                                    int64_t mask_words, int64_t* out_ids, void* out_scores,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  switch (dtype) {
    case 0:
      return blocked_scan_i8(queries, B, items, N, D, k, mask, mask_words, out_ids, out_scores,
                             workspace, workspace_bytes, stream);
    case 1:
      return blocked_scan_bf16(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                               out_scores, workspace, workspace_bytes, stream);
    case 2:
      return blocked_scan_f16(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                              out_scores, workspace, workspace_bytes, stream);
    case 3:
      return blocked_scan_f32(queries, B, items, N, 4 * D, k, mask, mask_words, out_ids,
                              out_scores, workspace, workspace_bytes, stream);
    default:
      set_error("blocked scan dtype must be 0 (int8), 1 (bf16), 2 (fp16) or 3 (fp32), got %d",
                dtype);
      return kInvalidType;
  }
}


// The blocked scan with the exact clause filter of rt_clause_filter tested per candidate that
// passes the mask (required): the clause prep pass writes the row sets after the scan's
// workspace.
extern "C" size_t rt_blocked_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t row_bytes,
                                                         int64_t k, int64_t C, int64_t V) {
  return align_up(rt_blocked_scan_topk_workspace(B, N, row_bytes, k, 1), 256) +
         clause_prep_workspace(B, C, V);
}

extern "C" int rt_blocked_scan_topk_clauses(const void* queries, int64_t B, const void* items,
                                            int64_t N, int64_t D, int64_t k, int dtype,
                                            const uint64_t* mask, int64_t mask_words,
                                            int64_t mask_t_stride, const void* item_attrs,
                                            int attr_bytes, int64_t C,
                                            int64_t A, const int8_t* clause_is_reverse,
                                            const int64_t* query_values, int64_t V,
                                            int64_t* out_ids, void* out_scores, void* workspace,
                                            size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(dtype >= 0 && dtype <= 3, "blocked scan dtype must be 0 (int8), 1 (bf16), 2 "
               "(fp16) or 3 (fp32), got %d", dtype);
  RT_CHECK_ARG(mask != nullptr, "the blocked scan tests exact clauses only together with a mask");
  RT_CHECK_ARG(B >= 0 && B <= (int64_t{1} << 21) && N >= 0, "B in [0, 2^21] and N >= 0");
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(C));
  RT_CHECK_ARG(A >= 0 && A <= 4096 && V >= 1 && V <= 4096, "A must be in [0, 4096] and V in "
               "[1, 4096]");
  RT_CHECK_ARG(attr_bytes == 2 || attr_bytes == 4 || attr_bytes == 8,
               "attr_bytes must be 2, 4 or 8 (int16, int32, int64 attributes)");
  if (B == 0) return kOk;
  RT_CHECK_ARG(C == 0 || (clause_is_reverse != nullptr && query_values != nullptr),
               "clause_is_reverse and query values must not be null");
  RT_CHECK_ARG(C * A == 0 || N == 0 || item_attrs != nullptr, "item attrs are null");
  const int64_t elem = dtype == 0 ? 1 : (dtype == 3 ? 4 : 2);
  const size_t scan_bytes = align_up(rt_blocked_scan_topk_workspace(B, N, elem * D, k, 1), 256);
  const size_t need = scan_bytes + clause_prep_workspace(B, C, V);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  ClauseCheck f;
  if (C > 0 && N > 0) {
    const int st = clause_prepare(query_values, B, C, V, clause_is_reverse,
                                  static_cast<char*>(workspace) + scan_bytes,
                                  workspace_bytes - scan_bytes, &f, stream);
    if (st != kOk) return st;
    f.attrs = item_attrs;
    f.attr_bytes = attr_bytes;
    f.A = static_cast<int>(A);
  }
  switch (dtype) {
    case 0:
      return blocked_scan_i8(queries, B, items, N, D, k, mask, mask_words, out_ids, out_scores,
                             workspace, scan_bytes, stream, f,
                             mask_t_stride);
    case 1:
      return blocked_scan_bf16(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                               out_scores, workspace, scan_bytes, stream, f, mask_t_stride);
    case 2:
      return blocked_scan_f16(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                              out_scores, workspace, scan_bytes, stream, f, mask_t_stride);
    default:
      return blocked_scan_f32(queries, B, items, N, 4 * D, k, mask, mask_words, out_ids,
                              out_scores, workspace, scan_bytes, stream, f, mask_t_stride);
  }
}
