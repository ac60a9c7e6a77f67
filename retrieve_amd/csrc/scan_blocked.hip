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

