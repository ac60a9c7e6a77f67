// The blocked scan over int8 rows (scan_blocked.h).
#include "scan_blocked.h"

namespace rt {

int blocked_scan_i8(const void* queries, int64_t B, const void* items, int64_t N,
                    int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                    hipStream_t stream, const ClauseCheck& clause, int64_t mask_t_stride) {
  return run_blocked<I8x32>(queries, B, items, N, row_bytes, k, mask, mask_words, out_ids,
                         out_scores, workspace, workspace_bytes, stream, I8x32::kind, clause,
                         mask_t_stride);
}

}  // namespace rt
