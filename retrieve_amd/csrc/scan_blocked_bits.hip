// The blocked scan over 512-bit codes on the fp4 matrix cores (scan_blocked.h).
#include "scan_blocked.h"

namespace rt {

bool blocked_hamming_fits(int64_t B, int64_t W, int64_t k, bool masked) {
  if (W != 8 || k < 1 || k > kMaxK) return false;
  const bool wide = blk_choose_wide(8 * W, B, k, true, masked);
  return blk_stages(8 * W, blk_capw(k, blk_rows(8 * W, wide, true)), wide, true, masked) != 0;
}

size_t blocked_hamming_workspace(int64_t B, int64_t N, int64_t W, int64_t k, bool masked) {
  return blk_plan(B, N, k, 8 * W, kMaxResidentWorkgroups, true, masked).total;
}

int blocked_hamming(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
                    int64_t W, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, int score_kind, void* workspace,
                    size_t workspace_bytes, hipStream_t stream, const ClauseCheck& clause,
                    int64_t mask_t_stride) {
  return run_blocked<BitsF4>(query_bits, B, item_bits, N, 8 * W, k, mask, mask_words, out_ids,
                              out_scores, workspace, workspace_bytes, stream, score_kind, clause,
                              mask_t_stride);
}

}  // namespace rt
