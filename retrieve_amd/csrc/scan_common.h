// The scan → merge pipeline shared by the int8, bf16 and Hamming scans: launch planning,
// workspace layout and the merge kernel's interface.
//
// One top-k call is up to four launches on the caller's stream, with no host sync:
//   1. seed scan over a strided sample of the items (only when N is large),
//   2. seed merge: the exact k-th best composite of the sample per query (a lower bound on the
//      k-th best over all items),
//   3. main scan over all items, appending only composites >= that bound,
//   4. final merge: the exact top-k over the main scan's lists.
#pragma once

#include <cmath>

#include "bloom_prog.h"
#include "clause_check.h"
#include "rt_common.h"

namespace rt {

constexpr int kScanWaves = 4;       // waves per scan workgroup
constexpr int kScanThreads = kScanWaves * kWave;
constexpr int kTile = 16;           // items per MFMA tile
constexpr int kMergeThreads = 512;
constexpr int64_t kMaxK = 1024;
// The 1-bit full scan's bound: above kMaxK it selects by counting scores (a score takes only
// 64 W + 1 values).
constexpr int64_t kMaxKHamming = 8192;
constexpr int64_t kMaxMergeSlots = 8192;  // lists a query's merge reads

// The scan kernels' arguments (the element type of queries/items is the kernel's).
struct ScanArgs {
  const void* queries;     // [B, D]
  int64_t B;
  const void* items;       // [N, D] (or [N, W] words)
  int64_t n_rows;          // rows of this pass's index space
  int64_t row_stride;      // item index = row * row_stride (the seed's sample strides)
  int64_t strip;           // rows per workgroup, a multiple of kTile
  int k;
  int qpw;                 // queries per wave (a query group), for scans that vary it
  int capw;                // list capacity (>= k + the appends one tile can make)
  const uint64_t* tau_in;  // [B] lower bounds (composites) or null
  const uint64_t* mask;    // [B, mask_words] item bits, item d at bit 63 - d % 64, or null
  int64_t mask_words;
  const uint64_t* mask_t;  // the mask transposed, [ceil(N/64), mask_t_stride] (blocked scan)
  int64_t mask_t_stride;
  int64_t mask_t_rows;     // its word rows, ceil(N/64)
  uint64_t* lists;         // [slots, qpw, capw]
  int* counts;             // [slots, qpw]
  ClauseCheck clause;      // exact clauses tested per candidate (active null: none; the
                           // scans of scan_mfma.hip)
  BloomProbe probe;        // Bloom plans probed per candidate, plan b for query b (doc_bits
                           // null: none; the scans of scan_mfma.hip)
  int probe_lds;           // main pass: the query group's Bloom clause tables copied to LDS
  int clause_lds;          // main pass: the query group's set bitmaps copied to LDS
  const uint32_t* run_if;  // not null: the pass runs only if *run_if != 0 (a fallback pass)
};

enum ScoreKind : int {
  kScoreI32 = 0,       // the key is an int32 score; write int32
  kScoreF32FromI32 = 1,  // the key is an int32 score; write it as float
  kScoreF32 = 2,       // the key is a float score; write float
};

struct MergeArgs {
  const uint64_t* lists;
  const int* counts;   // per-list lengths (unused when flat)
  bool flat;           // lists is [B, gx * waves] one-entry lists, contiguous per query
  int capw;
  int qpw;          // queries per list slot (a slot holds one list per such query)
  int64_t S;        // list slots per query: query q's lists are slots [q/qpw * S, +S)
  int64_t B;
  int k;
  uint64_t* tau_out;   // threshold mode: [B]
  bool tau_keep;       // threshold mode: write max(tau_base[q] (or tau_out[q]), the new bound)
  const uint64_t* tau_base;  // threshold mode with tau_keep: the bound to keep, or null
  uint64_t* tau2_out;  // threshold mode, not null: also the k2-th composite (k2 < k), at least
  int k2;              // the k-th (0 when fewer than k2 entries exist)
  const uint32_t* run_if;    // not null: the merge runs only if *run_if != 0 (a fallback merge)
  // Speculative bounds: in threshold mode block 0 clears *spec_flag; in final mode a query that
  // holds fewer than k entries although its bound spec_tau[q] is above the safe safe_tau[q]
  // sets it (its scan may have dropped items between the two bounds).
  uint32_t* spec_flag;
  const uint64_t* spec_tau;
  const uint64_t* safe_tau;  // null: 0 (no bound)
  int64_t* out_ids;    // final mode: [B, k]
  void* out_scores;    // final mode: [B, k]
  int score_kind;
  ClauseCheck clause;  // lists (not flat) whose entries may fail exact clauses: those entries
                       // count as empty (active null: none)
  // Room for a split merge (null: none): [B, kMergeParts, k] composites. launch_merge then
  // splits a small batch's lists into parts, each a workgroup keeping its part's best k there,
  // and merges those (flat) in a second launch.
  uint64_t* part_buf;
  // (set by launch_merge) parts per query, and the parts' output in the first launch
  int parts;
  uint64_t* part_out;
};

// Parts of a split merge at most, and the largest batch that splits.
constexpr int kMergeParts = 8;
constexpr int64_t kMergeSplitMaxB = 32;

// The seed pass samples blocks of kSeedBlock consecutive rows spread evenly over the table
// (row_stride = N / sample rows > 1), so each block is read as one contiguous run; sample row r
// is item sample_item(r, stride). The sample's k-th best is a lower bound of the table's for any
// choice of rows. The sample size is a multiple of kSeedBlock, and the last block ends at most at
// N - 1 - (kSeedBlock - 1) (stride - 1).
constexpr int64_t kSeedBlock = 256;

__host__ __device__ inline int64_t sample_item(int64_t r, int64_t stride) {
  return stride == 1 ? r : (r / kSeedBlock) * (kSeedBlock * stride) + (r % kSeedBlock);
}

// The rank m whose m-th best sampled composite bounds the k-th best of all items with
// overwhelming probability when one item in `stride` is sampled: the top k hold about
// lam = k / stride sampled items (Poisson), and m = lam + 5 sqrt(lam) + 4 exceeds that count
// all but very rarely. A query that nevertheless ends with fewer than k entries behind the bound
// raises a flag, and a fallback pass without it keeps the results exact.
inline int sample_rank(int64_t k, int64_t stride) {
  const double lam = static_cast<double>(k) / static_cast<double>(stride);
  const int64_t m = static_cast<int64_t>(std::ceil(lam + 5.0 * std::sqrt(lam) + 4.0));
  return static_cast<int>(m < k ? m : k);
}

// One pass of a scan: its grid and list geometry.
struct PassPlan {
  int64_t n_rows = 0;
  int64_t row_stride = 1;
  int64_t strip = 0;
  int64_t gx = 0;
  int64_t S = 0;           // lists per query
  int capw = 0;
  size_t lists_bytes = 0;
  size_t counts_bytes = 0;
};

struct ScanPlan {
  int64_t qpg = 16;        // queries per workgroup row (grid.y groups)
  int64_t n_qgroups = 0;
  bool seeded = false;
  PassPlan seed;
  PassPlan main;
  // workspace layout (byte offsets)
  size_t off_lists = 0, off_counts = 0, off_tau = 0, off_flag = 0, off_parts = 0, total = 0;
  bool split = false;  // room for a split merge at off_parts
};

// Upper bound on a main pass's workgroups (the workspace functions size for it).
constexpr int64_t kMaxResidentWorkgroups = 4096;
// Main-pass workgroups per CU: two, each streaming its share of every window of the table
// (measured best on MI355X; more workgroups only add candidate lists).
constexpr int64_t kMainWorkgroupsPerCU = 2;

// Main-pass workgroups for the current device: CUs x kMainWorkgroupsPerCU.
int64_t main_workgroups();

// The 1-bit Hamming top-k on the int8 matrix cores (scan_blocked_bits.hip): codes of W 64-bit
// words (W == 8), scores 64 W - 2 popcount(q ^ x) written as score_kind (kScoreI32 or
// kScoreF32FromI32); `clause`: exact clauses tested per candidate (with a mask only).
bool blocked_hamming_fits(int64_t B, int64_t W, int64_t k, bool masked);  // lists fit in LDS
size_t blocked_hamming_workspace(int64_t B, int64_t N, int64_t W, int64_t k, bool masked);
// The 1-bit Hamming top-k of small batches (B >= 1) over 512-bit codes on the fp4 matrix cores,
// one wave per stream of tiles (scan_bits_mfma.hip); k <= kMaxK, an optional mask of
// mask_words words a query.
size_t bits_mfma_workspace(int64_t B, int64_t N, int64_t k);
int bits_mfma(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
              int64_t k, const uint64_t* mask, int64_t mask_words, int64_t* out_ids,
              void* out_scores, int score_kind, void* workspace, size_t workspace_bytes,
              hipStream_t stream);
// The 1-bit full scan for kMaxK < k <= kMaxKHamming (scan_hamming_large.hip).
size_t hamming_large_k_workspace(int64_t B, int64_t N, int64_t W);
int hamming_large_k(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
                    int64_t W, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, int score_kind, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);
int blocked_hamming(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
                    int64_t W, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, int score_kind, void* workspace,
                    size_t workspace_bytes, hipStream_t stream,
                    const ClauseCheck& clause = ClauseCheck{},
                    int64_t mask_t_stride = 0);

// Sizes the passes for B queries over N rows and top-k. A workgroup row (grid.y) covers qpg
// queries and each workgroup keeps lists_per_wg candidate lists (of main_capw entries in the
// main pass); the main pass runs target_wgs workgroups in all; a seed workgroup scores at
// least seed_rows_per_wg sampled rows.
// Rows of the seed sample (at least, and kSeedRowsPerK * k at least): the main pass then keeps
// about k * N / seed rows composites a query (in expectation, for items in random order).
constexpr int64_t kSeedRows = 1 << 18;
ScanPlan plan_scan(int64_t B, int64_t N, int64_t k, int64_t qpg, int64_t lists_per_wg,
                   int64_t target_wgs, int main_capw, int64_t seed_rows_per_wg,
                   int64_t seed_rows_min = kSeedRows);

// Writes the -1 / sentinel pads of an empty result.
int launch_pad(int64_t* out_ids, void* out_scores, int64_t B, int64_t k, int score_kind,
               hipStream_t stream);

// Launches the merge (threshold mode when tau_out != null).
int launch_merge(const MergeArgs& m, hipStream_t stream);

}  // namespace rt
