// Candidate handling for scans whose scores come out of a 16x16 MFMA tile with the items as
// the A operand: lane l holds the scores of query (l % 16) for items 4 * (l / 16) + r, r < 4.
// Shared by the int8 and bf16 scans.
#pragma once

#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

template <class Score>
struct KeyOps;

template <>
struct KeyOps<int32_t> {
  __device__ static uint32_t key(int32_t s) { return key_of_i32(s); }
  __device__ static int32_t score(uint32_t k) { return i32_of_key(k); }
};

template <>
struct KeyOps<float> {
  __device__ static uint32_t key(float s) { return key_of_f32(s); }
  // keys below -inf's (only the no-bound key 0 occurs) test as -inf; keys above +inf's
  // (the padding key ~0) are NaN and never pass
  __device__ static float score(uint32_t k) {
    return k <= key_of_f32(-INFINITY) ? -INFINITY : f32_of_key(k);
  }
};

// One wave's candidate state for its 16 queries.
template <class Score>
struct WaveTopK16 {
  uint64_t* lists;         // [16, capw] in global memory
  int* cnt;                // [16] in LDS
  uint64_t* scratch;       // [capw] in LDS
  int capw;
  int k;
  uint64_t tau;            // this lane's query: lower bound (composite); ~0 = padding column
  Score ts;                // its score part (the fast-path test is score >= ts)
  const uint64_t* qmask;   // this lane's query's item bits (bit 63 - d % 64), or null
  ClauseCheck clause;      // exact clauses tested per candidate, where `clauses`
  ClauseRow crow;          // this lane's query's clause state
  bool clauses;

  __device__ void set_tau(uint64_t t) {
    tau = t;
    ts = KeyOps<Score>::score(composite_key(t));
  }

  // Scores acc[r] of rows row0 + r (r < 4) for this lane's query; rows >= r1 are past the
  // pass. item = row * row_stride. Appends composites >= tau that pass the mask and the
  // clauses (tested only for such composites); compacts lists that could overflow on the next
  // tile. The filters run once per tile for all four rows: one mask word when the rows are
  // four consecutive items from a multiple of four (they share a word), and the clause tests
  // one candidate per lane per pass (a wave rarely has more than one per lane).
  __device__ void push(const Score acc[4], int64_t row0, int64_t r1, int64_t row_stride) {
    const Score m01 = acc[0] > acc[1] ? acc[0] : acc[1];
    const Score m23 = acc[2] > acc[3] ? acc[2] : acc[3];
    const bool hit = (m01 > m23 ? m01 : m23) >= ts;
    if (!__any(hit)) return;
    const int col = lane_id() & 15;
    uint64_t cs[4];
    uint32_t cand = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = row0 + r;
      cs[r] = composite(KeyOps<Score>::key(acc[r]), static_cast<uint32_t>(row * row_stride));
      cand |= row < r1 && acc[r] >= ts && cs[r] >= tau ? 1u << r : 0u;
    }
    if (qmask != nullptr && cand != 0u) {
      const int64_t item0 = row0 * row_stride;
      if (row_stride == 1 && (row0 & 3) == 0) {
        const uint64_t w = qmask[item0 >> 6];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          cand &= (w >> (63 - ((item0 + r) & 63))) & 1ull ? ~0u : ~(1u << r);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t item = (row0 + r) * row_stride;
          if ((cand >> r) & 1u) {
            cand &= (qmask[item >> 6] >> (63 - (item & 63))) & 1ull ? ~0u : ~(1u << r);
          }
        }
      }
    }
    uint32_t todo = clauses ? cand : 0u;
    while (__any(todo != 0u)) {
      if (todo != 0u) {
        const int r = __builtin_ctz(todo);
        todo &= todo - 1u;
        if (!clause_pass(clause, crow, (row0 + r) * row_stride)) cand &= ~(1u << r);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if ((cand >> r) & 1u) {
        const int pos = atomicAdd(&cnt[col], 1);
        lists[col * capw + pos] = cs[r];
      }
    }
    wave_sync_memory();
    const bool full = cnt[col] > capw - kTile;
    uint64_t need = __ballot(full) & 0xffffull;
    while (need != 0ull) {
      const int c = __builtin_ctzll(need);
      need &= need - 1;
      const uint64_t nt = wave_compact(lists + c * capw, &cnt[c], scratch, capw, k);
      if (col == c && nt > tau) set_tau(nt);
    }
  }
};

}  // namespace rt
