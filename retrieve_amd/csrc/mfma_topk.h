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
  // the Bloom plan of this lane's query (its clause table, an LDS copy or the tables' global
  // copy), probed per candidate by the whole wave where `probing` (after the clauses: the
  // filter is their AND, and the clause test is one attribute-row load; a passing candidate's
  // row bits are one uniform load); probe_on (wave-uniform) false: no probe
  const uint64_t* doc_bits = nullptr;
  const uint64_t* table = nullptr;  // this lane's query's table (global memory)
  lds_cu64* lds = nullptr;          // the group's tables in LDS, when tables_lds (uniform)
  int lds_at = 0;                   // this lane's query's table there
  bool tables_lds = false;
  bool probe_on = false;
  bool probing = false;

  __device__ void set_tau(uint64_t t) {
    tau = t;
    ts = KeyOps<Score>::score(composite_key(t));
  }

  // Scores acc[r] of rows row0 + r (r < 4) for this lane's query; rows >= r1 are past the
  // pass. item = row * row_stride. Appends composites >= tau that pass the mask, the clauses
  // and the Bloom probe (tested only for such composites); compacts lists that could overflow
  // on the next tile. The filters run once per tile for all four rows: one mask word when the
  // rows are four consecutive items from a multiple of four (they share a word), and the clause
  // and probe tests one candidate per lane per pass (a wave rarely has more than one per lane).
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
    const bool held = clauses && clause.held;
    if (held && cand != 0u) {
      // every candidate's attribute row in one round of loads, then the tests on them
      AttrRow rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if ((cand >> r) & 1u) rows[r] = load_attr_row(clause, (row0 + r) * row_stride);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if ((cand >> r) & 1u && !clause_pass_held(clause, crow, rows[r])) cand &= ~(1u << r);
      }
    }
    uint32_t todo = (clauses && !held) || probing ? cand : 0u;
    while (__any(todo != 0u)) {
      int r = -1;
      bool ok = false;
      if (todo != 0u) {
        r = __builtin_ctz(todo);
        todo &= todo - 1u;
        ok = held || !clauses || clause_pass(clause, crow, (row0 + r) * row_stride);
      }
      if (probe_on) {  // each candidate that passed, one at a time, by the whole wave
        const uint64_t item = static_cast<uint64_t>((row0 + (r < 0 ? 0 : r)) * row_stride);
        uint64_t need = __ballot(ok && probing);
        while (need != 0ull) {
          const int l = static_cast<int>(__builtin_ctzll(need));
          need &= need - 1ull;
          // the candidate's row bits: one uniform (scalar) load, waited for on its own
          const uint64_t f = doc_bits[readlane64(item, l)];
          bool pass;
          if (tables_lds) {
            pass = probe_wave(lds + __builtin_amdgcn_readlane(lds_at, l), f, lane_id());
          } else {
            const uint64_t* t = reinterpret_cast<const uint64_t*>(
                readlane64(reinterpret_cast<uint64_t>(table), l));
            pass = probe_wave(t, f, lane_id());
          }
          if (lane_id() == l) ok = pass;
        }
      }
      if (r >= 0 && !ok) cand &= ~(1u << r);
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
