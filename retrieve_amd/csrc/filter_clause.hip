// Exact clause filter over item attributes, and the packed-mask compaction.
//
// Predicate (functional.py:173-185; fork_filters.cuh:15-41), generalised to value sets: query
// row b holds V values per clause c (-1 pads). Clause c is active for b iff some value is not
// -1; it matches an item iff one of the item's A values for c equals one of the row's values,
// XOR clause_is_reverse[c]. An item passes iff every active clause matches. With V == 1 this is
// the reference's [B, C] query (-1 = inactive clause).
//
// Layout: lane <-> item. A workgroup takes 256 consecutive items, loads each item's C * A
// attributes into registers once, and loops over its query rows; a row's values are
// wave-uniform (scalar loads), so inactive clauses cost a scalar branch. Outputs:
//   packed bits [B, ceil(N/64)] (item d at bit 63 - d % 64, the scans' mask layout): one
//     ballot per wave and query, bit-reversed;
//   bool [B, N], or masked scores [B, N] (scores where the row passes, -inf elsewhere).
// The compaction turns packed bits into ascending item ids per row in three launches: chunk
// popcounts, a per-row exclusive scan, and a scatter where each 64-item word is expanded by one
// wave with coalesced writes.
#include "clause_check.h"
#include "rt_common.h"

namespace rt {

constexpr int kClauseThreads = 256;
constexpr int kRegAttrs = 16;  // one value per clause (A == 1), C up to this: held in registers
constexpr int kCompactWords = 128;  // 64-bit mask words per compaction chunk (one wave)
// (rows whose values all lie in [0, kSetDomain) test membership in a per-clause bitmap staged
// in LDS, instead of walking the value list)
constexpr int kMaxBitmapLds = 64 * 1024;

enum ClauseMode : int { kClauseBits = 0, kClauseBool = 1, kClauseScores = 2 };

struct ClauseArgs {
  const void* attrs;  // [N, C, A] of int16, int32 or int64 (the kernel's T)
  int64_t N;
  int C;
  int A;
  const int8_t* reverse;  // [C] 0/1
  const int64_t* qvals;   // [B, C, V], -1 pads
  int64_t B;
  int V;
  // per row, from the prep pass: the active clauses, and each clause's values without pads
  const uint32_t* active;  // [B]
  const int32_t* nv;       // [B, C]
  const int64_t* qc;       // [B, C, V], clause c's first nv[b, c] entries
  const uint32_t* small;   // [B]: every value of the row in [0, kSetDomain)
  const uint32_t* rev_mask;  // [1]: bit c = clause_is_reverse[c]
  const uint64_t* bitmaps;  // [B, C, kSetWords]: the row's value set of clause c (small rows)
  int64_t rows_per_wg;     // query rows each workgroup loops over
  const uint64_t* and_mask;  // [B, and_words] or null (bits mode)
  int64_t and_words;
  const float* scores;       // [B, N] (scores mode)
  void* out;
  int64_t W;
  int mode;  // ClauseMode (the row kernel branches on it; the others take it as a template)
};

template <bool REG, class T>
__device__ inline int64_t item_attr(const int64_t (&at)[kRegAttrs], const T* row, int i) {
  if constexpr (REG) {
    return at[i];
  } else {
    return static_cast<int64_t>(row[i]);
  }
}

// Per query row (one workgroup each, one wave per clause): each clause's values with the -1
// pads removed (ballot compaction, in order), its 1024-bit set bitmap (LDS atomics), and the
// row's active clause mask and whether every value lies in [0, kSetDomain).
constexpr int kPrepThreads = 256;

__global__ void __launch_bounds__(kPrepThreads) clause_prep_kernel(
    const int64_t* qvals, int64_t B, int C, int V, const int8_t* reverse, uint32_t* active,
    int32_t* nv, int64_t* qc, uint32_t* small, uint64_t* bitmaps, uint32_t* rev_mask) {
  __shared__ uint64_t bm[kPrepThreads / kWave][kSetWords];
  __shared__ uint32_t clause_act[kMaxClauses];
  __shared__ uint32_t clause_fits[kMaxClauses];
  const int64_t b = blockIdx.x;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  if (b == 0 && threadIdx.x == 0) {
    uint32_t r = 0;
    for (int c = 0; c < C; ++c) r |= reverse[c] != 0 ? 1u << c : 0u;
    rev_mask[0] = r;
  }
  for (int c = wave; c < C; c += kPrepThreads / kWave) {
    if (lane < kSetWords) bm[wave][lane] = 0ull;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const int64_t* src = qvals + (b * C + c) * V;
    int64_t* dst = qc + (b * C + c) * V;
    int n = 0;
    bool fits = true;
    for (int v0 = 0; v0 < V; v0 += kWave) {
      const int64_t x = v0 + lane < V ? src[v0 + lane] : -1;
      const bool keep = x != -1;
      const uint64_t mask = __ballot(keep);
      const int pos = n + static_cast<int>(__popcll(mask & ((1ull << lane) - 1ull)));
      if (keep) dst[pos] = x;
      n += static_cast<int>(__popcll(mask));
      const bool in_set = keep && x >= 0 && x < kSetDomain;
      fits &= __ballot(keep && !in_set) == 0ull;
      if (in_set) atomicOr(&bm[wave][x >> 6], 1ull << (x & 63));
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (lane < kSetWords) bitmaps[(b * C + c) * kSetWords + lane] = bm[wave][lane];
    if (lane == 0) {
      nv[b * C + c] = n;
      clause_act[c] = n > 0 ? 1u : 0u;
      clause_fits[c] = fits ? 1u : 0u;
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t act = 0u;
    bool fits = true;
    for (int c = 0; c < C; ++c) {
      act |= clause_act[c] << c;
      fits &= clause_fits[c] != 0u;
    }
    active[b] = act;
    small[b] = fits ? 1u : 0u;
  }
}

// One query row against this lane's item: 1 iff every active clause matches.
template <bool REG, class T>
__device__ inline bool clause_pass(const ClauseArgs& a, const int64_t (&at)[kRegAttrs],
                                   const T* row, int64_t b, uint32_t rev_mask,
                                   const uint64_t* bm, uint32_t active) {
  // (active == 0: no clause, every item passes)
  const int32_t* nvb = a.nv + b * a.C;
  const int64_t* qcb = a.qc + b * a.C * a.V;
  uint32_t match = 0;
  if (bm != nullptr) {
    // the row's sets as bitmaps (LDS): one lookup per attribute value
    if constexpr (REG) {  // A == 1: register i holds clause i's value
#pragma unroll
      for (int i = 0; i < kRegAttrs; ++i) {
        const int64_t x = at[i];
        if (((active >> i) & 1u) && x >= 0 && x < kSetDomain) {
          match |= ((bm[i * kSetWords + (x >> 6)] >> (x & 63)) & 1ull) ? 1u << i : 0u;
        }
      }
    } else {
      for (int c = 0; c < a.C; ++c) {
        if (((active >> c) & 1u) == 0u) continue;
        for (int x = 0; x < a.A; ++x) {
          const int64_t v = item_attr<REG, T>(at, row, c * a.A + x);
          if (v >= 0 && v < kSetDomain && ((bm[c * kSetWords + (v >> 6)] >> (v & 63)) & 1ull)) {
            match |= 1u << c;
          }
        }
      }
    }
    return ((match ^ rev_mask) & active) == active;
  }
  if constexpr (REG) {  // A == 1: unrolled so the registers are indexed statically
#pragma unroll
    for (int i = 0; i < kRegAttrs; ++i) {
      if ((active >> i) & 1u) {
        const int64_t* vals = qcb + i * a.V;
        const int n = nvb[i];
        bool eq = false;
        for (int v = 0; v < n; ++v) eq |= at[i] == vals[v];
        match |= eq ? 1u << i : 0u;
      }
    }
  } else {
    for (int c = 0; c < a.C; ++c) {
      if (((active >> c) & 1u) == 0u) continue;
      const int64_t* vals = qcb + c * a.V;
      const int n = nvb[c];
      bool eq = false;
      for (int v = 0; v < n; ++v) {
        for (int x = 0; x < a.A; ++x) eq |= item_attr<REG, T>(at, row, c * a.A + x) == vals[v];
      }
      match |= eq ? 1u << c : 0u;
    }
  }
  return ((match ^ rev_mask) & active) == active;
}

// Each workgroup stages its query rows' set bitmaps in LDS once, then walks 256-item chunks
// round-robin with the other workgroups of its row range.
template <int MODE, bool REG, class T>
__global__ void __launch_bounds__(kClauseThreads) clause_kernel(ClauseArgs a) {
  const int lane = lane_id();
  const int ca = a.C * a.A;
  const uint32_t rev_mask = a.C > 0 ? a.rev_mask[0] : 0u;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.rows_per_wg;
  const int64_t b1 = b0 + a.rows_per_wg < a.B ? b0 + a.rows_per_wg : a.B;
  extern __shared__ uint64_t bm_lds[];
  __shared__ uint32_t row_active[kWave];
  __shared__ uint32_t row_small[kWave];
  const int64_t row_words = static_cast<int64_t>(a.C) * kSetWords;
  if (a.C > 0) {
    for (int64_t i = threadIdx.x; i < (b1 - b0) * row_words; i += kClauseThreads) {
      bm_lds[i] = a.bitmaps[b0 * row_words + i];
    }
    for (int64_t i = threadIdx.x; i < b1 - b0; i += kClauseThreads) {
      row_active[i] = a.active[b0 + i];
      row_small[i] = a.small[b0 + i];
    }
  }
  __syncthreads();

  const int nrows = static_cast<int>(b1 - b0);  // <= kWave (rows_per_wg is capped)
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kClauseThreads; base < a.N;
       base += static_cast<int64_t>(gridDim.x) * kClauseThreads) {
    const int64_t d = base + threadIdx.x;
    const bool valid = d < a.N;
    // bits mode: lane j handles row b0 + j's word of this wave's 64 items -- its AND-mask word
    // is loaded here for all rows at once, and the row words are stored together after the loop
    const int64_t wword = (d - lane) >> 6;
    uint64_t am = ~0ull;
    uint64_t mine = 0ull;
    if constexpr (MODE == kClauseBits) {
      if (a.and_mask != nullptr && lane < nrows && wword < a.W) {
        am = a.and_mask[(b0 + lane) * a.and_words + wword];
      }
    }
    // lanes past the end read item 0 (no divergent loads) and are masked out
    const T* row = static_cast<const T*>(a.attrs) + (valid ? d : 0) * ca;
    int64_t at[kRegAttrs];
    if constexpr (REG) {
      // unconditional in-row loads (slot min(i, C - 1)) and a branch-free select, so the
      // loads issue back to back
#pragma unroll
      for (int i = 0; i < kRegAttrs; ++i) {
        const int64_t x = static_cast<int64_t>(row[i < ca ? i : ca - 1]);
        const int64_t keep = -static_cast<int64_t>(i < ca);  // all ones or zero
        at[i] = (x & keep) | ~keep;                           // x, or -1 past the row
      }
    }
    for (int64_t b = b0; b < b1; ++b) {
      const bool small = a.C > 0 && row_small[b - b0] != 0u;
      const uint32_t active = a.C > 0 ? row_active[b - b0] : 0u;
      const uint64_t* bm = small ? bm_lds + (b - b0) * row_words : nullptr;
      const bool pass = valid && clause_pass<REG, T>(a, at, row, b, rev_mask, bm, active);
      if constexpr (MODE == kClauseBits) {
        // item (wave base + l) at bit 63 - l of its word, kept by lane b - b0
        const uint64_t word = __builtin_bitreverse64(__ballot(pass));
        mine = lane == static_cast<int>(b - b0) ? word : mine;
      } else if constexpr (MODE == kClauseBool) {
        if (valid) static_cast<uint8_t*>(a.out)[b * a.N + d] = pass ? 1 : 0;
      } else {
        if (valid) {
          static_cast<float*>(a.out)[b * a.N + d] = pass ? a.scores[b * a.N + d] : -INFINITY;
        }
      }
    }
    if constexpr (MODE == kClauseBits) {
      if (lane < nrows && wword < a.W) {
        static_cast<uint64_t*>(a.out)[(b0 + lane) * a.W + wword] = mine & am;
      }
    }
  }
}

// Query-mask form (C <= kQmaskClauses): a workgroup takes up to 32 query rows and builds in LDS
// qm[c][x] = the rows whose clause-c set holds x, for x in [0, kSetDomain). An item then costs
// one LDS lookup per attribute value for all its rows at once:
//   pass_c = (OR over its values x of qm[c][x]) XOR (rev[c] ? ~0 : 0), OR the rows where c is
//   inactive; the item's row mask is the AND over c.
// Rows with a value outside [0, kSetDomain) take the value-list path row by row.
constexpr int kQmaskRows = 32;
constexpr int kQmaskClauses = 16;

template <int MODE, bool REG, class T>
__global__ void __launch_bounds__(kClauseThreads) clause_qmask_kernel(ClauseArgs a) {
  const int lane = lane_id();
  const int ca = a.C * a.A;
  const uint32_t rev_mask = a.C > 0 ? a.rev_mask[0] : 0u;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * kQmaskRows;
  const int nrows = static_cast<int>(b0 + kQmaskRows < a.B ? kQmaskRows : a.B - b0);
  extern __shared__ uint32_t qm[];  // [C][kSetDomain]
  __shared__ uint32_t clause_xor[kQmaskClauses];
  __shared__ uint32_t clause_or[kQmaskClauses];
  __shared__ uint32_t row_active[kQmaskRows];
  __shared__ uint32_t slow_rows;
  for (int i = threadIdx.x; i < a.C * kSetDomain; i += kClauseThreads) qm[i] = 0u;
  if (threadIdx.x < kQmaskRows) {
    const int r = threadIdx.x;
    row_active[r] = r < nrows ? a.active[b0 + r] : 0u;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t slow = 0u;
    for (int r = 0; r < nrows; ++r) slow |= a.small[b0 + r] != 0u ? 0u : 1u << r;
    slow_rows = slow;
    for (int c = 0; c < a.C; ++c) {
      uint32_t inactive = slow;  // slow rows: any value here, replaced below
      for (int r = 0; r < nrows; ++r) inactive |= (row_active[r] >> c) & 1u ? 0u : 1u << r;
      clause_xor[c] = (rev_mask >> c) & 1u ? ~0u : 0u;
      clause_or[c] = inactive;
    }
  }
  // every (row, clause) value of the fast rows sets its row's bit
  for (int rc = threadIdx.x; rc < nrows * a.C; rc += kClauseThreads) {
    const int r = rc / a.C;
    const int c = rc - r * a.C;
    const int64_t b = b0 + r;
    if (a.small[b] == 0u) continue;
    const int64_t* vals = a.qc + (b * a.C + c) * a.V;
    const int n = a.nv[b * a.C + c];
    for (int v = 0; v < n; ++v) atomicOr(&qm[c * kSetDomain + vals[v]], 1u << r);
  }
  __syncthreads();
  const uint32_t slow = slow_rows;
  const uint32_t fast = ~slow;

  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kClauseThreads; base < a.N;
       base += static_cast<int64_t>(gridDim.x) * kClauseThreads) {
    const int64_t d = base + threadIdx.x;
    const bool valid = d < a.N;
    const int64_t wword = (d - lane) >> 6;
    uint64_t am = ~0ull;
    if constexpr (MODE == kClauseBits) {
      if (a.and_mask != nullptr && lane < nrows && wword < a.W) {
        am = a.and_mask[(b0 + lane) * a.and_words + wword];
      }
    }
    const T* row = static_cast<const T*>(a.attrs) + (valid ? d : 0) * ca;
    int64_t at[kRegAttrs];
    uint32_t m = ~0u;
    if constexpr (REG) {
#pragma unroll
      for (int i = 0; i < kRegAttrs; ++i) {
        const int64_t x = static_cast<int64_t>(row[i < ca ? i : ca - 1]);
        const int64_t keep = -static_cast<int64_t>(i < ca);
        at[i] = (x & keep) | ~keep;
      }
#pragma unroll
      for (int c = 0; c < kRegAttrs; ++c) {
        if (c < a.C) {
          const uint64_t x = static_cast<uint64_t>(at[c]);
          const uint32_t h = x < static_cast<uint64_t>(kSetDomain) ? qm[c * kSetDomain + x] : 0u;
          m &= (h ^ clause_xor[c]) | clause_or[c];
        }
      }
    } else {
      for (int c = 0; c < a.C; ++c) {
        uint32_t h = 0u;
        for (int j = 0; j < a.A; ++j) {
          const uint64_t x = static_cast<uint64_t>(static_cast<int64_t>(row[c * a.A + j]));
          h |= x < static_cast<uint64_t>(kSetDomain) ? qm[c * kSetDomain + x] : 0u;
        }
        m &= (h ^ clause_xor[c]) | clause_or[c];
      }
    }
    m &= fast;
    for (uint32_t rest = slow; rest != 0u; rest &= rest - 1u) {
      const int r = __builtin_ctz(rest);
      const bool pass = clause_pass<REG, T>(a, at, row, b0 + r, rev_mask, nullptr, row_active[r]);
      m |= pass ? 1u << r : 0u;
    }
    if (!valid) m = 0u;

    if constexpr (MODE == kClauseBits) {
      // row r's word of this wave's 64 items, kept by lane r and stored by all rows at once
      uint64_t mine = 0ull;
      for (int r = 0; r < nrows; ++r) {
        const uint64_t word = __builtin_bitreverse64(__ballot((m >> r) & 1u));
        mine = lane == r ? word : mine;
      }
      if (lane < nrows && wword < a.W) {
        static_cast<uint64_t*>(a.out)[(b0 + lane) * a.W + wword] = mine & am;
      }
    } else if (valid) {
      for (int r = 0; r < nrows; ++r) {
        const int64_t b = b0 + r;
        const bool pass = (m >> r) & 1u;
        if constexpr (MODE == kClauseBool) {
          static_cast<uint8_t*>(a.out)[b * a.N + d] = pass ? 1 : 0;
        } else {
          static_cast<float*>(a.out)[b * a.N + d] = pass ? a.scores[b * a.N + d] : -INFINITY;
        }
      }
    }
  }
}

// ---- one value per clause (A == 1), C <= 16: the row kernel --------------------------
//
// The query-mask form with C and T known at compile time. An item's C values arrive with the
// widest loads its row size allows; the table holds, per clause, kSetDomain + 1 row masks with
// the clause's reverse flag and its unconstrained rows (inactive clause, list rows) folded in:
//   tab[c][x] = (qm[c][x] XOR rev[c]) OR unconstrained[c],  tab[c][kSetDomain]: values outside
// [0, kSetDomain), which no bitmap row holds. An item's row mask is the AND of C lookups.
// Lane l of a wave takes item (wave base + 63 - l), so a ballot is a mask word as it is stored
// (item d at bit 63 - d % 64); lane r keeps row r's word and the rows store together.
constexpr int kTabStride = kSetDomain + 1;
constexpr int kRowUnroll = 4;  // 64-item words per wave per step of the row kernel

template <class T, int C>
struct RowShape {
  static constexpr int kBytes = C * static_cast<int>(sizeof(T));
  static constexpr int kLoad =
      kBytes % 16 == 0 ? 16 : kBytes % 8 == 0 ? 8 : kBytes % 4 == 0 ? 4 : 2;
  static constexpr int kWords = (kBytes + 3) / 4;
};

typedef uint32_t v4w __attribute__((ext_vector_type(4)));

typedef uint32_t v2w __attribute__((ext_vector_type(2)));

template <class T, int C>
__device__ inline void load_row(const char* p, uint32_t (&w)[RowShape<T, C>::kWords]) {
  using S = RowShape<T, C>;
  if constexpr (S::kLoad == 16) {
#pragma unroll
    for (int j = 0; j < S::kBytes / 16; ++j) {
      const v4w x = *reinterpret_cast<const v4w*>(p + 16 * j);
      w[4 * j] = x[0];
      w[4 * j + 1] = x[1];
      w[4 * j + 2] = x[2];
      w[4 * j + 3] = x[3];
    }
  } else if constexpr (S::kLoad == 8) {
#pragma unroll
    for (int j = 0; j < S::kBytes / 8; ++j) {
      const v2w x = *reinterpret_cast<const v2w*>(p + 8 * j);
      w[2 * j] = x[0];
      w[2 * j + 1] = x[1];
    }
  } else if constexpr (S::kLoad == 4) {
#pragma unroll
    for (int j = 0; j < S::kBytes / 4; ++j) w[j] = reinterpret_cast<const uint32_t*>(p)[j];
  } else {
#pragma unroll
    for (int j = 0; j < S::kWords; ++j) w[j] = 0u;
#pragma unroll
    for (int j = 0; j < S::kBytes / 2; ++j) {
      w[j / 2] |= static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(p)[j]) << (16 * (j % 2));
    }
  }
}

// Clause c's value: its table slot, and the value itself (for the list rows).
template <class T, int C>
__device__ inline uint32_t row_slot(const uint32_t (&w)[RowShape<T, C>::kWords], int c,
                                    int64_t& value) {
  if constexpr (sizeof(T) == 2) {
    const int32_t x = static_cast<int16_t>(w[c / 2] >> (16 * (c % 2)));
    value = x;
    return static_cast<uint32_t>(x) < static_cast<uint32_t>(kSetDomain) ? static_cast<uint32_t>(x)
                                                                          : kSetDomain;
  } else if constexpr (sizeof(T) == 4) {
    const int32_t x = static_cast<int32_t>(w[c]);
    value = x;
    return static_cast<uint32_t>(x) < static_cast<uint32_t>(kSetDomain) ? static_cast<uint32_t>(x)
                                                                          : kSetDomain;
  } else {
    const uint32_t lo = w[2 * c];
    const uint32_t hi = w[2 * c + 1];
    value = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    return hi == 0u && lo < static_cast<uint32_t>(kSetDomain) ? lo : kSetDomain;
  }
}

// In-wave transpose of a 64 x 64 bit matrix: lane i holds row i (bit j = column j); after six
// exchange stages lane j holds column j (bit i = row i's bit j). Stage s swaps the off-diagonal
// s x s blocks between lanes i and i ^ s.
__device__ inline uint64_t wave_transpose64(uint64_t x, int lane) {
  constexpr uint64_t kKeep[6] = {0x5555555555555555ull, 0x3333333333333333ull,
                                 0x0f0f0f0f0f0f0f0full, 0x00ff00ff00ff00ffull,
                                 0x0000ffff0000ffffull, 0x00000000ffffffffull};
#pragma unroll
  for (int t = 5; t >= 0; --t) {
    const int s = 1 << t;
    const uint64_t m = kKeep[t];  // the bits j with (j & s) == 0
    const uint64_t y = __shfl_xor(x, s);
    x = (lane & s) ? (((y >> s) & m) | (x & ~m)) : ((x & m) | ((y & m) << s));
  }
  return x;
}

// The same for 32 rows: lane l holds 32 row bits; lane r < 32 ends with row r's 64-bit word
// (bit l = lane l's bit r). A 32 x 32 transpose within each half-wave (five stages, partners
// reached by ds_swizzle's xor mode, which stays within 32 lanes), then the upper half's word of
// row r moves to lane r as the high dword.
template <int T>
__device__ inline uint32_t transpose32_stage(uint32_t x, int lane) {
  constexpr int s = 1 << T;
  // the bits j with (j & s) == 0
  constexpr uint32_t m = T == 0   ? 0x55555555u
                         : T == 1 ? 0x33333333u
                         : T == 2 ? 0x0f0f0f0fu
                         : T == 3 ? 0x00ff00ffu
                                  : 0x0000ffffu;
  const uint32_t y =
      static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(x), 0x1f | (s << 10)));
  return (lane & s) ? (((y >> s) & m) | (x & ~m)) : ((x & m) | ((y & m) << s));
}

__device__ inline uint64_t wave_transpose32(uint32_t x, int lane) {
  x = transpose32_stage<4>(x, lane);
  x = transpose32_stage<3>(x, lane);
  x = transpose32_stage<2>(x, lane);
  x = transpose32_stage<1>(x, lane);
  x = transpose32_stage<0>(x, lane);
  const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(x), (lane + 32) & 63));
  return (static_cast<uint64_t>(hi) << 32) | x;
}

// ROWS query rows per workgroup (32, or 64 for the bit masks of larger batches), M their mask
// word type.
template <class T, int C, int ROWS>
__global__ void __launch_bounds__((ROWS == 64 ? 2 : 1) * kClauseThreads)
    clause_row_kernel(ClauseArgs a) {
  // eight waves for the 64-row groups (their tables fill LDS to two workgroups per CU)
  constexpr int kThreads = (ROWS == 64 ? 2 : 1) * kClauseThreads;
  using S = RowShape<T, C>;
  using M = typename std::conditional<ROWS == 64, uint64_t, uint32_t>::type;
  extern __shared__ __attribute__((aligned(8))) uint32_t tab_raw[];
  M* tab = reinterpret_cast<M*>(tab_raw);  // [C][kTabStride]
  __shared__ uint32_t row_active[ROWS];
  __shared__ M clause_fold[2][C];  // XOR, then OR, per clause
  __shared__ M slow_rows;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const uint32_t rev_mask = a.rev_mask[0];
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * ROWS;
  const int nrows = static_cast<int>(b0 + ROWS < a.B ? ROWS : a.B - b0);
  constexpr M kOne = 1;

  for (int i = tid; i < C * kTabStride; i += kThreads) tab[i] = 0;
  if (tid == 0) slow_rows = 0;
  if (tid < ROWS) row_active[tid] = tid < nrows ? a.active[b0 + tid] : 0u;
  __syncthreads();
  if (tid < nrows && a.small[b0 + tid] == 0u) atomicOr(&slow_rows, kOne << tid);
  // every (row, clause) value of the bitmap rows sets its row's bit
  for (int rc = tid; rc < nrows * C; rc += kThreads) {
    const int r = rc / C;
    const int c = rc - r * C;
    const int64_t b = b0 + r;
    if (a.small[b] == 0u) continue;
    const int64_t* vals = a.qc + (b * C + c) * a.V;
    const int n = a.nv[b * C + c];
    for (int v = 0; v < n; ++v) atomicOr(&tab[c * kTabStride + vals[v]], kOne << r);
  }
  __syncthreads();
  const M slow = slow_rows;
  if (tid < C) {
    M unconstrained = slow;
    for (int r = 0; r < nrows; ++r) unconstrained |= (row_active[r] >> tid) & 1u ? 0 : kOne << r;
    clause_fold[0][tid] = (rev_mask >> tid) & 1u ? ~M{0} : M{0};
    clause_fold[1][tid] = unconstrained;
  }
  __syncthreads();
  for (int i = tid; i < C * kTabStride; i += kThreads) {
    const int c = i / kTabStride;
    tab[i] = (tab[i] ^ clause_fold[0][c]) | clause_fold[1][c];
  }
  __syncthreads();
  const M fast = ~slow;

  // Each workgroup takes one contiguous run of 64-item words, each wave kRowUnroll consecutive
  // words per step with every load of the step issued first: enough bytes in flight per CU to
  // cover HBM latency, and a workgroup's mask stores fill whole lines of each row.
  const int64_t words = (a.N + kWave - 1) / kWave;
  constexpr int kStepWords = kRowUnroll * (kThreads / kWave);
  const int64_t steps = (words + kStepWords - 1) / kStepWords;
  const int64_t per_wg = (steps + gridDim.x - 1) / gridDim.x * kStepWords;
  const int64_t w_lo = static_cast<int64_t>(blockIdx.x) * per_wg;
  const int64_t w_hi = w_lo + per_wg < words ? w_lo + per_wg : words;
  const bool bits = a.mode == kClauseBits;
  for (int64_t w0 = w_lo + wave * kRowUnroll; w0 < w_hi; w0 += kStepWords) {
    uint32_t w[kRowUnroll][S::kWords];
    uint64_t am[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t d = (w0 + u) * kWave + (kWave - 1 - lane);
      const bool valid = w0 + u < w_hi && d < a.N;
      load_row<T, C>(static_cast<const char*>(a.attrs) + (valid ? d : 0) * S::kBytes, w[u]);
      am[u] = ~0ull;
      if (bits && a.and_mask != nullptr && lane < nrows && w0 + u < w_hi) {
        am[u] = a.and_mask[(b0 + lane) * a.and_words + w0 + u];
      }
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t wword = w0 + u;
      const int64_t d = wword * kWave + (kWave - 1 - lane);
      const bool valid = wword < w_hi && d < a.N;
      uint32_t slot[C];
      int64_t at[kRegAttrs];
#pragma unroll
      for (int c = 0; c < kRegAttrs; ++c) at[c] = -1;
#pragma unroll
      for (int c = 0; c < C; ++c) slot[c] = row_slot<T, C>(w[u], c, at[c]);
      M m = fast;
#pragma unroll
      for (int c = 0; c < C; ++c) m &= tab[c * kTabStride + slot[c]];
      for (M rest = slow; rest != 0; rest &= rest - 1) {
        const int r = ROWS == 64 ? __builtin_ctzll(rest) : __builtin_ctz(rest);
        const bool pass = clause_pass<true, T>(a, at, nullptr, b0 + r, rev_mask, nullptr,
                                               row_active[r]);
        m |= pass ? kOne << r : M{0};
      }
      if (!valid) m = 0;

      if (bits) {
        uint64_t mine = 0ull;
        if (nrows > 6) {
          // lane l holds item (word base + 63 - l)'s row bits: the transpose gives lane r row
          // r's word with item d at bit 63 - d % 64, as stored
          if constexpr (ROWS == 64) {
            mine = wave_transpose64(m, lane);
          } else {
            mine = wave_transpose32(m, lane);
          }
        } else {
          for (int r = 0; r < nrows; ++r) {
            const uint64_t word = __ballot((m >> r) & 1u);
            mine = lane == r ? word : mine;
          }
        }
        if (lane < nrows && wword < w_hi) {
          static_cast<uint64_t*>(a.out)[(b0 + lane) * a.W + wword] = mine & am[u];
        }
      } else if (valid) {
        for (int r = 0; r < nrows; ++r) {
          const int64_t b = b0 + r;
          const bool pass = (m >> r) & 1u;
          if (a.mode == kClauseBool) {
            static_cast<uint8_t*>(a.out)[b * a.N + d] = pass ? 1 : 0;
          } else {
            static_cast<float*>(a.out)[b * a.N + d] = pass ? a.scores[b * a.N + d] : -INFINITY;
          }
        }
      }
    }
  }
}

template <class T, int C>
static bool launch_row_kernel(const ClauseArgs& a, dim3 grid, hipStream_t stream) {
  if (reinterpret_cast<uintptr_t>(a.attrs) % RowShape<T, C>::kLoad != 0) return false;
  if (a.rows_per_wg == 64) {
    const size_t lds = static_cast<size_t>(C) * kTabStride * sizeof(uint64_t);
    if (lds > 65536) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&clause_row_kernel<T, C, 64>),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds));
    }
    clause_row_kernel<T, C, 64><<<grid, 2 * kClauseThreads, lds, stream>>>(a);
  } else {
    const size_t lds = static_cast<size_t>(C) * kTabStride * sizeof(uint32_t);
    clause_row_kernel<T, C, 32><<<grid, kClauseThreads, lds, stream>>>(a);
  }
  return true;
}

// The row kernel for A == 1 and 1 <= C <= 16 (false: the attribute table is not aligned for its
// loads, or the shape is not one it takes).
template <class T>
static bool launch_row_typed(const ClauseArgs& a, dim3 grid, hipStream_t stream) {
  if (a.A != 1) return false;
  switch (a.C) {
    case 1: return launch_row_kernel<T, 1>(a, grid, stream);
    case 2: return launch_row_kernel<T, 2>(a, grid, stream);
    case 3: return launch_row_kernel<T, 3>(a, grid, stream);
    case 4: return launch_row_kernel<T, 4>(a, grid, stream);
    case 5: return launch_row_kernel<T, 5>(a, grid, stream);
    case 6: return launch_row_kernel<T, 6>(a, grid, stream);
    case 7: return launch_row_kernel<T, 7>(a, grid, stream);
    case 8: return launch_row_kernel<T, 8>(a, grid, stream);
    case 9: return launch_row_kernel<T, 9>(a, grid, stream);
    case 10: return launch_row_kernel<T, 10>(a, grid, stream);
    case 11: return launch_row_kernel<T, 11>(a, grid, stream);
    case 12: return launch_row_kernel<T, 12>(a, grid, stream);
    case 13: return launch_row_kernel<T, 13>(a, grid, stream);
    case 14: return launch_row_kernel<T, 14>(a, grid, stream);
    case 15: return launch_row_kernel<T, 15>(a, grid, stream);
    case 16: return launch_row_kernel<T, 16>(a, grid, stream);
    default: return false;
  }
}

// Whether the row kernel's widest loads fit the attribute table's alignment (RowShape's kLoad).
static bool row_loads_aligned(const void* attrs, int attr_bytes, int64_t C) {
  const int64_t bytes = C * attr_bytes;
  const int64_t load = bytes % 16 == 0 ? 16 : bytes % 8 == 0 ? 8 : bytes % 4 == 0 ? 4 : 2;
  return reinterpret_cast<uintptr_t>(attrs) % static_cast<uintptr_t>(load) == 0;
}

template <int MODE, class T>
static void launch_clause(const ClauseArgs& a, dim3 grid, hipStream_t stream) {
  if (a.C >= 1 && a.C <= kQmaskClauses && launch_row_typed<T>(a, grid, stream)) return;
  if (a.C >= 1 && a.C <= kQmaskClauses) {
    const size_t qlds = static_cast<size_t>(a.C) * kSetDomain * sizeof(uint32_t);
    if (a.A == 1) {
      clause_qmask_kernel<MODE, true, T><<<grid, kClauseThreads, qlds, stream>>>(a);
    } else {
      clause_qmask_kernel<MODE, false, T><<<grid, kClauseThreads, qlds, stream>>>(a);
    }
    return;
  }
  const size_t lds = static_cast<size_t>(a.rows_per_wg) * a.C * kSetWords * sizeof(uint64_t);
  if (a.A == 1 && a.C <= kRegAttrs) {
    clause_kernel<MODE, true, T><<<grid, kClauseThreads, lds, stream>>>(a);
  } else {
    clause_kernel<MODE, false, T><<<grid, kClauseThreads, lds, stream>>>(a);
  }
}

template <int MODE>
static void launch_clause_typed(const ClauseArgs& a, int attr_bytes, dim3 grid,
                                hipStream_t stream) {
  if (attr_bytes == 2) {
    launch_clause<MODE, int16_t>(a, grid, stream);
  } else if (attr_bytes == 4) {
    launch_clause<MODE, int32_t>(a, grid, stream);
  } else {
    launch_clause<MODE, int64_t>(a, grid, stream);
  }
}

// ---- the clause-major int32 slot layout of st::search -------------------------------------
//
// fork_clause_attrs (retrieve/src/retrieve/ops/official/adapter.py:68-89): slots [R, N] int32,
// clause c in rows clause_slots[c] .. clause_slots[c+1], each doc's values sorted descending
// with -1 pads last; queries [B, C] int32, -1 = inactive clause (INT32_MIN, for values no doc can
// hold, matches nothing). The exact_pass of fork_filters.cuh:15-41. Lane <-> doc: the doc's R
// values are read coalesced (row r of the table) into registers once.
constexpr int kRegSlots = 16;

struct SlotClauseArgs {
  const int32_t* slots;  // [R, N]
  int64_t N;
  int R;
  const int64_t* clause_slots;  // [C + 1]
  int C;
  const int8_t* reverse;  // [C]
  const int32_t* q;       // [B, C]
  int64_t B;
  int64_t rows_per_wg;
  const uint64_t* and_mask;
  int64_t and_words;
  uint64_t* out;  // [B, W]
  int64_t W;
};

template <bool REG>
__global__ void __launch_bounds__(kClauseThreads) slot_clause_kernel(SlotClauseArgs a) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kClauseThreads + threadIdx.x;
  const bool valid = d < a.N;
  const int lane = lane_id();
  int32_t v[kRegSlots];
  if constexpr (REG) {
#pragma unroll
    for (int r = 0; r < kRegSlots; ++r) v[r] = (r < a.R && valid) ? a.slots[r * a.N + d] : -1;
  }
  uint32_t rev_mask = 0;
  for (int c = 0; c < a.C; ++c) rev_mask |= a.reverse[c] != 0 ? 1u << c : 0u;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.rows_per_wg;
  const int64_t b1 = b0 + a.rows_per_wg < a.B ? b0 + a.rows_per_wg : a.B;
  for (int64_t b = b0; b < b1; ++b) {
    const int32_t* qb = a.q + b * a.C;
    uint32_t active = 0;
    uint32_t match = 0;
    for (int c = 0; c < a.C; ++c) {
      const int32_t val = qb[c];
      if (val == -1) continue;
      active |= 1u << c;
      const int r0 = static_cast<int>(a.clause_slots[c]);
      const int r1 = static_cast<int>(a.clause_slots[c + 1]);
      bool eq = false;
      if constexpr (REG) {
#pragma unroll
        for (int r = 0; r < kRegSlots; ++r) eq |= r >= r0 && r < r1 && v[r] == val;
      } else {
        for (int r = r0; r < r1 && valid; ++r) eq |= a.slots[r * a.N + d] == val;
      }
      match |= eq ? 1u << c : 0u;
    }
    const bool pass = valid && ((match ^ rev_mask) & active) == active;
    uint64_t word = __builtin_bitreverse64(__ballot(pass));
    const int64_t w = (d - lane) >> 6;
    if (lane == 0 && w < a.W) {
      if (a.and_mask != nullptr) word &= a.and_mask[b * a.and_words + w];
      a.out[b * a.W + w] = word;
    }
  }
}

// ---- packed mask -> ascending ids ------------------------------------------------------

// Word w of a row with the bits of items >= N cleared (a caller's mask may set them).
__device__ inline uint64_t row_word(const uint64_t* m, int64_t w, int64_t W, int64_t N) {
  const uint64_t x = m[w];
  const int tail = static_cast<int>(N - (W - 1) * 64);  // items in the last word, 1..64
  return (w == W - 1 && tail < 64) ? x & (~0ull << (64 - tail)) : x;
}

// chunk_counts[b, t] = set bits in words [t * 128, +128) of row b. One wave per chunk.
__global__ void __launch_bounds__(256) mask_count_kernel(const uint64_t* mask, int64_t W,
                                                         int64_t N, int64_t T,
                                                         int32_t* chunk_counts) {
  const int lane = lane_id();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (t >= T) return;
  const uint64_t* m = mask + b * W;
  int c = 0;
  for (int i = lane; i < kCompactWords; i += kWave) {
    const int64_t w = t * kCompactWords + i;
    if (w < W) c += __popcll(row_word(m, w, W, N));
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) c += __shfl_xor(c, off);
  if (lane == 0) chunk_counts[b * T + t] = c;
}

// Per row: exclusive scan of the chunk counts (int64 offsets) and the row total.
__global__ void __launch_bounds__(1024) mask_scan_kernel(const int32_t* chunk_counts, int64_t T,
                                                         int64_t* chunk_offsets, int64_t* counts) {
  __shared__ int64_t wave_sums[1024 / kWave];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  int64_t carry = 0;
  for (int64_t base = 0; base < T; base += 1024) {
    const int64_t t = base + tid;
    const int64_t v = t < T ? chunk_counts[b * T + t] : 0;
    // inclusive scan within the wave
    int64_t x = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int64_t y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == kWave - 1) wave_sums[wave] = x;
    __syncthreads();
    int64_t before = carry;
    int64_t total = carry;
    for (int w = 0; w < 1024 / kWave; ++w) {
      if (w < wave) before += wave_sums[w];
      total += wave_sums[w];
    }
    if (t < T) chunk_offsets[b * T + t] = before + x - v;
    carry = total;
    __syncthreads();
  }
  if (tid == 0) counts[b] = carry;
}

// Writes row b's set items in ascending order at out[b, chunk_offsets[b, t] + ...]. One wave per
// chunk walks its words in order (each word is wave-uniform); lane l owns item 64 w + l.
__global__ void __launch_bounds__(256) mask_scatter_kernel(const uint64_t* mask, int64_t W,
                                                           int64_t T, int64_t N,
                                                           const int64_t* chunk_offsets,
                                                           int64_t* out) {
  const int lane = lane_id();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (t >= T) return;
  const uint64_t* m = mask + b * W;
  int64_t* o = out + b * N + chunk_offsets[b * T + t];
  const int64_t w_end = (t + 1) * kCompactWords < W ? (t + 1) * kCompactWords : W;
  for (int64_t w = t * kCompactWords; w < w_end; ++w) {
    const uint64_t word = row_word(m, w, W, N);
    if (word == 0ull) continue;
    // set bits above this lane's bit = items of the word before this lane's item
    const int before = lane == 0 ? 0 : __popcll(word >> (64 - lane));
    if ((word >> (63 - lane)) & 1ull) o[before] = w * 64 + lane;
    o += __popcll(word);
  }
}

static int64_t compact_chunks(int64_t N) { return cdiv(cdiv(N, 64), kCompactWords); }

// (a kernel, not hipMemsetAsync: the calls stay safe to capture in a HIP graph)
__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

struct ClauseWs {
  size_t nv, qc, small, bitmaps, rev, total;
};

static ClauseWs clause_ws_parts(int64_t B, int64_t C, int64_t V) {
  ClauseWs w;
  w.nv = align_up(static_cast<size_t>(B) * sizeof(uint32_t), 256);
  w.qc = w.nv + align_up(static_cast<size_t>(B * C) * sizeof(int32_t), 256);
  w.small = w.qc + align_up(static_cast<size_t>(B * C * V) * sizeof(int64_t), 256);
  w.bitmaps = w.small + align_up(static_cast<size_t>(B) * sizeof(uint32_t), 256);
  w.rev = w.bitmaps + align_up(static_cast<size_t>(B * C) * kSetWords * sizeof(uint64_t), 256);
  w.total = w.rev + 256;
  return w;
}

size_t clause_prep_workspace(int64_t B, int64_t C, int64_t V) {
  if (B <= 0 || C <= 0 || V <= 0) return 256;
  return clause_ws_parts(B, C, V).total;
}

int clause_prepare(const int64_t* query_values, int64_t B, int64_t C, int64_t V,
                   const int8_t* clause_is_reverse, void* workspace, size_t workspace_bytes,
                   ClauseCheck* out, hipStream_t stream) {
  if (B <= 0 || C <= 0) return kOk;
  const ClauseWs p = clause_ws_parts(B, C, V);
  if (workspace_bytes < p.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, p.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint32_t* active = reinterpret_cast<uint32_t*>(ws);
  int32_t* nv = reinterpret_cast<int32_t*>(ws + p.nv);
  int64_t* qc = reinterpret_cast<int64_t*>(ws + p.qc);
  uint32_t* small = reinterpret_cast<uint32_t*>(ws + p.small);
  uint64_t* bitmaps = reinterpret_cast<uint64_t*>(ws + p.bitmaps);
  uint32_t* rev = reinterpret_cast<uint32_t*>(ws + p.rev);
  clause_prep_kernel<<<static_cast<unsigned>(B), kPrepThreads, 0, stream>>>(
      query_values, B, static_cast<int>(C), static_cast<int>(V), clause_is_reverse, active, nv,
      qc, small, bitmaps, rev);
  RT_CHECK_HIP(hipGetLastError());
  out->C = static_cast<int>(C);
  out->V = static_cast<int>(V);
  out->active = active;
  out->nv = nv;
  out->qc = qc;
  out->small = small;
  out->bitmaps = bitmaps;
  out->rev_mask = rev;
  return kOk;
}

}  // namespace rt

using namespace rt;

extern "C" size_t rt_clause_filter_workspace(int64_t B, int64_t C, int64_t V) {
  return clause_prep_workspace(B, C, V);
}

extern "C" int rt_clause_filter(const void* item_attrs, int attr_bytes, int64_t N, int64_t C,
                                int64_t A,
                                const int8_t* clause_is_reverse, const int64_t* query_values,
                                int64_t B, int64_t V, int mode, const float* scores,
                                const uint64_t* and_mask, int64_t and_mask_words, void* out,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && B >= 0, "N and B must be >= 0");
  RT_CHECK_ARG(B <= (int64_t{1} << 21), "B must be <= 2^21 query rows");
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(C));
  RT_CHECK_ARG(A >= 0 && A <= 4096 && V >= 1 && V <= 4096, "A must be >= 0 and V >= 1");
  RT_CHECK_ARG(mode >= kClauseBits && mode <= kClauseScores, "mode must be 0, 1 or 2");
  RT_CHECK_ARG(attr_bytes == 2 || attr_bytes == 4 || attr_bytes == 8,
               "attr_bytes must be 2, 4 or 8 (int16, int32, int64 attributes)");
  RT_CHECK_ARG(mode != kClauseScores || scores != nullptr, "scores mode needs scores");
  RT_CHECK_ARG(and_mask == nullptr || and_mask_words >= cdiv(N, 64),
               "and_mask rows must have >= ceil(N/64) words");
  RT_CHECK_ARG(N < (int64_t{1} << 40), "N too large");
  if (B == 0 || N == 0) return kOk;
  RT_CHECK_ARG(C == 0 || clause_is_reverse != nullptr, "clause_is_reverse is null");
  RT_CHECK_ARG(C == 0 || query_values != nullptr, "query values are null");
  RT_CHECK_ARG(C * A == 0 || item_attrs != nullptr, "item attrs are null");
  ClauseArgs a{};
  a.attrs = item_attrs;
  a.N = N;
  a.C = static_cast<int>(C);
  a.A = static_cast<int>(A);
  a.reverse = clause_is_reverse;
  a.qvals = query_values;
  a.B = B;
  a.V = static_cast<int>(V);
  a.and_mask = and_mask;
  a.and_words = and_mask_words;
  a.scores = scores;
  a.out = out;
  a.W = cdiv(N, 64);
  a.mode = mode;
  if (C > 0) {
    ClauseCheck f;
    const int st = clause_prepare(query_values, B, C, V, clause_is_reverse, workspace,
                                  workspace_bytes, &f, stream);
    if (st != kOk) return st;
    a.active = f.active;
    a.nv = f.nv;
    a.qc = f.qc;
    a.small = f.small;
    a.bitmaps = f.bitmaps;
    a.rev_mask = f.rev_mask;
  }
  // about 4096 workgroups in all, each looping over item chunks (the staging is amortized)
  int64_t gx = cdiv(N, kClauseThreads);
  gx = gx < 4096 ? gx : 4096;
  // split the rows when the items alone give too few workgroups
  int64_t gy = cdiv(4096, gx);
  gy = gy < 1 ? 1 : gy;
  gy = gy > B ? B : gy;
  gy = gy > 65535 ? 65535 : gy;
  a.rows_per_wg = cdiv(B, gy);
  // the rows' bitmaps staged per workgroup stay within kMaxBitmapLds
  if (C > 0) {
    const int64_t max_rows =
        kMaxBitmapLds / (C * kSetWords * static_cast<int64_t>(sizeof(uint64_t)));
    a.rows_per_wg = a.rows_per_wg < max_rows ? a.rows_per_wg : max_rows;
  }
  // a wave's lanes carry the rows' words (bits mode) and the staged row flags
  a.rows_per_wg = a.rows_per_wg < kWave ? a.rows_per_wg : kWave;
  if (C >= 1 && C <= kQmaskClauses) {
    // the query-mask form: 32 rows per workgroup, the table built once per workgroup; 64 rows
    // (the row kernel's 64-bit tables, masks written through an in-wave transpose) for the bit
    // masks of larger batches when its loads are aligned
    a.rows_per_wg = kQmaskRows;
    if (mode == kClauseBits && B > kQmaskRows && A == 1 &&
        row_loads_aligned(item_attrs, attr_bytes, C)) {
      a.rows_per_wg = 64;
    }
    gx = cdiv(N, kClauseThreads);
    gx = gx < 2048 ? gx : 2048;
  }
  gy = cdiv(B, a.rows_per_wg);
  RT_CHECK_ARG(gy <= 65535, "too many query rows");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (mode == kClauseBits) {
    launch_clause_typed<kClauseBits>(a, attr_bytes, grid, stream);
  } else if (mode == kClauseBool) {
    launch_clause_typed<kClauseBool>(a, attr_bytes, grid, stream);
  } else {
    launch_clause_typed<kClauseScores>(a, attr_bytes, grid, stream);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// [B, N] 0/1 bytes -> [B, ceil(N/64)] mask words, item d at bit 63 - d % 64: lane l of a wave
// takes item (wave base + 63 - l), so its ballot is the word as stored.
__global__ void __launch_bounds__(kClauseThreads) pack_mask_kernel(const uint8_t* valid,
                                                                   int64_t N, int64_t W,
                                                                   uint64_t* words) {
  const int lane = lane_id();
  const int64_t b = blockIdx.y;
  const int64_t w = (static_cast<int64_t>(blockIdx.x) * kClauseThreads + threadIdx.x) / kWave;
  if (w >= W) return;  // whole waves
  const int64_t d = w * kWave + (kWave - 1 - lane);
  const bool v = d < N && valid[b * N + d] != 0;
  const uint64_t word = __ballot(v);
  if (lane == 0) words[b * W + w] = word;
}

extern "C" int rt_pack_mask(const uint8_t* valid, int64_t B, int64_t N, uint64_t* words,
                            hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(B <= 65535, "B must be <= 65535");
  const int64_t W = cdiv(N, 64);
  if (B == 0 || W == 0) return kOk;
  const int64_t gx = cdiv(W * kWave, kClauseThreads);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "N too large");
  pack_mask_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(B)), kClauseThreads, 0,
                     stream>>>(valid, N, W, words);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" size_t rt_mask_compact_workspace(int64_t B, int64_t N) {
  if (B <= 0 || N <= 0) return 256;
  const int64_t T = compact_chunks(N);
  return align_up(static_cast<size_t>(B * T) * sizeof(int32_t), 256) +
         align_up(static_cast<size_t>(B * T) * sizeof(int64_t), 256);
}

extern "C" int rt_mask_compact(const uint64_t* mask, int64_t B, int64_t N, int64_t* out_indices,
                               int64_t* counts, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && B >= 0, "N and B must be >= 0");
  RT_CHECK_ARG(B <= 65535, "B must be <= 65535");
  if (B == 0) return kOk;
  if (N == 0) {
    fill_i64_kernel<<<static_cast<unsigned>(cdiv(B, 256)), 256, 0, stream>>>(counts, B, 0);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  const size_t need = rt_mask_compact_workspace(B, N);
  if (workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  const int64_t W = cdiv(N, 64);
  const int64_t T = compact_chunks(N);
  int32_t* chunk_counts = static_cast<int32_t*>(workspace);
  int64_t* chunk_offsets = reinterpret_cast<int64_t*>(
      static_cast<char*>(workspace) + align_up(static_cast<size_t>(B * T) * sizeof(int32_t), 256));
  const dim3 grid(static_cast<unsigned>(cdiv(T, 4)), static_cast<unsigned>(B));
  mask_count_kernel<<<grid, 256, 0, stream>>>(mask, W, N, T, chunk_counts);
  RT_CHECK_HIP(hipGetLastError());
  mask_scan_kernel<<<static_cast<unsigned>(B), 1024, 0, stream>>>(chunk_counts, T, chunk_offsets,
                                                                  counts);
  RT_CHECK_HIP(hipGetLastError());
  mask_scatter_kernel<<<grid, 256, 0, stream>>>(mask, W, T, N, chunk_offsets, out_indices);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_clause_slots_filter(const int32_t* slots, int64_t R, int64_t N,
                                      const int64_t* clause_slots, int64_t C,
                                      const int8_t* clause_is_reverse, const int32_t* query_values,
                                      int64_t B, const uint64_t* and_mask, int64_t and_mask_words,
                                      uint64_t* out, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && B >= 0 && R >= 0, "N, B and R must be >= 0");
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d]", kMaxClauses);
  RT_CHECK_ARG(R <= (int64_t{1} << 20), "too many slot rows");
  RT_CHECK_ARG(and_mask == nullptr || and_mask_words >= cdiv(N, 64),
               "and_mask rows must have >= ceil(N/64) words");
  if (B == 0 || N == 0) return kOk;
  SlotClauseArgs a{};
  a.slots = slots;
  a.N = N;
  a.R = static_cast<int>(R);
  a.clause_slots = clause_slots;
  a.C = static_cast<int>(C);
  a.reverse = clause_is_reverse;
  a.q = query_values;
  a.B = B;
  a.and_mask = and_mask;
  a.and_words = and_mask_words;
  a.out = out;
  a.W = cdiv(N, 64);
  const int64_t gx = cdiv(N, kClauseThreads);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "N too large");
  int64_t gy = cdiv(4096, gx);
  gy = gy < 1 ? 1 : (gy > B ? B : gy);
  gy = gy > 65535 ? 65535 : gy;
  a.rows_per_wg = cdiv(B, gy);
  gy = cdiv(B, a.rows_per_wg);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (R <= kRegSlots) {
    slot_clause_kernel<true><<<grid, kClauseThreads, 0, stream>>>(a);
  } else {
    slot_clause_kernel<false><<<grid, kClauseThreads, 0, stream>>>(a);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
