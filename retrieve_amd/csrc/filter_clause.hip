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
#include "rt_common.h"

namespace rt {

constexpr int kClauseThreads = 256;
constexpr int kRegAttrs = 16;  // C * A up to this is held in registers
constexpr int kMaxClauses = 32;
constexpr int kCompactWords = 128;  // 64-bit mask words per compaction chunk (one wave)

enum ClauseMode : int { kClauseBits = 0, kClauseBool = 1, kClauseScores = 2 };

struct ClauseArgs {
  const int64_t* attrs;  // [N, C, A]
  int64_t N;
  int C;
  int A;
  const int8_t* reverse;  // [C] 0/1
  const int64_t* qvals;   // [B, C, V], -1 pads
  int64_t B;
  int V;
  int64_t rows_per_wg;     // query rows each workgroup loops over
  const uint64_t* and_mask;  // [B, and_words] or null (bits mode)
  int64_t and_words;
  const float* scores;       // [B, N] (scores mode)
  void* out;
  int64_t W;
};

template <bool REG>
__device__ inline int64_t item_attr(const int64_t (&at)[kRegAttrs], const int64_t* row, int i) {
  if constexpr (REG) {
    return at[i];
  } else {
    return row[i];
  }
}

// One query row against this lane's item: 1 iff every active clause matches.
template <bool REG>
__device__ inline bool clause_pass(const ClauseArgs& a, const int64_t (&at)[kRegAttrs],
                                   const int64_t* row, int64_t b, uint32_t rev_mask) {
  const int64_t* q = a.qvals + b * a.C * a.V;
  uint32_t active = 0;
  uint32_t match = 0;
  if constexpr (REG) {
    // attribute slot i belongs to clause i / A: unrolled so the registers are indexed statically
#pragma unroll
    for (int i = 0; i < kRegAttrs; ++i) {
      if (i < a.C * a.A) {
        const int c = i / a.A;
        const int64_t* qc = q + c * a.V;
        bool eq = false;
        for (int v = 0; v < a.V; ++v) {
          const int64_t val = qc[v];
          if (val == -1) continue;
          active |= 1u << c;
          eq |= at[i] == val;
        }
        match |= eq ? 1u << c : 0u;
      }
    }
  } else {
    for (int c = 0; c < a.C; ++c) {
      const int64_t* qc = q + c * a.V;
      bool eq = false;
      for (int v = 0; v < a.V; ++v) {
        const int64_t val = qc[v];
        if (val == -1) continue;
        active |= 1u << c;
        for (int x = 0; x < a.A; ++x) eq |= item_attr<REG>(at, row, c * a.A + x) == val;
      }
      match |= eq ? 1u << c : 0u;
    }
  }
  return ((match ^ rev_mask) & active) == active;
}

template <int MODE, bool REG>
__global__ void __launch_bounds__(kClauseThreads) clause_kernel(ClauseArgs a) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kClauseThreads + threadIdx.x;
  const bool valid = d < a.N;
  const int ca = a.C * a.A;
  const int64_t* row = a.attrs + (valid ? d : 0) * ca;
  int64_t at[kRegAttrs];
  if constexpr (REG) {
#pragma unroll
    for (int i = 0; i < kRegAttrs; ++i) at[i] = (i < ca && valid) ? row[i] : -1;
  }
  uint32_t rev_mask = 0;
  for (int c = 0; c < a.C; ++c) rev_mask |= a.reverse[c] != 0 ? 1u << c : 0u;

  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.rows_per_wg;
  const int64_t b1 = b0 + a.rows_per_wg < a.B ? b0 + a.rows_per_wg : a.B;
  const int lane = lane_id();
  for (int64_t b = b0; b < b1; ++b) {
    const bool pass = valid && clause_pass<REG>(a, at, row, b, rev_mask);
    if constexpr (MODE == kClauseBits) {
      // item (wave base + l) at bit 63 - l of its word
      uint64_t word = __builtin_bitreverse64(__ballot(pass));
      const int64_t w = (d - lane) >> 6;
      if (lane == 0 && w < a.W) {
        if (a.and_mask != nullptr) word &= a.and_mask[b * a.and_words + w];
        static_cast<uint64_t*>(a.out)[b * a.W + w] = word;
      }
    } else if constexpr (MODE == kClauseBool) {
      if (valid) static_cast<uint8_t*>(a.out)[b * a.N + d] = pass ? 1 : 0;
    } else {
      if (valid) {
        static_cast<float*>(a.out)[b * a.N + d] = pass ? a.scores[b * a.N + d] : -INFINITY;
      }
    }
  }
}

template <int MODE>
static void launch_clause(const ClauseArgs& a, dim3 grid, hipStream_t stream) {
  if (a.C * a.A <= kRegAttrs) {
    clause_kernel<MODE, true><<<grid, kClauseThreads, 0, stream>>>(a);
  } else {
    clause_kernel<MODE, false><<<grid, kClauseThreads, 0, stream>>>(a);
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

}  // namespace rt

using namespace rt;

extern "C" int rt_clause_filter(const int64_t* item_attrs, int64_t N, int64_t C, int64_t A,
                                const int8_t* clause_is_reverse, const int64_t* query_values,
                                int64_t B, int64_t V, int mode, const float* scores,
                                const uint64_t* and_mask, int64_t and_mask_words, void* out,
                                hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && B >= 0, "N and B must be >= 0");
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(C));
  RT_CHECK_ARG(A >= 0 && A <= 4096 && V >= 1 && V <= 4096, "A must be >= 0 and V >= 1");
  RT_CHECK_ARG(mode >= kClauseBits && mode <= kClauseScores, "mode must be 0, 1 or 2");
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
  const int64_t gx = cdiv(N, kClauseThreads);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "N too large");
  // enough workgroups to fill the device: split the rows when the items alone are too few
  int64_t gy = cdiv(4096, gx);
  gy = gy < 1 ? 1 : gy;
  gy = gy > B ? B : gy;
  gy = gy > 65535 ? 65535 : gy;
  a.rows_per_wg = cdiv(B, gy);
  gy = cdiv(B, a.rows_per_wg);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (mode == kClauseBits) {
    launch_clause<kClauseBits>(a, grid, stream);
  } else if (mode == kClauseBool) {
    launch_clause<kClauseBool>(a, grid, stream);
  } else {
    launch_clause<kClauseScores>(a, grid, stream);
  }
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
