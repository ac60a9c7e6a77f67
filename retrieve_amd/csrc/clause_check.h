// The exact clause predicate for one (query row, item) pair, for the scans that test it where a
// candidate beats its query's threshold instead of reading a precomputed mask.
//
// Predicate (functional.py:173-185; fork_filters.cuh:15-41), with value sets: clause c of row b
// is active iff its set is not empty, and matches an item iff one of the item's A values for c
// is in the set, XOR clause_is_reverse[c]; the item passes iff every active clause matches
// (a row with no active clause passes every item). The sets come from the clause filter's prep
// pass (filter_clause.hip): per row the active mask, each clause's values with the -1 pads
// removed, and, for rows whose values all lie in [0, kSetDomain), one bitmap per clause.
#pragma once

#include "rt_common.h"

namespace rt {

constexpr int kMaxClauses = 32;
// Rows whose values all lie in [0, kSetDomain) test membership in a per-clause bitmap.
constexpr int kSetDomain = 1024;
constexpr int kSetWords = kSetDomain / 64;

struct ClauseCheck {
  const void* attrs = nullptr;  // [N, C, A] int16, int32 or int64
  int attr_bytes = 0;
  int C = 0;
  int A = 0;
  int V = 0;
  const uint32_t* active = nullptr;   // [B] bit c: clause c active; null: no clause filter
  const int32_t* nv = nullptr;        // [B, C] values per set
  const int64_t* qc = nullptr;        // [B, C, V] the set's values first
  const uint32_t* small = nullptr;    // [B] non-zero: the row's values lie in [0, kSetDomain)
  const uint64_t* bitmaps = nullptr;  // [B, C, kSetWords] value v at bit v % 64 of word v / 64
  const uint32_t* rev_mask = nullptr;  // [1] bit c: clause c is reversed
  int held = 0;  // rows of 4, 8 or 16 bytes at an address aligned to them: tests on held rows
};

// Whether an attribute table's rows can be held in registers (AttrRow below).
inline int attr_rows_held(const void* attrs, int attr_bytes, int64_t C, int64_t A) {
  const int64_t bytes = C * A * attr_bytes;
  return (bytes == 16 || bytes == 8 || bytes == 4) &&
         reinterpret_cast<uintptr_t>(attrs) % static_cast<uintptr_t>(bytes) == 0;
}

__device__ inline int64_t clause_attr(const ClauseCheck& f, const char* row, int i) {
  if (f.attr_bytes == 2) return reinterpret_cast<const int16_t*>(row)[i];
  if (f.attr_bytes == 4) return reinterpret_cast<const int32_t*>(row)[i];
  return reinterpret_cast<const int64_t*>(row)[i];
}

// One query row's clause state, loaded once per lane: its active and reverse masks, its set
// form, and where its bitmaps are (global memory, or a copy in LDS).
struct ClauseRow {
  uint32_t act = 0u;
  uint32_t rev = 0u;
  bool small = false;
  const uint64_t* bm = nullptr;  // [C, kSetWords]
  const int32_t* nv = nullptr;   // [C]
  const int64_t* qc = nullptr;   // [C, V]
};

// Row b's state; `bm` replaces the bitmaps' global address when not null.
__device__ inline ClauseRow clause_row(const ClauseCheck& f, int64_t b,
                                       const uint64_t* bm = nullptr) {
  ClauseRow r;
  r.act = f.active[b];
  r.rev = f.rev_mask[0];
  r.small = f.small[b] != 0u;
  r.bm = bm != nullptr ? bm : f.bitmaps + b * f.C * kSetWords;
  r.nv = f.nv + b * f.C;
  r.qc = f.qc + b * f.C * f.V;
  return r;
}

// Whether `item` passes the row's clauses (called per lane, lanes free to diverge).
__device__ inline bool clause_pass(const ClauseCheck& f, const ClauseRow& r, int64_t item) {
  if (r.act == 0u) return true;
  const char* row = static_cast<const char*>(f.attrs) +
                    item * static_cast<int64_t>(f.C) * f.A * f.attr_bytes;
  uint32_t match = 0u;
  for (uint32_t m = r.act; m != 0u; m &= m - 1u) {
    const int c = __builtin_ctz(m);
    bool eq = false;
    for (int x = 0; x < f.A; ++x) {
      const int64_t v = clause_attr(f, row, c * f.A + x);
      if (r.small) {
        eq |= v >= 0 && v < kSetDomain && ((r.bm[c * kSetWords + (v >> 6)] >> (v & 63)) & 1ull);
      } else {
        const int64_t* vals = r.qc + c * f.V;
        const int n = r.nv[c];
        for (int i = 0; i < n; ++i) eq |= v == vals[i];
      }
    }
    match |= eq ? 1u << c : 0u;
  }
  return ((match ^ r.rev) & r.act) == r.act;
}

// An item's attribute row held in registers, for tables whose rows are 4, 8 or 16 bytes
// (C * A * attr_bytes): one aligned load, so the clause tests of several candidates wait on
// one round of loads instead of one each.
struct AttrRow {
  uint32_t w[4];
};

__device__ inline AttrRow load_attr_row(const ClauseCheck& f, int64_t item) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int bytes = f.C * f.A * f.attr_bytes;
  const char* row = static_cast<const char*>(f.attrs) + item * bytes;
  AttrRow r{{0u, 0u, 0u, 0u}};
  if (bytes == 16) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(row);
    r.w[0] = v[0];
    r.w[1] = v[1];
    r.w[2] = v[2];
    r.w[3] = v[3];
  } else if (bytes == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(row);
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else {
    r.w[0] = *reinterpret_cast<const uint32_t*>(row);
  }
  return r;
}

// load_attr_row for rows of HB bytes (4, 8 or 16; a compile-time size: no branch).
template <int HB>
__device__ inline AttrRow load_attr_row_n(const ClauseCheck& f, int64_t item) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  static_assert(HB == 4 || HB == 8 || HB == 16, "held rows are 4, 8 or 16 bytes");
  const char* row = static_cast<const char*>(f.attrs) + item * HB;
  AttrRow r{{0u, 0u, 0u, 0u}};
  if constexpr (HB == 16) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(row);
    r.w[0] = v[0];
    r.w[1] = v[1];
    r.w[2] = v[2];
    r.w[3] = v[3];
  } else if constexpr (HB == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(row);
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else {
    r.w[0] = *reinterpret_cast<const uint32_t*>(row);
  }
  return r;
}

// Word i of a held row (a select chain: no indexed private array).
__device__ inline uint32_t row_word(const AttrRow& r, int i) {
  return i == 0 ? r.w[0] : i == 1 ? r.w[1] : i == 2 ? r.w[2] : r.w[3];
}

// Attribute value i of a held row.
__device__ inline int64_t held_attr(const ClauseCheck& f, const AttrRow& r, int i) {
  if (f.attr_bytes == 2) {
    const uint32_t w = row_word(r, i >> 1);
    return static_cast<int16_t>((w >> (16 * (i & 1))) & 0xFFFFu);
  }
  if (f.attr_bytes == 4) return static_cast<int32_t>(row_word(r, i));
  return static_cast<int64_t>((static_cast<uint64_t>(row_word(r, 2 * i + 1)) << 32) |
                              row_word(r, 2 * i));
}

// clause_pass over a held row (tables with f.held set).
__device__ inline bool clause_pass_held(const ClauseCheck& f, const ClauseRow& r,
                                        const AttrRow& row) {
  if (r.act == 0u) return true;
  uint32_t match = 0u;
  for (uint32_t m = r.act; m != 0u; m &= m - 1u) {
    const int c = __builtin_ctz(m);
    bool eq = false;
    for (int x = 0; x < f.A; ++x) {
      const int64_t v = held_attr(f, row, c * f.A + x);
      if (r.small) {
        eq |= v >= 0 && v < kSetDomain && ((r.bm[c * kSetWords + (v >> 6)] >> (v & 63)) & 1ull);
      } else {
        const int64_t* vals = r.qc + c * f.V;
        const int n = r.nv[c];
        for (int i = 0; i < n; ++i) eq |= v == vals[i];
      }
    }
    match |= eq ? 1u << c : 0u;
  }
  return ((match ^ r.rev) & r.act) == r.act;
}

// Whether `item` passes row b's clauses.
__device__ inline bool clause_check(const ClauseCheck& f, int64_t b, int64_t item) {
  return clause_pass(f, clause_row(f, b), item);
}

// Workspace of the prep pass for B rows of C clauses with V values, and the pass itself: it
// fills `out`'s set fields from query_values [B, C, V] (-1 pads) and clause_is_reverse [C] on
// `stream` (filter_clause.hip).
size_t clause_prep_workspace(int64_t B, int64_t C, int64_t V);
int clause_prepare(const int64_t* query_values, int64_t B, int64_t C, int64_t V,
                   const int8_t* clause_is_reverse, void* workspace, size_t workspace_bytes,
                   ClauseCheck* out, hipStream_t stream);

}  // namespace rt
