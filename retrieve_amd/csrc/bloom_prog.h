// Compiled Bloom plans: the program words bloom.hip's prep pass writes for each plan, read by
// the column search (bloom.hip) and by the host pass that derives the clause tables of the fused
// scans' per-candidate probe (retrieve_amd/st.py, probe_tables); the probe itself (scan_mfma.hip,
// bloom.hip's probe search).
//
// Post-order evaluation pushes every child of an n-ary AND / OR before the operator pops them,
// so an OR of 30 terms needs 30 stack slots. Folding a node's value into its previous sibling
// as soon as it is complete (AND / OR are associative and commutative) gives the same result
// with at most one slot per tree level. The prep pass checks each plan exactly as the stack
// evaluation does (a malformed plan matches nothing), marks every node "push" (a first child,
// or the root) or "fold into the top with the parent's operator", and writes two program words
// per op, leaving out the AND / OR nodes flattened into a parent of the same operator (so the
// fan-out-limited chains of a long value set are one run of folding TERMs). A TERM's positions
// p (for the width of bundle 0) are stored as the byte offsets p * 256 of their words in a
// staged bundle column, 14 bits each, the first repeated past the term's distinct positions
// (AND is idempotent):
//   word 0: bits 0-1 kind: TERM, EMPTY, PASS (an AND / OR whose children are folded into the
//           top: pop it), NOT (pop, invert); bits 2-3 place: push, AND into the top, OR into
//           the top; bits 4-17 offset 0; bits 18-31 offset 1
//   word 1: bits 0-13 offset 2; bits 16-29 offset 3
// Plans the program cannot hold (more than kFoldDepth levels, more than 4 positions a term,
// bundle 0 wider than 64 bits, more than kProgMaxOps ops) are left to the stack evaluation.
//
// A compiled buffer holds the headers ([plan_count, 4] int32: status, op count, first hash
// word lo / hi) and, from the next multiple of 256 bytes, each plan's program slot of
// kProgMaxOps word pairs.
#pragma once

#include "rt_common.h"

namespace rt {

constexpr int kFoldDepth = 4;
constexpr int kProgMaxPos = 4;
constexpr int kColMaxWidth = 64;
constexpr int kProgMaxOps = 2048;
constexpr uint32_t kColPosBytes = 32 * sizeof(uint64_t);  // a position's words in a column: 256

enum PlanStatus : int32_t { kPlanProgram = 0, kPlanNone = 1, kPlanStack = 2 };
enum ProgKind : uint32_t { kKindTerm = 0, kKindEmpty = 1, kKindPass = 2, kKindNot = 3 };
enum ProgPlace : uint32_t { kPlacePush = 0, kPlaceAnd = 1, kPlaceOr = 2 };

// Byte offset of the program slots in a compiled buffer of plan_count plans.
__host__ __device__ inline size_t compiled_prog_offset(int64_t plan_count) {
  return (static_cast<size_t>(plan_count) * 16 + 255) / 256 * 256;
}

// The per-document Bloom probe of a fused scan, over clause tables: a plan that is an AND of
// at most 64 clauses (an OR of terms, a term, or the NOT of either; none: EMPTY). The tables of
// a batch are one uint64 array: words 0 .. plan_count hold each plan's table offset (in words,
// from the array's start; plan b's ends where plan b + 1's begins), then the tables. A table is
// a 4-word header -- word 0: bit 0 the plan matches nothing (a malformed plan), bits 1-31 its
// chunk count; word 1: the clauses in use (bit j: clause j); word 2: the negated clauses;
// word 3: 0 -- and per chunk of 64 terms (the plan's terms in clause order) 128 words:
//   [0, 64)   term l's position bits (all ones past the last term),
//   [64, 128) the chunk's lanes holding clause j's terms (indexed by clause j).
// A document with bits f passes when every clause holds a term whose bits f all has, XOR the
// clause's NOT: the column search's verdict for that document (bloom.hip), one document at a
// time, evaluated by the whole wave (lane l tests term l of each chunk, lane j gathers clause
// j's hits, and a ballot decides).
constexpr int kProbeHeaderWords = 4;
constexpr int kProbeChunkWords = 128;

struct BloomProbe {
  const uint64_t* doc_bits = nullptr;  // [N]: bit p = the document's position p; null: no probe
  const uint64_t* tables = nullptr;    // the batch's tables (offsets first)
};

// Lane l's value of v in every lane (l wave-uniform).
__device__ inline uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), l));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// An LDS copy of probe tables (address space 3: its reads wait on LDS only, not behind the
// scan's outstanding global loads as flat reads would).
typedef __attribute__((address_space(3))) const uint64_t lds_cu64;

// The plan of table t (global memory, or an LDS copy) for a document with bits f (the same t and
// f in every lane; every lane of the wave calls it).
template <class Ptr>
__device__ inline bool probe_wave(Ptr t, uint64_t f, int lane) {
  const uint64_t head = t[0];
  const uint64_t used = t[1];
  const uint64_t neg = t[2];
  const int chunks = static_cast<int>(head >> 1);
  Ptr c = t + kProbeHeaderWords;
  bool any = false;  // lane j: clause j holds a hit
  for (int i = 0; i < chunks; ++i, c += kProbeChunkWords) {
    const uint64_t tm = c[lane];
    const uint64_t hits = __ballot((f & tm) == tm);
    any = any || (hits & c[64 + lane]) != 0ull;
  }
  // a clause fails when whether it holds a hit equals its NOT
  const bool bad = ((used >> lane) & 1ull) != 0ull && any == (((neg >> lane) & 1ull) != 0ull);
  return __ballot(bad) == 0ull && (head & 1ull) == 0ull;
}

}  // namespace rt
