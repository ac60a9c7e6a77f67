// Large-batch dense scans with the exact fused top-k: register-blocked 32x32 MFMA tiles.
//
// A workgroup owns 256 queries, eight 32-query column tiles. Item tiles of 64 rows are dealt
// round-robin to the workgroups of a query group; a tile is read once from HBM with coalesced
// loads straight into LDS (3-8 stages in flight). Each wave holds the B-operand fragments of two
// column tiles in registers for the whole kernel and multiplies staged rows against them in
// 32x32 output tiles (v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_{bf16,f16}: each instruction
// consumes 32 bytes of K per row). Two layouts, both with two waves per SIMD:
// - wide (up to 128 queries): eight waves, one workgroup per CU; wave w takes row half w & 1 of
//   every 64-row tile against column tiles w / 2 and w / 2 + 4. With fewer than 256 queries the
//   live column tiles are the low ones, so 64 queries keep one wave per SIMD busy and 128 all
//   eight.
// - narrow (larger batches): four waves, two workgroups per CU, each on its own tiles, so one
//   workgroup's score tests overlap the other's MFMAs (a workgroup's waves move in step through
//   its per-tile barrier). Wave w takes every row of a tile against column tiles w and w + 4:
//   64-row tiles (two row tiles per wave) below 512-byte rows, 32-row tiles at 512 bytes, where
//   the fragments of two column tiles leave registers for one row tile and four stages fit in
//   half the LDS.
// Lane l of an output tile holds query (col tile * 32 + l % 32) and, in register i, item
// (row tile * 32 + (i/4)*8 + (l/32)*4 + i%4). Per MFMA, lane l feeds bytes
// [32 s + 16 (l / 32), +16) of its row on both sides.
//
// Operand reuse: each staged item byte feeds 64 queries per wave and each register-held query
// byte feeds every item of the grid row, so the matrix cores, not LDS or HBM, bound the
// kernel at large batches.
#pragma once

#include <cmath>
#include <type_traits>

#include "bits_fp4.h"
#include "profile.h"
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {
// Each translation unit that includes this file instantiates the kernel for its own operand
// types (scan_blocked_*.hip); the definitions are internal to it.
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kBlkRows = 64;      // items per staged tile (at most)
constexpr int kBlkQpw = 64;       // queries per wave (two 32-query column tiles)
constexpr int kBlkCols = 8;       // 32-query column tiles per workgroup
constexpr int kBlkQpg = kBlkCols * 32;  // queries per workgroup (query group)
// Up to this many queries, rows narrower than 512 bytes take the wide layout; bit codes up to
// kBlkWideMaxBatchBits (their wide layout covers two column tiles).
constexpr int64_t kBlkWideMaxBatch = 128;
constexpr int64_t kBlkWideMaxBatchBits = 64;

// Rows per staged tile: 32 for narrow 512-byte rows, so four stages fit in half the LDS; 128
// for the wide layout below 512-byte rows (its row quarters are 32 rows); 64 otherwise; for
// 64-byte bit-code rows 256 wide (eight 32-row parts) and 64 narrow (two row tiles per wave: half
// the tile barriers and waits of 32-row tiles per MFMA, and whole 64-bit mask words per query).
constexpr int blk_rows(int64_t row_bytes, bool wide, bool bits) {
  return bits ? (wide ? 256 : 64)
              : (wide ? (row_bytes < 512 ? 128 : 64) : (row_bytes >= 512 ? 32 : 64));
}

// Row parts a tile is split into over the waves (a query's lists per workgroup): the wide
// layout's eight waves take 2 row halves x 4 column-tile pairs at 512-byte rows, and 4 row
// quarters x 2 column-tile pairs below, so from 33 queries on every wave holds a real column
// tile; for bit codes 8 row parts x column tiles 0 and 1 (up to 64 queries: every wave busy from
// one query on, and two column tiles share each expansion from 33); the narrow layout's four
// waves take whole tiles.
constexpr int blk_halves(int64_t row_bytes, bool wide, bool bits = false) {
  return wide ? (bits ? 8 : (row_bytes < 512 ? 4 : 2)) : 1;
}

template <bool WIDE, int RB, bool BITS>
struct BlkLayout {
  static constexpr int waves = WIDE ? 8 : 4;
  static constexpr int threads = waves * kWave;
  static constexpr int halves = blk_halves(RB, WIDE, BITS);
  // a wave's two column tiles: jt and jt + cstride (jt < 8 / cstride)
  static constexpr int cstride = halves == 8 ? 1 : (halves == 4 ? 2 : 4);
  static constexpr int rows = blk_rows(RB, WIDE, BITS);
  static constexpr int rtw = rows / 32 / halves;  // 32-row tiles per wave
  static constexpr int per_cu = WIDE ? 1 : 2;     // resident workgroups per CU
};

static_assert(kBlkWideMaxBatch <= kBlkQpg / 2, "the row-quarter layout covers 4 column tiles");
static_assert(kBlkWideMaxBatchBits <= 64, "the bit codes' wide layout covers 2 column tiles");

static bool blk_wide(int64_t row_bytes, int64_t B) {
  (void)row_bytes;
  return B <= kBlkWideMaxBatch;
}
// Cache-policy bits of the main pass's direct-to-LDS loads (streamed once: nontemporal).
constexpr int kNontemporal = 2;
// Word 3 of a raw buffer descriptor (stride 0, byte offsets; out-of-range loads return zeros).
constexpr int kBufferWord3 = 0x00020000;

// BYTES per lane from base + voffset (out-of-range past base + range: zeros) straight into LDS at
// lds + lane * BYTES (lds wave-uniform); NT: nontemporal. (The builtin's size and cache-policy
// operands must be literals, not template parameters.)
template <int BYTES, bool NT>
__device__ inline void buffer_load_lds(const void* base, int range, int voffset, void* lds) {
  static_assert(BYTES == 4 || BYTES == 16, "load size");
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, range, kBufferWord3);
  auto* l = (__attribute__((address_space(3))) void*)(lds);
  if constexpr (BYTES == 4) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, l, 4, voffset, 0, 0, 0);
  } else if constexpr (NT) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, l, 16, voffset, 0, 0, kNontemporal);
  } else {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, l, 16, voffset, 0, 0, 0);
  }
}

struct I8x32 {
  using Score = int32_t;
  using Acc = v16i;
  static constexpr int kind = kScoreI32;
  __device__ static Acc zero() { return Acc{}; }
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t key(Score s) { return key_of_i32(s); }
  __device__ static Score thresh(uint64_t tau) { return i32_of_key(composite_key(tau)); }
  // scores are already ordered ints: the hit test takes maxima of the raw values
  static constexpr bool kIntScores = true;
  __device__ static int32_t skey(Score s) { return s; }
  static constexpr bool kBits = false;
};

// 1-bit codes of 64 W bits (rows of 8 W bytes) on the fp4 matrix cores
// (v_mfma_scale_f32_32x32x64_f8f6f4 with e2m1 operands and unit scales): an item's bits expand
// to {0, 1.0} nibbles, a query's to {-2.0, +2.0}, and the fp32 accumulator starts at
// 64 W - 2 popcount(q), so it ends at the Hamming score 64 W - 2 popcount(q ^ x) exactly (the sum
// over bits of x (4 q - 2) is 4 popcount(x & q) - 2 popcount(x), and every partial sum is an
// integer of magnitude below 2^24). A lane's half of a row is bytes [4 W half, +4 W); K step s
// takes its 32 bits, dword s of that half (64 K elements a step over the two lane halves; the K
// order inside an operand is free, the same on both sides). The scores leave the accumulator as
// int32, so the rest of the scan is the int8 scan's.
struct BitsF4 : I8x32 {
  static constexpr bool kBits = true;
  static constexpr int kStepBits = 32;  // bits per lane per K step
  using MAcc = v16f;
  __device__ static MAcc mstart(int32_t start) { return mstart_f(static_cast<float>(start)); }
  __device__ static MAcc mstart_f(float start) {
    MAcc c;
#pragma unroll
    for (int e = 0; e < 16; ++e) c[e] = start;
    return c;
  }
  __device__ static MAcc mma(v4i a, v4i b, MAcc c) {
    // (the fp4 form reads the low four registers of each operand)
    const v8i a8 = __builtin_shufflevector(a, a, 0, 1, 2, 3, 0, 1, 2, 3);
    const v8i b8 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 0, 1, 2, 3);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, 0, 0x7f7f7f7f, 0,
                                                          0x7f7f7f7f);
  }
  // The main pass's MFMAs for output tile p = 2 i + j (row tile i, column tile j), the query
  // operand scaled and the accumulators started from an inline constant (fp4::hit_bias).
  __device__ static float hit_bias(int p) { return fp4::hit_bias(p); }
  __device__ static MAcc mma_hit(v4i a, v4i b, MAcc c, int p) {
    const v8i a8 = __builtin_shufflevector(a, a, 0, 1, 2, 3, 0, 1, 2, 3);
    const v8i b8 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 0, 1, 2, 3);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, fp4::kFmt, fp4::kFmt, 0,
                                                          fp4::kUnitScale, 0, fp4::hit_scale(p));
  }
  __device__ static int32_t hit_score(float v, int32_t acc0, int p) {
    return fp4::hit_score(v, acc0, p);
  }
  __device__ static int32_t hit_thresh(int32_t th, int32_t acc0, int p) {
    return fp4::hit_thresh(th, acc0, p);
  }
  // The main pass's mask as one more MFMA per 32 x 32 tile: the item operand is a one-hot -1.0
  // at row m's slot (lane m of the lower half), the query operand the mask word's failing rows
  // in the same in-place layout (item_frag of the inverted word: 0.5, 1.0, 2.0, 2.0 per set
  // bit), scaled by 2^14, so a row that fails its query's mask gains at most -8192.
  __device__ static MAcc mask_mma(v4i onehot, uint32_t mask_word, MAcc c) {
    const v4i b = item_frag(~mask_word);
    const v8i a8 = __builtin_shufflevector(onehot, onehot, 0, 1, 2, 3, 0, 1, 2, 3);
    const v8i b8 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 0, 1, 2, 3);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, 0, 0x7f7f7f7f, 0,
                                                          0x8d8d8d8d);
  }
  // the one-hot operand of this lane: row c32's bit 31 - c32 of a mask word sits in nibble
  // (31 - c32) / 4 of dword (31 - c32) % 4; -1.0 is e2m1 0b1010; the upper half is zero
  __device__ static v4i mask_onehot(int c32, int half) {
    const int b = 31 - c32;
    const uint32_t v = half == 0 ? 0xau << (4 * (b >> 2)) : 0u;
    v4i r;
#pragma unroll
    for (int n = 0; n < 4; ++n) r[n] = static_cast<int>((b & 3) == n ? v : 0u);
    return r;
  }
  __device__ static Acc finish(MAcc c) {
    Acc r;
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = static_cast<int32_t>(c[e]);
    return r;
  }
  // A step's 32 bits per lane fill the 32 nibbles of the fp4 operand (fp4::item_frag and
  // fp4::query_frag: an item 1 adds +-2 with the query bit, an item 0 adds 0).
  __device__ static v4i item_frag(uint32_t b) { return fp4::item_frag(b); }
  __device__ static v4i query_frag(uint32_t b) { return fp4::query_frag(b); }
};

// The accumulator of an op's MFMAs: MAcc where the op has one (bit codes), else Acc.
template <class Op, class = void>
struct MAccOf {
  using type = typename Op::Acc;
};
template <class Op>
struct MAccOf<Op, std::void_t<typename Op::MAcc>> {
  using type = typename Op::MAcc;
};

struct BF16x32 {
  using Score = float;
  using Acc = v16f;
  static constexpr int kind = kScoreF32;
  __device__ static Acc zero() { return Acc{}; }
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                   __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  }
  __device__ static uint32_t key(Score s) { return key_of_f32(s); }
  __device__ static Score thresh(uint64_t tau) {
    const uint32_t k = composite_key(tau);
    return k <= key_of_f32(-INFINITY) ? -INFINITY : f32_of_key(k);
  }
  static constexpr bool kIntScores = false;
  static constexpr bool kBits = false;
  // Order-preserving map of a float to int32 (signed compare): the bits of a non-negative
  // float, the magnitude bits flipped for a negative one (-0.0 maps below +0.0, as in key order).
  __device__ static int32_t skey(Score s) {
    const int32_t b = __builtin_bit_cast(int32_t, s);
    return b >= 0 ? b : b ^ 0x7fffffff;
  }
};

struct F16x32 : BF16x32 {
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a),
                                                  __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
};

// fp32 rows on the fp32 matrix cores (v_mfma_f32_32x32x2_f32): a K step's 16 bytes per lane are
// four floats, lane half h holding elements 4 h + i of the step's eight; product i pairs element
// i of both halves, on both operands alike, so the four products sum the step's dot product (in
// another order than a sequential sum).
struct F32x32 : BF16x32 {
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    const v4f fa = __builtin_bit_cast(v4f, a);
    const v4f fb = __builtin_bit_cast(v4f, b);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.x, fb.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.y, fb.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.z, fb.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(fa.w, fb.w, c, 0, 0, 0);
  }
};

// Staged tiles: as many of 8, 4, 3 as fit in LDS beside the lists (more bytes in flight per CU);
// 2 for the small bit-code tiles when the lists of a large k leave no more.
constexpr int kBlkMinStages = 3;

// Mask words staged beside each tile of a masked main pass: a 32-bit word per query and 32
// rows.
constexpr int blk_mask_bytes(int rows) { return kBlkQpg * (rows / 32) * 4; }

// Waves per SIMD: two (one 8-wave or two 4-wave workgroups per CU).
constexpr int kBlkWavesPerSimd = 2;

__device__ inline int32_t imax(int32_t a, int32_t b) { return a > b ? a : b; }

// Max of 4 accumulator values in the signed-int key domain of Op::skey. RAW: take maxima of the
// raw bits as ints (v_max3_i32, no NaN canonicalisation) -- exact for every value with the sign
// bit clear and below every such value otherwise, so it decides "max >= threshold" whenever the
// threshold's key is >= 0. Else the float max (NaN drops out) mapped through skey.
// (by value: __builtin_bit_cast applied directly to a vector element v[i] reads element 0)
template <class S>
__device__ inline int32_t raw_bits(S s) {
  return __builtin_bit_cast(int32_t, s);
}

template <class Op, bool RAW, class Acc>
__device__ inline int32_t group_max(const Acc& v, int g) {
  if constexpr (RAW) {
    return imax(imax(imax(raw_bits(v[4 * g]), raw_bits(v[4 * g + 1])), raw_bits(v[4 * g + 2])),
                raw_bits(v[4 * g + 3]));
  } else {
    const float m = __builtin_fmaxf(__builtin_fmaxf(static_cast<float>(v[4 * g]),
                                                    static_cast<float>(v[4 * g + 1])),
                                    __builtin_fmaxf(static_cast<float>(v[4 * g + 2]),
                                                    static_cast<float>(v[4 * g + 3])));
    return Op::skey(static_cast<typename Op::Score>(m));
  }
}

// group_max over the rows of the group that pass the mask: bit 31 - 8 g - u of w is row u's
// mask bit; rows that fail count as INT32_MIN (below every threshold). Per row one signed
// bit-field extract (0 or -1) and one bit-field insert, then two 3-way maxima.
template <class Op, bool RAW, class Acc>
__device__ inline int32_t group_max_masked(const Acc& v, int g, uint32_t w) {
  int32_t kv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if constexpr (RAW) {
      kv[u] = raw_bits(v[4 * g + u]);
    } else {
      kv[u] = Op::skey(static_cast<typename Op::Score>(v[4 * g + u]));
    }
    const int32_t m = __builtin_amdgcn_sbfe(static_cast<int32_t>(w), 31 - 8 * g - u, 1);
    kv[u] = (kv[u] & m) | (INT32_MIN & ~m);
  }
  return imax(imax(imax(kv[0], kv[1]), kv[2]), kv[3]);
}

// s_waitcnt immediate: vmcnt <= N (N < 64), expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// vmcnt <= later * LOADS for a wave-uniform later in [0, MAXL] (the immediate must be constant).
template <int LOADS, int MAXL>
__device__ inline void wait_later(int later) {
  if constexpr (MAXL > 0) {
    if (later >= MAXL) {
      wait_vmcnt<MAXL * LOADS>();
      return;
    }
    wait_later<LOADS, MAXL - 1>(later);
  } else {
    wait_vmcnt<0>();
  }
}

// Workgroup barrier over the staged tiles: waits for this wave's LDS accesses (lgkmcnt(0)),
// then s_barrier. __syncthreads() would also wait for every outstanding global load (its
// workgroup release fence), draining the tiles still in flight; the direct-to-LDS loads of the
// tile about to be read are covered by the wait_vmcnt before this. The empty asm statements
// keep the compiler from moving memory accesses across the barrier.
__device__ inline void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// SEED: per query, each workgroup's best composite over the strided sample, written to
// lists[q * gridDim.x + workgroup] (one-entry lists); else candidate lists per (wave, query).
// MASKED: the tiles' mask words are staged and tested (seed and main pass); a separate
// instantiation keeps the unmasked kernel's registers free of it. CLAUSES (with a mask): the
// exact clauses of a.clause are tested on each seed lane's best, and the main pass's lists
// (candidates that pass the mask) drop the entries that fail them when compacted (and in the
// final merge); also a separate instantiation, for the registers of the kernels without.
template <class Op, int RB, bool SEED, int STAGES, bool WIDE, bool MASKED, bool CLAUSES>
__global__ void __launch_bounds__((BlkLayout<WIDE, RB, Op::kBits>::threads))
    __attribute__((amdgpu_waves_per_eu(kBlkWavesPerSimd, kBlkWavesPerSimd)))
    scan_blocked_kernel(ScanArgs a) {
  if (a.run_if != nullptr && *a.run_if == 0u) return;  // (uniform: the fallback is not needed)
  using Score = typename Op::Score;
  using L = BlkLayout<WIDE, RB, Op::kBits>;
  constexpr int ROWS = L::rows;
  // MFMA steps per row: 32 bytes of K each, or 64 bits of a bit-code row (32 a lane half)
  constexpr int KS = Op::kBits ? RB / 8 : RB / 32;
  constexpr int RTW = L::rtw;  // 32-row tiles per wave
  constexpr int kBlkWaves = L::waves;
  constexpr int kBlkThreads = L::threads;
  constexpr int kBlkRowHalves = L::halves;
  constexpr int TILE_BYTES = ROWS * RB;
  // waves that load tile data (a tile smaller than one 16-byte load per thread: the first ones)
  // and their 16-byte loads per thread per tile
  constexpr int TWAVES = TILE_BYTES >= kBlkThreads * 16 ? kBlkWaves : TILE_BYTES / (kWave * 16);
  constexpr int TLOADS = TILE_BYTES / (TWAVES * kWave * 16);
  // The main pass stages the tile's mask words too (always issued, from a dummy address when
  // there is no mask, so every tile is the same number of loads): MASK_DW 32-bit words per
  // query, one per 32 rows, MLOADS 4-byte loads per thread.
  constexpr int MASK_DW = ROWS / 32;
  constexpr int MASK_BYTES = blk_mask_bytes(ROWS);
  constexpr int MLOADS = MASKED ? kBlkQpg * MASK_DW / kBlkThreads : 0;
  constexpr int LOADS = TLOADS + MLOADS;  // loads per thread per tile, with a mask
  constexpr int CH = RB / 16;             // 16-byte chunks per row
  static_assert(TWAVES >= 1 && TILE_BYTES % (TWAVES * kWave * 16) == 0,
                "tile must split into 16-byte loads");
  static_assert(!MASKED || (kBlkQpg * MASK_DW) % kBlkThreads == 0, "mask words per thread");
  static_assert((STAGES - 1) * LOADS < 64, "vmcnt range");
  static_assert(!Op::kBits || 2 * 8 * RB < 4 * 512, "scaled bit-code sums stay below the bias");
  extern __shared__ __attribute__((aligned(16))) uint64_t smem[];
  int8_t* stage = reinterpret_cast<int8_t*>(smem);
  // with a mask: [STAGES][kBlkQpg][MASK_DW] mask words after the tiles (none otherwise)
  constexpr bool masked = MASKED;
  int8_t* mstage = stage + STAGES * TILE_BYTES;
  uint64_t* scratch =
      reinterpret_cast<uint64_t*>(mstage + (masked ? STAGES * MASK_BYTES : 0));
  const int tid = threadIdx.x;
  const int lane = lane_id();
  // wave-uniform, so what derives from it (row half, column tiles, list slots) lives in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int half = lane >> 5;
  int* cnt = reinterpret_cast<int*>(scratch + kBlkWaves * a.capw) + wave * kBlkQpw;
  // bit codes, masked main pass: the mask MFMA's item operand
  v4i onehot = v4i{0, 0, 0, 0};
  if constexpr (Op::kBits && !SEED && masked) onehot = Op::mask_onehot(c32, half);
  const int wr = WIDE ? wave % kBlkRowHalves : 0;  // this wave's row part of each tile
  const int jt = WIDE ? wave / kBlkRowHalves : wave;  // and its column tiles jt, jt + CST
  constexpr int CST = L::cstride;

  const int64_t wg = blockIdx.x;
  const int64_t nwg = gridDim.x;
  const int64_t qg0 = static_cast<int64_t>(blockIdx.y) * kBlkQpg;
  // query of this lane in column tile j (0, 1) of the wave: qg0 + 32 (jt + CST j) + c32
  const int64_t q0[2] = {qg0 + 32 * jt, qg0 + 32 * (jt + CST)};
  // this wave's column tiles that hold real queries (wave-uniform; tile 1 only with tile 0)
  const int cols = (q0[0] < a.B ? 1 : 0) + (q0[1] < a.B ? 1 : 0);
  const int8_t* Q = static_cast<const int8_t*>(a.queries);
  const int8_t* I = static_cast<const int8_t*>(a.items);

  v4i qf[2][KS];
  uint64_t tau[2];
  Score ts[2];
  int32_t acc0[2] = {0, 0};  // accumulator start per column tile (bit codes: 64 W - 2 |q|)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t q = q0[j] + c32;
    if (q < a.B) {
      if constexpr (Op::kBits) {
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(Q + q * RB + (RB / 2) * half);
#pragma unroll
        for (int s = 0; s < KS; ++s) qf[j][s] = Op::query_frag(qb[s]);
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(Q + q * RB);
        int pc = 0;
#pragma unroll
        for (int w = 0; w < RB / 4; ++w) pc += __builtin_popcount(qw[w]);
        acc0[j] = 8 * RB - 2 * pc;
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          qf[j][s] = *reinterpret_cast<const v4i*>(Q + q * RB + 32 * s + 16 * half);
        }
      }
      tau[j] = a.tau_in != nullptr ? a.tau_in[q] : 0ull;
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[j][s] = v4i{0, 0, 0, 0};
      tau[j] = ~0ull;
    }
    ts[j] = Op::thresh(tau[j]);
  }
  // thresholds in the skey domain, and whether the raw-bits group maxima decide the hit test
  int32_t th[2] = {Op::skey(ts[0]), Op::skey(ts[1])};
  bool raw = Op::kIntScores || __all(th[0] >= 0 && th[1] >= 0);
  // bit codes, main pass: the fp32 accumulators start at BitsF4::hit_bias instead of the
  // column's 64 W - 2 popcount(q), with the sums scaled down (BitsF4::mma_hit), so a row that passes
  // the mask ends positive and one that fails it negative (the mask MFMA's -8192 or less); the
  // hit test takes signed int maxima of the raw bits, exact among positive floats and below them
  // for negative ones, against the threshold moved into the same domain (INT32_MIN: every row
  // hits, when the threshold is not positive there)
  int32_t thr[2][2] = {{INT32_MIN, INT32_MIN}, {INT32_MIN, INT32_MIN}};  // [row tile][column]
  if constexpr (Op::kBits) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) thr[i][j] = Op::hit_thresh(th[j], acc0[j], 2 * i + j);
  }
  uint64_t best[2] = {0ull, 0ull};  // SEED
  // list slots of this wave, one per column tile: a 32-query column tile g = q / 32 has slots
  // g * S + s, s = wg * 2 + wr (S = 2 nwg), each holding 32 lists of capw entries
  int64_t slot[2];
  uint64_t* lists[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t g = static_cast<int64_t>(blockIdx.y) * kBlkCols + jt + CST * j;
    slot[j] = (g * nwg + wg) * kBlkRowHalves + wr;
    lists[j] = a.lists + slot[j] * 32 * static_cast<int64_t>(a.capw);
  }
  // list lengths of this lane's two queries (the same in both halves of the wave): each list
  // belongs to this wave alone, so appends take positions from ballots, not atomics
  int nq[2] = {0, 0};

  const int64_t n = a.n_rows;
  const int64_t ntiles = cdiv(n, ROWS);
  // Staged tile layout (no padding): row r's 16-byte chunk c sits at r * RB + (c ^ (r % CH)) * 16,
  // so the 32 rows of an MFMA read start on different banks. A wave's direct-to-LDS load writes
  // 1 KiB contiguously in lane order, so the swizzle goes into the global address each lane
  // fetches (a permutation within the row: still one contiguous 1 KiB span per instruction).
  int toff[TLOADS];  // this lane's byte offset in a full tile (row r, swizzled chunk c)
#pragma unroll
  for (int l = 0; l < TLOADS; ++l) {
    const int sidx = (l * TWAVES + wave) * kWave + lane;  // 16-byte slot (loading waves)
    const int r = sidx / CH;
    toff[l] = r * RB + ((sidx % CH) ^ (r % CH)) * 16;
  }
  // Several query groups (gridDim.y > 1) read the same tiles from this XCD's L2: keep the lines
  // (temporal loads); with one group each tile is read once and streams past (nontemporal).
  const bool shared_tiles = gridDim.y > 1;
  auto issue_mask = [&](int64_t tt, int st) {
    // word e of the stage: query qg0 + e / MASK_DW, the tile's items i0 + 32 (e % MASK_DW) +
    // 0..31 at bits 31..0 (the high half of a 64-bit mask word holds its first 32 items); the
    // seed's tiles lie whole in its sample blocks, so their items are consecutive too
    const int64_t i0 = SEED ? sample_item(tt * ROWS, a.row_stride) : tt * ROWS;
    const int64_t last = a.mask_t_rows - 1;  // the transposed mask's last word row
    const int64_t w0 = i0 >> 6;              // the tile's first word row (<= last)
    const int64_t avail = (last - w0 + 1) * a.mask_t_stride * 8;
    const uint64_t* mbase = a.mask_t + w0 * a.mask_t_stride;
    const int mrange = static_cast<int>(avail < INT32_MAX ? avail : INT32_MAX);
#pragma unroll
    for (int l = 0; l < MLOADS; ++l) {
      const int e = (l * kBlkWaves + wave) * kWave + lane;
      // from the transposed mask: a tile's words for the group's queries are contiguous
      const int64_t r0 = i0 + 32 * (e % MASK_DW);
      int64_t w = r0 >> 6;
      w = w < last ? w : last;  // rows past the end: never scored
      const int off = static_cast<int>(((w - w0) * a.mask_t_stride + qg0 + e / MASK_DW) * 8) +
                      ((r0 & 63) ? 0 : 4);
      int8_t* dst = mstage + st * MASK_BYTES + (l * kBlkWaves + wave) * kWave * 4;
      buffer_load_lds<4, false>(mbase, mrange, off, dst);
    }
  };
  auto issue = [&](int64_t lt, int st) {
    const int64_t tt = lt;  // the tile in the item table
    int8_t* base = stage + st * TILE_BYTES;
    if constexpr (masked) issue_mask(tt, st);
    // One buffer descriptor per tile: base = its first row, range = its rows present. A tile's
    // rows are consecutive (the seed's sample blocks hold whole tiles, and only the last tile
    // is partial); rows past the end read as zeros and are never scored. Buffer loads rather
    // than global ones: the compiler counts a pending global load to LDS as an access to both
    // memories and then waits for every LDS read at once (lgkmcnt(0)), which would serialize
    // the fragment reads of the MFMA loop.
    static_assert(kSeedBlock % ROWS == 0, "seed sample blocks hold whole tiles");
    const int64_t rows_here = n - tt * ROWS < ROWS ? n - tt * ROWS : ROWS;
    const int8_t* tile = I + sample_item(tt * ROWS, a.row_stride) * static_cast<int64_t>(RB);
    const int range = static_cast<int>(rows_here * RB);
    if (wave >= TWAVES) return;  // (wave-uniform)
#pragma unroll
    for (int l = 0; l < TLOADS; ++l) {
      int8_t* dst = base + (l * TWAVES + wave) * kWave * 16;
      if (shared_tiles) {
        buffer_load_lds<16, false>(tile, range, toff[l], dst);
      } else {
        buffer_load_lds<16, true>(tile, range, toff[l], dst);
      }
    }
  };

  int64_t t = wg;
  // this workgroup's tiles: wg, wg + nwg, ...
  const int64_t my_tiles = wg < ntiles ? cdiv(ntiles - wg, nwg) : 0;
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st) {
    if (t + st * nwg < ntiles) issue(t + st * nwg, st);
  }
  static_assert(STAGES >= 2 && STAGES <= 8, "stage count");
  for (int it = 0; t < ntiles; ++it, t += nwg) {
    // Tile t has landed once at most the loads of this workgroup's later tiles issued so far
    // (up to STAGES - 2 of them) are outstanding: vmcnt retires in issue order on this
    // architecture, one counter for loads and stores, so list stores issued in between only
    // make the wait stricter.
    const int64_t after = my_tiles - 1 - it;  // this workgroup's tiles after t
    const int later = static_cast<int>(after < STAGES - 2 ? after : STAGES - 2);
    // (a wave that loads no tile data waits for its mask words only)
    if constexpr (masked) {
      if (wave < TWAVES) {
        wait_later<LOADS, STAGES - 2>(later);
      } else {
        wait_later<MLOADS, STAGES - 2>(later);
      }
    } else {
      if (wave < TWAVES) wait_later<TLOADS, STAGES - 2>(later);
    }
    // every wave's share of tile t is in LDS, and every wave is done reading tile t - nwg, whose
    // stage the next load goes into
    tile_barrier();
    const int64_t tn = t + (STAGES - 1) * nwg;
    if (tn < ntiles) issue(tn, (it + STAGES - 1) % STAGES);

    // only the 32-query column tiles that hold real queries are multiplied (NC of them; a
    // wave of padding only helps with the loads)
    auto tile_body = [&](auto nc) {
      constexpr int NC = decltype(nc)::value;
      const int8_t* src = stage + (it % STAGES) * TILE_BYTES;
      // 2 x 2 output tiles (rows 32 i + ..., this wave's query columns 32 j + ...): four
      // independent accumulator chains keep the matrix pipeline full
      typename Op::Acc acc[RTW][NC];
      // the main pass's scores in fp32 from zero (bit codes): the hit test reads them as they are
      constexpr bool FHIT = Op::kBits && !SEED;
      typename MAccOf<Op>::type macc[RTW][NC];
      // the staged mask bits of this lane's query over each 32-row tile (bit 31 - x: row x)
      uint32_t mw[RTW][NC];
      if constexpr (masked) {
        const uint32_t* ms =
            reinterpret_cast<const uint32_t*>(mstage + (it % STAGES) * MASK_BYTES);
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            mw[i][j] = ms[(32 * (jt + CST * j) + c32) * MASK_DW + wr * RTW + i];
          }
      }
      if constexpr (Op::kBits) {
        // fp32 accumulators: the seed pass's from 64 W - 2 popcount(q), the scores taken out as
        // int32 after; the main pass's from hit_bias(2 i + j), which its first MFMA reads as an
        // inline constant
        if constexpr (!FHIT) {
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) macc[i][j] = Op::mstart(acc0[j]);
        }
        // this lane's half of each of its rows (RB / 2 bytes), read once into registers; step s
        // masks its dword s into the four operand dwords (five VALU, no table)
        constexpr int HC = CH / 2;  // 16-byte chunks per half row
        v4i hb[RTW][HC];
#pragma unroll
        for (int i = 0; i < RTW; ++i) {
          const int r = 32 * (wr * RTW + i) + c32;
#pragma unroll
          for (int m = 0; m < HC; ++m) {
            hb[i][m] = *reinterpret_cast<const v4i*>(src + r * RB +
                                                     (((HC * half + m) ^ (r % CH)) * 16));
          }
        }
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          v4i cur[RTW];
#pragma unroll
          for (int i = 0; i < RTW; ++i) {
            cur[i] = Op::item_frag(static_cast<uint32_t>(hb[i][s / 4][s % 4]));
          }
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) {
              if constexpr (FHIT) {
                macc[i][j] = Op::mma_hit(
                    cur[i], qf[j][s], s == 0 ? Op::mstart_f(Op::hit_bias(2 * i + j)) : macc[i][j],
                    2 * i + j);
              } else {
                macc[i][j] = Op::mma(cur[i], qf[j][s], macc[i][j]);
              }
            }
        }
        if constexpr (FHIT && masked) {
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) macc[i][j] = Op::mask_mma(onehot, mw[i][j], macc[i][j]);
        }
        if constexpr (!FHIT) {
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) acc[i][j] = Op::finish(macc[i][j]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int j = 0; j < NC; ++j) acc[i][j] = Op::zero();
        // row fragments of step s: lane l reads bytes [32 s + 16 (l / 32), +16) of its row;
        // PF steps are read ahead so the LDS latency hides behind the MFMAs
        auto frag = [&](int s, int i) {
          const int r = 32 * (wr * RTW + i) + c32;
          return *reinterpret_cast<const v4i*>(src + r * RB +
                                               (((2 * s + half) ^ (r % CH)) * 16));
        };
        constexpr int PF = KS < 4 ? KS : 4;
        v4i af[PF][RTW];
#pragma unroll
        for (int s = 0; s < PF; ++s)
#pragma unroll
          for (int i = 0; i < RTW; ++i) af[s][i] = frag(s, i);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          v4i cur[RTW];
#pragma unroll
          for (int i = 0; i < RTW; ++i) {
            cur[i] = af[s % PF][i];
            if (s + PF < KS) af[s % PF][i] = frag(s + PF, i);
          }
          // keep the read of step s + PF ahead of step s's MFMAs (the scheduler would otherwise
          // sink it next to its use to save registers)
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) acc[i][j] = Op::mma(cur[i], qf[j][s], acc[i][j]);
        }
      }
      // register r of tile (i, j) holds row t * 64 + 32 i + (r / 4) * 8 + 4 half + r % 4
      const int64_t rt = t * ROWS + 4 * half;
      if constexpr (SEED) {
        // the mask words with this lane's half shifted out of the way (bit 31 - 8 g - u: row
        // 8 g + 4 half + u)
        uint32_t mwh[RTW][NC];
        if constexpr (masked) {
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j) mwh[i][j] = mw[i][j] << (4 * half);
        }
        // A lane's best over the tile is its largest key at the lowest of its rows holding it
        // (rows rise with the register index, and later tiles hold later items, which lose
        // ties), so the keys' maximum decides whether the tile can raise the lane's best and
        // the composite is built only where it does.
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            uint32_t keys[16];
            uint32_t mx = 0u;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              keys[r] = Op::key(acc[i][j][r]);
              if constexpr (masked) {
                // a row that fails the mask keeps key 0, below every score
                const int32_t m = __builtin_amdgcn_sbfe(static_cast<int32_t>(mwh[i][j]),
                                                        31 - (r / 4) * 8 - (r % 4), 1);
                keys[r] &= static_cast<uint32_t>(m);
              }
              mx = keys[r] > mx ? keys[r] : mx;
            }
            const bool up = mx > static_cast<uint32_t>(best[j] >> 32);
            if (__any(up)) {
              int rr = 15;
#pragma unroll
              for (int r = 15; r >= 0; --r) rr = keys[r] == mx ? r : rr;
              const int64_t row = rt + 32 * (wr * RTW + i) + (rr / 4) * 8 + (rr % 4);
              // (the seed's sample is whole tiles: row < n holds; checked all the same)
              if (up && row < n) {
                best[j] = composite(mx, static_cast<uint32_t>(sample_item(row, a.row_stride)));
              }
            }
          }
      } else {
        // fast path: the max of each group of 4 registers (rows 8 g + 4 half + 0..3), and one
        // compare per tile column against the max of its 4 group maxima
        int32_t gm[RTW][NC][4];
        int32_t thv[RTW][2];  // per row tile and column tile
        bool hit = false;
        // (with a mask, the maxima over the rows that pass it: a low masked bound would
        // otherwise send every group whose best row fails the mask to the slow path)
        auto maxima = [&](auto raw_c) {
          constexpr bool RAWV = decltype(raw_c)::value;
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                if constexpr (masked) {
                  gm[i][j][g] = group_max_masked<Op, RAWV>(acc[i][j], g, mw[i][j] << (4 * half));
                } else {
                  gm[i][j][g] = group_max<Op, RAWV>(acc[i][j], g);
                }
              }
        };
        if constexpr (FHIT) {
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) gm[i][j][g] = group_max<Op, true>(macc[i][j], g);
#pragma unroll
          for (int i = 0; i < RTW; ++i) {
            thv[i][0] = thr[i][0];
            thv[i][1] = thr[i][1];
          }
        } else {
          if (raw) {
            maxima(std::true_type{});
          } else {
            maxima(std::false_type{});
          }
#pragma unroll
          for (int i = 0; i < RTW; ++i) {
            thv[i][0] = th[0];
            thv[i][1] = th[1];
          }
        }
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            hit |= imax(imax(gm[i][j][0], gm[i][j][1]), imax(gm[i][j][2], gm[i][j][3])) >=
                   thv[i][j];
          }
        if (__any(hit)) {
          // slow path, narrowed by wave-uniform ballots: groups with a hit, then their registers
#pragma unroll
          for (int i = 0; i < RTW; ++i)
#pragma unroll
            for (int j = 0; j < NC; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                if (__ballot(gm[i][j][g] >= thv[i][j]) == 0ull) continue;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  Score sc;
                  if constexpr (FHIT) {
                    sc = Op::hit_score(macc[i][j][4 * g + u], acc0[j], 2 * i + j);
                  } else {
                    sc = acc[i][j][4 * g + u];
                  }
                  if (__ballot(sc >= ts[j]) == 0ull) continue;
                  const int64_t row = rt + 32 * (wr * RTW + i) + 8 * g + u;
                  const uint32_t item = static_cast<uint32_t>(row);
                  const uint64_t c = composite(Op::key(sc), item);
                  bool keep = row < n && sc >= ts[j] && c >= tau[j];
                  if constexpr (masked) {
                    keep = keep && ((mw[i][j] >> (31 - 8 * g - 4 * half - u)) & 1u);
                  }
                  // lanes l and l ^ 32 score the same query: the upper half's entry goes second
                  const uint64_t kb = __ballot(keep);
                  const int lo = static_cast<int>(static_cast<uint32_t>(kb) >> c32 & 1u);
                  const int hi = static_cast<int>(static_cast<uint32_t>(kb >> 32) >> c32 & 1u);
                  if (keep) {
                    lists[j][c32 * static_cast<int64_t>(a.capw) + nq[j] + (half ? lo : 0)] = c;
                  }
                  nq[j] += lo + hi;
                }
              }
          // a query gains at most 32 entries per tile: compact the lists that could overflow on
          // the next one (wave_compact waits for the stores above before reading them back)
#pragma unroll
          for (int jq = 0; jq < NC; ++jq) {
            uint64_t need = __ballot(nq[jq] > a.capw - 32 * RTW) & 0xffffffffull;
            while (need != 0ull) {
              const int c = __builtin_ctzll(need);
              need &= need - 1;
              const int q = 32 * jq + c;
              if (lane == c) cnt[q] = nq[jq];
              // (the lists hold candidates that pass the mask: with exact clauses, those that
              // fail them leave the list here and in the final merge)
              uint64_t* lq = lists[jq] + c * static_cast<int64_t>(a.capw);
              uint64_t nt;
              if constexpr (CLAUSES && masked) {
                const int64_t gq = q0[jq] + c;
                const bool cl = gq < a.B;
                nt = wave_compact(lq, &cnt[q], scratch + wave * a.capw, a.capw, a.k,
                                  [&](uint64_t v) {
                                    return !cl || clause_check(a.clause, gq, composite_item(v));
                                  });
              } else {
                nt = wave_compact(lq, &cnt[q], scratch + wave * a.capw, a.capw, a.k);
              }
              if (c32 == c) {
                nq[jq] = cnt[q];
                if (nt > tau[jq]) {
                  tau[jq] = nt;
                  ts[jq] = Op::thresh(nt);
                  th[jq] = Op::skey(ts[jq]);
                  if constexpr (FHIT) {
                    thr[0][jq] = Op::hit_thresh(th[jq], acc0[jq], jq);
                    thr[1][jq] = Op::hit_thresh(th[jq], acc0[jq], 2 + jq);
                  }
                }
              }
            }
          }
          raw = Op::kIntScores || __all(th[0] >= 0 && th[1] >= 0);
        }
      }
    };
    if (cols == 2) {
      tile_body(std::integral_constant<int, 2>{});
    } else if (cols == 1) {
      tile_body(std::integral_constant<int, 1>{});
    }
  }

  if constexpr (SEED) {
    if constexpr (CLAUSES) {
      // the maxima were taken over the mask alone: a lane whose best item fails its query's
      // clauses offers no bound (0), which keeps the bound a lower one (the merge takes the
      // k-th of at least 2 k maxima a query)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t q = q0[j] + c32;
        if (q < a.B && best[j] != 0ull &&
            !clause_check(a.clause, q, composite_item(best[j]))) {
          best[j] = 0ull;
        }
      }
    }
    // flat one-entry lists: a query's maxima, one per workgroup, at lists[q * nwg + wg]
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint64_t o = __shfl_xor(best[j], 32);
      const uint64_t b = o > best[j] ? o : best[j];
      const int64_t q = q0[j] + c32;
      if (half == 0 && q < a.B) a.lists[(q * nwg + wg) * kBlkRowHalves + wr] = b;
    }
  } else if (half == 0) {
    a.counts[slot[0] * 32 + c32] = nq[0];
    a.counts[slot[1] * 32 + c32] = nq[1];
  }
}

constexpr size_t kMaxLds = 160 * 1024;

static size_t blk_lds(int64_t row_bytes, int stages, int capw, bool wide, bool bits,
                      bool masked) {
  const int rows = blk_rows(row_bytes, wide, bits);
  return static_cast<size_t>(stages) * (rows * row_bytes + (masked ? blk_mask_bytes(rows) : 0)) +
         (wide ? 8 : 4) * (capw * sizeof(uint64_t) + kBlkQpw * sizeof(int));
}

// The deepest staging that fits a workgroup's share of LDS (all of it wide, half narrow, so two
// narrow workgroups stay resident), 0 when even three stages do not fit in the whole LDS.
static int blk_stages(int64_t row_bytes, int capw, bool wide, bool bits, bool masked) {
  const size_t share = wide ? kMaxLds : kMaxLds / 2;
  for (int s : {4, 3}) {
    if (blk_lds(row_bytes, s, capw, wide, bits, masked) <= share) return s;
  }
  // two stages: the small bit-code tiles, and the wide layout's 32 KiB tiles, beside the lists
  // of a large k
  const bool two = bits || (wide && row_bytes < 512);
  if (two && blk_lds(row_bytes, 2, capw, wide, bits, masked) <= share) return 2;
  return blk_lds(row_bytes, kBlkMinStages, capw, wide, bits, masked) <= kMaxLds ? kBlkMinStages
                                                                                 : 0;
}

// List capacity: k plus a tile's appends (one per row and query), a power of two (sorted
// whole).
static int blk_capw(int64_t k, int rows) { return static_cast<int>(next_pow2(k + rows)); }


// The layout of a batch: wide up to kBlkWideMaxBatch queries; bit codes up to
// kBlkWideMaxBatchBits, and only where k's lists fit beside the wide layout's 16 KiB tiles (the
// narrow layout's take less LDS).
static bool blk_choose_wide(int64_t row_bytes, int64_t B, int64_t k, bool bits, bool masked) {
  if (!bits) return blk_wide(row_bytes, B);
  return B <= kBlkWideMaxBatchBits &&
         blk_stages(row_bytes, blk_capw(k, blk_rows(row_bytes, true, true)), true, true,
                    masked) != 0;
}

template <class Op, int RB, bool SEED, int STAGES, bool WIDE, bool MASKED, bool CLAUSES>
static int launch_blk_kernel(const ScanArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  const void* fn = reinterpret_cast<const void*>(
      scan_blocked_kernel<Op, RB, SEED, STAGES, WIDE, MASKED, CLAUSES>);
  if (lds > 65536) {
    RT_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  scan_blocked_kernel<Op, RB, SEED, STAGES, WIDE, MASKED, CLAUSES>
      <<<grid, BlkLayout<WIDE, RB, Op::kBits>::threads, lds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// (exact clauses come with a mask only: run_blocked checks)
template <class Op, int RB, bool SEED, int STAGES, bool WIDE>
static int launch_blk_staged(const ScanArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  const bool clauses = a.clause.active != nullptr;
  if constexpr (!SEED) {
    if (a.mask != nullptr) {
      return clauses ? launch_blk_kernel<Op, RB, false, STAGES, WIDE, true, true>(a, grid, lds,
                                                                                  stream)
                     : launch_blk_kernel<Op, RB, false, STAGES, WIDE, true, false>(a, grid, lds,
                                                                                   stream);
    }
  } else {
    // (the seed takes its maxima over the staged mask too)
    if (a.mask != nullptr) {
      return clauses ? launch_blk_kernel<Op, RB, true, STAGES, WIDE, true, true>(a, grid, lds,
                                                                                 stream)
                     : launch_blk_kernel<Op, RB, true, STAGES, WIDE, true, false>(a, grid, lds,
                                                                                  stream);
    }
  }
  return launch_blk_kernel<Op, RB, SEED, STAGES, WIDE, false, false>(a, grid, lds, stream);
}

template <class Op, int RB, bool SEED, bool WIDE>
static int launch_blk_layout(const ScanArgs& a, dim3 grid, int capw, hipStream_t stream) {
  constexpr bool kBits = Op::kBits;
  if constexpr (SEED) {  // no lists in LDS: four stages always fit
    return launch_blk_staged<Op, RB, true, 4, WIDE>(
        a, grid, blk_lds(RB, 4, 0, WIDE, kBits, a.mask != nullptr), stream);
  } else {
    // the stage counts compiled: 4 or 3; 2 for bit codes and the wide layout below 512-byte rows
    // with the lists of a large k
    const bool masked = a.mask != nullptr;
    const int stages = blk_stages(RB, capw, WIDE, kBits, masked);
    const size_t lds = blk_lds(RB, stages, capw, WIDE, kBits, masked);
    if (stages == 4) return launch_blk_staged<Op, RB, false, 4, WIDE>(a, grid, lds, stream);
    if (stages == 3) return launch_blk_staged<Op, RB, false, 3, WIDE>(a, grid, lds, stream);
    if constexpr (kBits || (WIDE && RB < 512)) {
      if (stages == 2) return launch_blk_staged<Op, RB, false, 2, WIDE>(a, grid, lds, stream);
    }
    set_error("the blocked scan's lists do not fit in LDS at %d-byte rows", RB);
    return kInvalidArgument;
  }
}

template <class Op, int RB>
static int launch_blk(const ScanArgs& a, const PassPlan& p, int64_t nqg, bool seed, bool wide,
                      hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.gx), static_cast<unsigned>(nqg));
  const int capw = seed ? 0 : p.capw;
  if (wide) {
    return seed ? launch_blk_layout<Op, RB, true, true>(a, grid, capw, stream)
                : launch_blk_layout<Op, RB, false, true>(a, grid, capw, stream);
  }
  return seed ? launch_blk_layout<Op, RB, true, false>(a, grid, capw, stream)
              : launch_blk_layout<Op, RB, false, false>(a, grid, capw, stream);
}

template <class Op>
static int dispatch_blk(int64_t row_bytes, const ScanArgs& a, const PassPlan& p, int64_t nqg,
                        bool seed, bool wide, hipStream_t stream) {
  if constexpr (Op::kBits) {
    // (only 64-byte rows are instantiated for bit codes)
    if (row_bytes == 64) return launch_blk<Op, 64>(a, p, nqg, seed, wide, stream);
    set_error("the blocked bit-code scan supports 512-bit codes, got %lld bits",
              static_cast<long long>(8 * row_bytes));
    return kInvalidArgument;
  } else {
    switch (row_bytes) {
      case 128: return launch_blk<Op, 128>(a, p, nqg, seed, wide, stream);
      case 256: return launch_blk<Op, 256>(a, p, nqg, seed, wide, stream);
      case 512: return launch_blk<Op, 512>(a, p, nqg, seed, wide, stream);
      default:
        set_error("blocked scan supports rows of 128, 256 or 512 bytes, got %lld",
                  static_cast<long long>(row_bytes));
        return kInvalidArgument;
    }
  }
}

// The mask transposed for the main pass, [ceil(N/64)][stride] with stride = B rounded up to
// whole query groups: a 64 x 64 block of words per workgroup through LDS, each thread's sixteen
// loads issued before any LDS store. Padding queries are 0.
__global__ void __launch_bounds__(256) mask_transpose_kernel(const uint64_t* mask, int64_t B,
                                                             int64_t mask_words, int64_t W,
                                                             uint64_t* out, int64_t stride) {
  __shared__ uint64_t tile[64][65];
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int tx = threadIdx.x & 63;
  const int ty = threadIdx.x >> 6;
  uint64_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // row q0 + ty + 4 i of the mask, words w0 + tx
    const int64_t q = q0 + ty + 4 * i;
    const int64_t w = w0 + tx;
    v[i] = q < B && w < W ? __builtin_nontemporal_load(mask + q * mask_words + w) : 0ull;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) tile[ty + 4 * i][tx] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = tile[tx][ty + 4 * i];
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // row w0 + ty + 4 i of the output, queries q0 + tx
    const int64_t w = w0 + ty + 4 * i;
    if (w < W) out[w * stride + q0 + tx] = v[i];
  }
}


// The plan, and with a mask the transposed mask's place at the end of the workspace.
// The plan; after its own areas the speculative bounds [B] and the fallback flag, then, with a
// mask, the transposed mask.
static ScanPlan blk_plan(int64_t B, int64_t N, int64_t k, int64_t row_bytes, int64_t target_cus,
                         bool bits, bool masked, size_t* off_mask_t = nullptr,
                         size_t* off_spec = nullptr) {
  const bool wide = blk_choose_wide(row_bytes, B, k, bits, masked);
  // the row-quarter layout covers column tiles 0-3 only (B <= kBlkWideMaxBatch = 128), the bit
  // codes' eight row parts tiles 0-1 (B <= 64): their lists are sized for those queries
  const int halves = blk_halves(row_bytes, wide, bits);
  const int64_t qpg = halves == 8 ? kBlkQpg / 4 : (halves == 4 ? kBlkQpg / 2 : kBlkQpg);
  ScanPlan p = plan_scan(B, N, k, qpg, halves * qpg, target_cus * (wide ? 1 : 2),
                         blk_capw(k, blk_rows(row_bytes, wide, bits)), kBlkRows);
  if (off_spec != nullptr) *off_spec = align_up(p.total, 256);
  p.total = align_up(p.total, 256) + align_up(static_cast<size_t>(B) * sizeof(uint64_t), 256) +
            256;
  if (off_mask_t != nullptr) *off_mask_t = align_up(p.total, 256);
  if (masked) {
    p.total = align_up(p.total, 256) +
              static_cast<size_t>(cdiv(N, 64)) * static_cast<size_t>(cdiv(B, kBlkQpg) * kBlkQpg) *
                  sizeof(uint64_t);
  }
  return p;
}





template <class Op>
static int run_blocked(const void* queries, int64_t B, const void* items, int64_t N,
                       int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                       int64_t* out_ids, void* out_scores, void* workspace,
                       size_t workspace_bytes, hipStream_t stream, int score_kind = Op::kind,
                       const ClauseCheck& clause = ClauseCheck{}, int64_t mask_t_stride = 0) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(items) % 16 == 0,
               "queries and items must be 16-byte aligned");
  RT_CHECK_ARG(mask == nullptr || mask_words >= cdiv(N, 64), "mask must have ceil(N/64) words");
  // (the seed pass takes its maxima over the mask and tests only each lane's best against the
  // clauses: without a mask that bound would rarely hold)
  RT_CHECK_ARG(clause.active == nullptr || mask != nullptr,
               "the blocked scan tests exact clauses only together with a mask");
  if (B == 0) return kOk;
  RT_CHECK_ARG(out_ids != nullptr && out_scores != nullptr, "out_ids and out_scores are null");
  if (N == 0) return launch_pad(out_ids, out_scores, B, k, score_kind, stream);
  RT_CHECK_ARG(queries != nullptr && items != nullptr && workspace != nullptr,
               "queries, items and workspace must not be null");
  int dev = 0;
  int cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  }
  const bool wide = blk_choose_wide(row_bytes, B, k, Op::kBits, mask != nullptr);
  size_t off_mask_t = 0;
  size_t off_spec = 0;
  const ScanPlan plan = blk_plan(B, N, k, row_bytes, cus, Op::kBits, mask != nullptr,
                                 &off_mask_t, &off_spec);
  RT_CHECK_ARG(blk_stages(row_bytes, plan.main.capw, wide, Op::kBits, mask != nullptr) != 0,
               "k = %lld is too large for the blocked scan at %lld-byte rows",
               static_cast<long long>(k), static_cast<long long>(row_bytes));
  if (workspace_bytes < plan.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, plan.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* lists = reinterpret_cast<uint64_t*>(ws + plan.off_lists);
  int* counts = reinterpret_cast<int*>(ws + plan.off_counts);
  uint64_t* tau = reinterpret_cast<uint64_t*>(ws + plan.off_tau);
  uint64_t* spec = reinterpret_cast<uint64_t*>(ws + off_spec);
  uint32_t* spec_flag = reinterpret_cast<uint32_t*>(
      ws + off_spec + align_up(static_cast<size_t>(B) * sizeof(uint64_t), 256));

  ScanArgs a{};
  a.queries = queries;
  a.B = B;
  a.items = items;
  a.k = static_cast<int>(k);
  a.qpw = kBlkQpw;
  a.mask = mask;
  a.mask_words = mask_words;
  a.lists = lists;
  a.counts = counts;
  a.clause = clause;
  if (mask != nullptr && mask_t_stride > 0) {
    // the mask given transposed: [mask_words >= ceil(N/64) rows, mask_t_stride >= the padded
    // batch] (rt_bloom_search_t's layout)
    RT_CHECK_ARG(mask_t_stride >= cdiv(B, kBlkQpg) * kBlkQpg,
                 "a transposed mask needs a stride of at least %lld, got %lld",
                 static_cast<long long>(cdiv(B, kBlkQpg) * kBlkQpg),
                 static_cast<long long>(mask_t_stride));
    a.mask_t = mask;
    a.mask_t_stride = mask_t_stride;
    a.mask_t_rows = mask_words;
  } else if (mask != nullptr) {
    const int64_t W = cdiv(N, 64);
    const int64_t stride = cdiv(B, kBlkQpg) * kBlkQpg;
    uint64_t* mask_t = reinterpret_cast<uint64_t*>(ws + off_mask_t);
    RT_CHECK_ARG(cdiv(W, 64) < (int64_t{1} << 31), "N too large");
    mask_transpose_kernel<<<dim3(static_cast<unsigned>(cdiv(W, 64)),
                                 static_cast<unsigned>(stride / 64)),
                            256, 0, stream>>>(mask, B, mask_words, W, mask_t, stride);
    RT_CHECK_HIP(hipGetLastError());
    a.mask_t = mask_t;
    a.mask_t_stride = stride;
    a.mask_t_rows = W;
  }

  MergeArgs m{};
  m.lists = lists;
  m.counts = counts;
  m.clause = clause;  // (the main pass's lists hold candidates that pass the mask)
  m.qpw = 32;  // one list per query per slot; a slot is (32-query column tile, workgroup, half)
  m.B = B;
  m.k = static_cast<int>(k);

  if (plan.seeded) {
    a.n_rows = plan.seed.n_rows;
    a.row_stride = plan.seed.row_stride;
    a.capw = 1;
    a.tau_in = nullptr;
    int st = dispatch_blk<Op>(row_bytes, a, plan.seed, plan.n_qgroups, true, wide, stream);
    if (st != kOk) return st;
    m.capw = 1;
    m.flat = true;
    m.S = plan.seed.S;
    m.tau_out = tau;
    // the speculative bound from the same lists (below)
    const int rank = sample_rank(k, plan.seed.row_stride);
    if (rank < k) {
      m.tau2_out = spec;
      m.k2 = rank;
      m.spec_flag = spec_flag;  // (cleared)
    }
    st = launch_merge(m, stream);
    if (st != kOk) return st;
    m.tau_out = nullptr;
    m.tau2_out = nullptr;
    m.spec_flag = nullptr;
    m.flat = false;
  }
  a.n_rows = N;
  a.row_stride = 1;
  a.capw = plan.main.capw;
  a.tau_in = plan.seeded ? tau : nullptr;
  // The speculative bound: the seed's rank-th best (sample_rank of its row stride) beside its
  // k-th, both from the seed merge above (the rank-th at least the k-th). The lists hold each
  // seed workgroup's best over its strip of the sample, so the rank-th of them is at most the
  // sample's rank-th best; the main pass then keeps about rank * stride candidates a query
  // instead of N k / (seed rows). A query that ends with fewer than k entries although its
  // bound was above the seed's k-th raises a flag, and the fallback (the main pass and the
  // merge again behind the k-th, both returning at once on the device while the flag is clear)
  // keeps every result exact.
  const bool speculative = plan.seeded && sample_rank(k, plan.seed.row_stride) < k;
  if (speculative) a.tau_in = spec;
  hipEvent_t stop;
  profile_begin(stream, &stop);
  int st = dispatch_blk<Op>(row_bytes, a, plan.main, plan.n_qgroups, false, wide, stream);
  profile_end(stream, stop);
  if (st != kOk) return st;
  m.capw = plan.main.capw;
  m.S = plan.main.S;
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = score_kind;
  if (speculative) {
    m.spec_flag = spec_flag;
    m.spec_tau = spec;
    m.safe_tau = tau;
  }
  st = launch_merge(m, stream);
  if (st != kOk || !speculative) return st;
  // the fallback behind the seed's bound (returns at once while the flag is clear)
  a.tau_in = tau;
  a.run_if = spec_flag;
  st = dispatch_blk<Op>(row_bytes, a, plan.main, plan.n_qgroups, false, wide, stream);
  if (st != kOk) return st;
  m.spec_flag = nullptr;
  m.run_if = spec_flag;
  return launch_merge(m, stream);
}

}  // namespace
}  // namespace rt

namespace rt {

// One translation unit per operand type (scan_blocked_{i8,bf16,f16,f32}.hip): row_bytes = D
// times the element size; `clause`: exact clauses tested per candidate (with a mask only).
int blocked_scan_i8(const void* queries, int64_t B, const void* items, int64_t N,
                    int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                    hipStream_t stream, const ClauseCheck& clause = ClauseCheck{},
                    int64_t mask_t_stride = 0);
int blocked_scan_bf16(const void* queries, int64_t B, const void* items, int64_t N,
                      int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                      int64_t* out_ids, void* out_scores, void* workspace,
                      size_t workspace_bytes, hipStream_t stream,
                      const ClauseCheck& clause = ClauseCheck{},
                    int64_t mask_t_stride = 0);
int blocked_scan_f16(const void* queries, int64_t B, const void* items, int64_t N,
                     int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                     int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                     hipStream_t stream, const ClauseCheck& clause = ClauseCheck{},
                    int64_t mask_t_stride = 0);
int blocked_scan_f32(const void* queries, int64_t B, const void* items, int64_t N,
                     int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                     int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                     hipStream_t stream, const ClauseCheck& clause = ClauseCheck{},
                    int64_t mask_t_stride = 0);

}  // namespace rt
