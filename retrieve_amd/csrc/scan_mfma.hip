// Dense full scans with the exact fused top-k, on the matrix cores: int8 × int8 → int32
// (SilverTorch's int8 scorer semantics: int32 accumulation; v_mfma_i32_16x16x64_i8) and
// bf16 / fp16 × same → fp32 (LiNR's dense scores; v_mfma_f32_16x16x32_bf16 / _f16). Ties go to
// the lower item index.
//
// Each wave multiplies 16-item tiles of the item table against its 16 queries (items as the
// A operand, queries as B), so after a tile lane l holds the scores of query l % 16 for items
// 4 * (l / 16) + r, r < 4. Every MFMA consumes 64 bytes of each row: lane l feeds bytes
// [64 s + 16 (l / 16), +16) of its item row and of its query row at step s, the same bytes on
// both sides (the K order inside an operand is free: exact for integers, and within the fp32
// rounding the tolerance covers for the float types).
//
// Main pass: a tile (16 contiguous rows, 16 * D bytes) is read with coalesced nontemporal
// 16-byte loads (each instruction 1 KiB contiguous), staged in the wave's LDS with rows padded
// by 16 bytes, and read back in the MFMA layout. Tiles are dealt round-robin over all waves of
// a query group, so the whole GPU streams one contiguous window of the table at a time.
// Seed pass: the strided sample, read directly in the MFMA layout (rows are not contiguous).
#include <mutex>

#include "mfma_topk.h"
#include "profile.h"
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// One MFMA step (64 bytes of K) per element type. Score is the per-item score type.
struct I8Op {
  using Score = int32_t;
  using Acc = v4i;
  static constexpr int kind = kScoreI32;
  __device__ static Acc zero() { return Acc{0, 0, 0, 0}; }
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

struct BF16Op {
  using Score = float;
  using Acc = v4f;
  static constexpr int kind = kScoreF32;
  __device__ static Acc zero() { return Acc{0.f, 0.f, 0.f, 0.f}; }
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                   __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  }
};

struct F16Op {
  using Score = float;
  using Acc = v4f;
  static constexpr int kind = kScoreF32;
  __device__ static Acc zero() { return Acc{0.f, 0.f, 0.f, 0.f}; }
  __device__ static Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a),
                                                  __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
};

// KSTEPS = row bytes / 64 (D * element size / 64).
template <int KSTEPS>
__device__ inline void load_query_fragments(const ScanArgs& a, int64_t qrow, int grp, v4i* qf) {
  constexpr int64_t D = KSTEPS * 64;  // row bytes
  const int8_t* Q = static_cast<const int8_t*>(a.queries);
  if (qrow < a.B) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      qf[s] = *reinterpret_cast<const v4i*>(Q + qrow * D + s * 64 + grp * 16);
    }
  } else {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qf[s] = v4i{0, 0, 0, 0};
  }
}

// Seed pass over the strided sample: each wave keeps, per query, only its best composite over
// its rows and writes it to a.lists[qrow * S + wave index] (S = waves of the grid row); the
// k-th largest of those maxima is a lower bound on the k-th best item (k distinct waves each
// hold an item at least that good).
template <class Op, int KSTEPS>
__global__ void __launch_bounds__(kScanThreads) seed_mfma_kernel(ScanArgs a) {
  using Score = typename Op::Score;
  constexpr int64_t D = KSTEPS * 64;  // row bytes
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int8_t* I = static_cast<const int8_t*>(a.items);
  const int64_t qrow = static_cast<int64_t>(blockIdx.y) * 16 + col;
  v4i qf[KSTEPS];
  load_query_fragments<KSTEPS>(a, qrow, grp, qf);
  const uint64_t* qmask =
      a.mask != nullptr && qrow < a.B ? a.mask + qrow * a.mask_words : nullptr;
  const bool clauses = a.clause.active != nullptr && qrow < a.B;
  const uint64_t* bm = nullptr;
  if (a.clause.active != nullptr && a.clause_lds) {
    // the group's set bitmaps in LDS (the host sized the launch for them)
    extern __shared__ __attribute__((aligned(16))) uint64_t seed_bm[];
    const int per_row = a.clause.C * kSetWords;
    const int64_t g0 = static_cast<int64_t>(blockIdx.y) * 16;
    for (int i = threadIdx.x; i < 16 * per_row; i += kScanThreads) {
      const int64_t b = g0 + i / per_row;
      seed_bm[i] = b < a.B ? a.clause.bitmaps[b * per_row + i % per_row] : 0ull;
    }
    __syncthreads();
    bm = seed_bm + col * per_row;
  }
  const ClauseRow crow = clauses ? clause_row(a.clause, qrow, bm) : ClauseRow{};
  const bool held = clauses && a.clause.held;

  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * a.strip;
  const int64_t r1 = r0 + a.strip < a.n_rows ? r0 + a.strip : a.n_rows;
  const int64_t ntiles = r1 > r0 ? cdiv(r1 - r0, kTile) : 0;
  uint64_t best = 0ull;
  // Tile t's loads: its rows' fragments, this lane's four rows' attributes (held rows: loaded
  // before it is known which rows are candidates, so the tests wait on the same round of
  // loads) and their mask word (four sample rows from a multiple of four are consecutive items
  // of one word). A wave takes tiles wave, + kScanWaves, ... with two tiles' loads in flight:
  // buffers A and B alternate, each reloaded with the tile two ahead right after it is scored;
  // past the strip a buffer reloads the last tile (never used), so every load is unconditional
  // and the waits before a tile cover only the loads issued before its own.
  struct SeedTile {
    v4i af[KSTEPS];
    AttrRow rows[4];
    uint64_t mw;
  };
  // HB: the held rows' bytes (0: not held), MASKED: a mask; both compile-time, so no branch
  // sits between a tile's loads and the waits before it is scored
  auto run = [&](auto hb_c, auto masked_c) {
  constexpr int HB = decltype(hb_c)::value;
  constexpr bool MASKED = decltype(masked_c)::value;
  auto fetch = [&](int64_t t, SeedTile& b) {
    const int64_t rb = r0 + (t < ntiles ? t : ntiles - 1) * kTile;
    const int64_t lr = rb + col < r1 ? rb + col : r1 - 1;
    const int8_t* ip = I + sample_item(lr, a.row_stride) * D + grp * 16;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) b.af[s] = *reinterpret_cast<const v4i*>(ip + s * 64);
    const int64_t row0 = rb + 4 * grp;
    if constexpr (HB > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = row0 + r;
        b.rows[r] = load_attr_row_n<HB>(a.clause,
                                        sample_item(row < r1 ? row : r1 - 1, a.row_stride));
      }
    }
    if constexpr (MASKED) {
      b.mw = qmask[sample_item(row0 < r1 ? row0 : r1 - 1, a.row_stride) >> 6];
    } else {
      b.mw = ~0ull;
    }
  };
  auto score = [&](int64_t t, const SeedTile& b) {
    const int64_t rb = r0 + t * kTile;
    typename Op::Acc acc = Op::zero();
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) acc = Op::mma(b.af[s], qf[s], acc);
    // the rows whose composite would raise the maximum, then the filters on them only: the
    // mask word, then the clauses from the best row down until one passes
    uint64_t cs[4];
    uint32_t cand = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = rb + 4 * grp + r;
      cs[r] = composite(KeyOps<Score>::key(acc[r]),
                        static_cast<uint32_t>(sample_item(row, a.row_stride)));
      cand |= row < r1 && cs[r] > best ? 1u << r : 0u;
    }
    if (MASKED && cand != 0u) {
      const int64_t item0 = sample_item(rb + 4 * grp, a.row_stride);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        cand &= (b.mw >> (63 - ((item0 + r) & 63))) & 1ull ? ~0u : ~(1u << r);
      }
    }
    if (HB > 0 && cand != 0u) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if ((cand >> r) & 1u && !clause_pass_held(a.clause, crow, b.rows[r])) {
          cand &= ~(1u << r);
        }
      }
    }
    if (!clauses || HB > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) best = (cand >> r) & 1u && cs[r] > best ? cs[r] : best;
    }
    while (__any(clauses && HB == 0 && cand != 0u)) {
      if (clauses && HB == 0 && cand != 0u) {
        int rb_ = 0;
        uint64_t cb = 0ull;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if ((cand >> r) & 1u && cs[r] > cb) {
            cb = cs[r];
            rb_ = r;
          }
        }
        cand &= ~(1u << rb_);
        if (clause_pass(a.clause, crow, sample_item(rb + 4 * grp + rb_, a.row_stride))) {
          best = cb;
          cand = 0u;
        }
      }
    }
  };
  SeedTile ba;
  SeedTile bb;
  fetch(wave, ba);
  fetch(wave + kScanWaves, bb);
  for (int64_t t = wave; t < ntiles; t += 2 * kScanWaves) {
    score(t, ba);
    fetch(t + 2 * kScanWaves, ba);
    if (t + kScanWaves >= ntiles) break;
    score(t + kScanWaves, bb);
    fetch(t + 3 * kScanWaves, bb);
  }
  };
  // (uniform: the row size and the mask are the launch's)
  const int hb = held ? a.clause.C * a.clause.A * a.clause.attr_bytes : 0;
  auto run_hb = [&](auto masked_c) {
    if (hb == 16) {
      run(std::integral_constant<int, 16>{}, masked_c);
    } else if (hb == 8) {
      run(std::integral_constant<int, 8>{}, masked_c);
    } else if (hb == 4) {
      run(std::integral_constant<int, 4>{}, masked_c);
    } else {
      run(std::integral_constant<int, 0>{}, masked_c);
    }
  };
  if (ntiles > 0) {
    if (qmask != nullptr) {
      run_hb(std::true_type{});
    } else {
      run_hb(std::false_type{});
    }
  }
  uint64_t o = __shfl_xor(best, 16);
  best = o > best ? o : best;
  o = __shfl_xor(best, 32);
  best = o > best ? o : best;
  const int64_t S = static_cast<int64_t>(gridDim.x) * kScanWaves;
  if (lane < 16 && qrow < a.B) {
    a.lists[qrow * S + static_cast<int64_t>(blockIdx.x) * kScanWaves + wave] = best;
  }
}

// LDS row pitch of a staged tile: D + 16 bytes, so the 16 rows of an MFMA read start on
// different banks.
template <int KSTEPS>
constexpr int tile_pitch() {
  return KSTEPS * 64 + 16;
}

template <int KSTEPS>
constexpr size_t main_static_lds() {
  return static_cast<size_t>(kScanWaves) * kTile * tile_pitch<KSTEPS>();
}

// LDS of the clause bitmaps a main-pass workgroup copies (its 16 queries).
__host__ __device__ inline size_t clause_lds_bytes(int C) {
  return static_cast<size_t>(16) * C * kSetWords * sizeof(uint64_t);
}

// Main pass: every item (row_stride 1), candidate lists per wave.
template <class Op, int KSTEPS>
__global__ void __launch_bounds__(kScanThreads) scan_mfma_kernel(ScanArgs a) {
  using Score = typename Op::Score;
  constexpr int64_t D = KSTEPS * 64;  // row bytes
  constexpr int P = tile_pitch<KSTEPS>();
  if (a.run_if != nullptr && *a.run_if == 0u) return;  // (uniform: the fallback is not needed)
  constexpr int LOADS = KSTEPS;  // 16-byte loads per lane per tile: 16 * D / 1024
  extern __shared__ __attribute__((aligned(16))) uint64_t smem[];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  int8_t* base = reinterpret_cast<int8_t*>(smem);
  int8_t* stage = base + wave * kTile * P;
  uint64_t* scratch = reinterpret_cast<uint64_t*>(base + main_static_lds<KSTEPS>()) + wave * a.capw;
  int* cnt = reinterpret_cast<int*>(base + main_static_lds<KSTEPS>() +
                                    kScanWaves * a.capw * sizeof(uint64_t)) + wave * 16;
  const int64_t wave_in_group = static_cast<int64_t>(blockIdx.x) * kScanWaves + wave;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kScanWaves;
  const int64_t slot = static_cast<int64_t>(blockIdx.y) * waves + wave_in_group;
  if (lane < 16) cnt[lane] = 0;

  const int8_t* I = static_cast<const int8_t*>(a.items);
  const int64_t qrow = static_cast<int64_t>(blockIdx.y) * 16 + col;
  v4i qf[KSTEPS];
  load_query_fragments<KSTEPS>(a, qrow, grp, qf);
  WaveTopK16<Score> top;
  top.lists = a.lists + slot * 16 * a.capw;
  top.cnt = cnt;
  top.scratch = scratch;
  top.capw = a.capw;
  top.k = a.k;
  top.qmask = a.mask != nullptr && qrow < a.B ? a.mask + qrow * a.mask_words : nullptr;
  top.clause = a.clause;
  top.clauses = a.clause.active != nullptr && qrow < a.B;  // a padding column tests nothing
  if (a.clause.active != nullptr) {
    // the group's set bitmaps in LDS (after the lists' counts) when the host planned room
    const uint64_t* bm = nullptr;
    if (a.clause_lds) {
      uint64_t* lds_bm = reinterpret_cast<uint64_t*>(
          base + main_static_lds<KSTEPS>() + kScanWaves * a.capw * sizeof(uint64_t) +
          kScanWaves * 16 * sizeof(int));
      const int per_row = a.clause.C * kSetWords;
      const int64_t g0 = static_cast<int64_t>(blockIdx.y) * 16;
      for (int i = threadIdx.x; i < 16 * per_row; i += kScanThreads) {
        const int64_t b = g0 + i / per_row;
        lds_bm[i] = b < a.B ? a.clause.bitmaps[b * per_row + i % per_row] : 0ull;
      }
      __syncthreads();
      bm = lds_bm + col * per_row;
    }
    if (top.clauses) top.crow = clause_row(a.clause, qrow, bm);
  }
  if (a.probe.doc_bits != nullptr) {
    // the group's Bloom clause tables copied to LDS (after the set bitmaps) while they fit, in
    // query order; the others are read where they are
    uint64_t* tl = reinterpret_cast<uint64_t*>(
        base + main_static_lds<KSTEPS>() + kScanWaves * a.capw * sizeof(uint64_t) +
        kScanWaves * 16 * sizeof(int) + (a.clause_lds ? clause_lds_bytes(a.clause.C) : 0));
    const int cap = a.probe_lds / static_cast<int>(sizeof(uint64_t));
    const uint64_t* tables = a.probe.tables;
    const int64_t g0 = static_cast<int64_t>(blockIdx.y) * 16;
    const int64_t g1 = g0 + 16 < a.B ? g0 + 16 : a.B;
    const int64_t o0 = static_cast<int64_t>(tables[g0]);
    const int words = static_cast<int>(static_cast<int64_t>(tables[g1]) - o0);
    top.tables_lds = words <= cap;  // (uniform: the group's tables are contiguous)
    if (top.tables_lds) {
      for (int w = threadIdx.x; w < words; w += kScanThreads) tl[w] = tables[o0 + w];
      __syncthreads();
      top.lds = (lds_cu64*)(tl);
    }
    if (qrow < a.B) {
      const int64_t o = static_cast<int64_t>(tables[qrow]);
      top.table = tables + o;
      top.lds_at = static_cast<int>(o - o0);
    }
    top.doc_bits = a.probe.doc_bits;
    top.probe_on = true;
    top.probing = qrow < a.B;
  }
  top.set_tau(qrow < a.B ? (a.tau_in != nullptr ? a.tau_in[qrow] : 0ull) : ~0ull);
  wave_sync_memory();

  const int64_t n = a.n_rows;
  const int64_t ntiles = cdiv(n, kTile);
  // load j of a tile covers its bytes [1024 j + 16 lane, +16): row (1024 j + 16 lane) / D
  auto load_tile = [&](int64_t t, v4i (&v)[LOADS]) {
    const int64_t base_row = t * kTile;
    const v4i* src = reinterpret_cast<const v4i*>(I + base_row * D) + lane;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int off = 1024 * j + 16 * lane;
      const int64_t row = base_row + off / D;
      v[j] = row < n ? __builtin_nontemporal_load(src + 64 * j) : v4i{0, 0, 0, 0};
    }
  };
  // one tile: staged from registers, the registers reloaded with tile `next` (when it exists),
  // then the MFMAs and the candidates
  auto tile = [&](int64_t t, v4i (&v)[LOADS], int64_t next) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int off = 1024 * j + 16 * lane;
      *reinterpret_cast<v4i*>(stage + (off / D) * P + off % D) = v[j];
    }
    wave_sync_memory();
    v4i af[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      af[s] = *reinterpret_cast<const v4i*>(stage + col * P + grp * 16 + s * 64);
    }
    if (next < ntiles) load_tile(next, v);
    typename Op::Acc acc = Op::zero();
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) acc = Op::mma(af[s], qf[s], acc);
    const Score sc[4] = {acc[0], acc[1], acc[2], acc[3]};
    top.push(sc, t * kTile + 4 * grp, n, 1);
    wave_sync_memory();
  };

  // rows up to 512 bytes keep two tiles in flight per wave (two register sets), wider rows one
  v4i va[LOADS];
  int64_t t = wave_in_group;
  if constexpr (KSTEPS <= 8) {
    v4i vb[LOADS];
    if (t < ntiles) load_tile(t, va);
    if (t + waves < ntiles) load_tile(t + waves, vb);
    for (; t < ntiles; t += 2 * waves) {
      tile(t, va, t + 2 * waves);
      if (t + waves >= ntiles) break;
      tile(t + waves, vb, t + 3 * waves);
    }
  } else {
    if (t < ntiles) load_tile(t, va);
    for (; t < ntiles; t += waves) tile(t, va, t + waves);
  }
  wave_sync_memory();
  if (lane < 16) a.counts[slot * 16 + lane] = cnt[lane];
}

template <int KSTEPS>
static size_t main_lds_bytes(int capw) {
  return main_static_lds<KSTEPS>() + kScanWaves * (capw * sizeof(uint64_t) + 16 * sizeof(int));
}

// The most the main pass gives the LDS copies below: they are made only while two workgroups
// still fit a CU.
constexpr size_t kMainLdsForTwo = 80 * 1024;
// The most LDS the seed pass gives its copies of the set bitmaps.
constexpr size_t kSeedClauseLds = 32 * 1024;
// LDS for a main-pass workgroup's copies of its queries' Bloom clause tables: none below the
// minimum, at most the maximum, within the two-workgroup budget.
constexpr size_t kProbeLdsMin = 4 * 1024;
constexpr size_t kProbeLdsMax = 24 * 1024;

template <class Op, int KSTEPS>
static int launch_mfma(const ScanArgs& a, const PassPlan& p, int64_t n_qgroups, bool seed,
                       hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.gx), static_cast<unsigned>(n_qgroups));
  if (seed) {
    // the seed copies its group's set bitmaps to LDS when they are small
    ScanArgs s = a;
    const size_t bm = a.clause.active != nullptr ? clause_lds_bytes(a.clause.C) : 0;
    s.clause_lds = bm > 0 && bm <= kSeedClauseLds;
    seed_mfma_kernel<Op, KSTEPS><<<grid, kScanThreads, s.clause_lds ? bm : 0, stream>>>(s);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  ScanArgs m = a;
  size_t lds = main_lds_bytes<KSTEPS>(p.capw);
  m.clause_lds =
      a.clause.active != nullptr && lds + clause_lds_bytes(a.clause.C) <= kMainLdsForTwo;
  if (m.clause_lds) lds += clause_lds_bytes(a.clause.C);
  m.probe_lds = 0;
  if (a.probe.doc_bits != nullptr && lds + kProbeLdsMin <= kMainLdsForTwo) {
    const size_t room = kMainLdsForTwo - lds;
    m.probe_lds = static_cast<int>((room < kProbeLdsMax ? room : kProbeLdsMax) / 16 * 16);
    lds += m.probe_lds;
  }
  if (lds > 65536) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(scan_mfma_kernel<Op, KSTEPS>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  scan_mfma_kernel<Op, KSTEPS><<<grid, kScanThreads, lds, stream>>>(m);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// Row sizes supported: 64, 128, 256, 512, 768, 1024 bytes (int8 D; half the D for 16-bit).
template <class Op>
static int dispatch_mfma(int64_t row_bytes, const ScanArgs& a, const PassPlan& p, int64_t nqg,
                         bool seed, hipStream_t stream) {
  switch (row_bytes) {
    case 64: return launch_mfma<Op, 1>(a, p, nqg, seed, stream);
    case 128: return launch_mfma<Op, 2>(a, p, nqg, seed, stream);
    case 256: return launch_mfma<Op, 4>(a, p, nqg, seed, stream);
    case 512: return launch_mfma<Op, 8>(a, p, nqg, seed, stream);
    case 768: return launch_mfma<Op, 12>(a, p, nqg, seed, stream);
    case 1024: return launch_mfma<Op, 16>(a, p, nqg, seed, stream);
    default:
      set_error("dense scan supports rows of 64, 128, 256, 512, 768 or 1024 bytes, got %lld",
                static_cast<long long>(row_bytes));
      return kInvalidArgument;
  }
}

// List capacity: k kept after a compaction plus room for the next tiles' appends (a tile adds
// at most 16 per query), a power of two (the compaction sorts it whole).
static int mfma_capw(int64_t k) { return static_cast<int>(next_pow2(k + 2 * kTile)); }

// Seed rows: half the default sample. Behind the sample's rank-th best (sample_rank) the main
// pass keeps about k + 5 sqrt(k * stride) + 4 * stride candidates a query, few enough that the
// smaller sample's cheaper seed pass wins (filtered int8 at B = 16 over 30M rows: 2.362 ms a
// step with 2^19 rows, 2.347 with 2^18, 2.344 with 2^17; int8 at B = 1 2.266 / 2.247 / 2.242).
static int64_t mfma_seed_rows(int64_t B, int64_t N) {
  (void)B;
  (void)N;
  return kSeedRows / 2;
}

// Rows of the seed sample a workgroup takes: kSeedTiles 16-row tiles a wave, two tiles' loads
// in flight (2048 one-entry lists a query from 2^17 sampled rows). Four tiles keep four waves a
// SIMD for the clause tests' dependent LDS lookups; one tile a wave (8192 lists) merged slower,
// eight (one wave a SIMD) left the clause seed latency-bound: the filtered int8 step at B = 16
// 2.349-2.352 ms with eight, 2.338-2.341 ms with four (the plain int8 scan 2.253 / 2.260 ms).
constexpr int kSeedTiles = 4;

// The plan of a scan of B queries over N rows, top-k, over target_wgs main-pass workgroups.
static ScanPlan mfma_plan(int64_t B, int64_t N, int64_t k, int64_t target_wgs) {
  return plan_scan(B, N, k, 16, kScanWaves * 16, target_wgs, mfma_capw(k),
                   kScanWaves * kTile * kSeedTiles, mfma_seed_rows(B, N));
}

// seed scan → seed threshold merge → main scan → final merge, on `stream`, no host sync
template <class Op>
static int run_mfma_scan(const void* queries, int64_t B, const void* items, int64_t N,
                         int64_t row_bytes, int64_t k, const uint64_t* mask, int64_t mask_words,
                         int64_t* out_ids, void* out_scores, void* workspace,
                         size_t workspace_bytes, hipStream_t stream,
                         const ClauseCheck& clause = ClauseCheck{},
                         const BloomProbe& probe = BloomProbe{}) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(items) % 16 == 0,
               "queries and items must be 16-byte aligned");
  RT_CHECK_ARG(mask == nullptr || mask_words >= cdiv(N, 64), "mask must have ceil(N/64) words");
  if (B == 0) return kOk;
  RT_CHECK_ARG(out_ids != nullptr && out_scores != nullptr, "out_ids and out_scores are null");
  if (N == 0) return launch_pad(out_ids, out_scores, B, k, Op::kind, stream);
  RT_CHECK_ARG(queries != nullptr && items != nullptr && workspace != nullptr,
               "queries, items and workspace must not be null");
  const ScanPlan plan = mfma_plan(B, N, k, main_workgroups());
  if (workspace_bytes < plan.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, plan.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* lists = reinterpret_cast<uint64_t*>(ws + plan.off_lists);
  int* counts = reinterpret_cast<int*>(ws + plan.off_counts);
  uint64_t* tau = reinterpret_cast<uint64_t*>(ws + plan.off_tau);
  uint32_t* spec_flag = reinterpret_cast<uint32_t*>(ws + plan.off_flag);
  // The seed's bound is its sample's rank-th best (sample_rank: k -> about 13 at k = 100 and one
  // row in 57 sampled), not its k-th: the main pass then keeps about rank * stride candidates a
  // query instead of k * stride. With the Bloom probe the seed also takes its bound over the
  // exact clauses alone (a sampled item that passes them is not probed), which bounds the
  // filter's k-th best only where the plans pass every item the clauses pass. A query that
  // ends with fewer than k entries behind a bound above 0 raises a flag, and a fallback main
  // pass and merge without the bound (both returning at once while the flag is clear) keep the
  // results exact.
  const int rank = plan.seeded ? sample_rank(k, plan.seed.row_stride) : static_cast<int>(k);
  const bool speculative = plan.seeded && (rank < k || probe.doc_bits != nullptr);

  ScanArgs a{};
  a.queries = queries;
  a.B = B;
  a.items = items;
  a.k = static_cast<int>(k);
  a.qpw = 16;
  a.mask = mask;
  a.mask_words = mask_words;
  a.lists = lists;
  a.counts = counts;
  a.clause = clause;

  MergeArgs m{};
  m.lists = lists;
  m.counts = counts;
  m.qpw = 16;
  m.B = B;
  m.k = static_cast<int>(k);

  if (plan.seeded) {
    a.n_rows = plan.seed.n_rows;
    a.row_stride = plan.seed.row_stride;
    a.strip = plan.seed.strip;
    a.capw = 1;
    a.tau_in = nullptr;
    int st = dispatch_mfma<Op>(row_bytes, a, plan.seed, plan.n_qgroups, true, stream);
    if (st != kOk) return st;
    m.capw = 1;
    m.flat = true;  // one entry per seed wave, contiguous per query
    m.S = plan.seed.S;
    m.tau_out = tau;
    m.k = rank;
    m.spec_flag = speculative ? spec_flag : nullptr;  // (cleared)
    st = launch_merge(m, stream);
    if (st != kOk) return st;
    m.k = static_cast<int>(k);
    m.tau_out = nullptr;
    m.flat = false;
    m.spec_flag = nullptr;
  }
  a.probe = probe;
  a.n_rows = N;
  a.row_stride = 1;
  a.strip = plan.main.strip;
  a.capw = plan.main.capw;
  // the final merge over the main pass's lists split into parts (small batches); the seed's
  // flat merge above is one launch (its 1024 one-entry lists a query merge faster whole)
  m.part_buf = plan.split ? reinterpret_cast<uint64_t*>(ws + plan.off_parts) : nullptr;
  a.clause_lds = 0;  // the main pass's launch decides
  a.tau_in = plan.seeded ? tau : nullptr;
  hipEvent_t stop;
  profile_begin(stream, &stop);
  int st = dispatch_mfma<Op>(row_bytes, a, plan.main, plan.n_qgroups, false, stream);
  profile_end(stream, stop);
  if (st != kOk) return st;
  m.capw = plan.main.capw;
  m.S = plan.main.S;
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = Op::kind;
  if (speculative) {
    m.spec_flag = spec_flag;
    m.spec_tau = tau;
    m.safe_tau = nullptr;
  }
  st = launch_merge(m, stream);
  if (st != kOk || !speculative) return st;
  a.tau_in = nullptr;
  a.run_if = spec_flag;
  st = dispatch_mfma<Op>(row_bytes, a, plan.main, plan.n_qgroups, false, stream);
  if (st != kOk) return st;
  m.spec_flag = nullptr;
  m.run_if = spec_flag;
  m.part_buf = nullptr;  // (one launch: it returns at once while the flag is clear)
  return launch_merge(m, stream);
}

}  // namespace rt

using namespace rt;

extern "C" size_t rt_int8_scan_topk_workspace(int64_t B, int64_t N, int64_t D, int64_t k) {
  (void)D;
  return mfma_plan(B, N, k, kMaxResidentWorkgroups)
      .total;
}

extern "C" int rt_int8_scan_topk(const int8_t* queries, int64_t B, const int8_t* items,
                                 int64_t N, int64_t D, int64_t k, const uint64_t* mask,
                                 int64_t mask_words, int64_t* out_ids, int32_t* out_scores,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return run_mfma_scan<I8Op>(queries, B, items, N, D, k, mask, mask_words, out_ids, out_scores,
                             workspace, workspace_bytes, stream);
}

// ---- allocation-free int8 scan ------------------------------------------------------------
//
// Scratch of rt_int8_scan_topk_noalloc: the candidate lists, their lengths and the seed bounds
// (the workspace of rt_int8_scan_topk) in a file-scope device array. Each GPU the library runs
// on holds its own copy until the process ends. The main pass splits a fixed number of
// workgroups (two per CU) over the 16-query groups, so the lists hardly grow with the batch:
// on a 256-CU part they take 64 MiB at k <= 224 and 128 MiB at k <= 480, and 160 MiB holds
// the plan of up to 8192 queries at k <= 224 and 4096 at k <= 480; nothing in it needs clearing
// (every list length, list entry read and bound is written by the call before it is read).
constexpr size_t kNoAllocScratchBytes = size_t{160} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kNoAllocMaxDevices = 64;
std::once_flag g_scratch_once[kNoAllocMaxDevices];
void* g_scratch_ptr[kNoAllocMaxDevices];
hipError_t g_scratch_status[kNoAllocMaxDevices];

// The device address of the current GPU's copy of `scratch`, looked up once per device (with
// that device current, on its first call). Host code uses only this address: the array's name is
// a host-side stand-in.
int noalloc_scratch(void** out) {
  int dev = 0;
  RT_CHECK_HIP(hipGetDevice(&dev));
  RT_CHECK_ARG(dev >= 0 && dev < kNoAllocMaxDevices, "device %d: the allocation-free entry "
               "point supports devices 0-%d", dev, kNoAllocMaxDevices - 1);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = p;
  });
  if (g_scratch_status[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr) {
    set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
              hipGetErrorString(g_scratch_status[dev]));
    return kLaunchFailed;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

}  // namespace

extern "C" int rt_int8_scan_topk_noalloc(const int8_t* queries, int64_t B, const int8_t* items,
                                         int64_t N, int64_t D, int64_t k, const uint64_t* mask,
                                         int64_t mask_words, int64_t* out_ids,
                                         int32_t* out_scores, hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(B == 0 || (out_ids != nullptr && out_scores != nullptr &&
                          (N == 0 || (queries != nullptr && items != nullptr))),
               "queries, items, out_ids and out_scores must not be null");
  const size_t need = mfma_plan(B, N, k, main_workgroups())
                          .total;
  RT_CHECK_ARG(need <= kNoAllocScratchBytes,
               "rt_int8_scan_topk_noalloc: B = %lld, N = %lld, k = %lld need %zu bytes of "
               "scratch, above its fixed %zu bytes (call rt_int8_scan_topk with a workspace)",
               static_cast<long long>(B), static_cast<long long>(N), static_cast<long long>(k),
               need, kNoAllocScratchBytes);
  void* ws = nullptr;
  const int st = noalloc_scratch(&ws);
  if (st != kOk) return st;
  return run_mfma_scan<I8Op>(queries, B, items, N, D, k, mask, mask_words, out_ids, out_scores,
                             ws, kNoAllocScratchBytes, stream);
}

// ---- scans with the exact clause filter tested per candidate --------------------------------

static size_t mfma_plan_bytes(int64_t B, int64_t N, int64_t k) {
  return mfma_plan(B, N, k, kMaxResidentWorkgroups)
      .total;
}

extern "C" size_t rt_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t D, int64_t k,
                                                 int64_t C, int64_t V) {
  (void)D;
  if (k < 1 || k > kMaxK || B < 0 || N < 0) return 256;
  return align_up(mfma_plan_bytes(B, N, k), 256) + clause_prep_workspace(B, C, V);
}

// The clause scans' shared body: rt_scan_topk_clauses (mask) and rt_scan_topk_bloom_clauses
// (Bloom probe).
static int scan_clauses(const void* queries, int64_t B, const void* items, int64_t N, int64_t D,
                        int64_t k, int dtype, const uint64_t* mask, int64_t mask_words,
                        const BloomProbe& probe, const void* item_attrs, int attr_bytes,
                        int64_t C, int64_t A, const int8_t* clause_is_reverse,
                        const int64_t* query_values, int64_t V, int64_t* out_ids,
                        void* out_scores, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  RT_CHECK_ARG(dtype >= 0 && dtype <= 2, "dtype must be 0 (int8), 1 (bf16) or 2 (fp16), got %d",
               dtype);
  RT_CHECK_ARG(B >= 0 && N >= 0 && k >= 1 && k <= kMaxK, "B, N >= 0 and k in [1, %lld]",
               static_cast<long long>(kMaxK));
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(C));
  RT_CHECK_ARG(A >= 0 && A <= 4096 && V >= 1 && V <= 4096, "A must be in [0, 4096] and V in "
               "[1, 4096]");
  RT_CHECK_ARG(attr_bytes == 2 || attr_bytes == 4 || attr_bytes == 8,
               "attr_bytes must be 2, 4 or 8 (int16, int32, int64 attributes)");
  RT_CHECK_ARG(B <= (int64_t{1} << 21), "B must be <= 2^21 query rows");
  if (B == 0) return kOk;
  RT_CHECK_ARG(C == 0 || (clause_is_reverse != nullptr && query_values != nullptr),
               "clause_is_reverse and query values must not be null");
  RT_CHECK_ARG(C * A == 0 || N == 0 || item_attrs != nullptr, "item attrs are null");
  const size_t scan_bytes = align_up(mfma_plan_bytes(B, N, k), 256);
  const size_t need = scan_bytes + clause_prep_workspace(B, C, V);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  ClauseCheck f;
  if (C > 0 && N > 0) {
    const int st = clause_prepare(query_values, B, C, V, clause_is_reverse,
                                  static_cast<char*>(workspace) + scan_bytes,
                                  workspace_bytes - scan_bytes, &f, stream);
    if (st != kOk) return st;
    f.attrs = item_attrs;
    f.attr_bytes = attr_bytes;
    f.A = static_cast<int>(A);
    f.held = attr_rows_held(item_attrs, attr_bytes, C, A);
  }
  if (dtype == 0) {
    return run_mfma_scan<I8Op>(queries, B, items, N, D, k, mask, mask_words, out_ids,
                               out_scores, workspace, scan_bytes, stream, f, probe);
  }
  if (dtype == 1) {
    return run_mfma_scan<BF16Op>(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                                 out_scores, workspace, scan_bytes, stream, f, probe);
  }
  return run_mfma_scan<F16Op>(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                              out_scores, workspace, scan_bytes, stream, f, probe);
}

extern "C" int rt_scan_topk_clauses(const void* queries, int64_t B, const void* items, int64_t N,
                                    int64_t D, int64_t k, int dtype, const uint64_t* mask,
                                    int64_t mask_words, const void* item_attrs, int attr_bytes,
                                    int64_t C, int64_t A, const int8_t* clause_is_reverse,
                                    const int64_t* query_values, int64_t V, int64_t* out_ids,
                                    void* out_scores, void* workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  return scan_clauses(queries, B, items, N, D, k, dtype, mask, mask_words, BloomProbe{},
                      item_attrs, attr_bytes, C, A, clause_is_reverse, query_values, V, out_ids,
                      out_scores, workspace, workspace_bytes, stream);
}

extern "C" int rt_scan_topk_bloom_clauses(
    const void* queries, int64_t B, const void* items, int64_t N, int64_t D, int64_t k,
    int dtype, const uint64_t* doc_bits, const uint64_t* probe_tables, int64_t plan_count,
    const void* item_attrs, int attr_bytes, int64_t C, int64_t A,
    const int8_t* clause_is_reverse, const int64_t* query_values, int64_t V, int64_t* out_ids,
    void* out_scores, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(plan_count == B, "one Bloom plan per query: plan_count %lld != B %lld",
               static_cast<long long>(plan_count), static_cast<long long>(B));
  RT_CHECK_ARG(N == 0 || B == 0 || (doc_bits != nullptr && probe_tables != nullptr),
               "doc_bits and probe_tables must not be null");
  BloomProbe probe;
  probe.doc_bits = doc_bits;
  probe.tables = probe_tables;
  return scan_clauses(queries, B, items, N, D, k, dtype, nullptr, 0, probe, item_attrs,
                      attr_bytes, C, A, clause_is_reverse, query_values, V, out_ids, out_scores,
                      workspace, workspace_bytes, stream);
}

extern "C" size_t rt_dense_scan_topk_workspace(int64_t B, int64_t N, int64_t D, int64_t k) {
  (void)D;
  return mfma_plan(B, N, k, kMaxResidentWorkgroups)
      .total;
}

extern "C" int rt_dense_scan_topk(const void* queries, int64_t B, const void* items, int64_t N,
                                  int64_t D, int64_t k, int dtype, const uint64_t* mask,
                                  int64_t mask_words, int64_t* out_ids, float* out_scores,
                                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (dtype == 0) {
    return run_mfma_scan<BF16Op>(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                                 out_scores, workspace, workspace_bytes, stream);
  }
  if (dtype == 1) {
    return run_mfma_scan<F16Op>(queries, B, items, N, 2 * D, k, mask, mask_words, out_ids,
                                out_scores, workspace, workspace_bytes, stream);
  }
  set_error("dense scan dtype must be 0 (bf16) or 1 (fp16), got %d", dtype);
  return kInvalidType;
}
