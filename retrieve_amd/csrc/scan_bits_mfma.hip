// 1-bit Hamming top-k of small batches over 512-bit codes on the fp4 matrix cores, one wave per
// stream of tiles (v_mfma_scale_f32_16x16x128_f8f6f4, e2m1 operands; the nibble layout and the
// scaled, biased accumulators of bits_fp4.h). Scores 512 - 2 popcount(q ^ x), exact; ties to the
// lower item index.
//
// A 16-row group of codes is 1 KiB: lane l loads the 16 bytes [16 (l / 16), +16) of row l % 16,
// so each wave-wide load is one contiguous 1 KiB and lands in MFMA order -- no LDS staging and
// no workgroup barriers. MFMA step s (s < 4) takes dword s of each lane's 16 bytes as its 32 K
// elements (items as the A operand, rows l % 16); the query operand holds the same dwords of
// query l % 16's code (the K order inside an operand is free when both sides share it). After
// the four steps lane l holds the sums of query l % 16 for rows 4 (l / 16) + r, r < 4, of the
// group (the layout of the int8 scan's 16x16 tiles).
//
// Each wave scores up to four 16-query groups (NQ) against every group of rows it reads, so the
// expansion of a row word (five VALU per 32 bits) feeds NQ MFMAs. A wave streams 128-row tiles
// (8 KiB, one 16-byte load per lane per group; 64-row tiles for two or three query groups where
// three workgroups fit a CU) dealt round-robin over every wave of the grid, with two or three
// tiles in registers: the one being scored and the others in flight. The hit test is one
// signed-int maximum of the four raw accumulator bits per query group against the threshold in
// the same domain; candidates (composites >= the query's bound, passing the mask) are appended
// to per-wave lists and compacted as in every scan (wave_lists.h).
#include "bits_fp4.h"
#include "profile.h"
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kCodeBytes = 64;                        // a 512-bit code
constexpr int kGroupRows = 16;                        // rows of one MFMA
constexpr int kTileGroups = 8;                        // row groups of a main-pass tile
constexpr int kTileRows = kGroupRows * kTileGroups;  // 128 rows, 8 KiB
constexpr int kMaxQGroups = 4;                        // 16-query groups of a wave
// Two or three query groups whose lists leave room for three workgroups a CU: 64-row tiles (four
// groups), so the kernel fits three waves a SIMD (168 VGPRs at three groups; four spill);
// B = 17-32 0.343-0.353 -> 0.335-0.348 ms a call.
constexpr int kTileGroupsSmall = 4;
constexpr int kWavesSmall = 3;
constexpr size_t kLdsPerCU = 160 * 1024;
// Word 3 of a raw buffer descriptor (stride 0, byte offsets; out-of-range loads return zeros),
// and the cache-policy bits of a streamed load (nontemporal).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kNontemporal = 2;

// One MFMA step of output tile p (query group p of the wave): items x query, the query operand
// at the scale of tile p (fp4::hit_scale). The fp4 form reads the low four registers of each
// operand.
__device__ inline v4f bits_mma(v4i a, v4i b, v4f c, int p) {
  const v8i a8 = __builtin_shufflevector(a, a, 0, 1, 2, 3, 0, 1, 2, 3);
  const v8i b8 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 0, 1, 2, 3);
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, c, fp4::kFmt, fp4::kFmt, 0,
                                                         fp4::kUnitScale, 0, fp4::hit_scale(p));
}

__device__ inline int32_t raw_bits(float v) { return __builtin_bit_cast(int32_t, v); }
__device__ inline int32_t imax(int32_t a, int32_t b) { return a > b ? a : b; }

// Calls f(std::integral_constant<int, i>) for i < N (constant indices into register arrays).
template <int I, int N, class F>
__device__ inline void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// A 16-row group's item operands: this lane's 16 bytes x of its row, dword s as step s's.
struct GroupOps {
  v4i xs[4];
};
__device__ inline GroupOps expand(const v4i x) {
  GroupOps o;
#pragma unroll
  for (int s = 0; s < 4; ++s) o.xs[s] = fp4::item_frag(static_cast<uint32_t>(x[s]));
  return o;
}

// The group's sums against the wave's NQ query groups: acc[j] holds query 16 j + l % 16's
// values for rows 4 (l / 16) + r, r < 4.
template <int NQ>
__device__ inline void group_sums(const GroupOps& o, const v4i (&qf)[NQ][4], v4f (&acc)[NQ]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const float b = fp4::hit_bias(j);
      acc[j] = bits_mma(o.xs[s], qf[j][s], s == 0 ? v4f{b, b, b, b} : acc[j], j);
    }
  }
}

// This lane's query of each group: the operand fragments (dwords 4 (l / 16) + s of its code),
// the start 512 - 2 popcount(q), and its mask row (null without a mask or for padding).
template <int NQ>
struct BitsQueries {
  v4i qf[NQ][4];
  int32_t acc0[NQ];
  const uint64_t* qmask[NQ];
  __device__ void load(const ScanArgs& a, int64_t q0, int col, int grp) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int64_t q = q0 + 16 * j + col;
      if (q < a.B) {
        const uint32_t* qw =
            reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(a.queries) +
                                              q * kCodeBytes);
#pragma unroll
        for (int s = 0; s < 4; ++s) qf[j][s] = fp4::query_frag(qw[4 * grp + s]);
        int pc = 0;
#pragma unroll
        for (int w = 0; w < kCodeBytes / 4; ++w) pc += __builtin_popcount(qw[w]);
        acc0[j] = 8 * kCodeBytes - 2 * pc;
        qmask[j] = a.mask != nullptr ? a.mask + q * a.mask_words : nullptr;
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) qf[j][s] = v4i{0, 0, 0, 0};
        acc0[j] = 0;
        qmask[j] = nullptr;
      }
    }
  }
};

// Seed pass over the strided sample: per query, each wave's best composite over its rows,
// written to a.lists[q * S + wave index] (S = waves of the grid row). The sample is cut into
// chunks of kTileRows rows from row 0 (a sample block of kSeedBlock consecutive items holds
// whole chunks); a workgroup's waves take the parts of the chunks within its strip (a multiple
// of 16 rows from a multiple of 16) in turn, every load of a part issued before its sums. With
// strips of 512 rows: 1024 lists a query from the default 2^17 sampled rows, few to merge, and
// far more than the rank whose best the merge takes.
template <int NQ>
__global__ void __launch_bounds__(kScanThreads) bits_seed_kernel(ScanArgs a) {
  constexpr int QPW = 16 * NQ;
  static_assert(kSeedBlock % kTileRows == 0, "sample blocks hold whole chunks");
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * QPW;
  BitsQueries<NQ> qs;
  qs.load(a, q0, col, grp);
  const int8_t* I = static_cast<const int8_t*>(a.items);
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * a.strip;
  const int64_t s1 = s0 + a.strip < a.n_rows ? s0 + a.strip : a.n_rows;
  uint64_t best[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) best[j] = 0ull;
  const int64_t c1 = s1 > s0 ? (s1 - 1) / kTileRows : -1;  // the strip's last chunk
  for (int64_t c = s0 / kTileRows + wave; c <= c1; c += kScanWaves) {
    const int64_t r0 = c * kTileRows > s0 ? c * kTileRows : s0;
    const int64_t r1 = c * kTileRows + kTileRows < s1 ? c * kTileRows + kTileRows : s1;
    // the part's rows are consecutive items from sample_item(r0): one descriptor, rows past
    // r1 read as zeros and are never kept
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(I + sample_item(r0, a.row_stride) * kCodeBytes), 0,
        static_cast<int>((r1 - r0) * kCodeBytes), kBufferWord3);
    v4i x[kTileGroups];
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) {
      x[g] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(
                   rs, col * kCodeBytes + grp * 16 + g * kGroupRows * kCodeBytes, 0, 0));
    }
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) {
      if (r0 + g * kGroupRows >= r1) break;  // (uniform)
      v4f acc[NQ];
      group_sums<NQ>(expand(x[g]), qs.qf, acc);
      const int64_t row0 = r0 + g * kGroupRows + 4 * grp;  // this lane's rows row0 + r
      const int64_t item0 = sample_item(r0, a.row_stride) + (row0 - r0);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        // rows from a multiple of 4: items item0 + r share one mask word
        const uint64_t w =
            qs.qmask[j] != nullptr && row0 < r1 ? qs.qmask[j][item0 >> 6] : ~0ull;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint64_t c = composite(key_of_i32(fp4::hit_score(acc[j][r], qs.acc0[j], j)),
                                       static_cast<uint32_t>(item0 + r));
          const bool ok = row0 + r < r1 && ((w >> (63 - ((item0 + r) & 63))) & 1ull) != 0ull;
          best[j] = ok && c > best[j] ? c : best[j];
        }
      }
    }
  }
  const int64_t S = static_cast<int64_t>(gridDim.x) * kScanWaves;
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    uint64_t o = __shfl_xor(best[j], 16);
    best[j] = o > best[j] ? o : best[j];
    o = __shfl_xor(best[j], 32);
    best[j] = o > best[j] ? o : best[j];
    const int64_t q = q0 + 16 * j + col;
    if (lane < 16 && q < a.B) {
      a.lists[q * S + static_cast<int64_t>(blockIdx.x) * kScanWaves + wave] = best[j];
    }
  }
}

// Main pass: every item, candidate lists per (wave, query). List of query 16 j + c of this
// wave's group row: lists[(slot * QPW + 16 j + c) * capw], its length cnt[16 j + c] (LDS).
template <int NQ, int TG = kTileGroups>
__global__ void __launch_bounds__(kScanThreads)
    __attribute__((amdgpu_waves_per_eu(TG == kTileGroupsSmall ? kWavesSmall : 2)))
    bits_scan_kernel(ScanArgs a) {
  if (a.run_if != nullptr && *a.run_if == 0u) return;  // (uniform: the fallback is not needed)
  constexpr int QPW = 16 * NQ;
  constexpr int TR = kGroupRows * TG;  // rows of a tile
  extern __shared__ __attribute__((aligned(16))) uint64_t smem[];
  const int lane = lane_id();
  // wave-uniform, so the tile indices and buffer descriptors derived from it live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int capw = a.capw;
  uint64_t* scratch = smem + wave * capw;
  int* cnt = reinterpret_cast<int*>(smem + kScanWaves * capw) + wave * QPW;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kScanWaves;
  const int64_t wave_in_row = static_cast<int64_t>(blockIdx.x) * kScanWaves + wave;
  const int64_t slot = static_cast<int64_t>(blockIdx.y) * waves + wave_in_row;
  for (int i = lane; i < QPW; i += kWave) cnt[i] = 0;
  uint64_t* lists = a.lists + slot * QPW * static_cast<int64_t>(capw);

  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * QPW;
  BitsQueries<NQ> qs;
  qs.load(a, q0, col, grp);
  // per query group: the bound (composite), its score part, and the hit threshold
  uint64_t tau[NQ];
  int32_t ts[NQ];
  int32_t thr[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int64_t q = q0 + 16 * j + col;
    tau[j] = q < a.B ? (a.tau_in != nullptr ? a.tau_in[q] : 0ull) : ~0ull;
    ts[j] = i32_of_key(composite_key(tau[j]));
    thr[j] = fp4::hit_thresh(ts[j], qs.acc0[j], j);
  }
  wave_sync_memory();

  const int64_t n = a.n_rows;
  const int k = a.k;
  // Query group j's candidates among rows row0 + r (r < 4) of this lane: appended when their
  // composite reaches the bound and they pass the mask; lists that could overflow on the next
  // group are compacted, raising the bound to their k-th best.
  auto push = [&](auto jc, const v4f& v, int64_t row0) {
    constexpr int j = decltype(jc)::value;
    uint64_t cs[4];
    uint32_t cand = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t sc = fp4::hit_score(v[r], qs.acc0[j], j);
      cs[r] = composite(key_of_i32(sc), static_cast<uint32_t>(row0 + r));
      cand |= row0 + r < n && sc >= ts[j] && cs[r] >= tau[j] ? 1u << r : 0u;
    }
    if (qs.qmask[j] != nullptr && cand != 0u) {
      const uint64_t w = qs.qmask[j][row0 >> 6];  // (row0 is a multiple of 4: one word)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        cand &= (w >> (63 - ((row0 + r) & 63))) & 1ull ? ~0u : ~(1u << r);
      }
    }
    int* c_mine = &cnt[16 * j + col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if ((cand >> r) & 1u) {
        const int pos = atomicAdd(c_mine, 1);
        lists[(16 * j + col) * static_cast<int64_t>(capw) + pos] = cs[r];
      }
    }
    // the lengths after every lane's appends: the wave's LDS atomics done (lgkmcnt(0)); not a
    // memory fence, which would also wait for the tiles in flight (wave_compact fences before
    // it reads the lists back)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    uint64_t need = __ballot(*c_mine > capw - kGroupRows) & 0xffffull;
    while (need != 0ull) {
      const int c = __builtin_ctzll(need);
      need &= need - 1;
      const uint64_t nt = wave_compact(lists + (16 * j + c) * static_cast<int64_t>(capw),
                                       &cnt[16 * j + c], scratch, capw, k);
      if (col == c && nt > tau[j]) {
        tau[j] = nt;
        ts[j] = i32_of_key(composite_key(nt));
        thr[j] = fp4::hit_thresh(ts[j], qs.acc0[j], j);
      }
    }
  };
  const int8_t* I = static_cast<const int8_t*>(a.items);
  const int loff = col * kCodeBytes + grp * 16;  // this lane's bytes in a 16-row group
  // One buffer descriptor per tile (base = its first row, range = its rows present: rows past
  // the end read as zeros and are never kept; a tile past the table has range 0 and reads no
  // memory), so a lane's offsets are 32-bit constants and every load is issued unconditionally:
  // the waits before each group then count exactly the loads issued after it.
  auto load = [&](int64_t tt, v4i(&v)[TG]) {
    const int64_t rt = tt * TR;
    const int64_t left = rt < n ? (n - rt) * kCodeBytes : 0;
    const int range = static_cast<int>(left < TR * kCodeBytes ? left : TR * kCodeBytes);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(I + rt * kCodeBytes), 0, range, kBufferWord3);
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      v[g] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, loff + g * kGroupRows * kCodeBytes, 0,
                                                     kNontemporal));
    }
  };
  // the hit test of 16-row group g of tile t (the group's sums acc), then its candidates
  auto test = [&](int64_t t, int g, const v4f (&acc)[NQ]) {
    const int64_t row0 = t * TR + g * kGroupRows + 4 * grp;
    bool hit[NQ];
    bool any = false;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int32_t m = imax(imax(raw_bits(acc[j][0]), raw_bits(acc[j][1])),
                             imax(raw_bits(acc[j][2]), raw_bits(acc[j][3])));
      hit[j] = m >= thr[j];
      any = any || hit[j];
    }
    if (__any(any)) {
      static_for<0, NQ>([&](auto jc) {
        if (__any(hit[decltype(jc)::value])) push(jc, acc[decltype(jc)::value], row0);
      });
    }
  };

  // NB tiles in registers (three for one query group, two above, which keeps two waves a SIMD
  // without spills): the one being scored and the others in flight. Each group's registers are reloaded
  // with the same group of the tile NB ahead as soon as the group's operands are expanded, so
  // close to NB tiles stay in flight; the scheduling barriers keep each reload where it is.
  constexpr int NB = NQ <= 1 ? 3 : 2;
  const int64_t ntiles = cdiv(n, TR);
  v4i v0[TG], v1[TG], v2[TG];
  int64_t t = wave_in_row;
  load(t, v0);
  load(t + waves, v1);
  if constexpr (NB == 3) load(t + 2 * waves, v2);
  auto step = [&](int64_t tt, v4i(&v)[TG]) {
    // tile tt from v, v refilled with tile tt + NB waves
    const int64_t rn = (tt + NB * waves) * TR;
    const int64_t left = rn < n ? (n - rn) * kCodeBytes : 0;
    const int range = static_cast<int>(left < TR * kCodeBytes ? left : TR * kCodeBytes);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(I + rn * kCodeBytes), 0, range, kBufferWord3);
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      // the group's operands first, so its registers are free for the refill (no copies of a
      // load still in flight)
      const GroupOps ops = expand(v[g]);
      __builtin_amdgcn_sched_barrier(0);
      v[g] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, loff + g * kGroupRows * kCodeBytes, 0,
                                                     kNontemporal));
      __builtin_amdgcn_sched_barrier(0);
      v4f acc[NQ];
      group_sums<NQ>(ops, qs.qf, acc);
      test(tt, g, acc);
    }
  };
  for (; t < ntiles; t += NB * waves) {
    step(t, v0);
    if (t + waves >= ntiles) break;
    step(t + waves, v1);
    if constexpr (NB == 3) {
      if (t + 2 * waves >= ntiles) break;
      step(t + 2 * waves, v2);
    }
  }
  wave_sync_memory();
  static_assert(QPW <= kWave, "a lane per list length");
  if (lane < QPW) a.counts[slot * QPW + lane] = cnt[lane];
}

// List capacity: k plus room for the next group's appends (at most 16 a query), a power of two.
int bits_capw(int64_t k) { return static_cast<int>(next_pow2(k + 2 * kGroupRows)); }

// 16-query groups a wave scores: all of the batch up to kMaxQGroups.
int bits_qgroups(int64_t B) {
  const int64_t g = cdiv(B, 16);
  return static_cast<int>(g < kMaxQGroups ? g : kMaxQGroups);
}

ScanPlan bits_plan(int64_t B, int64_t N, int64_t k, int64_t target_wgs) {
  const int64_t qpg = 16 * bits_qgroups(B);
  return plan_scan(B, N, k, qpg, kScanWaves * qpg, target_wgs, bits_capw(k),
                   kScanWaves * kTileRows, kSeedRows / 2);
}

// LDS of a main-pass workgroup: each wave's compaction scratch and list lengths.
size_t bits_main_lds(int capw, int nq) {
  return kScanWaves * (static_cast<size_t>(capw) * sizeof(uint64_t) + 16 * nq * sizeof(int));
}

// The 64-row-tile form: two or three query groups whose lists leave room for three
// workgroups a CU.
bool bits_small_tiles(int nq, int capw) {
  return (nq == 2 || nq == 3) && kWavesSmall * bits_main_lds(capw, nq) <= kLdsPerCU;
}

template <int NQ, int TG>
int launch_main(const ScanArgs& a, const dim3 grid, size_t lds, hipStream_t stream) {
  if (lds > 65536) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(bits_scan_kernel<NQ, TG>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  bits_scan_kernel<NQ, TG><<<grid, kScanThreads, lds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

template <int NQ>
int launch_bits(const ScanArgs& a, const PassPlan& p, int64_t nqg, bool seed,
                hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.gx), static_cast<unsigned>(nqg));
  if (seed) {
    bits_seed_kernel<NQ><<<grid, kScanThreads, 0, stream>>>(a);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  const size_t lds = bits_main_lds(p.capw, NQ);
  if constexpr (NQ == 2 || NQ == 3) {
    if (bits_small_tiles(NQ, p.capw)) return launch_main<NQ, kTileGroupsSmall>(a, grid, lds, stream);
  }
  return launch_main<NQ, kTileGroups>(a, grid, lds, stream);
}

int dispatch_bits(int nq, const ScanArgs& a, const PassPlan& p, int64_t nqg, bool seed,
                  hipStream_t stream) {
  switch (nq) {
    case 1: return launch_bits<1>(a, p, nqg, seed, stream);
    case 2: return launch_bits<2>(a, p, nqg, seed, stream);
    case 3: return launch_bits<3>(a, p, nqg, seed, stream);
    default: return launch_bits<4>(a, p, nqg, seed, stream);
  }
}

}  // namespace

size_t bits_mfma_workspace(int64_t B, int64_t N, int64_t k) {
  return bits_plan(B > 0 ? B : 1, N, k, kMaxResidentWorkgroups).total;
}

// seed scan → rank-th bound merge → main scan → final merge (→ fallback scan and merge while
// the flag is set), on `stream`, no host sync. The seed's bound is its sample's rank-th best
// (sample_rank), not its k-th: the main pass then keeps about rank * stride candidates a query
// instead of k * stride. A query that ends with fewer than k entries behind a bound above 0
// raises the flag, and the fallback main pass and merge without the bound (both returning at
// once while the flag is clear) keep the results exact.
int bits_mfma(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
              int64_t k, const uint64_t* mask, int64_t mask_words, int64_t* out_ids,
              void* out_scores, int score_kind, void* workspace, size_t workspace_bytes,
              hipStream_t stream) {
  RT_CHECK_ARG(B >= 1 && N >= 1 && k >= 1 && k <= kMaxK, "bits_mfma: B, N >= 1, k in [1, %lld]",
               static_cast<long long>(kMaxK));
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(query_bits) % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(item_bits) % 16 == 0,
               "query_bits must be 4-byte and item_bits 16-byte aligned");
  const int nq = bits_qgroups(B);
  // (the 64-row-tile form: three workgroups a CU, its occupancy)
  const bool small_tiles = bits_small_tiles(nq, bits_capw(k));
  const ScanPlan plan =
      bits_plan(B, N, k, small_tiles ? main_workgroups() * kWavesSmall / 2 : main_workgroups());
  if (workspace_bytes < plan.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, plan.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* lists = reinterpret_cast<uint64_t*>(ws + plan.off_lists);
  int* counts = reinterpret_cast<int*>(ws + plan.off_counts);
  uint64_t* tau = reinterpret_cast<uint64_t*>(ws + plan.off_tau);
  uint32_t* spec_flag = reinterpret_cast<uint32_t*>(ws + plan.off_flag);
  const int rank = plan.seeded ? sample_rank(k, plan.seed.row_stride) : static_cast<int>(k);
  const bool speculative = plan.seeded && rank < k;

  ScanArgs a{};
  a.queries = query_bits;
  a.B = B;
  a.items = item_bits;
  a.k = static_cast<int>(k);
  a.qpw = static_cast<int>(plan.qpg);
  a.mask = mask;
  a.mask_words = mask_words;
  a.lists = lists;
  a.counts = counts;

  MergeArgs m{};
  m.lists = lists;
  m.counts = counts;
  m.qpw = static_cast<int>(plan.qpg);
  m.B = B;
  m.k = static_cast<int>(k);

  if (plan.seeded) {
    a.n_rows = plan.seed.n_rows;
    a.row_stride = plan.seed.row_stride;
    a.strip = plan.seed.strip;
    a.capw = 1;
    a.tau_in = nullptr;
    int st = dispatch_bits(nq, a, plan.seed, plan.n_qgroups, true, stream);
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
  a.n_rows = N;
  a.row_stride = 1;
  a.strip = plan.main.strip;
  a.capw = plan.main.capw;
  a.tau_in = plan.seeded ? tau : nullptr;
  // the final merge over the main pass's lists split into parts (small batches); the seed's
  // flat merge above is one launch (its 1024 one-entry lists a query merge faster whole)
  m.part_buf = plan.split ? reinterpret_cast<uint64_t*>(ws + plan.off_parts) : nullptr;
  hipEvent_t stop;
  profile_begin(stream, &stop);
  int st = dispatch_bits(nq, a, plan.main, plan.n_qgroups, false, stream);
  profile_end(stream, stop);
  if (st != kOk) return st;
  m.capw = plan.main.capw;
  m.S = plan.main.S;
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = score_kind;
  if (speculative) {
    m.spec_flag = spec_flag;
    m.spec_tau = tau;
    m.safe_tau = nullptr;
  }
  st = launch_merge(m, stream);
  if (st != kOk || !speculative) return st;
  a.tau_in = nullptr;
  a.run_if = spec_flag;
  st = dispatch_bits(nq, a, plan.main, plan.n_qgroups, false, stream);
  if (st != kOk) return st;
  m.spec_flag = nullptr;
  m.run_if = spec_flag;
  m.part_buf = nullptr;  // (one launch: it returns at once while the flag is clear)
  return launch_merge(m, stream);
}

}  // namespace rt
