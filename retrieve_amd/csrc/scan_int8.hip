// int8 × int8 → int32 full scan with the exact fused top-k (SilverTorch's int8 scorer
// semantics: int32 accumulation, ties to the lower item index).
//
// Each wave multiplies 16-item tiles of the item table against its 16 queries with
// v_mfma_i32_16x16x64_i8 (items as the A operand, queries as B), so after a tile lane l holds
// the scores of query l % 16 for items 4 * (l / 16) + r, r < 4. The K order inside an
// operand is free (integer sums are exact): lane l feeds bytes [64 s + 16 (l / 16), +16) of
// its item row and of its query row at step s, the same bytes on both sides.
#include "profile.h"
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));

// SEED: the sample pass. Instead of candidate lists each wave keeps, per query, only its best
// composite over its rows and writes it as a one-entry list (a.capw == 1); the k-th largest of
// those maxima is a lower bound on the k-th best item (k distinct waves each hold an item at
// least that good).
template <int KSTEPS, bool SEED>
__global__ void __launch_bounds__(kScanThreads) scan_int8_kernel(ScanArgs a) {
  constexpr int QPW = 16;
  constexpr int64_t D = KSTEPS * 64;
  extern __shared__ uint64_t smem[];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  uint64_t* scratch = smem + wave * a.capw;
  int* cnt = reinterpret_cast<int*>(smem + kScanWaves * a.capw) + wave * QPW;
  const int64_t slot = (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * kScanWaves +
                       wave;
  uint64_t* lists = a.lists + slot * QPW * a.capw;
  if constexpr (!SEED) {
    if (lane < QPW) cnt[lane] = 0;
  }

  const int8_t* Q = static_cast<const int8_t*>(a.queries);
  const int8_t* I = static_cast<const int8_t*>(a.items);
  const int64_t qrow = static_cast<int64_t>(blockIdx.y) * QPW + col;
  v4i qf[KSTEPS];
  uint64_t tau = ~0ull;  // padding query columns never pass
  if (qrow < a.B) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      qf[s] = *reinterpret_cast<const v4i*>(Q + qrow * D + s * 64 + grp * 16);
    }
    tau = a.tau_in != nullptr ? a.tau_in[qrow] : 0ull;
  } else {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qf[s] = v4i{0, 0, 0, 0};
  }
  int32_t ts = i32_of_key(composite_key(tau));
  const uint64_t* qmask =
      a.mask != nullptr && qrow < a.B ? a.mask + qrow * a.mask_words : nullptr;
  wave_sync_memory();

  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * a.strip;
  const int64_t r1 = r0 + a.strip < a.n_rows ? r0 + a.strip : a.n_rows;
  const int64_t ntiles = r1 > r0 ? cdiv(r1 - r0, kTile) : 0;

  uint64_t best = 0ull;  // SEED only
  for (int64_t t = wave; t < ntiles; t += kScanWaves) {
    const int64_t rb = r0 + t * kTile;
    int64_t lr = rb + col;
    lr = lr < r1 ? lr : r1 - 1;
    const int8_t* ip = I + lr * a.row_stride * D + grp * 16;
    v4i af[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) af[s] = *reinterpret_cast<const v4i*>(ip + s * 64);
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[s], qf[s], acc, 0, 0, 0);
    }
    if constexpr (SEED) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = rb + 4 * grp + r;
        const uint32_t item = static_cast<uint32_t>(row * a.row_stride);
        bool ok = row < r1;
        if (ok && qmask != nullptr) ok = (qmask[item >> 6] >> (63 - (item & 63))) & 1ull;
        const uint64_t c = composite(key_of_i32(acc[r]), item);
        best = ok && c > best ? c : best;
      }
      continue;
    }
    const bool hit = acc[0] >= ts || acc[1] >= ts || acc[2] >= ts || acc[3] >= ts;
    if (!__any(hit)) continue;

    // slow path: exact composite test, filter bit, append
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = rb + 4 * grp + r;
      if (row < r1 && acc[r] >= ts) {
        const uint32_t item = static_cast<uint32_t>(row * a.row_stride);
        const uint64_t c = composite(key_of_i32(acc[r]), item);
        bool keep = c >= tau;
        if (keep && qmask != nullptr) {
          keep = (qmask[item >> 6] >> (63 - (item & 63))) & 1ull;
        }
        if (keep) {
          const int pos = atomicAdd(&cnt[col], 1);
          lists[col * a.capw + pos] = c;
        }
      }
    }
    wave_sync_memory();
    const bool full = cnt[col] > a.capw - kTile;
    uint64_t need = __ballot(full) & 0xffffull;
    while (need != 0ull) {
      const int c = __builtin_ctzll(need);
      need &= need - 1;
      const uint64_t nt = wave_compact(lists + c * a.capw, &cnt[c], scratch, a.capw, a.k);
      if (col == c && nt > tau) {
        tau = nt;
        ts = i32_of_key(composite_key(nt));
      }
    }
  }
  if constexpr (SEED) {
    uint64_t o = __shfl_xor(best, 16);
    best = o > best ? o : best;
    o = __shfl_xor(best, 32);
    best = o > best ? o : best;
    if (lane < QPW) lists[lane] = best;
    return;
  }
  wave_sync_memory();
  if (lane < QPW) a.counts[slot * QPW + lane] = cnt[lane];
}

template <int KSTEPS>
static int launch_scan_int8(const ScanArgs& a, const PassPlan& p, int64_t n_qgroups, bool seed,
                            hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.gx), static_cast<unsigned>(n_qgroups));
  if (seed) {
    scan_int8_kernel<KSTEPS, true><<<grid, kScanThreads, 0, stream>>>(a);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  const size_t lds = kScanWaves * (p.capw * sizeof(uint64_t) + 16 * sizeof(int));
  if (lds > 65536) {
    RT_CHECK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void*>(scan_int8_kernel<KSTEPS, false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  }
  scan_int8_kernel<KSTEPS, false><<<grid, kScanThreads, lds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

static int dispatch_scan_int8(int64_t D, const ScanArgs& a, const PassPlan& p, int64_t nqg,
                              bool seed, hipStream_t stream) {
  switch (D) {
    case 64: return launch_scan_int8<1>(a, p, nqg, seed, stream);
    case 128: return launch_scan_int8<2>(a, p, nqg, seed, stream);
    case 256: return launch_scan_int8<4>(a, p, nqg, seed, stream);
    case 512: return launch_scan_int8<8>(a, p, nqg, seed, stream);
    case 768: return launch_scan_int8<12>(a, p, nqg, seed, stream);
    case 1024: return launch_scan_int8<16>(a, p, nqg, seed, stream);
    default:
      set_error("int8 scan supports D in {64, 128, 256, 512, 768, 1024}, got %lld",
                static_cast<long long>(D));
      return kInvalidArgument;
  }
}

}  // namespace rt

using namespace rt;

extern "C" size_t rt_int8_scan_topk_workspace(int64_t B, int64_t N, int64_t D, int64_t k) {
  (void)D;
  return plan_scan(B, N, k, 16).total;
}

extern "C" int rt_int8_scan_topk(const int8_t* queries, int64_t B, const int8_t* items,
                                 int64_t N, int64_t D, int64_t k, const uint64_t* mask,
                                 int64_t mask_words, int64_t* out_ids, int32_t* out_scores,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(items) % 16 == 0,
               "queries and items must be 16-byte aligned");
  RT_CHECK_ARG(mask == nullptr || mask_words >= cdiv(N, 64), "mask must have ceil(N/64) words");
  if (B == 0) return kOk;
  const ScanPlan plan = plan_scan(B, N, k, 16);
  if (workspace_bytes < plan.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, plan.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* lists = reinterpret_cast<uint64_t*>(ws + plan.off_lists);
  int* counts = reinterpret_cast<int*>(ws + plan.off_counts);
  uint64_t* tau = reinterpret_cast<uint64_t*>(ws + plan.off_tau);

  ScanArgs a{};
  a.queries = queries;
  a.B = B;
  a.items = items;
  a.k = static_cast<int>(k);
  a.mask = mask;
  a.mask_words = mask_words;
  a.lists = lists;
  a.counts = counts;

  MergeArgs m{};
  m.lists = lists;
  m.counts = counts;
  m.qpw = 16;
  m.B = B;
  m.k = static_cast<int>(k);

  if (N == 0) {
    // nothing to score: -1 / INT32_MIN pads
    return launch_pad(out_ids, out_scores, B, k, kScoreI32, stream);
  }
  {
    if (plan.seeded) {
      a.n_rows = plan.seed.n_rows;
      a.row_stride = plan.seed.row_stride;
      a.strip = plan.seed.strip;
      a.capw = plan.seed.capw;
      a.tau_in = nullptr;
      int st = dispatch_scan_int8(D, a, plan.seed, plan.n_qgroups, true, stream);
      if (st != kOk) return st;
      m.capw = 1;
      m.counts = nullptr;  // one entry per list: each seed wave's best
      m.gx = plan.seed.gx;
      m.tau_out = tau;
      st = launch_merge(m, stream);
      if (st != kOk) return st;
      m.tau_out = nullptr;
      m.counts = counts;
    }
    a.n_rows = plan.main.n_rows;
    a.row_stride = 1;
    a.strip = plan.main.strip;
    a.capw = plan.main.capw;
    a.tau_in = plan.seeded ? tau : nullptr;
    hipEvent_t stop;
    profile_begin(stream, &stop);
    int st = dispatch_scan_int8(D, a, plan.main, plan.n_qgroups, false, stream);
    profile_end(stream, stop);
    if (st != kOk) return st;
    m.capw = plan.main.capw;
    m.gx = plan.main.gx;
  }
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = kScoreI32;
  return launch_merge(m, stream);
}
