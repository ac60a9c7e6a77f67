// 1-bit Hamming full scan with the exact fused top-k: score = 64 W - 2 popcount(q ^ item)
// (Sign-OPORP / SimHash codes of W 64-bit words; retrieve/src/retrieve/ops/reference/
// oporp_1bit_match_topk.py:9-17), ties to the lower item index.
//
// Each lane scores its own item (its 2W dwords in VGPRs) against one wave-uniform query at a
// time: v_xor_b32 with the query dword (an SGPR, read by scalar loads through the constant
// address space) and v_bcnt_u32_b32 accumulating the popcount, 2 VALU per dword. A query's
// fast-path test is ham <= its threshold; the rare candidates go to the per-(wave, query) lists
// of uniform_topk.h and the shared merge.
#include "profile.h"
#include "scan_common.h"
#include "uniform_topk.h"
#include "wave_lists.h"

namespace rt {

constexpr int kHamTile = kWave;  // items per tile: one per lane
constexpr int kHamMaxQpw = 64;   // queries a wave scores (a query group)

// A row of W words: 16-byte loads when W is even (rows 16-byte aligned), 8-byte loads when odd.
template <int W>
__device__ inline void load_codes(const uint32_t* __restrict__ I, int64_t item, uint32_t* iw) {
  const uint4* p = reinterpret_cast<const uint4*>(I + item * (2 * W));
  if constexpr (W % 2 == 1) {
    const uint2* p2 = reinterpret_cast<const uint2*>(I + item * (2 * W));
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const uint2 v = p2[j];
      iw[2 * j] = v.x;
      iw[2 * j + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < W / 2; ++j) {
      const uint4 v = p[j];
      iw[4 * j] = v.x;
      iw[4 * j + 1] = v.y;
      iw[4 * j + 2] = v.z;
      iw[4 * j + 3] = v.w;
    }
  }
}

// Query codes through the constant address space: with a wave-uniform address the loads are
// scalar (s_load into SGPRs), so the XORs take the query dword as their scalar operand and no
// LDS bandwidth goes to broadcasting it. The queries are never written by the scan.
typedef __attribute__((address_space(4))) const uint32_t ku32;

template <int W, class Q>
__device__ inline int hamming(const uint32_t* iw, Q qw) {
  int h = 0;
#pragma unroll
  for (int d = 0; d < 2 * W; ++d) h = __builtin_popcount(iw[d] ^ qw[d]) + h;
  return h;
}

// ham <= hamming_limit(ts)  <=>  64 W - 2 ham >= ts
template <int W>
__device__ inline int hamming_limit(uint64_t tau) {
  const int64_t ts = i32_of_key(composite_key(tau));
  const int64_t lim = (64 * W - ts);
  return lim < 0 ? -1 : static_cast<int>(lim >> 1 < 0x7fffffff ? lim >> 1 : 0x7fffffff);
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off);
    v = o > v ? o : v;
  }
  return v;
}

// Seed pass over the strided sample: tiles of 64 sampled rows dealt round-robin to the grid
// row's waves; each wave keeps, per query, its best composite (LDS) and writes it to
// lists[q * S + wave index] (S = waves of the grid row).
template <int W>
__global__ void __launch_bounds__(kScanThreads) seed_hamming_kernel(ScanArgs a) {
  __shared__ uint64_t best[kScanWaves][kHamMaxQpw];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  ku32* Q = (ku32*)(a.queries);
  const uint32_t* I = static_cast<const uint32_t*>(a.items);
  const int64_t wi = static_cast<int64_t>(blockIdx.x) * kScanWaves + wave;
  const int64_t S = static_cast<int64_t>(gridDim.x) * kScanWaves;
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * a.qpw;
  const int nq = static_cast<int>(a.B - q0 < a.qpw ? a.B - q0 : a.qpw);
  for (int i = lane; i < kHamMaxQpw; i += kWave) best[wave][i] = 0ull;
  wave_sync_memory();
  const int64_t ntiles = cdiv(a.n_rows, kHamTile);
  for (int64_t t = wi; t < ntiles; t += S) {
    const int64_t row = t * kHamTile + lane;
    const bool valid = row < a.n_rows;
    const uint32_t item = static_cast<uint32_t>(sample_item(valid ? row : 0, a.row_stride));
    uint32_t iw[2 * W];
    load_codes<W>(I, item, iw);
    for (int qi = 0; qi < nq; ++qi) {
      const int64_t q = q0 + qi;
      const int h = hamming<W>(iw, Q + q * (2 * W));
      bool ok = valid;
      if (ok && a.mask != nullptr) {
        ok = (a.mask[q * a.mask_words + (item >> 6)] >> (63 - (item & 63))) & 1ull;
      }
      const uint64_t c = ok ? composite(key_of_i32(64 * W - 2 * h), item) : 0ull;
      const uint64_t m = wave_max_u64(c);
      if (lane == 0 && m > best[wave][qi]) best[wave][qi] = m;
    }
  }
  wave_sync_memory();
  for (int qi = lane; qi < nq; qi += kWave) a.lists[(q0 + qi) * S + wi] = best[wave][qi];
}

// Main pass over every item: tiles of 64 rows dealt round-robin to the group's waves; queries
// go two at a time, their codes in SGPRs, each query's popcount limit in lane q of a VGPR (read
// back with v_readlane).
template <int W>
__global__ void __launch_bounds__(kScanThreads) scan_hamming_kernel(ScanArgs a, int scratch_n) {
  extern __shared__ __attribute__((aligned(16))) uint64_t smem[];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qpw = a.qpw;
  uint64_t* rest = smem;
  uint64_t* scratch = rest + wave * scratch_n;
  uint64_t* tau = rest + kScanWaves * scratch_n + wave * qpw;
  int* cnt = reinterpret_cast<int*>(rest + kScanWaves * (scratch_n + qpw)) +
             kScanWaves * qpw + wave * qpw;
  const int64_t wave_in_group = static_cast<int64_t>(blockIdx.x) * kScanWaves + wave;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kScanWaves;
  const int64_t slot = static_cast<int64_t>(blockIdx.y) * waves + wave_in_group;
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * qpw;
  const int nq = static_cast<int>(a.B - q0 < qpw ? a.B - q0 : qpw);
  ku32* qcodes = (ku32*)(a.queries) + q0 * 2 * W;  // [nq][2W]
  int hlim = -1;  // lane q: query q's popcount limit (qpw <= kWave)
  for (int i = lane; i < qpw; i += kWave) {
    const uint64_t t = i < nq ? (a.tau_in != nullptr ? a.tau_in[q0 + i] : 0ull) : ~0ull;
    tau[i] = t;
    hlim = i < nq ? hamming_limit<W>(t) : -1;
    cnt[i] = 0;
  }
  WaveTopKUniform top;
  top.lists = a.lists + slot * qpw * static_cast<int64_t>(a.capw);
  top.cnt = cnt;
  top.tau = tau;
  top.scratch = scratch;
  top.capw = a.capw;
  top.scratch_n = scratch_n;
  top.k = a.k;
  __syncthreads();

  const uint32_t* I = static_cast<const uint32_t*>(a.items);
  const int64_t n = a.n_rows;
  const int64_t ntiles = cdiv(n, kHamTile);
  auto handle = [&](int qi, bool ok, int h, uint32_t item) {
    if (!__any(ok)) return;
    const uint64_t before = tau[qi];
    const uint64_t after =
        top.push(qi, ok, key_of_i32(64 * W - 2 * h), item,
                 a.mask != nullptr ? a.mask + (q0 + qi) * a.mask_words : nullptr);
    if (after != before) hlim = lane == qi ? hamming_limit<W>(after) : hlim;
  };
  for (int64_t t = wave_in_group; t < ntiles; t += waves) {
    const int64_t row = t * kHamTile + lane;
    const bool valid = row < n;
    const uint32_t item = static_cast<uint32_t>(valid ? row : n - 1);
    uint32_t iw[2 * W];
    load_codes<W>(I, item, iw);
    int qi = 0;
    for (; qi + 1 < nq; qi += 2) {
      const int h0 = hamming<W>(iw, qcodes + qi * 2 * W);
      const int h1 = hamming<W>(iw, qcodes + (qi + 1) * 2 * W);
      const bool ok0 = valid && h0 <= __builtin_amdgcn_readlane(hlim, qi);
      const bool ok1 = valid && h1 <= __builtin_amdgcn_readlane(hlim, qi + 1);
      if (__any(ok0 || ok1)) {
        handle(qi, ok0, h0, item);
        handle(qi + 1, ok1, h1, item);
      }
    }
    if (qi < nq) {
      const int h = hamming<W>(iw, qcodes + qi * 2 * W);
      handle(qi, valid && h <= __builtin_amdgcn_readlane(hlim, qi), h, item);
    }
  }
  wave_sync_memory();
  for (int i = lane; i < qpw; i += kWave) a.counts[slot * qpw + i] = cnt[i];
}

static int ham_capw(int64_t k) {
  return static_cast<int>(align_up(static_cast<size_t>(k) + kWave, 64));
}

static size_t ham_lds(int qpw, int scratch_n) {
  return kScanWaves * (scratch_n * sizeof(uint64_t) + qpw * (sizeof(uint64_t) + 2 * sizeof(int)));
}

template <int W>
static int launch_ham(const ScanArgs& a, const PassPlan& p, int64_t nqg, bool seed,
                      hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.gx), static_cast<unsigned>(nqg));
  if (seed) {
    seed_hamming_kernel<W><<<grid, kScanThreads, 0, stream>>>(a);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  const int scratch_n = static_cast<int>(next_pow2(a.capw));
  const size_t lds = ham_lds(a.qpw, scratch_n);
  if (lds > 65536) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(scan_hamming_kernel<W>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  scan_hamming_kernel<W><<<grid, kScanThreads, lds, stream>>>(a, scratch_n);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

constexpr int kHamMaxWords = 16;

template <int W>
static int dispatch_ham_from(int64_t w, const ScanArgs& a, const PassPlan& p, int64_t nqg,
                             bool seed, hipStream_t stream) {
  if (w == W) return launch_ham<W>(a, p, nqg, seed, stream);
  if constexpr (W < kHamMaxWords) {
    return dispatch_ham_from<W + 1>(w, a, p, nqg, seed, stream);
  } else {
    set_error("Hamming scan supports W (64-bit words per code) in [1, %d], got %lld",
              kHamMaxWords, static_cast<long long>(w));
    return kInvalidArgument;
  }
}

static int dispatch_ham(int64_t W, const ScanArgs& a, const PassPlan& p, int64_t nqg, bool seed,
                        hipStream_t stream) {
  return dispatch_ham_from<1>(W, a, p, nqg, seed, stream);
}

static int ham_qpw(int64_t B) { return static_cast<int>(B < kHamMaxQpw ? B : kHamMaxQpw); }

// From this batch on, the blocked scan on the fp4 matrix cores (bits as e2m1 nibbles) takes the
// 512-bit batches the per-wave scan below does not (more than kBitsMfmaMaxBatch queries, and the
// scans with exact clauses or a transposed mask); below, one XOR + popcount pass per query and word. Measured over
// 30M codes (k = 100, a call): the popcount pass costs ~0.33 ms + ~35-48 us per query
// (VALU-bound: 2 VALU per 32 bits; B=4 0.46 ms, B=8 0.59 ms, B=12 0.76 ms), the blocked path
// ~0.46-0.52 ms from B=12 to B=32, so it takes over from 8 queries.
constexpr int64_t kHamMfmaMinBatch = 8;

static bool ham_mfma(int64_t B, int64_t W, int64_t k, bool masked) {
  return W == 8 && B >= kHamMfmaMinBatch && blocked_hamming_fits(B, W, k, masked);
}

// Batches of 512-bit codes from kBitsMfmaMinBatch to kBitsMfmaMaxBatch queries run the per-wave
// fp4 scan (scan_bits_mfma.hip: no workgroup barriers, every 16-row group read straight into
// MFMA order), ahead of the blocked scan and the popcount pass. Over 30M codes, k = 100, a call:
// B = 1-16 0.34-0.35 ms (main pass 0.29 ms, 6.7 TB/s), B = 32 0.37 ms, B = 64 0.49 ms (k = 1000
// 0.51 ms), B = 128 0.89 ms; the blocked scan took 0.47 / 0.44 / 0.60 (1.08) / 1.09 ms and the
// popcount pass 0.38 ms at B = 1. From 256 queries the blocked scan is faster (1.54 against
// 1.69 ms).
constexpr int64_t kBitsMfmaMinBatch = 1;
constexpr int64_t kBitsMfmaMaxBatch = 128;

static bool ham_bits_mfma(int64_t B, int64_t W, int64_t k) {
  return W == 8 && B >= kBitsMfmaMinBatch && B <= kBitsMfmaMaxBatch && k <= kMaxK;
}

}  // namespace rt

using namespace rt;

extern "C" size_t rt_hamming_scan_topk_workspace(int64_t B, int64_t N, int64_t W, int64_t k,
                                                 int masked) {
  if (k > kMaxK) return hamming_large_k_workspace(B > 0 ? B : 1, N, W);
  if (ham_bits_mfma(B, W, k)) return bits_mfma_workspace(B, N, k);
  if (ham_mfma(B, W, k, masked != 0)) {
    return blocked_hamming_workspace(B, N, W, k, masked != 0);
  }
  const int qpw = ham_qpw(B > 0 ? B : 1);
  return plan_scan(B, N, k, qpw, kScanWaves * qpw, kMaxResidentWorkgroups, ham_capw(k),
                   kScanWaves * kHamTile)
      .total;
}

extern "C" int rt_hamming_scan_topk(const uint64_t* query_bits, int64_t B,
                                    const uint64_t* item_bits, int64_t N, int64_t W, int64_t k,
                                    const uint64_t* mask,
                                    int64_t mask_words, int64_t* out_ids, void* out_scores,
                                    int score_f32, void* workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0, "B and N must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxKHamming, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxKHamming), static_cast<long long>(k));
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  RT_CHECK_ARG(W >= 1 && W <= kHamMaxWords,
               "W (64-bit words per code) must be in [1, %d], got %lld", kHamMaxWords,
               static_cast<long long>(W));
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(item_bits) % (W % 2 ? 8 : 16) == 0,
               "item_bits must be %d-byte aligned", W % 2 ? 8 : 16);
  RT_CHECK_ARG(mask == nullptr || mask_words >= cdiv(N, 64), "mask must have ceil(N/64) words");
  if (B == 0) return kOk;
  const int kind = score_f32 ? kScoreF32FromI32 : kScoreI32;
  if (N == 0) return launch_pad(out_ids, out_scores, B, k, kind, stream);
  if (k > kMaxK) {
    return hamming_large_k(query_bits, B, item_bits, N, W, k, mask, mask_words, out_ids,
                           out_scores, kind, workspace, workspace_bytes, stream);
  }
  if (ham_bits_mfma(B, W, k)) {
    return bits_mfma(query_bits, B, item_bits, N, k, mask, mask_words, out_ids, out_scores, kind,
                     workspace, workspace_bytes, stream);
  }
  if (ham_mfma(B, W, k, mask != nullptr)) {
    return blocked_hamming(query_bits, B, item_bits, N, W, k, mask, mask_words, out_ids,
                           out_scores, kind, workspace, workspace_bytes, stream);
  }
  const int qpw = ham_qpw(B);
  const ScanPlan plan = plan_scan(B, N, k, qpw, kScanWaves * qpw, main_workgroups(), ham_capw(k),
                                  kScanWaves * kHamTile);
  if (workspace_bytes < plan.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, plan.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* lists = reinterpret_cast<uint64_t*>(ws + plan.off_lists);
  int* counts = reinterpret_cast<int*>(ws + plan.off_counts);
  uint64_t* tau = reinterpret_cast<uint64_t*>(ws + plan.off_tau);

  ScanArgs a{};
  a.queries = query_bits;
  a.B = B;
  a.items = item_bits;
  a.k = static_cast<int>(k);
  a.qpw = qpw;
  a.mask = mask;
  a.mask_words = mask_words;
  a.lists = lists;
  a.counts = counts;

  MergeArgs m{};
  m.lists = lists;
  m.counts = counts;
  m.qpw = qpw;
  m.B = B;
  m.k = static_cast<int>(k);

  if (plan.seeded) {
    a.n_rows = plan.seed.n_rows;
    a.row_stride = plan.seed.row_stride;
    a.capw = 1;
    a.tau_in = nullptr;
    int st = dispatch_ham(W, a, plan.seed, plan.n_qgroups, true, stream);
    if (st != kOk) return st;
    m.capw = 1;
    m.flat = true;
    m.S = plan.seed.S;
    m.tau_out = tau;
    st = launch_merge(m, stream);
    if (st != kOk) return st;
    m.tau_out = nullptr;
    m.flat = false;
  }
  a.n_rows = N;
  a.row_stride = 1;
  a.capw = plan.main.capw;
  a.tau_in = plan.seeded ? tau : nullptr;
  hipEvent_t stop;
  profile_begin(stream, &stop);
  int st = dispatch_ham(W, a, plan.main, plan.n_qgroups, false, stream);
  profile_end(stream, stop);
  if (st != kOk) return st;
  m.capw = plan.main.capw;
  m.S = plan.main.S;
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = kind;
  return launch_merge(m, stream);
}

// The 1-bit scan on the matrix cores with the exact clause filter tested per candidate that
// passes the mask (required), where the blocked kernel takes the batch (fused != 0).
extern "C" int rt_hamming_scan_topk_clauses_fused(int64_t B, int64_t W, int64_t k) {
  return k <= kMaxK && ham_mfma(B, W, k, true) ? 1 : 0;
}

extern "C" size_t rt_hamming_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t W,
                                                         int64_t k, int64_t C, int64_t V) {
  if (!(k <= kMaxK && ham_mfma(B, W, k, true))) return 256;
  return align_up(blocked_hamming_workspace(B, N, W, k, true), 256) +
         clause_prep_workspace(B, C, V);
}

extern "C" int rt_hamming_scan_topk_clauses(const uint64_t* query_bits, int64_t B,
                                            const uint64_t* item_bits, int64_t N, int64_t W,
                                            int64_t k, const uint64_t* mask, int64_t mask_words,
                                            int64_t mask_t_stride, const void* item_attrs,
                                            int attr_bytes, int64_t C,
                                            int64_t A, const int8_t* clause_is_reverse,
                                            const int64_t* query_values, int64_t V,
                                            int64_t* out_ids, void* out_scores, int score_f32,
                                            void* workspace, size_t workspace_bytes,
                                            hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && B <= (int64_t{1} << 21) && N >= 0, "B in [0, 2^21] and N >= 0");
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  RT_CHECK_ARG(mask != nullptr && mask_words >= cdiv(N, 64),
               "the fused clause filter needs a mask of ceil(N/64) words a row (rows, when "
               "transposed)");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK && ham_mfma(B, W, k, true),
               "the fused clause filter runs where the matrix-core scan takes the batch "
               "(rt_hamming_scan_topk_clauses_fused)");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(item_bits) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(query_bits) % 16 == 0,
               "query_bits and item_bits must be 16-byte aligned");
  RT_CHECK_ARG(C >= 0 && C <= kMaxClauses, "C must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(C));
  RT_CHECK_ARG(A >= 0 && A <= 4096 && V >= 1 && V <= 4096, "A must be in [0, 4096] and V in "
               "[1, 4096]");
  RT_CHECK_ARG(attr_bytes == 2 || attr_bytes == 4 || attr_bytes == 8,
               "attr_bytes must be 2, 4 or 8 (int16, int32, int64 attributes)");
  if (B == 0) return kOk;
  const int kind = score_f32 ? kScoreF32FromI32 : kScoreI32;
  if (N == 0) return launch_pad(out_ids, out_scores, B, k, kind, stream);
  RT_CHECK_ARG(C == 0 || (clause_is_reverse != nullptr && query_values != nullptr),
               "clause_is_reverse and query values must not be null");
  RT_CHECK_ARG(C * A == 0 || item_attrs != nullptr, "item attrs are null");
  const size_t scan_bytes = align_up(blocked_hamming_workspace(B, N, W, k, true), 256);
  const size_t need = scan_bytes + clause_prep_workspace(B, C, V);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  ClauseCheck f;
  if (C > 0) {
    const int st = clause_prepare(query_values, B, C, V, clause_is_reverse,
                                  static_cast<char*>(workspace) + scan_bytes,
                                  workspace_bytes - scan_bytes, &f, stream);
    if (st != kOk) return st;
    f.attrs = item_attrs;
    f.attr_bytes = attr_bytes;
    f.A = static_cast<int>(A);
  }
  return blocked_hamming(query_bits, B, item_bits, N, W, k, mask, mask_words, out_ids,
                         out_scores, kind, workspace, scan_bytes, stream, f, mask_t_stride);
}
