// The exact top-k merge over the scan waves' lists, launch planning, and the library's error
// store.
#include <cstdarg>
#include <cstdlib>

#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

// ---- errors -----------------------------------------------------------------------------

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_error; }

// ---- planning ---------------------------------------------------------------------------

// Workgroups a seed pass aims for, and the main pass's when the device cannot be queried.
static constexpr int64_t kTargetWorkgroups = 2048;
// At least this many sampled rows per wanted item (keeps the main pass's candidates near
// k * N / seed_rows for large k).
static constexpr int64_t kSeedRowsPerK = 1024;
// Upper bound on the candidate lists' workspace (a pass may exceed it only at one workgroup
// per query group).
static constexpr int64_t kMaxListBytes = int64_t{2} << 30;

static PassPlan plan_pass(int64_t n_rows, int64_t row_stride, int64_t n_qgroups, int64_t min_rows,
                          int capw, int64_t lists_per_wg, int64_t lists_per_query_per_wg,
                          int64_t target_wgs, int64_t min_gx = 1) {
  PassPlan p;
  p.n_rows = n_rows;
  p.row_stride = row_stride;
  p.capw = capw;
  int64_t gx = target_wgs / (n_qgroups > 0 ? n_qgroups : 1);
  gx = gx < min_gx ? min_gx : gx;
  const int64_t by_rows = cdiv(n_rows, min_rows);
  gx = gx < by_rows ? gx : by_rows;
  const int64_t by_slots = kMaxMergeSlots / lists_per_query_per_wg;
  gx = gx < by_slots ? gx : by_slots;
  // keep the lists within kMaxListBytes (fewer workgroups for large k or batch)
  const int64_t per_wg = n_qgroups * lists_per_wg * static_cast<int64_t>(capw) *
                         static_cast<int64_t>(sizeof(uint64_t));
  const int64_t by_bytes = kMaxListBytes / (per_wg > 0 ? per_wg : 1);
  gx = gx < by_bytes ? gx : by_bytes;
  gx = gx < 1 ? 1 : gx;
  p.strip = align_up(static_cast<size_t>(cdiv(n_rows, gx)), kTile);
  if (p.strip == 0) p.strip = kTile;
  p.gx = cdiv(n_rows, p.strip);
  if (p.gx < 1) p.gx = 1;
  p.S = p.gx * lists_per_query_per_wg;
  p.lists_bytes = static_cast<size_t>(p.gx) * n_qgroups * lists_per_wg * capw * sizeof(uint64_t);
  p.counts_bytes = static_cast<size_t>(p.gx) * n_qgroups * lists_per_wg * sizeof(int);
  // the seed's flat one-entry lists: [B rounded up to groups][S]
  return p;
}

int64_t main_workgroups() {
  int dev = 0;
  int cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0) {
    return kTargetWorkgroups;
  }
  const int64_t t = static_cast<int64_t>(cus) * kMainWorkgroupsPerCU;
  return t < kMaxResidentWorkgroups ? t : kMaxResidentWorkgroups;
}

ScanPlan plan_scan(int64_t B, int64_t N, int64_t k, int64_t qpg, int64_t lists_per_wg,
                   int64_t target_wgs, int main_capw, int64_t seed_rows_per_wg,
                   int64_t seed_rows_min) {
  ScanPlan s;
  s.qpg = qpg;
  s.n_qgroups = cdiv(B, qpg);
  // a query's lists per workgroup: every wave scores all of the row's queries (lists_per_wg ==
  // waves * qpg), or one wave owns each query (lists_per_wg == qpg)
  const int64_t lpq = lists_per_wg / qpg;
  const int64_t seed_rows =
      seed_rows_min > kSeedRowsPerK * k ? seed_rows_min : kSeedRowsPerK * k;
  s.seeded = N >= 8 * seed_rows;
  if (s.seeded) {
    // one-entry lists (each seed wave's best); at least 2k of them per query (their k-th is the
    // safe bound, their rank-th the speculative one; 4k cost configuration 5's step 1.5 % in
    // seed workgroups, each loading the group's queries)
    s.seed = plan_pass(seed_rows, N / seed_rows, s.n_qgroups, seed_rows_per_wg, 1, lists_per_wg,
                       lpq, kTargetWorkgroups, cdiv(2 * k, lpq));
  }
  s.main = plan_pass(N, 1, s.n_qgroups, 1024, main_capw, lists_per_wg, lpq, target_wgs);
  const size_t lists = s.main.lists_bytes > s.seed.lists_bytes ? s.main.lists_bytes
                                                              : s.seed.lists_bytes;
  const size_t counts = s.main.counts_bytes > s.seed.counts_bytes ? s.main.counts_bytes
                                                                 : s.seed.counts_bytes;
  s.off_lists = 0;
  s.off_counts = align_up(lists, 256);
  s.off_tau = s.off_counts + align_up(counts, 256);
  s.off_flag = s.off_tau + align_up(static_cast<size_t>(B) * sizeof(uint64_t), 256);
  s.off_parts = s.off_flag + 256;
  s.split = B <= kMergeSplitMaxB;
  s.total = s.off_parts +
            (s.split ? align_up(static_cast<size_t>(B) * kMergeParts * k * sizeof(uint64_t), 256)
                     : 0);
  return s;
}

// ---- merge ------------------------------------------------------------------------------

constexpr int kMergeChunk = 10240;  // list entries gathered into LDS per round
// The light form for grids of more queries than CUs whose queries read at most
// kMergeSlotsLight lists: rounds of kMergeChunkLight entries, ~30 KB of LDS for k <= 128
// against ~140 KB, so four workgroups share a CU instead of one.
constexpr int kMergeChunkLight = 2048;
constexpr int kMergeSlotsLight = 1024;
constexpr int64_t kMergeLightMinBlocks = 256;
constexpr int kMergeWaves = kMergeThreads / kWave;

// Block-wide min and max of keys[0, n) (LDS). Every thread calls it; all get the results.
__device__ void block_minmax(const uint64_t* keys, int n, uint64_t* red, uint64_t* lo,
                             uint64_t* hi) {
  const int tid = threadIdx.x;
  uint64_t a = ~0ull;
  uint64_t b = 0ull;
  for (int i = tid; i < n; i += blockDim.x) {
    const uint64_t v = keys[i];
    a = v < a ? v : a;
    b = v > b ? v : b;
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const uint64_t oa = __shfl_xor(a, off);
    const uint64_t ob = __shfl_xor(b, off);
    a = oa < a ? oa : a;
    b = ob > b ? ob : b;
  }
  if ((tid & (kWave - 1)) == 0) {
    red[2 * (tid / kWave)] = a;
    red[2 * (tid / kWave) + 1] = b;
  }
  __syncthreads();
  a = ~0ull;
  b = 0ull;
  for (int w = 0; w < static_cast<int>(blockDim.x) / kWave; ++w) {
    a = red[2 * w] < a ? red[2 * w] : a;
    b = red[2 * w + 1] > b ? red[2 * w + 1] : b;
  }
  *lo = a;
  *hi = b;
  __syncthreads();
}

// Appends v at dst[*counter + j] when keep, j counting the keeping lanes of the wave before
// this one: one LDS atomic a wave. Every lane of the wave calls it.
__device__ __forceinline__ void wave_append(uint64_t* dst, int* counter, bool keep, uint64_t v) {
  const uint64_t b = __ballot(keep);
  if (b == 0ull) return;
  const int before = static_cast<int>(__builtin_amdgcn_mbcnt_hi(
      static_cast<uint32_t>(b >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b), 0u)));
  int base = 0;
  if ((threadIdx.x & (kWave - 1)) == 0) base = atomicAdd(counter, __popcll(b));
  base = __shfl(base, 0);
  if (keep) dst[base + before] = v;
}

// Block-wide radix select over keys[0, n) in LDS, MSB-first digits of up to 8 bits, starting
// below the bits every key shares (min and max agree there). Returns a bound T with at
// most kth keys > T and at least kth keys >= T (exactly kth for distinct keys): the kth
// largest key counted with repeats, or, when a digit pass finds the kth largest key's bucket
// holding exactly the keys still wanted, that bucket's lowest possible value (the search
// stops there).
// 1 <= kth <= n. Every thread of the block calls it.
__device__ uint64_t block_select_desc(const uint64_t* keys, int n, int kth, unsigned* hist,
                                      int* sh, uint64_t* red) {
  const int tid = threadIdx.x;
  uint64_t kmin;
  uint64_t kmax;
  block_minmax(keys, n, red, &kmin, &kmax);
  const uint64_t diff = kmin ^ kmax;
  if (diff == 0ull) return kmin;
  int top = 63 - __builtin_clzll(diff);  // highest bit where keys differ
  uint64_t mask = top == 63 ? 0ull : ~((2ull << top) - 1ull);
  uint64_t prefix = kmin & mask;
  if (tid == 0) {
    sh[1] = kth;
    sh[3] = 0;
  }
  __syncthreads();
  while (true) {
    const int low = top >= 7 ? top - 7 : 0;
    const int width = top - low + 1;
    const uint64_t dmask = (1ull << width) - 1ull;
    for (int i = tid; i < 256; i += blockDim.x) hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < n; i += blockDim.x) {
      const uint64_t v = keys[i];
      if ((v & mask) == prefix) atomicAdd(&hist[(v >> low) & dmask], 1u);
    }
    __syncthreads();
    if (tid < kWave) {
      // lane l covers digits 255 - 4l - j, j < 4 (descending digit order across the wave)
      const int lane = tid;
      unsigned c[4];
      unsigned sum = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[255 - 4 * lane - j];
        sum += c[j];
      }
      unsigned incl = sum;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const unsigned t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
      }
      const unsigned excl = incl - sum;
      const unsigned want = static_cast<unsigned>(sh[1]);
      if (excl < want && want <= incl) {
        unsigned run = excl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (run + c[j] >= want) {
            sh[0] = 255 - 4 * lane - j;
            sh[1] = static_cast<int>(want - run);
            sh[3] = c[j] == want - run;  // the bucket is exactly the keys still wanted
            break;
          }
          run += c[j];
        }
      }
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(sh[0]) << low;
    mask |= dmask << low;
    const bool done = sh[3] != 0 || low == 0;
    __syncthreads();
    if (done) break;
    top = low - 1;
  }
  return prefix;
}

// The exact top-k of one query over all its scan lists. Rounds of up to kMergeChunk list
// entries are gathered behind the current best (at most k entries), the k-th largest of the
// union is found by radix select and only the entries >= it are kept; the survivors are
// sorted at the end. With tau_out set, only the k-th composite is written (0 when fewer than
// k entries exist: no bound; with tau_keep, the larger of it and the bound already there).
template <int KP, int CHUNK = kMergeChunk, int SLOTS = kMaxMergeSlots>
__global__ void __launch_bounds__(kMergeThreads) merge_kernel(MergeArgs m) {
  __shared__ uint64_t buf[KP + CHUNK];
  __shared__ uint64_t tmp[KP];
  __shared__ int pre[SLOTS];
  __shared__ short owner[CHUNK];
  __shared__ unsigned hist[256];
  __shared__ int part[kMergeThreads];
  __shared__ uint64_t red[2 * kMergeWaves];
  __shared__ int sh[4];
  __shared__ int fill;
  const int tid = threadIdx.x;
  if (m.run_if != nullptr && *m.run_if == 0u) return;  // (uniform: the fallback is not needed)
  // a split merge's first launch: block = (query, part), the part's lists [s_lo, s_lo + S)
  const int parts = m.part_out != nullptr ? m.parts : 1;
  const int64_t q = blockIdx.x / parts;
  const int my_part = static_cast<int>(blockIdx.x % parts);
  const int span = static_cast<int>((m.S + parts - 1) / parts);
  const int s_lo = my_part * span;
  const int S = static_cast<int>(m.S - s_lo < span ? (m.S - s_lo > 0 ? m.S - s_lo : 0) : span);
  const int64_t g = q / m.qpw;
  const int qi = static_cast<int>(q % m.qpw);
  const int64_t slot0 = g * m.S + s_lo;
  const int k = m.k;

  // list lengths → inclusive prefix sums over this query's lists (flat: S one-entry lists
  // stored contiguously per query, lists + q * S)
  int total = S;
  if (!m.flat) {
    const int per = (S + kMergeThreads - 1) / kMergeThreads;
    int run = 0;
    for (int i = 0; i < per; ++i) {
      const int s = tid * per + i;
      if (s < S) {
        int c = m.counts[(slot0 + s) * m.qpw + qi];
        c = c < m.capw ? c : m.capw;
        run += c;
        pre[s] = run;
      }
    }
    // exclusive prefix of the threads' runs: a scan within each wave, then the waves' totals
    int incl = run;
    const int lane = tid & (kWave - 1);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int t = __shfl_up(incl, off);
      incl += lane >= off ? t : 0;
    }
    if (lane == kWave - 1) part[tid / kWave] = incl;
    __syncthreads();
    int base = incl - run;
    for (int w = 0; w < tid / kWave; ++w) base += part[w];
    for (int i = 0; i < per; ++i) {
      const int s = tid * per + i;
      if (s < S) pre[s] += base;
    }
    __syncthreads();
    total = S > 0 ? pre[S - 1] : 0;
  }

  // Entries <= thr cannot enter the top k: once a round has kept the best k, thr is their
  // bound (k entries >= thr, and an entry equal to it is the same composite again), so
  // later rounds gather only what beats it and their selects run over a few survivors.
  // Empty entries (0) are dropped from the start.
  uint64_t thr = 0ull;
  int held = 0;
  for (int e0 = 0; e0 < total; e0 += CHUNK) {
    const int n = total - e0 < CHUNK ? total - e0 : CHUNK;
    if (!m.flat) {
      // owner[] maps each entry of the window to its list (LDS only)
      for (int s = tid; s < S; s += kMergeThreads) {
        const int lo = s == 0 ? 0 : pre[s - 1];
        const int hi = pre[s];
        const int a = lo > e0 ? lo : e0;
        const int b = hi < e0 + n ? hi : e0 + n;
        for (int e = a; e < b; ++e) owner[e - e0] = static_cast<short>(s);
      }
    }
    if (tid == 0) fill = 0;
    __syncthreads();
    // every thread loads independent entries, four in flight; the trip count is the same for
    // the whole block, so every lane of a wave takes part in each append
    const uint64_t* row = m.lists + q * m.S + s_lo + e0;
    const int rounds = (n + 4 * kMergeThreads - 1) / (4 * kMergeThreads);
    for (int r = 0; r < rounds; ++r) {
      const int i0 = r * 4 * kMergeThreads + tid;
      uint64_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kMergeThreads;
        v[u] = 0ull;
        if (i < n) {
          if (m.flat) {
            v[u] = row[i];
          } else {
            const int s = owner[i];
            const int lo = s == 0 ? 0 : pre[s - 1];
            v[u] = m.lists[((slot0 + s) * m.qpw + qi) * static_cast<int64_t>(m.capw) +
                           (e0 + i - lo)];
          }
        }
      }
      if (!m.flat && m.clause.active != nullptr) {
        // an entry that fails the query's clauses is empty (0, below every composite); flat
        // lists (a seed pass's maxima) were tested where they were written
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (v[u] > thr && !clause_check(m.clause, q, composite_item(v[u]))) v[u] = 0ull;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) wave_append(buf + held, &fill, v[u] > thr, v[u]);
    }
    __syncthreads();
    const int cnt = held + fill;
    if (cnt > k) {
      const uint64_t kth = block_select_desc(buf, cnt, k, hist, sh, red);
      thr = kth;
      if (tid == 0) sh[2] = 0;
      __syncthreads();
      // at most k entries are above kth; equal entries (repeated empty seed entries, or a
      // candidate listed twice) fill the remaining places, any copy being as good as another
      for (int i = tid; i < cnt; i += kMergeThreads) {
        const uint64_t v = buf[i];
        if (v > kth) tmp[atomicAdd(&sh[2], 1)] = v;
      }
      __syncthreads();
      for (int i = tid; i < cnt; i += kMergeThreads) {
        const uint64_t v = buf[i];
        if (v == kth) {
          const int p = atomicAdd(&sh[2], 1);
          if (p < k) tmp[p] = v;
        }
      }
      __syncthreads();
      for (int i = tid; i < k; i += kMergeThreads) buf[i] = tmp[i];
      held = k;
    } else {
      held = cnt;
    }
    __syncthreads();
  }

  if (m.part_out != nullptr) {
    // the part's best k (or all it holds), the rest empty
    uint64_t* out = m.part_out + blockIdx.x * static_cast<int64_t>(k);
    for (int i = tid; i < k; i += kMergeThreads) out[i] = i < held ? buf[i] : 0ull;
    return;
  }
  if (m.tau_out != nullptr) {
    // only the k-th composite: held <= k entries remain, the best k of everything when held == k
    uint64_t lo = 0ull;
    uint64_t hi = 0ull;
    if (held == k) block_minmax(buf, held, red, &lo, &hi);
    // and the k2-th over the same held entries, the best k2 of everything (a radix select:
    // block-uniform, as held is)
    const uint64_t t2 = m.tau2_out != nullptr && held >= m.k2
                            ? block_select_desc(buf, held, m.k2, hist, sh, red)
                            : 0ull;
    if (tid == 0) {
      const uint64_t t = held == k ? lo : 0ull;
      const uint64_t old =
          m.tau_keep ? (m.tau_base != nullptr ? m.tau_base[q] : m.tau_out[q]) : 0ull;
      m.tau_out[q] = t > old ? t : old;
      if (m.tau2_out != nullptr) m.tau2_out[q] = t2 > t ? t2 : t;
      if (m.spec_flag != nullptr && q == 0) *m.spec_flag = 0u;
    }
    return;
  }
  for (int i = held + tid; i < KP; i += kMergeThreads) buf[i] = 0ull;
  __syncthreads();
  for (int size = 2; size <= KP; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < (KP >> 1); t += kMergeThreads) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint64_t a = buf[i];
        const uint64_t b = buf[j];
        if ((a < b) == desc) {
          buf[i] = b;
          buf[j] = a;
        }
      }
      __syncthreads();
    }
  }

  if (m.spec_flag != nullptr && tid == 0 && buf[k - 1] == 0ull &&
      m.spec_tau[q] > (m.safe_tau != nullptr ? m.safe_tau[q] : 0ull)) {
    atomicOr(m.spec_flag, 1u);
  }
  for (int j = tid; j < k; j += kMergeThreads) {
    const uint64_t c = buf[j];
    const bool ok = c != 0ull;
    m.out_ids[q * k + j] = ok ? static_cast<int64_t>(composite_item(c)) : -1;
    const uint32_t key = composite_key(c);
    if (m.score_kind == kScoreI32) {
      static_cast<int32_t*>(m.out_scores)[q * k + j] = ok ? i32_of_key(key) : INT32_MIN;
    } else if (m.score_kind == kScoreF32FromI32) {
      static_cast<float*>(m.out_scores)[q * k + j] =
          ok ? static_cast<float>(i32_of_key(key)) : -INFINITY;
    } else {
      static_cast<float*>(m.out_scores)[q * k + j] = ok ? f32_of_key(key) : -INFINITY;
    }
  }
}

__global__ void pad_kernel(int64_t* ids, void* scores, int64_t n, int score_kind) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  ids[i] = -1;
  if (score_kind == kScoreI32) {
    static_cast<int32_t*>(scores)[i] = INT32_MIN;
  } else {
    static_cast<float*>(scores)[i] = -INFINITY;
  }
}

int launch_pad(int64_t* out_ids, void* out_scores, int64_t B, int64_t k, int score_kind,
               hipStream_t stream) {
  const int64_t n = B * k;
  if (n == 0) return kOk;
  pad_kernel<<<static_cast<unsigned>(cdiv(n, 256)), 256, 0, stream>>>(out_ids, out_scores, n,
                                                                     score_kind);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

static int launch_merge_grid(const MergeArgs& m, int64_t blocks, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(blocks));
#ifndef RT_MERGE_LIGHT
#define RT_MERGE_LIGHT 1
#endif
  if (RT_MERGE_LIGHT && m.k <= 128 && m.S <= kMergeSlotsLight && blocks > kMergeLightMinBlocks) {
    merge_kernel<128, kMergeChunkLight, kMergeSlotsLight><<<grid, kMergeThreads, 0, stream>>>(m);
    RT_CHECK_HIP(hipGetLastError());
    return kOk;
  }
  if (m.k <= 128) {
    merge_kernel<128><<<grid, kMergeThreads, 0, stream>>>(m);
  } else if (m.k <= 256) {
    merge_kernel<256><<<grid, kMergeThreads, 0, stream>>>(m);
  } else if (m.k <= 512) {
    merge_kernel<512><<<grid, kMergeThreads, 0, stream>>>(m);
  } else {
    merge_kernel<1024><<<grid, kMergeThreads, 0, stream>>>(m);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// A small batch's merge is split when the caller gave room: each query's lists go to up to
// kMergeParts workgroups (a part at least kMergeMinPartSlots lists), each keeping its part's
// best k in part_buf, then one workgroup per query merges those (flat, kMergeParts * k
// entries) with the call's own outputs. Same results: the best k of the union is among the
// parts' best k.
constexpr int64_t kMergeMinPartSlots = 256;

int launch_merge(const MergeArgs& m, hipStream_t stream) {
  RT_CHECK_ARG(m.k >= 1 && m.k <= kMaxK, "k must be in [1, %lld], got %d",
               static_cast<long long>(kMaxK), m.k);
  RT_CHECK_ARG(m.S >= 1 && m.S <= kMaxMergeSlots, "too many scan lists per query");
  if (m.B == 0) return kOk;
  int64_t parts = m.S / kMergeMinPartSlots;
  parts = parts < kMergeParts ? parts : kMergeParts;
  if (m.part_buf == nullptr || m.B > kMergeSplitMaxB || parts < 2) {
    MergeArgs one = m;
    one.parts = 1;
    one.part_out = nullptr;
    return launch_merge_grid(one, m.B, stream);
  }
  MergeArgs first = m;
  first.parts = static_cast<int>(parts);
  first.part_out = m.part_buf;
  first.tau_out = nullptr;
  first.spec_flag = nullptr;
  int st = launch_merge_grid(first, m.B * parts, stream);
  if (st != kOk) return st;
  MergeArgs second = m;
  second.lists = m.part_buf;
  second.counts = nullptr;
  second.flat = true;
  second.capw = 1;
  second.S = parts * m.k;
  second.clause = ClauseCheck{};  // (the first launch tested them)
  second.parts = 1;
  second.part_out = nullptr;
  return launch_merge_grid(second, m.B, stream);
}

}  // namespace rt

extern "C" const char* rt_last_error(void) { return rt::last_error(); }
