// 1-bit Hamming full-scan top-k for k above the list-based scans' 1024 (up to 8192): LiNR V3's
// candidate pools (retrieve/src/retrieve/modules/linr.py:112-162, candidate_pool = 5000 by
// default; the shortlist is oporp_1bit_match_topk_full, ops/triton/oporp_1bit_match_topk.py:
// 261-273, then torch.topk). Same result as the scan: top-k by (score desc, id asc) of
// score = 64 W - 2 popcount(q ^ item) over the items that pass the mask.
//
// A Hamming score takes only 64 W + 1 values, so the k-th score is found by counting:
//   1. histogram pass: per query, the number of passing items at each popcount h;
//   2. cut: the popcount h* of the k-th best, lt = #(h < h*), need = k - lt;
//   3. emit pass: items with h < h* appended (at most k - 1 of them); the items with h == h*
//      counted per bin of 8192 ids;
//   4. cut: the id bin b* where the ties reach `need`, need2 = what bin b* must give;
//   5. emit pass: the ties in bins below b* appended (fewer than need), those of bin b* apart
//      (at most 8192);
//   6. per query: bin b*'s ties sorted (their composites order by id), the first need2 kept,
//      everything sorted by composite and written.
// Each pass is the popcount scan of the small-batch path (lane <-> item, query codes in SGPRs);
// the appends go through global atomics and are rare (at most k + 8192 per query).
#include "scan_common.h"

namespace rt {
namespace {

constexpr int kLkThreads = 256;
constexpr int kLkWaves = kLkThreads / kWave;
constexpr int kLkQpw = 8;        // queries a workgroup scores per pass
constexpr int kLkIdShift = 13;   // bins of 8192 ids for the ties at the cut
constexpr int kLkCap = 8192;     // entries per query of each buffer (>= k and >= a bin)
constexpr int kLkFinalThreads = 1024;
constexpr int kLkMaxGx = 512;    // workgroups per query group (each flushes one histogram)

typedef __attribute__((address_space(4))) const uint32_t ku32;

struct LkArgs {
  const uint64_t* q;
  int64_t B;
  const uint64_t* items;
  int64_t N;
  int k;
  const uint64_t* mask;
  int64_t mask_words;
  int nb;            // 64 W + 1 popcount bins
  int64_t nbin;      // id bins
  uint32_t* hist;    // [B][nb] (N < 2^32 items: a count fits)
  int32_t* cnt;      // [B][4]: appends to A, B, C
  uint32_t* idhist;  // [B][nbin]
  int32_t* cut;      // [B][8]: h*, lt, need, b*, need2
  uint64_t* buf_a;   // [B][kLkCap]: h < h*
  uint64_t* buf_b;   // [B][kLkCap]: h == h*, id bin < b*
  uint64_t* buf_c;   // [B][kLkCap]: h == h*, id bin == b*
};

template <int W>
__device__ inline void lk_load(const uint32_t* __restrict__ I, int64_t item, uint32_t* iw) {
  if constexpr (W % 2 == 1) {
    const uint2* p = reinterpret_cast<const uint2*>(I + item * (2 * W));
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const uint2 v = p[j];
      iw[2 * j] = v.x;
      iw[2 * j + 1] = v.y;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(I + item * (2 * W));
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

// MODE 0: histogram; 1: append h < h*, count the ties per id bin; 2: append the ties of the
// bins up to b*.
template <int W, int MODE>
__global__ void __launch_bounds__(kLkThreads) lk_pass_kernel(LkArgs a) {
  extern __shared__ uint32_t lh[];  // MODE 0: [kLkQpw][nb]
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * kLkQpw;
  const int nq = static_cast<int>(a.B - q0 < kLkQpw ? a.B - q0 : kLkQpw);
  if constexpr (MODE == 0) {
    for (int i = threadIdx.x; i < kLkQpw * a.nb; i += kLkThreads) lh[i] = 0;
    __syncthreads();
  }
  ku32* qc = (ku32*)(a.q) + q0 * 2 * W;
  const uint32_t* I = reinterpret_cast<const uint32_t*>(a.items);
  const int64_t ntiles = (a.N + kWave - 1) / kWave;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * kLkWaves + wave; t < ntiles;
       t += static_cast<int64_t>(gridDim.x) * kLkWaves) {
    const int64_t row = t * kWave + lane;
    const bool valid = row < a.N;
    uint32_t iw[2 * W];
    lk_load<W>(I, valid ? row : a.N - 1, iw);
    for (int qi = 0; qi < nq; ++qi) {
      const int64_t q = q0 + qi;
      int h = 0;
#pragma unroll
      for (int d = 0; d < 2 * W; ++d) h = __builtin_popcount(iw[d] ^ qc[qi * 2 * W + d]) + h;
      bool ok = valid;
      if (ok && a.mask != nullptr) {
        ok = (a.mask[q * a.mask_words + (row >> 6)] >> (63 - (row & 63))) & 1ull;
      }
      if constexpr (MODE == 0) {
        if (ok) atomicAdd(&lh[qi * a.nb + h], 1u);
      } else {
        const int hs = a.cut[q * 8];
        if (!__any(ok && h <= hs)) continue;
        const uint64_t c = composite(key_of_i32(64 * W - 2 * h), static_cast<uint32_t>(row));
        if constexpr (MODE == 1) {
          if (ok && h < hs) {
            const int pos = atomicAdd(&a.cnt[q * 4], 1);
            if (pos < kLkCap) a.buf_a[q * kLkCap + pos] = c;
          } else if (ok && h == hs) {
            atomicAdd(&a.idhist[q * a.nbin + (row >> kLkIdShift)], 1u);
          }
        } else {
          const int64_t bs = a.cut[q * 8 + 3];
          const int64_t bin = row >> kLkIdShift;
          if (ok && h == hs && bin <= bs) {
            const int which = bin < bs ? 1 : 2;
            const int pos = atomicAdd(&a.cnt[q * 4 + which], 1);
            uint64_t* dst = which == 1 ? a.buf_b : a.buf_c;
            if (pos < kLkCap) dst[q * kLkCap + pos] = c;
          }
        }
      }
    }
  }
  if constexpr (MODE == 0) {
    __syncthreads();
    for (int i = threadIdx.x; i < nq * a.nb; i += kLkThreads) {
      const uint32_t v = lh[i];
      if (v != 0u) atomicAdd(&a.hist[(q0 + i / a.nb) * a.nb + i % a.nb], v);
    }
  }
}

// Inclusive prefix sum over the wave (64-bit: the counts of up to 2^32 items).
__device__ inline uint64_t lk_wave_scan(uint64_t x) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t y = __shfl_up(x, off);
    x += lane >= off ? y : 0ull;
  }
  return x;
}

// The first index of counts[0, n) at which the running sum reaches `want` (>= 1), and the sum
// before it (< want); n when the counts never reach it. One wave.
__device__ inline void lk_find(const uint32_t* counts, int64_t n, int want, int64_t* at,
                               int* before) {
  const int lane = lane_id();
  uint64_t run = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kWave) {
    const uint64_t v = c0 + lane < n ? counts[c0 + lane] : 0u;
    const uint64_t incl = lk_wave_scan(v);
    const uint64_t hit = __ballot(run + incl >= static_cast<uint64_t>(want));
    if (hit != 0ull) {
      const int f = __builtin_ctzll(hit);
      *at = c0 + f;
      *before = static_cast<int>(run + __shfl(incl - v, f));
      return;
    }
    run += __shfl(incl, kWave - 1);
  }
  *at = n;
  *before = static_cast<int>(run < static_cast<uint64_t>(want) ? run : want);
}

// Step 2: h*, lt, need per query (one wave each).
__global__ void __launch_bounds__(kWave) lk_cut_kernel(LkArgs a) {
  const int64_t q = blockIdx.x;
  const uint32_t* h = a.hist + q * a.nb;
  uint64_t total = 0;
  for (int i = lane_id(); i < a.nb; i += kWave) total += h[i];
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) total += __shfl_xor(total, off);
  const int kk = total < static_cast<uint64_t>(a.k) ? static_cast<int>(total) : a.k;
  int64_t hs = -1;  // no passing item: nothing is emitted
  int lt = 0;
  if (kk > 0) lk_find(h, a.nb, kk, &hs, &lt);
  if (lane_id() == 0) {
    a.cut[q * 8] = static_cast<int32_t>(hs);
    a.cut[q * 8 + 1] = lt;
    a.cut[q * 8 + 2] = kk - lt;
    a.cut[q * 8 + 3] = -1;
    a.cut[q * 8 + 4] = 0;
  }
}

// Step 4: b*, need2 per query (one wave each).
__global__ void __launch_bounds__(kWave) lk_cut2_kernel(LkArgs a) {
  const int64_t q = blockIdx.x;
  const int need = a.cut[q * 8 + 2];
  if (need <= 0) return;
  int64_t bs = 0;
  int before = 0;
  lk_find(a.idhist + q * a.nbin, a.nbin, need, &bs, &before);
  if (lane_id() == 0) {
    a.cut[q * 8 + 3] = static_cast<int32_t>(bs);
    a.cut[q * 8 + 4] = need - before;
  }
}

// Descending bitonic sort of s[0, n) (n a power of two) by the whole workgroup.
__device__ inline void lk_block_sort(uint64_t* s, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < (n >> 1); t += kLkFinalThreads) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint64_t x = s[i];
        const uint64_t y = s[j];
        if ((x < y) == desc) {
          s[i] = y;
          s[j] = x;
        }
      }
      __syncthreads();
    }
  }
}

__device__ inline int lk_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// Step 6: one workgroup per query.
__global__ void __launch_bounds__(kLkFinalThreads) lk_final_kernel(LkArgs a, int64_t* out_ids,
                                                                   void* out_scores,
                                                                   int score_kind) {
  extern __shared__ uint64_t sm[];
  uint64_t* tie = sm;             // [kLkCap]
  uint64_t* all = sm + kLkCap;    // [kLkCap]
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const int need2 = a.cut[q * 8 + 4];
  const int na = a.cnt[q * 4] < kLkCap ? a.cnt[q * 4] : kLkCap;  // == lt
  const int nb_ = a.cnt[q * 4 + 1] < kLkCap ? a.cnt[q * 4 + 1] : kLkCap;
  const int nc = a.cnt[q * 4 + 2] < kLkCap ? a.cnt[q * 4 + 2] : kLkCap;
  const int take = need2 < nc ? need2 : nc;
  if (take > 0) {
    const int p = lk_pow2(nc);
    for (int i = tid; i < p; i += kLkFinalThreads) tie[i] = i < nc ? a.buf_c[q * kLkCap + i] : 0ull;
    __syncthreads();
    lk_block_sort(tie, p);  // one score: descending composites = ascending ids
  }
  int n = na + nb_ + take;
  n = n < kLkCap ? n : kLkCap;
  const int p = lk_pow2(n > 0 ? n : 1);
  for (int i = tid; i < p; i += kLkFinalThreads) {
    uint64_t v = 0ull;
    if (i < na) {
      v = a.buf_a[q * kLkCap + i];
    } else if (i < na + nb_) {
      v = a.buf_b[q * kLkCap + (i - na)];
    } else if (i < n) {
      v = tie[i - na - nb_];
    }
    all[i] = v;
  }
  __syncthreads();
  lk_block_sort(all, p);
  for (int i = tid; i < a.k; i += kLkFinalThreads) {
    const int64_t o = q * a.k + i;
    if (i < n && all[i] != 0ull) {
      out_ids[o] = composite_item(all[i]);
      const int32_t s = i32_of_key(composite_key(all[i]));
      if (score_kind == kScoreI32) {
        static_cast<int32_t*>(out_scores)[o] = s;
      } else {
        static_cast<float*>(out_scores)[o] = static_cast<float>(s);
      }
    } else {
      out_ids[o] = -1;
      if (score_kind == kScoreI32) {
        static_cast<int32_t*>(out_scores)[o] = INT32_MIN;
      } else {
        static_cast<float*>(out_scores)[o] = -INFINITY;
      }
    }
  }
}

__global__ void __launch_bounds__(256) lk_zero_kernel(int32_t* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    p[i] = 0;
  }
}

struct LkLayout {
  size_t hist, cnt, idhist, zero_end, cut, a, b, c, total;
};

LkLayout lk_layout(int64_t B, int64_t N, int64_t W) {
  LkLayout l{};
  const int64_t nb = 64 * W + 1;
  const int64_t nbin = (N + (int64_t{1} << kLkIdShift) - 1) >> kLkIdShift;
  l.hist = 0;
  l.cnt = l.hist + static_cast<size_t>(B * nb) * 4;
  l.idhist = l.cnt + static_cast<size_t>(B) * 16;
  l.zero_end = l.idhist + static_cast<size_t>(B * (nbin > 0 ? nbin : 1)) * 4;
  l.cut = align_up(l.zero_end, 256);
  l.a = align_up(l.cut + static_cast<size_t>(B) * 32, 256);
  l.b = l.a + static_cast<size_t>(B) * kLkCap * 8;
  l.c = l.b + static_cast<size_t>(B) * kLkCap * 8;
  l.total = l.c + static_cast<size_t>(B) * kLkCap * 8;
  return l;
}

template <int W>
int lk_passes(const LkArgs& a, dim3 grid, hipStream_t stream, int mode) {
  if (mode == 0) {
    const size_t lds = static_cast<size_t>(kLkQpw) * a.nb * sizeof(int32_t);
    lk_pass_kernel<W, 0><<<grid, kLkThreads, lds, stream>>>(a);
  } else if (mode == 1) {
    lk_pass_kernel<W, 1><<<grid, kLkThreads, 0, stream>>>(a);
  } else {
    lk_pass_kernel<W, 2><<<grid, kLkThreads, 0, stream>>>(a);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

template <int W>
int lk_dispatch(int64_t w, const LkArgs& a, dim3 grid, hipStream_t stream, int mode) {
  if (w == W) return lk_passes<W>(a, grid, stream, mode);
  if constexpr (W < 16) {
    return lk_dispatch<W + 1>(w, a, grid, stream, mode);
  } else {
    set_error("Hamming scan supports W in [1, 16], got %lld", static_cast<long long>(w));
    return kInvalidArgument;
  }
}

}  // namespace

size_t hamming_large_k_workspace(int64_t B, int64_t N, int64_t W) {
  return lk_layout(B, N, W).total;
}

int hamming_large_k(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits, int64_t N,
                    int64_t W, int64_t k, const uint64_t* mask, int64_t mask_words,
                    int64_t* out_ids, void* out_scores, int score_kind, void* workspace,
                    size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(k > kMaxK && k <= kMaxKHamming, "k must be in (%lld, %lld] here",
               static_cast<long long>(kMaxK), static_cast<long long>(kMaxKHamming));
  const LkLayout l = lk_layout(B, N, W);
  if (workspace_bytes < l.total) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, l.total);
    return kWorkspaceTooSmall;
  }
  char* ws = static_cast<char*>(workspace);
  LkArgs a{};
  a.q = query_bits;
  a.B = B;
  a.items = item_bits;
  a.N = N;
  a.k = static_cast<int>(k);
  a.mask = mask;
  a.mask_words = mask_words;
  a.nb = static_cast<int>(64 * W + 1);
  a.nbin = (N + (int64_t{1} << kLkIdShift) - 1) >> kLkIdShift;
  a.hist = reinterpret_cast<uint32_t*>(ws + l.hist);
  a.cnt = reinterpret_cast<int32_t*>(ws + l.cnt);
  a.idhist = reinterpret_cast<uint32_t*>(ws + l.idhist);
  a.cut = reinterpret_cast<int32_t*>(ws + l.cut);
  a.buf_a = reinterpret_cast<uint64_t*>(ws + l.a);
  a.buf_b = reinterpret_cast<uint64_t*>(ws + l.b);
  a.buf_c = reinterpret_cast<uint64_t*>(ws + l.c);

  const int64_t nzero = static_cast<int64_t>(l.zero_end / 4);
  const int64_t zg = cdiv(nzero, 256) < 4096 ? cdiv(nzero, 256) : 4096;
  lk_zero_kernel<<<static_cast<unsigned>(zg), 256, 0, stream>>>(
      reinterpret_cast<int32_t*>(ws + l.hist), nzero);
  RT_CHECK_HIP(hipGetLastError());

  const int64_t tiles = cdiv(N, kWave);
  int64_t gx = cdiv(tiles, kLkWaves);
  gx = gx < kLkMaxGx ? gx : kLkMaxGx;
  const int64_t gy = cdiv(B, kLkQpw);
  RT_CHECK_ARG(gy <= 65535, "too many queries");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  int st = lk_dispatch<1>(W, a, grid, stream, 0);
  if (st != kOk) return st;
  lk_cut_kernel<<<static_cast<unsigned>(B), kWave, 0, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  st = lk_dispatch<1>(W, a, grid, stream, 1);
  if (st != kOk) return st;
  lk_cut2_kernel<<<static_cast<unsigned>(B), kWave, 0, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  st = lk_dispatch<1>(W, a, grid, stream, 2);
  if (st != kOk) return st;
  const size_t lds = 2 * kLkCap * sizeof(uint64_t);
  RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&lk_final_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(lds)));
  lk_final_kernel<<<static_cast<unsigned>(B), kLkFinalThreads, lds, stream>>>(
      a, out_ids, out_scores, score_kind);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

}  // namespace rt
