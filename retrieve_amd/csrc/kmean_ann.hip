// SilverTorch's raw scorer, st::fused_kmean_ann / st::fused_kmean_ann_with_partial_masks
// (silvertorch/silvertorch/ops/csrc/fused_kmean_ann_cuda.cu:2126-2501, schemas
// fused_kmean_ann.cpp:420-460): every probed doc's score written to its slot of a [B, width]
// buffer, with the doc's table position beside it.
//
// Slots (the reference's write indices, fused_kmean_ann_cuda.cu:592-598 for the full warps and
// :443-453 for the remainders): row b's probes p hold cluster_length[b, p] docs from
// cluster_offsets[cluster_ids[b, p]]; the full 32-doc warps of every probe come first, in probe
// order, then every probe's remaining docs, in probe order. A doc that fails the filter leaves its
// slot as a pad, as do slots past the row's docs: the score type's lowest value (INT32_MIN,
// fp16 -65504, bf16 / fp32 -max) and `invalid_index_value`. The reference requires a row's docs
// to fit `width`; slots past it are dropped here.
//
// Scores: int8 rows give the exact int32 dot; with divisor_for_int8 != -1, fp16(float(dot) /
// divisor) (index_mm_helpers.cuh:48-65); with a per-doc fp16 scale, fp16(float(fp16(dot)) /
// float(scale)), the reference's Half arithmetic. 16-bit and fp32 rows accumulate in fp32 and
// round once to the row type (the reference accumulates fp16 / bf16 in pairs of the row type,
// simple_index_mm.cuh:98-149, so those scores agree to the row type's rounding, not bit for bit).
//
// Layout: a group of L lanes (L * 16 bytes of a row per step) scores one slot, 64 / L slots a
// wave; the query row is staged in LDS; partial sums meet by xor-shuffles.
#include "profile.h"
#include "scan_common.h"

namespace rt {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kKmThreads = 256;
constexpr int kKmWaves = kKmThreads / kWave;
constexpr int kKmMaxProbe = 1024;
constexpr int kKmMaxRowBytes = 8192;

enum KmElem : int { kElemI8 = 0, kElemBf16 = 1, kElemF16 = 2, kElemF32 = 3 };
enum KmOut : int { kOutI32 = 0, kOutF16 = 1, kOutBf16 = 2, kOutF32 = 3 };
constexpr int kKeepF32 = 16;

struct KmArgs {
  const int8_t* queries;  // [B, RB]
  const int8_t* emb;      // [N, RB]
  int64_t B;
  int64_t N;
  int RB;
  int L;  // lanes per slot (a power of two, L * 16 <= RB rounded up)
  const int64_t* cluster_offsets;
  int64_t n_offsets;
  const int64_t* cluster_ids;     // [B, P]
  const int64_t* cluster_length;  // [B, P]
  int64_t P;
  int64_t width;
  // a full-N mask: row mask_index[b] (or b) of [mask_rows, mask_words], doc d at bit 63 - d % 64
  const uint64_t* mask;
  int64_t mask_rows;
  int64_t mask_words;
  const int64_t* mask_index;
  // partial masks (the Bloom search over the probed clusters' columns): cluster entry
  // e = mask_row * P + p spans words pcum[e - 1] .. pcum[e) of pwords, its first doc at bit
  // position pfirst[e] of the first word
  const int32_t* pcum;
  const int8_t* pfirst;
  const uint64_t* pwords;
  int64_t p_entries;
  int64_t p_words;
  int divisor;                // -1: none
  const uint16_t* scale16;    // [N] fp16 per-doc scales, or null
  int32_t invalid;
  int out_kind;
  void* out_scores;  // [B, width]
  int32_t* out_idx;  // [B, width]
};

__device__ inline float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
__device__ inline float f16_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
__device__ inline float f16_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// The slot's ranges (as search.hip's load_ranges, with per-row lengths): range j < P is probe
// j's full warps, range P + j its remainder; start[r] the first position, prefix[r] the slots
// before it (clamped at width). start[j] (j < P) is also probe j's cluster start, from which the
// partial masks count docs.
__device__ inline int64_t km_ranges(const KmArgs& a, int64_t b, int64_t* start, int64_t* prefix) {
  const int tid = threadIdx.x;
  const int64_t np = a.P;
  for (int64_t j = tid; j < np; j += blockDim.x) {
    const int64_t c = a.cluster_ids[b * np + j];
    int64_t s = 0;
    int64_t len = 0;
    if (c >= 0 && c < a.n_offsets) {
      s = a.cluster_offsets[c];
      len = a.cluster_length[b * np + j];
      if (s < 0 || len < 0 || s > a.N || len > a.N - s) len = 0;
    }
    const int64_t full = len / 32 * 32;
    start[j] = s;
    prefix[j + 1] = full;
    start[np + j] = s + full;
    prefix[np + j + 1] = len - full;
  }
  __syncthreads();
  if (tid == 0) {
    prefix[0] = 0;
    for (int64_t r = 0; r < 2 * np; ++r) {
      const int64_t t = prefix[r] + prefix[r + 1];
      prefix[r + 1] = t < a.width ? t : a.width;
    }
  }
  __syncthreads();
  return prefix[2 * np];
}

__device__ inline int64_t km_range_of(const int64_t* prefix, int64_t n, int64_t s) {
  int64_t lo = 0;
  int64_t hi = n - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= s) {
      lo = mid;
    } else {
      hi = mid - 1;
    }
  }
  return lo;
}

__device__ inline void km_store(const KmArgs& a, int64_t at, int32_t dot, float acc, int64_t pos,
                                bool written) {
  switch (a.out_kind) {
    case kOutI32:
      static_cast<int32_t*>(a.out_scores)[at] = written ? dot : INT32_MIN;
      break;
    case kOutF16: {
      uint16_t bits = 0xfbffu;  // -65504
      if (written) {
        _Float16 h;
        if (a.scale16 != nullptr) {
          const _Float16 hd = static_cast<_Float16>(static_cast<float>(dot));
          const float sc = static_cast<float>(
              __builtin_bit_cast(_Float16, a.scale16[pos]));
          h = static_cast<_Float16>(static_cast<float>(hd) / sc);
        } else if (a.divisor != -1) {
          h = static_cast<_Float16>(static_cast<float>(dot) / static_cast<float>(a.divisor));
        } else {
          h = static_cast<_Float16>(acc);
        }
        bits = __builtin_bit_cast(uint16_t, h);
      }
      static_cast<uint16_t*>(a.out_scores)[at] = bits;
      break;
    }
    case kOutBf16: {
      uint16_t bits = 0xff7fu;  // the lowest finite bf16
      if (written) bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(acc));
      static_cast<uint16_t*>(a.out_scores)[at] = bits;
      break;
    }
    default:
      static_cast<float*>(a.out_scores)[at] = written ? acc : -3.40282347e+38f;
      break;
  }
  a.out_idx[at] = written ? static_cast<int32_t>(pos) : a.invalid;
}

template <int ELEM>
__global__ void __launch_bounds__(kKmThreads) fused_kmean_ann_kernel(KmArgs a) {
  extern __shared__ __attribute__((aligned(16))) int64_t kmem[];
  const int64_t nr = 2 * a.P;
  // the query row first (16-byte aligned, RB a multiple of 16), then the ranges
  int8_t* qs = reinterpret_cast<int8_t*>(kmem);
  int64_t* start = reinterpret_cast<int64_t*>(qs + a.RB);
  int64_t* prefix = start + nr;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int L = a.L;
  const int R = kWave / L;
  const int grp = lane / L;
  const int gl = lane % L;
  const int nchunks = a.RB / 16;

  for (int c = tid; c < nchunks; c += kKmThreads) {
    reinterpret_cast<v4i*>(qs)[c] = reinterpret_cast<const v4i*>(a.queries + b * a.RB)[c];
  }
  const int64_t total = km_ranges(a, b, start, prefix);  // (its barriers cover the staging)

  int64_t mrow = b;
  if (a.mask_index != nullptr) mrow = a.mask_index[b];
  const uint64_t* mwords = nullptr;
  if (a.mask != nullptr && mrow >= 0 && mrow < a.mask_rows) mwords = a.mask + mrow * a.mask_words;

  const int64_t step = static_cast<int64_t>(gridDim.x) * kKmWaves * R;
  for (int64_t base = (static_cast<int64_t>(blockIdx.x) * kKmWaves + wave) * R;
       base < a.width; base += step) {
    const int64_t s = base + grp;
    bool ok = s < total;
    int64_t pos = 0;
    if (ok) {
      const int64_t j = km_range_of(prefix, nr, s);
      pos = start[j] + (s - prefix[j]);
      if (a.mask != nullptr) {
        ok = mwords != nullptr && (pos >> 6) < a.mask_words &&
             ((mwords[pos >> 6] >> (63 - (pos & 63))) & 1ull);
      } else if (a.pwords != nullptr) {
        const int64_t p = j < a.P ? j : j - a.P;
        const int64_t e = mrow * a.P + p;
        ok = mrow >= 0 && e < a.p_entries;
        if (ok) {
          const int64_t w0 = e == 0 ? 0 : static_cast<int64_t>(a.pcum[e - 1]);
          const int64_t bit = static_cast<int64_t>(a.pfirst[e]) + (pos - start[p]);
          const int64_t w = w0 + (bit >> 6);
          ok = bit >= 0 && w >= 0 && w < a.p_words &&
               ((a.pwords[w] >> (63 - (bit & 63))) & 1ull);
        }
      }
    }
    int32_t dot = 0;
    float acc = 0.f;
    if (ok) {
      const int8_t* row = a.emb + pos * a.RB;
      for (int c = gl; c < nchunks; c += L) {
        const v4i x = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row) + c);
        const v4i q = reinterpret_cast<const v4i*>(qs)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t xe = static_cast<uint32_t>(x[e]);
          const uint32_t qe = static_cast<uint32_t>(q[e]);
          if constexpr (ELEM == kElemI8) {
            dot = __builtin_amdgcn_sdot4(x[e], q[e], dot, false);
          } else if constexpr (ELEM == kElemBf16) {
            acc = __builtin_fmaf(bf16_lo(xe), bf16_lo(qe), acc);
            acc = __builtin_fmaf(bf16_hi(xe), bf16_hi(qe), acc);
          } else if constexpr (ELEM == kElemF16) {
            acc = __builtin_fmaf(f16_lo(xe), f16_lo(qe), acc);
            acc = __builtin_fmaf(f16_hi(xe), f16_hi(qe), acc);
          } else {
            acc = __builtin_fmaf(__builtin_bit_cast(float, xe), __builtin_bit_cast(float, qe),
                                 acc);
          }
        }
      }
    }
    for (int off = L / 2; off > 0; off >>= 1) {
      if constexpr (ELEM == kElemI8) {
        dot += __shfl_xor(dot, off);
      } else {
        acc += __shfl_xor(acc, off);
      }
    }
    if (gl == 0 && s < a.width) km_store(a, b * a.width + s, dot, acc, pos, ok);
  }
}

}  // namespace
}  // namespace rt

using namespace rt;

extern "C" int rt_fused_kmean_ann(
    const void* queries, const void* embeddings, int elem, int64_t B, int64_t N, int64_t D,
    const int64_t* cluster_offsets, int64_t n_offsets, const int64_t* cluster_ids,
    const int64_t* cluster_length, int64_t n_probe, int64_t width, const uint64_t* mask,
    int64_t mask_rows, int64_t mask_words, const int64_t* mask_index,
    const int32_t* partial_counts_cumsum, const int8_t* partial_first_offsets,
    const uint64_t* partial_words, int64_t partial_entries, int64_t partial_n_words,
    int64_t divisor, const uint16_t* per_embedding_scale, int64_t invalid_index, void* out_scores,
    int32_t* out_indices, hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0 && n_probe >= 0 && n_offsets >= 0 && width >= 0,
               "sizes must be >= 0");
  // elem + kKeepF32: float rows store their fp32 accumulators (the library's top-k above 1024)
  const bool keep_f32 = elem >= kKeepF32;
  if (keep_f32) elem -= kKeepF32;
  RT_CHECK_ARG(elem >= kElemI8 && elem <= kElemF32 && !(keep_f32 && elem == kElemI8),
               "element kind must be 0-3, or 17-19 for fp32 scores of float rows");
  const int64_t esz = elem == kElemI8 ? 1 : (elem == kElemF32 ? 4 : 2);
  const int64_t rb = D * esz;
  RT_CHECK_ARG(D >= 1 && rb % 16 == 0 && rb <= kKmMaxRowBytes,
               "rows must be a multiple of 16 bytes, at most %d (D = %lld)", kKmMaxRowBytes,
               static_cast<long long>(D));
  RT_CHECK_ARG(n_probe <= kKmMaxProbe, "at most %d probes per row, got %lld", kKmMaxProbe,
               static_cast<long long>(n_probe));
  RT_CHECK_ARG(N < (int64_t{1} << 31), "N must be < 2**31 (int32 indices)");
  RT_CHECK_ARG(divisor == -1 || (divisor >= 1 && divisor < (int64_t{1} << 31)),
               "divisor_for_int8 must be -1 or positive");
  RT_CHECK_ARG(mask == nullptr || partial_words == nullptr, "one mask at most");
  RT_CHECK_ARG(B <= 65535, "B must be <= 65535");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(embeddings) % 16 == 0,
               "queries and embeddings must be 16-byte aligned");
  if (B == 0 || width == 0) return kOk;
  RT_CHECK_ARG(out_scores != nullptr && out_indices != nullptr, "outputs must not be null");
  RT_CHECK_ARG(n_probe == 0 || (queries != nullptr && embeddings != nullptr &&
                                cluster_offsets != nullptr && cluster_ids != nullptr &&
                                cluster_length != nullptr),
               "inputs must not be null");
  KmArgs a{};
  a.queries = static_cast<const int8_t*>(queries);
  a.emb = static_cast<const int8_t*>(embeddings);
  a.B = B;
  a.N = N;
  a.RB = static_cast<int>(rb);
  int lanes = 1;
  while (lanes < kWave && lanes * 16 < rb) lanes <<= 1;
  a.L = lanes;
  a.cluster_offsets = cluster_offsets;
  a.n_offsets = n_offsets;
  a.cluster_ids = cluster_ids;
  a.cluster_length = cluster_length;
  a.P = n_probe;
  a.width = width;
  a.mask = mask;
  a.mask_rows = mask_rows;
  a.mask_words = mask_words;
  a.mask_index = mask_index;
  a.pcum = partial_counts_cumsum;
  a.pfirst = partial_first_offsets;
  a.pwords = partial_words;
  a.p_entries = partial_entries;
  a.p_words = partial_n_words;
  // (the divisor and the per-doc scales apply to int8 rows only)
  a.divisor = elem == kElemI8 ? static_cast<int>(divisor) : -1;
  a.scale16 = elem == kElemI8 ? per_embedding_scale : nullptr;
  a.invalid = static_cast<int32_t>(invalid_index);
  if (elem == kElemI8) {
    a.out_kind = (divisor == -1 && per_embedding_scale == nullptr) ? kOutI32 : kOutF16;
  } else {
    a.out_kind = keep_f32 ? kOutF32
                          : (elem == kElemBf16 ? kOutBf16 : (elem == kElemF16 ? kOutF16 : kOutF32));
  }
  a.out_scores = out_scores;
  a.out_idx = out_indices;
  // slots per workgroup row: enough workgroups to cover the widest row a few times over
  const int64_t per_wg = static_cast<int64_t>(kKmWaves) * (kWave / lanes) * 8;
  int64_t gx = cdiv(width, per_wg);
  const int64_t cap = cdiv(4096, B);
  gx = gx < cap ? gx : cap;
  gx = gx < 1 ? 1 : gx;
  const size_t lds = static_cast<size_t>(4 * n_probe + 1) * sizeof(int64_t) + rb;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(B));
  hipEvent_t stop;
  profile_begin(stream, &stop);
  switch (elem) {
    case kElemI8:
      fused_kmean_ann_kernel<kElemI8><<<grid, kKmThreads, lds, stream>>>(a);
      break;
    case kElemBf16:
      fused_kmean_ann_kernel<kElemBf16><<<grid, kKmThreads, lds, stream>>>(a);
      break;
    case kElemF16:
      fused_kmean_ann_kernel<kElemF16><<<grid, kKmThreads, lds, stream>>>(a);
      break;
    default:
      fused_kmean_ann_kernel<kElemF32><<<grid, kKmThreads, lds, stream>>>(a);
      break;
  }
  profile_end(stream, stop);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
