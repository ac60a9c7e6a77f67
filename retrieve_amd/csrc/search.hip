// SilverTorch's search after phase 1 (silvertorch/.../ops/csrc/fork_search_cuda.cu:1256-1524):
// query quantization, the int8 scorer over each query's probed clusters, the selection by
// (key desc, slot asc) and the epilogue id = sort_perm[position], score = dequantized dot.
//
// Slots: query row b's probed clusters c_j = probe_ids[b, j] hold the items at sorted positions
// cluster_offsets[c_j] .. + cluster_sizes[c_j]. The row's slots are the reference scorer's write
// order: the full 32-item warps of every probed cluster in probe order, then every cluster's
// remaining (< 32) items in probe order (fork_search_cuda.cu:989-991 and :1051-1053;
// fused_kmean_ann_cuda.cu:592-598 and :443-453). Ties go to the lower slot. The row holds at most
// `width` slots (max_tensor_size_per_row rounded up to 32, as the reference's score buffer); the
// reference requires a row's clusters to fit its width, and slots at or past it are dropped here.
// A filtered-out item keeps its slot (the scorer skips it), so the filter never renumbers slots.
//
// Keys: the int32 dot (divisor -1), or the fp16 score fp16(float(dot) / divisor) of the serving
// path (index_mm_helpers.cuh:48-65), ordered as fp16 values (ties merge distinct dots).
//
// The range scan is the candidate kernel's layout: a group of L lanes loads one item row with
// 16-byte loads and reduces its v_dot4 partial sums by xor-shuffles; every wave keeps a
// candidate list under a rising threshold; the shared merge picks the k best composites.
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kQuantThreads = 256;
constexpr int kIvfThreads = 256;
constexpr int kIvfWaves = kIvfThreads / kWave;
constexpr int kIvfMaxProbe = 1024;
constexpr int kIvfMaxWgsPerRow = 64;

// ---- query quantization (A1 / A2) ------------------------------------------------------------

// Per row: abs_max = max(max |x|, 1e-8); scale = abs_max * fp32(1/127); code =
// clamp(rint(fp32(fp64(x) / fp64(abs_max)) * 127), -128, 127) (fork_search_cuda.cu:680-699;
// retrieve/src/retrieve/indexing/quantize.py:9-18). One workgroup per row.
// scale_div: scales = abs_max / 127 (quantize_int8, indexing/quantize.py:9-18); else
// abs_max * fp32(1/127) (probe_prep_kernel, fork_search_cuda.cu:689). The codes are the same.
__global__ void __launch_bounds__(kQuantThreads) quantize_rows_kernel(const float* x,
                                                                      int64_t dim, int8_t* codes,
                                                                      float* scales,
                                                                      int scale_div) {
  __shared__ float red[kQuantThreads / kWave];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * dim;
  float m = 0.f;
  for (int64_t d = threadIdx.x; d < dim; d += kQuantThreads) m = fmaxf(m, fabsf(xr[d]));
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane_id() == 0) red[threadIdx.x / kWave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < kQuantThreads / kWave; ++w) m = fmaxf(m, red[w]);
  m = fmaxf(m, 1e-8f);
  if (threadIdx.x == 0) scales[row] = scale_div ? m / 127.0f : m * (1.0f / 127.0f);
  const double a = static_cast<double>(m);
  int8_t* out = codes + row * dim;
  for (int64_t d = threadIdx.x; d < dim; d += kQuantThreads) {
    float v = static_cast<float>(static_cast<double>(xr[d]) / a) * 127.0f;
    v = fminf(fmaxf(rintf(v), -128.0f), 127.0f);
    out[d] = static_cast<int8_t>(v);
  }
}

// One scale for the whole table (quantize_int8_global, retrieve/src/retrieve/indexing/quantize.py:
// 25-52): abs_max = max(max x, -min x) floored at 1e-8 (fabsf's maximum, the same value), code
// = clamp(rint(fp32(x / abs_max) * 127), -128, 127) in fp32, row i of the codes from row
// perm[i] of x when a permutation is given. NaN inputs are outside the contract (max ignores
// them here; the reference's int8 cast of a NaN code is unspecified).
constexpr int kGlobalThreads = 256;

__global__ void abs_max_init_kernel(uint32_t* bits) { bits[0] = 0u; }

// Grid-stride max |x| over n floats, 16-byte loads when x is 16-byte aligned; one atomic per
// workgroup on the bits of the (non-negative) float, whose unsigned order is the float order.
__global__ void __launch_bounds__(kGlobalThreads) abs_max_kernel(const float* x, int64_t n,
                                                                 uint32_t* bits) {
  __shared__ float red[kGlobalThreads / kWave];
  float m = 0.f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGlobalThreads;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kGlobalThreads + threadIdx.x;
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    const int64_t n4 = n / 4;
    for (int64_t i = t0; i < n4; i += stride) {
      const v4f v = __builtin_nontemporal_load(x4 + i);
      m = fmaxf(fmaxf(m, fmaxf(fabsf(v[0]), fabsf(v[1]))), fmaxf(fabsf(v[2]), fabsf(v[3])));
    }
    for (int64_t i = 4 * n4 + t0; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
  } else {
    for (int64_t i = t0; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane_id() == 0) red[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kGlobalThreads / kWave; ++w) m = fmaxf(m, red[w]);
    atomicMax(bits, __float_as_uint(m));
  }
}

__global__ void __launch_bounds__(kGlobalThreads) quantize_global_kernel(
    const float* x, int64_t rows, int64_t dim, const int64_t* perm, const uint32_t* bits,
    int8_t* codes, float* abs_max_out) {
  const float m = fmaxf(__uint_as_float(bits[0]), 1e-8f);
  const int64_t total = rows * dim;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGlobalThreads;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kGlobalThreads + threadIdx.x;
  if (t0 == 0) abs_max_out[0] = m;
  for (int64_t i = t0; i < total; i += stride) {
    const int64_t r = i / dim;
    const int64_t c = i - r * dim;
    const int64_t src = perm != nullptr ? perm[r] : r;
    float v = (x[src * dim + c] / m) * 127.0f;
    v = fminf(fmaxf(rintf(v), -128.0f), 127.0f);
    codes[i] = static_cast<int8_t>(v);
  }
}

// Sign bits of float rows, LSB-first: bit b of word w of row r is x[r, 64 w + b] > 0
// (_pack_signs_to_int64, retrieve/src/retrieve/indexing/quantize.py:63-72). One wave per word:
// lane b reads element 64 w + b and the ballot is the word (NaN and -0 give 0 bits, as the
// reference's comparison does).
__global__ void __launch_bounds__(256) pack_signs_kernel(const float* x, int64_t words_total,
                                                         uint64_t* words) {
  const int64_t w = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / kWave;
  if (w >= words_total) return;  // whole waves
  const bool pos = x[w * kWave + lane_id()] > 0.0f;
  const uint64_t word = __ballot(pos);
  if (lane_id() == 0) words[w] = word;
}

// ---- range scan ------------------------------------------------------------------------------

struct IvfArgs {
  const int8_t* q;  // [B, RB] codes
  int64_t B;
  const int8_t* items;  // [N, RB]
  int64_t N;
  int RB;
  const int64_t* probe_ids;  // [B, n_probe]
  int64_t n_probe;
  const int64_t* cluster_offsets;  // [n_lists]
  const int64_t* cluster_sizes;    // [n_lists]
  int64_t n_lists;
  int64_t width;
  const uint64_t* mask;  // [B, mask_words], item position d at bit 63 - d % 64, or null
  int64_t mask_words;
  // or the probed payloads' Bloom words (rt_bloom_search_columns' layout): entry e = b * n_probe
  // + j covers probe j's docs from bit pfirst[e] of words pcum[e - 1] ... (null: none)
  const int32_t* pcum;
  const int8_t* pfirst;
  const uint64_t* pwords;
  int64_t p_entries;
  int64_t p_words;
  // and / or the exact clauses in the slot layout (slots [R, N] int32, clause c in rows
  // cslots[c] .. cslots[c + 1], query values qv [B, C], -1 inactive; null: none)
  const int32_t* slots;
  int64_t R;
  const int64_t* cslots;
  int C;
  const int8_t* reverse;  // [C], non-zero: a reverse clause
  const int32_t* qv;
  int divisor;  // -1: int32 keys
  int k;
  int capw;
  uint64_t* lists;
  int* list_counts;
};

// The row's 2 n_probe slot ranges in slot order: range j < n_probe is probe j's full warps
// (its first len_j / 32 * 32 items), range n_probe + j probe j's remaining len_j % 32 items.
// start[r] is range r's first sorted position and prefix[r] the slots before it (prefix[2n] =
// total, clamped at width). Invalid clusters, or clusters reaching outside the table, are empty.
__device__ inline int64_t load_ranges(const IvfArgs& a, int64_t b, int64_t* start,
                                      int64_t* prefix) {
  const int tid = threadIdx.x;
  const int64_t np = a.n_probe;
  for (int64_t j = tid; j < np; j += blockDim.x) {
    const int64_t c = a.probe_ids[b * np + j];
    int64_t s = 0;
    int64_t len = 0;
    if (c >= 0 && c < a.n_lists) {
      s = a.cluster_offsets[c];
      len = a.cluster_sizes[c];
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

// LDS bytes of a row's ranges (start[2 n], prefix[2 n + 1]).
inline size_t ranges_lds(int64_t n_probe) {
  return static_cast<size_t>(4 * n_probe + 1) * sizeof(int64_t);
}

// the range holding slot s: the last j with prefix[j] <= s
__device__ inline int64_t range_of(const int64_t* prefix, int64_t n, int64_t s) {
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

__device__ inline uint32_t search_key(int32_t dot, int divisor) {
  if (divisor == -1) return key_of_i32(dot);
  const _Float16 h = static_cast<_Float16>(static_cast<float>(dot) / static_cast<float>(divisor));
  return key_of_f32(static_cast<float>(h));
}

// Bit `off` of probe j's payload in row b's Bloom words (out of range: no match), as
// fused_kmean_ann_with_partial_masks reads it (fused_kmean_ann_cuda.cu:2264-2501).
__device__ inline bool payload_bit(const IvfArgs& a, int64_t b, int64_t j, int64_t off) {
  const int64_t e = b * a.n_probe + j;
  if (e >= a.p_entries) return false;
  const int64_t w0 = e == 0 ? 0 : static_cast<int64_t>(a.pcum[e - 1]);
  const int64_t bit = static_cast<int64_t>(a.pfirst[e]) + off;
  const int64_t w = w0 + (bit >> 6);
  return bit >= 0 && w < a.p_words && ((a.pwords[w] >> (63 - (bit & 63))) & 1ull);
}

// The exact recheck of one probed doc (fork_filters.cuh:15-41): every active clause matches
// (one of the doc's values equals the query's), negated for a reverse clause.
__device__ inline bool exact_pass(const IvfArgs& a, int64_t b, int64_t pos, uint32_t rev_mask) {
  const int32_t* q = a.qv + b * a.C;
  uint32_t active = 0;
  uint32_t match = 0;
  for (int c = 0; c < a.C; ++c) {
    const int32_t v = q[c];
    if (v == -1) continue;
    active |= 1u << c;
    bool eq = false;
    const int64_t r0 = a.cslots[c] > 0 ? a.cslots[c] : 0;
    const int64_t r1 = a.cslots[c + 1] < a.R ? a.cslots[c + 1] : a.R;  // rows inside the table
    for (int64_t r = r0; r < r1; ++r) eq |= a.slots[r * a.N + pos] == v;
    match |= eq ? 1u << c : 0u;
  }
  return ((match ^ rev_mask) & active) == active;
}

template <int L, int NC>
__global__ void __launch_bounds__(kIvfThreads) ivf_scan_kernel(IvfArgs a) {
  constexpr int R = kWave / L;
  extern __shared__ uint64_t smem[];
  const int64_t nr = 2 * a.n_probe;  // slot ranges
  int64_t* start = reinterpret_cast<int64_t*>(smem);
  int64_t* prefix = start + nr;
  uint64_t* scratch = reinterpret_cast<uint64_t*>(prefix + nr + 1);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int grp = lane / L;
  const int gl = lane % L;
  int* cnt_lds = reinterpret_cast<int*>(scratch + kIvfWaves * a.capw);
  const int64_t b = blockIdx.y;
  const int64_t gx = gridDim.x;
  const int64_t S = gx * kIvfWaves;
  const int64_t slot_list = static_cast<int64_t>(blockIdx.x) * kIvfWaves + wave;
  uint64_t* list = a.lists + (b * S + slot_list) * a.capw;
  scratch += wave * a.capw;

  const int64_t total = load_ranges(a, b, start, prefix);
  const int nchunks = a.RB / 16;
  v4i qv[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = gl + j * L;
    qv[j] = c < nchunks ? *reinterpret_cast<const v4i*>(a.q + b * a.RB + c * 16)
                        : v4i{0, 0, 0, 0};
  }
  const uint64_t* mrow = a.mask != nullptr ? a.mask + b * a.mask_words : nullptr;
  uint32_t rev_mask = 0;
  if (a.qv != nullptr) {
    for (int c = 0; c < a.C; ++c) rev_mask |= a.reverse[c] != 0 ? 1u << c : 0u;
  }

  uint64_t tau = 0;
  int cnt = 0;
  const int64_t step = gx * kIvfWaves * R;
  for (int64_t base = slot_list * R; base < total; base += step) {
    const int64_t s = base + grp;
    bool ok = s < total;
    int64_t pos = 0;
    if (ok) {
      const int64_t j = range_of(prefix, nr, s);
      pos = start[j] + (s - prefix[j]);
      if (mrow != nullptr) {
        ok = (mrow[pos >> 6] >> (63 - (pos & 63))) & 1ull;
      } else if (a.pwords != nullptr) {
        const int64_t p = j < a.n_probe ? j : j - a.n_probe;  // the probe of range j
        ok = payload_bit(a, b, p, pos - start[p]);
      }
      if (ok && a.qv != nullptr) ok = exact_pass(a, b, pos, rev_mask);
    }
    int32_t dot = 0;
    if (ok) {
      const int8_t* row = a.items + pos * a.RB;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = gl + j * L;
        if (c < nchunks) {
          const v4i x = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row + c * 16));
#pragma unroll
          for (int e = 0; e < 4; ++e) dot = __builtin_amdgcn_sdot4(x[e], qv[j][e], dot, false);
        }
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
    const uint64_t c = composite(search_key(dot, a.divisor), static_cast<uint32_t>(s));
    const bool keep = ok && gl == 0 && c >= tau;
    const uint64_t bal = __ballot(keep);
    if (bal != 0ull) {
      const int before = __popcll(bal & ((1ull << lane) - 1ull));
      if (keep) list[cnt + before] = c;
      cnt += __popcll(bal);
      if (cnt > a.capw - R) {
        if (lane == 0) cnt_lds[wave] = cnt;
        const uint64_t nt = wave_compact(list, &cnt_lds[wave], scratch, a.capw, a.k);
        cnt = cnt_lds[wave];
        tau = nt > tau ? nt : tau;
      }
    }
  }
  if (lane == 0) a.list_counts[b * S + slot_list] = cnt;
}

// ---- epilogue -------------------------------------------------------------------------------

struct EpiArgs {
  int64_t* ids;     // in: slots (ranges) or positions, -1 empty; out: sort_perm ids
  const void* raw;  // [B, k] int32 dots, or float fp16 scores
  float* scores;    // out [B, k]
  int64_t B;
  int64_t k;
  bool ranges;  // ids are slots of the probed ranges (else item positions)
  IvfArgs a;    // the ranges (when `ranges`)
  const int64_t* sort_perm;
  int64_t n_perm;
  const float* q_scales;
  const float* global_scale;
  int divisor;
};

// One workgroup per row. Scores (fork_search_cuda.cu:585-591): int32 path
// (fp32(dot) * q_scale) * global_scale; fp16 path score16 * ((q_scale * divisor) *
// global_scale), each product rounded to nearest.
__global__ void __launch_bounds__(kIvfThreads) search_epilogue_kernel(EpiArgs e) {
  extern __shared__ uint64_t smem[];
  const int64_t b = blockIdx.x;
  const int64_t nr = e.ranges ? 2 * e.a.n_probe : 0;  // slot ranges
  int64_t* start = reinterpret_cast<int64_t*>(smem);
  int64_t* prefix = start + nr;
  if (e.ranges) load_ranges(e.a, b, start, prefix);
  const float qs = e.q_scales[b];
  const float gs = e.global_scale[0];
  for (int64_t i = threadIdx.x; i < e.k; i += blockDim.x) {
    const int64_t x = e.ids[b * e.k + i];
    int64_t id = -1;
    float score = -INFINITY;
    if (x >= 0) {
      int64_t pos = x;
      if (e.ranges) {
        const int64_t j = range_of(prefix, nr, x);
        pos = start[j] + (x - prefix[j]);
      }
      if (pos >= 0 && pos < e.n_perm) {
        id = e.sort_perm[pos];
        if (e.divisor == -1) {
          const float dot = static_cast<float>(static_cast<const int32_t*>(e.raw)[b * e.k + i]);
          score = __fmul_rn(__fmul_rn(dot, qs), gs);
        } else {
          const float s16 = static_cast<const float*>(e.raw)[b * e.k + i];
          score = __fmul_rn(s16, __fmul_rn(__fmul_rn(qs, static_cast<float>(e.divisor)), gs));
        }
      }
    }
    e.ids[b * e.k + i] = id;
    e.scores[b * e.k + i] = score;
  }
}

template <int L, int NC>
static void launch_ivf(const IvfArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  if (lds > 64 * 1024) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&ivf_scan_kernel<L, NC>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  }
  ivf_scan_kernel<L, NC><<<grid, kIvfThreads, lds, stream>>>(a);
}

static int ivf_capw(int64_t k) { return static_cast<int>(next_pow2(k + kWave)); }

static int64_t ivf_gx(int64_t B, int64_t width) {
  int64_t gx = cdiv(2048, B > 0 ? B : 1);
  const int64_t by_rows = cdiv(width, 1024);
  gx = gx < by_rows ? gx : by_rows;
  gx = gx < 1 ? 1 : gx;
  return gx < kIvfMaxWgsPerRow ? gx : kIvfMaxWgsPerRow;
}

}  // namespace rt

using namespace rt;

extern "C" int rt_quantize_int8_rows(const float* x, int64_t rows, int64_t dim, int8_t* codes,
                                     float* scales, int scale_div, hipStream_t stream) {
  RT_CHECK_ARG(rows >= 0 && dim >= 1, "rows must be >= 0 and dim >= 1");
  RT_CHECK_ARG(rows <= (int64_t{1} << 31) - 1, "too many rows");
  if (rows == 0) return kOk;
  quantize_rows_kernel<<<static_cast<unsigned>(rows), kQuantThreads, 0, stream>>>(
      x, dim, codes, scales, scale_div);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_quantize_int8_global(const float* x, int64_t rows, int64_t dim,
                                       const int64_t* perm, int8_t* codes, float* abs_max,
                                       uint32_t* scratch4, hipStream_t stream) {
  RT_CHECK_ARG(rows >= 0 && dim >= 1, "rows must be >= 0 and dim >= 1");
  RT_CHECK_ARG(abs_max != nullptr && scratch4 != nullptr, "abs_max and scratch4 must be given");
  RT_CHECK_ARG(rows == 0 || (x != nullptr && codes != nullptr), "x and codes must not be null");
  const int64_t total = rows * dim;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  }
  const int64_t want = cdiv(total, kGlobalThreads * 4);
  const unsigned grid = static_cast<unsigned>(want < 8 * cus ? (want > 0 ? want : 1) : 8 * cus);
  abs_max_init_kernel<<<1, 1, 0, stream>>>(scratch4);
  if (total > 0) abs_max_kernel<<<grid, kGlobalThreads, 0, stream>>>(x, total, scratch4);
  quantize_global_kernel<<<grid, kGlobalThreads, 0, stream>>>(x, rows, dim, perm, scratch4,
                                                              codes, abs_max);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_pack_signs(const float* x, int64_t rows, int64_t dim, uint64_t* words,
                             hipStream_t stream) {
  RT_CHECK_ARG(rows >= 0 && dim >= 1, "rows must be >= 0 and dim >= 1");
  RT_CHECK_ARG(dim % 64 == 0, "dim must be a multiple of 64, got %lld",
               static_cast<long long>(dim));
  const int64_t total = rows * (dim / 64);
  if (total == 0) return kOk;
  const int64_t blocks = cdiv(total * kWave, 256);
  RT_CHECK_ARG(blocks < (int64_t{1} << 31), "too many rows");
  pack_signs_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(x, total, words);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" size_t rt_ivf_search_workspace(int64_t B, int64_t width, int64_t k) {
  if (B <= 0 || k <= 0) return 256;
  const int64_t S = ivf_gx(B, width) * kIvfWaves;
  return align_up(static_cast<size_t>(B * S) * ivf_capw(k) * sizeof(uint64_t), 256) +
         align_up(static_cast<size_t>(B * S) * sizeof(int), 256) +
         align_up(static_cast<size_t>(B * k) * sizeof(float), 256);
}

// Top-k over each row's probed ranges of int8 codes (slots, ties to the lower slot), then the
// epilogue: out_ids = sort_perm[position] (-1 pads), out_scores dequantized (-inf pads).
static int ivf_search(const int8_t* q_codes, const float* q_scales, int64_t B,
                      const int8_t* item_codes, int64_t N, int64_t D, const int64_t* probe_ids,
                      int64_t n_probe, const int64_t* cluster_offsets,
                      const int64_t* cluster_sizes, int64_t n_lists, int64_t width,
                      const uint64_t* mask, int64_t mask_words, const IvfArgs& filters,
                      int64_t divisor, const int64_t* sort_perm, int64_t n_perm,
                      const float* global_scale, int64_t k, int64_t* out_ids, float* out_scores,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0 && n_probe >= 0 && n_lists >= 0 && width >= 0,
               "sizes must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(D % 16 == 0 && D >= 16 && D <= 8192, "D must be a multiple of 16 in [16, 8192]");
  RT_CHECK_ARG(n_probe <= kIvfMaxProbe, "n_probe must be <= %d", kIvfMaxProbe);
  RT_CHECK_ARG(divisor == -1 || divisor >= 1, "divisor_for_int8 must be -1 or >= 1");
  RT_CHECK_ARG(width < 0xffffffffll, "width must be < 2**32 - 1");
  RT_CHECK_ARG(mask == nullptr || mask_words >= cdiv(N, 64), "mask must cover every item");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(item_codes) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(q_codes) % 16 == 0,
               "codes must be 16-byte aligned");
  RT_CHECK_ARG(B <= 65535, "B must be <= 65535");
  if (B == 0) return kOk;
  const size_t need = rt_ivf_search_workspace(B, width, k);
  if (workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  const int64_t gx = ivf_gx(B, width);
  const int64_t S = gx * kIvfWaves;
  const int capw = ivf_capw(k);
  IvfArgs a{};
  a.q = q_codes;
  a.B = B;
  a.items = item_codes;
  a.N = N;
  a.RB = static_cast<int>(D);
  a.probe_ids = probe_ids;
  a.n_probe = n_probe;
  a.cluster_offsets = cluster_offsets;
  a.cluster_sizes = cluster_sizes;
  a.n_lists = n_lists;
  a.width = width;
  a.mask = mask;
  a.mask_words = mask_words;
  a.pcum = filters.pcum;
  a.pfirst = filters.pfirst;
  a.pwords = filters.pwords;
  a.p_entries = filters.p_entries;
  a.p_words = filters.p_words;
  a.slots = filters.slots;
  a.R = filters.R;
  a.cslots = filters.cslots;
  a.C = filters.C;
  a.reverse = filters.reverse;
  a.qv = filters.qv;
  a.divisor = static_cast<int>(divisor);
  a.k = static_cast<int>(k);
  a.capw = capw;
  char* ws = static_cast<char*>(workspace);
  a.lists = reinterpret_cast<uint64_t*>(ws);
  ws += align_up(static_cast<size_t>(B * S) * capw * sizeof(uint64_t), 256);
  a.list_counts = reinterpret_cast<int*>(ws);
  ws += align_up(static_cast<size_t>(B * S) * sizeof(int), 256);
  void* raw = ws;
  const int score_kind = divisor == -1 ? kScoreI32 : kScoreF32;
  if (n_probe > 0) {
    const size_t lds = ranges_lds(n_probe) +
                       static_cast<size_t>(kIvfWaves) * capw * sizeof(uint64_t) +
                       kIvfWaves * sizeof(int);
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(B));
    if (D <= 1024) {
      switch (D) {
        case 16: launch_ivf<1, 1>(a, grid, lds, stream); break;
        case 32: launch_ivf<2, 1>(a, grid, lds, stream); break;
        case 64: launch_ivf<4, 1>(a, grid, lds, stream); break;
        case 128: launch_ivf<8, 1>(a, grid, lds, stream); break;
        case 256: launch_ivf<16, 1>(a, grid, lds, stream); break;
        case 512: launch_ivf<32, 1>(a, grid, lds, stream); break;
        default: launch_ivf<64, 1>(a, grid, lds, stream); break;
      }
    } else if (D <= 2048) {
      launch_ivf<64, 2>(a, grid, lds, stream);
    } else if (D <= 4096) {
      launch_ivf<64, 4>(a, grid, lds, stream);
    } else {
      launch_ivf<64, 8>(a, grid, lds, stream);
    }
    RT_CHECK_HIP(hipGetLastError());
    MergeArgs m{};
    m.lists = a.lists;
    m.counts = a.list_counts;
    m.capw = capw;
    m.qpw = 1;
    m.S = S;
    m.B = B;
    m.k = static_cast<int>(k);
    m.out_ids = out_ids;
    m.out_scores = raw;
    m.score_kind = score_kind;
    const int st = launch_merge(m, stream);
    if (st != kOk) return st;
  } else {
    const int st = launch_pad(out_ids, raw, B, k, score_kind, stream);
    if (st != kOk) return st;
  }
  EpiArgs e{};
  e.ids = out_ids;
  e.raw = raw;
  e.scores = out_scores;
  e.B = B;
  e.k = k;
  e.ranges = true;
  e.a = a;
  e.sort_perm = sort_perm;
  e.n_perm = n_perm;
  e.q_scales = q_scales;
  e.global_scale = global_scale;
  e.divisor = static_cast<int>(divisor);
  const size_t lds = ranges_lds(n_probe);
  search_epilogue_kernel<<<static_cast<unsigned>(B), kIvfThreads, lds, stream>>>(e);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_ivf_search(const int8_t* q_codes, const float* q_scales, int64_t B,
                             const int8_t* item_codes, int64_t N, int64_t D,
                             const int64_t* probe_ids, int64_t n_probe,
                             const int64_t* cluster_offsets, const int64_t* cluster_sizes,
                             int64_t n_lists, int64_t width, const uint64_t* mask,
                             int64_t mask_words, int64_t divisor, const int64_t* sort_perm,
                             int64_t n_perm, const float* global_scale, int64_t k,
                             int64_t* out_ids, float* out_scores, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  const IvfArgs none{};
  return ivf_search(q_codes, q_scales, B, item_codes, N, D, probe_ids, n_probe, cluster_offsets,
                    cluster_sizes, n_lists, width, mask, mask_words, none, divisor, sort_perm,
                    n_perm, global_scale, k, out_ids, out_scores, workspace, workspace_bytes,
                    stream);
}

// rt_ivf_search with the reference's per-payload filters in place of a full-N mask: the probed
// payloads' Bloom words (partial response, may be null) and / or the exact clause recheck over
// the probed docs (slot layout, may be null); a doc is scored when both pass.
extern "C" int rt_ivf_search_payload_filters(
    const int8_t* q_codes, const float* q_scales, int64_t B, const int8_t* item_codes, int64_t N,
    int64_t D, const int64_t* probe_ids, int64_t n_probe, const int64_t* cluster_offsets,
    const int64_t* cluster_sizes, int64_t n_lists, int64_t width,
    const int32_t* partial_counts_cumsum, const int8_t* partial_first_offsets,
    const uint64_t* partial_words, int64_t partial_entries, int64_t partial_n_words,
    const int32_t* clause_slot_values, int64_t R, const int64_t* clause_slots, int64_t C,
    const int8_t* clause_is_reverse, const int32_t* query_clause_values, int64_t divisor,
    const int64_t* sort_perm, int64_t n_perm, const float* global_scale, int64_t k,
    int64_t* out_ids, float* out_scores, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
  RT_CHECK_ARG(partial_words == nullptr ||
                   (partial_counts_cumsum != nullptr && partial_first_offsets != nullptr &&
                    partial_entries >= 0 && partial_n_words >= 0),
               "the partial masks need their counts and first offsets");
  RT_CHECK_ARG(query_clause_values == nullptr ||
                   (clause_slots != nullptr && clause_is_reverse != nullptr && C >= 0 &&
                    C <= 32 && R >= 0 && (R == 0 || clause_slot_values != nullptr)),
               "the exact clauses need slots, clause_slots and clause_is_reverse, C <= 32");
  IvfArgs f{};
  f.pcum = partial_counts_cumsum;
  f.pfirst = partial_first_offsets;
  f.pwords = partial_words;
  f.p_entries = partial_entries;
  f.p_words = partial_n_words;
  f.slots = clause_slot_values;
  f.R = R;
  f.cslots = clause_slots;
  f.C = static_cast<int>(C);
  f.reverse = clause_is_reverse;
  f.qv = query_clause_values;
  return ivf_search(q_codes, q_scales, B, item_codes, N, D, probe_ids, n_probe, cluster_offsets,
                    cluster_sizes, n_lists, width, nullptr, 0, f, divisor, sort_perm, n_perm,
                    global_scale, k, out_ids, out_scores, workspace, workspace_bytes, stream);
}

// The epilogue alone, for a full scan's results: in_ids are item positions (-1 empty), raw the
// int32 dots [B, k].
extern "C" int rt_search_epilogue(int64_t* ids, const int32_t* raw_dots, float* out_scores,
                                  int64_t B, int64_t k, const int64_t* sort_perm, int64_t n_perm,
                                  const float* q_scales, const float* global_scale,
                                  hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && k >= 1, "B must be >= 0 and k >= 1");
  if (B == 0) return kOk;
  EpiArgs e{};
  e.ids = ids;
  e.raw = raw_dots;
  e.scores = out_scores;
  e.B = B;
  e.k = k;
  e.ranges = false;
  e.sort_perm = sort_perm;
  e.n_perm = n_perm;
  e.q_scales = q_scales;
  e.global_scale = global_scale;
  e.divisor = -1;
  search_epilogue_kernel<<<static_cast<unsigned>(B), kIvfThreads, 0, stream>>>(e);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
