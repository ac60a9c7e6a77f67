// Bloom index over bit-sliced 2048-doc bundles: build, and the plan search that turns a batch of
// AND/OR/NOT term expressions into the scans' packed mask.
//
// Layout (bloom_indexer.cpp:79-110): bundle beta = d / 2048 is w_beta = off[beta+1] - off[beta]
// bits per doc; bit position p of doc d is word (off[beta] + p) * 32 + (d % 2048) / 64, bit
// 63 - d % 64. So word (off[beta] + p) * 32 + j holds position p of the 64 docs of global column
// 32 beta + j, in the bit order of the scans' mask words.
//
// Terms: a token (feature id f, value v) hashes to murmur(f, v, seed) = h1 ^ h2 of
// MurmurHash3_x64_128 (Austin Appleby's published algorithm, public domain) over the 16-byte
// key f || v (little-endian words), seeds 0, 1, ... (bloom_index_util.cuh:60-107). Build: the
// first k distinct hash % w_beta over seeds 0, 1, ... (:185-208). Search: the first k distinct
// hash % w_beta among the hash_k stored hashes (bloom_index_search_cuda.cu:305-349); a term
// holds for a doc iff all its positions are set.
//
// Build: one wave per 64-doc column (lane <-> doc). Each lane gathers its doc's positions into
// a bit mask; position p of the column is then one ballot, bit-reversed, written once by lane
// 0 -- every word of the index is written exactly once, with no atomics and no clearing pass.
//
// Plans (the parser's encoding, retrieve_amd/bloom.py): per plan 8 byte offsets [ops, offsets,
// parameters, hashes] x [begin, end) into the data, each segment 8-aligned; ops are uint8
// AND=1 OR=2 NOT=3 TERM=4 EMPTY=5 in post-order (bloom_index_util.h:49-56), offsets int32 [ops
// + 1] (parameter ranges: AND/OR take offsets[j+1] - offsets[j] children), hashes uint64
// [terms * hash_k] in the order the terms appear. Search: lane <-> column, a workgroup loops over
// its plans (wave-uniform instruction stream), the evaluation stack lives in LDS. When every
// bundle has the same width a resolve pass first turns each term's stored hashes into its k
// positions once, so the column pass does no 64-bit division.
#include "rt_common.h"

namespace rt {

constexpr int kBloomDocsPerBundle = 2048;
constexpr int kBloomWordsPerBundle = 32;
constexpr int kBloomMaxK = 10;            // positions per term (MAX_K_V2)
constexpr int kBloomMaxBuildWidth = 256;  // bits per doc the build keeps in registers
constexpr int kBloomMaxStack = 64;
constexpr int kBloomThreads = 256;
constexpr int kBloomMaxSeeds = 4096;  // build: bound on the seeds tried for k distinct positions

enum BloomOp : uint8_t { kOpAnd = 1, kOpOr = 2, kOpNot = 3, kOpTerm = 4, kOpEmpty = 5 };

__host__ __device__ inline uint64_t rotl64(uint64_t x, int r) {
  return (x << r) | (x >> (64 - r));
}

__host__ __device__ inline uint64_t fmix64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// MurmurHash3_x64_128 of the one 16-byte block x || y, folded h1 ^ h2.
__host__ __device__ inline uint64_t murmur_2x64(uint64_t x, uint64_t y, uint64_t seed) {
  const uint64_t c1 = 0x87c37b91114253d5ull;
  const uint64_t c2 = 0x4cf5ad432745937full;
  uint64_t h1 = seed;
  uint64_t h2 = seed;
  uint64_t k1 = x * c1;
  k1 = rotl64(k1, 31);
  k1 *= c2;
  h1 ^= k1;
  h1 = rotl64(h1, 27);
  h1 += h2;
  h1 = h1 * 5 + 0x52dce729;
  uint64_t k2 = y * c2;
  k2 = rotl64(k2, 33);
  k2 *= c1;
  h2 ^= k2;
  h2 = rotl64(h2, 31);
  h2 += h1;
  h2 = h2 * 5 + 0x38495ab5;
  h1 ^= 16;
  h2 ^= 16;
  h1 += h2;
  h2 += h1;
  h1 = fmix64(h1);
  h2 = fmix64(h2);
  h1 += h2;
  h2 += h1;
  return h1 ^ h2;
}

// ---- build --------------------------------------------------------------------------------

// max over the bundle's docs of the doc's value count (all features). One workgroup per bundle.
__global__ void __launch_bounds__(kBloomThreads) bloom_terms_kernel(const int64_t* fo, int64_t N,
                                                                    int C, int64_t* max_terms) {
  __shared__ int64_t red[kBloomThreads / kWave];
  const int64_t beta = blockIdx.x;
  int64_t m = 0;
  for (int i = threadIdx.x; i < kBloomDocsPerBundle; i += kBloomThreads) {
    const int64_t d = beta * kBloomDocsPerBundle + i;
    if (d < N) {
      const int64_t t = fo[(d + 1) * C] - fo[d * C];
      m = t > m ? t : m;
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(m, off);
    m = o > m ? o : m;
  }
  if (lane_id() == 0) red[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBloomThreads / kWave; ++w) m = red[w] > m ? red[w] : m;
    max_terms[beta] = m;
  }
}

struct BloomBuildArgs {
  const int32_t* feature_ids;  // [C]
  int C;
  const int64_t* fo;  // [N * C + 1] value ranges per (doc, feature)
  const int64_t* values;
  int64_t N;
  const int64_t* bundle_off;  // [nb + 1]
  int k;
  uint64_t* words;
};

// grid covers every doc slot of every bundle (nb * 2048), so the words of columns past the last
// doc are written too (as zeros)
__global__ void __launch_bounds__(kBloomThreads) bloom_build_kernel(BloomBuildArgs a) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kBloomThreads + threadIdx.x;
  const int lane = lane_id();
  const int64_t beta = d / kBloomDocsPerBundle;
  const int j = static_cast<int>((d % kBloomDocsPerBundle) / 64);
  const int64_t off = a.bundle_off[beta];
  const int64_t w = a.bundle_off[beta + 1] - off;  // the same for the whole wave
  uint64_t pm[kBloomMaxBuildWidth / 64] = {0ull, 0ull, 0ull, 0ull};
  if (d < a.N && w > 0) {
    const uint64_t uw = static_cast<uint64_t>(w);
    for (int c = 0; c < a.C; ++c) {
      const uint64_t f = static_cast<uint64_t>(static_cast<int64_t>(a.feature_ids[c]));
      const int64_t i1 = a.fo[d * a.C + c + 1];
      for (int64_t i = a.fo[d * a.C + c]; i < i1; ++i) {
        const uint64_t v = static_cast<uint64_t>(a.values[i]);
        int got = 0;
        uint32_t pos[kBloomMaxK];
        for (int seed = 0; got < a.k && seed < kBloomMaxSeeds; ++seed) {
          const uint32_t p = static_cast<uint32_t>(murmur_2x64(f, v, seed) % uw);
          bool dup = false;
          for (int q = 0; q < got; ++q) dup |= pos[q] == p;
          if (!dup) {
            pos[got++] = p;
            const uint64_t bit = 1ull << (p & 63);
            // (a select per slot keeps pm in registers)
#pragma unroll
            for (int s = 0; s < kBloomMaxBuildWidth / 64; ++s) pm[s] |= (p >> 6) == s ? bit : 0ull;
          }
        }
      }
    }
  }
  for (int64_t p = 0; p < w; ++p) {
    const uint64_t m = pm[p >> 6];
    const uint64_t word = __builtin_bitreverse64(__ballot((m >> (p & 63)) & 1ull));
    if (lane == 0) a.words[(off + p) * kBloomWordsPerBundle + j] = word;
  }
}

// ---- search -------------------------------------------------------------------------------

struct BloomSearchArgs {
  const uint64_t* words;
  const int64_t* bundle_off;  // [nb + 1]
  int64_t nb;
  const int64_t* plan_offsets;  // [plan_count, 8] byte offsets into data
  const int8_t* data;
  int64_t data_bytes;
  int64_t plan_count;
  int64_t plans_per_wg;
  int max_stack;
  int k;
  int hash_k;
  const int32_t* resolved;  // [data_bytes / 8] positions parallel to the hash words, or null
  const int32_t* uniform;   // [1]: 1 iff every bundle has the same width (resolve pass)
  int64_t* out_mask;        // [plan_count, nb * 32] or null
  uint8_t* out_bool;        // [plan_count, nb * 32 * 64] or null
};

// The first k distinct hash % w among a term's stored hashes (fewer if they do not hold k).
__device__ inline int resolve_positions(const uint64_t* h, int hash_k, int k, uint64_t w,
                                        uint32_t (&pos)[kBloomMaxK]) {
  int got = 0;
  for (int s = 0; s < hash_k && got < k; ++s) {
    const uint32_t p = static_cast<uint32_t>(h[s] % w);
    bool dup = false;
    for (int q = 0; q < got; ++q) dup |= pos[q] == p;
    if (!dup) pos[got++] = p;
  }
  return got;
}

// A plan's offsets are inside the data, ordered, and aligned for their element types.
__device__ inline bool plan_ok(const int64_t* o, int64_t data_bytes) {
  bool ok = true;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    ok &= o[2 * s] >= 0 && o[2 * s] <= o[2 * s + 1] && o[2 * s + 1] <= data_bytes;
  }
  return ok && (o[2] % 4) == 0 && (o[4] % 4) == 0 && (o[6] % 8) == 0;
}

// One workgroup: whether all bundles share a width, and if so every term's positions for it
// (resolved[hash word index of the term's first hash + i], -1 past the distinct ones).
__global__ void __launch_bounds__(kBloomThreads) bloom_resolve_kernel(BloomSearchArgs a,
                                                                      int32_t* resolved,
                                                                      int32_t* uniform) {
  __shared__ int all_same;
  if (threadIdx.x == 0) all_same = 1;
  __syncthreads();
  const int64_t w0 = a.bundle_off[1] - a.bundle_off[0];
  for (int64_t beta = threadIdx.x; beta < a.nb; beta += kBloomThreads) {
    if (a.bundle_off[beta + 1] - a.bundle_off[beta] != w0) all_same = 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) uniform[0] = all_same;
  if (!all_same || w0 <= 0) return;
  const int kk = a.k < a.hash_k ? a.k : a.hash_k;  // positions a term can resolve
  for (int64_t b = threadIdx.x; b < a.plan_count; b += kBloomThreads) {
    const int64_t* o = a.plan_offsets + 8 * b;
    if (!plan_ok(o, a.data_bytes)) continue;
    const int64_t h0 = o[6] / 8;
    const int64_t nh = (o[7] - o[6]) / 8;
    const uint64_t* hashes = reinterpret_cast<const uint64_t*>(a.data) + h0;
    for (int64_t t = 0; (t + 1) * a.hash_k <= nh; ++t) {
      uint32_t pos[kBloomMaxK];
      const int got = resolve_positions(hashes + t * a.hash_k, a.hash_k, a.k,
                                        static_cast<uint64_t>(w0), pos);
      for (int i = 0; i < kk; ++i) {
        resolved[h0 + t * a.hash_k + i] = i < got ? static_cast<int32_t>(pos[i]) : -1;
      }
    }
  }
}

__global__ void __launch_bounds__(kBloomThreads) bloom_search_kernel(BloomSearchArgs a) {
  extern __shared__ uint64_t stk[];  // [max_stack][kBloomThreads]
  const int tid = threadIdx.x;
  const int64_t ncol = a.nb * kBloomWordsPerBundle;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kBloomThreads + tid;
  const bool valid = col < ncol;
  const int64_t beta = valid ? col / kBloomWordsPerBundle : 0;
  const int j = static_cast<int>(col % kBloomWordsPerBundle);
  const int64_t off = a.bundle_off[beta];
  const int64_t w = a.bundle_off[beta + 1] - off;
  const bool uniform = a.uniform[0] != 0;
  const uint64_t* wcol = a.words + off * kBloomWordsPerBundle + j;  // position p at wcol[32 p]

  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.plans_per_wg;
  const int64_t b1 = b0 + a.plans_per_wg < a.plan_count ? b0 + a.plans_per_wg : a.plan_count;
  for (int64_t b = b0; b < b1; ++b) {
    const int64_t* o = a.plan_offsets + 8 * b;
    // a malformed plan evaluates to no match instead of reading out of bounds
    bool bad = !plan_ok(o, a.data_bytes);
    const uint8_t* ops = reinterpret_cast<const uint8_t*>(a.data + o[0]);
    const int64_t n_ops = bad ? 0 : o[1] - o[0];
    const int32_t* offs = reinterpret_cast<const int32_t*>(a.data + o[2]);
    const int64_t n_offs = (o[3] - o[2]) / 4;
    const int64_t h0 = o[6] / 8;
    const int64_t nh = (o[7] - o[6]) / 8;
    int sp = 0;
    int64_t term = 0;
    for (int64_t i = 0; i < n_ops && !bad; ++i) {
      const uint8_t op = ops[i];
      uint64_t r = 0ull;
      if (op == kOpTerm) {
        if ((term + 1) * a.hash_k > nh) {
          bad = true;
          break;
        }
        if (w <= 0) {
          r = 0ull;  // a bundle with no bits holds no term
        } else if (uniform) {
          r = ~0ull;
          const int32_t* rp = a.resolved + h0 + term * a.hash_k;
          const int kk = a.k < a.hash_k ? a.k : a.hash_k;
          for (int q = 0; q < kk; ++q) {
            const int32_t p = rp[q];
            if (p < 0) break;
            r &= wcol[static_cast<int64_t>(p) * kBloomWordsPerBundle];
          }
        } else {
          r = ~0ull;
          uint32_t pos[kBloomMaxK];
          const uint64_t* h = reinterpret_cast<const uint64_t*>(a.data) + h0 + term * a.hash_k;
          const int got = resolve_positions(h, a.hash_k, a.k, static_cast<uint64_t>(w), pos);
          for (int q = 0; q < got; ++q) {
            r &= wcol[static_cast<int64_t>(pos[q]) * kBloomWordsPerBundle];
          }
        }
        ++term;
      } else if (op == kOpAnd || op == kOpOr) {
        if (i + 1 >= n_offs) {
          bad = true;
          break;
        }
        const int n = offs[i + 1] - offs[i];  // children on the stack
        if (n < 1 || n > sp) {
          bad = true;
          break;
        }
        r = op == kOpAnd ? ~0ull : 0ull;
        for (int q = 0; q < n; ++q) {
          const uint64_t x = stk[(--sp) * kBloomThreads + tid];
          r = op == kOpAnd ? (r & x) : (r | x);
        }
      } else if (op == kOpNot) {
        if (sp < 1) {
          bad = true;
          break;
        }
        r = ~stk[(--sp) * kBloomThreads + tid];
      } else if (op == kOpEmpty) {
        r = ~0ull;
      } else {
        bad = true;
        break;
      }
      if (sp >= a.max_stack) {
        bad = true;
        break;
      }
      stk[(sp++) * kBloomThreads + tid] = r;
    }
    const uint64_t res = (!bad && sp == 1) ? stk[tid] : 0ull;
    if (valid) {
      if (a.out_mask != nullptr) a.out_mask[b * ncol + col] = static_cast<int64_t>(res);
      if (a.out_bool != nullptr) {
        // 64 bytes per column, doc 64 col + q at byte q (bit 63 - q of the word)
        uint4* ob = reinterpret_cast<uint4*>(a.out_bool + (b * ncol + col) * 64);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          uint32_t x[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            uint32_t y = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int q = 16 * v + 4 * u + t;
              y |= static_cast<uint32_t>((res >> (63 - q)) & 1ull) << (8 * t);
            }
            x[u] = y;
          }
          ob[v] = make_uint4(x[0], x[1], x[2], x[3]);
        }
      }
    }
  }
}

}  // namespace rt

using namespace rt;

extern "C" int rt_bloom_bundle_terms(const int64_t* feature_offsets, int64_t N, int64_t C,
                                     int64_t* max_terms, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && C >= 1 && C <= (int64_t{1} << 20), "N must be >= 0 and C >= 1");
  const int64_t nb = cdiv(N, kBloomDocsPerBundle);
  if (nb == 0) return kOk;
  bloom_terms_kernel<<<static_cast<unsigned>(nb), kBloomThreads, 0, stream>>>(
      feature_offsets, N, static_cast<int>(C), max_terms);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_bloom_build(const int32_t* feature_ids, int64_t C,
                              const int64_t* feature_offsets, const int64_t* feature_values,
                              int64_t N, const int64_t* bundle_b_offsets, int64_t max_width,
                              int64_t k, uint64_t* words, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && C >= 1 && C <= (int64_t{1} << 20), "N must be >= 0 and C >= 1");
  RT_CHECK_ARG(k >= 1 && k <= kBloomMaxK, "k must be in [1, %d], got %lld", kBloomMaxK,
               static_cast<long long>(k));
  RT_CHECK_ARG(max_width >= 0 && max_width <= kBloomMaxBuildWidth,
               "bits per doc must be <= %d, got %lld", kBloomMaxBuildWidth,
               static_cast<long long>(max_width));
  const int64_t nb = cdiv(N, kBloomDocsPerBundle);
  if (nb == 0 || max_width == 0) return kOk;
  BloomBuildArgs a{};
  a.feature_ids = feature_ids;
  a.C = static_cast<int>(C);
  a.fo = feature_offsets;
  a.values = feature_values;
  a.N = N;
  a.bundle_off = bundle_b_offsets;
  a.k = static_cast<int>(k);
  a.words = words;
  const int64_t grid = nb * kBloomDocsPerBundle / kBloomThreads;
  RT_CHECK_ARG(grid < (int64_t{1} << 31), "N too large");
  bloom_build_kernel<<<static_cast<unsigned>(grid), kBloomThreads, 0, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" size_t rt_bloom_search_workspace(int64_t data_bytes) {
  const int64_t words = data_bytes > 0 ? data_bytes / 8 : 0;
  return 256 + align_up(static_cast<size_t>(words) * sizeof(int32_t), 256);
}

extern "C" int rt_bloom_search(const uint64_t* words, const int64_t* bundle_b_offsets,
                               int64_t n_bundles, const int64_t* plan_offsets,
                               const int8_t* plan_data, int64_t data_bytes, int64_t plan_count,
                               int64_t max_stack, int64_t k, int64_t hash_k, int64_t* out_mask,
                               uint8_t* out_bool, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  RT_CHECK_ARG(n_bundles >= 0 && plan_count >= 0 && data_bytes >= 0, "sizes must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kBloomMaxK, "k must be in [1, %d], got %lld", kBloomMaxK,
               static_cast<long long>(k));
  RT_CHECK_ARG(hash_k >= 1 && hash_k <= 64, "hash_k must be in [1, 64], got %lld",
               static_cast<long long>(hash_k));
  RT_CHECK_ARG(max_stack >= 1 && max_stack <= kBloomMaxStack,
               "max_stack_size must be in [1, %d], got %lld", kBloomMaxStack,
               static_cast<long long>(max_stack));
  RT_CHECK_ARG(out_mask != nullptr || out_bool != nullptr, "no output");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(plan_data) % 8 == 0, "plan data must be 8-aligned");
  if (n_bundles == 0 || plan_count == 0) return kOk;
  const size_t need = rt_bloom_search_workspace(data_bytes);
  if (workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  BloomSearchArgs a{};
  a.words = words;
  a.bundle_off = bundle_b_offsets;
  a.nb = n_bundles;
  a.plan_offsets = plan_offsets;
  a.data = plan_data;
  a.data_bytes = data_bytes;
  a.plan_count = plan_count;
  a.max_stack = static_cast<int>(max_stack);
  a.k = static_cast<int>(k);
  a.hash_k = static_cast<int>(hash_k);
  a.uniform = static_cast<int32_t*>(workspace);
  a.resolved = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + 256);
  a.out_mask = out_mask;
  a.out_bool = out_bool;
  bloom_resolve_kernel<<<1, kBloomThreads, 0, stream>>>(
      a, const_cast<int32_t*>(a.resolved), const_cast<int32_t*>(a.uniform));
  RT_CHECK_HIP(hipGetLastError());
  const int64_t gx = cdiv(n_bundles * kBloomWordsPerBundle, kBloomThreads);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "too many bundles");
  int64_t gy = cdiv(2048, gx);
  gy = gy < 1 ? 1 : gy;
  gy = gy > plan_count ? plan_count : gy;
  gy = gy > 65535 ? 65535 : gy;
  a.plans_per_wg = cdiv(plan_count, gy);
  gy = cdiv(plan_count, a.plans_per_wg);
  const size_t lds = static_cast<size_t>(max_stack) * kBloomThreads * sizeof(uint64_t);
  if (lds > 64 * 1024) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&bloom_search_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  bloom_search_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                        kBloomThreads, lds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
