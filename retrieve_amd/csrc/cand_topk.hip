// Exact top-k over per-query candidate lists: score item rows gathered through
// positive_indices[b, 0:counts[b]] against query b, keep the best k by (score desc, item id
// asc).
//
// The LiNR V2 / V3 operators fused_masked_knn_topk and oporp_1bit_match_topk_indirect
// (retrieve/src/retrieve/ops/reference/fused_masked_knn_topk.py:9-29,
// ops/reference/oporp_1bit_match_topk.py:29-41) and SilverTorch's int8 re-rank of given ids
// (modules/silvertorch.py:363-379). Each query has its own rows, so the work is a gather:
// a group of L lanes loads one row, 16 bytes per lane per step, dots it with the query chunks
// it holds in registers and reduces across the group with xor-shuffles; a wave scores 64 / L
// rows per step. A workgroup scans one query's positions round-robin with the other
// workgroups of that query; every wave keeps a candidate list under a running threshold (no
// seed: the list fills, is compacted to the best k and the threshold rises), and the shared
// merge picks the final k. The item id rides in the composites, so ties go to the lower item
// id whatever the candidates' order (a re-rank's candidates arrive in score order).
#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kCandThreads = 256;
constexpr int kCandWaves = kCandThreads / kWave;
constexpr int kCandMaxWgsPerQuery = 64;
constexpr int kCandMaxChunks = 8;  // 16-byte chunks per lane: rows up to 64 * 16 * 8 bytes

enum CandKind : int {
  kCandF16 = 0,
  kCandBF16 = 1,
  kCandF32 = 2,
  kCandI8 = 3,
  kCandBits = 4,
  kCandI8Scaled = 5,  // int8 dots keyed on the float score (dot * query scale) * global scale
};

// (by value: __builtin_bit_cast applied directly to a vector element x[i] reads element 0)
__device__ inline float as_float(int32_t v) { return __builtin_bit_cast(float, v); }

// Partial score of one 16-byte chunk of a row against the query chunk (fp32 query for the
// floating kinds, raw bytes otherwise).
template <int KIND>
struct CandOp;

template <>
struct CandOp<kCandF16> {
  using Acc = float;
  __device__ static float chunk(v4i x, const float* q) {
    const _Float16* h = reinterpret_cast<const _Float16*>(&x);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = __builtin_fmaf(static_cast<float>(h[i]), q[i], s);
    return s;
  }
};

template <>
struct CandOp<kCandBF16> {
  using Acc = float;
  __device__ static float chunk(v4i x, const float* q) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = static_cast<uint32_t>(x[i]);
      s = __builtin_fmaf(__builtin_bit_cast(float, w << 16), q[2 * i], s);
      s = __builtin_fmaf(__builtin_bit_cast(float, w & 0xffff0000u), q[2 * i + 1], s);
    }
    return s;
  }
};

template <>
struct CandOp<kCandF32> {
  using Acc = float;
  __device__ static float chunk(v4i x, const float* q) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_fmaf(as_float(x[i]), q[i], s);
    return s;
  }
};

template <>
struct CandOp<kCandI8> {
  using Acc = int32_t;
  __device__ static int32_t chunk(v4i x, v4i q) {
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_sdot4(x[i], q[i], s, false);
    return s;
  }
};

template <>
struct CandOp<kCandI8Scaled> : CandOp<kCandI8> {};

template <>
struct CandOp<kCandBits> {
  using Acc = int32_t;
  // -2 popcount(q ^ x) of the chunk; the row's 8 * RB bits are added once after the reduction,
  // so a half chunk (zeros in both halves) counts only its own 64 bits
  __device__ static int32_t chunk(v4i x, v4i q) {
    int32_t d = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) d += __builtin_popcount(static_cast<uint32_t>(x[i] ^ q[i]));
    return -2 * d;
  }
};

typedef int v2i __attribute__((ext_vector_type(2)));

// 16-byte chunk c of a row of rb bytes; the last chunk of a row of 8 (mod 16) bytes is loaded as
// 8 bytes and zero-extended.
template <bool NT>
__device__ inline v4i load_chunk(const int8_t* row, int c, int rb) {
  if (16 * c + 8 == rb) {
    const v2i h = NT ? __builtin_nontemporal_load(reinterpret_cast<const v2i*>(row + 16 * c))
                     : *reinterpret_cast<const v2i*>(row + 16 * c);
    return v4i{h[0], h[1], 0, 0};
  }
  return NT ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row + 16 * c))
            : *reinterpret_cast<const v4i*>(row + 16 * c);
}

struct CandArgs {
  const void* queries;  // [B, RB] bytes (float32 rows for the floating kinds)
  int64_t B;
  const void* items;  // [N, RB] bytes
  int64_t N;
  int RB;  // item row bytes (a multiple of 16)
  const int64_t* ids;  // [B, P] candidate item ids
  int64_t P;
  const int64_t* counts;  // [B]
  const int64_t* rows;    // [N] item id -> row of items, or null (row = id)
  const float* qscale;    // [B], kCandI8Scaled only
  const float* gscale;    // [1], kCandI8Scaled only
  int k;
  int capw;
  uint64_t* lists;  // [B, S, capw]
  int* list_counts;  // [B, S]
};

template <int KIND, int L, int NC>
__global__ void __launch_bounds__(kCandThreads) cand_scan_kernel(CandArgs a) {
  using Op = CandOp<KIND>;
  constexpr bool kFloat = KIND == kCandF16 || KIND == kCandBF16 || KIND == kCandF32;
  constexpr int R = kWave / L;  // rows per wave step
  // elements of a 16-byte item chunk, and the query floats they meet
  constexpr int QF = KIND == kCandF32 ? 4 : 8;
  extern __shared__ uint64_t smem[];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int grp = lane / L;  // row within the step
  const int gl = lane % L;   // lane within the row's group
  uint64_t* scratch = smem + wave * a.capw;
  int* cnt_lds = reinterpret_cast<int*>(smem + kCandWaves * a.capw);
  const int64_t b = blockIdx.y;
  const int64_t gx = gridDim.x;
  const int64_t S = gx * kCandWaves;
  const int64_t slot = static_cast<int64_t>(blockIdx.x) * kCandWaves + wave;
  uint64_t* list = a.lists + (b * S + slot) * a.capw;

  int64_t count = a.counts[b];
  count = count < 0 ? 0 : (count > a.P ? a.P : count);

  // this lane's query chunks: c = gl + j * L
  const int nchunks = (a.RB + 15) / 16;
  v4i qb[NC];
  float qf[NC][QF];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = gl + j * L;
    if constexpr (kFloat) {
      const float* q =
          static_cast<const float*>(a.queries) + b * (a.RB / (KIND == kCandF32 ? 4 : 2));
#pragma unroll
      for (int e = 0; e < QF; ++e) qf[j][e] = c < nchunks ? q[c * QF + e] : 0.f;
    } else {
      const int8_t* q = static_cast<const int8_t*>(a.queries) + b * a.RB;
      qb[j] = c < nchunks ? load_chunk<false>(q, c, a.RB) : v4i{0, 0, 0, 0};
    }
  }

  float qs = 0.f, gs = 0.f;
  if constexpr (KIND == kCandI8Scaled) {
    qs = a.qscale[b];
    gs = a.gscale[0];
  }
  uint64_t tau = 0;  // composites below it cannot reach this wave's best k
  int cnt = 0;
  const int64_t step = gx * kCandWaves * R;
  const int64_t first = slot * R;
  const int8_t* I = static_cast<const int8_t*>(a.items);
  for (int64_t base = first; base < count; base += step) {
    const int64_t p = base + grp;
    bool ok = p < count;
    int64_t item = ok ? a.ids[b * a.P + p] : 0;
    ok = ok && item >= 0 && item < a.N;  // ids outside the table are skipped, not read
    int64_t r = item;
    if (a.rows != nullptr && ok) {
      r = a.rows[item];
      ok = r >= 0 && r < a.N;
    }
    typename Op::Acc s = 0;
    if (ok) {
      const int8_t* row = I + r * a.RB;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = gl + j * L;
        if (c < nchunks) {
          const v4i x = load_chunk<true>(row, c, a.RB);
          if constexpr (kFloat) {
            s += Op::chunk(x, qf[j]);
          } else {
            s += Op::chunk(x, qb[j]);
          }
        }
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if constexpr (KIND == kCandBits) s += 8 * a.RB;
    uint64_t c = 0;
    if constexpr (kFloat) {
      c = composite(key_of_f32(static_cast<float>(s)), static_cast<uint32_t>(item));
    } else if constexpr (KIND == kCandI8Scaled) {
      // two roundings in this order, as (dots * q_scales) * global_scale in fp32
      const float v = (static_cast<float>(s) * qs) * gs;
      c = composite(key_of_f32(v), static_cast<uint32_t>(item));
    } else {  // int8 dots and bit-code scores are exact int32
      c = composite(key_of_i32(static_cast<int32_t>(s)), static_cast<uint32_t>(item));
    }
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
  if (lane == 0) a.list_counts[b * S + slot] = cnt;
}

// A winner with a non-finite float score becomes id -1 (functional.py:81-82).
__global__ void cand_ids_kernel(int64_t* ids, const float* scores, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n && !__builtin_isfinite(scores[i])) ids[i] = -1;
}

template <int KIND, int L, int NC>
static void launch_cand(const CandArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  if (lds > 64 * 1024) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&cand_scan_kernel<KIND, L, NC>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  }
  cand_scan_kernel<KIND, L, NC><<<grid, kCandThreads, lds, stream>>>(a);
}

template <int KIND>
static int dispatch_cand(const CandArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  // L lanes per row (16 bytes each, up to 64), NC 16-byte chunks per lane
  switch ((a.RB + 15) / 16 * 16) {
    case 16: launch_cand<KIND, 1, 1>(a, grid, lds, stream); break;
    case 32: launch_cand<KIND, 2, 1>(a, grid, lds, stream); break;
    case 64: launch_cand<KIND, 4, 1>(a, grid, lds, stream); break;
    case 128: launch_cand<KIND, 8, 1>(a, grid, lds, stream); break;
    case 256: launch_cand<KIND, 16, 1>(a, grid, lds, stream); break;
    case 512: launch_cand<KIND, 32, 1>(a, grid, lds, stream); break;
    default:
      if (a.RB <= 1024) {
        launch_cand<KIND, 64, 1>(a, grid, lds, stream);
      } else if (a.RB <= 2048) {
        launch_cand<KIND, 64, 2>(a, grid, lds, stream);
      } else if (a.RB <= 4096) {
        launch_cand<KIND, 64, 4>(a, grid, lds, stream);
      } else {
        launch_cand<KIND, 64, 8>(a, grid, lds, stream);
      }
  }
  return kOk;
}

static int cand_capw(int64_t k) { return static_cast<int>(next_pow2(k + kWave)); }

// Workgroups per query: ~2048 in all, at most one per 128 candidates (a wave's rows are an id
// load then the row's loads, one step after another: the grid, not the loop, hides that latency).
static int64_t cand_gx(int64_t B, int64_t P) {
  int64_t gx = cdiv(2048, B > 0 ? B : 1);
  const int64_t by_rows = cdiv(P, 128);
  gx = gx < by_rows ? gx : by_rows;
  gx = gx < 1 ? 1 : gx;
  return gx < kCandMaxWgsPerQuery ? gx : kCandMaxWgsPerQuery;
}

}  // namespace rt

using namespace rt;

extern "C" size_t rt_cand_topk_workspace(int64_t B, int64_t P, int64_t k) {
  if (B <= 0 || P <= 0 || k <= 0) return 256;
  const int64_t S = cand_gx(B, P) * kCandWaves;
  return align_up(static_cast<size_t>(B * S) * cand_capw(k) * sizeof(uint64_t), 256) +
         align_up(static_cast<size_t>(B * S) * sizeof(int), 256);
}

namespace rt {

static int cand_topk(const void* queries, int64_t B, const void* items, int64_t N, int64_t D,
                     int kind, const int64_t* positive_indices, int64_t P, const int64_t* counts,
                     const int64_t* rows, const float* qscale, const float* gscale, int64_t k,
                     int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  RT_CHECK_ARG(B >= 0 && N >= 0 && P >= 0 && D >= 1, "B, N, P must be >= 0 and D >= 1");
  RT_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be in [1, %lld], got %lld",
               static_cast<long long>(kMaxK), static_cast<long long>(k));
  RT_CHECK_ARG(kind >= kCandF16 && kind <= kCandI8Scaled, "kind must be in [0, 5]");
  static const int elem[] = {2, 2, 4, 1, 8, 1};
  const int64_t rb = D * elem[kind];
  // bit codes: any number of 64-bit words; the other kinds whole 16-byte chunks
  const int64_t unit = kind == kCandBits ? 8 : 16;
  RT_CHECK_ARG(rb % unit == 0 && rb <= 64 * 16 * kCandMaxChunks,
               "row bytes (D * element size = %lld) must be a multiple of %lld and <= %d",
               static_cast<long long>(rb), static_cast<long long>(unit),
               64 * 16 * kCandMaxChunks);
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(items) % unit == 0 &&
                   reinterpret_cast<uintptr_t>(queries) % unit == 0,
               "queries and items must be %lld-byte aligned", static_cast<long long>(unit));
  RT_CHECK_ARG(N < 0xffffffffll, "N must be < 2**32 - 1");
  // bit codes score as exact int32 keys, written as float
  const int score_kind =
      kind == kCandI8 ? kScoreI32 : (kind == kCandBits ? kScoreF32FromI32 : kScoreF32);
  RT_CHECK_ARG(kind != kCandI8Scaled || (qscale != nullptr && gscale != nullptr),
               "the scaled int8 kind needs query and global scales");
  if (B == 0) return kOk;
  if (P == 0 || N == 0) return launch_pad(out_ids, out_scores, B, k, score_kind, stream);
  const size_t need = rt_cand_topk_workspace(B, P, k);
  if (workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  const int64_t gx = cand_gx(B, P);
  const int64_t S = gx * kCandWaves;
  const int capw = cand_capw(k);
  RT_CHECK_ARG(B <= 65535, "B must be <= 65535");
  CandArgs a{};
  a.queries = queries;
  a.B = B;
  a.items = items;
  a.N = N;
  a.RB = static_cast<int>(rb);
  a.ids = positive_indices;
  a.P = P;
  a.counts = counts;
  a.rows = rows;
  a.qscale = qscale;
  a.gscale = gscale;
  a.k = static_cast<int>(k);
  a.capw = capw;
  a.lists = static_cast<uint64_t*>(workspace);
  a.list_counts = reinterpret_cast<int*>(
      static_cast<char*>(workspace) +
      align_up(static_cast<size_t>(B * S) * capw * sizeof(uint64_t), 256));
  const size_t lds = static_cast<size_t>(kCandWaves) * capw * sizeof(uint64_t) +
                     kCandWaves * sizeof(int);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(B));
  switch (kind) {
    case kCandF16: dispatch_cand<kCandF16>(a, grid, lds, stream); break;
    case kCandBF16: dispatch_cand<kCandBF16>(a, grid, lds, stream); break;
    case kCandF32: dispatch_cand<kCandF32>(a, grid, lds, stream); break;
    case kCandI8: dispatch_cand<kCandI8>(a, grid, lds, stream); break;
    case kCandI8Scaled: dispatch_cand<kCandI8Scaled>(a, grid, lds, stream); break;
    default: dispatch_cand<kCandBits>(a, grid, lds, stream); break;
  }
  RT_CHECK_HIP(hipGetLastError());
  MergeArgs m{};
  m.lists = a.lists;
  m.counts = a.list_counts;
  m.flat = false;
  m.capw = capw;
  m.qpw = 1;
  m.S = S;
  m.B = B;
  m.k = static_cast<int>(k);
  m.out_ids = out_ids;
  m.out_scores = out_scores;
  m.score_kind = score_kind;
  int st = launch_merge(m, stream);
  if (st != kOk) return st;
  if (score_kind == kScoreF32) {
    cand_ids_kernel<<<static_cast<unsigned>(cdiv(B * k, 256)), 256, 0, stream>>>(
        out_ids, static_cast<const float*>(out_scores), B * k);
    RT_CHECK_HIP(hipGetLastError());
  }
  return kOk;
}

}  // namespace rt

// kind: 0 fp16, 1 bf16, 2 fp32 items with float32 queries [B, D] (float scores); 3 int8
// (int32 scores); 4 bit codes of D 64-bit words (score 64 D - 2 popcount, float scores).
extern "C" int rt_cand_topk(const void* queries, int64_t B, const void* items, int64_t N,
                            int64_t D, int kind, const int64_t* positive_indices, int64_t P,
                            const int64_t* counts, int64_t k, int64_t* out_ids, void* out_scores,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
  RT_CHECK_ARG(kind >= kCandF16 && kind <= kCandBits, "kind must be in [0, 4]");
  return cand_topk(queries, B, items, N, D, kind, positive_indices, P, counts, nullptr, nullptr,
                   nullptr, k, out_ids, out_scores, workspace, workspace_bytes, stream);
}

// SilverTorch's re-rank of given ids: candidate id c (-1 = padding) is scored from row
// item_rows[c] of item_codes (the cluster-sorted table), key (float(dot) * q_scales[b]) *
// global_scale[0], ties to the lower id.
extern "C" int rt_int8_rerank_topk(const int8_t* q_codes, const float* q_scales, int64_t B,
                                   const int8_t* item_codes, int64_t N, int64_t D,
                                   const int64_t* item_rows, const float* global_scale,
                                   const int64_t* candidate_ids, int64_t P, const int64_t* counts,
                                   int64_t k, int64_t* out_ids, float* out_scores,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return cand_topk(q_codes, B, item_codes, N, D, kCandI8Scaled, candidate_ids, P, counts,
                   item_rows, q_scales, global_scale, k, out_ids, out_scores, workspace,
                   workspace_bytes, stream);
}
