// [1, N] fp32 dense scores of one fp16 query against the [D, N] fp16 item table, one fp32 FMA
// per k in order k = 0 .. D-1 (retrieve/src/retrieve/ops/triton/gemv_scores.py:19-43): the
// arithmetic of cuBLAS's gemv2N, so the scores equal torch.mm(q, E_t, out_dtype=fp32) where
// cuBLAS runs that kernel.
//
// HBM-bound (2 D bytes per item): lane <-> 8 consecutive items, so each k is one 16-byte load
// per lane and 1 KiB per wave instruction; the k loop is unrolled 8 deep for loads in flight.
// Tables whose rows are not 16-byte aligned (N % 8 != 0) take 2-byte loads.
#include "rt_common.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemvThreads = 256;
constexpr int kGemvItems = 8;  // items per lane
constexpr int kGemvUnroll = 8;

__device__ inline float half_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

template <bool VEC>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const uint16_t* __restrict__ q,
                                                            const uint16_t* __restrict__ e,
                                                            int64_t D, int64_t N,
                                                            float* __restrict__ out) {
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * kGemvThreads + threadIdx.x) * kGemvItems;
  if (n0 >= N) return;
  float acc[kGemvItems];
#pragma unroll
  for (int i = 0; i < kGemvItems; ++i) acc[i] = 0.f;
  const bool full = n0 + kGemvItems <= N;
  for (int64_t k0 = 0; k0 < D; k0 += kGemvUnroll) {
    uint16_t x[kGemvUnroll][kGemvItems];
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u) {
      const int64_t k = k0 + u;
      const uint16_t* row = e + k * N + n0;
      if (k < D) {
        if (VEC && full) {
          const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row));
#pragma unroll
          for (int i = 0; i < kGemvItems; ++i) {
            x[u][i] = static_cast<uint16_t>(static_cast<uint32_t>(v[i / 2]) >> (16 * (i % 2)));
          }
        } else {
#pragma unroll
          for (int i = 0; i < kGemvItems; ++i) x[u][i] = n0 + i < N ? row[i] : uint16_t{0};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u) {
      const int64_t k = k0 + u;
      if (k < D) {
        const float qk = half_to_float(q[k]);
#pragma unroll
        for (int i = 0; i < kGemvItems; ++i) {
          acc[i] = __builtin_fmaf(qk, half_to_float(x[u][i]), acc[i]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kGemvItems; ++i) {
    if (n0 + i < N) out[n0 + i] = acc[i];
  }
}

}  // namespace rt

using namespace rt;

extern "C" int rt_gemv_scores(const uint16_t* query, const uint16_t* item_embs_t, int64_t D,
                              int64_t N, float* out, hipStream_t stream) {
  RT_CHECK_ARG(D >= 1 && N >= 0, "D must be >= 1 and N >= 0");
  if (N == 0) return kOk;
  const int64_t grid = cdiv(cdiv(N, kGemvItems), kGemvThreads);
  RT_CHECK_ARG(grid < (int64_t{1} << 31), "N too large");
  const bool vec = N % kGemvItems == 0 && reinterpret_cast<uintptr_t>(item_embs_t) % 16 == 0;
  if (vec) {
    gemv_kernel<true><<<static_cast<unsigned>(grid), kGemvThreads, 0, stream>>>(
        query, item_embs_t, D, N, out);
  } else {
    gemv_kernel<false><<<static_cast<unsigned>(grid), kGemvThreads, 0, stream>>>(
        query, item_embs_t, D, N, out);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
