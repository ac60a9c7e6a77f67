// Per-wave candidate lists: the exact top-k machinery every scan kernel shares.
//
// A scan wave owns, for each query it scores, one list of `capw` composites in global memory
// and a count in LDS. A scored (query, item) whose composite is >= the query's threshold is
// appended; when a count could overflow on the next tile the wave sorts that list in its LDS
// scratch, keeps the best k and raises the threshold to the k-th composite. Appends are rare
// once the threshold is seeded from a sample, so the lists are usually a few entries long.
// The final top-k is the best k over all of a query's lists (merge kernel): every item of the
// true top-k is in some list, because a wave's threshold never exceeds its own k-th best.
#pragma once

#include <type_traits>

#include "rt_common.h"

namespace rt {

// Relaxed agent-scope load: bypasses the non-coherent vector L1, so a wave reads back the
// list entries its other lanes stored earlier.
__device__ inline uint64_t load_coherent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bitonic sort of `n` (a power of two) composites in LDS, descending, by one wave.
__device__ inline void wave_sort_desc(uint64_t* s, int n) {
  const int lane = lane_id();
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = lane; t < (n >> 1); t += kWave) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint64_t a = s[i];
        const uint64_t b = s[j];
        if ((a < b) == desc) {
          s[i] = b;
          s[j] = a;
        }
      }
      wave_sync_memory();
    }
  }
}

// Every composite is kept by wave_compact's default filter.
struct KeepAll {
  __device__ bool operator()(uint64_t) const { return true; }
};

// Sorts list[0, *count) (global) through `scratch` (LDS, sort_n entries: a power of two >=
// *count), keeps the best min(count, k) of the entries `keep_entry` accepts (the others drop
// out), and returns the k-th composite (0 while fewer than k are held). Called by the whole
// wave with a wave-uniform list.
template <class Keep = KeepAll>
__device__ inline uint64_t wave_compact(uint64_t* list, int* count, uint64_t* scratch, int sort_n,
                                        int k, Keep keep_entry = Keep{}) {
  const int lane = lane_id();
  wave_sync_memory();
  int n = *count;
  if constexpr (std::is_same<Keep, KeepAll>::value) {
    for (int i = lane; i < sort_n; i += kWave) {
      scratch[i] = i < n ? load_coherent(list + i) : 0ull;
    }
  } else {
    int held = 0;
    for (int i = lane; i < sort_n; i += kWave) {
      const uint64_t v = i < n ? load_coherent(list + i) : 0ull;
      const bool kept = i < n && keep_entry(v);
      held += kept ? 1 : 0;
      scratch[i] = kept ? v : 0ull;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) held += __shfl_xor(held, off);
    n = held;
  }
  wave_sync_memory();
  wave_sort_desc(scratch, sort_n);
  const int keep = n < k ? n : k;
  for (int i = lane; i < keep; i += kWave) {
    list[i] = scratch[i];
  }
  const uint64_t tau = n >= k ? scratch[k - 1] : 0ull;
  wave_sync_memory();
  if (lane == 0) {
    *count = keep;
  }
  wave_sync_memory();
  return tau;
}

}  // namespace rt
