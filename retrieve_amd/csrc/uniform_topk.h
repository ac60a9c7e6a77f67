// Candidate handling for scans where each lane scores its own item against one wave-uniform
// query at a time (the Hamming scan): per-query thresholds and list counts live in LDS.
#pragma once

#include "scan_common.h"
#include "wave_lists.h"

namespace rt {

// One wave's candidate state for `nq` queries (nq <= its LDS capacity).
struct WaveTopKUniform {
  uint64_t* lists;         // [nq, capw] in global memory
  int* cnt;                // [nq] in LDS
  uint64_t* tau;           // [nq] in LDS: lower bound per query (composite)
  uint64_t* scratch;       // [scratch_n] in LDS (power of two >= capw)
  int capw;
  int scratch_n;
  int k;

  // `ok`: this lane's item is a candidate for query qi (score >= the fast-path threshold and
  // inside the pass). Appends its composite if >= tau[qi] and it passes the filter bits
  // (qmask: query qi's item bits, bit 63 - d % 64, or null); compacts the list when it could
  // overflow on the next tile (at most 64 appends). Returns the (possibly raised) tau[qi].
  __device__ uint64_t push(int qi, bool ok, uint32_t key, uint32_t item, const uint64_t* qmask) {
    const uint64_t t = tau[qi];
    if (ok) {
      const uint64_t c = composite(key, item);
      bool keep = c >= t;
      if (keep && qmask != nullptr) keep = (qmask[item >> 6] >> (63 - (item & 63))) & 1ull;
      if (keep) {
        const int pos = atomicAdd(&cnt[qi], 1);
        lists[static_cast<int64_t>(qi) * capw + pos] = c;
      }
    }
    wave_sync_memory();
    if (cnt[qi] > capw - kWave) {
      const uint64_t nt =
          wave_compact(lists + static_cast<int64_t>(qi) * capw, &cnt[qi], scratch, scratch_n, k);
      if (lane_id() == 0 && nt > t) tau[qi] = nt;
      wave_sync_memory();
    }
    return tau[qi];
  }
};

}  // namespace rt
