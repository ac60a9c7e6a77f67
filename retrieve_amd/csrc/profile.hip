// Optional HIP-event timing of the dominant kernel of each call (the main scan), for the
// benchmark's live roofline figure. Off by default; when on, each main-scan launch is
// bracketed by an event pair recorded on the launch stream.
#include <vector>

#include "rt_common.h"
#include "profile.h"

namespace rt {

namespace {
bool g_enabled = false;
std::vector<hipEvent_t> g_pool;  // pairs: start, stop
size_t g_used = 0;               // events in use (2 per launch)
}  // namespace

bool profile_on() { return g_enabled; }

void profile_begin(hipStream_t stream, hipEvent_t* stop_out) {
  *stop_out = nullptr;
  if (!g_enabled) return;
  while (g_pool.size() < g_used + 2) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    g_pool.push_back(e);
  }
  hipEvent_t start = g_pool[g_used];
  hipEvent_t stop = g_pool[g_used + 1];
  g_used += 2;
  (void)hipEventRecord(start, stream);
  *stop_out = stop;
}

void profile_end(hipStream_t stream, hipEvent_t stop) {
  if (stop != nullptr) (void)hipEventRecord(stop, stream);
}

}  // namespace rt

extern "C" int rt_profile_enable(int on) {
  rt::g_enabled = on != 0;
  rt::g_used = 0;
  return rt::kOk;
}

extern "C" int rt_profile_collect(double* total_ms, int64_t* launches) {
  double total = 0.0;
  const int64_t n = static_cast<int64_t>(rt::g_used / 2);
  for (int64_t i = 0; i < n; ++i) {
    RT_CHECK_HIP(hipEventSynchronize(rt::g_pool[2 * i + 1]));
    float ms = 0.f;
    RT_CHECK_HIP(hipEventElapsedTime(&ms, rt::g_pool[2 * i], rt::g_pool[2 * i + 1]));
    total += ms;
  }
  *total_ms = total;
  *launches = n;
  rt::g_used = 0;
  return rt::kOk;
}
