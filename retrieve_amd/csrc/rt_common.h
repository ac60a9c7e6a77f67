// Shared device/host helpers of the retrieve_amd HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

namespace rt {

// ---- status / errors (host) -------------------------------------------------------------

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,  // shape / size / range problem: ValueError on the Python side
  kInvalidType = 2,      // unsupported dtype or width: TypeError
  kLaunchFailed = 3,     // a HIP call failed: RuntimeError
  kWorkspaceTooSmall = 4,
};

void set_error(const char* fmt, ...);
const char* last_error();

#define RT_CHECK_ARG(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      ::rt::set_error(__VA_ARGS__);          \
      return ::rt::kInvalidArgument;         \
    }                                        \
  } while (0)

#define RT_CHECK_HIP(expr)                                                          \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess) {                                                         \
      ::rt::set_error("%s failed: %s", #expr, hipGetErrorString(e_));               \
      return ::rt::kLaunchFailed;                                                   \
    }                                                                               \
  } while (0)

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---- order-preserving keys (device + host) ----------------------------------------------
//
// A score is turned into a uint32 that orders like the score; the selection runs on the
// composite (key << 32) | (0xffffffff - item), which orders by (score desc, item asc) when
// sorted descending, so every stage breaks ties toward the lower item index. Composite 0 is
// below every real entry and marks an empty slot.

__host__ __device__ inline uint32_t key_of_i32(int32_t v) {
  return static_cast<uint32_t>(v) ^ 0x80000000u;
}
__host__ __device__ inline int32_t i32_of_key(uint32_t k) {
  return static_cast<int32_t>(k ^ 0x80000000u);
}
__host__ __device__ inline uint32_t key_of_f32(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__host__ __device__ inline float f32_of_key(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  float f;
  memcpy(&f, &b, 4);
  return f;
}
__host__ __device__ inline uint64_t composite(uint32_t key, uint32_t item) {
  return (static_cast<uint64_t>(key) << 32) | (0xffffffffu - item);
}
__host__ __device__ inline uint32_t composite_item(uint64_t c) {
  return 0xffffffffu - static_cast<uint32_t>(c);
}
__host__ __device__ inline uint32_t composite_key(uint64_t c) {
  return static_cast<uint32_t>(c >> 32);
}

// ---- wave helpers -----------------------------------------------------------------------

constexpr int kWave = 64;

__device__ inline int lane_id() { return __lane_id(); }

// Orders this wave's earlier LDS/global writes before its later reads by other lanes of the
// same wave (the wave's memory operations complete in order once issued; the fence keeps the
// compiler from moving accesses across it and waits for outstanding ones).
__device__ inline void wave_sync_memory() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

}  // namespace rt
