// 1-bit codes on the fp4 matrix cores (v_mfma_scale_f32_{32x32x64,16x16x128}_f8f6f4 with e2m1
// operands): the nibble layout of a 32-bit word of a code, and the scaled, biased accumulators
// of the scans' main passes. Shared by the blocked scan (scan_blocked.h) and the per-wave scan
// of small batches (scan_bits_mfma.hip).
//
// A lane feeds 32 K elements of an operand per MFMA: 32 nibbles in four dwords. A 32-bit word b
// of an item fills them in place -- nibble e of dword n holds bit 4 e + n (the K order inside an
// operand is free when items and queries share it), masked to e2m1 0.5, 1.0, 2.0 for n = 0, 1,
// 2 and, for dword 3, bit 3 moved one place down (2.0; bit 3 is the sign): five VALU per 32 bits,
// no table. The query nibble of the same slot is +-4.0, +-2.0, +-1.0, +-1.0 (sign set for a 0
// bit), so every product of an item 1 with a query bit is +-2 exactly and an item 0 adds 0: the
// sum over the code is 4 popcount(x & q) - 2 popcount(x), and the Hamming score
// 64 W - 2 popcount(q ^ x) is that sum plus the query's start acc0 = 64 W - 2 popcount(q).
#pragma once

#include <cstdint>

namespace rt {
namespace fp4 {

typedef int v4i __attribute__((ext_vector_type(4)));

// e2m1 format code of the MFMA's cbsz / blgp operands
constexpr int kFmt = 4;
// unit block scale (e8m0 0x7f = 2^0) in each byte
constexpr int kUnitScale = 0x7f7f7f7f;

__device__ inline v4i item_frag(uint32_t b) {
  return v4i{static_cast<int>(b & 0x11111111u), static_cast<int>(b & 0x22222222u),
             static_cast<int>(b & 0x44444444u), static_cast<int>((b >> 1) & 0x44444444u)};
}

// +4.0 0b0110, +2.0 0b0100, +1.0 0b0010; the sign (bit 3) set where the query bit is 0
__device__ inline v4i query_frag(uint32_t b) {
  constexpr uint32_t kMag[4] = {0x66666666u, 0x44444444u, 0x22222222u, 0x22222222u};
  v4i r;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    r[n] = static_cast<int>((kMag[n] | 0x88888888u) ^ (((b >> n) & 0x11111111u) << 3));
  }
  return r;
}

// Main passes: the accumulator of output tile p (p < 4, a different one per tile a wave holds
// in flight) starts at the inline constant hit_bias(p) = 4.0 / 2^p and the query operand runs
// at block scale 2^-(9 + p) (e8m0 0x76 - p in each byte), so a 512-bit row's sum
// sum_x (4 q - 2) 2^-(9 + p) lies in [-2, 2] / 2^p, in multiples of 2^-(8 + p) (exact in fp32),
// and a row ends in [2, 6] / 2^p, positive (a mask term of -8192 or less makes it negative).
// Positive floats order as their bits do as signed ints, and negative ones fall below them, so
// the hit test is signed-int maxima of the raw accumulator bits against hit_thresh.
// (A different constant per tile: the compiler would otherwise keep a shared one in registers
// and copy it into every accumulator.)
__device__ constexpr float hit_bias(int p) { return 4.0f / static_cast<float>(1 << p); }
__device__ constexpr int hit_scale(int p) { return 0x76767676 - 0x01010101 * p; }

// The score of tile p's accumulator value v for a query whose sum starts at acc0 (exact: v minus
// the bias is a multiple of 2^-(8 + p) below 2^14 in magnitude).
__device__ inline int32_t hit_score(float v, int32_t acc0, int p) {
  return static_cast<int32_t>((v - hit_bias(p)) * static_cast<float>(512 << p)) + acc0;
}

// Tile p's threshold for the score threshold th: hit_bias(p) + (th - acc0) 2^-(9 + p) as the
// signed int of its bits; INT32_MIN (every row hits) when that is not positive (th below every
// score: no bound yet).
__device__ inline int32_t hit_thresh(int32_t th, int32_t acc0, int p) {
  const float t = hit_bias(p) + (static_cast<float>(th) - static_cast<float>(acc0)) /
                                    static_cast<float>(512 << p);
  return t > 0.0f ? __builtin_bit_cast(int32_t, t) : INT32_MIN;
}

}  // namespace fp4
}  // namespace rt
