// RoPE arithmetic shared by the rotary kernel (rope.hip) and the fused
// QK-Norm + RoPE kernels (norm.hip), so that both evaluate the same float
// expressions and give the same bits.  Pairs are (i, i + D/2), the reference's
// non-interleaved layout (src/ops/rope.cu:17-56).
#pragma once

#include <cstdint>

namespace ember {

constexpr int kRopeMaxPairs = 128;  // D <= 256

// The D/2 pair frequencies, computed on the host (ember_rope_freqs_host) and
// passed by value.
struct RopeFreqs {
  float f[kRopeMaxPairs];
};

// sin and cos of float(pos) * freq (the reference's fp32 angle, rope.cu:49),
// sin multiplied by sign (+1 forward, -1 for the transpose).
__device__ __forceinline__ void rope_sincos(int64_t pos, float freq, float sign, float& sn,
                                            float& cs) {
  const float ang = static_cast<float>(pos) * freq;
  sincosf(ang, &sn, &cs);
  sn *= sign;
}

// Rotated pair: a is element i, b element i + D/2.  The roundings are
// spelled out (one product rounded, the other fused into the add) so that
// every kernel using these gets the same bits, whatever the compiler would
// otherwise contract in its context.
__device__ __forceinline__ float rope_first(float a, float b, float cs, float sn) {
#pragma clang fp contract(off)
  return fmaf(a, cs, -(b * sn));
}
__device__ __forceinline__ float rope_second(float a, float b, float cs, float sn) {
#pragma clang fp contract(off)
  return fmaf(b, cs, a * sn);
}

}  // namespace ember
