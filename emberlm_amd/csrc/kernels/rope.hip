// Rotary position embedding (non-interleaved pairs (i, i+D/2)) with llama3
// frequency scaling.
//
// Reference: rope_kernel_f32 (src/ops/rope.cu:17-56) launches one 64-thread
// block per (b,t,h) slot and re-evaluates __powf/__sinf/__cosf per element.
// Here the D/2 frequencies are computed once on the host with the same float
// formula (rope.cu:37-46) and passed by value; a thread owns one pair index i
// of one token, evaluates the angle float(pos)*freq[i] (the reference's fp32
// rounding, rope.cu:49) and an accurate sincos once, and rotates that pair in
// every head of the token.  For a fixed head the threads of a token touch
// consecutive floats, so every access is coalesced.
#include <cmath>

#include "common.h"
#include "rope_math.h"

using namespace ember;

namespace {

constexpr int kMaxPairs = kRopeMaxPairs;
using Freqs = RopeFreqs;

__global__ __launch_bounds__(256) void rope_kernel(const float* x,
                                                   float* y, int64_t BT, int64_t T,
                                                   int H, int D, int64_t pos0, int pairs_pow2,
                                                   Freqs fr, float sign) {
  const int per_block = 256 / pairs_pow2;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * per_block + threadIdx.x / pairs_pow2;
  const int i = threadIdx.x % pairs_pow2;
  const int half = D / 2;
  if (tok >= BT || i >= half) return;
  const int64_t t = tok % T;
  float sn, cs;
  rope_sincos(pos0 + t, fr.f[i], sign, sn, cs);
  const float* xb = x + tok * H * D;
  float* yb = y + tok * H * D;
  // Up to kHeads heads' pairs are loaded before any is stored (y may be x,
  // which otherwise keeps each head's loads behind the previous head's stores).
  constexpr int kHeads = 8;
  for (int h0 = 0; h0 < H; h0 += kHeads) {
    float a[kHeads], b[kHeads];
#pragma unroll
    for (int j = 0; j < kHeads; ++j)
      if (h0 + j < H) {
        a[j] = xb[(h0 + j) * D + i];
        b[j] = xb[(h0 + j) * D + i + half];
      }
#pragma unroll
    for (int j = 0; j < kHeads; ++j)
      if (h0 + j < H) {
        yb[(h0 + j) * D + i] = rope_first(a[j], b[j], cs, sn);
        yb[(h0 + j) * D + i + half] = rope_second(a[j], b[j], cs, sn);
      }
  }
}

}  // namespace

extern "C" int ember_rope_freqs_host(float* freqs_out, int D, float theta, float factor,
                                     float low_freq_factor, float high_freq_factor,
                                     int original_max_pos) {
  if (!freqs_out || D <= 0 || D % 2 != 0) return EMBER_EINVAL;
  const float low_wl = static_cast<float>(original_max_pos) / low_freq_factor;
  const float high_wl = static_cast<float>(original_max_pos) / high_freq_factor;
  for (int i = 0; i < D / 2; ++i) {
    const float base = std::pow(theta, -(2.0f * static_cast<float>(i)) / static_cast<float>(D));
    float freq = base;
    if (factor > 1.0f) {
      const float wavelen = 6.2831853f / base;
      if (wavelen > low_wl) {
        freq = base / factor;
      } else if (wavelen > high_wl) {
        const float smooth = (wavelen - high_wl) / (low_wl - high_wl);
        freq = (1.0f - smooth) * base + smooth * (base / factor);
      }
    }
    freqs_out[i] = freq;
  }
  return EMBER_OK;
}

extern "C" int ember_rope(const float* x, float* y, int64_t B, int64_t T, int64_t H, int64_t D,
                          int64_t pos0, const float* freqs_host, float sign, ember_stream_t s) {
  if (B < 0 || T < 0 || H <= 0 || D <= 0 || D % 2 != 0 || D / 2 > kMaxPairs || !freqs_host)
    return EMBER_EINVAL;
  const int64_t BT = B * T;
  if (BT == 0) return EMBER_OK;
  if (!x || !y || H > 0x7fffffff) return EMBER_EINVAL;
  Freqs fr;
  for (int i = 0; i < kMaxPairs; ++i) fr.f[i] = i < D / 2 ? freqs_host[i] : 0.f;
  int p2 = 1;
  while (p2 < D / 2) p2 <<= 1;
  const int per_block = 256 / p2;
  const int64_t nb = (BT + per_block - 1) / per_block;
  if (nb > 0x7fffffff) return EMBER_EINVAL;
  rope_kernel<<<static_cast<unsigned>(nb), 256, 0, as_stream(s)>>>(
      x, y, BT, T, static_cast<int>(H), static_cast<int>(D), pos0, p2, fr, sign);
  return launch_status();
}
