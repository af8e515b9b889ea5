// Greedy token choice on the device.
//
// Reference: argmax_cpu (src/core/sampling.cpp:12-19) scans a row copied to
// the host: best = 0, and index i replaces it only when x[i] > x[best].  So
// the result is the first index of the largest non-NaN value, NaNs never win,
// and a NaN at index 0 wins by default (nothing compares greater).  Here one
// workgroup reduces a row with the same order on (value, index) -- larger
// value first, then smaller index, NaN below everything -- which is
// associative, so the parallel reduction returns the scan's index exactly,
// and only the B int64 results cross PCIe instead of B*V floats.
#include <cmath>

#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;

struct Best {
  float v;
  int64_t i;
};

// True when (v, i) precedes (bv, bi): larger value, then smaller index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  if (v != v) return false;    // NaN never wins
  if (bv != bv) return true;   // anything beats a NaN placeholder
  return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(kThreads) void argmax_rows_kernel(const float* __restrict__ x,
                                                               int64_t n,
                                                               int64_t* __restrict__ out) {
  __shared__ float sv[kThreads / kWave];
  __shared__ int64_t si[kThreads / kWave];
  const float* row = x + static_cast<int64_t>(blockIdx.x) * n;
  float bv = NAN;
  int64_t bi = INT64_MAX;
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    const float v = row[i];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int64_t oi = __shfl_xor(bi, o, kWave);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kThreads / kWave; ++k)
      if (better(sv[k], si[k], bv, bi)) {
        bv = sv[k];
        bi = si[k];
      }
    // A NaN first element is never replaced by the scan; all-NaN rows give 0 too.
    out[blockIdx.x] = (row[0] != row[0] || bi == INT64_MAX) ? 0 : bi;
  }
}

}  // namespace

extern "C" int ember_argmax_rows(const float* x, int64_t rows, int64_t n, int64_t* out,
                                 ember_stream_t s) {
  if (rows < 0 || n < 0) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (n == 0 || !x || !out || rows > 0x7fffffff) return EMBER_EINVAL;
  argmax_rows_kernel<<<static_cast<unsigned>(rows), kThreads, 0, as_stream(s)>>>(x, n, out);
  return launch_status();
}
