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

constexpr int kThreads = 1024;  // one workgroup per row; 16 waves keep many loads in flight
constexpr int kUnroll = 4;

// True when (v, i) precedes (bv, bi): larger value, then smaller index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  if (v != v) return false;    // NaN never wins
  if (bv != bv) return true;   // anything beats a NaN placeholder
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void take(float v, int64_t i, float& bv, int64_t& bi) {
  if (better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void argmax_rows_kernel(const float* __restrict__ x,
                                                               int64_t n,
                                                               int64_t* __restrict__ out) {
  __shared__ float sv[kThreads / kWave];
  __shared__ int64_t si[kThreads / kWave];
  const float* row = x + static_cast<int64_t>(blockIdx.x) * n;
  float bv = NAN;
  int64_t bi = INT64_MAX;
  if (VEC) {
    // float4 chunks, kUnroll loads issued before any comparison.
    const f32x4* r4 = reinterpret_cast<const f32x4*>(row);
    const int64_t n4 = n / 4;
    for (int64_t c0 = threadIdx.x; c0 < n4; c0 += static_cast<int64_t>(kThreads) * kUnroll) {
      f32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kThreads;
        v[u] = c < n4 ? r4[c] : f32x4{NAN, NAN, NAN, NAN};
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t base = 4 * (c0 + static_cast<int64_t>(u) * kThreads);
#pragma unroll
        for (int e = 0; e < 4; ++e) take(v[u][e], base + e, bv, bi);
      }
    }
    for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += kThreads) take(row[i], i, bv, bi);
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kThreads) take(row[i], i, bv, bi);
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int64_t oi = __shfl_xor(bi, o, kWave);
    take(ov, oi, bv, bi);
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kThreads / kWave; ++k) take(sv[k], si[k], bv, bi);
    // A NaN first element is never replaced by the scan; all-NaN rows give 0 too.
    out[blockIdx.x] = (row[0] != row[0] || bi == INT64_MAX) ? 0 : bi;
  }
}

// Two-stage form for long rows: workgroup (p, row) reduces slice p of the row
// to a packed key -- order-preserving bits of the value above, the inverted
// index below, NaN as 0 -- so the larger key is the scan's winner; stage 2
// takes the largest key of each row.  +0 and -0 compare equal in the scan and
// are packed alike.
constexpr int kPartThreads = 256;
constexpr int64_t kPartChunk = 8192;  // elements per stage-1 workgroup (at least)
constexpr int kMaxParts = 64;

__device__ __forceinline__ uint64_t pack_key(float v, int64_t i) {
  if (v != v) return 0;
  const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
}

int64_t parts_for(int64_t n) {
  int64_t p = (n + kPartChunk - 1) / kPartChunk;
  return p < 1 ? 1 : (p > kMaxParts ? kMaxParts : p);
}

template <bool VEC>
__global__ __launch_bounds__(kPartThreads) void argmax_part_kernel(const float* __restrict__ x,
                                                                   int64_t n, int64_t chunk,
                                                                   uint64_t* __restrict__ keys) {
  __shared__ uint64_t sk[kPartThreads / kWave];
  const int64_t row = blockIdx.y;
  const float* r = x + row * n;
  const int64_t b = blockIdx.x * chunk;
  const int64_t e = b + chunk < n ? b + chunk : n;
  float bv = NAN;
  int64_t bi = INT64_MAX;
  if (VEC) {  // chunk and n are multiples of 4 here
    const f32x4* r4 = reinterpret_cast<const f32x4*>(r);
    for (int64_t c0 = b / 4 + threadIdx.x; c0 < e / 4; c0 += kPartThreads * kUnroll) {
      f32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kPartThreads;
        v[u] = c < e / 4 ? r4[c] : f32x4{NAN, NAN, NAN, NAN};
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          take(v[u][q], 4 * (c0 + static_cast<int64_t>(u) * kPartThreads) + q, bv, bi);
    }
  } else {
    for (int64_t i = b + threadIdx.x; i < e; i += kPartThreads) take(r[i], i, bv, bi);
  }
  uint64_t key = bi == INT64_MAX ? 0 : pack_key(bv, bi);
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const uint64_t ok = __shfl_xor(key, o, kWave);
    key = ok > key ? ok : key;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) sk[threadIdx.x / kWave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kPartThreads / kWave; ++w) key = sk[w] > key ? sk[w] : key;
    keys[row * gridDim.x + blockIdx.x] = key;
  }
}

__global__ __launch_bounds__(kWave) void argmax_final_kernel(const float* __restrict__ x,
                                                             int64_t n, const uint64_t* keys,
                                                             int parts, int64_t* __restrict__ out) {
  const int64_t row = blockIdx.x;
  uint64_t key = 0;
  for (int p = threadIdx.x; p < parts; p += kWave) {
    const uint64_t k = keys[row * parts + p];
    key = k > key ? k : key;
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const uint64_t ok = __shfl_xor(key, o, kWave);
    key = ok > key ? ok : key;
  }
  if (threadIdx.x == 0) {
    const float x0 = x[row * n];
    out[row] = (x0 != x0 || key == 0) ? 0
                                      : static_cast<int64_t>(0xFFFFFFFFu -
                                                             static_cast<uint32_t>(key));
  }
}

}  // namespace

extern "C" size_t ember_argmax_rows_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  const int64_t p = parts_for(n);
  return p > 1 ? static_cast<size_t>(rows * p) * sizeof(uint64_t) : 0;
}

extern "C" int ember_argmax_rows_ws(const float* x, int64_t rows, int64_t n, int64_t* out,
                                    void* workspace, size_t workspace_bytes, ember_stream_t s) {
  if (rows < 0 || n < 0) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (n == 0 || !x || !out || rows > 65535 || n > 0xFFFFFFFFLL) return EMBER_EINVAL;
  const int64_t parts = parts_for(n);
  const size_t need = ember_argmax_rows_workspace_bytes(rows, n);
  if (parts == 1 || !workspace || workspace_bytes < need)
    return ember_argmax_rows(x, rows, n, out, s);
  hipStream_t st = as_stream(s);
  int64_t chunk = (n + parts - 1) / parts;
  chunk = (chunk + 3) / 4 * 4;
  const dim3 grid(static_cast<unsigned>(parts), static_cast<unsigned>(rows));
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  if (aligned16(x) && n % 4 == 0)
    argmax_part_kernel<true><<<grid, kPartThreads, 0, st>>>(x, n, chunk, keys);
  else
    argmax_part_kernel<false><<<grid, kPartThreads, 0, st>>>(x, n, chunk, keys);
  int rc = launch_status();
  if (rc) return rc;
  argmax_final_kernel<<<static_cast<unsigned>(rows), kWave, 0, st>>>(x, n, keys,
                                                                    static_cast<int>(parts), out);
  return launch_status();
}

extern "C" int ember_argmax_rows(const float* x, int64_t rows, int64_t n, int64_t* out,
                                 ember_stream_t s) {
  if (rows < 0 || n < 0) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (n == 0 || !x || !out || rows > 0x7fffffff) return EMBER_EINVAL;
  if (aligned16(x) && n % 4 == 0)
    argmax_rows_kernel<true><<<static_cast<unsigned>(rows), kThreads, 0, as_stream(s)>>>(x, n, out);
  else
    argmax_rows_kernel<false><<<static_cast<unsigned>(rows), kThreads, 0, as_stream(s)>>>(x, n,
                                                                                        out);
  return launch_status();
}
