// Shared helpers for the gfx950 kernels behind include/ember_hip.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ember_hip.h"

namespace ember {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Global-memory views of a pointer the compiler cannot place (one loaded from
// a table in device memory is a generic pointer): accesses through them are
// global_* instructions, not flat_* ones, which also count on the LDS wait
// counter and so hold up the kernel's LDS waits until the stores complete.
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) f32x4 gf32x4;
__device__ __forceinline__ gfloat* as_global(float* p) { return (gfloat*)p; }
__device__ __forceinline__ const gfloat* as_global(const float* p) { return (const gfloat*)p; }

inline int status_of(hipError_t e) { return e == hipSuccess ? EMBER_OK : static_cast<int>(e); }

// Status of the most recent launch on this thread.
inline int launch_status() { return status_of(hipGetLastError()); }

inline hipStream_t as_stream(ember_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Copies `bytes` of host memory to device memory on stream st through a
// page-locked staging buffer owned by the library, so the caller's host
// memory may be reused as soon as this returns.  The staging buffer is
// reused by the next call once this copy has left (an event, waited on by
// the next call).  Small tables only (launch descriptors).
int upload_async(void* dev_dst, const void* host_src, size_t bytes, hipStream_t st);

inline unsigned grid_1d(int64_t n, int threads, int64_t cap = 1 << 20) {
  int64_t g = (n + threads - 1) / threads;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

// Full-wave (64-lane) reductions through DPP-free shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum for blockDim.x = 64 * nwaves; result valid in every lane.
// `smem` holds at least nwaves floats.  Fixed reduction order (deterministic).
__device__ __forceinline__ float block_sum(float v, float* smem) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < nw; ++i) t += smem[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* smem) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, smem[i]);
  return t;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace ember
