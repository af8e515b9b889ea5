// AdamW update and the grad-norm sum of squares.
//
// Reference: adamw_step_kernel_f32 (src/core/optim.cu:54-73) and
// sum_sq_kernel_f32 + atomicAdd (optim.cu:221-239).  The AdamW kernel is the
// same element formula streamed as float4 (28 bytes per parameter of HBM
// traffic); the sum of squares is a two-stage fixed-order reduction so the
// clip norm is reproducible.
#include "common.h"

// No FMA contraction in this file: the float4 and scalar paths (taken for
// chunks that start off a 16-byte boundary) must round identically, so an
// offloaded, chunked update equals the on-device one bit for bit.
#pragma clang fp contract(off)

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kSumsqBlocksPerTensor = 256;

__device__ __forceinline__ void adamw_one(float& p, float g, float& m, float& v, float b1, float b2,
                                          float lr, float wd, float eps, float bc1, float bc2) {
  const float mi = b1 * m + (1.0f - b1) * g;
  const float vi = b2 * v + (1.0f - b2) * g * g;
  m = mi;
  v = vi;
  const float mh = mi / bc1;
  const float vh = vi / bc2;
  const float upd = mh / (sqrtf(vh) + eps);
  p = p - lr * (upd + wd * p);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void adamw_kernel(float* __restrict__ p,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ m,
                                                         float* __restrict__ v, int64_t n,
                                                         float lr, float b1, float b2, float eps,
                                                         float wd, float bc1, float bc2) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (VEC) {
    const int64_t n4 = n / 4;
    for (int64_t i = tid; i < n4; i += stride) {
      f32x4 pp = reinterpret_cast<f32x4*>(p)[i];
      const f32x4 gg = reinterpret_cast<const f32x4*>(g)[i];
      f32x4 mm = reinterpret_cast<f32x4*>(m)[i];
      f32x4 vv = reinterpret_cast<f32x4*>(v)[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pp[e], me = mm[e], ve = vv[e];
        adamw_one(pe, gg[e], me, ve, b1, b2, lr, wd, eps, bc1, bc2);
        pp[e] = pe;
        mm[e] = me;
        vv[e] = ve;
      }
      reinterpret_cast<f32x4*>(p)[i] = pp;
      reinterpret_cast<f32x4*>(m)[i] = mm;
      reinterpret_cast<f32x4*>(v)[i] = vv;
    }
    for (int64_t i = n4 * 4 + tid; i < n; i += stride)
      adamw_one(p[i], g[i], m[i], v[i], b1, b2, lr, wd, eps, bc1, bc2);
  } else {
    for (int64_t i = tid; i < n; i += stride)
      adamw_one(p[i], g[i], m[i], v[i], b1, b2, lr, wd, eps, bc1, bc2);
  }
}

__global__ __launch_bounds__(kThreads) void sumsq_partial(const float* __restrict__ x, int64_t n,
                                                          float* __restrict__ part) {
  __shared__ float red[kThreads / kWave];
  float a = 0.f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    a += x[i] * x[i];
  a = block_sum(a, red);
  if (threadIdx.x == 0) part[blockIdx.x] = a;
}

__global__ __launch_bounds__(kThreads) void sum_parts(const float* __restrict__ part, int64_t np,
                                                      float* __restrict__ out) {
  __shared__ double red[kThreads];
  double a = 0.0;
  for (int64_t i = threadIdx.x; i < np; i += kThreads) a += part[i];
  red[threadIdx.x] = a;
  __syncthreads();
  for (int o = kThreads / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = static_cast<float>(red[0]);
}

}  // namespace

extern "C" int ember_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr,
                           float beta1, float beta2, float eps, float wd, float bc1, float bc2,
                           ember_stream_t s) {
  return ember_adamw_bounded(p, g, m, v, n, lr, beta1, beta2, eps, wd, bc1, bc2, 0, s);
}

extern "C" int ember_adamw_bounded(float* p, const float* g, float* m, float* v, int64_t n,
                                   float lr, float beta1, float beta2, float eps, float wd,
                                   float bc1, float bc2, int max_blocks, ember_stream_t s) {
  if (n < 0 || max_blocks < 0) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  if (!p || !g || !m || !v) return EMBER_EINVAL;
  // A bounded launch shares the GPU with another kernel, so it takes the
  // scalar form: 22 registers per lane instead of 62 lets its waves sit next
  // to a GEMM's or the attention forward's on the same SIMD.
  const bool vec = max_blocks == 0 && aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v);
  const unsigned grid = grid_1d(vec ? (n + 3) / 4 : n, kThreads, max_blocks > 0 ? max_blocks : 8192);
  if (vec)
    adamw_kernel<true><<<grid, kThreads, 0, as_stream(s)>>>(p, g, m, v, n, lr, beta1, beta2, eps,
                                                            wd, bc1, bc2);
  else
    adamw_kernel<false><<<grid, kThreads, 0, as_stream(s)>>>(p, g, m, v, n, lr, beta1, beta2, eps,
                                                             wd, bc1, bc2);
  return launch_status();
}

extern "C" size_t ember_sumsq_workspace_bytes(int count) {
  return count > 0 ? static_cast<size_t>(count) * kSumsqBlocksPerTensor * sizeof(float) : 0;
}

extern "C" int ember_sumsq_multi(const float* const* ptrs_host, const int64_t* sizes_host, int count,
                                 float* out, void* workspace, size_t workspace_bytes,
                                 ember_stream_t s) {
  if (count < 0 || !out || (count > 0 && (!ptrs_host || !sizes_host))) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (count == 0) return ember_fill(out, 1, 0.f, s);
  if (!workspace || workspace_bytes < ember_sumsq_workspace_bytes(count)) return EMBER_EWORKSPACE;
  float* part = static_cast<float*>(workspace);
  int64_t np = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t n = sizes_host[i];
    if (n < 0 || (n > 0 && !ptrs_host[i])) return EMBER_EINVAL;
    if (n == 0) continue;
    int64_t nb = (n + kThreads * 8 - 1) / (kThreads * 8);
    if (nb > kSumsqBlocksPerTensor) nb = kSumsqBlocksPerTensor;
    sumsq_partial<<<static_cast<unsigned>(nb), kThreads, 0, st>>>(ptrs_host[i], n, part + np);
    const int rc = launch_status();
    if (rc) return rc;
    np += nb;
  }
  sum_parts<<<1, kThreads, 0, st>>>(part, np, out);
  return launch_status();
}
