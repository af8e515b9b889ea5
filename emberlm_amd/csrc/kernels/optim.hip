// AdamW update, SGD, and the gradient-clipping sum of squares and scale.
//
// Reference: adamw_step_kernel_f32 (src/core/optim.cu:54-73) and
// sum_sq_kernel_f32 + atomicAdd (optim.cu:221-239).  The AdamW kernel is the
// same element formula streamed as float4 (28 bytes per parameter of HBM
// traffic); the sum of squares is a two-stage fixed-order reduction so the
// clip norm is reproducible, all of a model's gradients in one launch (the
// reference launches one kernel per parameter, optim.cu:262-270, and scales
// them one by one, optim.cu:277-289).
#include <vector>

#include "common.h"

// No FMA contraction in this file: the float4 and scalar paths (taken for
// chunks that start off a 16-byte boundary) must round identically, so an
// offloaded, chunked update equals the on-device one bit for bit.
#pragma clang fp contract(off)

using namespace ember;

namespace {

constexpr int kThreads = 256;
// Sum of squares: each lane keeps four float4 loads in flight, and a tensor
// gets one workgroup per 16 floats per lane up to this many, enough loads in
// flight to stream the gradients of a 1.7B-parameter model at HBM rate.
constexpr int kSumsqBlocksPerTensor = 1024;
constexpr int kSumsqPerThread = 16;

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

// One tensor of a batched launch: its elements, the first block of the
// launch that is its (also its first partial), its number of blocks, and
// whether its float4 loads are aligned.
struct ListItem {
  const float* x;
  int64_t n;
  int64_t first;
  int32_t blocks;
  int32_t vec;
};

// The tensor that block `blk` of a batched launch works on (items sorted by
// `first`, which starts at 0).
__device__ __forceinline__ ListItem find_item(const ListItem* __restrict__ items, int count,
                                              int64_t blk) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (items[mid].first <= blk) lo = mid;
    else hi = mid - 1;
  }
  return items[lo];
}

// Block b of nb: its sum of x[i]^2 over a fixed set of i, in a fixed order
// (four running sums per lane, then a fixed tree), so the total does not
// depend on timing or on how the tensors are grouped into launches.
template <bool VEC>
__device__ __forceinline__ float sumsq_block(const gfloat* __restrict__ x, int64_t n, int64_t b,
                                             int64_t nb, float* red) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  const int64_t stride = nb * kThreads;
  const int64_t tid = b * kThreads + threadIdx.x;
  int64_t tail = 0;
  if (VEC) {
    const int64_t n4 = n / 4;
    const gf32x4* x4 = reinterpret_cast<const gf32x4*>(x);
    int64_t i = tid;
    for (; i + 3 * stride < n4; i += 4 * stride) {
      const f32x4 v0 = x4[i], v1 = x4[i + stride], v2 = x4[i + 2 * stride], v3 = x4[i + 3 * stride];
      a0 += v0[0] * v0[0] + v0[1] * v0[1] + v0[2] * v0[2] + v0[3] * v0[3];
      a1 += v1[0] * v1[0] + v1[1] * v1[1] + v1[2] * v1[2] + v1[3] * v1[3];
      a2 += v2[0] * v2[0] + v2[1] * v2[1] + v2[2] * v2[2] + v2[3] * v2[3];
      a3 += v3[0] * v3[0] + v3[1] * v3[1] + v3[2] * v3[2] + v3[3] * v3[3];
    }
    for (; i < n4; i += stride) {
      const f32x4 v = x4[i];
      a0 += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
    tail = n4 * 4;
  }
  for (int64_t j = tail + tid; j < n; j += stride) a0 += x[j] * x[j];
  return block_sum((a0 + a1) + (a2 + a3), red);
}

// All tensors of a list in one launch: part[block] = that block's partial.
__global__ __launch_bounds__(kThreads) void sumsq_list(const ListItem* __restrict__ items,
                                                       int count, float* __restrict__ part) {
  __shared__ float red[kThreads / kWave];
  const ListItem it = find_item(items, count, blockIdx.x);
  const int64_t b = static_cast<int64_t>(blockIdx.x) - it.first;
  const float a = it.vec ? sumsq_block<true>(as_global(it.x), it.n, b, it.blocks, red)
                         : sumsq_block<false>(as_global(it.x), it.n, b, it.blocks, red);
  if (threadIdx.x == 0) part[blockIdx.x] = a;
}

// x *= alpha for every tensor of a list in one launch.
__global__ __launch_bounds__(kThreads) void scale_list(const ListItem* __restrict__ items,
                                                       int count, float alpha) {
  const ListItem it = find_item(items, count, blockIdx.x);
  gfloat* x = as_global(const_cast<float*>(it.x));  // a pointer from the table
  const int64_t stride = static_cast<int64_t>(it.blocks) * kThreads;
  const int64_t tid = (static_cast<int64_t>(blockIdx.x) - it.first) * kThreads + threadIdx.x;
  int64_t tail = 0;
  if (it.vec) {
    gf32x4* x4 = reinterpret_cast<gf32x4*>(x);
    const int64_t n4 = it.n / 4;
    for (int64_t i = tid; i < n4; i += stride) x4[i] = x4[i] * alpha;
    tail = n4 * 4;
  }
  for (int64_t j = tail + tid; j < it.n; j += stride) x[j] = x[j] * alpha;
}

// out[0] = sum of the np partials in double, in a fixed order: four running
// sums per lane over a fixed stride, then a fixed tree.
constexpr int kPartsThreads = 1024;
__global__ __launch_bounds__(kPartsThreads) void sum_parts(const float* __restrict__ part,
                                                           int64_t np, float* __restrict__ out) {
  __shared__ double red[kPartsThreads];
  constexpr int64_t K = kPartsThreads;
  double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
  int64_t i = threadIdx.x;
  for (; i + 3 * K < np; i += 4 * K) {
    a0 += part[i];
    a1 += part[i + K];
    a2 += part[i + 2 * K];
    a3 += part[i + 3 * K];
  }
  for (; i < np; i += K) a0 += part[i];
  red[threadIdx.x] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  for (int o = kPartsThreads / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = static_cast<float>(red[0]);
}

}  // namespace

namespace {

// p -= lr * g as one fused multiply-add, fma(-lr, g, p): the single rounding
// nvcc gives the reference's sgd_step_kernel_f32 (src/core/optim.cu:14-20),
// whose p[i] -= lr * g[i] it contracts by default (-fmad=true).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void sgd_kernel(float* __restrict__ p,
                                                       const float* __restrict__ g, int64_t n,
                                                       float lr) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (VEC) {
    for (int64_t i = tid; i < n / 4; i += stride) {
      f32x4 pp = reinterpret_cast<f32x4*>(p)[i];
      const f32x4 gg = reinterpret_cast<const f32x4*>(g)[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) pp[e] = __builtin_fmaf(-lr, gg[e], pp[e]);
      reinterpret_cast<f32x4*>(p)[i] = pp;
    }
    for (int64_t i = n / 4 * 4 + tid; i < n; i += stride) p[i] = __builtin_fmaf(-lr, g[i], p[i]);
  } else {
    for (int64_t i = tid; i < n; i += stride) p[i] = __builtin_fmaf(-lr, g[i], p[i]);
  }
}

}  // namespace

extern "C" int ember_sgd(float* p, const float* g, int64_t n, float lr, ember_stream_t s) {
  if (n < 0) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  if (!p || !g) return EMBER_EINVAL;
  const bool vec = aligned16(p) && aligned16(g);
  const unsigned grid = grid_1d(vec ? (n + 3) / 4 : n, kThreads, 65536);
  if (vec)
    sgd_kernel<true><<<grid, kThreads, 0, as_stream(s)>>>(p, g, n, lr);
  else
    sgd_kernel<false><<<grid, kThreads, 0, as_stream(s)>>>(p, g, n, lr);
  return launch_status();
}

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
  const unsigned grid = grid_1d(vec ? (n + 3) / 4 : n, kThreads, max_blocks > 0 ? max_blocks : 65536);
  if (vec)
    adamw_kernel<true><<<grid, kThreads, 0, as_stream(s)>>>(p, g, m, v, n, lr, beta1, beta2, eps,
                                                            wd, bc1, bc2);
  else
    adamw_kernel<false><<<grid, kThreads, 0, as_stream(s)>>>(p, g, m, v, n, lr, beta1, beta2, eps,
                                                             wd, bc1, bc2);
  return launch_status();
}

namespace {

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Builds the item table of `count` tensors (blocks per tensor from
// blocks_of(n); empty tensors are left out) and copies it to `dev_items` on
// stream st; returns the total number of blocks, or a negative status.
template <typename BlocksOf>
int64_t upload_items(const float* const* ptrs, const int64_t* sizes, int count, ListItem* dev_items,
                     hipStream_t st, BlocksOf blocks_of, int* kept) {
  std::vector<ListItem> items;
  items.reserve(static_cast<size_t>(count));
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t n = sizes[i];
    if (n < 0 || (n > 0 && !ptrs[i])) return -EMBER_EINVAL;
    if (n == 0) continue;
    const int64_t nb = blocks_of(n);
    items.push_back(ListItem{ptrs[i], n, total, static_cast<int32_t>(nb),
                             aligned16(ptrs[i]) ? 1 : 0});
    total += nb;
  }
  *kept = static_cast<int>(items.size());
  if (items.empty()) return 0;
  const int rc = upload_async(dev_items, items.data(), items.size() * sizeof(ListItem), st);
  return rc ? -rc : total;
}

int64_t sumsq_blocks_of(int64_t n) {
  const int64_t nb = (n + kThreads * kSumsqPerThread - 1) / (kThreads * kSumsqPerThread);
  return nb < kSumsqBlocksPerTensor ? nb : kSumsqBlocksPerTensor;
}

int64_t scale_blocks_of(int64_t n) {
  const int64_t nb = (n + kThreads * 16 - 1) / (kThreads * 16);
  return nb < 1024 ? nb : 1024;
}

}  // namespace

extern "C" size_t ember_sumsq_workspace_bytes(int count) {
  if (count <= 0) return 0;
  return align256(static_cast<size_t>(count) * kSumsqBlocksPerTensor * sizeof(float)) +
         static_cast<size_t>(count) * sizeof(ListItem);
}

extern "C" int ember_sumsq_multi(const float* const* ptrs_host, const int64_t* sizes_host, int count,
                                 float* out, void* workspace, size_t workspace_bytes,
                                 ember_stream_t s) {
  if (count < 0 || !out || (count > 0 && (!ptrs_host || !sizes_host))) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (count == 0) return ember_fill(out, 1, 0.f, s);
  if (!workspace || workspace_bytes < ember_sumsq_workspace_bytes(count)) return EMBER_EWORKSPACE;
  float* part = static_cast<float*>(workspace);
  ListItem* items = reinterpret_cast<ListItem*>(
      static_cast<char*>(workspace) +
      align256(static_cast<size_t>(count) * kSumsqBlocksPerTensor * sizeof(float)));
  int kept = 0;
  const int64_t np = upload_items(ptrs_host, sizes_host, count, items, st, sumsq_blocks_of, &kept);
  if (np < 0) return static_cast<int>(-np);
  if (np == 0) return ember_fill(out, 1, 0.f, s);
  sumsq_list<<<static_cast<unsigned>(np), kThreads, 0, st>>>(items, kept, part);
  int rc = launch_status();
  if (rc) return rc;
  sum_parts<<<1, kPartsThreads, 0, st>>>(part, np, out);
  return launch_status();
}

extern "C" size_t ember_scale_multi_workspace_bytes(int count) {
  return count > 0 ? static_cast<size_t>(count) * sizeof(ListItem) : 0;
}

extern "C" int ember_scale_multi(float* const* ptrs_host, const int64_t* sizes_host, int count,
                                 float alpha, void* workspace, size_t workspace_bytes,
                                 ember_stream_t s) {
  if (count < 0 || (count > 0 && (!ptrs_host || !sizes_host))) return EMBER_EINVAL;
  if (count == 0) return EMBER_OK;
  if (!workspace || workspace_bytes < ember_scale_multi_workspace_bytes(count))
    return EMBER_EWORKSPACE;
  hipStream_t st = as_stream(s);
  ListItem* items = static_cast<ListItem*>(workspace);
  int kept = 0;
  const int64_t nb = upload_items(const_cast<const float* const*>(ptrs_host), sizes_host, count,
                                  items, st, scale_blocks_of, &kept);
  if (nb < 0) return static_cast<int>(-nb);
  if (nb == 0) return EMBER_OK;
  scale_list<<<static_cast<unsigned>(nb), kThreads, 0, st>>>(items, kept, alpha);
  return launch_status();
}
