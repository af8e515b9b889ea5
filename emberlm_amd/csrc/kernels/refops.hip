// The reference's unfused attention-chain ops, kept for the ops:: API:
// softmax (src/ops/softmax.cu:17-80), causal mask (src/ops/mask.cu:15-52),
// repeat_kv / group sum (src/ops/repeat_kv.cu:16-43) and permute
// (src/ops/permute.cu:20-127).  The training block uses the fused attention
// kernels instead; these exist so the reference's op-level API and tests
// stay available.  Offsets are 64-bit (the reference's mask launch overflows
// grid.y at B*H*T/8 > 65535, mask.cu:71-73), and permute takes its shape and
// permutation by value instead of three cudaMalloc/cudaMemcpy round trips and
// a device synchronize per call (permute.cu:76-100).
#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void softmax_fwd_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y, int64_t rows,
                                                               int64_t N) {
  __shared__ float red[kThreads / kWave];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float* xr = x + r * N;
    float* yr = y + r * N;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < N; i += kThreads) m = fmaxf(m, xr[i]);
    m = block_max(m, red);
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < N; i += kThreads) s += expf(xr[i] - m);
    s = block_sum(s, red);
    const float inv = 1.0f / s;
    for (int64_t i = threadIdx.x; i < N; i += kThreads) yr[i] = expf(xr[i] - m) * inv;
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void softmax_bwd_kernel(const float* __restrict__ y,
                                                               const float* __restrict__ g,
                                                               float* __restrict__ dx,
                                                               int64_t rows, int64_t N) {
  __shared__ float red[kThreads / kWave];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float* yr = y + r * N;
    const float* gr = g + r * N;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < N; i += kThreads) s += gr[i] * yr[i];
    s = block_sum(s, red);
    for (int64_t i = threadIdx.x; i < N; i += kThreads) dx[r * N + i] = yr[i] * (gr[i] - s);
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void causal_mask_kernel(const float* in, float* out,
                                                               int64_t total, int64_t Tq,
                                                               int64_t Tk, int64_t q0, float fill) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t k = i % Tk;
    const int64_t q = (i / Tk) % Tq;
    out[i] = (k > q0 + q) ? fill : in[i];
  }
}

__global__ __launch_bounds__(kThreads) void repeat_kv_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y, int64_t total,
                                                             int64_t Hk, int64_t group, int64_t D) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t H = Hk * group;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t d = i % D;
    const int64_t h = (i / D) % H;
    const int64_t bt = i / (D * H);
    y[i] = x[(bt * Hk + h / group) * D + d];
  }
}

__global__ __launch_bounds__(kThreads) void repeat_kv_sum_kernel(const float* __restrict__ y,
                                                                 float* __restrict__ x,
                                                                 int64_t total, int64_t Hk,
                                                                 int64_t group, int64_t D) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t d = i % D;
    const int64_t hk = (i / D) % Hk;
    const int64_t bt = i / (D * Hk);
    float a = 0.f;
    for (int64_t j = 0; j < group; ++j) a += y[((bt * Hk * group) + hk * group + j) * D + d];
    x[i] = a;
  }
}

struct PermuteArgs {
  int ndim;
  int64_t out_shape[6];
  int64_t in_stride_of_out_dim[6];
};

__global__ __launch_bounds__(kThreads) void permute_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, int64_t total,
                                                           PermuteArgs a) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += stride) {
    int64_t rem = i, src = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % a.out_shape[d];
      rem /= a.out_shape[d];
      src += c * a.in_stride_of_out_dim[d];
    }
    y[i] = x[src];
  }
}

unsigned rows_grid(int64_t rows) { return static_cast<unsigned>(rows < 262144 ? rows : 262144); }

}  // namespace

extern "C" int ember_softmax_fwd(const float* x, float* y, int64_t rows, int64_t N,
                                 ember_stream_t s) {
  if (rows < 0 || N <= 0) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (!x || !y) return EMBER_EINVAL;
  softmax_fwd_kernel<<<rows_grid(rows), kThreads, 0, as_stream(s)>>>(x, y, rows, N);
  return launch_status();
}

extern "C" int ember_softmax_bwd(const float* y, const float* g, float* dx, int64_t rows,
                                 int64_t N, ember_stream_t s) {
  if (rows < 0 || N <= 0) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  if (!y || !g || !dx) return EMBER_EINVAL;
  softmax_bwd_kernel<<<rows_grid(rows), kThreads, 0, as_stream(s)>>>(y, g, dx, rows, N);
  return launch_status();
}

extern "C" int ember_causal_mask(const float* in, float* out, int64_t rows, int64_t Tq,
                                 int64_t Tk, int64_t q0, float fill, ember_stream_t s) {
  if (rows < 0 || Tq <= 0 || Tk <= 0) return EMBER_EINVAL;
  const int64_t total = rows * Tk;
  if (total == 0) return EMBER_OK;
  if (!in || !out) return EMBER_EINVAL;
  causal_mask_kernel<<<grid_1d(total, kThreads, 65536), kThreads, 0, as_stream(s)>>>(
      in, out, total, Tq, Tk, q0, fill);
  return launch_status();
}

extern "C" int ember_repeat_kv(const float* x, float* y, int64_t BT, int64_t Hk, int64_t group,
                               int64_t D, ember_stream_t s) {
  if (BT < 0 || Hk <= 0 || group <= 0 || D <= 0) return EMBER_EINVAL;
  const int64_t total = BT * Hk * group * D;
  if (total == 0) return EMBER_OK;
  if (!x || !y) return EMBER_EINVAL;
  repeat_kv_kernel<<<grid_1d(total, kThreads, 65536), kThreads, 0, as_stream(s)>>>(x, y, total, Hk,
                                                                                   group, D);
  return launch_status();
}

extern "C" int ember_repeat_kv_sum(const float* y, float* x, int64_t BT, int64_t Hk,
                                   int64_t group, int64_t D, ember_stream_t s) {
  if (BT < 0 || Hk <= 0 || group <= 0 || D <= 0) return EMBER_EINVAL;
  const int64_t total = BT * Hk * D;
  if (total == 0) return EMBER_OK;
  if (!x || !y) return EMBER_EINVAL;
  repeat_kv_sum_kernel<<<grid_1d(total, kThreads, 65536), kThreads, 0, as_stream(s)>>>(
      y, x, total, Hk, group, D);
  return launch_status();
}

extern "C" int ember_permute(const float* x, float* y, int ndim, const int64_t* shape_host,
                             const int* perm_host, ember_stream_t s) {
  if (ndim < 1 || ndim > 6 || !shape_host || !perm_host) return EMBER_EINVAL;
  int64_t in_stride[6];
  in_stride[ndim - 1] = 1;
  for (int i = ndim - 2; i >= 0; --i) in_stride[i] = in_stride[i + 1] * shape_host[i + 1];
  PermuteArgs a{};
  a.ndim = ndim;
  int64_t total = 1;
  bool seen[6] = {false, false, false, false, false, false};
  for (int i = 0; i < ndim; ++i) {
    const int p = perm_host[i];
    if (p < 0 || p >= ndim || seen[p] || shape_host[i] < 0) return EMBER_EINVAL;
    seen[p] = true;
    a.out_shape[i] = shape_host[p];
    a.in_stride_of_out_dim[i] = in_stride[p];
    total *= shape_host[i];
  }
  if (total == 0) return EMBER_OK;
  if (!x || !y) return EMBER_EINVAL;
  permute_kernel<<<grid_1d(total, kThreads, 65536), kThreads, 0, as_stream(s)>>>(x, y, total, a);
  return launch_status();
}
