// Token embedding gather and its deterministic scatter-add backward.
//
// Reference: embedding_kernel_f32 / embedding_backward_kernel_f32
// (src/ops/embedding.cu:15-39), whose backward atomically adds every token's
// gradient row into dW[id] (order-dependent fp32 sums).  Here each block owns
// a range of kIdsPerBlock vocabulary rows, scans the id list in order, compacts
// the positions that hit its range with a wave ballot (keeping ascending
// order), and adds those dy rows into its dW rows one after another, so every
// dW row is the same left-to-right sum on every run.
#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kIdsPerBlock = 128;

__global__ __launch_bounds__(kThreads) void embedding_fwd_kernel(const int64_t* __restrict__ ids,
                                                                 const float* __restrict__ w,
                                                                 float* __restrict__ out,
                                                                 int64_t n, int64_t H, int64_t V) {
  // One block per token row (grid-stride); ids outside [0,V) give zero rows.
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const int64_t id = ids[r];
    const bool ok = id >= 0 && id < V;
    for (int64_t c = threadIdx.x; c < H; c += kThreads)
      out[r * H + c] = ok ? w[id * H + c] : 0.f;
  }
}

__global__ __launch_bounds__(kThreads) void embedding_bwd_kernel(const int64_t* __restrict__ ids,
                                                                 const float* __restrict__ dy,
                                                                 float* __restrict__ dw, int64_t n,
                                                                 int64_t H, int64_t V) {
  __shared__ int hits[kThreads];
  __shared__ int wave_base[kThreads / kWave + 1];
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kIdsPerBlock;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int64_t base = 0; base < n; base += kThreads) {
    const int64_t i = base + threadIdx.x;
    const int64_t id = i < n ? ids[i] : -1;
    const bool hit = id >= v0 && id < v0 + kIdsPerBlock && id < V;
    const uint64_t ballot = __ballot(hit);
    const int before = __popcll(ballot & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (lane == 0) wave_base[wid] = __popcll(ballot);
    __syncthreads();
    if (threadIdx.x == 0) {
      int acc = 0;
      for (int w_ = 0; w_ < kThreads / kWave; ++w_) {
        const int c = wave_base[w_];
        wave_base[w_] = acc;
        acc += c;
      }
      wave_base[kThreads / kWave] = acc;
    }
    __syncthreads();
    if (hit) hits[wave_base[wid] + before] = static_cast<int>(threadIdx.x);
    __syncthreads();
    const int nh = wave_base[kThreads / kWave];
    for (int h = 0; h < nh; ++h) {  // ascending token order
      const int64_t r = base + hits[h];
      const int64_t row = ids[r];
      for (int64_t c = threadIdx.x; c < H; c += kThreads) dw[row * H + c] += dy[r * H + c];
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" int ember_embedding_fwd(const int64_t* ids, const float* w, float* out, int64_t n,
                                   int64_t H, int64_t V, ember_stream_t s) {
  if (n < 0 || H <= 0 || V <= 0) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  if (!ids || !w || !out) return EMBER_EINVAL;
  const unsigned g = static_cast<unsigned>(n < 65536 * 4 ? n : 65536 * 4);
  embedding_fwd_kernel<<<g, kThreads, 0, as_stream(s)>>>(ids, w, out, n, H, V);
  return launch_status();
}

extern "C" size_t ember_embedding_bwd_workspace_bytes(int64_t n, int64_t V) {
  (void)n;
  (void)V;
  return 0;
}

extern "C" int ember_embedding_bwd(const int64_t* ids, const float* dy, float* dw, int64_t n,
                                   int64_t H, int64_t V, int accumulate, void* workspace,
                                   size_t workspace_bytes, ember_stream_t s) {
  (void)workspace;
  (void)workspace_bytes;
  if (n < 0 || H <= 0 || V <= 0 || !dw) return EMBER_EINVAL;
  if (n > 0 && (!ids || !dy)) return EMBER_EINVAL;
  if (!accumulate) {
    const int rc = ember_fill(dw, V * H, 0.f, s);
    if (rc) return rc;
  }
  if (n == 0) return EMBER_OK;
  const int64_t nb = (V + kIdsPerBlock - 1) / kIdsPerBlock;
  if (nb > 0x7fffffff) return EMBER_EINVAL;
  embedding_bwd_kernel<<<static_cast<unsigned>(nb), kThreads, 0, as_stream(s)>>>(ids, dy, dw, n, H,
                                                                                 V);
  return launch_status();
}
