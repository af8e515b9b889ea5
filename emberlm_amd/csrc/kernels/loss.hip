// Masked cross-entropy over [N,V] logits (the LM-head loss).
//
// Reference: ce_masked_fwd/mean/bwd kernels (src/ops/loss.cu:253-329).  The
// reference runs max, exp-sum and probability passes, writes an [N,V]
// probability tensor, reduces the loss with two atomicAdds and a <<<1,1>>>
// divide, and indexes row*V in 32-bit int.  Here the forward is one online
// (max, sum) pass per row that keeps only lse[N]; rows whose mask is 0 are
// skipped (their loss term is 0); the loss is a fixed-order reduction (no
// atomics); the backward recomputes exp(logit - lse) and can write dlogits in
// place over the logits.  All offsets are 64-bit.
#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

// Rows of the compacted LM head: row j of a chunk is row idx[base + j] of the
// batch; the chunk holds n = clamp(*count - base, 0, N) of them.
struct RowMap {
  const int64_t* idx;
  const int64_t* count;
  int64_t base;
  __device__ __forceinline__ int64_t rows(int64_t N) const {
    return idx ? min(max(*count - base, int64_t{0}), N) : N;
  }
  __device__ __forceinline__ int64_t src(int64_t j) const { return idx ? idx[base + j] : j; }
};

// lse[j] and the logits are per row of the chunk; mask, tgt and row_loss are
// indexed by the batch row map.src(j).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void ce_fwd_rows(const float* __restrict__ logits,
                                                        const int64_t* __restrict__ tgt,
                                                        const float* __restrict__ mask,
                                                        int64_t N, int64_t V,
                                                        float* __restrict__ lse,
                                                        float* __restrict__ row_loss,
                                                        RowMap map) {
  __shared__ float red[kThreads / kWave];
  const int64_t n = map.rows(N);
  for (int64_t row = blockIdx.x; row < n; row += gridDim.x) {
    const int64_t b = map.src(row);
    const float mk = mask[b];
    if (mk == 0.0f) {  // uniform per block
      if (threadIdx.x == 0) {
        lse[row] = 0.f;
        row_loss[b] = 0.f;
      }
      continue;
    }
    const float* lr = logits + row * V;
    float m = -INFINITY, s = 0.f;
    if (VEC) {
      const f32x4* l4 = reinterpret_cast<const f32x4*>(lr);
      for (int64_t c = threadIdx.x; c < V / 4; c += kThreads) {
        const f32x4 v = l4[c];
        const float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (mx > m) {
          s *= exp2f((m - mx) * kLog2e);
          m = mx;
        }
        s += exp2f((v[0] - m) * kLog2e) + exp2f((v[1] - m) * kLog2e) +
             exp2f((v[2] - m) * kLog2e) + exp2f((v[3] - m) * kLog2e);
      }
    } else {
      for (int64_t i = threadIdx.x; i < V; i += kThreads) {
        const float v = lr[i];
        if (v > m) {
          s *= exp2f((m - v) * kLog2e);
          m = v;
        }
        s += exp2f((v - m) * kLog2e);
      }
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.f : s * exp2f((m - M) * kLog2e);
    const float S = block_sum(part, red);
    if (threadIdx.x == 0) {
      const float l = M + logf(S);
      lse[row] = l;
      const int64_t t = tgt[b];
      row_loss[b] = (t >= 0 && t < V) ? mk * (l - lr[t]) : 0.f;
    }
    __syncthreads();
  }
}

// One block: loss = sum(row_loss) / sum(mask) in a fixed order (double accumulators).
__global__ __launch_bounds__(1024) void ce_reduce(const float* __restrict__ row_loss,
                                                  const float* __restrict__ mask, int64_t N,
                                                  float* __restrict__ loss,
                                                  float* __restrict__ mask_sum) {
  __shared__ double sl[1024];
  __shared__ double sm[1024];
  double a = 0.0, b = 0.0;
  for (int64_t i = threadIdx.x; i < N; i += 1024) {
    if (row_loss) a += row_loss[i];
    b += mask[i];
  }
  sl[threadIdx.x] = a;
  sm[threadIdx.x] = b;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      sl[threadIdx.x] += sl[threadIdx.x + o];
      sm[threadIdx.x] += sm[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double ms = sm[0];
    loss[0] = ms > 0.0 ? static_cast<float>(sl[0] / ms) : 0.0f;
    mask_sum[0] = static_cast<float>(ms);
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void ce_bwd_rows(const float* logits,
                                                        const int64_t* __restrict__ tgt,
                                                        const float* __restrict__ mask,
                                                        const float* __restrict__ lse,
                                                        const float* __restrict__ dloss,
                                                        const float* __restrict__ mask_sum,
                                                        int64_t N, int64_t V, float* dlogits,
                                                        RowMap map) {
  const float alpha = dloss[0] / mask_sum[0];
  const int64_t n = map.rows(N);
  for (int64_t row = blockIdx.x; row < n; row += gridDim.x) {
    const int64_t b = map.src(row);
    const float sc = alpha * mask[b];
    float* dr = dlogits + row * V;
    const float* lr = logits + row * V;
    const int64_t t = tgt[b];
    if (mask[b] == 0.0f) {
      if (VEC) {
        for (int64_t c = threadIdx.x; c < V / 4; c += kThreads)
          reinterpret_cast<f32x4*>(dr)[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        for (int64_t i = threadIdx.x; i < V; i += kThreads) dr[i] = 0.f;
      }
      continue;
    }
    const float l2 = lse[row] * kLog2e;
    if (VEC) {
      for (int64_t c = threadIdx.x; c < V / 4; c += kThreads) {
        const f32x4 v = reinterpret_cast<const f32x4*>(lr)[c];
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float p = exp2f(v[e] * kLog2e - l2);
          if (4 * c + e == t) p -= 1.0f;
          o[e] = sc * p;
        }
        reinterpret_cast<f32x4*>(dr)[c] = o;
      }
    } else {
      for (int64_t i = threadIdx.x; i < V; i += kThreads) {
        float p = exp2f(lr[i] * kLog2e - l2);
        if (i == t) p -= 1.0f;
        dr[i] = sc * p;
      }
    }
  }
}

unsigned row_grid(int64_t N) { return static_cast<unsigned>(N < 65536 * 4 ? N : 65536 * 4); }

// idx[0 .. count) = the rows with mask != 0 (NaN included), ascending.  One
// workgroup: thread t owns rows [t*per, (t+1)*per), counts its hits, and a
// block-wide exclusive scan of the counts gives where its indices go.
constexpr int kScan = 1024;
__global__ __launch_bounds__(kScan) void mask_rows_kernel(const float* __restrict__ mask,
                                                           int64_t N, int64_t* __restrict__ idx,
                                                           int64_t* __restrict__ count) {
  __shared__ int64_t part[kScan];
  const int t = threadIdx.x;
  const int64_t per = (N + kScan - 1) / kScan;
  const int64_t b = min(N, t * per), e = min(N, b + per);
  int64_t c = 0;
  for (int64_t i = b; i < e; ++i) c += mask[i] != 0.0f;
  part[t] = c;
  __syncthreads();
  for (int o = 1; o < kScan; o <<= 1) {  // inclusive Hillis-Steele scan
    const int64_t v = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int64_t pos = part[t] - c;
  for (int64_t i = b; i < e; ++i)
    if (mask[i] != 0.0f) idx[pos++] = i;
  if (t == kScan - 1) *count = part[kScan - 1];
}

// dst row j (of R, H floats, contiguous) = src row idx[base + j] for j < n;
// zeros for j in [n, round_up(n, 256)) so that the GEMM row tile holding row
// n - 1 reads zeros past it; rows after that are left alone.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void rows_gather_kernel(const float* __restrict__ src,
                                                               int64_t ld, int64_t H,
                                                               RowMap map, int64_t R,
                                                               float* __restrict__ dst) {
  const int64_t n = map.rows(R);
  const int64_t fill = min(R, (n + 255) / 256 * 256);
  for (int64_t j = blockIdx.x; j < fill; j += gridDim.x) {
    float* d = dst + j * H;
    if (j < n) {
      const float* sr = src + map.src(j) * ld;
      if (VEC) {
        for (int64_t c = threadIdx.x; c < H / 4; c += kThreads)
          reinterpret_cast<f32x4*>(d)[c] = reinterpret_cast<const f32x4*>(sr)[c];
      } else {
        for (int64_t c = threadIdx.x; c < H; c += kThreads) d[c] = sr[c];
      }
    } else {
      if (VEC) {
        for (int64_t c = threadIdx.x; c < H / 4; c += kThreads)
          reinterpret_cast<f32x4*>(d)[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        for (int64_t c = threadIdx.x; c < H; c += kThreads) d[c] = 0.f;
      }
    }
  }
}

// dst row idx[base + j] = src row j (contiguous, H floats) for j < n.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void rows_scatter_kernel(const float* __restrict__ src,
                                                                int64_t H, RowMap map, int64_t R,
                                                                float* __restrict__ dst,
                                                                int64_t ld) {
  const int64_t n = map.rows(R);
  for (int64_t j = blockIdx.x; j < n; j += gridDim.x) {
    const float* sr = src + j * H;
    float* d = dst + map.src(j) * ld;
    if (VEC) {
      for (int64_t c = threadIdx.x; c < H / 4; c += kThreads)
        reinterpret_cast<f32x4*>(d)[c] = reinterpret_cast<const f32x4*>(sr)[c];
    } else {
      for (int64_t c = threadIdx.x; c < H; c += kThreads) d[c] = sr[c];
    }
  }
}

}  // namespace

extern "C" size_t ember_ce_masked_fwd_workspace_bytes(int64_t N) {
  return N > 0 ? static_cast<size_t>(N) * sizeof(float) : 0;
}

extern "C" int ember_ce_masked_fwd(const float* logits, const int64_t* tgt, const float* mask,
                                   int64_t N, int64_t V, float* lse, float* loss, float* mask_sum,
                                   void* workspace, size_t workspace_bytes, ember_stream_t s) {
  if (N < 0 || V <= 0 || !loss || !mask_sum) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (N > 0) {
    if (!logits || !tgt || !mask || !lse) return EMBER_EINVAL;
    if (!workspace || workspace_bytes < static_cast<size_t>(N) * sizeof(float))
      return EMBER_EWORKSPACE;
    float* row_loss = static_cast<float*>(workspace);
    const bool vec = V % 4 == 0 && aligned16(logits);
    if (vec)
      ce_fwd_rows<true><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, N, V, lse, row_loss,
                                                        RowMap{});
    else
      ce_fwd_rows<false><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, N, V, lse, row_loss,
                                                        RowMap{});
    int rc = launch_status();
    if (rc) return rc;
    ce_reduce<<<1, 1024, 0, st>>>(row_loss, mask, N, loss, mask_sum);
  } else {
    ce_reduce<<<1, 1024, 0, st>>>(nullptr, nullptr, 0, loss, mask_sum);
  }
  return launch_status();
}

extern "C" int ember_ce_masked_bwd(const float* logits, const int64_t* tgt, const float* mask,
                                   const float* lse, const float* dloss, const float* mask_sum,
                                   int64_t N, int64_t V, float* dlogits, ember_stream_t s) {
  if (N < 0 || V <= 0) return EMBER_EINVAL;
  if (N == 0) return EMBER_OK;
  if (!logits || !tgt || !mask || !lse || !dloss || !mask_sum || !dlogits) return EMBER_EINVAL;
  const bool vec = V % 4 == 0 && aligned16(logits) && aligned16(dlogits);
  hipStream_t st = as_stream(s);
  if (vec)
    ce_bwd_rows<true><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, lse, dloss, mask_sum, N,
                                                        V, dlogits, RowMap{});
  else
    ce_bwd_rows<false><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, lse, dloss, mask_sum,
                                                         N, V, dlogits, RowMap{});
  return launch_status();
}

extern "C" int ember_ce_masked_rows(const float* logits, const int64_t* tgt, const float* mask,
                                    int64_t N, int64_t V, float* lse, float* row_loss,
                                    ember_stream_t s) {
  if (N < 0 || V <= 0) return EMBER_EINVAL;
  if (N == 0) return EMBER_OK;
  if (!logits || !tgt || !mask || !lse || !row_loss) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (V % 4 == 0 && aligned16(logits))
    ce_fwd_rows<true><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, N, V, lse, row_loss,
                                                        RowMap{});
  else
    ce_fwd_rows<false><<<row_grid(N), kThreads, 0, st>>>(logits, tgt, mask, N, V, lse, row_loss,
                                                        RowMap{});
  return launch_status();
}

extern "C" int ember_ce_masked_reduce(const float* row_loss, const float* mask, int64_t N,
                                      float* loss, float* mask_sum, ember_stream_t s) {
  if (N < 0 || !loss || !mask_sum || (N > 0 && !mask)) return EMBER_EINVAL;
  ce_reduce<<<1, 1024, 0, as_stream(s)>>>(row_loss, mask, N, loss, mask_sum);
  return launch_status();
}

extern "C" int ember_mask_rows(const float* mask, int64_t N, int64_t* idx, int64_t* count,
                               ember_stream_t s) {
  if (N < 0 || !count || (N > 0 && (!mask || !idx))) return EMBER_EINVAL;
  mask_rows_kernel<<<1, kScan, 0, as_stream(s)>>>(mask, N, idx, count);
  return launch_status();
}

extern "C" int ember_rows_gather(const float* src, int64_t ld, int64_t H, const int64_t* idx,
                                 const int64_t* count, int64_t base, int64_t R, float* dst,
                                 ember_stream_t s) {
  if (H < 0 || R < 0 || ld < H || base < 0 || !idx || !count) return EMBER_EINVAL;
  if (R == 0 || H == 0) return EMBER_OK;
  if (!src || !dst) return EMBER_EINVAL;
  const RowMap map{idx, count, base};
  const bool vec = H % 4 == 0 && ld % 4 == 0 && aligned16(src) && aligned16(dst);
  if (vec)
    rows_gather_kernel<true><<<row_grid(R), kThreads, 0, as_stream(s)>>>(src, ld, H, map, R, dst);
  else
    rows_gather_kernel<false><<<row_grid(R), kThreads, 0, as_stream(s)>>>(src, ld, H, map, R, dst);
  return launch_status();
}

extern "C" int ember_rows_scatter(const float* src, int64_t H, const int64_t* idx,
                                  const int64_t* count, int64_t base, int64_t R, float* dst,
                                  int64_t ld, ember_stream_t s) {
  if (H < 0 || R < 0 || ld < H || base < 0 || !idx || !count) return EMBER_EINVAL;
  if (R == 0 || H == 0) return EMBER_OK;
  if (!src || !dst) return EMBER_EINVAL;
  const RowMap map{idx, count, base};
  const bool vec = H % 4 == 0 && ld % 4 == 0 && aligned16(src) && aligned16(dst);
  if (vec)
    rows_scatter_kernel<true><<<row_grid(R), kThreads, 0, as_stream(s)>>>(src, H, map, R, dst, ld);
  else
    rows_scatter_kernel<false><<<row_grid(R), kThreads, 0, as_stream(s)>>>(src, H, map, R, dst, ld);
  return launch_status();
}

extern "C" int ember_ce_masked_rows_idx(const float* logits, const int64_t* tgt,
                                        const float* mask, const int64_t* idx,
                                        const int64_t* count, int64_t base, int64_t R, int64_t V,
                                        float* lse, float* row_loss, ember_stream_t s) {
  if (R < 0 || V <= 0 || base < 0 || !idx || !count) return EMBER_EINVAL;
  if (R == 0) return EMBER_OK;
  if (!logits || !tgt || !mask || !lse || !row_loss) return EMBER_EINVAL;
  const RowMap map{idx, count, base};
  hipStream_t st = as_stream(s);
  if (V % 4 == 0 && aligned16(logits))
    ce_fwd_rows<true><<<row_grid(R), kThreads, 0, st>>>(logits, tgt, mask, R, V, lse, row_loss, map);
  else
    ce_fwd_rows<false><<<row_grid(R), kThreads, 0, st>>>(logits, tgt, mask, R, V, lse, row_loss,
                                                         map);
  return launch_status();
}

extern "C" int ember_ce_masked_bwd_idx(const float* logits, const int64_t* tgt,
                                       const float* mask, const float* lse, const int64_t* idx,
                                       const int64_t* count, int64_t base, int64_t R, int64_t V,
                                       const float* dloss, const float* mask_sum, float* dlogits,
                                       ember_stream_t s) {
  if (R < 0 || V <= 0 || base < 0 || !idx || !count) return EMBER_EINVAL;
  if (R == 0) return EMBER_OK;
  if (!logits || !tgt || !mask || !lse || !dloss || !mask_sum || !dlogits) return EMBER_EINVAL;
  const RowMap map{idx, count, base};
  const bool vec = V % 4 == 0 && aligned16(logits) && aligned16(dlogits);
  hipStream_t st = as_stream(s);
  if (vec)
    ce_bwd_rows<true><<<row_grid(R), kThreads, 0, st>>>(logits, tgt, mask, lse, dloss, mask_sum, R,
                                                        V, dlogits, map);
  else
    ce_bwd_rows<false><<<row_grid(R), kThreads, 0, st>>>(logits, tgt, mask, lse, dloss, mask_sum,
                                                         R, V, dlogits, map);
  return launch_status();
}
