// Fused kernels for a decode step (at most 8 token rows per call).
//
// A decode step reads every weight once and does almost nothing else, so its
// cost is HBM streaming plus a fixed latency per launch (about 3 us on
// MI355X for the smallest kernel).  The reference runs each module op as its
// own kernel (include/ctd/nn/transformer_block.h:17-24, attention.h:43-97,
// mlp.h:16-21: 19 launches per layer).  These kernels fold the small ops into
// the weight-streaming ones, leaving per layer: RMSNorm+Q/K/V GEMV, QK-Norm+
// RoPE+cache write, attention, O GEMV+residual, RMSNorm+gate/up GEMV+SwiGLU,
// down GEMV+residual.
//
// GEMV layout: a workgroup's waves form row groups of kRows rows of each
// weight stream, the kKSplit waves of a group each taking a slice of K; every
// lane streams float4s of the rows (1 KB per row per wave load, kUnroll loads
// in flight) and dots them with the token rows of x (a few KB, L1/L2
// resident).  Partial sums meet in LDS in wave order (deterministic).  A fused RMSNorm uses W (x * w * rstd) = rstd * (W (x * w)):
// the lanes accumulate sum(x^2) over their K range in the same pass and the
// row's rstd = 1/sqrt(mean(x^2) + eps) scales the dot product at the end, so
// the norm adds no pass over x and no latency.
#include <algorithm>
#include <cmath>

#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 2;     // weight rows per row group and stream
constexpr int kKSplit = 4;   // waves sharing a row group, each a 1/kKSplit slice of K
constexpr int kGroups = kWaves / kKSplit;  // row groups per workgroup
constexpr int kBlockRows = kRows * kGroups;
constexpr int kUnroll = 2;   // float4 loads per row in flight per lane
constexpr int64_t kMaxGrid = 1 << 30;  // workgroups per launch; more row groups loop
constexpr int kMaxM = 8;     // token rows per call
constexpr int kMaxSeg = 3;   // weight streams of one ember_decode_gemv call

struct Segs {
  const float* W[kMaxSeg];
  float* y[kMaxSeg];
  const float* res[kMaxSeg];
  int64_t N[kMaxSeg];
  int64_t blocks[kMaxSeg + 1];  // prefix sums of workgroups per segment
  int nseg;
};

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * (1.0f / (1.0f + expf(-g))) * u;
}

// Streams S weight row sets (S = 1 plain, 2 gate+up) of kRows rows each over
// this wave's K slice; the wave's row group starts at n0 + (w / kKSplit) *
// kRows.  acc[s][r][m] = sum_k W_s[n, k] xw[m, k], where xw = x * norm_w when
// NORM; ss[m] = sum_k x[m,k]^2 over the same range.
template <int MR, int S, bool NORM>
__device__ __forceinline__ void gemv_stream(const float* __restrict__ x, int M, int64_t K,
                                            const float* __restrict__ norm_w,
                                            const float* const (&W)[S], int64_t n0, int64_t N,
                                            float (&acc)[S][kRows][MR], float (&ss)[MR]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int64_t K4 = K / 4;
  const int64_t slice = (K4 + kKSplit - 1) / kKSplit;
  const int64_t kb = (w % kKSplit) * slice;
  const int64_t ke = kb + slice < K4 ? kb + slice : K4;
  n0 += (w / kKSplit) * kRows;
  const f32x4* rows[S][kRows];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int64_t n = n0 + r < N ? n0 + r : N - 1;  // rows past N re-read the last one
      rows[s][r] = reinterpret_cast<const f32x4*>(W[s] + n * K);
    }
  const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
  const f32x4* w4 = reinterpret_cast<const f32x4*>(norm_w);
  for (int64_t i0 = kb + lane; i0 < ke; i0 += kUnroll * kWave) {
    f32x4 b[kUnroll][S][kRows];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kWave;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int r = 0; r < kRows; ++r)
          b[u][s][r] = i < ke ? rows[s][r][i] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kWave;
      if (i >= ke) break;
      const f32x4 nw = NORM ? w4[i] : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m < M) {
          const f32x4 xv = x4[m * K4 + i];
          if (NORM) ss[m] += dot4(xv, xv);
          const f32x4 xw = NORM ? xv * nw : xv;
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int r = 0; r < kRows; ++r) acc[s][r][m] += dot4(b[u][s][r], xw);
        }
      }
    }
  }
}

// Sums acc / ss over each row group's kKSplit waves (lanes by shuffles, waves
// through LDS in wave order).  Afterwards thread t < kGroups * kRows * MR
// holds, in acc[.][0][0] / ss[0], the totals of item t: group t / (kRows*MR),
// row (t / MR) % kRows, token row t % MR (of every stream s).
template <int MR, int S, bool NORM>
__device__ __forceinline__ void block_reduce(float (&acc)[S][kRows][MR], float (&ss)[MR]) {
  constexpr int NV = S * kRows * MR + (NORM ? MR : 0);
  __shared__ float red[kWaves][NV];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float v = wave_sum(acc[s][r][m]);
        if (lane == 0) red[w][(s * kRows + r) * MR + m] = v;
      }
  if (NORM) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = wave_sum(ss[m]);
      if (lane == 0) red[w][S * kRows * MR + m] = v;
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < kGroups * kRows * MR) {
    const int g = t / (kRows * MR), rm = t % (kRows * MR);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < kKSplit; ++q) sum += red[g * kKSplit + q][s * kRows * MR + rm];
      acc[s][0][0] = sum;
    }
    if (NORM) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < kKSplit; ++q) sum += red[g * kKSplit + q][S * kRows * MR + rm % MR];
      ss[0] = sum;
    }
  }
}

template <int MR, bool NORM>
__global__ __launch_bounds__(kThreads) void decode_gemv_kernel(const float* __restrict__ x,
                                                               int M, int64_t K,
                                                               const float* __restrict__ norm_w,
                                                               float eps, Segs sg) {
  for (int64_t bid = blockIdx.x; bid < sg.blocks[sg.nseg]; bid += gridDim.x) {
    int seg = 0;
    while (seg + 1 < sg.nseg && bid >= sg.blocks[seg + 1]) ++seg;
    const int64_t N = sg.N[seg];
    const int64_t n0 = (bid - sg.blocks[seg]) * kBlockRows;
    const float* const W[1] = {sg.W[seg]};
    float acc[1][kRows][MR] = {};
    float ss[MR] = {};
    gemv_stream<MR, 1, NORM>(x, M, K, norm_w, W, n0, N, acc, ss);
    block_reduce<MR, 1, NORM>(acc, ss);
    const int t = threadIdx.x;
    if (t < kGroups * kRows * MR) {
      const int m = t % MR;
      const int64_t n = n0 + t / MR;  // group-major rows: (t / (kRows*MR)) * kRows + row
      if (m < M && n < N) {
        float v = acc[0][0][0];
        if (NORM) v *= 1.0f / sqrtf(ss[0] / static_cast<float>(K) + eps);
        const float* res = sg.res[seg];
        sg.y[seg][m * N + n] = res ? res[m * N + n] + v : v;
      }
    }
    __syncthreads();  // the next row group reuses the reduction buffer
  }
}

template <int MR, bool NORM>
__global__ __launch_bounds__(kThreads) void decode_gateup_kernel(
    const float* __restrict__ x, int M, int64_t K, const float* __restrict__ norm_w, float eps,
    const float* __restrict__ Wg, const float* __restrict__ Wu, int64_t I,
    float* __restrict__ out) {
  const int64_t nblocks = (I + kBlockRows - 1) / kBlockRows;
  for (int64_t bid = blockIdx.x; bid < nblocks; bid += gridDim.x) {
    const int64_t n0 = bid * kBlockRows;
    const float* const W[2] = {Wg, Wu};
    float acc[2][kRows][MR] = {};
    float ss[MR] = {};
    gemv_stream<MR, 2, NORM>(x, M, K, norm_w, W, n0, I, acc, ss);
    block_reduce<MR, 2, NORM>(acc, ss);
    const int t = threadIdx.x;
    if (t < kGroups * kRows * MR) {
      const int m = t % MR;
      const int64_t n = n0 + t / MR;
      if (m < M && n < I) {
        const float sc = NORM ? 1.0f / sqrtf(ss[0] / static_cast<float>(K) + eps) : 1.0f;
        out[m * I + n] = silu_mul(acc[0][0][0] * sc, acc[1][0][0] * sc);
      }
    }
    __syncthreads();  // the next row group reuses the reduction buffer
  }
}

// ------------------------------------------------ QK-Norm + RoPE + cache write
constexpr int kMaxPairs = 128;  // D <= 256
struct Freqs {
  float f[kMaxPairs];
};

// One wave per (token row, head): heads [0, H) are query heads, [H, H+Hk)
// key heads, [H+Hk, H+2Hk) value heads; a workgroup takes 4 consecutive
// (row, head) items.  Lane i < D/2 owns the rotation pair (i, i + D/2): the
// angle float(pos + t) * freq[i] and its sincos are those of the standalone
// RoPE kernel, so the rotation rounds the same way.
__global__ __launch_bounds__(kThreads) void qkv_post_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    int64_t rows, int64_t T, int H, int Hk, int D, const float* __restrict__ qn_w,
    const float* __restrict__ kn_w, float eps, Freqs fr, int64_t pos, float* __restrict__ q_out,
    float* __restrict__ ck, float* __restrict__ cv, int64_t S) {
  const int heads = H + 2 * Hk;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
  if (item >= rows * heads) return;  // whole waves leave; no barrier follows
  const int64_t m = item / heads;
  const int hh = static_cast<int>(item % heads);
  const int64_t b = m / T, t = m % T;
  const int lane = threadIdx.x & (kWave - 1);
  const int half = D / 2;
  if (hh >= H + Hk) {  // value head: straight copy into the cache
    const int h = hh - H - Hk;
    const float* src = v + (m * Hk + h) * D;
    float* dst = cv + ((b * Hk + h) * S + pos + t) * D;
    for (int i = lane; i < D; i += kWave) dst[i] = src[i];
    return;
  }
  const bool isq = hh < H;
  const int h = isq ? hh : hh - H;
  const float* src = isq ? q + (m * H + h) * D : k + (m * Hk + h) * D;
  const float* nw = isq ? qn_w : kn_w;
  float a[2], c[2], sn[2] = {0.f, 0.f}, cs[2] = {1.f, 1.f};
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + j * kWave;
    a[j] = i < half ? src[i] : 0.f;
    c[j] = i < half ? src[i + half] : 0.f;
    part += a[j] * a[j] + c[j] * c[j];
    if (i < half) sincosf(static_cast<float>(pos + t) * fr.f[i], &sn[j], &cs[j]);
  }
  if (nw) {
    const float rs = 1.0f / sqrtf(wave_sum(part) / static_cast<float>(D) + eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = lane + j * kWave;
      if (i < half) {
        a[j] = a[j] * rs * nw[i];
        c[j] = c[j] * rs * nw[i + half];
      }
    }
  }
  float* dst = isq ? q_out + (m * H + h) * D : ck + ((b * Hk + h) * S + pos + t) * D;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + j * kWave;
    if (i < half) {
      dst[i] = a[j] * cs[j] - c[j] * sn[j];
      dst[i + half] = a[j] * sn[j] + c[j] * cs[j];
    }
  }
}

template <bool NORM>
int launch_gemv(int64_t M, const float* x, int64_t K, const float* nw, float eps, const Segs& sg,
                hipStream_t st) {
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(sg.blocks[sg.nseg], kMaxGrid));
  const int m = static_cast<int>(M);
  if (M == 1) decode_gemv_kernel<1, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, sg);
  else if (M == 2) decode_gemv_kernel<2, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, sg);
  else if (M <= 4) decode_gemv_kernel<4, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, sg);
  else decode_gemv_kernel<8, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, sg);
  return launch_status();
}

template <bool NORM>
int launch_gateup(int64_t M, const float* x, int64_t K, const float* nw, float eps,
                  const float* Wg, const float* Wu, int64_t I, float* out, hipStream_t st) {
  const unsigned grid =
      static_cast<unsigned>(std::min<int64_t>((I + kBlockRows - 1) / kBlockRows, kMaxGrid));
  const int m = static_cast<int>(M);
  if (M == 1)
    decode_gateup_kernel<1, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, Wg, Wu, I, out);
  else if (M == 2)
    decode_gateup_kernel<2, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, Wg, Wu, I, out);
  else if (M <= 4)
    decode_gateup_kernel<4, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, Wg, Wu, I, out);
  else
    decode_gateup_kernel<8, NORM><<<grid, kThreads, 0, st>>>(x, m, K, nw, eps, Wg, Wu, I, out);
  return launch_status();
}

bool vec_ok(const void* p) { return p == nullptr || aligned16(p); }

}  // namespace

extern "C" int ember_decode_gemv(const float* x, int64_t M, int64_t K, const float* norm_w,
                                 float eps, int nseg, const float* const* W, const int64_t* N,
                                 float* const* y, const float* const* residual,
                                 ember_stream_t s) {
  if (M < 0 || M > kMaxM || K <= 0 || K % 4 != 0 || nseg < 1 || nseg > kMaxSeg || !W || !N || !y)
    return EMBER_EINVAL;
  if (M == 0) return EMBER_OK;
  if (!x || !aligned16(x) || !vec_ok(norm_w)) return EMBER_EINVAL;
  Segs sg{};
  sg.nseg = nseg;
  sg.blocks[0] = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!W[i] || !y[i] || N[i] < 1 || !aligned16(W[i])) return EMBER_EINVAL;
    sg.W[i] = W[i];
    sg.y[i] = y[i];
    sg.res[i] = residual ? residual[i] : nullptr;
    sg.N[i] = N[i];
    sg.blocks[i + 1] = sg.blocks[i] + (N[i] + kBlockRows - 1) / kBlockRows;
  }
  if (sg.blocks[nseg] > 0x7fffffff) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  return norm_w ? launch_gemv<true>(M, x, K, norm_w, eps, sg, st)
                : launch_gemv<false>(M, x, K, nullptr, eps, sg, st);
}

extern "C" int ember_decode_gateup(const float* x, int64_t M, int64_t K, const float* norm_w,
                                   float eps, const float* Wg, const float* Wu, int64_t I,
                                   float* out, ember_stream_t s) {
  if (M < 0 || M > kMaxM || K <= 0 || K % 4 != 0 || I < 1) return EMBER_EINVAL;
  if (M == 0) return EMBER_OK;
  if (!x || !Wg || !Wu || !out || !aligned16(x) || !aligned16(Wg) || !aligned16(Wu) ||
      !vec_ok(norm_w))
    return EMBER_EINVAL;
  if ((I + kBlockRows - 1) / kBlockRows > 0x7fffffff) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  return norm_w ? launch_gateup<true>(M, x, K, norm_w, eps, Wg, Wu, I, out, st)
                : launch_gateup<false>(M, x, K, nullptr, eps, Wg, Wu, I, out, st);
}

extern "C" int ember_decode_qkv_post(const float* q, const float* k, const float* v, int64_t B,
                                     int64_t T, int64_t H, int64_t Hk, int64_t D,
                                     const float* q_norm_w, const float* k_norm_w, float eps,
                                     const float* freqs_host, int64_t pos, float* q_out,
                                     float* cache_k, float* cache_v, int64_t S,
                                     ember_stream_t s) {
  if (B < 0 || T < 0 || H < 1 || Hk < 1 || D < 2 || D % 2 != 0 || D > 2 * kMaxPairs || pos < 0 ||
      pos + T > S || !freqs_host)
    return EMBER_EINVAL;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !q_out || !cache_k || !cache_v || B * T * (H + 2 * Hk) > 0x1fffffff)
    return EMBER_EINVAL;
  Freqs fr{};
  for (int64_t i = 0; i < D / 2; ++i) fr.f[i] = freqs_host[i];
  const int64_t items = B * T * (H + 2 * Hk);
  qkv_post_kernel<<<static_cast<unsigned>((items + kWaves - 1) / kWaves), kThreads, 0,
                    as_stream(s)>>>(q, k, v, B * T, T, static_cast<int>(H), static_cast<int>(Hk),
                                    static_cast<int>(D), q_norm_w, k_norm_w, eps, fr, pos, q_out,
                                    cache_k, cache_v, S);
  return launch_status();
}
