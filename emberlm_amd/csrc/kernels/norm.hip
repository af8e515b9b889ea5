// RMSNorm forward/backward (block norms and per-head QK-Norm).
//
// Reference: rms_norm_kernel_f32 / rms_norm_backward_kernel_f32
// (src/ops/norm.cu:17-106).  The reference gives every row a 256-thread block
// (half idle at H = 128) and sums dw with atomicAdd.  Here a row is owned by a
// group of LPR lanes (LPR = 64 for H >= 256, fewer for the 64/128-wide
// QK-Norm rows, so one wave covers several rows), rows are read as float4,
// and dw is reduced deterministically: each block sums its rows in a fixed
// order into a workspace row, then one pass sums the workspace rows in order.
#include <mutex>

#include "common.h"
#include "rope_math.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBwdBlocks = 1024;
// The float4 path on rows of 1024 floats or more: fewer blocks running more
// rows each (and half the dw partials for the column sum): 0.1545 against
// 0.1725 ms at 32768 x 2048 with the non-temporal loads below.
constexpr int kMaxBwdBlocksWide = 512;

__device__ __forceinline__ float group_sum(float v, int lpr) {
  for (int o = lpr >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Lanes per row for a row of H floats read as float4 (H % 4 == 0).
inline int lanes_per_row(int64_t H) {
  int64_t c = H / 4;
  int lpr = 1;
  while (lpr < 64 && lpr < c) lpr <<= 1;
  return lpr;
}

template <int LPR>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_vec(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ y,
                                                            float* __restrict__ rstd,
                                                            int64_t rows, int64_t H, float eps) {
  constexpr int RPB = kThreads / LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t nc = H / 4;
  const bool live = row < rows;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + (live ? row : 0) * H);
  float ss = 0.f;
  if (live)
    for (int64_t c = sub; c < nc; c += LPR) {
      const f32x4 v = xr[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = fmaf(v[e], v[e], ss);
    }
  ss = group_sum(ss, LPR);
  if (!live) return;
  const float s = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  if (rstd && sub == 0) rstd[row] = s;
  f32x4* yr = reinterpret_cast<f32x4*>(y + row * H);
  const f32x4* wv = reinterpret_cast<const f32x4*>(w);
  for (int64_t c = sub; c < nc; c += LPR) {
    const f32x4 v = xr[c], ww = wv[c];
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[e] * s * ww[e];
    yr[c] = o;
  }
}

// The same with the row held in registers: MAXC float4 chunks per lane, all
// loaded before the sum of squares and written from there, so x is read
// once and its loads are in flight together.  Same arithmetic, same order.
template <int LPR, int MAXC>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_reg(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ y,
                                                            float* __restrict__ rstd,
                                                            int64_t rows, int64_t H, float eps) {
  constexpr int RPB = kThreads / LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t nc = H / 4;
  const bool live = row < rows;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + (live ? row : 0) * H);
  f32x4 v[MAXC];
  float ss = 0.f;
  if (live) {
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
      const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
      // non-temporal: read once (0.084 against 0.103 ms at 32768 x 2048)
      v[j] = ci < nc ? __builtin_nontemporal_load(xr + ci) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
      if (sub + static_cast<int64_t>(j) * LPR < nc)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(v[j][e], v[j][e], ss);
  }
  ss = group_sum(ss, LPR);
  if (!live) return;
  const float s = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  if (rstd && sub == 0) rstd[row] = s;
  f32x4* yr = reinterpret_cast<f32x4*>(y + row * H);
  const f32x4* wv = reinterpret_cast<const f32x4*>(w);
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
    if (ci < nc) {
      const f32x4 ww = wv[ci];
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[j][e] * s * ww[e];
      yr[ci] = o;
    }
  }
}

// Any H: one block per row, scalar accesses.
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_scalar(const float* __restrict__ x,
                                                               const float* __restrict__ w,
                                                               float* __restrict__ y,
                                                               float* __restrict__ rstd,
                                                               int64_t rows, int64_t H, float eps) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * H;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += kThreads) ss = fmaf(xr[i], xr[i], ss);
  ss = block_sum(ss, red);
  const float s = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  if (rstd && threadIdx.x == 0) rstd[row] = s;
  for (int64_t i = threadIdx.x; i < H; i += kThreads) y[row * H + i] = xr[i] * s * w[i];
}

// The backward's per-element arithmetic with its roundings spelled out (the
// products written here are rounded, the rest is fused), so that this file's
// two backward kernels give the same bits whatever the compiler would
// contract in each context:  c += g w x,  dx = s (g w - x k),  dw += g x s.
__device__ __forceinline__ float bwd_c_term(float c, float g, float w, float x) {
#pragma clang fp contract(off)
  return fmaf(x, g * w, c);
}
__device__ __forceinline__ float bwd_dx(float s, float g, float w, float x, float k) {
#pragma clang fp contract(off)
  return s * fmaf(g, w, -(x * k));
}
__device__ __forceinline__ float bwd_dw_term(float acc, float g, float x, float s) {
#pragma clang fp contract(off)
  return fmaf(g * x, s, acc);
}

// Backward, float4 path.  Block b handles rows b*RPB + slot + k*grid*RPB,
// NR of them (k, k+1, ...) per pass of the loop so that a lane has NR rows'
// loads in flight; the dw partials still take the rows in increasing k, the
// same order (and sums) for any NR.  MAXC = float4 chunks per lane (H/4/LPR
// rounded up) kept as dw partials.  ACC: dx += the gradient (dx holds a
// running sum, read with the row; one row per pass keeps its registers).
template <int LPR, int MAXC, bool ACC>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_vec(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, float* __restrict__ dx, float* __restrict__ dw_part,
    int64_t rows, int64_t H, float eps) {
  constexpr int RPB = kThreads / LPR;
  constexpr int NR = ACC ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) float red[];  // [RPB][H]
  const int slot = threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t nc = H / 4;
  const float invH = 1.0f / static_cast<float>(H);
  const f32x4* wv = reinterpret_cast<const f32x4*>(w);
  f32x4 acc[MAXC];
#pragma unroll
  for (int j = 0; j < MAXC; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t step = static_cast<int64_t>(gridDim.x) * RPB;
  for (int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB; row0 < rows; row0 += NR * step) {
    int64_t rr[NR];
    bool live[NR];
    // The rows' x and dy chunks stay in registers for the dx pass below.
    f32x4 xv[NR][MAXC], gv[NR][MAXC], ov[ACC ? MAXC : 1];  // ov: dx's running sum (ACC)
    float ss[NR], c[NR];
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      rr[u] = row0 + u * step + slot;
      live[u] = rr[u] < rows;
      ss[u] = 0.f;
      c[u] = 0.f;
      const f32x4* xr = reinterpret_cast<const f32x4*>(x + (live[u] ? rr[u] : 0) * H);
      const f32x4* gr = reinterpret_cast<const f32x4*>(dy + (live[u] ? rr[u] : 0) * H);
#pragma unroll
      for (int j = 0; j < MAXC; ++j) {
        const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
        // read once: non-temporal loads (x and dy do not displace the dx
        // running sum the accumulating form reads back)
        xv[u][j] = live[u] && ci < nc ? __builtin_nontemporal_load(xr + ci)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
        gv[u][j] = live[u] && ci < nc ? __builtin_nontemporal_load(gr + ci)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if constexpr (ACC) {  // loaded with the row, not behind the sums below
#pragma unroll
      for (int j = 0; j < MAXC; ++j) {
        const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
        ov[j] = live[0] && ci < nc ? reinterpret_cast<const f32x4*>(dx + rr[0] * H)[ci]
                                   : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      if (!live[u]) continue;
#pragma unroll
      for (int j = 0; j < MAXC; ++j) {
        const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
        if (ci < nc) {
          const f32x4 v = xv[u][j], g = gv[u][j], ww = wv[ci];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ss[u] = fmaf(v[e], v[e], ss[u]);
            c[u] = bwd_c_term(c[u], g[e], ww[e], v[e]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {  // every lane takes part in the group sums
      ss[u] = group_sum(ss[u], LPR);
      c[u] = group_sum(c[u], LPR);
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      if (!live[u]) continue;
      const int64_t row = rr[u];
      const float s = rstd ? rstd[row] : 1.0f / sqrtf(ss[u] / static_cast<float>(H) + eps);
      const float k = s * s * c[u] * invH;
#pragma unroll
      for (int j = 0; j < MAXC; ++j) {
        const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
        if (ci < nc) {
          const f32x4 v = xv[u][j], g = gv[u][j], ww = wv[ci];
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[e] = bwd_dx(s, g[e], ww[e], v[e], k);
            acc[j][e] = bwd_dw_term(acc[j][e], g[e], v[e], s);
          }
          if (dx) {
            if constexpr (ACC) {  // dx += this gradient (one add, as ember_accumulate)
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e] = ov[j][e] + o[e];
            }
            reinterpret_cast<f32x4*>(dx + row * H)[ci] = o;
          }
        }
      }
    }
  }
  if (!dw_part) return;
  // Combine the RPB row slots of this block in slot order.
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int64_t ci = sub + static_cast<int64_t>(j) * LPR;
    if (ci < nc) reinterpret_cast<f32x4*>(red + slot * H)[ci] = acc[j];
  }
  __syncthreads();
  for (int64_t col = threadIdx.x; col < H; col += kThreads) {
    float t = 0.f;
    for (int sl = 0; sl < RPB; ++sl) t += red[sl * H + col];
    dw_part[static_cast<int64_t>(blockIdx.x) * H + col] = t;
  }
}

// Any H (slow path): block per row for dx; dw partial per block of rows.
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_scalar(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, float* __restrict__ dx, float* __restrict__ dw_part,
    int64_t rows, int64_t H, float eps, bool acc_dx) {
  __shared__ float red[kThreads / kWave];
  const float invH = 1.0f / static_cast<float>(H);
  for (int64_t col0 = 0; col0 < H; col0 += kThreads) {
    if (dw_part && col0 + threadIdx.x < H) dw_part[blockIdx.x * H + col0 + threadIdx.x] = 0.f;
  }
  __syncthreads();
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * H;
    const float* gr = dy + row * H;
    float ss = 0.f, c = 0.f;
    for (int64_t i = threadIdx.x; i < H; i += kThreads) {
      ss = fmaf(xr[i], xr[i], ss);
      c += gr[i] * w[i] * xr[i];
    }
    ss = block_sum(ss, red);
    c = block_sum(c, red);
    const float s = rstd ? rstd[row] : 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
    for (int64_t i = threadIdx.x; i < H; i += kThreads) {
      if (dx) {
        const float d = s * (gr[i] * w[i] - xr[i] * s * s * c * invH);
        dx[row * H + i] = acc_dx ? dx[row * H + i] + d : d;
      }
      if (dw_part) dw_part[blockIdx.x * H + i] += gr[i] * xr[i] * s;
    }
  }
}

// ------------------------------------------------ QK-Norm + RoPE, fused
// Per-head RMSNorm and then the rotation in one pass over q or k: rows of
// H = 4 * LPR floats, one float4 per lane (LPR = 16 or 32: D = 64 or 128),
// row r = (b * T + t) * heads + h.  The norm is rmsnorm_fwd_reg<LPR, 1>'s
// arithmetic and the rotation rope_kernel's (rope_math.h), so the result is
// bitwise those two kernels run one after the other.  Element i's partner
// i +- D/2 sits in lane sub ^ LPR/2 of the same row and comes over by a lane
// shuffle; pair index i = 4 (sub % (LPR/2)) + e.  A workgroup's rows cover
// few tokens (one when heads is a multiple of its row count), so it computes
// each of their D/2 sines and cosines once, into LDS.
struct RopeRows {
  int64_t T, pos0;
  int heads;
  float sign;  // a run-time value, as in rope_kernel, so both compile alike
  RopeFreqs fr;
};

template <int LPR>
struct RopeTable {
  static constexpr int kRows = kThreads / LPR, kPairs = 2 * LPR;
  float cs[kRows][kPairs], sn[kRows][kPairs];
};

// Sines and cosines of the tokens of rows [row0, row0 + kRows) (clipped to
// rows), token j at tok0 + j; the workgroup's threads share the work.
template <int LPR>
__device__ __forceinline__ void fill_rope_table(RopeTable<LPR>& tb, int64_t row0, int64_t rows,
                                                const RopeRows& rr, int64_t& tok0) {
  constexpr int P = RopeTable<LPR>::kPairs;
  tok0 = row0 / rr.heads;
  const int64_t last = min(row0 + RopeTable<LPR>::kRows, rows) - 1;
  const int ntok = static_cast<int>(last / rr.heads - tok0 + 1);
  for (int idx = threadIdx.x; idx < ntok * P; idx += kThreads) {
    const int j = idx / P, i = idx % P;
    float sn, cs;
    rope_sincos(rr.pos0 + (tok0 + j) % rr.T, rr.fr.f[i], rr.sign, sn, cs);
    tb.cs[j][i] = cs;
    tb.sn[j][i] = sn;
  }
}

template <int LPR>
__device__ __forceinline__ f32x4 rotate_row_chunk(const f32x4& o, int sub, int j,
                                                  const RopeTable<LPR>& tb) {
  constexpr int HALF = LPR / 2;
  f32x4 p, out;
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = __shfl_xor(o[e], HALF, kWave);
  const bool first = sub < HALF;
  const int i0 = 4 * (sub % HALF);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float cs = tb.cs[j][i0 + e], sn = tb.sn[j][i0 + e];
    out[e] = first ? rope_first(o[e], p[e], cs, sn) : rope_second(p[e], o[e], cs, sn);
  }
  return out;
}

// The same rotation with the sines computed in registers: lanes sub and
// sub ^ LPR/2 need the same four, so each computes two and they swap.  (For
// the backward's grid-stride loop, where a shared table costs a barrier per
// step.)
template <int LPR>
__device__ __forceinline__ f32x4 rotate_row_chunk_regs(const f32x4& o, int sub, int64_t row,
                                                       const RopeRows& rr) {
  constexpr int HALF = LPR / 2;
  const bool first = sub < HALF;
  const int i0 = 4 * (sub % HALF);
  const int64_t pos = rr.pos0 + (row / rr.heads) % rr.T;
  float cs[4], sn[4];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int mine = first ? q : 2 + q, theirs = first ? 2 + q : q;
    rope_sincos(pos, rr.fr.f[i0 + mine], rr.sign, sn[mine], cs[mine]);
    cs[theirs] = __shfl_xor(cs[mine], HALF, kWave);
    sn[theirs] = __shfl_xor(sn[mine], HALF, kWave);
  }
  f32x4 p, out;
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = __shfl_xor(o[e], HALF, kWave);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    out[e] = first ? rope_first(o[e], p[e], cs[e], sn[e]) : rope_second(p[e], o[e], cs[e], sn[e]);
  return out;
}

template <int LPR>
__global__ __launch_bounds__(kThreads) void qknorm_rope_fwd(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ y,
                                                            float* __restrict__ rstd,
                                                            int64_t rows, float eps,
                                                            RopeRows rr) {
  constexpr int RPB = kThreads / LPR;
  constexpr int64_t H = 4 * LPR;
  __shared__ RopeTable<LPR> tb;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB;
  const int64_t row = row0 + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const bool live = row < rows;  // the same for every lane of a row's group
  const int64_t r = live ? row : rows - 1;
  // the row's load is in flight while the block computes its sine table
  const f32x4 v = reinterpret_cast<const f32x4*>(x + r * H)[sub];
  int64_t tok0;
  fill_rope_table<LPR>(tb, row0, rows, rr, tok0);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss = fmaf(v[e], v[e], ss);
  ss = group_sum(ss, LPR);
  const float s = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  if (live && rstd && sub == 0) rstd[row] = s;
  const f32x4 ww = reinterpret_cast<const f32x4*>(w)[sub];
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = v[e] * s * ww[e];
  __syncthreads();  // the table is filled
  const f32x4 out = rotate_row_chunk<LPR>(o, sub, static_cast<int>(r / rr.heads - tok0), tb);
  if (live) reinterpret_cast<f32x4*>(y + row * H)[sub] = out;
}

// Backward (rr.sign = -1): dy through the rotation's transpose (rope_kernel
// with sign -1), then rmsnorm_bwd_vec<LPR, 1>'s arithmetic, dw partials per
// block likewise.
template <int LPR>
__global__ __launch_bounds__(kThreads) void qknorm_rope_bwd(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, float* __restrict__ dx, float* __restrict__ dw_part,
    int64_t rows, float eps, RopeRows rr) {
  constexpr int RPB = kThreads / LPR;
  constexpr int64_t H = 4 * LPR;
  extern __shared__ __attribute__((aligned(16))) float red[];  // [RPB][H]
  const int slot = threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  const float invH = 1.0f / static_cast<float>(H);
  const f32x4 ww = reinterpret_cast<const f32x4*>(w)[sub];
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  // NR rows per pass (rows k, k+1, ... of the slot, so the dw partials take
  // them in the same order as one at a time), loaded (non-temporal: read
  // once) before any is reduced.  q of Qwen3-1.7B at B=8, T=4096: 0.148 ms
  // with two rows, 0.195 with four, 0.198 with one.
  constexpr int NR = 2;
  const int64_t step = static_cast<int64_t>(gridDim.x) * RPB;
  for (int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB; row0 < rows; row0 += NR * step) {
    f32x4 v[NR], graw[NR];
    int64_t rr_[NR];
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int64_t row = row0 + u * step + slot;
      rr_[u] = row < rows ? row : rows - 1;
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + rr_[u] * H) + sub);
      graw[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dy + rr_[u] * H) + sub);
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int64_t row = row0 + u * step + slot;
      const bool live = row < rows;
      const f32x4 g = rotate_row_chunk_regs<LPR>(graw[u], sub, rr_[u], rr);
      float ss = 0.f, c = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ss = fmaf(v[u][e], v[u][e], ss);
        c = bwd_c_term(c, g[e], ww[e], v[u][e]);
      }
      ss = group_sum(ss, LPR);
      c = group_sum(c, LPR);
      if (!live) continue;
      const float s = rstd ? rstd[row] : 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
      const float k = s * s * c * invH;
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = bwd_dx(s, g[e], ww[e], v[u][e], k);
        acc[e] = bwd_dw_term(acc[e], g[e], v[u][e], s);
      }
      if (dx) reinterpret_cast<f32x4*>(dx + row * H)[sub] = o;
    }
  }
  if (!dw_part) return;
  reinterpret_cast<f32x4*>(red + slot * H)[sub] = acc;
  __syncthreads();
  for (int64_t col = threadIdx.x; col < H; col += kThreads) {
    float t = 0.f;
    for (int sl = 0; sl < RPB; ++sl) t += red[sl * H + col];
    dw_part[static_cast<int64_t>(blockIdx.x) * H + col] = t;
  }
}

// dw = column sums of the [nrows, H] partials.  A workgroup owns 64 columns;
// its 16 waves take the rows r = j (mod 16), each lane one column (256 B
// coalesced per wave load, kColUnroll loads in flight), and the 16 partial
// sums meet in LDS in slice order: a fixed order, so dw is reproducible.
constexpr int kColThreads = 1024;
constexpr int kColSlices = kColThreads / kWave;
constexpr int kColUnroll = 8;

__global__ __launch_bounds__(kColThreads) void column_sum(const float* __restrict__ part,
                                                          float* __restrict__ out,
                                                          int64_t nrows, int64_t H) {
  __shared__ float s_part[kColSlices][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int j = threadIdx.x / kWave;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kWave + lane;
  float t = 0.f;
  if (col < H) {
    for (int64_t r0 = j; r0 < nrows; r0 += kColSlices * kColUnroll) {
      float v[kColUnroll];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) {
        const int64_t r = r0 + static_cast<int64_t>(u) * kColSlices;
        v[u] = r < nrows ? part[r * H + col] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) t += v[u];
    }
  }
  s_part[j][lane] = t;
  __syncthreads();
  if (j == 0 && col < H) {
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < kColSlices; ++q) sum += s_part[q][lane];
    out[col] = sum;
  }
}

bool vec_ok(int64_t H, const void* a, const void* b) {
  return H % 4 == 0 && aligned16(a) && aligned16(b);
}

int64_t bwd_blocks(int64_t rows, int64_t H, bool vec) {
  const int64_t rpb = vec ? kThreads / lanes_per_row(H) : 1;
  int64_t nb = (rows + rpb - 1) / rpb;
  const int64_t cap = vec && H >= 1024 ? kMaxBwdBlocksWide : kMaxBwdBlocks;
  if (nb > cap) nb = cap;
  if (nb < 1) nb = 1;
  return nb;
}

template <int LPR>
int launch_bwd_lpr(int64_t nb, const float* dy, const float* x, const float* w, const float* rstd,
                   float* dx, float* part, int64_t rows, int64_t H, float eps, bool acc_dx,
                   hipStream_t st) {
  const int64_t chunks = (H / 4 + LPR - 1) / LPR;
  const size_t lds = static_cast<size_t>(kThreads / LPR) * H * sizeof(float);
  if (lds > 64 * 1024) return EMBER_EINVAL;
#define EMBER_BWD_CASE(MC)                                                                     \
  if (chunks <= MC) {                                                                          \
    auto kern = acc_dx ? rmsnorm_bwd_vec<LPR, MC, true> : rmsnorm_bwd_vec<LPR, MC, false>;     \
    kern<<<static_cast<unsigned>(nb), kThreads, part ? lds : 0, st>>>(dy, x, w, rstd, dx, part, \
                                                                     rows, H, eps);            \
    return launch_status();                                                                    \
  }
  EMBER_BWD_CASE(1)
  EMBER_BWD_CASE(2)
  EMBER_BWD_CASE(4)
  EMBER_BWD_CASE(8)
  EMBER_BWD_CASE(16)
#undef EMBER_BWD_CASE
  return EMBER_EINVAL;
}

}  // namespace

extern "C" int ember_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd,
                                 int64_t rows, int64_t H, float eps, ember_stream_t s) {
  if (rows < 0 || H <= 0 || (rows > 0 && (!x || !w || !y))) return EMBER_EINVAL;
  if (rows == 0) return EMBER_OK;
  hipStream_t st = as_stream(s);
  if (vec_ok(H, x, y) && aligned16(w)) {
    const int lpr = lanes_per_row(H);
    const unsigned nb = static_cast<unsigned>((rows + kThreads / lpr - 1) / (kThreads / lpr));
    const int64_t chunks = (H / 4 + lpr - 1) / lpr;  // > 1 only at lpr = 64
#define EMBER_FWD_REG(L, MC)                                                               \
  rmsnorm_fwd_reg<L, MC><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps);            \
  return launch_status();
    if (chunks == 1) {
      switch (lpr) {
        case 1: EMBER_FWD_REG(1, 1)
        case 2: EMBER_FWD_REG(2, 1)
        case 4: EMBER_FWD_REG(4, 1)
        case 8: EMBER_FWD_REG(8, 1)
        case 16: EMBER_FWD_REG(16, 1)
        case 32: EMBER_FWD_REG(32, 1)
        default: EMBER_FWD_REG(64, 1)
      }
    }
    if (chunks <= 2) { EMBER_FWD_REG(64, 2) }
    if (chunks <= 4) { EMBER_FWD_REG(64, 4) }
    if (chunks <= 8) { EMBER_FWD_REG(64, 8) }
    if (chunks <= 16) { EMBER_FWD_REG(64, 16) }
#undef EMBER_FWD_REG
    switch (lpr) {  // wider rows: the chunk loop
      case 1: rmsnorm_fwd_vec<1><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      case 2: rmsnorm_fwd_vec<2><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      case 4: rmsnorm_fwd_vec<4><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      case 8: rmsnorm_fwd_vec<8><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      case 16: rmsnorm_fwd_vec<16><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      case 32: rmsnorm_fwd_vec<32><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
      default: rmsnorm_fwd_vec<64><<<nb, kThreads, 0, st>>>(x, w, y, rstd, rows, H, eps); break;
    }
  } else {
    if (rows > 0x7fffffff) return EMBER_EINVAL;
    rmsnorm_fwd_scalar<<<static_cast<unsigned>(rows), kThreads, 0, st>>>(x, w, y, rstd, rows, H,
                                                                         eps);
  }
  return launch_status();
}

// Scratch of ember_rmsnorm_bwd_noalloc: the dw partials in a file-scope device
// array instead of a caller workspace.  Every GPU the library runs on holds
// its own copy at its own address until the process ends.  Host code must not
// pass the array's name to a kernel (on the host it is a stand-in, not a
// device address): each device's address is looked up once with
// hipGetSymbolAddress and cached below.
static __device__ __align__(256) float scratch[EMBER_RMSNORM_BWD_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// Address of `scratch` on the current device, looked up on first use there.
int scratch_on_current_device(hipStream_t st, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return status_of(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return EMBER_EINVAL;
  if (st) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return status_of(e);
    if (sdev != dev) return EMBER_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return status_of(e);
    if (!p) return EMBER_EINVAL;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return EMBER_OK;
}

}  // namespace

extern "C" size_t ember_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t H) {
  if (rows <= 0 || H <= 0) return 0;
  const bool vec = H % 4 == 0 && H / 4 <= 16 * 64;
  return static_cast<size_t>(bwd_blocks(rows, H, vec)) * H * sizeof(float);
}

namespace {

int rmsnorm_bwd_run(const float* dy, const float* x, const float* w, const float* rstd, float* dx,
                    float* dw, int64_t rows, int64_t H, float eps, bool acc_dx, void* workspace,
                    size_t workspace_bytes, ember_stream_t s) {
  if (rows < 0 || H <= 0 || !w) return EMBER_EINVAL;
  if (rows > 0 && (!dy || !x)) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (rows == 0) {
    if (dw) return ember_fill(dw, H, 0.f, s);
    return EMBER_OK;
  }
  const bool vec = H % 4 == 0 && H / 4 <= 16 * 64 && aligned16(dy) && aligned16(x) &&
                   aligned16(w) && (!dx || aligned16(dx));
  float* part = nullptr;
  const int64_t nb = bwd_blocks(rows, H, H % 4 == 0 && H / 4 <= 16 * 64);
  if (dw) {
    const size_t need = static_cast<size_t>(nb) * H * sizeof(float);
    if (!workspace || workspace_bytes < need) return EMBER_EWORKSPACE;
    part = static_cast<float*>(workspace);
  }
  int rc;
  if (vec) {
    int (*fn)(int64_t, const float*, const float*, const float*, const float*, float*, float*,
              int64_t, int64_t, float, bool, hipStream_t);
    switch (lanes_per_row(H)) {
      case 1: fn = launch_bwd_lpr<1>; break;
      case 2: fn = launch_bwd_lpr<2>; break;
      case 4: fn = launch_bwd_lpr<4>; break;
      case 8: fn = launch_bwd_lpr<8>; break;
      case 16: fn = launch_bwd_lpr<16>; break;
      case 32: fn = launch_bwd_lpr<32>; break;
      default: fn = launch_bwd_lpr<64>; break;
    }
    rc = fn(nb, dy, x, w, rstd, dx, part, rows, H, eps, acc_dx, st);
  } else {
    rmsnorm_bwd_scalar<<<static_cast<unsigned>(nb), kThreads, 0, st>>>(dy, x, w, rstd, dx, part,
                                                                       rows, H, eps, acc_dx);
    rc = launch_status();
  }
  if (rc || !dw) return rc;
  column_sum<<<static_cast<unsigned>((H + kWave - 1) / kWave), kColThreads, 0, st>>>(part, dw, nb,
                                                                                  H);
  return launch_status();
}

}  // namespace

extern "C" int ember_rmsnorm_bwd(const float* dy, const float* x, const float* w,
                                 const float* rstd, float* dx, float* dw, int64_t rows, int64_t H,
                                 float eps, void* workspace, size_t workspace_bytes,
                                 ember_stream_t s) {
  return rmsnorm_bwd_run(dy, x, w, rstd, dx, dw, rows, H, eps, false, workspace, workspace_bytes,
                         s);
}

extern "C" int ember_rmsnorm_bwd_accumulate(const float* dy, const float* x, const float* w,
                                            const float* rstd, float* dx, float* dw,
                                            int64_t rows, int64_t H, float eps, void* workspace,
                                            size_t workspace_bytes, ember_stream_t s) {
  if (!dx) return EMBER_EINVAL;
  return rmsnorm_bwd_run(dy, x, w, rstd, dx, dw, rows, H, eps, true, workspace, workspace_bytes,
                         s);
}

namespace {

// Checks shared by the fused QK-Norm + RoPE entries; fills the rows' RoPE
// arguments.
int qknorm_rope_rows(int64_t rows, int64_t heads, int64_t T, int64_t D, int64_t pos0,
                     const float* freqs_host, float sign, RopeRows* rr) {
  if (rows < 0 || heads <= 0 || T <= 0 || (D != 64 && D != 128) || !freqs_host ||
      heads > 0x7fffffff || rows % (heads * T) != 0)
    return EMBER_EINVAL;
  rr->T = T;
  rr->pos0 = pos0;
  rr->heads = static_cast<int>(heads);
  rr->sign = sign;
  for (int i = 0; i < kRopeMaxPairs; ++i) rr->fr.f[i] = i < D / 2 ? freqs_host[i] : 0.f;
  return EMBER_OK;
}

}  // namespace

extern "C" int ember_qknorm_rope_fwd(const float* x, const float* w, float* y, float* rstd,
                                     int64_t rows, int64_t heads, int64_t T, int64_t D, float eps,
                                     int64_t pos0, const float* freqs_host, ember_stream_t s) {
  RopeRows rr;
  int rc = qknorm_rope_rows(rows, heads, T, D, pos0, freqs_host, 1.0f, &rr);
  if (rc || rows == 0) return rc;
  if (!x || !w || !y) return EMBER_EINVAL;
  if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return EMBER_EALIGN;
  const int lpr = static_cast<int>(D / 4);
  const int64_t nb = (rows + kThreads / lpr - 1) / (kThreads / lpr);
  if (nb > 0x7fffffff) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (D == 64)
    qknorm_rope_fwd<16><<<static_cast<unsigned>(nb), kThreads, 0, st>>>(x, w, y, rstd, rows, eps,
                                                                       rr);
  else
    qknorm_rope_fwd<32><<<static_cast<unsigned>(nb), kThreads, 0, st>>>(x, w, y, rstd, rows, eps,
                                                                       rr);
  return launch_status();
}

extern "C" int ember_qknorm_rope_bwd(const float* dy, const float* x, const float* w,
                                     const float* rstd, float* dx, float* dw, int64_t rows,
                                     int64_t heads, int64_t T, int64_t D, float eps,
                                     int64_t pos0, const float* freqs_host, void* workspace,
                                     size_t workspace_bytes, ember_stream_t s) {
  RopeRows rr;
  int rc = qknorm_rope_rows(rows, heads, T, D, pos0, freqs_host, -1.0f, &rr);
  if (rc) return rc;
  if (!w) return EMBER_EINVAL;
  if (rows == 0) return dw ? ember_fill(dw, D, 0.f, s) : EMBER_OK;
  if (!dy || !x) return EMBER_EINVAL;
  if (!aligned16(dy) || !aligned16(x) || !aligned16(w) || (dx && !aligned16(dx)))
    return EMBER_EALIGN;
  const int64_t nb = bwd_blocks(rows, D, true);
  float* part = nullptr;
  if (dw) {
    if (!workspace || workspace_bytes < static_cast<size_t>(nb) * D * sizeof(float))
      return EMBER_EWORKSPACE;
    part = static_cast<float*>(workspace);
  }
  hipStream_t st = as_stream(s);
  const size_t lds = part ? static_cast<size_t>(kThreads) * 4 * sizeof(float) : 0;  // [RPB][D]
  if (D == 64)
    qknorm_rope_bwd<16><<<static_cast<unsigned>(nb), kThreads, lds, st>>>(dy, x, w, rstd, dx,
                                                                         part, rows, eps, rr);
  else
    qknorm_rope_bwd<32><<<static_cast<unsigned>(nb), kThreads, lds, st>>>(dy, x, w, rstd, dx,
                                                                         part, rows, eps, rr);
  if ((rc = launch_status()) || !dw) return rc;
  column_sum<<<static_cast<unsigned>((D + kWave - 1) / kWave), kColThreads, 0, st>>>(part, dw, nb,
                                                                                  D);
  return launch_status();
}

extern "C" int ember_rmsnorm_bwd_noalloc(const float* dy, const float* x, const float* w,
                                         const float* rstd, float* dx, float* dw, int64_t rows,
                                         int64_t H, float eps, ember_stream_t s) {
  if (rows < 0 || H <= 0 || !w) return EMBER_EINVAL;
  if (rows > 0 && (!dy || !x)) return EMBER_EINVAL;
  const size_t need = ember_rmsnorm_bwd_workspace_bytes(rows, H);
  if (!dw || need == 0)
    return ember_rmsnorm_bwd(dy, x, w, rstd, dx, dw, rows, H, eps, nullptr, 0, s);
  if (need > EMBER_RMSNORM_BWD_SCRATCH_BYTES) return EMBER_ESCRATCH;
  float* ws = nullptr;
  const int rc = scratch_on_current_device(as_stream(s), &ws);
  if (rc) return rc;
  // Every partial row the kernels read is written first by the same call (the
  // float4 kernel stores all H columns of each workgroup's row, the scalar one
  // zeroes its row before adding), so nothing left by an earlier call is read.
  return ember_rmsnorm_bwd(dy, x, w, rstd, dx, dw, rows, H, eps, ws, need, s);
}
