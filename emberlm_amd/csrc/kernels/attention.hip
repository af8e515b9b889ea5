// Fused causal GQA attention, forward and backward, on fp32 MFMA (32x32x2).
//
// Replaces the reference's materialised chain (include/ctd/nn/attention.h:100-143):
// repeat_kv_heads + permute (x3), bmm(Q,K^T), mul_scalar(1/sqrt(D)),
// apply_causal_mask, softmax, bmm(P,V), permute, plus all of their backward
// nodes (src/ops/matmul.cpp:137-152, softmax.cu:54-80, mask.cu:41-52,
// repeat_kv.cu:29-43).  Nothing of size [B*H,T,T] is ever written; the
// forward saves O and the log-sum-exp per query row.
//
// Layout: q, o, dq [B,T,H,D]; k, v, dk, dv [B,T,Hk,D]; lse, delta [B,H,T].
//
// MFMA fragment conventions (v_mfma_f32_32x32x2_f32, wave64): A operand lane
// (g = lane/32, r = lane%32) holds A[m=r][k=g]; B operand holds B[k=g][n=r];
// accumulator register e holds C[m = 8*(e/4) + 4*g + (e%4)][n = r].
//
// Forward, per wave of 32 queries: S^T = K Q^T puts the query index in the
// lane (n = r), so the online-softmax statistics of a query live in one lane
// pair (g = 0/1) and the probabilities come out exactly in the B-operand
// layout of O^T += V^T P^T: accumulator register e of S^T is the B value of
// the MFMA step that contracts over keys {8*(e/4)+(e%4), 8*(e/4)+4+(e%4)}.
// Q stays in registers (pre-multiplied by scale*log2(e)), K and V tiles of 64
// keys are staged through LDS and shared by the block's 4 waves.
//
// Backward (no atomics, so dK/dV/dQ are bitwise reproducible):
//   attn_delta:  delta = rowsum(dO * O);
//   attn_bwd_dq: per 32 queries, S^T = K Q^T and dP^T = V dO^T, then
//                dQ^T += K^T dS^T (same orientation as the forward);
//   attn_bwd_dkdv: per 32 keys, S = Q K^T and dP = dO V^T put the key in the
//                lane, so dV^T += dO^T P and dK^T += Q^T dS accumulate in
//                registers across every query tile and every query head of
//                the KV head's group, in a fixed order.
#include "common.h"

using namespace ember;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int e, int g) { return 8 * (e >> 2) + 4 * g + (e & 3); }

__device__ __forceinline__ void zero16(f32x16& a) {
#pragma unroll
  for (int e = 0; e < 16; ++e) a[e] = 0.f;
}

// Copy `rows` rows of D floats (row stride `gstride` floats) into LDS rows of
// stride `ls`, zero rows at or beyond `valid`.
template <int D>
__device__ __forceinline__ void stage_rows(float* __restrict__ lds, int ls,
                                           const float* __restrict__ src, int64_t gstride,
                                           int rows, int valid) {
  for (int c = threadIdx.x; c < rows * (D / 4); c += blockDim.x) {
    const int row = c / (D / 4), c4 = c % (D / 4);
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (row < valid) v = reinterpret_cast<const f32x4*>(src + row * gstride)[c4];
    *reinterpret_cast<f32x4*>(lds + row * ls + 4 * c4) = v;
  }
}

// Write LDS rows [rows][D] (stride ls) to global rows, skipping rows >= valid.
template <int D>
__device__ __forceinline__ void unstage_rows(const float* __restrict__ lds, int ls,
                                             float* __restrict__ dst, int64_t gstride, int rows,
                                             int valid) {
  for (int c = threadIdx.x; c < rows * (D / 4); c += blockDim.x) {
    const int row = c / (D / 4), c4 = c % (D / 4);
    if (row < valid)
      reinterpret_cast<f32x4*>(dst + row * gstride)[c4] =
          *reinterpret_cast<const f32x4*>(lds + row * ls + 4 * c4);
  }
}

// Load the D/2 values of row `row` starting at column `col0` into registers,
// times `mul`; zeros when row >= T.
template <int HALF>
__device__ __forceinline__ void load_half(float (&reg)[HALF], const float* __restrict__ base,
                                          int64_t stride, int row, int T, int col0, float mul) {
  if (row < T) {
    const f32x4* src = reinterpret_cast<const f32x4*>(base + row * stride + col0);
#pragma unroll
    for (int c = 0; c < HALF / 4; ++c) {
      const f32x4 t = src[c];
#pragma unroll
      for (int j = 0; j < 4; ++j) reg[4 * c + j] = t[j] * mul;
    }
  } else {
#pragma unroll
    for (int c = 0; c < HALF; ++c) reg[c] = 0.f;
  }
}

// ------------------------------------------------------------------ forward
template <int D>
struct FwdCfg {
  static constexpr int kBQ = 128, kBK = 64, kKS = D + 4, kVS = D + 8, kOS = D + 4;
  static constexpr int kTile = kBK * (kKS + kVS);
  static constexpr int kOut = kBQ * kOS;
  static constexpr int kSmem = kTile > kOut ? kTile : kOut;
};

template <int D>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const float* __restrict__ q,
                                                       const float* __restrict__ k,
                                                       const float* __restrict__ v,
                                                       float* __restrict__ o,
                                                       float* __restrict__ lse, int T, int H,
                                                       int Hk, float scale_log2) {
  using C = FwdCfg<D>;
  constexpr int HALF = D / 2, NDT = D / 32;
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];
  float* Ks = smem;
  float* Vs = smem + C::kBK * C::kKS;

  const int nqb = (T + C::kBQ - 1) / C::kBQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);  // longest rows first
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hk);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, r = lane & 31;
  const int q0 = qb * C::kBQ, qw0 = q0 + 32 * w, myq = qw0 + r;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const float* qbase = q + static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
  const float* kbase = k + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const float* vbase = v + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;

  float qreg[HALF];
  load_half<HALF>(qreg, qbase, qs, myq, T, HALF * g, scale_log2);

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) zero16(acc[dt]);
  float m_run = -INFINITY, l_run = 0.f;

  const int kend = min(T, q0 + C::kBQ);
  const int nkb = (kend + C::kBK - 1) / C::kBK;
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * C::kBK;
    stage_rows<D>(Ks, C::kKS, kbase + static_cast<int64_t>(k0) * ks, ks, C::kBK, T - k0);
    stage_rows<D>(Vs, C::kVS, vbase + static_cast<int64_t>(k0) * ks, ks, C::kBK, T - k0);
    __syncthreads();
    if (k0 <= qw0 + 31) {
      f32x16 s[2];
      zero16(s[0]);
      zero16(s[1]);
#pragma unroll
      for (int s4 = 0; s4 < HALF / 4; ++s4) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const f32x4 kf =
              *reinterpret_cast<const f32x4*>(Ks + (mt * 32 + r) * C::kKS + HALF * g + 4 * s4);
#pragma unroll
          for (int j = 0; j < 4; ++j) s[mt] = mfma32(kf[j], qreg[4 * s4 + j], s[mt]);
        }
      }
      const bool need_mask = (k0 + C::kBK - 1 > qw0) || (k0 + C::kBK > T);
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + mt * 32 + acc_row(e, g);
          if (need_mask && (key > myq || key >= T)) s[mt][e] = -INFINITY;
          tmax = fmaxf(tmax, s[mt][e]);
        }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = exp2f(m_run - m_new);
      float psum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = exp2f(s[mt][e] - m_new);
          s[mt][e] = p;
          psum += p;
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[dt][e] *= alpha;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float* vrow = Vs + (mt * 32 + acc_row(e, g)) * C::kVS + r;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma32(vrow[dt * 32], s[mt][e], acc[dt]);
        }
    }
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = 1.0f / l_tot;
  if (g == 0 && myq < T)
    lse[(static_cast<int64_t>(b) * H + h) * T + myq] = (m_run + log2f(l_tot)) * kLn2;
  float* Os = smem;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      Os[(32 * w + r) * C::kOS + dt * 32 + acc_row(e, g)] = acc[dt][e] * inv;
  __syncthreads();
  unstage_rows<D>(Os, C::kOS, o + static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(q0) * qs +
                                  static_cast<int64_t>(h) * D,
                  qs, C::kBQ, T - q0);
}

// --------------------------------------------------------------- backward
// delta[b,h,t] = sum_d dO[b,t,h,d] * O[b,t,h,d]; LPR = D/4 lanes per row.
template <int D>
__global__ __launch_bounds__(256) void attn_delta_kernel(const float* __restrict__ o,
                                                         const float* __restrict__ dout,
                                                         float* __restrict__ delta, int64_t rows,
                                                         int T, int H) {
  constexpr int LPR = D / 4, RPB = 256 / LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  float a = 0.f;
  if (row < rows) {
    const f32x4 x = reinterpret_cast<const f32x4*>(o + row * D)[sub];
    const f32x4 y = reinterpret_cast<const f32x4*>(dout + row * D)[sub];
    a = x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
  }
  for (int off = LPR / 2; off > 0; off >>= 1) a += __shfl_xor(a, off, kWave);
  if (row < rows && sub == 0) {
    const int64_t h = row % H;
    const int64_t bt = row / H;
    const int64_t t = bt % T, b = bt / T;
    delta[(b * H + h) * T + t] = a;
  }
}

template <int D>
struct DqCfg {
  static constexpr int kBQ = 128, kBK = 32, kKS = D + 4, kVS = D + 4, kOS = D + 4;
  static constexpr int kTile = kBK * (kKS + kVS);
  static constexpr int kOut = kBQ * kOS;
  static constexpr int kSmem = kTile > kOut ? kTile : kOut;
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dq, int T, int H, int Hk, float scale_log2, float scale) {
  using C = DqCfg<D>;
  constexpr int HALF = D / 2, NDT = D / 32;
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];
  float* Ks = smem;
  float* Vs = smem + C::kBK * C::kKS;

  const int nqb = (T + C::kBQ - 1) / C::kBQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hk);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, r = lane & 31;
  const int q0 = qb * C::kBQ, qw0 = q0 + 32 * w, myq = qw0 + r;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const int64_t qoff = static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
  const float* kbase = k + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const float* vbase = v + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;

  float qreg[HALF], doreg[HALF];
  load_half<HALF>(qreg, q + qoff, qs, myq, T, HALF * g, scale_log2);
  load_half<HALF>(doreg, dout + qoff, qs, myq, T, HALF * g, 1.0f);
  const int64_t srow = (static_cast<int64_t>(b) * H + h) * T;
  const float lse2 = myq < T ? lse[srow + myq] * kLog2e : 0.f;
  const float dlt = myq < T ? delta[srow + myq] : 0.f;

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) zero16(acc[dt]);

  const int kend = min(T, q0 + C::kBQ);
  const int nkb = (kend + C::kBK - 1) / C::kBK;
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * C::kBK;
    stage_rows<D>(Ks, C::kKS, kbase + static_cast<int64_t>(k0) * ks, ks, C::kBK, T - k0);
    stage_rows<D>(Vs, C::kVS, vbase + static_cast<int64_t>(k0) * ks, ks, C::kBK, T - k0);
    __syncthreads();
    if (k0 <= qw0 + 31) {
      f32x16 s, dp;
      zero16(s);
      zero16(dp);
#pragma unroll
      for (int s4 = 0; s4 < HALF / 4; ++s4) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(Ks + r * C::kKS + HALF * g + 4 * s4);
        const f32x4 vf = *reinterpret_cast<const f32x4*>(Vs + r * C::kVS + HALF * g + 4 * s4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s = mfma32(kf[j], qreg[4 * s4 + j], s);
          dp = mfma32(vf[j], doreg[4 * s4 + j], dp);
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + acc_row(e, g);
        const float p = (key > myq || key >= T) ? 0.f : exp2f(s[e] - lse2);
        s[e] = p * (dp[e] - dlt);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float* krow = Ks + acc_row(e, g) * C::kKS + r;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma32(krow[dt * 32], s[e], acc[dt]);
      }
    }
    __syncthreads();
  }

  float* Os = smem;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      Os[(32 * w + r) * C::kOS + dt * 32 + acc_row(e, g)] = acc[dt][e] * scale;
  __syncthreads();
  unstage_rows<D>(Os, C::kOS, dq + qoff + static_cast<int64_t>(q0) * qs, qs, C::kBQ, T - q0);
}

template <int D>
struct DkvCfg {
  static constexpr int kBKeys = 128, kBQ = 32, kQS = D + 4, kOS = D + 4;
  static constexpr int kTile = 2 * kBQ * kQS + 2 * kBQ;
  static constexpr int kOut = kBKeys * kOS;
  static constexpr int kSmem = kTile > kOut ? kTile : kOut;
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dk, float* __restrict__ dv, int T, int H, int Hk, float scale_log2,
    float scale) {
  using C = DkvCfg<D>;
  constexpr int HALF = D / 2, NDT = D / 32;
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];
  float* Qs = smem;
  float* Ds = smem + C::kBQ * C::kQS;
  float* Ls = smem + 2 * C::kBQ * C::kQS;
  float* Es = Ls + C::kBQ;

  const int kb = blockIdx.x;  // small key blocks see the most queries: launched first
  const int hk = blockIdx.y, b = blockIdx.z;
  const int group = H / Hk;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, r = lane & 31;
  const int key0 = kb * C::kBKeys, kw0 = key0 + 32 * w, mykey = kw0 + r;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const int64_t koff = static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;

  float kreg[HALF], vreg[HALF];
  load_half<HALF>(kreg, k + koff, ks, mykey, T, HALF * g, scale_log2);
  load_half<HALF>(vreg, v + koff, ks, mykey, T, HALF * g, 1.0f);

  f32x16 adk[NDT], adv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    zero16(adk[dt]);
    zero16(adv[dt]);
  }

  for (int hh = 0; hh < group; ++hh) {
    const int h = hk * group + hh;
    const int64_t qoff = static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
    const int64_t srow = (static_cast<int64_t>(b) * H + h) * T;
    for (int qt0 = key0; qt0 < T; qt0 += C::kBQ) {
      stage_rows<D>(Qs, C::kQS, q + qoff + static_cast<int64_t>(qt0) * qs, qs, C::kBQ, T - qt0);
      stage_rows<D>(Ds, C::kQS, dout + qoff + static_cast<int64_t>(qt0) * qs, qs, C::kBQ, T - qt0);
      if (threadIdx.x < C::kBQ) {
        const int t = qt0 + threadIdx.x;
        Ls[threadIdx.x] = t < T ? lse[srow + t] * kLog2e : 0.f;
        Es[threadIdx.x] = t < T ? delta[srow + t] : 0.f;
      }
      __syncthreads();
      if (qt0 + C::kBQ - 1 >= kw0) {
        f32x16 s, dp;
        zero16(s);
        zero16(dp);
#pragma unroll
        for (int s4 = 0; s4 < HALF / 4; ++s4) {
          const f32x4 qf = *reinterpret_cast<const f32x4*>(Qs + r * C::kQS + HALF * g + 4 * s4);
          const f32x4 of = *reinterpret_cast<const f32x4*>(Ds + r * C::kQS + HALF * g + 4 * s4);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            s = mfma32(qf[j], kreg[4 * s4 + j], s);
            dp = mfma32(of[j], vreg[4 * s4 + j], dp);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int ql = acc_row(e, g);
          const int qq = qt0 + ql;
          const float p = (qq < mykey || qq >= T) ? 0.f : exp2f(s[e] - Ls[ql]);
          s[e] = p;
          dp[e] = p * (dp[e] - Es[ql]);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int ql = acc_row(e, g);
          const float* orow = Ds + ql * C::kQS + r;
          const float* qrow = Qs + ql * C::kQS + r;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            adv[dt] = mfma32(orow[dt * 32], s[e], adv[dt]);
            adk[dt] = mfma32(qrow[dt * 32], dp[e], adk[dt]);
          }
        }
      }
      __syncthreads();
    }
  }

  float* Os = smem;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      Os[(32 * w + r) * C::kOS + dt * 32 + acc_row(e, g)] = adk[dt][e] * scale;
  __syncthreads();
  unstage_rows<D>(Os, C::kOS, dk + koff + static_cast<int64_t>(key0) * ks, ks, C::kBKeys, T - key0);
  __syncthreads();
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) Os[(32 * w + r) * C::kOS + dt * 32 + acc_row(e, g)] = adv[dt][e];
  __syncthreads();
  unstage_rows<D>(Os, C::kOS, dv + koff + static_cast<int64_t>(key0) * ks, ks, C::kBKeys, T - key0);
}

int check_shapes(int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D) {
  if (B < 0 || T < 0 || H <= 0 || Hk <= 0 || H % Hk != 0) return EMBER_EINVAL;
  if (D != 64 && D != 128) return EMBER_EINVAL;
  if (T > 0x7fffffff / 2 || H > 65535 || Hk > 65535 || B > 65535) return EMBER_EINVAL;
  return EMBER_OK;
}

}  // namespace

extern "C" int ember_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                              int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                              ember_stream_t s) {
  int rc = check_shapes(B, T, H, Hk, D);
  if (rc) return rc;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !o || !lse) return EMBER_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return EMBER_EALIGN;
  const dim3 grid(static_cast<unsigned>((T + 127) / 128), static_cast<unsigned>(H),
                  static_cast<unsigned>(B));
  const float sl = scale * kLog2e;
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H), Hki = static_cast<int>(Hk);
  if (D == 64)
    attn_fwd_kernel<64><<<grid, 256, 0, as_stream(s)>>>(q, k, v, o, lse, Ti, Hi, Hki, sl);
  else
    attn_fwd_kernel<128><<<grid, 256, 0, as_stream(s)>>>(q, k, v, o, lse, Ti, Hi, Hki, sl);
  return launch_status();
}

extern "C" size_t ember_attn_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return static_cast<size_t>(B * T * H) * sizeof(float);
}

extern "C" int ember_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                              const float* lse, const float* dout, float* dq, float* dk, float* dv,
                              int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                              void* workspace, size_t workspace_bytes, ember_stream_t s) {
  int rc = check_shapes(B, T, H, Hk, D);
  if (rc) return rc;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return EMBER_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dout) ||
      !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return EMBER_EALIGN;
  if (!workspace || workspace_bytes < ember_attn_bwd_workspace_bytes(B, T, H))
    return EMBER_EWORKSPACE;
  float* delta = static_cast<float*>(workspace);
  hipStream_t st = as_stream(s);
  const int64_t rows = B * T * H;
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H), Hki = static_cast<int>(Hk);
  const float sl = scale * kLog2e;
  const dim3 gq(static_cast<unsigned>((T + 127) / 128), static_cast<unsigned>(H),
                static_cast<unsigned>(B));
  const dim3 gk(static_cast<unsigned>((T + 127) / 128), static_cast<unsigned>(Hk),
                static_cast<unsigned>(B));
  if (D == 64) {
    attn_delta_kernel<64><<<static_cast<unsigned>((rows + 15) / 16), 256, 0, st>>>(o, dout, delta,
                                                                                  rows, Ti, Hi);
    if ((rc = launch_status())) return rc;
    attn_bwd_dq_kernel<64><<<gq, 256, 0, st>>>(q, k, v, dout, lse, delta, dq, Ti, Hi, Hki, sl,
                                               scale);
    if ((rc = launch_status())) return rc;
    attn_bwd_dkdv_kernel<64><<<gk, 256, 0, st>>>(q, k, v, dout, lse, delta, dk, dv, Ti, Hi, Hki,
                                                 sl, scale);
  } else {
    attn_delta_kernel<128><<<static_cast<unsigned>((rows + 7) / 8), 256, 0, st>>>(o, dout, delta,
                                                                                 rows, Ti, Hi);
    if ((rc = launch_status())) return rc;
    attn_bwd_dq_kernel<128><<<gq, 256, 0, st>>>(q, k, v, dout, lse, delta, dq, Ti, Hi, Hki, sl,
                                                scale);
    if ((rc = launch_status())) return rc;
    attn_bwd_dkdv_kernel<128><<<gk, 256, 0, st>>>(q, k, v, dout, lse, delta, dk, dv, Ti, Hi, Hki,
                                                  sl, scale);
  }
  return launch_status();
}
