// KV cache and cached (decode) attention for the inference forward.
//
// Reference: write_kv_kernel / read_kv_expanded_kernel (src/ops/kv_cache.cu:13-48)
// and the chain Attention::forward runs over the cache
// (include/ctd/nn/attention.h:43-97): read_kv_expanded -> bmm -> mul_scalar ->
// apply_causal_mask(position_start) -> softmax -> bmm.
//
// The cache keeps the reference's layout [B, Hk, S, D]: one KV head's keys are
// contiguous, which is what a decode step streams.  ember_attn_decode reads it
// in place (no GQA expansion, no [B*H, T, L] scores): a workgroup owns one
// (batch, KV head, key split) and every query row of that KV head's group, so
// each key and value row is read from HBM once per step whatever the group
// size.  Inside the workgroup a row of D floats is spread over D/4 lanes
// (one float4 each), so a wave covers 64*4/D keys per load; each lane group
// runs its own online softmax (exp2 domain, queries pre-scaled by
// scale*log2(e)), the groups and the 4 waves are merged through LDS in a fixed
// order, and the key splits are merged by a second kernel in split order, so
// results are reproducible bit for bit.
#include <cmath>

#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRowTile = 4;        // query rows per pass over the split's keys (a GQA group)
constexpr int kUnroll = 4;         // key loads in flight per lane before use
// Split plan (measured on MI355X, B=1, 8 KV heads, D=128): about 512
// workgroups in all, and at least 32 keys each.  Fewer, longer splits leave
// HBM idle at the start; more, shorter ones spend their time in the per-split
// setup and the merge.
constexpr int kMinKeysPerSplit = 32;
constexpr int kTargetBlocks = 512;

// ---------------------------------------------------------------- KV writes
// src [B,T,Hk,D] -> cache [B,Hk,S,D] rows [pos, pos+T).  One thread per VEC
// floats of src, in src order.
template <int VEC>
__global__ __launch_bounds__(kThreads) void kv_write_kernel(const float* __restrict__ src,
                                                            float* __restrict__ cache, int64_t n,
                                                            int64_t T, int64_t Hk, int64_t D,
                                                            int64_t S, int64_t pos) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    const int64_t e = i * VEC;
    const int64_t d = e % D;
    const int64_t h = (e / D) % Hk;
    const int64_t t = (e / (D * Hk)) % T;
    const int64_t b = e / (D * Hk * T);
    const int64_t dst = ((b * Hk + h) * S + pos + t) * D + d;
    if (VEC == 4)
      *reinterpret_cast<f32x4*>(cache + dst) = *reinterpret_cast<const f32x4*>(src + e);
    else
      cache[dst] = src[e];
  }
}

// cache [B,Hk,S,D] rows [0,L) -> out [B, Hk*group, L, D], head h reading KV head h/group.
template <int VEC>
__global__ __launch_bounds__(kThreads) void kv_read_expanded_kernel(
    const float* __restrict__ cache, float* __restrict__ out, int64_t n, int64_t Hk,
    int64_t group, int64_t L, int64_t D, int64_t S) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t H = Hk * group;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    const int64_t e = i * VEC;
    const int64_t d = e % D;
    const int64_t t = (e / D) % L;
    const int64_t h = (e / (D * L)) % H;
    const int64_t b = e / (D * L * H);
    const int64_t src = ((b * Hk + h / group) * S + t) * D + d;
    if (VEC == 4)
      *reinterpret_cast<f32x4*>(out + e) = *reinterpret_cast<const f32x4*>(cache + src);
    else
      out[e] = cache[src];
  }
}

// ------------------------------------------------------- decode attention
struct DecodeArgs {
  const float* q;    // [B, T, H, D]
  const float* k;    // key row (b, hk, j) at k + b*kv_sb + hk*kv_sh + j*kv_st
  const float* v;
  float* o;          // [B, T, H, D] (written here when nsplit == 1)
  float* part_o;     // [B*T*H, nsplit, D]   unnormalised split outputs
  float* part_ml;    // [B*T*H, nsplit, 2]   split (max, sum) in log2 units
  int64_t T, H, Hk, L, pos;
  int64_t kv_sb, kv_sh, kv_st;
  int64_t kps;       // keys per split
  int nsplit;
  float qscale;      // scale * log2(e)
};

// Sum over the LPK lanes of one key group (aligned blocks of LPK lanes).
template <int LPK>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int o = LPK / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// The QK-Norm + RoPE + cache write of a decode step, folded into the
// attention launch (ember_attn_decode_qkv): q is then the raw query
// projection and the new key/value rows [pos, pos + T) come from kn / vn.
constexpr int kMaxRopePairs = 64;  // D <= 128
constexpr int kFoldRows = 8;       // new rows per call (T): a decode step's
struct QkvFold {
  const float* kn;    // [B, T, Hk, D] key projection
  const float* vn;    // [B, T, Hk, D] value projection
  const float* qn_w;  // [D] QK-Norm weights, or null (no norm)
  const float* kn_w;
  float* ck;          // the caches that DecodeArgs::k / v read
  float* cv;
  float eps;
  float freqs[kMaxRopePairs];
};

// One D-float row spread over the LPK lanes of a key group, a float4 each:
// RMSNorm with weight w (skipped when w is null), then the rotation of each
// pair (i, i + D/2) by the angle whose cosine and sine are cs[i] and sn[i],
// lanes d4 < LPK/2 holding the first halves and lane d4 + LPK/2 the partners.
// With cs, sn the sincosf of float(position) * freq[i], the products are those
// of the standalone QK-Norm and RoPE kernels; only the order of the norm's sum
// of squares differs.
template <int LPK>
__device__ __forceinline__ f32x4 norm_rope(f32x4 x, int d4, const float* w, float eps,
                                           const float* cs, const float* sn) {
  if (w) {
    const float rs =
        1.0f / sqrtf(group_sum<LPK>(dot4(x, x)) / static_cast<float>(4 * LPK) + eps);
    const f32x4 wv = *reinterpret_cast<const f32x4*>(w + 4 * d4);
    x = f32x4{x.x * rs * wv.x, x.y * rs * wv.y, x.z * rs * wv.z, x.w * rs * wv.w};
  }
  const f32x4 y = {__shfl_xor(x.x, LPK / 2, kWave), __shfl_xor(x.y, LPK / 2, kWave),
                   __shfl_xor(x.z, LPK / 2, kWave), __shfl_xor(x.w, LPK / 2, kWave)};
  const bool first = d4 < LPK / 2;
  const int f0 = 4 * (d4 % (LPK / 2));
  f32x4 out;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float cv = cs[f0 + c], sv = sn[f0 + c];
    out[c] = first ? x[c] * cv - y[c] * sv : y[c] * sv + x[c] * cv;
  }
  return out;
}

template <int D, bool FOLD>
__device__ __forceinline__ void attn_decode_body(const DecodeArgs& a, const QkvFold& f) {
  constexpr int LPK = D / 4;          // lanes per key row
  constexpr int KPW = kWave / LPK;    // keys per wave load
  constexpr int NG = kWaves * KPW;    // independent softmax groups per workgroup
  constexpr int HALF = D / 2;
  __shared__ float s_ml[NG][kRowTile][2];
  __shared__ f32x4 s_o[NG][kRowTile][LPK];
  __shared__ float s_rot[FOLD ? kFoldRows : 1][2][HALF];  // fold: cos, sin per (new row, pair)

  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int sub = lane / LPK;
  const int d4 = lane % LPK;
  const int g_id = w * KPW + sub;

  const int64_t G = a.H / a.Hk;
  const int64_t split = blockIdx.x % a.nsplit;
  const int64_t bh = blockIdx.x / a.nsplit;
  const int64_t hk = bh % a.Hk;
  const int64_t b = bh / a.Hk;
  const int64_t ks = split * a.kps;
  const int64_t ke = ks + a.kps < a.L ? ks + a.kps : a.L;
  const float* kbase = a.k + b * a.kv_sb + hk * a.kv_sh + 4 * d4;
  const float* vbase = a.v + b * a.kv_sb + hk * a.kv_sh + 4 * d4;
  const int64_t R = G * a.T;  // query rows of this KV head: r -> (t = r / G, h = hk*G + r % G)

  // Raw q of a row tile; the first tile's is loaded before the fold's
  // barriers, so its latency overlaps them.
  f32x4 qraw[kRowTile];
  auto load_q = [&](int64_t r0) {
#pragma unroll
    for (int r = 0; r < kRowTile; ++r) {
      qraw[r] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (r0 + r < R) {
        const int64_t t = (r0 + r) / G;
        const int64_t h = hk * G + (r0 + r) % G;
        qraw[r] = *reinterpret_cast<const f32x4*>(a.q + ((b * a.T + t) * a.H + h) * D + 4 * d4);
      }
    }
  };
  load_q(0);

  if constexpr (FOLD) {
    // This split's share of the new rows [pos, pos + T) (ke <= L = pos + T):
    // normalised, rotated keys and the values into the cache, one row per
    // lane group.  No other workgroup reads these rows in this launch; this
    // one reads them after the second barrier.  The rotations' cosines and
    // sines are tabulated once per workgroup, T * D/2 sincosf in parallel,
    // while the raw rows load.
    const int64_t p0 = (ks > a.pos ? ks : a.pos) + g_id;
    f32x4 kraw = {0.f, 0.f, 0.f, 0.f}, vraw = {0.f, 0.f, 0.f, 0.f};
    const int64_t row0 = ((b * a.T + (p0 - a.pos)) * a.Hk + hk) * D + 4 * d4;
    if (p0 < ke) {
      kraw = *reinterpret_cast<const f32x4*>(f.kn + row0);
      vraw = *reinterpret_cast<const f32x4*>(f.vn + row0);
    }
    for (int e = threadIdx.x; e < a.T * HALF; e += kThreads) {
      const int t = e / HALF, i = e % HALF;
      float sn, cs;
      sincosf(static_cast<float>(a.pos + t) * f.freqs[i], &sn, &cs);
      s_rot[t][0][i] = cs;
      s_rot[t][1][i] = sn;
    }
    __syncthreads();
    for (int64_t p = p0; p < ke; p += NG) {
      const int64_t t = p - a.pos;
      if (p != p0) {
        const int64_t src = ((b * a.T + t) * a.Hk + hk) * D + 4 * d4;
        kraw = *reinterpret_cast<const f32x4*>(f.kn + src);
        vraw = *reinterpret_cast<const f32x4*>(f.vn + src);
      }
      const int64_t dst = b * a.kv_sb + hk * a.kv_sh + p * a.kv_st + 4 * d4;
      *reinterpret_cast<f32x4*>(f.ck + dst) =
          norm_rope<LPK>(kraw, d4, f.kn_w, f.eps, s_rot[t][0], s_rot[t][1]);
      *reinterpret_cast<f32x4*>(f.cv + dst) = vraw;
    }
    __syncthreads();
  }

  for (int64_t r0 = 0; r0 < R; r0 += kRowTile) {
    const int nr = static_cast<int>(R - r0 < kRowTile ? R - r0 : kRowTile);
    if (r0 > 0) load_q(r0);
    f32x4 q[kRowTile], acc[kRowTile];
    float m[kRowTile], l[kRowTile];
    int lim[kRowTile];  // keys j < lim[r] are visible to row r
    int jend = static_cast<int>(ks);
#pragma unroll
    for (int r = 0; r < kRowTile; ++r) {
      acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
      m[r] = -INFINITY;
      l[r] = 0.f;
      q[r] = f32x4{0.f, 0.f, 0.f, 0.f};
      lim[r] = static_cast<int>(ks);
      if (r < nr) {
        const int64_t t = (r0 + r) / G;
        q[r] = qraw[r];
        if constexpr (FOLD)
          q[r] = norm_rope<LPK>(q[r], d4, f.qn_w, f.eps, s_rot[t][0], s_rot[t][1]);
        q[r] *= a.qscale;
        const int64_t c = a.pos + t + 1;  // causal: key j <= pos + t
        lim[r] = static_cast<int>(c < ke ? c : ke);
        jend = lim[r] > jend ? lim[r] : jend;
      }
    }
    // Keys of this lane group: ks + (it*kWaves + w)*KPW + sub.
    for (int j0 = static_cast<int>(ks) + w * KPW + sub; j0 < jend; j0 += kUnroll * kWaves * KPW) {
      f32x4 kf[kUnroll], vf[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = j0 + u * kWaves * KPW;
        if (j < jend) {
          kf[u] = *reinterpret_cast<const f32x4*>(kbase + static_cast<int64_t>(j) * a.kv_st);
          vf[u] = *reinterpret_cast<const f32x4*>(vbase + static_cast<int64_t>(j) * a.kv_st);
        } else {
          kf[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          vf[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
      // The kUnroll keys' scores are independent (their shuffles overlap);
      // the running max and the rescale are then updated once per batch.
#pragma unroll
      for (int r = 0; r < kRowTile; ++r) {
        if (r < nr) {
          float sc[kUnroll];
          float mx = m[r];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            sc[u] = group_sum<LPK>(dot4(q[r], kf[u]));
            if (j0 + u * kWaves * KPW < lim[r]) mx = fmaxf(mx, sc[u]);
          }
          if (mx != -INFINITY) {  // else no key of this row seen yet, none in the batch
            const float c = exp2f(m[r] - mx);
            float ps = 0.f;
            f32x4 pv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
              if (j0 + u * kWaves * KPW < lim[r]) {
                const float pr = exp2f(sc[u] - mx);
                ps += pr;
                pv += vf[u] * pr;
              }
            }
            l[r] = l[r] * c + ps;
            acc[r] = acc[r] * c + pv;
            m[r] = mx;
          }
        }
      }
    }
    // Merge the NG groups: publish, then each thread finishes (row, float4) items.
    __syncthreads();  // previous row tile's readers are done with LDS
#pragma unroll
    for (int r = 0; r < kRowTile; ++r) {
      if (r < nr) {
        s_o[g_id][r][d4] = acc[r];
        if (d4 == 0) {
          s_ml[g_id][r][0] = m[r];
          s_ml[g_id][r][1] = l[r];
        }
      }
    }
    __syncthreads();
    for (int it = threadIdx.x; it < nr * LPK; it += kThreads) {
      const int r = it / LPK;
      const int c4 = it % LPK;
      float M = -INFINITY;
      for (int g = 0; g < NG; ++g) M = fmaxf(M, s_ml[g][r][0]);
      float lsum = 0.f;
      f32x4 osum = {0.f, 0.f, 0.f, 0.f};
      if (M != -INFINITY) {
        for (int g = 0; g < NG; ++g) {
          const float e = exp2f(s_ml[g][r][0] - M);
          lsum += s_ml[g][r][1] * e;
          osum += s_o[g][r][c4] * e;
        }
      }
      const int64_t row = r0 + r;
      const int64_t t = row / G;
      const int64_t h = hk * G + row % G;
      const int64_t orow = (b * a.T + t) * a.H + h;
      if (a.nsplit == 1) {
        // Split 0 holds key 0, which every row sees: lsum >= 1.
        *reinterpret_cast<f32x4*>(a.o + orow * D + 4 * c4) = osum * (1.0f / lsum);
      } else {
        *reinterpret_cast<f32x4*>(a.part_o + (orow * a.nsplit + split) * D + 4 * c4) = osum;
        if (c4 == 0) {
          a.part_ml[(orow * a.nsplit + split) * 2 + 0] = M;
          a.part_ml[(orow * a.nsplit + split) * 2 + 1] = lsum;
        }
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(DecodeArgs a) {
  attn_decode_body<D, false>(a, QkvFold{});
}

template <int D>
__global__ __launch_bounds__(kThreads) void attn_decode_qkv_kernel(DecodeArgs a, QkvFold f) {
  attn_decode_body<D, true>(a, f);
}

// One wave per output row: merge the splits in split order.  The split
// weights exp2(m_s - M) are computed lane-parallel and kept in LDS, so the
// loop over splits only streams part_o with independent loads.
constexpr int kMaxSplits = 2048;

template <int D>
__global__ __launch_bounds__(kThreads) void attn_decode_combine(const float* __restrict__ part_o,
                                                                const float* __restrict__ part_ml,
                                                                float* __restrict__ o,
                                                                int64_t rows, int nsplit) {
  __shared__ float s_e[kWaves][kMaxSplits];
  const int w = threadIdx.x / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + w;
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= rows) return;  // whole waves leave; no block barrier follows
  const float* ml = part_ml + row * nsplit * 2;
  float M = -INFINITY;
  for (int s = lane; s < nsplit; s += kWave) M = fmaxf(M, ml[2 * s]);
  M = wave_max(M);
  float lpart = 0.f;
  for (int s = lane; s < nsplit; s += kWave) {
    const float ms = ml[2 * s];
    // A split with no visible key has m = -inf and l = 0: weight 0.
    const float e = ms == -INFINITY ? 0.f : exp2f(ms - M);
    s_e[w][s] = e;
    lpart += ml[2 * s + 1] * e;
  }
  const float lsum = wave_sum(lpart);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int PER = D / kWave;
  float acc[PER] = {};
  const float* po = part_o + row * nsplit * D + lane;
  int s = 0;
  for (; s + 4 <= nsplit; s += 4) {
    float x[4][PER];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int p = 0; p < PER; ++p) x[u][p] = po[(s + u) * D + p * kWave];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int p = 0; p < PER; ++p) acc[p] += x[u][p] * s_e[w][s + u];
  }
  for (; s < nsplit; ++s)
#pragma unroll
    for (int p = 0; p < PER; ++p) acc[p] += po[s * D + p * kWave] * s_e[w][s];
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int p = 0; p < PER; ++p) o[row * D + p * kWave + lane] = acc[p] * inv;
}

struct DecodePlan {
  int nsplit;
  int64_t kps;
};

DecodePlan decode_plan(int64_t B, int64_t Hk, int64_t L) {
  const int64_t heads = B * Hk;
  int64_t want = (kTargetBlocks + heads - 1) / heads;
  const int64_t most = (L + kMinKeysPerSplit - 1) / kMinKeysPerSplit;
  if (want > most) want = most;
  if (want < 1) want = 1;
  if (want > kMaxSplits) want = kMaxSplits;
  const int64_t kps = (L + want - 1) / want;
  return DecodePlan{static_cast<int>((L + kps - 1) / kps), kps};
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

extern "C" int ember_kv_write(const float* src, float* cache, int64_t B, int64_t T, int64_t Hk,
                              int64_t D, int64_t S, int64_t pos, ember_stream_t s) {
  if (B < 0 || T < 0 || Hk < 0 || D < 0 || pos < 0 || pos + T > S) return EMBER_EINVAL;
  const int64_t n = B * T * Hk * D;
  if (n == 0) return EMBER_OK;
  if (!src || !cache) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (D % 4 == 0 && aligned16(src) && aligned16(cache))
    kv_write_kernel<4><<<grid_1d(n / 4, kThreads), kThreads, 0, st>>>(src, cache, n / 4, T, Hk,
                                                                       D, S, pos);
  else
    kv_write_kernel<1><<<grid_1d(n, kThreads), kThreads, 0, st>>>(src, cache, n, T, Hk, D, S,
                                                                   pos);
  return launch_status();
}

extern "C" int ember_kv_read_expanded(const float* cache, float* out, int64_t B, int64_t Hk,
                                      int64_t group, int64_t L, int64_t D, int64_t S,
                                      ember_stream_t s) {
  if (B < 0 || Hk < 0 || group <= 0 || L < 0 || L > S || D < 0) return EMBER_EINVAL;
  const int64_t n = B * Hk * group * L * D;
  if (n == 0) return EMBER_OK;
  if (!cache || !out) return EMBER_EINVAL;
  hipStream_t st = as_stream(s);
  if (D % 4 == 0 && aligned16(cache) && aligned16(out))
    kv_read_expanded_kernel<4><<<grid_1d(n / 4, kThreads), kThreads, 0, st>>>(
        cache, out, n / 4, Hk, group, L, D, S);
  else
    kv_read_expanded_kernel<1><<<grid_1d(n, kThreads), kThreads, 0, st>>>(cache, out, n, Hk,
                                                                           group, L, D, S);
  return launch_status();
}

extern "C" size_t ember_attn_decode_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t Hk,
                                                    int64_t D, int64_t L) {
  if (B <= 0 || T <= 0 || H <= 0 || Hk <= 0 || D <= 0 || L <= 0) return 0;
  const DecodePlan p = decode_plan(B, Hk, L);
  if (p.nsplit == 1) return 0;
  return static_cast<size_t>(B * T * H) * p.nsplit * (D + 2) * sizeof(float);
}

namespace {

// Shared by ember_attn_decode and ember_attn_decode_qkv (fold != null): checks
// the split plan against the grid and the workspace, launches the split
// kernel, then the merge when there is more than one split.
int run_decode(const float* q, const float* k, const float* v, float* o, int64_t B, int64_t T,
               int64_t H, int64_t Hk, int64_t D, int64_t L, int64_t pos, int64_t kv_sb,
               int64_t kv_sh, int64_t kv_st, float scale, void* workspace,
               size_t workspace_bytes, const QkvFold* fold, hipStream_t st) {
  const DecodePlan p = decode_plan(B, Hk, L);
  const int64_t blocks = B * Hk * p.nsplit;
  if (blocks > 0x7fffffff) return EMBER_EINVAL;
  const size_t need = ember_attn_decode_workspace_bytes(B, T, H, Hk, D, L);
  if (need && (!workspace || workspace_bytes < need)) return EMBER_EINVAL;
  DecodeArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  const int64_t rows = B * T * H;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = need ? a.part_o + rows * p.nsplit * D : nullptr;
  a.T = T;
  a.H = H;
  a.Hk = Hk;
  a.L = L;
  a.pos = pos;
  a.kv_sb = kv_sb;
  a.kv_sh = kv_sh;
  a.kv_st = kv_st;
  a.kps = p.kps;
  a.nsplit = p.nsplit;
  a.qscale = scale * 1.4426950408889634f;
  const unsigned grid = static_cast<unsigned>(blocks);
  if (fold && D == 128)
    attn_decode_qkv_kernel<128><<<grid, kThreads, 0, st>>>(a, *fold);
  else if (fold)
    attn_decode_qkv_kernel<64><<<grid, kThreads, 0, st>>>(a, *fold);
  else if (D == 128)
    attn_decode_kernel<128><<<grid, kThreads, 0, st>>>(a);
  else
    attn_decode_kernel<64><<<grid, kThreads, 0, st>>>(a);
  int rc = launch_status();
  if (rc || p.nsplit == 1) return rc;
  const unsigned cgrid = static_cast<unsigned>(cdiv(rows, kWaves));
  if (D == 128)
    attn_decode_combine<128><<<cgrid, kThreads, 0, st>>>(a.part_o, a.part_ml, o, rows, p.nsplit);
  else
    attn_decode_combine<64><<<cgrid, kThreads, 0, st>>>(a.part_o, a.part_ml, o, rows, p.nsplit);
  return launch_status();
}

}  // namespace

extern "C" int ember_attn_decode(const float* q, const float* k, const float* v, float* o,
                                 int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D,
                                 int64_t L, int64_t pos, int64_t kv_sb, int64_t kv_sh,
                                 int64_t kv_st, float scale, void* workspace,
                                 size_t workspace_bytes, ember_stream_t s) {
  if (B < 0 || T < 0 || H <= 0 || Hk <= 0 || H % Hk != 0 || pos < 0) return EMBER_EINVAL;
  if (D != 64 && D != 128) return EMBER_EINVAL;
  if (B == 0 || T == 0) return EMBER_OK;
  if (L < 1 || !q || !k || !v || !o) return EMBER_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || kv_sb % 4 ||
      kv_sh % 4 || kv_st % 4)
    return EMBER_EINVAL;
  return run_decode(q, k, v, o, B, T, H, Hk, D, L, pos, kv_sb, kv_sh, kv_st, scale, workspace,
                    workspace_bytes, nullptr, as_stream(s));
}

extern "C" int ember_attn_decode_qkv(const float* q, const float* k, const float* v, int64_t B,
                                     int64_t T, int64_t H, int64_t Hk, int64_t D,
                                     const float* q_norm_w, const float* k_norm_w, float eps,
                                     const float* freqs_host, int64_t pos, float* cache_k,
                                     float* cache_v, int64_t S, float scale, float* o,
                                     void* workspace, size_t workspace_bytes, ember_stream_t s) {
  if (B < 0 || T < 0 || H <= 0 || Hk <= 0 || H % Hk != 0 || pos < 0 || pos + T > S ||
      !freqs_host)
    return EMBER_EINVAL;
  if ((D != 64 && D != 128) || T > kFoldRows) return EMBER_EINVAL;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !o || !cache_k || !cache_v) return EMBER_EINVAL;
  for (const float* ptr : {q, k, v, static_cast<const float*>(o),
                           static_cast<const float*>(cache_k), static_cast<const float*>(cache_v)})
    if (!aligned16(ptr)) return EMBER_EINVAL;
  if ((q_norm_w && !aligned16(q_norm_w)) || (k_norm_w && !aligned16(k_norm_w)))
    return EMBER_EINVAL;
  QkvFold f{};
  f.kn = k;
  f.vn = v;
  f.qn_w = q_norm_w;
  f.kn_w = k_norm_w;
  f.ck = cache_k;
  f.cv = cache_v;
  f.eps = eps;
  for (int64_t i = 0; i < D / 2; ++i) f.freqs[i] = freqs_host[i];
  return run_decode(q, cache_k, cache_v, o, B, T, H, Hk, D, pos + T, pos, Hk * S * D, S * D, D,
                    scale, workspace, workspace_bytes, &f, as_stream(s));
}
