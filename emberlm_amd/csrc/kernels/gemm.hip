// fp32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Replaces cublasSgemm / cublasSgemmStridedBatched behind ops::matmul and
// ops::bmm (reference src/ops/matmul.cpp:13-93).  One kernel template covers
// the four transpose cases: each operand is staged through LDS either
// K-contiguous ([rows][BK+4], read as b128 so one LDS read feeds four MFMA
// k-steps) or MN-contiguous ([BK][rows+8], read as b32 with consecutive lanes
// on consecutive rows).  The k index an MFMA step consumes is permuted so that
// lane group g = lane/32 owns k = 8*slab + 4*g + j for step j; A and B use the
// same permutation, so the contraction is unchanged.
//
// Block tile 128x128, 256 threads = 4 waves in 2x2, wave tile 64x64 = 2x2
// MFMA tiles of 32x32 (64 accumulator registers per lane).  Global loads for
// stage k+1 are issued before the MFMAs of stage k (double-buffered LDS, one
// barrier per stage).  Tiles are ordered so that tiles sharing A rows land
// on the same XCD (block b runs on XCD b % 8) and, within it, in groups of 8
// tile rows for L2 reuse.
#include "common.h"

using namespace ember;

namespace {

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC;
  float alpha, beta;
  int tiles_m, tiles_n;
};

template <bool KC, int ROWS, int BK>
struct Stage {
  static constexpr int kStride = KC ? (BK + 4) : (ROWS + 8);
  static constexpr int kSize = KC ? ROWS * (BK + 4) : BK * (ROWS + 8);
  static constexpr int kChunks = ROWS * BK / 4;           // float4 chunks per tile
  static constexpr int kPerThread = kChunks / kThreads;   // loads per thread
  static_assert(kChunks % kThreads == 0, "tile not divisible among threads");

  f32x4 reg[kPerThread];

  // Global -> registers.  Operand rows [row0, row0+ROWS) x k [k0, k0+BK),
  // zero outside [0,R) x [0,K).
  template <bool VEC>
  __device__ __forceinline__ void load(const float* __restrict__ X, int64_t ld, int64_t R,
                                       int64_t K, int64_t row0, int64_t k0) {
#pragma unroll
    for (int p = 0; p < kPerThread; ++p) {
      const int c = threadIdx.x + p * kThreads;
      int64_t r, k;
      if (KC) {
        r = row0 + c / (BK / 4);
        k = k0 + 4 * (c % (BK / 4));
      } else {
        k = k0 + c / (ROWS / 4);
        r = row0 + 4 * (c % (ROWS / 4));
      }
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (KC) {
        if (r < R) {
          const float* src = X + r * ld + k;
          if (VEC && k + 3 < K) {
            v = *reinterpret_cast<const f32x4*>(src);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (k + e < K) ? src[e] : 0.f;
          }
        }
      } else {
        if (k < K) {
          const float* src = X + k * ld + r;
          if (VEC && r + 3 < R) {
            v = *reinterpret_cast<const f32x4*>(src);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (r + e < R) ? src[e] : 0.f;
          }
        }
      }
      reg[p] = v;
    }
  }

  // Registers -> LDS in this operand's layout.
  __device__ __forceinline__ void store(float* __restrict__ lds) const {
#pragma unroll
    for (int p = 0; p < kPerThread; ++p) {
      const int c = threadIdx.x + p * kThreads;
      int off;
      if (KC) {
        off = (c / (BK / 4)) * kStride + 4 * (c % (BK / 4));
      } else {
        off = (c / (ROWS / 4)) * kStride + 4 * (c % (ROWS / 4));
      }
      *reinterpret_cast<f32x4*>(lds + off) = reg[p];
    }
  }

  // Fragment for MFMA steps j = 0..3 of k-slab `slab`, row `row` of the tile.
  __device__ __forceinline__ static f32x4 frag(const float* __restrict__ lds, int row, int slab,
                                               int g) {
    if (KC) {
      return *reinterpret_cast<const f32x4*>(lds + row * kStride + slab * 8 + 4 * g);
    } else {
      f32x4 v;
      const float* base = lds + (slab * 8 + 4 * g) * kStride + row;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = base[j * kStride];
      return v;
    }
  }
};

__device__ __forceinline__ void tile_coords(const GemmArgs& a, int& tm, int& tn) {
  const int tiles = a.tiles_m * a.tiles_n;
  int t = blockIdx.x;
  if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
  const int width = kGroupM * a.tiles_n;
  const int group = t / width;
  const int first = group * kGroupM;
  const int gsz = min(a.tiles_m - first, kGroupM);
  const int in = t - group * width;
  tm = first + in % gsz;
  tn = in / gsz;
}

template <bool A_KC, bool B_KC, bool VEC, int BK>
__global__ __launch_bounds__(kThreads) void gemm_f32_mfma(GemmArgs a) {
  using SA = Stage<A_KC, kBM, BK>;
  using SB = Stage<B_KC, kBN, BK>;
  __shared__ __attribute__((aligned(16))) float lds_a[2][SA::kSize];
  __shared__ __attribute__((aligned(16))) float lds_b[2][SB::kSize];

  int tm, tn;
  tile_coords(a, tm, tn);
  const int64_t bz = blockIdx.y;
  const float* __restrict__ A = a.A + bz * a.sA;
  const float* __restrict__ B = a.B + bz * a.sB;
  float* __restrict__ C = a.C + bz * a.sC;
  const int64_t m0 = static_cast<int64_t>(tm) * kBM;
  const int64_t n0 = static_cast<int64_t>(tn) * kBN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 5, r = lane & 31;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  SA sa;
  SB sb;
  const int64_t nk = (a.K + BK - 1) / BK;
  if (nk > 0) {
    sa.template load<VEC>(A, a.lda, a.M, a.K, m0, 0);
    sb.template load<VEC>(B, a.ldb, a.N, a.K, n0, 0);
    sa.store(lds_a[0]);
    sb.store(lds_b[0]);
  }
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = static_cast<int>(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      sa.template load<VEC>(A, a.lda, a.M, a.K, m0, (kt + 1) * BK);
      sb.template load<VEC>(B, a.ldb, a.N, a.K, n0, (kt + 1) * BK);
    }
    const float* la = lds_a[cur];
    const float* lb = lds_b[cur];
#pragma unroll
    for (int slab = 0; slab < BK / 8; ++slab) {
      f32x4 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = SA::frag(la, wm * 64 + i * 32 + r, slab, g);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = SB::frag(lb, wn * 64 + j * 32 + r, slab, g);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
    }
    if (more) {
      sa.store(lds_a[cur ^ 1]);
      sb.store(lds_b[cur ^ 1]);
    }
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA tile: lane (g, r), register e holds
  // row 8*(e/4) + 4*g + (e%4), column r.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + r;
      if (col >= a.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        if (row < a.M) {
          float* dst = C + row * a.ldc + col;
          const float v = a.alpha * acc[i][j][e];
          *dst = (a.beta != 0.f) ? v + a.beta * *dst : v;
        }
      }
    }
}

template <bool A_KC, bool B_KC>
int launch(const GemmArgs& a, int64_t batch, bool vec, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(a.tiles_m) * a.tiles_n, static_cast<unsigned>(batch));
  if (vec)
    gemm_f32_mfma<A_KC, B_KC, true, 16><<<grid, kThreads, 0, st>>>(a);
  else
    gemm_f32_mfma<A_KC, B_KC, false, 16><<<grid, kThreads, 0, st>>>(a);
  return launch_status();
}

}  // namespace

extern "C" int ember_gemm_f32(int transa, int transb, int64_t M, int64_t N, int64_t K,
                              float alpha, const float* A, int64_t lda, int64_t sA,
                              const float* B, int64_t ldb, int64_t sB, float beta, float* C,
                              int64_t ldc, int64_t sC, int64_t batch, ember_stream_t s) {
  if (M < 0 || N < 0 || K < 0 || batch < 1) return EMBER_EINVAL;
  if (M == 0 || N == 0) return EMBER_OK;
  if (!C || (K > 0 && (!A || !B))) return EMBER_EINVAL;
  if (lda < (transa ? M : K) || ldb < (transb ? K : N) || ldc < N) return EMBER_EINVAL;
  const int64_t tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
  if (tm * tn > 0x7fffffff || batch > 65535) return EMBER_EINVAL;
  GemmArgs a{A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, alpha, beta,
             static_cast<int>(tm), static_cast<int>(tn)};
  const bool vec = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                   (batch == 1 || (sA % 4 == 0 && sB % 4 == 0));
  hipStream_t st = as_stream(s);
  const bool a_kc = !transa, b_kc = transb != 0;
  if (a_kc && b_kc) return launch<true, true>(a, batch, vec, st);
  if (a_kc && !b_kc) return launch<true, false>(a, batch, vec, st);
  if (!a_kc && !b_kc) return launch<false, false>(a, batch, vec, st);
  return launch<false, true>(a, batch, vec, st);
}
