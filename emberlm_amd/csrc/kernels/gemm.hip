// fp32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Replaces cublasSgemm / cublasSgemmStridedBatched behind ops::matmul and
// ops::bmm (reference src/ops/matmul.cpp:13-93).  Kernel templates cover the
// four transpose cases: each operand tile is K-contiguous (read as b128, one
// LDS read feeds four MFMA k-steps) or MN-contiguous (read as b32 with
// consecutive lanes on consecutive rows).  The k index an MFMA step consumes
// is permuted so that lane group g = lane/32 owns k = 8*slab + 4*g + j for
// step j; A and B use the same permutation, so the contraction is unchanged.
//
// Block tiles 128x128 (three blocks per CU) or 256x128 (two per CU), 256
// threads = 4 waves in 2x2, wave tile (BM/2)x(BN/2) of 32x32 MFMA tiles held
// in accumulation registers.  A stage is BK = 16 = two k slabs, software
// pipelined inside one wave so the matrix core never waits on LDS (ordering
// fixed with sched_group_barrier): slab-0 MFMAs under the LDS reads of slab 1,
// one barrier, the next stage's slab-0 reads under the last slab-1 MFMAs.
//
// Main path, gemm_f32_dma: tiles are copied global -> LDS by
// global_load_lds_dwordx4 (no register staging, no LDS store instructions)
// into a 3-stage ring, two stages ahead of the MFMAs, with swizzled layouts
// instead of padding.  Fallback, gemm_f32_mfma (K % 16 != 0, unaligned or
// odd-width operands): global -> registers -> LDS, double-buffered, the
// stores interleaved with the MFMAs.  Both accumulate in the same k order,
// so they give identical bits.
//
// Tiles are ordered so that tiles sharing A rows land on the same XCD (block
// b runs on XCD b % 8) and, within it, in groups of 8 tile rows for L2 reuse.
// Small output grids with a long K (weight gradients: M, N = features,
// K = tokens) are split along K into a workspace of partial products that a
// second kernel sums in a fixed order, so results stay bitwise reproducible.
#include <type_traits>

#include "common.h"
#include "mfma_sched.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;
constexpr int kGroupM = 8;
constexpr int kCUs = 256;

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC;
  int64_t kchunk;  // > 0: blockIdx.y is a K split of this many k (last one clipped)
  float alpha, beta;
  int tiles_m, tiles_n;
  // Optional extent read from device memory at run time (LDS-DMA kernel and
  // the split-K reduce only): v = clamp(*dyn - dyn_base, 0, static extent);
  // dyn_dim 0: rows of C beyond v are not needed (whole tiles past v exit);
  // dyn_dim 1: K becomes v rounded up to 16 (operand rows up to there are read).
  const int64_t* dyn = nullptr;
  int64_t dyn_base = 0;
  int dyn_dim = 0;
  // Optional addend (single GEMMs only): C = alpha op(A) op(B) + beta D, with
  // D = C when null.  D may be C itself (ldd = ldc), never a shifted overlap.
  const float* D = nullptr;
  int64_t ldd = 0;
};

// The beta term's source for element (row, col) of the current C.
__device__ __forceinline__ const float* addend(const GemmArgs& a, const float* dst, int64_t row,
                                               int64_t col) {
  return a.D ? a.D + row * a.ldd + col : dst;
}

__device__ __forceinline__ int64_t dyn_extent(const GemmArgs& a, int64_t full) {
  return min(max(*a.dyn - a.dyn_base, int64_t{0}), full);
}

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

template <int BM, int BN>
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int& tm, int& tn) {
  const int tiles = a.tiles_m * a.tiles_n;
  int t = blockIdx.x;
  if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
  if (a.dyn && a.dyn_dim == 0) {
    // Row tiles past a count read on the device are skipped.  Each XCD takes
    // a range of whole columns (every row tile of them), so each keeps the
    // same share of the work that remains whatever the count; with groups of
    // tile rows per XCD, the XCDs holding the first rows would do it all.
    tm = t % a.tiles_m;
    tn = t / a.tiles_m;
    return;
  }
  const int width = kGroupM * a.tiles_n;
  const int group = t / width;
  const int first = group * kGroupM;
  const int gsz = min(a.tiles_m - first, kGroupM);
  const int in = t - group * width;
  tm = first + in % gsz;
  tn = in / gsz;
}

template <bool A_KC, bool B_KC, bool VEC, int BM, int BN, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void gemm_f32_mfma(GemmArgs a) {
  using SA = Stage<A_KC, BM, kBK>;
  using SB = Stage<B_KC, BN, kBK>;
  constexpr int FI = BM / 64, FJ = BN / 64;             // 32x32 tiles per wave
  constexpr int NR = FI * (A_KC ? 1 : 4) + FJ * (B_KC ? 1 : 4);  // LDS reads per slab
  constexpr int NW = SA::kPerThread + SB::kPerThread;   // LDS stores per stage
  constexpr int NM = 4 * FI * FJ;                       // MFMAs per slab
  __shared__ __attribute__((aligned(16))) float lds_a[2][SA::kSize];
  __shared__ __attribute__((aligned(16))) float lds_b[2][SB::kSize];

  int tm, tn;
  tile_coords<BM, BN>(a, tm, tn);
  const int64_t bz = blockIdx.y;
  const float* __restrict__ A = a.A + bz * a.sA;
  const float* __restrict__ B = a.B + bz * a.sB;
  float* __restrict__ C = a.C + bz * a.sC;
  const int64_t K = a.kchunk > 0 ? min(a.kchunk, a.K - bz * a.kchunk) : a.K;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 5, r = lane & 31;
  const int arow = wm * (BM / 2) + r, brow = wn * (BN / 2) + r;

  f32x16 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  SA sa;
  SB sb;
  const int64_t nk = (K + kBK - 1) / kBK;
  if (nk > 0) {
    sa.template load<VEC>(A, a.lda, a.M, K, m0, 0);
    sb.template load<VEC>(B, a.ldb, a.N, K, n0, 0);
    sa.store(lds_a[0]);
    sb.store(lds_b[0]);
  }
  __syncthreads();

  f32x4 fa0[FI], fb0[FJ], fa1[FI], fb1[FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i) fa0[i] = SA::frag(lds_a[0], arow + i * 32, 0, g);
#pragma unroll
  for (int j = 0; j < FJ; ++j) fb0[j] = SB::frag(lds_b[0], brow + j * 32, 0, g);

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = static_cast<int>(kt & 1);
    // Stage kt+1; the last iteration reloads its own stage into the idle
    // buffer, which nothing reads afterwards.
    const int64_t knext = (kt + 1 < nk ? kt + 1 : kt) * kBK;
    sa.template load<VEC>(A, a.lda, a.M, K, m0, knext);
    sb.template load<VEC>(B, a.ldb, a.N, K, n0, knext);
    const float* la = lds_a[cur];
    const float* lb = lds_b[cur];
    float* na = lds_a[cur ^ 1];
    float* nb = lds_b[cur ^ 1];

#pragma unroll
    for (int i = 0; i < FI; ++i) fa1[i] = SA::frag(la, arow + i * 32, 1, g);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb1[j] = SB::frag(lb, brow + j * 32, 1, g);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[i][s], fb0[j][s], acc[i][j], 0, 0, 0);
    interleave<NR, NM, 0x100>();

    sa.store(na);
    sb.store(nb);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[j][s], acc[i][j], 0, 0, 0);
    interleave<NW, NM / 2, 0x200>();
    __syncthreads();

#pragma unroll
    for (int i = 0; i < FI; ++i) fa0[i] = SA::frag(na, arow + i * 32, 0, g);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb0[j] = SB::frag(nb, brow + j * 32, 0, g);
#pragma unroll
    for (int s = 2; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[j][s], acc[i][j], 0, 0, 0);
    interleave<NR, NM / 2, 0x100>();
  }

  // Accumulator layout of a 32x32 MFMA tile: lane (g, r), register e holds
  // row 8*(e/4) + 4*g + (e%4), column r.
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const int64_t col = n0 + wn * (BN / 2) + j * 32 + r;
      if (col >= a.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
        if (row < a.M) {
          float* dst = C + row * a.ldc + col;
          const float v = a.alpha * acc[i][j][e];
          *dst = (a.beta != 0.f) ? v + a.beta * *addend(a, dst, row, col) : v;
        }
      }
    }
}


// ---------------------------------------------------------------- LDS DMA
// Operand tiles go global -> LDS with global_load_lds_dwordx4: lane L of a
// wave-instruction writes 16 bytes at LDS base + 16 L, so one instruction
// fills a contiguous 1 KB block and the choice of which global 16 bytes each
// lane fetches sets the layout.  No registers stage the tile and no LDS store
// instruction runs.
//   K-contiguous tile [ROWS][16]: 16-row blocks of 64 16-byte units; row x's
//     k-chunk c sits at unit 4 (x % 16) + (c ^ swz(x % 16)).
//   MN-contiguous tile [16][ROWS]: k-row k's chunk q (4 floats) sits at
//     chunk position q ^ (8 ((k >> 2) & 1)).
// Both keep the fragment reads free of bank conflicts without padding.
__device__ __forceinline__ int swz(int x) { return ((x >> 1) ^ (x >> 3)) & 3; }

//   BUF: the copies are buffer_load_dwordx4 ... lds through a buffer resource
//     based at the block's first row (K-contiguous) or column (MN-contiguous),
//     with 32-bit per-lane byte offsets and the stage's offset in an SGPR;
//     otherwise global_load_lds_dwordx4 with a 64-bit address per lane.  Same
//     bytes to the same LDS places: 1.3-2.1% faster on the c5 NT shapes (fewer
//     address registers and address operations per copy).  The launcher picks
//     BUF when every offset of the product stays below 2^31 bytes.
template <bool KC, int ROWS, bool BUF>
struct DmaTile {
  static constexpr int kFloats = ROWS * 16;   // one stage
  static constexpr int kInsts = ROWS / 64;    // wave-instructions per wave per stage
  const float* src[kInsts];                    // !BUF: this lane's 16 bytes, stage 0
  int64_t step;                                // !BUF: element stride between stages
  __amdgpu_buffer_rsrc_t rsrc;                 // BUF: the block's first row / column
  int voff[kInsts];                            // BUF: this lane's byte offset, stage 0
  int bstep;                                   // BUF: bytes between stages

  __device__ __forceinline__ void init(const float* X, int64_t ld, int64_t R, int64_t row0,
                                       int w, int lane) {
    const int64_t base = KC ? row0 * ld : row0;  // elements from X to the buffer's start
    if constexpr (BUF)
      rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + base), 0, 0x7fffffff,
                                               0x00020000);
#pragma unroll
    for (int q = 0; q < kInsts; ++q) {
      const int t = w + 4 * q;  // 1 KB block of the tile
      int64_t e;                // this lane's first element
      if (KC) {
        const int x = lane >> 2;
        const int64_t row = min(row0 + 16 * t + x, R - 1);  // rows past R: never stored
        e = row * ld + 4 * ((lane & 3) ^ swz(x));
      } else {
        constexpr int kRowsPer = 256 / ROWS;   // k-rows per 1 KB block
        constexpr int kLanesPer = 64 / kRowsPer;
        const int k = t * kRowsPer + lane / kLanesPer;
        const int q4 = (lane % kLanesPer) ^ (8 * ((k >> 2) & 1));
        const int64_t col = min(row0 + 4 * q4, R - 4);      // R % 4 == 0 on this path
        e = k * ld + col;
      }
      if constexpr (BUF)
        voff[q] = static_cast<int>((e - base) * 4);
      else
        src[q] = X + e;
    }
    step = KC ? 16 : 16 * ld;
    bstep = static_cast<int>(4 * step);
  }
  // Stage kt of this lane's loads into the stage buffer `dst` (LDS).
  __device__ __forceinline__ void issue(float* dst, int64_t kt, int w) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the kernel's launch stub
#pragma unroll
    for (int q = 0; q < kInsts; ++q) {
      float* d = dst + 256 * (w + 4 * q);
      if constexpr (BUF)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void*)d, 16, voff[q],
            static_cast<int>(kt) * bstep, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(src[q] + kt * step, d, 16, 0, 0);
    }
#endif
  }
};

// Fragment of 32-row tile `i` for MFMA steps j = 0..3 of slab s: one b128
// read at the lane's precomputed offset (K-contiguous), or four b32 reads of
// k-rows 8 s + 4 g + j at column position ((mb4 + 8 i) ^ 8 g) * 4 + r
// (MN-contiguous; mb4 = the wave's first column / 4).
template <bool KC, int ROWS>
__device__ __forceinline__ f32x4 dma_frag(const float* st, int off, int i, int s, int g, int r,
                                          int mb4) {
  if (KC) return *reinterpret_cast<const f32x4*>(st + off + i * 32 * 16);
  f32x4 v;
  const int q = (mb4 + 8 * i) ^ (8 * g);
  const float* p = st + (8 * s + 4 * g) * ROWS + (q << 2) + r;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = p[j * ROWS];
  return v;
}

template <bool A_KC, bool B_KC, int BM, int BN, int OCC, bool BUF>
__global__ __launch_bounds__(kThreads, OCC) void gemm_f32_dma(GemmArgs a) {
  using TA = DmaTile<A_KC, BM, BUF>;
  using TB = DmaTile<B_KC, BN, BUF>;
  constexpr int FI = BM / 64, FJ = BN / 64;
  // An M-contiguous A on 256-row tiles is read as b128 rows of four
  // consecutive tile rows (see load_a), one read per MFMA k-step of a slab.
  constexpr bool kPermA = !A_KC && FI == 4;
  constexpr int NR = (A_KC ? FI : kPermA ? 4 : 4 * FI) + FJ * (B_KC ? 1 : 4);
  constexpr int NM = 4 * FI * FJ;
  constexpr int kStage = TA::kFloats + TB::kFloats;
  __shared__ __attribute__((aligned(1024))) float lds[3 * kStage];  // 3-stage ring
  constexpr int NI = TA::kInsts + TB::kInsts;  // DMA instructions per wave per stage

  int tm, tn;
  tile_coords<BM, BN>(a, tm, tn);
  const int64_t bz = blockIdx.y;
  const float* __restrict__ A = a.A + bz * a.sA;
  const float* __restrict__ B = a.B + bz * a.sB;
  float* __restrict__ C = a.C + bz * a.sC;
  int64_t K = a.kchunk > 0 ? min(a.kchunk, a.K - bz * a.kchunk) : a.K;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;
  if (a.dyn) {  // uniform per block: the whole block leaves or none of it
    if (a.dyn_dim == 0) {
      if (m0 >= dyn_extent(a, a.M)) return;
    } else {
      K = min(K, (dyn_extent(a, K) + 15) / 16 * 16);
      if (K == 0 && a.beta == 1.f && !a.D) return;  // C stays as it is
    }
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // The wave index as a uniform (SGPR) value: the DMA's LDS address (M0) is then
  // computed on the scalar unit, not read back from a vector register per copy.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 5, r = lane & 31;

  TA ta;
  TB tb;
  ta.init(A, a.lda, a.M, m0, wave_s, lane);
  tb.init(B, a.ldb, a.N, n0, wave_s, lane);

  // Per-lane fragment offsets (floats) inside a stage's A / B tile.
  // K-contiguous: slab s reads unit 4 (r % 16) + ((2 s + g) ^ swz(r % 16)) of
  // 16-row block (row / 16); MN-contiguous: k-row 8 s + 4 g + j, float
  // ((mbase / 4) ^ 8 g) * 4 + r.
  int offA[2], offB[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int u = 4 * (4 * (r & 15) + ((2 * s + g) ^ swz(r & 15))) + (r >> 4) * 256;
    offA[s] = u + wm * (BM / 2) * 16;
    offB[s] = u + wn * (BN / 2) * 16;
  }
  const int mbA = (wm * (BM / 2)) >> 2, mbB = (wn * (BN / 2)) >> 2;
  // A fragments of slab s.  With kPermA, MFMA tile i's row slot x holds tile
  // row wm * (BM / 2) + 4x + i (not 32i + x): the b128 at k-row 8s + 4g + j,
  // chunk mbA + r (swizzled as stored) is then lane (g, r)'s k-step-j value
  // for all four tiles.  Each output element sums the same products in the
  // same k order either way; only the rows' places in the registers move,
  // which the epilogue undoes.
  auto load_a = [&](const float* st, int s, f32x4 (&fa)[FI]) {
    if constexpr (kPermA) {
      const int off = 4 * ((mbA + r) ^ (8 * g));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(st + (8 * s + 4 * g + j) * BM + off);
#pragma unroll
        for (int i = 0; i < FI; ++i) fa[i][j] = v[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < FI; ++i) fa[i] = dma_frag<A_KC, BM>(st, offA[s], i, s, g, r, mbA);
    }
  };
  f32x16 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int64_t nk = K / 16;
  if (nk > 0) {
    ta.issue(lds, 0, wave_s);
    tb.issue(lds + TA::kFloats, 0, wave_s);
  }
  if (nk > 1) {
    ta.issue(lds + kStage, 1, wave_s);
    tb.issue(lds + kStage + TA::kFloats, 1, wave_s);
    wait_vm_lgkm0<NI>();
  } else {
    wait_vm_lgkm0<0>();
  }
  block_barrier();
  float* st0 = lds;
  f32x4 fa0[FI], fb0[FJ], fa1[FI], fb1[FJ];
  load_a(st0, 0, fa0);
#pragma unroll
  for (int j = 0; j < FJ; ++j) fb0[j] = dma_frag<B_KC, BN>(st0 + TA::kFloats, offB[0], j, 0, g, r, mbB);

  // The k loop is peeled: stages 0 .. nk-3 issue the DMA of the stage two
  // ahead, the last two none, so the DMA instructions sit in straight-line
  // code the scheduler can spread among the MFMAs (one burst of them holds up
  // this wave's MFMA issue while the memory pipe takes them).  Where: among
  // the slab-1 MFMAs before the barrier (the late form), or among the slab-0
  // MFMAs.  With buffer-resource copies the late form is 0.2-1.7% faster on
  // both tile shapes; with 64-bit-address copies the slab-0 form was 1-3%
  // faster on 128-row tiles.  The arithmetic is the same either way.
  constexpr bool kLateDma = BUF || BM == 256;
  int ic = 0;  // kt % 3
  auto stage = [&](int64_t kt, auto with_dma) {
    constexpr bool kDma = decltype(with_dma)::value;
    float* cur = lds + ic * kStage;
    float* nxt = lds + (ic == 2 ? 0 : ic + 1) * kStage;
    float* nx2 = lds + (ic == 0 ? 2 : ic - 1) * kStage;
    load_a(cur, 1, fa1);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb1[j] = dma_frag<B_KC, BN>(cur + TA::kFloats, offB[1], j, 1, g, r, mbB);
    if constexpr (kDma && !kLateDma) {
      ta.issue(nx2, kt + 2, wave_s);
      tb.issue(nx2 + TA::kFloats, kt + 2, wave_s);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[i][s], fb0[j][s], acc[i][j], 0, 0, 0);
    if constexpr (kDma && !kLateDma)
      interleave2<NR, NI, NM>();
    else
      interleave_mfma_first<NR, NM, 0x100>();
    if constexpr (kDma && kLateDma) {
      ta.issue(nx2, kt + 2, wave_s);
      tb.issue(nx2 + TA::kFloats, kt + 2, wave_s);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[j][s], acc[i][j], 0, 0, 0);
    if constexpr (kDma && kLateDma) interleave<NI, NM / 2, 0x020>();
    // Stage kt+1's DMA has landed (only stage kt+2's may still be in flight)
    // and every wave is done reading stage kt's buffer.
    if constexpr (kDma)
      wait_vm_lgkm0<NI>();
    else
      wait_vm_lgkm0<0>();
    block_barrier();
    load_a(nxt, 0, fa0);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb0[j] = dma_frag<B_KC, BN>(nxt + TA::kFloats, offB[0], j, 0, g, r, mbB);
#pragma unroll
    for (int s = 2; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[j][s], acc[i][j], 0, 0, 0);
    interleave<NR, NM / 2, 0x100>();
    ic = ic == 2 ? 0 : ic + 1;
  };
  int64_t kt = 0;
  for (; kt + 2 < nk; ++kt) stage(kt, std::true_type{});
  for (; kt < nk; ++kt) stage(kt, std::false_type{});

  if constexpr (BUF) {
#if defined(__HIP_DEVICE_COMPILE__)
    // Stores (and the beta term's loads) through buffer resources based at
    // this wave's first output row of C (and of D): a row's byte offset splits
    // into a uniform part (the MFMA register's row slot, in an SGPR) and the
    // lane's part (computed once), with no 64-bit address arithmetic per
    // element.  Rows at or past M are skipped by an explicit test, made only on
    // the wave tiles that reach M.  Same values as the form below.
    const int wm_s = wave_s >> 1, wn_s = wave_s & 1;
    const int64_t rw0 = m0 + wm_s * (BM / 2), cw0 = n0 + wn_s * (BN / 2);
    if (rw0 < a.M) {
      const float* Dm = a.D ? a.D : C;
      const int64_t ldd = a.D ? a.ldd : a.ldc;
      const __amdgpu_buffer_rsrc_t rc =
          __builtin_amdgcn_make_buffer_rsrc(C + rw0 * a.ldc + cw0, 0, 0x7fffffff, 0x00020000);
      const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(Dm + rw0 * ldd + cw0), 0, 0x7fffffff, 0x00020000);
      const int lrow = kPermA ? 16 * g : 4 * g;  // the lane's part of the row
      const int lc = static_cast<int>((lrow * a.ldc + r) * 4);
      const int ld = static_cast<int>((lrow * ldd + r) * 4);
      const int rows_left = static_cast<int>(min(a.M - rw0, int64_t{BM}));
      // CHECKED: the wave tile reaches M.  BETA: the beta term is read, all 16
      // values of an MFMA tile before the first is used (one wait per tile).
      auto store_all = [&](auto checked, auto with_beta) {
        constexpr bool kChecked = decltype(checked)::value, kBeta = decltype(with_beta)::value;
#pragma unroll
        for (int j = 0; j < FJ; ++j) {
          if (cw0 + j * 32 + r >= a.N) continue;
#pragma unroll
          for (int i = 0; i < FI; ++i) {
            float d[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int ru = kPermA ? 4 * (8 * (e >> 2) + (e & 3)) + i
                                    : i * 32 + 8 * (e >> 2) + (e & 3);
              d[e] = 0.f;
              if (kBeta && !(kChecked && ru + lrow >= rows_left))
                d[e] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               rd, ld + 128 * j, static_cast<int>(ru * ldd * 4), 0));
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              // the row slot's uniform part; the lane's part is in lc / ld
              const int ru = kPermA ? 4 * (8 * (e >> 2) + (e & 3)) + i
                                    : i * 32 + 8 * (e >> 2) + (e & 3);
              if (kChecked && ru + lrow >= rows_left) continue;
              const float v = a.alpha * acc[i][j][e];
              const float out = kBeta ? v + a.beta * d[e] : v;
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out), rc,
                                                    lc + 128 * j,
                                                    static_cast<int>(ru * a.ldc * 4), 0);
            }
          }
        }
      };
      const bool full = rows_left >= BM / 2;
      if (a.beta != 0.f) {
        if (full) store_all(std::false_type{}, std::true_type{});
        else store_all(std::true_type{}, std::true_type{});
      } else {
        if (full) store_all(std::false_type{}, std::false_type{});
        else store_all(std::true_type{}, std::false_type{});
      }
    }
#endif
  } else {
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const int64_t col = n0 + wn * (BN / 2) + j * 32 + r;
        if (col >= a.N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int x = 8 * (e >> 2) + 4 * g + (e & 3);  // the MFMA tile's row slot
          const int64_t row = m0 + wm * (BM / 2) + (kPermA ? 4 * x + i : i * 32 + x);
          if (row < a.M) {
            float* dst = C + row * a.ldc + col;
            const float v = a.alpha * acc[i][j][e];
            *dst = (a.beta != 0.f) ? v + a.beta * *addend(a, dst, row, col) : v;
          }
        }
      }
  }
}

// C = alpha * sum_{s<S} P[s] + beta * D (D = C when null), the split partials
// summed in order.  P is [S][M][N] dense; four columns per thread when the
// rows allow it.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void splitk_reduce(const float* __restrict__ P, float* C,
                                                          int64_t M, int64_t N, int64_t ldc,
                                                          int S, float alpha, float beta,
                                                          const int64_t* dyn, int64_t dyn_base,
                                                          const float* D, int64_t ldd) {
  const int64_t per = VEC ? 4 : 1;
  const int64_t cols = N / per;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= M * cols) return;
  const int64_t m = i / cols, n = (i % cols) * per;
  // Rows past the device-side count are not needed, except up to its 16-row
  // group: a later dyn_dim 1 product reads K rounded up to 16, and those rows
  // (products of zero-filled operand rows) must hold their zeros, as the
  // unsplit tiles store them.
  if (dyn && m >= min((max(*dyn - dyn_base, int64_t{0}) + 15) / 16 * 16, M)) return;
  const int64_t plane = M * N;
  if (VEC) {
    f32x4 s = *reinterpret_cast<const f32x4*>(P + m * N + n);
    for (int k = 1; k < S; ++k) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(P + k * plane + m * N + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] += t[e];
    }
    f32x4* dst = reinterpret_cast<f32x4*>(C + m * ldc + n);
    const f32x4* src = D ? reinterpret_cast<const f32x4*>(D + m * ldd + n) : dst;
    f32x4 out;
    const f32x4 old = beta != 0.f ? *src : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = beta != 0.f ? alpha * s[e] + beta * old[e] : alpha * s[e];
    *dst = out;
  } else {
    float s = P[m * N + n];
    for (int k = 1; k < S; ++k) s += P[k * plane + m * N + n];
    float* dst = C + m * ldc + n;
    const float* src = D ? D + m * ldd + n : dst;
    *dst = beta != 0.f ? alpha * s + beta * *src : alpha * s;
  }
}

// Skinny NT product for M <= 8 rows (decode: one token per sequence):
// C[M,N] = alpha * A[M,K] B[N,K]^T + beta * C.  The MFMA tiles would run
// 1/128 full and only N/128 workgroups wide; this kernel is bound by streaming
// B from HBM (4*N*K bytes) instead.  A workgroup owns kSkinnyRows consecutive
// rows of B; its 4 waves take one K quarter each, every lane streams float4s of
// those rows (1 KB per row per wave load) and dots them with the M rows of A
// (a few KB, served by L1/L2).  Partial sums are reduced across the wave by
// shuffles and across the 4 waves through LDS in wave order.
constexpr int kSkinnyRows = 4;
constexpr int kSkinnyMaxM = 8;

template <int MR>
__global__ __launch_bounds__(kThreads) void gemm_skinny_nt(const float* __restrict__ A,
                                                           int64_t lda,
                                                           const float* __restrict__ B,
                                                           int64_t ldb, float* C, int64_t ldc,
                                                           int M, int64_t N, int64_t K,
                                                           float alpha, float beta,
                                                           const float* D, int64_t ldd) {
  constexpr int NR = kSkinnyRows;
  __shared__ float red[kThreads / kWave][NR * MR];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NR;
  const int64_t K4 = K / 4;
  const int64_t quarter = (K4 + 3) / 4;
  const int64_t kb = w * quarter;
  const int64_t ke = kb + quarter < K4 ? kb + quarter : K4;
  const f32x4* brow[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t n = n0 + r < N ? n0 + r : N - 1;  // rows past N re-read the last one
    brow[r] = reinterpret_cast<const f32x4*>(B + n * ldb);
  }
  float acc[NR][MR];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;

  for (int64_t i = kb + lane; i < ke; i += 2 * kWave) {
    const int64_t i1 = i + kWave;
    const bool two = i1 < ke;
    f32x4 b0[NR], b1[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      b0[r] = brow[r][i];
      b1[r] = two ? brow[r][i1] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const f32x4* arow = reinterpret_cast<const f32x4*>(A + m * lda);
        const f32x4 x0 = arow[i];
        const f32x4 x1 = two ? arow[i1] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          acc[r][m] += b0[r].x * x0.x + b0[r].y * x0.y + b0[r].z * x0.z + b0[r].w * x0.w;
          acc[r][m] += b1[r].x * x1.x + b1[r].y * x1.y + b1[r].z * x1.z + b1[r].w * x1.w;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const float s = wave_sum(acc[r][m]);
        if (lane == 0) red[w][r * MR + m] = s;
      }
    }
  __syncthreads();
  const int idx = threadIdx.x;
  if (idx < NR * MR) {
    const int r = idx / MR, m = idx % MR;
    const int64_t n = n0 + r;
    if (m < M && n < N) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < kThreads / kWave; ++q) s += red[q][idx];
      float* c = C + m * ldc + n;
      const float* src = D ? D + m * ldd + n : c;
      *c = beta != 0.f ? alpha * s + beta * *src : alpha * s;
    }
  }
}

template <int MR>
int launch_skinny(const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                  int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                  const float* D, int64_t ldd, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>((N + kSkinnyRows - 1) / kSkinnyRows);
  gemm_skinny_nt<MR><<<grid, kThreads, 0, st>>>(A, lda, B, ldb, C, ldc, static_cast<int>(M), N,
                                                 K, alpha, beta, D, ldd);
  return launch_status();
}

// Launch plan for one call.
struct Plan {
  bool big;         // 256x128 tiles (else 128x128)
  int64_t splits;   // 1 = no K split
  int64_t kchunk;   // k per split (multiple of kBK)
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

Plan make_plan(int64_t M, int64_t N, int64_t K, int64_t batch) {
  Plan p{false, 1, 0};
  const int64_t big_tiles = cdiv(M, 256) * cdiv(N, 128) * batch;
  if (big_tiles >= 4 * kCUs) {  // at least two full waves of 2 blocks per CU
    p.big = true;
    return p;
  }
  const int64_t tiles = cdiv(M, 128) * cdiv(N, 128) * batch;
  const int64_t target = 6 * kCUs;  // two waves of 3 blocks per CU
  // K chunks of at least 1024 from K = 4096 up.  A grid that would fill at
  // most half the CUs (e.g. the projections of a short prefill, M = 128) is
  // latency-bound on its one pass over K: chunks of at least 256 from K = 512.
  const bool few = 2 * tiles <= kCUs;
  const int64_t min_chunk = few ? 256 : 1024;
  // A K split on 256x128 tiles, in chunks of at least 1024, when a whole
  // number of waves of them (two per CU) is at least two waves: 2-4% faster
  // than the 128x128 split on the weight-gradient shapes that allows (e.g.
  // 1024x2048, 2048x2048 and 6144x2048 over 32768 tokens), which a partial
  // last wave made up to 8% slower.
  if (batch == 1 && K >= 4096) {
    int64_t s = cdiv(4 * kCUs, big_tiles);
    while (s < 16 && (big_tiles * s) % (2 * kCUs) != 0) ++s;
    if (s >= 2 && s <= K / 1024 && (big_tiles * s) % (2 * kCUs) == 0) {
      p.big = true;
      p.kchunk = cdiv(cdiv(K, s), kBK) * kBK;
      p.splits = cdiv(K, p.kchunk);
      return p;
    }
  }
  if (batch == 1 && tiles < target && K >= (few ? 2 * min_chunk : 4096)) {
    int64_t s = std::min<int64_t>(16, cdiv(target, tiles));
    s = std::min<int64_t>(s, K / min_chunk);
    if (s >= 2) {
      p.kchunk = cdiv(cdiv(K, s), kBK) * kBK;
      p.splits = cdiv(K, p.kchunk);
    }
  }
  return p;
}

template <bool A_KC, bool B_KC, int BM, int BN, int OCC>
int launch(const GemmArgs& a, int64_t ny, bool vec, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(a.tiles_m) * a.tiles_n, static_cast<unsigned>(ny));
  if (vec)
    gemm_f32_mfma<A_KC, B_KC, true, BM, BN, OCC><<<grid, kThreads, 0, st>>>(a);
  else
    gemm_f32_mfma<A_KC, B_KC, false, BM, BN, OCC><<<grid, kThreads, 0, st>>>(a);
  return launch_status();
}

template <int BM, int BN, int OCC>
int launch_t(GemmArgs a, bool a_kc, bool b_kc, int64_t ny, bool vec, hipStream_t st) {
  a.tiles_m = static_cast<int>(cdiv(a.M, BM));
  a.tiles_n = static_cast<int>(cdiv(a.N, BN));
  if (a_kc && b_kc) return launch<true, true, BM, BN, OCC>(a, ny, vec, st);
  if (a_kc && !b_kc) return launch<true, false, BM, BN, OCC>(a, ny, vec, st);
  if (!a_kc && !b_kc) return launch<false, false, BM, BN, OCC>(a, ny, vec, st);
  return launch<false, true, BM, BN, OCC>(a, ny, vec, st);
}

template <bool A_KC, bool B_KC, int BM, int BN, int OCC>
int launch_dma_t(GemmArgs a, int64_t ny, hipStream_t st) {
  a.tiles_m = static_cast<int>(cdiv(a.M, BM));
  a.tiles_n = static_cast<int>(cdiv(a.N, BN));
  dim3 grid(static_cast<unsigned>(a.tiles_m) * a.tiles_n, static_cast<unsigned>(ny));
  // Largest byte offset a block's buffer resource must reach: BM (BN) rows of
  // K plus K, or K rows of lda (ldb) plus the tile's columns.
  const int64_t span_a = A_KC ? BM * a.lda + a.K : a.K * a.lda + BM;
  const int64_t span_b = B_KC ? BN * a.ldb + a.K : a.K * a.ldb + BN;
  const int64_t span_c = BM * std::max(a.ldc, a.D ? a.ldd : int64_t{0});  // the epilogue's rows
  if (4 * std::max({span_a, span_b, span_c}) < (int64_t{1} << 31) - 256)
    gemm_f32_dma<A_KC, B_KC, BM, BN, OCC, true><<<grid, kThreads, 0, st>>>(a);
  else
    gemm_f32_dma<A_KC, B_KC, BM, BN, OCC, false><<<grid, kThreads, 0, st>>>(a);
  return launch_status();
}

template <int BM, int BN, int OCC>
int launch_dma(const GemmArgs& a, bool a_kc, bool b_kc, int64_t ny, hipStream_t st) {
  if (a_kc && b_kc) return launch_dma_t<true, true, BM, BN, OCC>(a, ny, st);
  if (a_kc && !b_kc) return launch_dma_t<true, false, BM, BN, OCC>(a, ny, st);
  if (!a_kc && !b_kc) return launch_dma_t<false, false, BM, BN, OCC>(a, ny, st);
  return launch_dma_t<false, true, BM, BN, OCC>(a, ny, st);
}

int check_args(int transa, int transb, int64_t M, int64_t N, int64_t K, const float* A,
               int64_t lda, const float* B, int64_t ldb, const float* C, int64_t ldc,
               int64_t batch) {
  if (M < 0 || N < 0 || K < 0 || batch < 1) return EMBER_EINVAL;
  if (M == 0 || N == 0) return EMBER_OK;
  if (!C || (K > 0 && (!A || !B))) return EMBER_EINVAL;
  if (lda < (transa ? M : K) || ldb < (transb ? K : N) || ldc < N) return EMBER_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > 0x7fffffff || batch > 65535) return EMBER_EINVAL;
  return EMBER_OK;
}

}  // namespace

extern "C" size_t ember_gemm_f32_workspace_bytes(int64_t M, int64_t N, int64_t K,
                                                 int64_t batch) {
  if (M <= 0 || N <= 0 || K <= 0 || batch < 1) return 0;
  const Plan p = make_plan(M, N, K, batch);
  return p.splits > 1 ? static_cast<size_t>(p.splits * M * N) * sizeof(float) : 0;
}

namespace {

// One GEMM call; `dyn` (may be null) is the device-side extent of GemmArgs.
int gemm_run(int transa, int transb, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb, int64_t sB,
             float beta, float* C, int64_t ldc, int64_t sC, int64_t batch, void* workspace,
             size_t workspace_bytes, const int64_t* dyn, int64_t dyn_base, int dyn_dim,
             const float* D, int64_t ldd, hipStream_t st) {
  int rc = EMBER_OK;
  GemmArgs a{A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, 0, alpha, beta, 0, 0};
  a.dyn = dyn;
  a.dyn_base = dyn_base;
  a.dyn_dim = dyn_dim;
  a.D = D;
  a.ldd = ldd;
  const bool vec = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                   (batch == 1 || (sA % 4 == 0 && sB % 4 == 0));
  const bool a_kc = !transa, b_kc = transb != 0;
  if (!dyn && batch == 1 && M <= kSkinnyMaxM && a_kc && b_kc && vec && K > 0 && K % 4 == 0 &&
      N <= int64_t{kSkinnyRows} * 0x7fffffff) {
    auto skinny = M == 1 ? launch_skinny<1>
                  : M == 2 ? launch_skinny<2>
                  : M <= 4 ? launch_skinny<4>
                           : launch_skinny<8>;
    return skinny(A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, D, ldd, st);
  }
  Plan p = make_plan(M, N, K, batch);
  if (p.splits > 1 &&
      ((dyn && dyn_dim == 1) || !workspace ||
       workspace_bytes < static_cast<size_t>(p.splits * M * N) * sizeof(float)))
    p.splits = 1;  // no room for partials, or K itself is decided on the device
  if (p.splits > 1) {
    // Split s computes A[:, s*kchunk ...] B[s*kchunk ..., :] into plane s.
    GemmArgs sp = a;
    sp.C = static_cast<float*>(workspace);
    sp.ldc = N;
    sp.sA = a_kc ? p.kchunk : p.kchunk * lda;
    sp.sB = b_kc ? p.kchunk : p.kchunk * ldb;
    sp.sC = M * N;
    sp.kchunk = p.kchunk;
    sp.alpha = 1.f;
    sp.beta = 0.f;
    const bool dma = vec && p.kchunk % 16 == 0 && K % 16 == 0 && (a_kc || M % 4 == 0) &&
                     (b_kc || N % 4 == 0);
    if ((rc = dma ? (p.big ? launch_dma<256, 128, 2>(sp, a_kc, b_kc, p.splits, st)
                           : launch_dma<128, 128, 3>(sp, a_kc, b_kc, p.splits, st))
                  : launch_t<128, 128, 3>(sp, a_kc, b_kc, p.splits, vec, st)))
      return rc;
    const bool rvec = (N % 4 == 0) && (ldc % 4 == 0) && aligned16(C) &&
                      (!D || (ldd % 4 == 0 && aligned16(D)));
    const int64_t items = M * (rvec ? N / 4 : N);
    const unsigned blocks = static_cast<unsigned>(cdiv(items, kThreads));
    const int64_t* rdyn = dyn_dim == 0 ? dyn : nullptr;
    if (rvec)
      splitk_reduce<true><<<blocks, kThreads, 0, st>>>(static_cast<const float*>(workspace), C, M,
                                                       N, ldc, static_cast<int>(p.splits),
                                                       alpha, beta, rdyn, dyn_base, D, ldd);
    else
      splitk_reduce<false><<<blocks, kThreads, 0, st>>>(static_cast<const float*>(workspace), C,
                                                        M, N, ldc, static_cast<int>(p.splits),
                                                        alpha, beta, rdyn, dyn_base, D, ldd);
    return launch_status();
  }
  const bool dma = vec && K % 16 == 0 && (a_kc || M % 4 == 0) && (b_kc || N % 4 == 0) &&
                   (batch == 1 || (sA % 4 == 0 && sB % 4 == 0));
  if (dma && p.big) return launch_dma<256, 128, 2>(a, a_kc, b_kc, batch, st);
  if (dma) return launch_dma<128, 128, 3>(a, a_kc, b_kc, batch, st);
  if (dyn) return EMBER_EINVAL;  // only the LDS-DMA kernels read a device-side extent
  if (p.big) return launch_t<256, 128, 2>(a, a_kc, b_kc, batch, vec, st);
  return launch_t<128, 128, 3>(a, a_kc, b_kc, batch, vec, st);
}

}  // namespace

extern "C" int ember_gemm_f32_ws(int transa, int transb, int64_t M, int64_t N, int64_t K,
                                 float alpha, const float* A, int64_t lda, int64_t sA,
                                 const float* B, int64_t ldb, int64_t sB, float beta, float* C,
                                 int64_t ldc, int64_t sC, int64_t batch, void* workspace,
                                 size_t workspace_bytes, ember_stream_t s) {
  int rc = check_args(transa, transb, M, N, K, A, lda, B, ldb, C, ldc, batch);
  if (rc || M == 0 || N == 0) return rc;
  return gemm_run(transa, transb, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, batch,
                  workspace, workspace_bytes, nullptr, 0, 0, nullptr, 0, as_stream(s));
}

extern "C" int ember_gemm_f32_add(int transa, int transb, int64_t M, int64_t N, int64_t K,
                                  float alpha, const float* A, int64_t lda, const float* B,
                                  int64_t ldb, const float* D, int64_t ldd, float* C, int64_t ldc,
                                  void* workspace, size_t workspace_bytes, ember_stream_t s) {
  int rc = check_args(transa, transb, M, N, K, A, lda, B, ldb, C, ldc, 1);
  if (rc || M == 0 || N == 0) return rc;
  if (!D || ldd < N) return EMBER_EINVAL;
  if (D != C) {  // D is C itself or lies wholly apart from it
    const auto c0 = reinterpret_cast<uintptr_t>(C), d0 = reinterpret_cast<uintptr_t>(D);
    const uintptr_t c1 = c0 + static_cast<uintptr_t>((M - 1) * ldc + N) * sizeof(float);
    const uintptr_t d1 = d0 + static_cast<uintptr_t>((M - 1) * ldd + N) * sizeof(float);
    if (d0 < c1 && c0 < d1) return EMBER_EINVAL;
  } else if (ldd != ldc) {
    return EMBER_EINVAL;
  }
  return gemm_run(transa, transb, M, N, K, alpha, A, lda, 0, B, ldb, 0, 1.0f, C, ldc, 0, 1,
                  workspace, workspace_bytes, nullptr, 0, 0, D, ldd, as_stream(s));
}

extern "C" int ember_gemm_f32_dyn(int transa, int transb, int64_t M, int64_t N, int64_t K,
                                  float alpha, const float* A, int64_t lda, const float* B,
                                  int64_t ldb, float beta, float* C, int64_t ldc,
                                  const int64_t* count, int64_t base, int dim, void* workspace,
                                  size_t workspace_bytes, ember_stream_t s) {
  int rc = check_args(transa, transb, M, N, K, A, lda, B, ldb, C, ldc, 1);
  if (rc) return rc;
  if (!count || (dim != 0 && dim != 1) || base < 0) return EMBER_EINVAL;
  // The LDS-DMA kernels' conditions: 16-byte rows and K in whole 16-k stages.
  const bool a_kc = !transa, b_kc = transb != 0;
  if (!aligned16(A) || !aligned16(B) || lda % 4 != 0 || ldb % 4 != 0 || K % 16 != 0 ||
      (!a_kc && M % 4 != 0) || (!b_kc && N % 4 != 0))
    return EMBER_EINVAL;
  if (M == 0 || N == 0) return EMBER_OK;
  return gemm_run(transa, transb, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1,
                  workspace, workspace_bytes, count, base, dim, nullptr, 0, as_stream(s));
}

extern "C" int ember_gemm_f32(int transa, int transb, int64_t M, int64_t N, int64_t K,
                              float alpha, const float* A, int64_t lda, int64_t sA,
                              const float* B, int64_t ldb, int64_t sB, float beta, float* C,
                              int64_t ldc, int64_t sC, int64_t batch, ember_stream_t s) {
  return ember_gemm_f32_ws(transa, transb, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc,
                           sC, batch, nullptr, 0, s);
}
