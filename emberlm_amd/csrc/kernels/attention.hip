// Fused causal GQA attention, forward and backward, on fp32 MFMA.
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
// The forward, dK/dV and recompute-dQ kernels run on v_mfma_f32_16x16x4_f32
// tiles (wave64; the dQ-from-dS kernel is a GEMM, described there): lane
// (g = lane/16, i = lane%16) holds A[m=i][k=g] and B[k=g][n=i]; accumulator
// register e holds C[m = 4*g + e][n = i].  A wave owns 16 rows (queries or
// keys), so its register-resident rows and accumulators take half of what 32
// rows on 32x32x2 tiles would, and at D = 128 two to four waves share a SIMD:
// one wave's softmax section and barrier waits run under another's MFMAs.
//
// Forward, per wave of 16 queries: S^T = K Q^T puts the query index in the
// lane (n = i), and the probabilities come out exactly in the B-operand layout
// of O^T += V^T P^T.  Q stays in registers (pre-multiplied by scale*log2(e)).
// K/V tiles of 32 keys are double-buffered in LDS: the global loads of tile
// i+1 are issued into registers before the MFMAs of tile i and written to the
// other buffer after them, so one barrier per tile remains and load latency
// is hidden.
//
// Backward (no atomics, so dK/dV/dQ are bitwise reproducible):
//   attn_delta:  delta = rowsum(dO * O);
//   attn_bwd_dkdv: per 16 keys, S = Q K^T and dP = dO V^T put the key in the
//                lane, so dV^T += dO^T P and dK^T += Q^T dS accumulate in
//                registers across every query tile and every query head of
//                the KV head's group, in a fixed order.  With a dS buffer it
//                also stores dS (fp32, the causal part only, see below);
//   attn_bwd_dq_gemm: dQ = dS K from the stored dS, a plain product in key
//                order on the GEMM kernel's 256 x D tiles;
//   attn_bwd_dq (no dS buffer): per 16 queries, S^T = K Q^T and dP^T =
//                V dO^T recomputed, then dQ^T += K^T dS^T.
// Counted in units of one T x T x D product per head, the algorithm needs 4
// (dV, dP, dQ, dK); with the stored dS the kernels execute 5 (S is computed
// again), with the recompute dQ kernel 7 (S and dP twice).
// dS layout, per (b, h) row: for each 64-key block kb a strip of 64 key rows
// by Lr = T32 - 64 kb query columns (T32 = T rounded up to 32), columns
// starting at query 64 kb, so only the causal part is kept; strips follow
// each other in kb order (ds_strip_offset).  The dK/dV kernel writes one
// float4 of four consecutive queries per lane; entries it skips (query tiles
// no key of a wave sees) are read, but zeroed with every other query < key
// entry, by the dQ kernel.  The table at the end of the workspace gives each
// (batch, KV head) row's dS region; the regions of one chunk of rows may lie
// in separate buffers (ember_attn_bwd_scattered).
// The dK/dV and recompute-dQ kernels take 64 rows per workgroup (two waves
// per SIMD at D = 128; 32 rows per wave on 32x32x2 tiles needed more than 256
// registers per lane there) and double-buffer their streamed tiles the same
// way.
#include <type_traits>
#include <vector>

#include "common.h"
#include "mfma_sched.h"

using namespace ember;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kThreads = 256;

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Accumulators over d with permuted row slots: tile 4hq + c, row slot
// x = 4g + e holds d = 64hq + 4x + c (so that one b128 LDS read of d = 64hq +
// 4i .. +3 is the A operand of four tiles).  Writes lane (g, i)'s values of
// one row (query or key i) as float4s at d = 64hq + 16g + 4e, times mul.
template <int NT>
__device__ __forceinline__ void store_d_row(f32x4* row, const f32x4 (&acc)[NT], int g,
                                            float mul) {
#pragma unroll
  for (int hq = 0; hq < NT / 4; ++hq)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      row[16 * hq + 4 * g + e] =
          f32x4{acc[4 * hq][e], acc[4 * hq + 1][e], acc[4 * hq + 2][e], acc[4 * hq + 3][e]} *
          mul;
}

// 2^x on the transcendental unit (inputs here are <= 0 or -inf).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Block order.  Every attention kernel runs a 1-D grid of (tile, row) work
// items, row = (b, head).  Blocks are dispatched in index order and dealt
// round-robin over the 8 XCDs (block i runs on XCD i % 8), so the index puts
// the heaviest tiles first (the causal triangle makes tile cost vary 32x) and
// gives every XCD the same mix of tiles; when the row count is a multiple of 8
// the rows are regrouped so that each XCD owns a contiguous range of (b, head)
// rows and the K/V of a GQA group stays in one L2.
struct WorkItem {
  int tile, row;
};
__device__ __forceinline__ WorkItem work_item(int ntiles) {
  const int L = static_cast<int>(blockIdx.x);
  const int rows = static_cast<int>(gridDim.x) / ntiles;
  int rr = L % rows;
  if (rows % 8 == 0) rr = (rr % 8) * (rows / 8) + rr / 8;
  return {L / rows, rr};
}

// dS strips of one (b, h) row (layout in the header comment).
__host__ __device__ __forceinline__ int64_t ds_t32(int64_t T) { return (T + 31) / 32 * 32; }
__host__ __device__ __forceinline__ int64_t ds_strip_offset(int64_t kb, int64_t T32) {
  return 64 * kb * T32 - 2048 * kb * (kb - 1);
}
__host__ __device__ __forceinline__ int64_t ds_row_floats(int64_t T) {
  return ds_strip_offset((T + 63) / 64, ds_t32(T));
}

// ROWS rows of D floats staged global -> registers -> LDS by a block of
// THREADS.  All loads of a tile are issued before the first wait; rows at or
// beyond `valid` are zero.
template <int D, int ROWS, int THREADS = kThreads>
struct RowTile {
  static constexpr int kChunks = ROWS * D / 4;
  static constexpr int kPer = kChunks / THREADS;
  static_assert(kChunks % THREADS == 0, "tile does not split evenly over the block");
  f32x4 r[kPer];

  __device__ __forceinline__ void load(const float* __restrict__ src, int64_t gstride, int valid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * THREADS;
      const int row = c / (D / 4), c4 = c % (D / 4);
      r[i] = row < valid ? reinterpret_cast<const f32x4*>(src + row * gstride)[c4]
                         : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ lds, int ls) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * THREADS;
      const int row = c / (D / 4), c4 = c % (D / 4);
      *reinterpret_cast<f32x4*>(lds + row * ls + 4 * c4) = r[i];
    }
  }
};

// ROWS rows of D floats copied global -> LDS by global_load_lds_dwordx4 (no
// registers, no LDS store instructions) by WAVES waves.  One wave
// instruction fills a 1 KB block with 1024 / (4 D) rows; row r sits in block
// r % kBlocks at (r / kBlocks) * D, and blocks are padded to 260 floats, so the
// b128 reads of 16 consecutive rows at one column (the K fragments) and of
// one row at 16 consecutive columns (V) both hit 16 distinct bank groups.
template <int D, int ROWS, int WAVES>
struct DmaTile {
  static constexpr int kChunks = D / 4;              // 16-byte chunks per row
  static constexpr int kRpi = 64 / kChunks;          // rows per block
  static constexpr int kBlocks = ROWS / kRpi;
  static constexpr int kBlockStride = 256 + 4;       // floats
  static constexpr int kFloats = kBlocks * kBlockStride;
  static constexpr int kInsts = kBlocks / WAVES;     // per wave
  static_assert(kRpi * kChunks == 64 && ROWS % kRpi == 0, "rows do not fill 1 KB blocks");
  static_assert(kBlocks % WAVES == 0, "tile does not split evenly over the waves");
  __device__ __forceinline__ static int at(int row, int col) {
    return (row % kBlocks) * kBlockStride + (row / kBlocks) * D + col;
  }
  // Rows [0, ROWS) of src (row stride gstride floats) into lds; rows at or
  // past valid (>= 1) read row valid - 1 again, whose products are masked.
  // buffer_load_dwordx4 ... lds through a buffer resource based at src, with
  // a 32-bit byte offset per lane (under ROWS * gstride * 4 bytes).
  __device__ __forceinline__ static void issue(float* lds, const float* src, int64_t gstride,
                                               int valid, int w, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the kernel's launch stub
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), 0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int q = 0; q < kInsts; ++q) {
      const int blk = w + WAVES * q;
      const int row = blk + kBlocks * (lane / kChunks);
      const int srow = min(row, valid - 1);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(lds + kBlockStride * blk), 16,
          static_cast<int>((srow * gstride + 4 * (lane % kChunks)) * 4), 0, 0, 0);
    }
#endif
  }
};

// One dword per lane copied global -> LDS by DMA: lane l's word lands at
// lds[l].
__device__ __forceinline__ void dma_dword(float* lds, const float* src) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the kernel's launch stub
  __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0);
#endif
}

// s_waitcnt vmcnt(0) lgkmcnt(0).
__device__ __forceinline__ void wait_all_mem() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (0 << 8));
}

// Max and sum over lanes i, i + 16, i + 32, i + 48 of a wave, the four
// 16-lane rows' values exchanged in registers: v_permlane16_swap trades rows
// 1 and 3 of its first operand for rows 0 and 2 of its second, so with x in
// both each lane holds x of rows {0, 1} or {2, 3}; v_permlane32_swap trades
// the upper 32 lanes of the first for the lower 32 of the second.  max and +
// of two operands are commutative, so every lane gets the same bits.
__device__ __forceinline__ float pair_rows16(float x, bool sum) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return sum ? a + b : fmaxf(a, b);
}
__device__ __forceinline__ float pair_rows32(float x, bool sum) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return sum ? a + b : fmaxf(a, b);
}
__device__ __forceinline__ float max_over_rows(float x) {
  return pair_rows32(pair_rows16(x, false), false);
}
__device__ __forceinline__ float sum_over_rows(float x) {
  return pair_rows32(pair_rows16(x, true), true);
}

// ------------------------------------------------------------------ forward
// Forward.  A wave owns 16 queries and a workgroup of eight waves 128, so
// every K/V tile in LDS serves 128 queries, and at 100 registers per lane
// (D = 128) four waves fit on a SIMD (32 queries per wave on 32x32x2 tiles
// took 239 and two waves: 1.14x slower at B=8, T=4096, H=16, Hk=8).  K and V
// tiles are copied global -> LDS by DMA into two buffers, the next tile's
// copy in flight during this one's MFMAs.  Per 32-key tile (halves kt of 16
// keys):
//   S^T = K Q^T (m = key, n = query): MFMA step 4t+j contracts over
//   d = 16t + 4g + j, each K fragment one b128 LDS read, Q in registers;
//   register e of s[kt] in lane (g, i) is the score of key 16kt + 4g + e for
//   query i: a query's running max is reduced over its four lanes (g), and
//   its running sum is kept per lane and added up at the end;
//   O^T += V^T P^T (m = d, n = query, contraction over the 4 keys
//   {16kt + 4g + e : g}): P is the B operand straight from s[kt]; the A
//   operand of tile 4hq + c, row slot x, is d = 64hq + 4x + c, so one b128
//   LDS read of V (d = 64hq + 4i .. +3) feeds the four tiles 4hq .. 4hq + 3.
//   Each element of O sums the same products in the same order as with
//   d = 16t + x; only its register moves.
template <int D>
struct FwdCfg {
  static constexpr int kThreads = 512, kBQ = 128, kBK = 32;
  using Tile = DmaTile<D, kBK, kThreads / 64>;
  static constexpr int kTile = Tile::kFloats;
  static constexpr int kBuf = 2 * kTile;  // one K+V stage
  static constexpr int kSmem = 2 * kBuf;
};

// SS: also store every computed score (log2 units, before the mask) in the
// dS layout of the KV row's region given by `s_rows` (attn_bwd_from_scores
// reads them back instead of computing S again).
template <int D, bool SS>
__global__ __launch_bounds__(FwdCfg<D>::kThreads, 2) void attn_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ lse, float* const* __restrict__ s_rows, int T,
    int H, int Hk, float scale_log2) {
  using C = FwdCfg<D>;
  constexpr int NT = D / 16;
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];

  const int nqb = (T + C::kBQ - 1) / C::kBQ;
  const WorkItem wi = work_item(nqb);
  const int qb = nqb - 1 - wi.tile;  // longest rows first
  const int h = wi.row % H, b = wi.row / H;
  const int hk = h / (H / Hk);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, i = lane & 15;
  const int q0 = qb * C::kBQ, qw0 = q0 + 16 * w, myq = qw0 + i;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const int64_t qoff = static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
  const float* kbase = k + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const float* vbase = v + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const int64_t T32 = ds_t32(T);
  gfloat* sregion = nullptr;  // this (b, h) row's strips
  if constexpr (SS)
    sregion = as_global(s_rows[b * Hk + hk]) + static_cast<int64_t>(h - hk * (H / Hk)) *
                                                   ds_row_floats(T);

  f32x4 qreg[NT];
  if (myq < T) {
    const f32x4* qr = reinterpret_cast<const f32x4*>(q + qoff + myq * qs);
#pragma unroll
    for (int t = 0; t < NT; ++t) qreg[t] = qr[4 * t + g] * scale_log2;
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) qreg[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const int kend = min(T, q0 + C::kBQ);
  const int nkb = (kend + C::kBK - 1) / C::kBK;
  using Tile = typename C::Tile;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int qw0u = q0 + 16 * wu;  // qw0, known wave-uniform
  Tile::issue(smem, kbase, ks, T, wu, lane);
  Tile::issue(smem + C::kTile, vbase, ks, T, wu, lane);
  wait_all_mem();
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * C::kBK;
    const bool more = kb + 1 < nkb;
    if (more) {  // the next K/V tile lands in the other buffer during this one
      float* nb = smem + ((kb + 1) & 1) * C::kBuf;
      const int64_t off = static_cast<int64_t>(k0 + C::kBK) * ks;
      Tile::issue(nb, kbase + off, ks, T - k0 - C::kBK, wu, lane);
      Tile::issue(nb + C::kTile, vbase + off, ks, T - k0 - C::kBK, wu, lane);
    }
    const float* Ks = smem + (kb & 1) * C::kBuf;
    const float* Vs = Ks + C::kTile;
    if (k0 <= qw0 + 15) {  // some key of the tile is seen by some query of this wave
      f32x4 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      // K fragments one d tile ahead: the reads of tile t + 1 are in flight
      // while the MFMAs of tile t run.
      f32x4 kf[2][2];
      auto read_k = [&](int t, f32x4 (&dst)[2]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          dst[kt] = *reinterpret_cast<const f32x4*>(Ks + Tile::at(16 * kt + i, 16 * t + 4 * g));
      };
      read_k(0, kf[0]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t + 1 < NT) read_k(t + 1, kf[(t + 1) & 1]);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j) s[kt] = mfma16(kf[t & 1][kt][j], qreg[t][j], s[kt]);
      }
      // Order: tile 0's reads, then per tile two MFMAs, a read of the next
      // tile, two MFMAs, the other read, four MFMAs (the wait for a tile's
      // reads comes before the next tile's are issued).
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int t = 0; t + 1 < NT; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      if constexpr (SS) {
        // The tile's 32 keys lie in one 64-key strip; this lane's query is at
        // or past the strip's first key whenever the tile is processed.
        if (myq < T) {
          const int sb = k0 >> 6;
          const int64_t lr = T32 - 64 * sb;
          gfloat* col = sregion + ds_strip_offset(sb, T32) + (myq - 64 * sb) +
                        static_cast<int64_t>(k0 - 64 * sb + 4 * g) * lr;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) col[(16 * kt + e) * lr] = s[kt][e];
        }
      }
      // Keys past min(myq, T - 1) are masked, on the tiles that reach them (a
      // wave-uniform test, so the other tiles skip it on a scalar branch).
      if (k0 + C::kBK - 1 > qw0u || k0 + C::kBK > T) {
        const int klim = min(myq, T - 1) - k0 - 4 * g;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) s[kt][e] = 16 * kt + e > klim ? -INFINITY : s[kt][e];
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, s[kt][e]);
      tmax = max_over_rows(tmax);
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = fast_exp2(m_run - m_new);
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = fast_exp2(s[kt][e] - m_new);
          s[kt][e] = pv;
          psum += pv;
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
      if (__any(alpha != 1.0f)) {  // the running max moved for some query of the wave
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] *= alpha;
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * kt + 4 * g + e;
#pragma unroll
          for (int hq = 0; hq < NT / 4; ++hq) {
            const f32x4 vv = *reinterpret_cast<const f32x4*>(Vs + Tile::at(row, 64 * hq + 4 * i));
#pragma unroll
            for (int c = 0; c < 4; ++c)
              acc[4 * hq + c] = mfma16(vv[c], s[kt][e], acc[4 * hq + c]);
          }
        }
    }
    wait_all_mem();  // this wave's DMA of the next tile has landed
    __syncthreads();
  }

  const float l_tot = sum_over_rows(l_run);
  if (myq < T) {
    if (g == 0) lse[(static_cast<int64_t>(b) * H + h) * T + myq] = (m_run + log2f(l_tot)) * kLn2;
    store_d_row(reinterpret_cast<f32x4*>(o + qoff + myq * qs), acc, g, 1.0f / l_tot);
  }
}

// --------------------------------------------------------------- backward
// delta[b,h,t] = sum_d dO[b,t,h,d] * O[b,t,h,d]; LPR = D/4 lanes per row.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_delta_kernel(const float* __restrict__ o,
                                                              const float* __restrict__ dout,
                                                              float* __restrict__ delta,
                                                              int64_t rows, int T, int H) {
  constexpr int LPR = D / 4, RPB = kThreads / LPR;
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

// dQ on 16x16x4 MFMA tiles (lane l: A[l%16][l/16], B[l/16][l%16],
// accumulator e = C[4*(l/16) + e][l%16]).  A wave owns 16 queries, a
// workgroup 64.  Per 32-key tile (halves kt of 16 keys):
//   S^T = K Q^T and dP^T = V dO^T (m = key, n = query): MFMA step 4t+j
//   contracts over d = 16t + 4g + j, so each K / V fragment is one b128 LDS
//   read and the Q / dO rows sit in registers in the matching order;
//   dS^T comes out with the query in the lane and keys 16kt + 4g + e in the
//   registers, which is the B operand of dQ^T += K^T dS^T (m = d, contraction
//   over the 4 keys {16kt + 4g + e : g}); its A operand comes from b128 LDS
//   reads of K, one per four d tiles (the permuted row slots of store_d_row).
// The query's lse and delta are per-lane scalars.
template <int D>
struct DqCfg {
  static constexpr int kBQ = 64, kBK = 32, kKS = D + 4;
  static constexpr int kBuf = 2 * kBK * kKS;  // one K+V stage
  static constexpr int kSmem = 2 * kBuf;
};

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_bwd_dq_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dq, int T, int H, int Hk, float scale_log2, float scale) {
  using C = DqCfg<D>;
  constexpr int NT = D / 16;  // d tiles; float4 groups of a lane's Q/dO row
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];

  const int nqb = (T + C::kBQ - 1) / C::kBQ;
  const WorkItem wi = work_item(nqb);
  const int qb = nqb - 1 - wi.tile;  // longest rows first
  const int h = wi.row % H, b = wi.row / H;
  const int hk = h / (H / Hk);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, i = lane & 15;
  const int q0 = qb * C::kBQ, qw0 = q0 + 16 * w, myq = qw0 + i;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const int64_t qoff = static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
  const float* kbase = k + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const float* vbase = v + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;

  f32x4 qreg[NT], doreg[NT];
  if (myq < T) {
    const f32x4* qr = reinterpret_cast<const f32x4*>(q + qoff + myq * qs);
    const f32x4* dr = reinterpret_cast<const f32x4*>(dout + qoff + myq * qs);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      qreg[t] = qr[4 * t + g] * scale_log2;
      doreg[t] = dr[4 * t + g];
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) qreg[t] = doreg[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int64_t srow = (static_cast<int64_t>(b) * H + h) * T;
  const float lse2 = myq < T ? lse[srow + myq] * kLog2e : 0.f;
  const float dlt = myq < T ? delta[srow + myq] : 0.f;

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kend = min(T, q0 + C::kBQ);
  const int nkb = (kend + C::kBK - 1) / C::kBK;
  RowTile<D, C::kBK> tk, tv;
  tk.load(kbase, ks, T);
  tv.load(vbase, ks, T);
  tk.store(smem, C::kKS);
  tv.store(smem + C::kBK * C::kKS, C::kKS);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * C::kBK;
    const bool more = kb + 1 < nkb;
    if (more) {
      tk.load(kbase + static_cast<int64_t>(k0 + C::kBK) * ks, ks, T - k0 - C::kBK);
      tv.load(vbase + static_cast<int64_t>(k0 + C::kBK) * ks, ks, T - k0 - C::kBK);
    }
    const float* Ks = smem + (kb & 1) * C::kBuf;
    const float* Vs = Ks + C::kBK * C::kKS;
    if (k0 <= qw0 + 15) {  // some key of the tile is seen by some query of this wave
      f32x4 s[2], dp[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) s[kt] = dp[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const f32x4 kf =
              *reinterpret_cast<const f32x4*>(Ks + (16 * kt + i) * C::kKS + 16 * t + 4 * g);
          const f32x4 vf =
              *reinterpret_cast<const f32x4*>(Vs + (16 * kt + i) * C::kKS + 16 * t + 4 * g);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            s[kt] = mfma16(kf[j], qreg[t][j], s[kt]);
            dp[kt] = mfma16(vf[j], doreg[t][j], dp[kt]);
          }
        }
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + 16 * kt + 4 * g + e;
          const float p = (key > myq || key >= T) ? 0.f : fast_exp2(s[kt][e] - lse2);
          s[kt][e] = p * (dp[kt][e] - dlt);
        }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = (16 * kt + 4 * g + e) * C::kKS;
#pragma unroll
          for (int hq = 0; hq < NT / 4; ++hq) {
            const f32x4 kv = *reinterpret_cast<const f32x4*>(Ks + row + 64 * hq + 4 * i);
#pragma unroll
            for (int c = 0; c < 4; ++c)
              acc[4 * hq + c] = mfma16(kv[c], s[kt][e], acc[4 * hq + c]);
          }
        }
    }
    if (more) {
      float* nb = smem + ((kb + 1) & 1) * C::kBuf;
      tk.store(nb, C::kKS);
      tv.store(nb + C::kBK * C::kKS, C::kKS);
    }
    __syncthreads();
  }

  if (myq < T) store_d_row(reinterpret_cast<f32x4*>(dq + qoff + myq * qs), acc, g, scale);
}

// dK/dV on 16x16x4 MFMA tiles.  A wave owns 16 keys, a workgroup 64, so a
// wave holds half the accumulators and half the K/V registers that 32 keys
// on 32x32x2 tiles would need (those spill past 256 VGPRs into AGPRs at
// D = 128, one wave per SIMD): two waves fit on a SIMD, and one wave's
// softmax section and barrier waits run under the other's MFMAs.  The Q and
// dO tiles of a step (and its lse and delta) are copied global -> LDS by DMA
// into two buffers, the next step's copy in flight during this one.  Per
// 32-query tile:
//   S = Q K^T and dP = dO V^T (m = query, n = key): MFMA step 4t+j contracts
//   over d = 16t + 4g + j, so each Q / dO fragment is one b128 LDS read and
//   the K / V rows sit in registers in the matching order;
//   P and dS come out with the key in the lane (n = l%16) and queries
//   16mt + 4g + e in the registers, which is exactly the B operand of
//   dV^T += dO^T P and dK^T += Q^T dS (m = d, n = key, contraction over the
//   4 queries {16mt + 4g + e : g}); their A operand comes from b128 LDS
//   reads of dO and Q, one per four d tiles (the permuted row slots of
//   store_d_row).
template <int D>
struct DkvCfg {
  static constexpr int kBKeys = 64, kBQ = 32;
  using Tile = DmaTile<D, kBQ, kThreads / 64>;
  static constexpr int kTile = Tile::kFloats;
  static constexpr int kBuf = 2 * kTile + 2 * kBQ;  // Q, dO, lse, delta
  static constexpr int kSmem = 2 * kBuf;
};

// DS: store dS.  FS: the dS buffers hold the forward's scores (attn_fwd_kernel
// with SS), which are read back instead of computing S = Q K^T, and dS is
// written over them.
template <int D, bool DS, bool FS>
__global__ __launch_bounds__(kThreads, 2) void attn_bwd_dkdv_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dk, float* __restrict__ dv, float* const* __restrict__ ds_rows, int row0,
    int T, int H, int Hk, float scale_log2, float scale) {
  using C = DkvCfg<D>;
  constexpr int NT = D / 16;  // d tiles; float4 groups of a lane's K/V row
  static_assert(DS || !FS, "the scores live in the dS buffers");
  __shared__ __attribute__((aligned(16))) float smem[C::kSmem];

  const WorkItem wi = work_item((T + C::kBKeys - 1) / C::kBKeys);
  const int kb = wi.tile;  // small key blocks see the most queries: launched first
  const int kvrow = row0 + wi.row;  // (b, hk) of this launch's chunk of rows
  const int hk = kvrow % Hk, b = kvrow / Hk;
  const int group = H / Hk;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, i = lane & 15;
  const int key0 = kb * C::kBKeys, kw0 = key0 + 16 * w, mykey = kw0 + i;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const int64_t koff = static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;

  f32x4 kreg[NT], vreg[NT];  // kreg: unused with FS
  if (mykey < T) {
    const f32x4* kr = reinterpret_cast<const f32x4*>(k + koff + mykey * ks);
    const f32x4* vr = reinterpret_cast<const f32x4*>(v + koff + mykey * ks);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (!FS) kreg[t] = kr[4 * t + g] * scale_log2;
      vreg[t] = vr[4 * t + g];
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) kreg[t] = vreg[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x4 adk[NT], adv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) adk[t] = adv[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // This lane's row of the key block's dS strip for the group's first query
  // head (a KV row's region holds its group's heads one after another; the
  // table gives each KV row's region); columns count queries from key0.
  const int64_t T32 = ds_t32(T), ds_row = ds_row_floats(T), lr = T32 - key0;
  // (DS is a template argument so that the stores are unconditional, without a
  // branch around them, and can be kept ahead of each half's products.)
  gfloat* ds_lane = DS ? as_global(ds_rows[kvrow]) + ds_strip_offset(kb, T32) +
                             static_cast<int64_t>(16 * w + i) * lr + 4 * g
                       : nullptr;

  // The streamed sequence: for each query head of the group, the query tiles
  // key0, key0 + 32, ... below T.
  const int ntile = (T - key0 + C::kBQ - 1) / C::kBQ;
  const int nsteps = group * ntile;
  using Tile = typename C::Tile;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // Step `step`'s Q and dO tiles, lse and delta copied global -> LDS by DMA
  // into `buf`.  Query rows at or past T read row T - 1 again (their P is
  // selected to 0 below, and their dQ rows are not stored); wave 0 copies
  // lse (lanes 0-31) and delta (lanes 32-63) in one dword instruction.
  auto issue = [&](int step, float* buf) {
    const int hh = step / ntile, qt0 = key0 + (step % ntile) * C::kBQ;
    const int h = hk * group + hh;
    const int64_t qoff = static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D +
                         static_cast<int64_t>(qt0) * qs;
    Tile::issue(buf, q + qoff, qs, T - qt0, wu, lane);
    Tile::issue(buf + C::kTile, dout + qoff, qs, T - qt0, wu, lane);
    if (wu == 0) {
      const int64_t srow = (static_cast<int64_t>(b) * H + h) * T;
      const int t = min(qt0 + (lane & (C::kBQ - 1)), T - 1);
      dma_dword(buf + 2 * C::kTile, (lane < C::kBQ ? lse : delta) + srow + t);
    }
  };
  // FS: this lane's scores of a step (queries qt0 + 16mt + 4g + (0..3), the
  // addresses its dS goes to), loaded one step ahead.
  f32x4 snext[2];
  auto load_scores = [&](int st) {
    const gfloat* src = ds_lane + (st / ntile) * ds_row + (st % ntile) * C::kBQ;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) snext[mt] = *reinterpret_cast<const gf32x4*>(src + 16 * mt);
  };
  issue(0, smem);
  if constexpr (FS) load_scores(0);
  wait_all_mem();
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int qt0 = key0 + (step % ntile) * C::kBQ;
    const bool more = step + 1 < nsteps;
    f32x4 scur[2];
    if constexpr (FS) {
      scur[0] = snext[0];
      scur[1] = snext[1];
    }
    if (more) {  // the next step's tiles land in the other buffer during this one
      issue(step + 1, smem + ((step + 1) & 1) * C::kBuf);
      if constexpr (FS) load_scores(step + 1);
    }
    const float* Qs = smem + (step & 1) * C::kBuf;
    const float* Ds = Qs + C::kTile;
    const float* Ls = Qs + 2 * C::kTile;
    const float* Es = Ls + C::kBQ;
    if (qt0 + C::kBQ - 1 >= kw0) {  // some query of the tile sees some key of this wave
      // The two 16-query halves in sequence: S and dP of half 1 are issued
      // before the softmax of half 0 and the dV/dK products of half 0 before
      // the softmax of half 1, so each softmax runs under MFMAs of this wave.
      // Every accumulator sums in the same order as with the halves together.
      f32x4 s[2], dp[2];
      auto scores = [&](int mt) {
        s[mt] = dp[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (FS) s[mt] = scur[mt];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const f32x4 of =
              *reinterpret_cast<const f32x4*>(Ds + Tile::at(16 * mt + i, 16 * t + 4 * g));
          if constexpr (FS) {
#pragma unroll
            for (int j = 0; j < 4; ++j) dp[mt] = mfma16(of[j], vreg[t][j], dp[mt]);
          } else {
            const f32x4 qf =
                *reinterpret_cast<const f32x4*>(Qs + Tile::at(16 * mt + i, 16 * t + 4 * g));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              s[mt] = mfma16(qf[j], kreg[t][j], s[mt]);
              dp[mt] = mfma16(of[j], vreg[t][j], dp[mt]);
            }
          }
        }
      };
      auto softmax = [&](int mt) {
        // lse (scaled to log2 units here; the product is rounded on its own,
        // not fused into the subtraction) and delta of this lane's queries
        // 16mt + 4g + e, read as float4s (a read per entry, inside the mask
        // test, serialised the softmax section on LDS round trips).
#pragma clang fp contract(off)
        const f32x4 lq = *reinterpret_cast<const f32x4*>(Ls + 16 * mt + 4 * g) * kLog2e;
        const f32x4 eq = *reinterpret_cast<const f32x4*>(Es + 16 * mt + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int qq = qt0 + 16 * mt + 4 * g + e;
          // exp2 on every entry, then a select: no branch around the LDS data
          const float pe = fast_exp2(s[mt][e] - lq[e]);
          const float p = (qq < mykey || qq >= T) ? 0.f : pe;
          s[mt][e] = p;
          dp[mt][e] = p * (dp[mt][e] - eq[e]);
        }
        if constexpr (DS) {  // queries qt0 + 16mt + 4g + (0..3) of this lane's key
          *reinterpret_cast<gf32x4*>(ds_lane + (step / ntile) * ds_row + (qt0 - key0) +
                                     16 * mt) = dp[mt];
          // Keep the store ahead of this half's dV/dK products: the write of
          // the next tile to LDS waits for every outstanding vector memory
          // operation (loads and stores share the counter), so a store sunk
          // to the end of the step would be waited for in full.
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      auto grads = [&](int mt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * mt + 4 * g + e;
#pragma unroll
          for (int hq = 0; hq < NT / 4; ++hq) {
            const f32x4 ov = *reinterpret_cast<const f32x4*>(Ds + Tile::at(row, 64 * hq + 4 * i));
            const f32x4 qv = *reinterpret_cast<const f32x4*>(Qs + Tile::at(row, 64 * hq + 4 * i));
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              adv[4 * hq + c] = mfma16(ov[c], s[mt][e], adv[4 * hq + c]);
              adk[4 * hq + c] = mfma16(qv[c], dp[mt][e], adk[4 * hq + c]);
            }
          }
        }
      };
      scores(0);
      scores(1);
      softmax(0);
      grads(0);
      softmax(1);
      grads(1);
    }
    wait_all_mem();  // this wave's DMA of the next step has landed
    __syncthreads();
  }

  if (mykey < T) {
    store_d_row(reinterpret_cast<f32x4*>(dk + koff + mykey * ks), adk, g, scale);
    store_d_row(reinterpret_cast<f32x4*>(dv + koff + mykey * ks), adv, g, 1.0f);
  }
}

// dQ = scale * dS K from the stored dS on the GEMM kernel's machinery
// (gemm.hip's gemm_f32_dma): m = query, n = d, contraction over keys; 256
// queries x D per workgroup, four waves in 2 x 2 on v_mfma_f32_32x32x2f32
// tiles; 16-key stages copied global -> LDS by global_load_lds_dwordx4 into a
// 3-stage ring two stages ahead of the MFMAs, up to the tile's last query.
//   A = dS^T: a key's row of its strip holds queries 64 sb ... contiguously,
//     so one 1 KB DMA block is one key's 256 queries (chunk q of key row k at
//     chunk position q ^ (8 ((k >> 2) & 1)), as the GEMM lays out an
//     M-contiguous tile), read back as b128 rows of four consecutive queries.
//   B = K rows (d contiguous), laid out the same way.
// Entries with query < key are zeroed in registers after the LDS read: the
// dK/dV kernel does not write all of them, and a tile's queries before a
// strip's first query read the end of the strip before it (inside the same
// (b, h) region); query columns past a strip row's end are clamped into it
// (they only reach rows past T, which are not stored), keys past T into the
// last key.  Every dQ element sums the same products in the same key order
// whatever the chunking or placement of dS.
template <int D>
struct DqGemmCfg {
  static constexpr int kBM = 256, kBN = D, FI = 4, FJ = D / 64;
  static constexpr int kAFloats = kBM * 16, kBFloats = kBN * 16;
  static constexpr int kStage = kAFloats + kBFloats;
  static constexpr int kInstA = kBM / 64, kInstB = kBN / 64;  // DMA per wave per stage
};

// BUF: the DMA goes through buffer resources based at the (b, h) region of dS
// and at the KV head's first key, with 32-bit byte offsets (the launcher
// checks that both regions are under 2^31 bytes); otherwise through 64-bit
// global addresses.  The same bytes either way.
template <int D, bool BUF>
__global__ __launch_bounds__(kThreads, 2) void attn_bwd_dq_gemm_kernel(
    const float* __restrict__ k, const float* const* __restrict__ ds_rows, float* __restrict__ dq,
    int row0, int T, int H, int Hk, float scale) {
  using C = DqGemmCfg<D>;
  constexpr int FI = C::FI, FJ = C::FJ, BM = C::kBM, BN = C::kBN;
  constexpr int NR = 4 + 4 * FJ;           // LDS reads per slab: A b128 x 4, B b32 x 4 FJ
  constexpr int NM = 4 * FI * FJ;          // MFMAs per slab
  constexpr int NI = C::kInstA + C::kInstB;
  __shared__ __attribute__((aligned(1024))) float lds[3 * C::kStage];

  // A workgroup takes query tiles nmt - 1 - p and p of its row (the middle
  // tile alone when nmt is odd): nmt + 1 key-tiles of work for every pair.
  const int nmt = (T + BM - 1) / BM;
  const WorkItem wi = work_item((nmt + 1) / 2);
  const int p = wi.tile;
  const int row = row0 + wi.row;     // (b, h)
  const int h = row % H, b = row / H;
  const int hk = h / (H / Hk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r = lane & 31;
  auto run_tile = [&](const int mt) {
  const int m0 = mt * BM;
  const int64_t qs = static_cast<int64_t>(H) * D, ks = static_cast<int64_t>(Hk) * D;
  const float* kbase = k + static_cast<int64_t>(b) * T * ks + static_cast<int64_t>(hk) * D;
  const int64_t T32 = ds_t32(T);
  const float* dsrow =
      ds_rows[b * Hk + hk] + static_cast<int64_t>(h - hk * (H / Hk)) * ds_row_floats(T);

  // DMA of stage kt (keys 16 kt ... 16 kt + 15, all in strip sb) into `dst`.
#if defined(__HIP_DEVICE_COMPILE__)
  __amdgpu_buffer_rsrc_t rs_ds, rs_k;
  if constexpr (BUF) {
    rs_ds = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(dsrow), 0, 0x7fffffff,
                                              0x00020000);
    rs_k = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kbase), 0, 0x7fffffff,
                                             0x00020000);
  }
#endif
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);  // M0 from the scalar unit
  auto issue = [&](float* dst, int kt) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the kernel's launch stub
    auto copy16 = [&](const __amdgpu_buffer_rsrc_t& rs, const float* base, int64_t e,
                      float* to) {
      if constexpr (BUF)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)to,
                                                 16, static_cast<int>(e * 4), 0, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(base + e, to, 16, 0, 0);
    };
    const int k0 = 16 * kt, sb = k0 >> 6;
    const int64_t lr = T32 - 64 * sb;
    const int64_t strip = ds_strip_offset(sb, T32);
#pragma unroll
    for (int q = 0; q < C::kInstA; ++q) {
      const int t = wave_s + 4 * q;  // key row of the stage = 1 KB block of the tile
      const int q4 = lane ^ (8 * ((t >> 2) & 1));
      const int64_t col = min(static_cast<int64_t>(m0 - 64 * sb + 4 * q4), lr - 4);
      copy16(rs_ds, dsrow, strip + (k0 + t - 64 * sb) * lr + col, dst + 256 * t);
    }
    constexpr int kRowsPer = 256 / BN, kLanesPer = 64 / kRowsPer;
#pragma unroll
    for (int q = 0; q < C::kInstB; ++q) {
      const int t = wave_s + 4 * q;
      const int kr = t * kRowsPer + lane / kLanesPer;
      const int q4 = (lane % kLanesPer) ^ (8 * ((kr >> 2) & 1));
      const int key = min(k0 + kr, T - 1);
      copy16(rs_k, kbase, static_cast<int64_t>(key) * ks + 4 * q4, dst + C::kAFloats + 256 * t);
    }
#endif
  };
  // A fragments of slab s: query m0 + 128 wm + 4 r + i at k-step j (key
  // 16 kt + 8 s + 4 g + j) in fa[i][j]; query < key zeroed where the slab
  // reaches past the wave's first query.
  const int qw = m0 + (BM / 2) * wm;
  auto load_a = [&](const float* st, int kt, int s, f32x4 (&fa)[FI]) {
    const int off = 4 * (((BM / 8) * wm + r) ^ (8 * g));  // chunk (qw - m0) / 4 + r
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(st + (8 * s + 4 * g + j) * BM + off);
#pragma unroll
      for (int i = 0; i < FI; ++i) fa[i][j] = v[i];
    }
    if (16 * kt + 8 * s + 7 > qw) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < FI; ++i)
          fa[i][j] = qw + 4 * r + i < 16 * kt + 8 * s + 4 * g + j ? 0.f : fa[i][j];
    }
  };
  const int mbB = (wn * (BN / 2)) >> 2;
  auto load_b = [&](const float* st, int s, f32x4 (&fb)[FJ]) {
#pragma unroll
    for (int jj = 0; jj < FJ; ++jj) {
      const int qc = (mbB + 8 * jj) ^ (8 * g);
      const float* p = st + C::kAFloats + (8 * s + 4 * g) * BN + (qc << 2) + r;
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[jj][j] = p[j * BN];
    }
  };

  f32x16 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int jj = 0; jj < FJ; ++jj)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][jj][e] = 0.f;

  const int kend = min(T, m0 + BM);
  const int nk = (kend + 15) / 16;
  issue(lds, 0);
  if (nk > 1) {
    issue(lds + C::kStage, 1);
    wait_vm_lgkm0<NI>();
  } else {
    wait_vm_lgkm0<0>();
  }
  block_barrier();
  f32x4 fa0[FI], fb0[FJ], fa1[FI], fb1[FJ];
  load_a(lds, 0, 0, fa0);
  load_b(lds, 0, fb0);

  // The GEMM kernel's stage: slab 1's reads, slab 0's MFMAs with them spread
  // among, the DMA two stages ahead, slab 1's first MFMAs, the barrier after
  // stage kt+1's copy has landed, the next stage's slab-0 reads under slab
  // 1's last MFMAs.
  int ic = 0;  // kt % 3
  auto stage = [&](int kt, auto with_dma) {
    constexpr bool kDma = decltype(with_dma)::value;
    float* cur = lds + ic * C::kStage;
    float* nxt = lds + (ic == 2 ? 0 : ic + 1) * C::kStage;
    float* nx2 = lds + (ic == 0 ? 2 : ic - 1) * C::kStage;
    load_a(cur, kt, 1, fa1);
    load_b(cur, 1, fb1);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int jj = 0; jj < FJ; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[i][s], fb0[jj][s], acc[i][jj], 0,
                                                            0, 0);
    interleave_mfma_first<NR, NM, 0x100>();
    if constexpr (kDma) issue(nx2, kt + 2);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int jj = 0; jj < FJ; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[jj][s], acc[i][jj], 0,
                                                            0, 0);
    if constexpr (kDma) interleave<NI, NM / 2, 0x020>();
    if constexpr (kDma)
      wait_vm_lgkm0<NI>();
    else
      wait_vm_lgkm0<0>();
    block_barrier();
    load_a(nxt, kt + 1, 0, fa0);  // past the last stage: unused reads inside the ring
    load_b(nxt, 0, fb0);
#pragma unroll
    for (int s = 2; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int jj = 0; jj < FJ; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[i][s], fb1[jj][s], acc[i][jj], 0,
                                                            0, 0);
    interleave<NR, NM / 2, 0x100>();
    ic = ic == 2 ? 0 : ic + 1;
  };
  int kt = 0;
  for (; kt + 2 < nk; ++kt) stage(kt, std::true_type{});
  for (; kt < nk; ++kt) stage(kt, std::false_type{});

  float* dqb = dq + static_cast<int64_t>(b) * T * qs + static_cast<int64_t>(h) * D;
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int jj = 0; jj < FJ; ++jj) {
      const int col = wn * (BN / 2) + jj * 32 + r;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int x = 8 * (e >> 2) + 4 * g + (e & 3);  // the MFMA tile's row slot
        const int q = qw + 4 * x + i;
        if (q < T) dqb[static_cast<int64_t>(q) * qs + col] = scale * acc[i][jj][e];
      }
    }
  };
  run_tile(nmt - 1 - p);
  if (nmt - 1 - p != p) {
    wait_vm_lgkm0<0>();  // every wave is done with the ring before it is refilled
    block_barrier();
    run_tile(p);
  }
}

int check_shapes(int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D) {
  if (B < 0 || T < 0 || H <= 0 || Hk <= 0 || H % Hk != 0) return EMBER_EINVAL;
  if (D != 64 && D != 128) return EMBER_EINVAL;
  if (T > 0x7fffffff / 2 || H > 65535 || Hk > 65535 || B > 65535) return EMBER_EINVAL;
  // 1-D grids: 128-query forward tiles, 64-row backward tiles, Hk <= H.
  if ((T + 63) / 64 * H * B > 0x7fffffff) return EMBER_EINVAL;
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
  static_assert(FwdCfg<64>::kBQ == 128 && FwdCfg<128>::kBQ == 128, "grid assumes 128 queries");
  const dim3 grid(static_cast<unsigned>((T + 127) / 128 * H * B));
  const float sl = scale * kLog2e;
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H), Hki = static_cast<int>(Hk);
  if (D == 64)
    attn_fwd_kernel<64, false><<<grid, FwdCfg<64>::kThreads, 0, as_stream(s)>>>(
        q, k, v, o, lse, nullptr, Ti, Hi, Hki, sl);
  else
    attn_fwd_kernel<128, false><<<grid, FwdCfg<128>::kThreads, 0, as_stream(s)>>>(
        q, k, v, o, lse, nullptr, Ti, Hi, Hki, sl);
  return launch_status();
}

namespace {

size_t delta_bytes(int64_t B, int64_t T, int64_t H) {
  return static_cast<size_t>((B * T * H * 4 + 255) / 256 * 256);
}
// The KV-row table: room for B*H pointers (B*Hk are used; H >= Hk keeps the
// workspace query independent of Hk).
size_t table_bytes(int64_t B, int64_t H) {
  return static_cast<size_t>((B * H * 8 + 255) / 256 * 256);
}
// dS bytes of one KV row: its group's (b, h) rows of causal strips.
size_t kv_row_ds_bytes(int64_t T, int64_t group) {
  return static_cast<size_t>(group * ds_row_floats(T)) * sizeof(float);
}

// The backward over buffers for dS (host array of device pointers and sizes;
// none: dQ recomputes dS).  `ws` holds rowsum(dO*O) and the KV-row table.
template <int D>
int launch_bwd(const float* q, const float* k, const float* v, const float* o, const float* lse,
               const float* dout, float* dq, float* dk, float* dv, int64_t B, int64_t T,
               int64_t H, int64_t Hk, float scale, char* ws, float* const* bufs,
               const size_t* buf_bytes, int nbufs, bool from_scores, hipStream_t st) {
  float* delta = reinterpret_cast<float*>(ws);
  float** table = reinterpret_cast<float**>(ws + delta_bytes(B, T, H));
  const int64_t rows = B * T * H;
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H), Hki = static_cast<int>(Hk);
  const float sl = scale * kLog2e;
  if (from_scores) {  // the scores of every KV row must be there: checked before any launch
    int64_t slots = 0;
    const size_t rb = kv_row_ds_bytes(T, H / Hk);
    for (int i = 0; i < nbufs; ++i) slots += static_cast<int64_t>(buf_bytes[i] / rb);
    if (slots < B * Hk) return EMBER_EWORKSPACE;
  }
  constexpr int RPB = kThreads / (D / 4);
  attn_delta_kernel<D><<<static_cast<unsigned>((rows + RPB - 1) / RPB), kThreads, 0, st>>>(
      o, dout, delta, rows, Ti, Hi);
  int rc = launch_status();
  if (rc) return rc;
  static_assert(DqCfg<D>::kBQ == 64, "recompute dQ grid assumes 64 queries");
  static_assert(DkvCfg<D>::kBKeys == 64, "dK/dV grid assumes 64 keys");
  const unsigned nqb = static_cast<unsigned>((T + 63) / 64);
  const unsigned nmt = static_cast<unsigned>((T + DqGemmCfg<D>::kBM - 1) / DqGemmCfg<D>::kBM);
  const int64_t group = H / Hk, kv_rows = B * Hk;
  const size_t row_bytes = kv_row_ds_bytes(T, group);
  // The dQ GEMM's 32-bit DMA offsets span one (b, h) region of dS and one KV
  // head's keys.
  const bool dq_buf =
      4 * std::max<int64_t>(ds_row_floats(T), T * Hk * D) < (int64_t{1} << 31) - 256;
  // KV-row slots in the buffers, in buffer order.
  int64_t chunk = 0;
  for (int i = 0; i < nbufs; ++i) chunk += static_cast<int64_t>(buf_bytes[i] / row_bytes);
  if (chunk < 1) {  // no room for dS: dQ recomputes S and dP
    attn_bwd_dq_kernel<D><<<dim3(nqb * static_cast<unsigned>(B * H)), kThreads, 0, st>>>(
        q, k, v, dout, lse, delta, dq, Ti, Hi, Hki, sl, scale);
    if ((rc = launch_status())) return rc;
    attn_bwd_dkdv_kernel<D, false, false><<<dim3(nqb * static_cast<unsigned>(kv_rows)), kThreads, 0, st>>>(
        q, k, v, dout, lse, delta, dk, dv, nullptr, 0, Ti, Hi, Hki, sl, scale);
    return launch_status();
  }
  // Chunks of KV rows whose dS fits, as equal as the room allows (a short
  // last chunk leaves its dK/dV launch too few workgroups for the causal
  // triangle's uneven blocks), in multiples of 8 rows where the room has 8,
  // which keeps the XCD regrouping of the work items.
  if (chunk >= kv_rows) {
    chunk = kv_rows;
  } else {
    if (chunk >= 8) chunk -= chunk % 8;
    const int64_t nch = (kv_rows + chunk - 1) / chunk;
    int64_t even = (kv_rows + nch - 1) / nch;
    if (chunk >= 8) even = (even + 7) / 8 * 8;
    chunk = even < chunk ? even : chunk;
  }
  // KV row r of a chunk takes slot r - r0: the same slots for every chunk.
  std::vector<float*> host_table(static_cast<size_t>(kv_rows));
  std::vector<float*> slot(static_cast<size_t>(chunk));
  {
    int64_t j = 0;
    for (int i = 0; i < nbufs && j < chunk; ++i)
      for (size_t off = 0; off + row_bytes <= buf_bytes[i] && j < chunk; off += row_bytes)
        slot[static_cast<size_t>(j++)] = bufs[i] + off / sizeof(float);
  }
  for (int64_t r = 0; r < kv_rows; ++r)
    host_table[static_cast<size_t>(r)] = slot[static_cast<size_t>(r % chunk)];
  if ((rc = upload_async(table, host_table.data(), host_table.size() * sizeof(float*), st)))
    return rc;
  for (int64_t r0 = 0; r0 < kv_rows; r0 += chunk) {
    const int64_t n = kv_rows - r0 < chunk ? kv_rows - r0 : chunk;
    if (from_scores)
      attn_bwd_dkdv_kernel<D, true, true><<<dim3(nqb * static_cast<unsigned>(n)), kThreads, 0,
                                             st>>>(q, k, v, dout, lse, delta, dk, dv, table,
                                                   static_cast<int>(r0), Ti, Hi, Hki, sl, scale);
    else
      attn_bwd_dkdv_kernel<D, true, false><<<dim3(nqb * static_cast<unsigned>(n)), kThreads, 0,
                                              st>>>(q, k, v, dout, lse, delta, dk, dv, table,
                                                    static_cast<int>(r0), Ti, Hi, Hki, sl, scale);
    if ((rc = launch_status())) return rc;
    const dim3 grid((nmt + 1) / 2 * static_cast<unsigned>(n * group));
    if (dq_buf)
      attn_bwd_dq_gemm_kernel<D, true><<<grid, kThreads, 0, st>>>(
          k, table, dq, static_cast<int>(r0 * group), Ti, Hi, Hki, scale);
    else
      attn_bwd_dq_gemm_kernel<D, false><<<grid, kThreads, 0, st>>>(
          k, table, dq, static_cast<int>(r0 * group), Ti, Hi, Hki, scale);
    if ((rc = launch_status())) return rc;
  }
  return EMBER_OK;
}

int attn_bwd_run(const float* q, const float* k, const float* v, const float* o, const float* lse,
                 const float* dout, float* dq, float* dk, float* dv, int64_t B, int64_t T,
                 int64_t H, int64_t Hk, int64_t D, float scale, void* workspace,
                 size_t workspace_bytes, float* const* bufs, const size_t* buf_bytes, int nbufs,
                 bool from_scores, ember_stream_t s) {
  int rc = check_shapes(B, T, H, Hk, D);
  if (rc) return rc;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return EMBER_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dout) ||
      !aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(workspace))
    return EMBER_EALIGN;
  if (!workspace || workspace_bytes < ember_attn_bwd_workspace_bytes_min(B, T, H))
    return EMBER_EWORKSPACE;
  if (nbufs < 0 || (nbufs > 0 && (!bufs || !buf_bytes))) return EMBER_EINVAL;
  for (int i = 0; i < nbufs; ++i) {
    if (buf_bytes[i] > 0 && !bufs[i]) return EMBER_EINVAL;
    if (!aligned16(bufs[i])) return EMBER_EALIGN;
  }
  char* ws = static_cast<char*>(workspace);
  if (D == 64)
    return launch_bwd<64>(q, k, v, o, lse, dout, dq, dk, dv, B, T, H, Hk, scale, ws, bufs,
                          buf_bytes, nbufs, from_scores, as_stream(s));
  return launch_bwd<128>(q, k, v, o, lse, dout, dq, dk, dv, B, T, H, Hk, scale, ws, bufs,
                         buf_bytes, nbufs, from_scores, as_stream(s));
}

}  // namespace

extern "C" size_t ember_attn_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return ember_attn_bwd_workspace_bytes_min(B, T, H) +
         static_cast<size_t>(B * H * ds_row_floats(T)) * sizeof(float);
}

extern "C" size_t ember_attn_bwd_workspace_bytes_min(int64_t B, int64_t T, int64_t H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return delta_bytes(B, T, H) + table_bytes(B, H);
}

extern "C" size_t ember_attn_bwd_ds_row_bytes(int64_t T, int64_t H, int64_t Hk) {
  if (T <= 0 || H <= 0 || Hk <= 0 || H % Hk) return 0;
  return kv_row_ds_bytes(T, H / Hk);
}

extern "C" int ember_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                              const float* lse, const float* dout, float* dq, float* dk, float* dv,
                              int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                              void* workspace, size_t workspace_bytes, ember_stream_t s) {
  // dS goes in the workspace after rowsum(dO*O) and the KV-row table.
  const size_t lo = ember_attn_bwd_workspace_bytes_min(B, T, H);
  float* buf = workspace && workspace_bytes > lo
                   ? reinterpret_cast<float*>(static_cast<char*>(workspace) + lo)
                   : nullptr;
  const size_t bytes = buf ? workspace_bytes - lo : 0;
  return attn_bwd_run(q, k, v, o, lse, dout, dq, dk, dv, B, T, H, Hk, D, scale, workspace,
                      workspace_bytes, &buf, &bytes, buf ? 1 : 0, false, s);
}

extern "C" int ember_attn_bwd_scattered(const float* q, const float* k, const float* v,
                                        const float* o, const float* lse, const float* dout,
                                        float* dq, float* dk, float* dv, int64_t B, int64_t T,
                                        int64_t H, int64_t Hk, int64_t D, float scale,
                                        void* workspace, size_t workspace_bytes,
                                        float* const* ds_bufs_host, const size_t* ds_bytes_host,
                                        int nbufs, ember_stream_t s) {
  return attn_bwd_run(q, k, v, o, lse, dout, dq, dk, dv, B, T, H, Hk, D, scale, workspace,
                      workspace_bytes, ds_bufs_host, ds_bytes_host, nbufs, false, s);
}

extern "C" size_t ember_attn_scores_workspace_bytes(int64_t B, int64_t H) {
  if (B <= 0 || H <= 0) return 0;
  return table_bytes(B, H);
}

extern "C" int ember_attn_fwd_scores(const float* q, const float* k, const float* v, float* o,
                                     float* lse, int64_t B, int64_t T, int64_t H, int64_t Hk,
                                     int64_t D, float scale, float* const* s_bufs_host,
                                     const size_t* s_bytes_host, int nbufs, void* workspace,
                                     size_t workspace_bytes, ember_stream_t s) {
  int rc = check_shapes(B, T, H, Hk, D);
  if (rc) return rc;
  if (B == 0 || T == 0) return EMBER_OK;
  if (!q || !k || !v || !o || !lse) return EMBER_EINVAL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return EMBER_EALIGN;
  if (!workspace || workspace_bytes < ember_attn_scores_workspace_bytes(B, H))
    return EMBER_EWORKSPACE;
  if (nbufs < 1 || !s_bufs_host || !s_bytes_host) return EMBER_EINVAL;
  const int64_t kv_rows = B * Hk;
  const size_t row_bytes = kv_row_ds_bytes(T, H / Hk);
  // Whole KV rows from the buffers in order, as the backward lays them out
  // when one chunk holds every row.
  std::vector<float*> host_table;
  for (int i = 0; i < nbufs && static_cast<int64_t>(host_table.size()) < kv_rows; ++i) {
    if (s_bytes_host[i] > 0 && !s_bufs_host[i]) return EMBER_EINVAL;
    if (!aligned16(s_bufs_host[i])) return EMBER_EALIGN;
    for (size_t off = 0; off + row_bytes <= s_bytes_host[i] &&
                         static_cast<int64_t>(host_table.size()) < kv_rows;
         off += row_bytes)
      host_table.push_back(s_bufs_host[i] + off / sizeof(float));
  }
  if (static_cast<int64_t>(host_table.size()) < kv_rows) return EMBER_EWORKSPACE;
  hipStream_t st = as_stream(s);
  float** table = static_cast<float**>(workspace);
  if ((rc = upload_async(table, host_table.data(), host_table.size() * sizeof(float*), st)))
    return rc;
  const dim3 grid(static_cast<unsigned>((T + 127) / 128 * H * B));
  const float sl = scale * kLog2e;
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H), Hki = static_cast<int>(Hk);
  if (D == 64)
    attn_fwd_kernel<64, true><<<grid, FwdCfg<64>::kThreads, 0, st>>>(q, k, v, o, lse, table, Ti,
                                                                      Hi, Hki, sl);
  else
    attn_fwd_kernel<128, true><<<grid, FwdCfg<128>::kThreads, 0, st>>>(q, k, v, o, lse, table, Ti,
                                                                        Hi, Hki, sl);
  return launch_status();
}

extern "C" int ember_attn_bwd_from_scores(const float* q, const float* k, const float* v,
                                          const float* o, const float* lse, const float* dout,
                                          float* dq, float* dk, float* dv, int64_t B, int64_t T,
                                          int64_t H, int64_t Hk, int64_t D, float scale,
                                          void* workspace, size_t workspace_bytes,
                                          float* const* s_bufs_host, const size_t* s_bytes_host,
                                          int nbufs, ember_stream_t s) {
  if (nbufs < 1) return EMBER_EINVAL;
  return attn_bwd_run(q, k, v, o, lse, dout, dq, dk, dv, B, T, H, Hk, D, scale, workspace,
                      workspace_bytes, s_bufs_host, s_bytes_host, nbufs, true, s);
}
