/*
 * ember_hip.h -- C ABI of the MI355X (gfx950) kernels for emberlm's training hot path.
 *
 * This is the drop-in boundary: the C++ Tensor/autograd/Module layer
 * (include/ctd/...) calls only these functions, and a foreign binding needs
 * nothing else.  Conventions:
 *   - every function returns an int status: EMBER_OK (0), a negative EMBER_E*
 *     code for a rejected argument, or a positive hipError_t value;
 *   - nothing throws and no kernel entry point allocates device memory;
 *     functions that need scratch take an explicit workspace and export a
 *     *_workspace_bytes() size query;
 *   - pointers are device pointers unless the name says host; all tensors are
 *     fp32 row-major contiguous unless stated (token ids are int64);
 *   - work is enqueued on the given stream (NULL = the default stream) and is
 *     asynchronous to the host;
 *   - 64-bit sizes and offsets throughout (the reference's int32 row*V
 *     indexing, src/ops/loss.cu:112-113 and 263-264, overflows at N*V > 2^31).
 * Each declaration cites the reference function it replaces.
 */
#ifndef EMBER_HIP_H
#define EMBER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ember_stream_t; /* hipStream_t */
typedef void* ember_event_t;  /* hipEvent_t */

enum {
  EMBER_OK = 0,
  EMBER_EINVAL = -1,     /* bad size, shape, null pointer or flag */
  EMBER_EWORKSPACE = -2, /* workspace missing or too small */
  EMBER_EALIGN = -3,     /* pointer alignment the kernel requires is not met */
  EMBER_EMASKSUM = -4,   /* sum(loss_mask) == 0 in cross-entropy backward */
  EMBER_ESCRATCH = -5,   /* problem larger than an allocation-free entry's fixed scratch */
  EMBER_NOTREADY = 600   /* ember_event_query: work before the event still pending */
};

/* Human-readable text for a status code (static storage). */
const char* ember_status_string(int status);

/* ------------------------------------------------------------------ runtime
 * Replace cudaMalloc/cudaFree/cudaMallocHost and cudaMemcpy of
 * src/core/allocator.cpp:14-57 and src/core/tensor.cpp:84-108. */
int ember_get_device_count(int* count);
int ember_set_device(int device);
int ember_get_device(int* device);
int ember_device_malloc(void** ptr, size_t bytes);
int ember_device_free(void* ptr);
/* Page-locked host memory (hipHostMalloc); the reference's offload path used
 * pageable memory instead (src/core/optim.cu:114-117). */
int ember_host_malloc_pinned(void** ptr, size_t bytes);
int ember_host_free_pinned(void* ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device, 3 host->host */
int ember_memcpy_async(void* dst, const void* src, size_t bytes, int kind, ember_stream_t s);
int ember_memcpy(void* dst, const void* src, size_t bytes, int kind);
int ember_mem_get_info(size_t* free_bytes, size_t* total_bytes);
int ember_device_synchronize(void);
/* Streams are created at the default priority. */
int ember_stream_create(ember_stream_t* s);
int ember_stream_destroy(ember_stream_t s);
int ember_stream_synchronize(ember_stream_t s);
int ember_event_create(ember_event_t* e);
int ember_event_destroy(ember_event_t e);
int ember_event_record(ember_event_t e, ember_stream_t s);
int ember_event_synchronize(ember_event_t e);
/* EMBER_OK once the work recorded before e has finished, EMBER_NOTREADY before. */
int ember_event_query(ember_event_t e);
int ember_stream_wait_event(ember_stream_t s, ember_event_t e);
int ember_event_elapsed_ms(float* ms, ember_event_t start, ember_event_t stop);
/* Device name / CU count / HBM bytes of the current device. */
int ember_device_info(char* name, size_t name_cap, int* cu_count, size_t* hbm_bytes);

/* ---------------------------------------------------------------- fills
 * Counter-based generator (SplitMix64 + Box-Muller): element i of a stream
 * depends only on (seed, offset + i), so host and device agree and any slice
 * can be regenerated.  Used for seeded synthetic weights and activations. */
int ember_fill_normal(float* p, int64_t n, uint64_t seed, uint64_t offset, float mean,
                      float stddev, ember_stream_t s);
int ember_fill(float* p, int64_t n, float value, ember_stream_t s);

/* ----------------------------------------------------------------- GEMM
 * C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b], fp32 operands, fp32 MFMA.
 * op(A) is MxK: A is stored [M,K] (lda >= K) or, when transa, [K,M] (lda >= M);
 * op(B) is KxN: B is stored [K,N] (ldb >= N) or, when transb, [N,K] (ldb >= K).
 * C is [M,N] with ldc >= N.  batch >= 1 with element strides sA/sB/sC.
 * Replaces cublasSgemm / cublasSgemmStridedBatched in ops::matmul_impl and
 * ops::bmm_impl (src/ops/matmul.cpp:13-49, 51-93; row-major trick 38-47). */
int ember_gemm_f32(int transa, int transb, int64_t M, int64_t N, int64_t K, float alpha,
                   const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb,
                   int64_t sB, float beta, float* C, int64_t ldc, int64_t sC, int64_t batch,
                   ember_stream_t s);
/* The same product with a workspace: when the output grid is too small to fill
 * the GPU and K is long (weight gradients, K = tokens), K is split into partial
 * products in `workspace` that are then summed in a fixed order, so results are
 * reproducible run to run.  ember_gemm_f32_workspace_bytes gives the size this
 * call can use (0: no split for this shape); a smaller or NULL workspace runs
 * the unsplit kernel.  ember_gemm_f32 is this call with no workspace. */
/* These entry points and ember_gemm_f32_add run products with at most 8 rows
 * (M <= 8, batch 1, A and B K-contiguous i.e. transa = 0 and transb = 1,
 * 16-byte aligned, K % 4 == 0: Linear forward of a decode step) on a skinny
 * kernel that streams B at HBM rate instead of on the MFMA tiles. */
size_t ember_gemm_f32_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t batch);
int ember_gemm_f32_ws(int transa, int transb, int64_t M, int64_t N, int64_t K, float alpha,
                      const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb,
                      int64_t sB, float beta, float* C, int64_t ldc, int64_t sC, int64_t batch,
                      void* workspace, size_t workspace_bytes, ember_stream_t s);
/* ember_gemm_f32_ws (batch 1) with one extent known only on the device, so a
 * caller can size a product by a count a kernel produced without waiting for
 * it on the host.  v = clamp(*count - base, 0, extent):
 *   dim 0: only rows [0, v) of C are wanted; whole row tiles past v are
 *          skipped, rows of a tile that straddles v are written too.
 *   dim 1: K becomes v rounded up to a multiple of 16; the operands' k rows
 *          [v, that) are read and must hold finite values (zeros contribute
 *          nothing).  With v = 0 and beta = 1, C is left untouched.
 * Requires 16-byte aligned A and B, lda and ldb multiples of 4, K % 16 == 0 and
 * M (N) % 4 == 0 when A (B) is MN-contiguous; otherwise EMBER_EINVAL.  The
 * workspace is ember_gemm_f32_ws's (a K split only with dim 0).  Used by
 * the LM head to compute only rows whose loss-mask value is nonzero.  Added in
 * this build; the reference sizes every product on the host. */
int ember_gemm_f32_dyn(int transa, int transb, int64_t M, int64_t N, int64_t K, float alpha,
                       const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                       float* C, int64_t ldc, const int64_t* count, int64_t base, int dim,
                       void* workspace, size_t workspace_bytes, ember_stream_t s);
/* C = alpha op(A) op(B) + D (batch 1): a product and a residual add in one
 * pass, the add done where the product is stored (the split-K reduce when K
 * is split).  Replaces the matmul + ops::add pairs of the block's residual
 * connections (include/ctd/nn/transformer_block.h:21, 24 with
 * src/ops/matmul.cpp:38-47 and the add kernel, src/ops/elementwise.cu:14-20,
 * 89-101); element for element the same float additions as the product
 * stored and then added, so the results are bitwise equal.  D is [M][ldd],
 * ldd >= N; it may be C itself (ldd == ldc, the same as beta = 1) but must
 * not otherwise overlap C (EMBER_EINVAL).  The workspace is
 * ember_gemm_f32_ws's. */
int ember_gemm_f32_add(int transa, int transb, int64_t M, int64_t N, int64_t K, float alpha,
                       const float* A, int64_t lda, const float* B, int64_t ldb, const float* D,
                       int64_t ldd, float* C, int64_t ldc, void* workspace,
                       size_t workspace_bytes, ember_stream_t s);

/* -------------------------------------------------------------- RMSNorm
 * y = x * rsqrt(mean(x^2) + eps) * w over rows of length H; rstd[rows] (may be
 * NULL) receives rsqrt(mean(x^2)+eps).  Replaces rms_norm_kernel_f32
 * (src/ops/norm.cu:17-49) for block norms and per-head QK-Norm. */
int ember_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd, int64_t rows,
                      int64_t H, float eps, ember_stream_t s);
/* dx and dw from dy (src/ops/norm.cu:51-106).  dw is written (not accumulated)
 * through a deterministic two-stage reduction in `workspace`; either dx or dw
 * may be NULL.  rstd may be NULL (recomputed). */
size_t ember_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t H);
int ember_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rstd,
                      float* dx, float* dw, int64_t rows, int64_t H, float eps, void* workspace,
                      size_t workspace_bytes, ember_stream_t s);
/* ember_rmsnorm_bwd with dx accumulated: dx += the input gradient (dx must
 * hold the running sum; one add per element, as ember_accumulate after
 * ember_rmsnorm_bwd, so the same bits).  For an input whose other consumers'
 * gradients already sit in dx, e.g. the residual stream of a block (the
 * reference's autograd adds them in its fan-in, src/core/autograd.cu:86-118). */
int ember_rmsnorm_bwd_accumulate(const float* dy, const float* x, const float* w,
                                 const float* rstd, float* dx, float* dw, int64_t rows, int64_t H,
                                 float eps, void* workspace, size_t workspace_bytes,
                                 ember_stream_t s);
/* ember_rmsnorm_bwd with no workspace argument and no allocation of any kind,
 * for callers that cannot allocate device memory: code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc.  No counterpart
 * in the reference.  The dw partials go to one fixed array of
 * EMBER_RMSNORM_BWD_SCRATCH_BYTES in device memory, one per GPU, held until
 * the process ends: sizes whose ember_rmsnorm_bwd_workspace_bytes(rows, H)
 * exceed it return EMBER_ESCRATCH (any row count fits for H <= 4096).  Results
 * are bitwise those of ember_rmsnorm_bwd.  Every call on a GPU uses that GPU's
 * one array, so calls that overlap on one GPU (two streams, two threads) race;
 * the stream must belong to the current device (else EMBER_EINVAL). */
#define EMBER_RMSNORM_BWD_SCRATCH_BYTES ((size_t)16 << 20)
int ember_rmsnorm_bwd_noalloc(const float* dy, const float* x, const float* w, const float* rstd,
                              float* dx, float* dw, int64_t rows, int64_t H, float eps,
                              ember_stream_t s);

/* ----------------------------------------------------------------- RoPE
 * Frequencies of the D/2 rotation pairs in float, following src/ops/rope.cu:37-46
 * (llama3 band scaling when factor > 1).  Host-only helper. */
int ember_rope_freqs_host(float* freqs_out, int D, float theta, float factor,
                          float low_freq_factor, float high_freq_factor,
                          int original_max_pos);
/* y = R(sign * angle) x for x [B,T,H,D], pairs (i, i+D/2), angle = float(pos0+t)*freq[i]
 * rounded to fp32 (rope.cu:49); sign = -1 is RopeBackward's transpose
 * (rope.cu:106-118).  freqs_host: D/2 values from ember_rope_freqs_host (passed
 * by value to the kernel).  y may equal x (in place, apply_rope_inplace).
 * D even and <= 256.  Replaces rope_kernel_f32 (src/ops/rope.cu:17-56). */
int ember_rope(const float* x, float* y, int64_t B, int64_t T, int64_t H, int64_t D,
               int64_t pos0, const float* freqs_host, float sign, ember_stream_t s);

/* Per-head QK-Norm followed by RoPE in one pass: y = R(angle) (x * rstd * w)
 * over rows = B*T*heads rows of D floats (row (b*T + t)*heads + h, position
 * pos0 + t), bitwise ember_rmsnorm_fwd then ember_rope (sign 1); rstd[rows]
 * may be NULL.  The backward is bitwise ember_rope (sign -1) then
 * ember_rmsnorm_bwd: dx and dw (either may be NULL; dw through the workspace
 * that ember_rmsnorm_bwd_workspace_bytes(rows, D) sizes).  D = 64 or 128,
 * 16-byte aligned rows, freqs_host as for ember_rope.  Replaces the
 * q_norm / k_norm then rope pair of Attention::forward_train and forward
 * (include/ctd/nn/attention.h:115-121 and 58-64 of the reference; norm.cu:17-49,
 * rope.cu:17-56) and the two backward nodes. */
int ember_qknorm_rope_fwd(const float* x, const float* w, float* y, float* rstd, int64_t rows,
                          int64_t heads, int64_t T, int64_t D, float eps, int64_t pos0,
                          const float* freqs_host, ember_stream_t s);
int ember_qknorm_rope_bwd(const float* dy, const float* x, const float* w, const float* rstd,
                          float* dx, float* dw, int64_t rows, int64_t heads, int64_t T,
                          int64_t D, float eps, int64_t pos0, const float* freqs_host,
                          void* workspace, size_t workspace_bytes, ember_stream_t s);

/* --------------------------------------------------------- elementwise
 * Replace src/ops/elementwise.cu:15-69, repeat_kv.cu:45-51 and
 * autograd.cu:88-93 (addinto). */
int ember_add(const float* a, const float* b, float* y, int64_t n, ember_stream_t s);
int ember_sub(const float* a, const float* b, float* y, int64_t n, ember_stream_t s);
int ember_mul(const float* a, const float* b, float* y, int64_t n, ember_stream_t s);
int ember_scale(const float* x, float alpha, float* y, int64_t n, ember_stream_t s);
/* y += x (autograd fan-in, autograd.cu:86-118). */
int ember_accumulate(float* y, const float* x, int64_t n, ember_stream_t s);
int ember_silu(const float* x, float* y, int64_t n, ember_stream_t s);
int ember_silu_bwd(const float* x, const float* g, float* dx, int64_t n, ember_stream_t s);
/* Fused SwiGLU: h = silu(g) * u (MLP::forward, include/ctd/nn/mlp.h:16-21).  h may
 * be g or u. */
int ember_swiglu_fwd(const float* g, const float* u, float* h, int64_t n, ember_stream_t s);
/* dg = dh * u * silu'(g), du = dh * silu(g) (MulBackward + SiluBackward,
 * elementwise.cu:57-69, 186-238).  dg may be g and du may be u (each element
 * is read before it is written); no other overlap is allowed. */
int ember_swiglu_bwd(const float* g, const float* u, const float* dh, float* dg, float* du,
                     int64_t n, ember_stream_t s);

/* ------------------------------------------------ unfused attention ops
 * The reference's attention chain, kept for the ops:: API and parity tests. */
/* Row softmax over the last dim N (src/ops/softmax.cu:17-52). */
int ember_softmax_fwd(const float* x, float* y, int64_t rows, int64_t N, ember_stream_t s);
/* dx = y * (g - sum(g*y)) (softmax.cu:54-80). */
int ember_softmax_bwd(const float* y, const float* g, float* dx, int64_t rows, int64_t N,
                      ember_stream_t s);
/* out = (k > q0 + q) ? fill : in, rows of [*, Tq, Tk] (src/ops/mask.cu:15-52);
 * backward uses fill = 0 on the upstream grad.  out may equal in. */
int ember_causal_mask(const float* in, float* out, int64_t rows, int64_t Tq, int64_t Tk,
                      int64_t q0, float fill, ember_stream_t s);
/* [BT,Hk,D] -> [BT,Hk*group,D] and its group-sum (src/ops/repeat_kv.cu:16-43). */
int ember_repeat_kv(const float* x, float* y, int64_t BT, int64_t Hk, int64_t group,
                    int64_t D, ember_stream_t s);
int ember_repeat_kv_sum(const float* y, float* x, int64_t BT, int64_t Hk, int64_t group,
                        int64_t D, ember_stream_t s);
/* Generic rank<=6 permutation y.shape[i] = shape[perm[i]] (src/ops/permute.cu:20-127);
 * shape/perm are host arrays, passed by value (no device allocation or sync). */
int ember_permute(const float* x, float* y, int ndim, const int64_t* shape_host,
                  const int* perm_host, ember_stream_t s);

/* ------------------------------------------------ fused causal attention
 * Causal GQA attention over q [B,T,H,D], k/v [B,T,Hk,D] -> o [B,T,H,D] with
 * lse [B,H,T] (natural-log log-sum-exp of the scaled, masked scores).  Equals
 * the reference chain bmm -> mul_scalar -> apply_causal_mask -> softmax -> bmm
 * with repeat_kv_heads/permute (include/ctd/nn/attention.h:100-143) without
 * materialising [B*H,T,T]; head h reads KV head h / (H/Hk).  D in {64, 128}. */
int ember_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                   int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                   ember_stream_t s);
/* Backward of ember_attn_fwd: dq [B,T,H,D], dk/dv [B,T,Hk,D] (written, summed
 * over each KV head's query group in a fixed order: deterministic).  Replaces
 * BmmBackward, SoftmaxBackward, CausalMaskBackward, MulScalarBackward,
 * RepeatKvBackward and PermuteBackward of the chain (matmul.cpp:137-152,
 * softmax.cu:54-80, mask.cu:41-52, repeat_kv.cu:29-43, permute.cu).
 * The workspace holds rowsum(dO*O) ([B,H,T]), a table of KV-row pointers and,
 * when it is large enough, dS for the causal part of as many KV heads' query
 * groups as fit (ember_attn_bwd_ds_row_bytes per (batch, KV head), about
 * group*4*T^2/2 bytes); the dQ product then reads dS instead of recomputing
 * it, and the work runs in chunks of KV heads.
 * ember_attn_bwd_workspace_bytes: the size that keeps all of dS (fastest);
 * ember_attn_bwd_workspace_bytes_min: the smallest accepted (no dS kept).
 * Any size in between works; dq, dk and dv do not depend on the chunking. */
size_t ember_attn_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H);
size_t ember_attn_bwd_workspace_bytes_min(int64_t B, int64_t T, int64_t H);
size_t ember_attn_bwd_ds_row_bytes(int64_t T, int64_t H, int64_t Hk);
int ember_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                   const float* lse, const float* dout, float* dq, float* dk, float* dv,
                   int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                   void* workspace, size_t workspace_bytes, ember_stream_t s);
/* ember_attn_bwd with dS in separate buffers (a host array of nbufs device
 * pointers and sizes; the workspace needs only ember_attn_bwd_workspace_bytes_min):
 * each buffer holds whole KV rows of dS (ember_attn_bwd_ds_row_bytes each), and
 * a chunk is as many KV rows as the buffers hold together, so dS can sit in
 * free blocks of the caller's allocator that no single block would hold.
 * Same results, bit for bit, as ember_attn_bwd with the same number of rows
 * per chunk.  Same replaced chain as ember_attn_bwd. */
int ember_attn_bwd_scattered(const float* q, const float* k, const float* v, const float* o,
                             const float* lse, const float* dout, float* dq, float* dk, float* dv,
                             int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                             void* workspace, size_t workspace_bytes, float* const* ds_bufs_host,
                             const size_t* ds_bytes_host, int nbufs, ember_stream_t s);
/* The forward that keeps its scores for the backward (an added option of the
 * same chain as ember_attn_fwd, for a forward whose backward follows while
 * memory allows, e.g. a checkpointed block's re-run): o and lse as
 * ember_attn_fwd, bit for bit; every score it computes, S = Q K^T scale log2(e)
 * before the causal mask, is also written in the dS layout into buffers that
 * together hold all B*Hk KV rows (ember_attn_bwd_ds_row_bytes each, whole rows
 * per buffer, taken in order).  `workspace` >= ember_attn_scores_workspace_bytes
 * holds the row table (enqueued, so it may be reused once the launch has run).
 * EMBER_EWORKSPACE when the buffers hold fewer rows. */
size_t ember_attn_scores_workspace_bytes(int64_t B, int64_t H);
int ember_attn_fwd_scores(const float* q, const float* k, const float* v, float* o, float* lse,
                          int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, float scale,
                          float* const* s_bufs_host, const size_t* s_bytes_host, int nbufs,
                          void* workspace, size_t workspace_bytes, ember_stream_t s);
/* ember_attn_bwd_scattered over the buffers ember_attn_fwd_scores filled (the
 * same buffers, in the same order): the dK/dV pass reads the kept scores
 * instead of computing S again and writes dS over them; one chunk of all rows.
 * dq, dk, dv agree with ember_attn_bwd to fp32 rounding (S is the forward's
 * rounding of the same products). */
int ember_attn_bwd_from_scores(const float* q, const float* k, const float* v, const float* o,
                               const float* lse, const float* dout, float* dq, float* dk,
                               float* dv, int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D,
                               float scale, void* workspace, size_t workspace_bytes,
                               float* const* s_bufs_host, const size_t* s_bytes_host, int nbufs,
                               ember_stream_t s);

/* ------------------------------------------------------ KV cache (inference)
 * Cache layout [B, Hk, S, D] (S = max_seq_len), fp32, as nn::KVCache holds it.
 * ember_kv_write copies src [B,T,Hk,D] into cache rows [pos, pos+T), folding
 * the axis permute into the copy; EMBER_EINVAL unless 0 <= pos and pos+T <= S.
 * Replaces write_kv_kernel / ops::write_kv_inplace (src/ops/kv_cache.cu:13-27,
 * 50-82). */
int ember_kv_write(const float* src, float* cache, int64_t B, int64_t T, int64_t Hk, int64_t D,
                   int64_t S, int64_t pos, ember_stream_t s);
/* out [B, Hk*group, L, D] = cache rows [0, L), KV head h/group for head h.
 * Replaces read_kv_expanded_kernel / ops::read_kv_expanded (kv_cache.cu:29-48,
 * 84-108); the inference attention below reads the cache without it. */
int ember_kv_read_expanded(const float* cache, float* out, int64_t B, int64_t Hk, int64_t group,
                           int64_t L, int64_t D, int64_t S, ember_stream_t s);
/* Attention of q [B,T,H,D] over L keys/values, query t seeing keys
 * j <= pos + t (and j < L); head h reads KV head h / (H/Hk).  Key/value row
 * (b, hk, j) sits at k + b*kv_sb + hk*kv_sh + j*kv_st floats: [B,Hk,S,D] cache
 * (kv_sb = Hk*S*D, kv_sh = S*D, kv_st = D) or [B,T,Hk,D] projections
 * (T*Hk*D, D, Hk*D).  o [B,T,H,D].  D in {64,128}; pointers 16-byte aligned,
 * strides multiples of 4.  Long key ranges are split over workgroups into
 * `workspace` (>= ember_attn_decode_workspace_bytes, 0 = none needed) and
 * merged in a fixed order: deterministic.  Replaces, for the inference
 * forward, read_kv_expanded -> bmm -> mul_scalar -> apply_causal_mask(pos)
 * -> softmax -> bmm (include/ctd/nn/attention.h:66-91). */
size_t ember_attn_decode_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D,
                                         int64_t L);
int ember_attn_decode(const float* q, const float* k, const float* v, float* o, int64_t B,
                      int64_t T, int64_t H, int64_t Hk, int64_t D, int64_t L, int64_t pos,
                      int64_t kv_sb, int64_t kv_sh, int64_t kv_st, float scale, void* workspace,
                      size_t workspace_bytes, ember_stream_t s);

/* ------------------------------------------------------ fused decode step
 * Kernels for calls of at most 8 token rows (decode), each streaming its
 * weights once with the small ops around it folded in.  No counterpart kernel
 * in the reference, which runs the per-module ops of
 * TransformerBlock::forward (include/ctd/nn/transformer_block.h:17-24) one
 * launch each; these compute the same functions.
 *
 * ember_decode_gemv: for s < nseg (1..3), y[s][M, N[s]] = W[s][N[s], K] xn
 * (+ residual[s][M, N[s]] when residual and residual[s] are non-NULL), where
 * xn = x [M, K] when norm_w is NULL, else RMSNorm(x) with weight norm_w [K] and
 * eps (src/ops/norm.cu:17-49 then Linear::forward).  M <= 8, K % 4 == 0,
 * x / W / norm_w 16-byte aligned.  Host arrays W, N, y, residual are read at
 * the call. */
int ember_decode_gemv(const float* x, int64_t M, int64_t K, const float* norm_w, float eps,
                      int nseg, const float* const* W, const int64_t* N, float* const* y,
                      const float* const* residual, ember_stream_t s);
/* out[M, I] = silu(Wg xn) * (Wu xn), xn as above: MLP::forward's gate, up and
 * silu*mul (include/ctd/nn/mlp.h:16-21) with the post-attention RMSNorm. */
int ember_decode_gateup(const float* x, int64_t M, int64_t K, const float* norm_w, float eps,
                        const float* Wg, const float* Wu, int64_t I, float* out,
                        ember_stream_t s);
/* Per token row (b, t) of q [B,T,H,D] and k, v [B,T,Hk,D]: per-head RMSNorm of
 * q and k with q_norm_w / k_norm_w [D] (skipped when NULL), RoPE at position
 * pos + t (freqs_host: D/2 values of ember_rope_freqs_host), rotated q to
 * q_out [B,T,H,D], rotated k and v to cache rows pos + t of cache_k / cache_v
 * [B,Hk,S,D].  Replaces Attention::forward's q_norm/k_norm, the two
 * apply_rope_inplace and the two write_kv_inplace (attention.h:55-72);
 * EMBER_EINVAL unless pos + T <= S. */
int ember_decode_qkv_post(const float* q, const float* k, const float* v, int64_t B, int64_t T,
                          int64_t H, int64_t Hk, int64_t D, const float* q_norm_w,
                          const float* k_norm_w, float eps, const float* freqs_host, int64_t pos,
                          float* q_out, float* cache_k, float* cache_v, int64_t S,
                          ember_stream_t s);
/* ember_decode_qkv_post then ember_attn_decode over the cache, in the
 * attention's launch: q [B,T,H,D] and k, v [B,T,Hk,D] are the raw
 * projections; the normalised, rotated k and v go to cache rows
 * [pos, pos + T) of cache_k / cache_v [B,Hk,S,D], and o [B,T,H,D] is the
 * attention of the normalised, rotated q over cache rows [0, pos + T), query t
 * seeing rows j <= pos + t.  Each workgroup writes, then reads, only the new
 * rows inside its own key split.  T <= 8, D in {64,128}; pointers 16-byte aligned;
 * `workspace` >= ember_attn_decode_workspace_bytes(B, T, H, Hk, D, pos + T).
 * Replaces Attention::forward's q_norm/k_norm, apply_rope_inplace,
 * write_kv_inplace and the attention over the cache (attention.h:55-91);
 * EMBER_EINVAL unless pos + T <= S. */
int ember_attn_decode_qkv(const float* q, const float* k, const float* v, int64_t B, int64_t T,
                          int64_t H, int64_t Hk, int64_t D, const float* q_norm_w,
                          const float* k_norm_w, float eps, const float* freqs_host, int64_t pos,
                          float* cache_k, float* cache_v, int64_t S, float scale, float* o,
                          void* workspace, size_t workspace_bytes, ember_stream_t s);

/* ------------------------------------------------------------- sampling
 * out[r] = index of the largest value of row r of x [rows, n], the first such
 * index on ties, NaNs skipped (0 when x[r,0] is NaN or the row is all NaN):
 * exactly the host scan argmax_cpu (src/core/sampling.cpp:12-19) that greedy
 * sampling (temperature <= 0) runs on the copied logits.  out is device int64. */
int ember_argmax_rows(const float* x, int64_t rows, int64_t n, int64_t* out, ember_stream_t s);
/* The same in two stages for long rows (a vocabulary of logits): slices of each
 * row are reduced by separate workgroups into `workspace` (>=
 * ember_argmax_rows_workspace_bytes; 0 = one stage suffices), then merged.  A
 * smaller or NULL workspace runs ember_argmax_rows.  n < 2^32, rows <= 65535. */
size_t ember_argmax_rows_workspace_bytes(int64_t rows, int64_t n);
int ember_argmax_rows_ws(const float* x, int64_t rows, int64_t n, int64_t* out, void* workspace,
                         size_t workspace_bytes, ember_stream_t s);

/* ---------------------------------------------------- masked cross-entropy
 * Per row r: lse[r] = log sum_v exp(logits[r,v]); loss[0] = sum_r mask[r]*(lse[r]
 * - logits[r,tgt[r]]) / sum_r mask[r] (0 when the mask sums to 0); mask_sum[0].
 * Deterministic (fixed-order reduction in workspace, no atomics).  Replaces
 * ce_masked_fwd/mean kernels (src/ops/loss.cu:253-310); no [N,V] probabilities
 * are written. */
size_t ember_ce_masked_fwd_workspace_bytes(int64_t N);
int ember_ce_masked_fwd(const float* logits, const int64_t* tgt, const float* mask, int64_t N,
                        int64_t V, float* lse, float* loss, float* mask_sum, void* workspace,
                        size_t workspace_bytes, ember_stream_t s);
/* dlogits = (dloss[0] / mask_sum[0]) * mask * (exp(logits - lse) - onehot(tgt))
 * (src/ops/loss.cu:312-329, 382-408), with dloss and mask_sum read on the device.
 * dlogits may equal logits (in place).  Targets outside [0,V) are rejected by
 * the forward's caller; the kernel skips them. */
int ember_ce_masked_bwd(const float* logits, const int64_t* tgt, const float* mask,
                        const float* lse, const float* dloss, const float* mask_sum, int64_t N,
                        int64_t V, float* dlogits, ember_stream_t s);

/* The two halves of ember_ce_masked_fwd, for callers that produce the logits
 * a slice of rows at a time (the chunked LM head + loss): per-row lse[N] and
 * row_loss[N] = mask * (lse - logit[tgt]); then loss[0] = sum(row_loss) /
 * sum(mask) and mask_sum[0] in the same fixed order (row_loss NULL: mask_sum
 * only, loss 0). */
int ember_ce_masked_rows(const float* logits, const int64_t* tgt, const float* mask, int64_t N,
                         int64_t V, float* lse, float* row_loss, ember_stream_t s);
int ember_ce_masked_reduce(const float* row_loss, const float* mask, int64_t N, float* loss,
                           float* mask_sum, ember_stream_t s);

/* Rows whose loss-mask value is 0 add nothing to the loss or to any gradient,
 * so the chunked LM head can compute the others only (added in this build; the
 * reference's ce_masked kernels run every row, loss.cu:253-329):
 *   ember_mask_rows: idx[0 .. *count) = the rows r < N with mask[r] != 0 (NaN
 *     counts as nonzero), ascending; idx holds N entries.
 * The calls below work on a chunk of R rows whose row j is batch row
 * idx[base + j], for j < n = clamp(*count - base, 0, R), all read on the device:
 *   ember_rows_gather: dst [R, H] contiguous; row j = src row idx[base + j]
 *     (src row stride ld) for j < n, zeros for j in [n, round_up(n, 256)) (the
 *     row tile of a GEMM over the chunk), later rows untouched.
 *   ember_rows_scatter: dst row idx[base + j] (stride ld) = src row j, j < n.
 *   ember_ce_masked_rows_idx / _bwd_idx: ember_ce_masked_rows / _bwd over the
 *     chunk's n rows of logits [R, V]; lse is per chunk row, tgt, mask and
 *     row_loss are per batch row (row_loss of other rows is not written). */
int ember_mask_rows(const float* mask, int64_t N, int64_t* idx, int64_t* count,
                    ember_stream_t s);
int ember_rows_gather(const float* src, int64_t ld, int64_t H, const int64_t* idx,
                      const int64_t* count, int64_t base, int64_t R, float* dst,
                      ember_stream_t s);
int ember_rows_scatter(const float* src, int64_t H, const int64_t* idx, const int64_t* count,
                       int64_t base, int64_t R, float* dst, int64_t ld, ember_stream_t s);
int ember_ce_masked_rows_idx(const float* logits, const int64_t* tgt, const float* mask,
                             const int64_t* idx, const int64_t* count, int64_t base, int64_t R,
                             int64_t V, float* lse, float* row_loss, ember_stream_t s);
int ember_ce_masked_bwd_idx(const float* logits, const int64_t* tgt, const float* mask,
                            const float* lse, const int64_t* idx, const int64_t* count,
                            int64_t base, int64_t R, int64_t V, const float* dloss,
                            const float* mask_sum, float* dlogits, ember_stream_t s);

/* -------------------------------------------------------------- embedding
 * out[i,:] = w[ids[i],:] (src/ops/embedding.cu:15-24). */
int ember_embedding_fwd(const int64_t* ids, const float* w, float* out, int64_t n, int64_t H,
                        int64_t V, ember_stream_t s);
/* dw[v,:] (+)= sum over i with ids[i]==v of dy[i,:] (deterministic, no
 * atomics); accumulate=0 zero-fills dw first.  Replaces the atomicAdd scatter
 * of src/ops/embedding.cu:28-39, 71-87.  With a workspace of
 * ember_embedding_bwd_workspace_bytes(n, H, V) (queried on the device that
 * runs the call; 0 when unavailable) the positions are sorted by id and each
 * id's rows summed in fixed-size windows of the sorted order, then across the
 * windows in order, so a much-repeated id costs no more than n/64 workgroups;
 * with none, one workgroup per 128 vocabulary rows sums its hits in
 * increasing i, one after another. */
size_t ember_embedding_bwd_workspace_bytes(int64_t n, int64_t H, int64_t V);
int ember_embedding_bwd(const int64_t* ids, const float* dy, float* dw, int64_t n, int64_t H,
                        int64_t V, int accumulate, void* workspace, size_t workspace_bytes,
                        ember_stream_t s);

/* -------------------------------------------------------------------- SGD
 * p -= lr * g as one fused multiply-add, fma(-lr, g, p) (sgd_step_kernel_f32,
 * src/core/optim.cu:14-20, launched per parameter by SGD::step, optim.cu:29-44,
 * whose p[i] -= lr * g[i] nvcc contracts to one FMA by default). */
int ember_sgd(float* p, const float* g, int64_t n, float lr, ember_stream_t s);

/* ------------------------------------------------------------------ AdamW
 * m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
 * p -= lr * ((m/bc1) / (sqrt(v/bc2) + eps) + wd * p)
 * (adamw_step_kernel_f32, src/core/optim.cu:54-73). */
int ember_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
                float beta2, float eps, float wd, float bc1, float bc2, ember_stream_t s);
/* The same update on at most max_blocks workgroups (0: ember_adamw; each
 * workgroup strides over the array), in a low-register form whose waves fit
 * next to a GEMM's or the attention forward's on one SIMD.  The offloaded
 * optimizer runs its chunk updates this way while the next step's forward
 * holds the GPU.  Results equal ember_adamw's bitwise. */
int ember_adamw_bounded(float* p, const float* g, float* m, float* v, int64_t n, float lr,
                        float beta1, float beta2, float eps, float wd, float bc1, float bc2,
                        int max_blocks, ember_stream_t s);

/* ------------------------------------------------------- grad-norm clip
 * out[0] = sum over tensors of sum(g^2), fixed-order two-stage reduction,
 * all tensors in one launch (plus the final sum).  ptrs/sizes are host
 * arrays of `count` device pointers and lengths; the call copies a table of
 * them into the workspace on stream s.  Replaces the per-parameter
 * sum_sq_kernel_f32 launches + atomicAdd of clip_grad_norm_
 * (src/core/optim.cu:221-239, 262-270). */
size_t ember_sumsq_workspace_bytes(int count);
int ember_sumsq_multi(const float* const* ptrs_host, const int64_t* sizes_host, int count,
                      float* out, void* workspace, size_t workspace_bytes, ember_stream_t s);
/* x *= alpha in place for every tensor of a host list (device pointers and
 * lengths), in one launch; the workspace holds the list's table.  Replaces
 * clip_grad_norm_'s per-parameter scale_kernel_f32 launches
 * (src/core/optim.cu:241-245, 277-289). */
size_t ember_scale_multi_workspace_bytes(int count);
int ember_scale_multi(float* const* ptrs_host, const int64_t* sizes_host, int count, float alpha,
                      void* workspace, size_t workspace_bytes, ember_stream_t s);

#ifdef __cplusplus
}
#endif
#endif /* EMBER_HIP_H */
