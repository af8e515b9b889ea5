/*
 * ember_oracle.h -- CPU restatement of emberlm's training math (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker for the HIP path, never part of it: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  Every
 * function restates the reference algorithm it cites, in double precision
 * (the reference's own CPU test oracles accumulate in double, e.g.
 * tests/test_norm.cpp:19, tests/test_softmax.cpp:20).  Layouts are the
 * reference's: row-major, contiguous, [B,T,H,D] for per-head tensors.
 *
 * Parity pins (tests/test_oracle.py): reference KATs, numpy/scipy/torch-CPU
 * library routines, closed forms and central finite differences.
 */
#ifndef EMBER_ORACLE_H
#define EMBER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C[M,N] = op(A)[M,K] . op(B)[K,N]; A stored [M,K] (or [K,M] if transa),
 * B stored [K,N] (or [N,K] if transb).  Follows matmul_cpu
 * (tests/test_matmul.cpp:14-22) and the transpose flags of ops::matmul
 * (src/ops/matmul.cpp:33-47). beta=0 overwrites, beta=1 accumulates. */
void orc_matmul(const double* a, const double* b, double* c, int64_t M, int64_t N,
                int64_t K, int transa, int transb, double beta);

/* Strided batched variant of the above (tests/test_bmm.cpp:13-26). */
void orc_bmm(const double* a, const double* b, double* c, int64_t batch, int64_t M,
             int64_t N, int64_t K, int transa, int transb);

/* y = x * 1/sqrt(mean(x^2)+eps) * w per row (tests/test_norm.cpp:14-23). */
void orc_rmsnorm_fwd(const double* x, const double* w, double* y, int64_t rows,
                     int64_t H, double eps);
/* dx, dw (dw overwritten, summed over rows) from src/ops/norm.cu:51-106. */
void orc_rmsnorm_bwd(const double* dy, const double* x, const double* w, double* dx,
                     double* dw, int64_t rows, int64_t H, double eps);

/* RoPE frequency for pair i, in float exactly as src/ops/rope.cu:37-46
 * computes it (llama3 scaling when factor > 1). */
float orc_rope_freq(int i, int D, float theta, float factor, float low_freq_factor,
                    float high_freq_factor, int original_max_pos);
/* y = R(sign*angle) x over [B,T,H,D], pairs (i, i+D/2) (tests/test_rope.cpp:15-32,
 * src/ops/rope.cu:17-56).  angle = float(pos0+t) * freq rounded to float as in
 * rope.cu:49; cos/sin evaluated in double. */
void orc_rope(const double* x, double* y, int64_t B, int64_t T, int64_t H, int64_t D,
              int64_t pos0, float theta, double sign, float factor, float low_freq_factor,
              float high_freq_factor, int original_max_pos);

/* Row softmax (tests/test_softmax.cpp:14-28) and its backward
 * dx = y*(g - sum(g*y)) (src/ops/softmax.cu:54-80). */
void orc_softmax_fwd(const double* x, double* y, int64_t rows, int64_t N);
void orc_softmax_bwd(const double* y, const double* g, double* dx, int64_t rows, int64_t N);

/* out = (k > q0+q) ? fill : in over rows of [*, Tq, Tk] (src/ops/mask.cu:28-52);
 * backward writes 0 at masked positions. */
void orc_causal_mask(const double* in, double* out, int64_t rows, int64_t Tq, int64_t Tk,
                     int64_t q0, double fill);

/* [BT, Hk, D] -> [BT, Hk*group, D] (src/ops/repeat_kv.cu:16-26) and the group
 * sum backward (repeat_kv.cu:29-43). */
void orc_repeat_kv(const double* x, double* y, int64_t BT, int64_t Hk, int64_t group,
                   int64_t D);
void orc_repeat_kv_sum(const double* y, double* x, int64_t BT, int64_t Hk, int64_t group,
                       int64_t D);

/* Generic rank<=6 permutation y.shape[i] = x.shape[perm[i]] (src/ops/permute.cu:20-38). */
void orc_permute(const double* x, double* y, int ndim, const int64_t* shape,
                 const int* perm);

/* silu(x) = x/(1+exp(-x)) (tests/test_activations.cpp:37) and
 * g * (s + x s (1-s)) (src/ops/elementwise.cu:57-69). */
void orc_silu(const double* x, double* y, int64_t n);
void orc_silu_bwd(const double* x, const double* g, double* dx, int64_t n);

/* Masked CE (src/ops/loss.cu:253-310): per row lse = max + log(sum exp);
 * returns sum(mask*(lse - logit[tgt])) / sum(mask) (0 if sum(mask)==0).
 * lse_out[N] and *mask_sum_out are optional. */
double orc_ce_masked_fwd(const double* logits, const int64_t* tgt, const double* mask,
                         int64_t N, int64_t V, double* lse_out, double* mask_sum_out);
/* dlogits = (dy/sum(mask)) * mask * (softmax - onehot) (loss.cu:312-329, 382-408). */
void orc_ce_masked_bwd(const double* logits, const int64_t* tgt, const double* mask,
                       int64_t N, int64_t V, double dy, double* dlogits);

/* out[i,:] = w[ids[i],:]; dw[v,:] = sum_{i: ids[i]==v} dy[i,:] (src/ops/embedding.cu:15-39). */
void orc_embedding_fwd(const int64_t* ids, const double* w, double* out, int64_t n,
                       int64_t H);
void orc_embedding_bwd(const int64_t* ids, const double* dy, double* dw, int64_t n,
                       int64_t H, int64_t V);

/* One AdamW element update (src/core/optim.cu:54-73). */
void orc_adamw(double* p, const double* g, double* m, double* v, int64_t n, double lr,
               double beta1, double beta2, double eps, double wd, double bc1, double bc2);

/* Causal GQA attention as composed in include/ctd/nn/attention.h:100-143:
 * scores = (Q K^T) * scale, causal mask, softmax, P V; head h reads KV head
 * h / (H/Hk).  q,o [B,T,H,D]; k,v [B,T,Hk,D]; lse [B,H,T] (optional). */
void orc_attention_fwd(const double* q, const double* k, const double* v, double* o,
                       double* lse, int64_t B, int64_t T, int64_t H, int64_t Hk,
                       int64_t D, double scale);
/* Chain rule through the same composition: bmm, mul_scalar, mask, softmax,
 * bmm, repeat_kv (src/ops/matmul.cpp:99-118, softmax.cu:54-80, mask.cu:41-52,
 * repeat_kv.cu:29-43).  dk/dv summed over each KV head's query group. */
void orc_attention_bwd(const double* q, const double* k, const double* v,
                       const double* dout, double* dq, double* dk, double* dv, int64_t B,
                       int64_t T, int64_t H, int64_t Hk, int64_t D, double scale);

/* The attention of Attention::forward with a KV cache (include/ctd/nn/attention.h:43-97):
 * scores = (Q K^T) * scale over L keys, apply_causal_mask(q0 = pos) hides key
 * j > pos + t (src/ops/mask.cu:15-37), softmax, P V.  q,o [B,T,H,D]; k,v
 * [B,L,Hk,D] (key rows in projection layout); head h reads KV head h/(H/Hk). */
void orc_attention_offset(const double* q, const double* k, const double* v, double* o,
                          int64_t B, int64_t T, int64_t L, int64_t H, int64_t Hk, int64_t D,
                          int64_t pos, double scale);

/* Decoder block / model shapes (include/ctd/nn/model.h:19-37). */
typedef struct {
  int64_t vocab;   /* V */
  int64_t hidden;  /* d */
  int64_t inter;   /* I */
  int64_t layers;
  int64_t heads;   /* H */
  int64_t kv_heads;/* Hk */
  int64_t head_dim;/* D */
  double eps;
  float theta;
  float rope_factor;     /* 0 = vanilla RoPE */
  float rope_low_freq;
  float rope_high_freq;
  int rope_orig_max_pos;
  int qk_norm;
} orc_cfg;

/* Block weights in the reference's collect_parameters order
 * (src/nn/model.cpp:81-94): input_layernorm, q, k, v, o, [q_norm, k_norm],
 * post_attention_layernorm, gate, up, down. */
enum { ORC_W_IN_NORM = 0, ORC_W_Q, ORC_W_K, ORC_W_V, ORC_W_O, ORC_W_Q_NORM, ORC_W_K_NORM,
       ORC_W_POST_NORM, ORC_W_GATE, ORC_W_UP, ORC_W_DOWN, ORC_W_COUNT };

/* y = h + mlp(rms2(h)), h = x + attn(rms1(x))  (include/ctd/nn/transformer_block.h:28-35),
 * x,y [B,T,d].  w[ORC_W_*]; q_norm/k_norm ignored unless cfg->qk_norm. */
void orc_block_fwd(const orc_cfg* cfg, const double* const* w, const double* x, double* y,
                   int64_t B, int64_t T);
/* Backward of orc_block_fwd for upstream dy: dx and dw[ORC_W_*] (overwritten). */
void orc_block_bwd(const orc_cfg* cfg, const double* const* w, const double* x,
                   const double* dy, double* dx, double* const* dw, int64_t B, int64_t T);

/* Number of parameter tensors of a model (collect_parameters order,
 * src/nn/model.cpp:63-100): embed, per layer 9 (11 with qk_norm), final norm. */
int64_t orc_model_num_params(const orc_cfg* cfg);
/* Full training loss of Model::forward_train_masked (include/ctd/nn/model.h:170-206)
 * with the tied LM head; grads (if non-NULL) in the same order as params. */
double orc_model_loss(const orc_cfg* cfg, const double* const* params, double* const* grads,
                      const int64_t* ids, const int64_t* targets, const double* mask,
                      int64_t B, int64_t T);

/* Logits [B,T,V] of Model::forward without a cache (include/ctd/nn/model.h:152-163):
 * embedding, blocks, final RMSNorm, tied head. */
void orc_model_logits(const orc_cfg* cfg, const double* const* params, const int64_t* ids,
                      double* logits, int64_t B, int64_t T);

#ifdef __cplusplus
}
#endif
#endif
