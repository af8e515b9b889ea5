/*
 * ref_f32.c -- the reference's scalar fp32 CPU ops as its unit tests write
 * them, composed into a decoder block's forward and backward, the tied LM head
 * with masked cross-entropy, and AdamW.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU baseline that bench.py times beside the
 * GPU (single-threaded, built -O2 by oracle/Makefile) and that
 * tests/test_ref_f32.py checks against the float64 oracle.  The product path
 * never links it.
 *
 * As written (float arithmetic, loop order and accumulation of the source):
 *   rf_mm          mm_cpu, tests/test_bmm.cpp:13-26 (matmul_cpu of
 *                  tests/test_matmul.cpp:14-22 is its ta = tb = 0 case)
 *   rf_rms_norm    rms_norm_cpu, tests/test_norm.cpp:14-23 (double sum of squares)
 *   rf_softmax     softmax_cpu, tests/test_softmax.cpp:14-28 (double sum)
 *   rf_rope        rope_cpu, tests/test_rope.cpp:15-32 (in place, std::pow)
 *   silu           x / (1 + exp(-x)), tests/test_activations.cpp:37
 *   rf_adamw       the closed form of tests/test_autograd.cpp:546-566 with the
 *                  decoupled weight decay of src/core/optim.cu:54-73
 * The reference's tests hold no CPU backward; the backward formulas below are
 * this file's scalar fp32 restatement of the reference kernels' math, each
 * citing the kernel it follows.  The composition follows
 * include/ctd/nn/attention.h:100-143 (repeat_kv, permute, bmm, scale, causal
 * mask, softmax, bmm), mlp.h:16-21, transformer_block.h:28-35.
 */
#include "ref_f32.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static float* fz(size_t n) {
  float* p = (float*)calloc(n ? n : 1, sizeof(float));
  if (!p) abort();
  return p;
}

/* ------------------------------------------------------------ unit-test ops */
void rf_mm(const float* a, const float* b, float* c, int M, int K, int N, int ta, int tb) {
  for (int i = 0; i < M; ++i) {
    for (int j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) {
        float av = ta ? a[k * M + i] : a[i * K + k];
        float bv = tb ? b[j * K + k] : b[k * N + j];
        acc += av * bv;
      }
      c[i * N + j] = acc;
    }
  }
}

void rf_rms_norm(const float* x, const float* w, float* y, int rows, int H, float eps) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * H;
    float* yr = y + (size_t)r * H;
    double acc = 0.0;
    for (int i = 0; i < H; ++i) acc += (double)xr[i] * xr[i];
    float scale = 1.0f / sqrtf((float)(acc / H) + eps);
    for (int i = 0; i < H; ++i) yr[i] = xr[i] * scale * w[i];
  }
}

void rf_softmax(const float* x, float* y, int rows, int N) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * N;
    float* yr = y + (size_t)r * N;
    float m = xr[0];
    for (int i = 1; i < N; ++i) m = fmaxf(m, xr[i]);
    double s = 0.0;
    for (int i = 0; i < N; ++i) {
      yr[i] = expf(xr[i] - m);
      s += yr[i];
    }
    float inv = (float)(1.0 / s);
    for (int i = 0; i < N; ++i) yr[i] *= inv;
  }
}

/* rope_cpu; sign = -1 gives the transpose RopeBackward applies
 * (src/ops/rope.cu:15, 106-118), this file's addition. */
static void rope_signed(float* x, int B, int T, int H, int D, int pos_start, float theta,
                        float sign) {
  const int Dh = D / 2;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t)
      for (int h = 0; h < H; ++h) {
        float* slot = x + (((int64_t)b * T + t) * H + h) * D;
        for (int i = 0; i < Dh; ++i) {
          float inv_freq = powf(theta, -(2.0f * i) / (float)D);
          float ang = (pos_start + t) * inv_freq;
          float c = cosf(ang), s = sign * sinf(ang);
          float a0 = slot[i], a1 = slot[i + Dh];
          slot[i] = a0 * c - a1 * s;
          slot[i + Dh] = a0 * s + a1 * c;
        }
      }
}

void rf_rope(float* x, int B, int T, int H, int D, int pos_start, float theta) {
  rope_signed(x, B, T, H, D, pos_start, theta, 1.0f);
}

static float silu(float v) { return v / (1.0f + expf(-v)); }

void rf_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float b1,
              float b2, float eps, float wd, int step) {
  const float bc1 = 1.0f - powf(b1, (float)step), bc2 = 1.0f - powf(b2, (float)step);
  for (int64_t i = 0; i < n; ++i) {
    m[i] = b1 * m[i] + (1.0f - b1) * g[i];
    v[i] = b2 * v[i] + (1.0f - b2) * g[i] * g[i];
    const float m_hat = m[i] / bc1, v_hat = v[i] / bc2;
    p[i] = p[i] - lr * (m_hat / (sqrtf(v_hat) + eps) + wd * p[i]);
  }
}

/* --------------------------------------------- backward formulas (this file) */
/* RMSNorm backward, src/ops/norm.cu:51-54 and 96-105: s = rsqrt(mean(x^2)+eps),
 * c = sum dy*w*x, dx = s*(dy*w - x*s^2*c/H) (added into dx), dw += dy*x*s. */
static void rms_norm_bwd(const float* dy, const float* x, const float* w, float* dx, float* dw,
                         int rows, int H, float eps) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * H;
    const float* gr = dy + (size_t)r * H;
    double acc = 0.0;
    float c = 0.0f;
    for (int i = 0; i < H; ++i) {
      acc += (double)xr[i] * xr[i];
      c += gr[i] * w[i] * xr[i];
    }
    const float s = 1.0f / sqrtf((float)(acc / H) + eps);
    for (int i = 0; i < H; ++i) {
      dx[(size_t)r * H + i] += s * (gr[i] * w[i] - xr[i] * s * s * c / (float)H);
      dw[i] += gr[i] * xr[i] * s;
    }
  }
}

/* softmax backward, src/ops/softmax.cu:54-80: dx = y*(g - sum(g*y)). */
static void softmax_bwd(const float* y, const float* g, float* dx, int rows, int N) {
  for (int r = 0; r < rows; ++r) {
    const float* yr = y + (size_t)r * N;
    const float* gr = g + (size_t)r * N;
    float dot = 0.0f;
    for (int i = 0; i < N; ++i) dot += gr[i] * yr[i];
    for (int i = 0; i < N; ++i) dx[(size_t)r * N + i] = yr[i] * (gr[i] - dot);
  }
}

/* silu backward, src/ops/elementwise.cu:57-69: g*(s + v*s*(1-s)). */
static float silu_grad(float v) {
  const float s = 1.0f / (1.0f + expf(-v));
  return s + v * s * (1.0f - s);
}

static void add_into(float* y, const float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] += x[i];
}

/* ------------------------------------------------------- one attention head */
/* Forward of one head over [T, D] q/k/v (after repeat_kv and permute):
 * scores = q k^T (bmm), * 1/sqrt(D) (mul_scalar), causal mask to -FLT_MAX
 * (mask.cu:28-52), softmax_cpu, o = P v (bmm).  P [T, T] is kept. */
static void attn_head_fwd(const float* q, const float* k, const float* v, float* P, float* o,
                          int T, int D) {
  const float scale = 1.0f / sqrtf((float)D);
  float* scores = fz((size_t)T * T);
  rf_mm(q, k, scores, T, D, T, 0, 1);
  for (size_t i = 0; i < (size_t)T * T; ++i) scores[i] *= scale;
  for (int r = 0; r < T; ++r)
    for (int c = r + 1; c < T; ++c) scores[(size_t)r * T + c] = -FLT_MAX;
  rf_softmax(scores, P, T, T);
  rf_mm(P, v, o, T, T, D, 0, 0);
  free(scores);
}

/* Its backward (BmmBackward, SoftmaxBackward, CausalMaskBackward,
 * MulScalarBackward): dP = do v^T, dv = P^T do, dS = softmax'(P, dP) masked
 * and scaled, dq = dS k, dk = dS^T q. */
static void attn_head_bwd(const float* q, const float* k, const float* v, const float* P,
                          const float* dout, float* dq, float* dk, float* dv, int T, int D) {
  const float scale = 1.0f / sqrtf((float)D);
  float* dp = fz((size_t)T * T);
  float* ds = fz((size_t)T * T);
  rf_mm(dout, v, dp, T, D, T, 0, 1);
  rf_mm(P, dout, dv, T, T, D, 1, 0);
  softmax_bwd(P, dp, ds, T, T);
  for (int r = 0; r < T; ++r)
    for (int c = 0; c < T; ++c) {
      float* e = ds + (size_t)r * T + c;
      *e = c > r ? 0.0f : *e * scale;
    }
  rf_mm(ds, k, dq, T, T, D, 0, 0);
  rf_mm(ds, q, dk, T, T, D, 1, 0);
  free(dp);
  free(ds);
}

void rf_attention_head(const float* q, const float* k, const float* v, const float* dout,
                       float* o, float* dq, float* dk, float* dv, int T, int D) {
  float* P = fz((size_t)T * T);
  attn_head_fwd(q, k, v, P, o, T, D);
  if (dout) attn_head_bwd(q, k, v, P, dout, dq, dk, dv, T, D);
  free(P);
}

/* ------------------------------------------------------------ the block */
typedef struct {
  float *h1, *q, *k, *v, *q3, *k3, *v3, *probs, *attn, *hres, *h2, *gate, *up, *act;
  float *qpre, *kpre; /* Q/K before QK-Norm */
} acts_t;

static void acts_free(acts_t* a) {
  float** f = (float**)a;
  for (size_t i = 0; i < sizeof(acts_t) / sizeof(float*); ++i) free(f[i]);
  memset(a, 0, sizeof *a);
}

/* Forward of one block over T tokens (B = 1): y = h + mlp(rms2(h)),
 * h = x + attn(rms1(x)).  Keeps the activations in *a. */
static void block_fwd(const rf_block_cfg* c, const rf_block_w* w, const float* x, float* y, int T,
                      acts_t* a) {
  const int d = c->d, H = c->H, Hk = c->Hk, D = c->Dh, I = c->I, G = H / Hk;
  const size_t nq = (size_t)T * H * D, nk = (size_t)T * Hk * D;
  a->h1 = fz((size_t)T * d);
  rf_rms_norm(x, w->ln1, a->h1, T, d, c->eps);
  a->q = fz(nq);
  a->k = fz(nk);
  a->v = fz(nk);
  rf_mm(a->h1, w->wq, a->q, T, d, H * D, 0, 1); /* Linear: x W^T */
  rf_mm(a->h1, w->wk, a->k, T, d, Hk * D, 0, 1);
  rf_mm(a->h1, w->wv, a->v, T, d, Hk * D, 0, 1);
  if (w->qn) { /* QK-Norm over each head's D values */
    a->qpre = fz(nq);
    a->kpre = fz(nk);
    memcpy(a->qpre, a->q, nq * sizeof(float));
    memcpy(a->kpre, a->k, nk * sizeof(float));
    rf_rms_norm(a->qpre, w->qn, a->q, T * H, D, c->eps);
    rf_rms_norm(a->kpre, w->kn, a->k, T * Hk, D, c->eps);
  }
  rf_rope(a->q, 1, T, H, D, 0, c->theta);
  rf_rope(a->k, 1, T, Hk, D, 0, c->theta);
  /* repeat_kv_heads then permute {0,2,1,3}: [H, T, D] */
  a->q3 = fz(nq);
  a->k3 = fz(nq);
  a->v3 = fz(nq);
  for (int h = 0; h < H; ++h)
    for (int t = 0; t < T; ++t)
      for (int e = 0; e < D; ++e) {
        a->q3[((size_t)h * T + t) * D + e] = a->q[((size_t)t * H + h) * D + e];
        a->k3[((size_t)h * T + t) * D + e] = a->k[((size_t)t * Hk + h / G) * D + e];
        a->v3[((size_t)h * T + t) * D + e] = a->v[((size_t)t * Hk + h / G) * D + e];
      }
  a->probs = fz((size_t)H * T * T);
  float* a3 = fz(nq);
  for (int h = 0; h < H; ++h)
    attn_head_fwd(a->q3 + (size_t)h * T * D, a->k3 + (size_t)h * T * D, a->v3 + (size_t)h * T * D,
                  a->probs + (size_t)h * T * T, a3 + (size_t)h * T * D, T, D);
  a->attn = fz(nq); /* permute back: [T, H*D] */
  for (int h = 0; h < H; ++h)
    for (int t = 0; t < T; ++t)
      memcpy(a->attn + ((size_t)t * H + h) * D, a3 + ((size_t)h * T + t) * D, D * sizeof(float));
  free(a3);
  a->hres = fz((size_t)T * d);
  rf_mm(a->attn, w->wo, a->hres, T, H * D, d, 0, 1);
  add_into(a->hres, x, (size_t)T * d);
  a->h2 = fz((size_t)T * d);
  rf_rms_norm(a->hres, w->ln2, a->h2, T, d, c->eps);
  a->gate = fz((size_t)T * I);
  a->up = fz((size_t)T * I);
  a->act = fz((size_t)T * I);
  rf_mm(a->h2, w->wg, a->gate, T, d, I, 0, 1);
  rf_mm(a->h2, w->wu, a->up, T, d, I, 0, 1);
  for (size_t i = 0; i < (size_t)T * I; ++i) a->act[i] = silu(a->gate[i]) * a->up[i];
  rf_mm(a->act, w->wd, y, T, I, d, 0, 1);
  add_into(y, a->hres, (size_t)T * d);
}

/* Backward of block_fwd for upstream dy: dx and the weight gradients (added). */
static void block_bwd(const rf_block_cfg* c, const rf_block_w* w, const float* x, const float* dy,
                      float* dx, rf_block_g* g, int T, const acts_t* a) {
  const int d = c->d, H = c->H, Hk = c->Hk, D = c->Dh, I = c->I, G = H / Hk;
  const size_t nq = (size_t)T * H * D, nk = (size_t)T * Hk * D;
  float* tmp = fz((size_t)d * (I > H * D ? I : H * D));
  /* y = hres + act W_d^T */
  rf_mm(dy, a->act, tmp, d, T, I, 1, 0); /* dW_d = dy^T act (MatmulBackward, matmul.cpp:99-118) */
  add_into(g->wd, tmp, (size_t)d * I);
  float* dact = fz((size_t)T * I);
  rf_mm(dy, w->wd, dact, T, d, I, 0, 0); /* d act = dy W_d */
  float* dgate = fz((size_t)T * I);
  float* dup = fz((size_t)T * I);
  for (size_t i = 0; i < (size_t)T * I; ++i) {
    dgate[i] = dact[i] * a->up[i] * silu_grad(a->gate[i]);
    dup[i] = dact[i] * silu(a->gate[i]);
  }
  rf_mm(dgate, a->h2, tmp, I, T, d, 1, 0);
  add_into(g->wg, tmp, (size_t)I * d);
  rf_mm(dup, a->h2, tmp, I, T, d, 1, 0);
  add_into(g->wu, tmp, (size_t)I * d);
  float* dh2 = fz((size_t)T * d);
  float* t2 = fz((size_t)T * d);
  rf_mm(dgate, w->wg, dh2, T, I, d, 0, 0);
  rf_mm(dup, w->wu, t2, T, I, d, 0, 0);
  add_into(dh2, t2, (size_t)T * d);
  float* dhres = fz((size_t)T * d);
  memcpy(dhres, dy, (size_t)T * d * sizeof(float)); /* AddBackward */
  rms_norm_bwd(dh2, a->hres, w->ln2, dhres, g->ln2, T, d, c->eps);
  /* hres = x + attn W_o^T */
  rf_mm(dhres, a->attn, tmp, d, T, H * D, 1, 0);
  add_into(g->wo, tmp, (size_t)d * H * D);
  float* dattn = fz(nq);
  rf_mm(dhres, w->wo, dattn, T, d, H * D, 0, 0);
  /* attention: per head, dP = dA V^T, dV = P^T dA, dS = softmax'(P, dP) * scale,
   * dQ = dS K, dK = dS^T Q (BmmBackward / SoftmaxBackward / CausalMaskBackward /
   * MulScalarBackward) */
  float* dq3 = fz(nq);
  float* dk3 = fz(nq);
  float* dv3 = fz(nq);
  float* da3 = fz((size_t)T * D);
  for (int h = 0; h < H; ++h) {
    for (int t = 0; t < T; ++t)
      memcpy(da3 + (size_t)t * D, dattn + ((size_t)t * H + h) * D, D * sizeof(float));
    const size_t o = (size_t)h * T * D;
    attn_head_bwd(a->q3 + o, a->k3 + o, a->v3 + o, a->probs + (size_t)h * T * T, da3, dq3 + o,
                  dk3 + o, dv3 + o, T, D);
  }
  /* permute back; repeat_kv backward sums each group (repeat_kv.cu:29-43) */
  float* dq = fz(nq);
  float* dk = fz(nk);
  float* dv = fz(nk);
  for (int h = 0; h < H; ++h)
    for (int t = 0; t < T; ++t)
      for (int e = 0; e < D; ++e) {
        dq[((size_t)t * H + h) * D + e] = dq3[((size_t)h * T + t) * D + e];
        dk[((size_t)t * Hk + h / G) * D + e] += dk3[((size_t)h * T + t) * D + e];
        dv[((size_t)t * Hk + h / G) * D + e] += dv3[((size_t)h * T + t) * D + e];
      }
  rope_signed(dq, 1, T, H, D, 0, c->theta, -1.0f); /* RopeBackward: rotate by -theta */
  rope_signed(dk, 1, T, Hk, D, 0, c->theta, -1.0f);
  if (w->qn) {
    float* t3 = fz(nq);
    rms_norm_bwd(dq, a->qpre, w->qn, t3, g->qn, T * H, D, c->eps);
    memcpy(dq, t3, nq * sizeof(float));
    memset(t3, 0, nq * sizeof(float));
    rms_norm_bwd(dk, a->kpre, w->kn, t3, g->kn, T * Hk, D, c->eps);
    memcpy(dk, t3, nk * sizeof(float));
    free(t3);
  }
  rf_mm(dq, a->h1, tmp, H * D, T, d, 1, 0);
  add_into(g->wq, tmp, (size_t)H * D * d);
  rf_mm(dk, a->h1, tmp, Hk * D, T, d, 1, 0);
  add_into(g->wk, tmp, (size_t)Hk * D * d);
  rf_mm(dv, a->h1, tmp, Hk * D, T, d, 1, 0);
  add_into(g->wv, tmp, (size_t)Hk * D * d);
  float* dh1 = fz((size_t)T * d);
  rf_mm(dq, w->wq, dh1, T, H * D, d, 0, 0);
  rf_mm(dk, w->wk, t2, T, Hk * D, d, 0, 0);
  add_into(dh1, t2, (size_t)T * d);
  rf_mm(dv, w->wv, t2, T, Hk * D, d, 0, 0);
  add_into(dh1, t2, (size_t)T * d);
  memcpy(dx, dhres, (size_t)T * d * sizeof(float));
  rms_norm_bwd(dh1, x, w->ln1, dx, g->ln1, T, d, c->eps);
  float* fr[] = {tmp, dact, dgate, dup, dh2, t2, dhres, dattn, dq3, dk3, dv3, da3, dq, dk, dv,
                 dh1};
  for (size_t i = 0; i < sizeof fr / sizeof fr[0]; ++i) free(fr[i]);
}

void rf_block_forward(const rf_block_cfg* c, const rf_block_w* w, const float* x, float* y,
                      int T) {
  acts_t a;
  memset(&a, 0, sizeof a);
  block_fwd(c, w, x, y, T, &a);
  acts_free(&a);
}

void rf_block_fwd_bwd(const rf_block_cfg* c, const rf_block_w* w, const float* x, const float* dy,
                      float* y, float* dx, rf_block_g* g, int T, int checkpoint) {
  acts_t a;
  memset(&a, 0, sizeof a);
  if (checkpoint) {
    /* CheckpointNode (autograd.cu:327-363): the forward keeps only x, the
     * backward runs the block's forward again before its backward */
    rf_block_forward(c, w, x, y, T);
    float* y2 = fz((size_t)T * c->d);
    block_fwd(c, w, x, y2, T, &a);
    free(y2);
  } else {
    block_fwd(c, w, x, y, T, &a);
  }
  block_bwd(c, w, x, dy, dx, g, T, &a);
  acts_free(&a);
}

/* Tied LM head and masked mean CE over n rows of h [n, d] with E [V, d]:
 * logits = h E^T (Linear), per row softmax_cpu, loss = sum mask*(-log p[t]) /
 * sum mask, dlogits = (p - onehot) * mask / sum mask (the closed form of
 * src/ops/loss.cu:253-329), dh = dlogits E, dE += dlogits^T h.  Returns the
 * loss. */
float rf_lm_head_ce(const float* h, const float* E, const int64_t* tgt, const float* mask,
                    float* dh, float* dE, int n, int d, int V) {
  float* logits = fz((size_t)n * V);
  float* p = fz((size_t)n * V);
  rf_mm(h, E, logits, n, d, V, 0, 1);
  rf_softmax(logits, p, n, V);
  float msum = 0.0f;
  for (int r = 0; r < n; ++r) msum += mask[r];
  double loss = 0.0;
  for (int r = 0; r < n; ++r) {
    loss += (double)mask[r] * -log((double)p[(size_t)r * V + tgt[r]]);
    const float k = msum > 0.0f ? mask[r] / msum : 0.0f;
    for (int j = 0; j < V; ++j) {
      float* e = p + (size_t)r * V + j;
      *e = (*e - (j == tgt[r] ? 1.0f : 0.0f)) * k;
    }
  }
  rf_mm(p, E, dh, n, V, d, 0, 0);
  float* t = fz((size_t)V * d);
  rf_mm(p, h, t, V, n, d, 1, 0);
  add_into(dE, t, (size_t)V * d);
  free(t);
  free(logits);
  free(p);
  return msum > 0.0f ? (float)(loss / msum) : 0.0f;
}
