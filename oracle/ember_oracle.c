/*
 * ember_oracle.c -- CPU restatement of emberlm's training math.
 *
 * TEST INFRASTRUCTURE ONLY.  Loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; the product path never links it.
 * Each function cites the reference file:line whose algorithm it restates.
 * Arithmetic is double precision throughout except where the reference's own
 * float rounding is part of the algorithm (RoPE angle, rope.cu:37-49).
 */
#include "ember_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static void* xcalloc(size_t n, size_t sz) {
  void* p = calloc(n ? n : 1, sz);
  if (!p) abort();
  return p;
}
#define DALLOC(n) ((double*)xcalloc((size_t)(n), sizeof(double)))

/* ---------------------------------------------------------------- GEMM */
/* matmul_cpu, tests/test_matmul.cpp:14-22, with the transpose flags of
 * src/ops/matmul.cpp:33-47 (op(A) is [M,K], op(B) is [K,N]). */
void orc_matmul(const double* a, const double* b, double* c, int64_t M, int64_t N,
                int64_t K, int transa, int transb, double beta) {
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double av = transa ? a[k * M + i] : a[i * K + k];
        const double bv = transb ? b[j * K + k] : b[k * N + j];
        acc += av * bv;
      }
      c[i * N + j] = (beta != 0.0 ? beta * c[i * N + j] : 0.0) + acc;
    }
  }
}

/* mm_cpu per batch, tests/test_bmm.cpp:13-26; ops::bmm (src/ops/matmul.cpp:51-93). */
void orc_bmm(const double* a, const double* b, double* c, int64_t batch, int64_t M,
             int64_t N, int64_t K, int transa, int transb) {
  for (int64_t s = 0; s < batch; ++s)
    orc_matmul(a + s * M * K, b + s * K * N, c + s * M * N, M, N, K, transa, transb, 0.0);
}

/* ------------------------------------------------------------- RMSNorm */
/* rms_norm_cpu, tests/test_norm.cpp:14-23. */
void orc_rmsnorm_fwd(const double* x, const double* w, double* y, int64_t rows,
                     int64_t H, double eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * H;
    double acc = 0.0;
    for (int64_t i = 0; i < H; ++i) acc += xr[i] * xr[i];
    const double s = 1.0 / sqrt(acc / (double)H + eps);
    for (int64_t i = 0; i < H; ++i) y[r * H + i] = xr[i] * s * w[i];
  }
}

/* src/ops/norm.cu:51-54 and 96-105:
 *   s = rsqrt(mean(x^2)+eps), c = sum_j dy_j w_j x_j,
 *   dx_i = s (dy_i w_i - x_i s^2 c / H),  dw_i = sum_rows dy_i x_i s. */
void orc_rmsnorm_bwd(const double* dy, const double* x, const double* w, double* dx,
                     double* dw, int64_t rows, int64_t H, double eps) {
  if (dw) memset(dw, 0, (size_t)H * sizeof(double));
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * H;
    const double* gr = dy + r * H;
    double acc = 0.0, c = 0.0;
    for (int64_t i = 0; i < H; ++i) acc += xr[i] * xr[i];
    const double s = 1.0 / sqrt(acc / (double)H + eps);
    for (int64_t i = 0; i < H; ++i) c += gr[i] * w[i] * xr[i];
    for (int64_t i = 0; i < H; ++i) {
      if (dx) dx[r * H + i] = s * (gr[i] * w[i] - xr[i] * s * s * c / (double)H);
      if (dw) dw[i] += gr[i] * xr[i] * s;
    }
  }
}

/* ---------------------------------------------------------------- RoPE */
/* Frequency of pair i (src/ops/rope.cu:37-46), evaluated in float as the
 * reference does; llama3 band split on wavelength when factor > 1. */
float orc_rope_freq(int i, int D, float theta, float factor, float low_freq_factor,
                    float high_freq_factor, int original_max_pos) {
  const float base = powf(theta, -(2.0f * (float)i) / (float)D);
  float freq = base;
  if (factor > 1.0f) {
    const float low_wl = (float)original_max_pos / low_freq_factor;
    const float high_wl = (float)original_max_pos / high_freq_factor;
    const float wavelen = 6.2831853f / base;
    if (wavelen > low_wl) {
      freq = base / factor;
    } else if (wavelen > high_wl) {
      const float smooth = (wavelen - high_wl) / (low_wl - high_wl);
      freq = (1.0f - smooth) * base + smooth * (base / factor);
    }
  }
  return freq;
}

/* rope_cpu, tests/test_rope.cpp:15-32; sign=-1 is the transpose used by
 * RopeBackward (src/ops/rope.cu:15, 106-118). */
void orc_rope(const double* x, double* y, int64_t B, int64_t T, int64_t H, int64_t D,
              int64_t pos0, float theta, double sign, float factor, float low_freq_factor,
              float high_freq_factor, int original_max_pos) {
  const int64_t Dh = D / 2;
  float* freq = (float*)xcalloc((size_t)Dh, sizeof(float));
  for (int64_t i = 0; i < Dh; ++i)
    freq[i] = orc_rope_freq((int)i, (int)D, theta, factor, low_freq_factor, high_freq_factor,
                            original_max_pos);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h) {
        const int64_t base = ((b * T + t) * H + h) * D;
        for (int64_t i = 0; i < Dh; ++i) {
          const float ang = (float)(pos0 + t) * freq[i]; /* rope.cu:49, float product */
          const double c = cos((double)ang), s = sign * sin((double)ang);
          const double a0 = x[base + i], a1 = x[base + i + Dh];
          y[base + i] = a0 * c - a1 * s;
          y[base + i + Dh] = a0 * s + a1 * c;
        }
      }
  free(freq);
}

/* ------------------------------------------------------------- Softmax */
/* softmax_cpu, tests/test_softmax.cpp:14-28. */
void orc_softmax_fwd(const double* x, double* y, int64_t rows, int64_t N) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * N;
    double* yr = y + r * N;
    double m = xr[0];
    for (int64_t i = 1; i < N; ++i) m = xr[i] > m ? xr[i] : m;
    double s = 0.0;
    for (int64_t i = 0; i < N; ++i) {
      yr[i] = exp(xr[i] - m);
      s += yr[i];
    }
    for (int64_t i = 0; i < N; ++i) yr[i] /= s;
  }
}

/* src/ops/softmax.cu:54-80. */
void orc_softmax_bwd(const double* y, const double* g, double* dx, int64_t rows, int64_t N) {
  for (int64_t r = 0; r < rows; ++r) {
    double s = 0.0;
    for (int64_t i = 0; i < N; ++i) s += g[r * N + i] * y[r * N + i];
    for (int64_t i = 0; i < N; ++i) dx[r * N + i] = y[r * N + i] * (g[r * N + i] - s);
  }
}

/* src/ops/mask.cu:28-52: rows of a [*, Tq, Tk] tensor, query index r % Tq. */
void orc_causal_mask(const double* in, double* out, int64_t rows, int64_t Tq, int64_t Tk,
                     int64_t q0, double fill) {
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t q = r % Tq;
    for (int64_t k = 0; k < Tk; ++k) out[r * Tk + k] = (k > q0 + q) ? fill : in[r * Tk + k];
  }
}

/* ------------------------------------------------------- GQA / permute */
/* src/ops/repeat_kv.cu:16-26: output head h reads input head h / group. */
void orc_repeat_kv(const double* x, double* y, int64_t BT, int64_t Hk, int64_t group,
                   int64_t D) {
  for (int64_t bt = 0; bt < BT; ++bt)
    for (int64_t h = 0; h < Hk * group; ++h)
      memcpy(y + (bt * Hk * group + h) * D, x + (bt * Hk + h / group) * D,
             (size_t)D * sizeof(double));
}

/* src/ops/repeat_kv.cu:29-43. */
void orc_repeat_kv_sum(const double* y, double* x, int64_t BT, int64_t Hk, int64_t group,
                       int64_t D) {
  for (int64_t bt = 0; bt < BT; ++bt)
    for (int64_t h = 0; h < Hk; ++h)
      for (int64_t d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int64_t j = 0; j < group; ++j) acc += y[((bt * Hk * group) + h * group + j) * D + d];
        x[(bt * Hk + h) * D + d] = acc;
      }
}

/* src/ops/permute.cu:20-38: y index -> x index via the permuted strides. */
void orc_permute(const double* x, double* y, int ndim, const int64_t* shape,
                 const int* perm) {
  int64_t xstr[8], yshape[8], n = 1;
  xstr[ndim - 1] = 1;
  for (int i = ndim - 2; i >= 0; --i) xstr[i] = xstr[i + 1] * shape[i + 1];
  for (int i = 0; i < ndim; ++i) {
    yshape[i] = shape[perm[i]];
    n *= shape[i];
  }
  for (int64_t idx = 0; idx < n; ++idx) {
    int64_t rem = idx, src = 0;
    for (int i = ndim - 1; i >= 0; --i) {
      const int64_t c = rem % yshape[i];
      rem /= yshape[i];
      src += c * xstr[perm[i]];
    }
    y[idx] = x[src];
  }
}

/* ------------------------------------------------------------ SwiGLU */
/* tests/test_activations.cpp:37. */
void orc_silu(const double* x, double* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] / (1.0 + exp(-x[i]));
}

/* src/ops/elementwise.cu:57-69. */
void orc_silu_bwd(const double* x, const double* g, double* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double s = 1.0 / (1.0 + exp(-x[i]));
    dx[i] = g[i] * (s + x[i] * s * (1.0 - s));
  }
}

/* ------------------------------------------------------- Masked CE */
static double row_lse(const double* lr, int64_t V) {
  double m = -DBL_MAX, s = 0.0;
  for (int64_t i = 0; i < V; ++i) m = lr[i] > m ? lr[i] : m;
  for (int64_t i = 0; i < V; ++i) s += exp(lr[i] - m);
  return m + log(s); /* loss.cu:291 */
}

/* src/ops/loss.cu:253-310. */
double orc_ce_masked_fwd(const double* logits, const int64_t* tgt, const double* mask,
                         int64_t N, int64_t V, double* lse_out, double* mask_sum_out) {
  double loss = 0.0, ms = 0.0;
  for (int64_t r = 0; r < N; ++r) {
    const double lse = row_lse(logits + r * V, V);
    if (lse_out) lse_out[r] = lse;
    loss += mask[r] * (lse - logits[r * V + tgt[r]]);
    ms += mask[r];
  }
  if (mask_sum_out) *mask_sum_out = ms;
  return ms > 0.0 ? loss / ms : 0.0;
}

/* src/ops/loss.cu:312-329 with alpha = dy / sum(mask) (loss.cu:389-399). */
void orc_ce_masked_bwd(const double* logits, const int64_t* tgt, const double* mask,
                       int64_t N, int64_t V, double dy, double* dlogits) {
  double ms = 0.0;
  for (int64_t r = 0; r < N; ++r) ms += mask[r];
  const double alpha = dy / ms;
  for (int64_t r = 0; r < N; ++r) {
    const double lse = row_lse(logits + r * V, V);
    const double sc = alpha * mask[r];
    for (int64_t i = 0; i < V; ++i) {
      double p = exp(logits[r * V + i] - lse);
      if (i == tgt[r]) p -= 1.0;
      dlogits[r * V + i] = sc * p;
    }
  }
}

/* --------------------------------------------------------- Embedding */
/* src/ops/embedding.cu:15-24. */
void orc_embedding_fwd(const int64_t* ids, const double* w, double* out, int64_t n,
                       int64_t H) {
  for (int64_t r = 0; r < n; ++r) memcpy(out + r * H, w + ids[r] * H, (size_t)H * sizeof(double));
}

/* src/ops/embedding.cu:28-39, 71-87 (fresh zeroed [V,H], scatter-add). */
void orc_embedding_bwd(const int64_t* ids, const double* dy, double* dw, int64_t n,
                       int64_t H, int64_t V) {
  memset(dw, 0, (size_t)(V * H) * sizeof(double));
  for (int64_t r = 0; r < n; ++r)
    for (int64_t i = 0; i < H; ++i) dw[ids[r] * H + i] += dy[r * H + i];
}

/* ------------------------------------------------------------- AdamW */
/* src/core/optim.cu:54-73 (decoupled decay uses the pre-update p). */
void orc_adamw(double* p, const double* g, double* m, double* v, int64_t n, double lr,
               double beta1, double beta2, double eps, double wd, double bc1, double bc2) {
  for (int64_t i = 0; i < n; ++i) {
    const double mi = beta1 * m[i] + (1.0 - beta1) * g[i];
    const double vi = beta2 * v[i] + (1.0 - beta2) * g[i] * g[i];
    m[i] = mi;
    v[i] = vi;
    const double upd = (mi / bc1) / (sqrt(vi / bc2) + eps);
    p[i] = p[i] - lr * (upd + wd * p[i]);
  }
}

/* --------------------------------------------------------- Attention */
/* Probabilities of one (b,h) row block: P[t][u] for u<=t, from the
 * composition in include/ctd/nn/attention.h:130-137.  Masked entries are
 * exactly 0 (exp(-FLT_MAX - max) underflows, src/ops/mask.cu:37). */
static void attn_probs(const double* q, const double* k, double* P, double* lse, int64_t b,
                       int64_t h, int64_t kvh, int64_t T, int64_t H, int64_t Hk, int64_t D,
                       double scale) {
  for (int64_t t = 0; t < T; ++t) {
    const double* qt = q + ((b * T + t) * H + h) * D;
    double m = -DBL_MAX;
    for (int64_t u = 0; u <= t; ++u) {
      const double* ku = k + ((b * T + u) * Hk + kvh) * D;
      double s = 0.0;
      for (int64_t d = 0; d < D; ++d) s += qt[d] * ku[d];
      s *= scale;
      P[t * T + u] = s;
      m = s > m ? s : m;
    }
    double sum = 0.0;
    for (int64_t u = 0; u <= t; ++u) {
      P[t * T + u] = exp(P[t * T + u] - m);
      sum += P[t * T + u];
    }
    for (int64_t u = 0; u <= t; ++u) P[t * T + u] /= sum;
    for (int64_t u = t + 1; u < T; ++u) P[t * T + u] = 0.0;
    if (lse) lse[(b * H + h) * T + t] = m + log(sum);
  }
}

void orc_attention_fwd(const double* q, const double* k, const double* v, double* o,
                       double* lse, int64_t B, int64_t T, int64_t H, int64_t Hk,
                       int64_t D, double scale) {
  const int64_t group = H / Hk;
  double* P = DALLOC(T * T);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t kvh = h / group;
      attn_probs(q, k, P, lse, b, h, kvh, T, H, Hk, D, scale);
      for (int64_t t = 0; t < T; ++t)
        for (int64_t d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t u = 0; u <= t; ++u) acc += P[t * T + u] * v[((b * T + u) * Hk + kvh) * D + d];
          o[((b * T + t) * H + h) * D + d] = acc;
        }
    }
  free(P);
}

void orc_attention_bwd(const double* q, const double* k, const double* v,
                       const double* dout, double* dq, double* dk, double* dv, int64_t B,
                       int64_t T, int64_t H, int64_t Hk, int64_t D, double scale) {
  const int64_t group = H / Hk;
  double* P = DALLOC(T * T);
  double* dS = DALLOC(T * T);
  memset(dk, 0, (size_t)(B * T * Hk * D) * sizeof(double));
  memset(dv, 0, (size_t)(B * T * Hk * D) * sizeof(double));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t kvh = h / group;
      attn_probs(q, k, P, NULL, b, h, kvh, T, H, Hk, D, scale);
      for (int64_t t = 0; t < T; ++t) {
        const double* dot = dout + ((b * T + t) * H + h) * D;
        /* dP = dO V^T (PV BmmBackward, matmul.cpp:99-102) */
        double rs = 0.0;
        for (int64_t u = 0; u <= t; ++u) {
          const double* vu = v + ((b * T + u) * Hk + kvh) * D;
          double dp = 0.0;
          for (int64_t d = 0; d < D; ++d) dp += dot[d] * vu[d];
          dS[t * T + u] = dp;
          rs += dp * P[t * T + u];
        }
        /* softmax backward (softmax.cu:54-80); masked entries have P=0 so
         * the mask backward (mask.cu:41-52) zeroes them; then MulScalar. */
        for (int64_t u = 0; u <= t; ++u) dS[t * T + u] = P[t * T + u] * (dS[t * T + u] - rs) * scale;
        /* dV_h = P^T dO, summed over the group (repeat_kv.cu:29-43) */
        for (int64_t u = 0; u <= t; ++u) {
          double* dvu = dv + ((b * T + u) * Hk + kvh) * D;
          for (int64_t d = 0; d < D; ++d) dvu[d] += P[t * T + u] * dot[d];
        }
      }
      for (int64_t t = 0; t < T; ++t) {
        double* dqt = dq + ((b * T + t) * H + h) * D;
        const double* qt = q + ((b * T + t) * H + h) * D;
        for (int64_t d = 0; d < D; ++d) dqt[d] = 0.0;
        for (int64_t u = 0; u <= t; ++u) {
          const double ds = dS[t * T + u];
          const double* ku = k + ((b * T + u) * Hk + kvh) * D;
          double* dku = dk + ((b * T + u) * Hk + kvh) * D;
          for (int64_t d = 0; d < D; ++d) {
            dqt[d] += ds * ku[d];  /* dQ = dS K */
            dku[d] += ds * qt[d];  /* dK = dS^T Q */
          }
        }
      }
    }
  free(P);
  free(dS);
}

/* ------------------------------------------------------ Decoder block */
typedef struct {
  double *h1, *q, *k, *v, *qn, *kn, *qr, *kr, *attn, *h, *h2, *g, *u, *s, *m;
} block_acts;

static void block_forward_acts(const orc_cfg* c, const double* const* w, const double* x,
                               double* y, int64_t B, int64_t T, block_acts* A) {
  const int64_t N = B * T, d = c->hidden, I = c->inter, H = c->heads, Hk = c->kv_heads,
                D = c->head_dim;
  A->h1 = DALLOC(N * d);
  A->q = DALLOC(N * H * D);
  A->k = DALLOC(N * Hk * D);
  A->v = DALLOC(N * Hk * D);
  A->qn = DALLOC(N * H * D);
  A->kn = DALLOC(N * Hk * D);
  A->qr = DALLOC(N * H * D);
  A->kr = DALLOC(N * Hk * D);
  A->attn = DALLOC(N * H * D);
  A->h = DALLOC(N * d);
  A->h2 = DALLOC(N * d);
  A->g = DALLOC(N * I);
  A->u = DALLOC(N * I);
  A->s = DALLOC(N * I);
  A->m = DALLOC(N * I);
  double* a = DALLOC(N * d);
  double* dn = DALLOC(N * d);

  /* transformer_block.h:29 */
  orc_rmsnorm_fwd(x, w[ORC_W_IN_NORM], A->h1, N, d, c->eps);
  /* attention.h:107-109 Linear = x W^T (linear.h:13-26) */
  orc_matmul(A->h1, w[ORC_W_Q], A->q, N, H * D, d, 0, 1, 0.0);
  orc_matmul(A->h1, w[ORC_W_K], A->k, N, Hk * D, d, 0, 1, 0.0);
  orc_matmul(A->h1, w[ORC_W_V], A->v, N, Hk * D, d, 0, 1, 0.0);
  /* attention.h:115-118 QK-Norm over head_dim */
  if (c->qk_norm) {
    orc_rmsnorm_fwd(A->q, w[ORC_W_Q_NORM], A->qn, N * H, D, c->eps);
    orc_rmsnorm_fwd(A->k, w[ORC_W_K_NORM], A->kn, N * Hk, D, c->eps);
  } else {
    memcpy(A->qn, A->q, (size_t)(N * H * D) * sizeof(double));
    memcpy(A->kn, A->k, (size_t)(N * Hk * D) * sizeof(double));
  }
  /* attention.h:120-121, pos0 = 0 */
  orc_rope(A->qn, A->qr, B, T, H, D, 0, c->theta, 1.0, c->rope_factor, c->rope_low_freq,
           c->rope_high_freq, c->rope_orig_max_pos);
  orc_rope(A->kn, A->kr, B, T, Hk, D, 0, c->theta, 1.0, c->rope_factor, c->rope_low_freq,
           c->rope_high_freq, c->rope_orig_max_pos);
  /* attention.h:123-141 */
  orc_attention_fwd(A->qr, A->kr, A->v, A->attn, NULL, B, T, H, Hk, D, 1.0 / sqrt((double)D));
  orc_matmul(A->attn, w[ORC_W_O], a, N, d, H * D, 0, 1, 0.0);
  for (int64_t i = 0; i < N * d; ++i) A->h[i] = x[i] + a[i]; /* transformer_block.h:31 */
  orc_rmsnorm_fwd(A->h, w[ORC_W_POST_NORM], A->h2, N, d, c->eps);
  /* mlp.h:16-21 */
  orc_matmul(A->h2, w[ORC_W_GATE], A->g, N, I, d, 0, 1, 0.0);
  orc_matmul(A->h2, w[ORC_W_UP], A->u, N, I, d, 0, 1, 0.0);
  orc_silu(A->g, A->s, N * I);
  for (int64_t i = 0; i < N * I; ++i) A->m[i] = A->s[i] * A->u[i];
  orc_matmul(A->m, w[ORC_W_DOWN], dn, N, d, I, 0, 1, 0.0);
  for (int64_t i = 0; i < N * d; ++i) y[i] = A->h[i] + dn[i]; /* transformer_block.h:34 */
  free(a);
  free(dn);
}

static void block_free_acts(block_acts* A) {
  double** f = (double**)A;
  for (size_t i = 0; i < sizeof(block_acts) / sizeof(double*); ++i) free(f[i]);
}

void orc_block_fwd(const orc_cfg* cfg, const double* const* w, const double* x, double* y,
                   int64_t B, int64_t T) {
  block_acts A;
  block_forward_acts(cfg, w, x, y, B, T, &A);
  block_free_acts(&A);
}

/* Chain rule through orc_block_fwd using the reference's backward formulas:
 * MatmulBackward for Linear (matmul.cpp:105-107: dX = dY W, dW = dY^T X),
 * MulBackward (dy*b, dy*a), SiluBackward, RmsNormBackward, RopeBackward
 * (transpose rotation), AddBackward (two copies of dy, elementwise.cu:177-184). */
void orc_block_bwd(const orc_cfg* c, const double* const* w, const double* x,
                   const double* dy, double* dx, double* const* dw, int64_t B, int64_t T) {
  const int64_t N = B * T, d = c->hidden, I = c->inter, H = c->heads, Hk = c->kv_heads,
                D = c->head_dim;
  block_acts A;
  double* y = DALLOC(N * d);
  block_forward_acts(c, w, x, y, B, T, &A);
  free(y);

  double* dh = DALLOC(N * d);
  double* dm = DALLOC(N * I);
  double* dg = DALLOC(N * I);
  double* du = DALLOC(N * I);
  double* ds = DALLOC(N * I);
  double* dh2 = DALLOC(N * d);
  double* tmp = DALLOC(N * d);
  double* dattn = DALLOC(N * H * D);
  double* dqr = DALLOC(N * H * D);
  double* dkr = DALLOC(N * Hk * D);
  double* dv = DALLOC(N * Hk * D);
  double* dqn = DALLOC(N * H * D);
  double* dkn = DALLOC(N * Hk * D);
  double* dq = DALLOC(N * H * D);
  double* dk = DALLOC(N * Hk * D);
  double* dh1 = DALLOC(N * d);

  memcpy(dh, dy, (size_t)(N * d) * sizeof(double));
  /* down_proj */
  orc_matmul(dy, w[ORC_W_DOWN], dm, N, I, d, 0, 0, 0.0);
  orc_matmul(dy, A.m, dw[ORC_W_DOWN], d, I, N, 1, 0, 0.0);
  /* m = s * u */
  for (int64_t i = 0; i < N * I; ++i) {
    ds[i] = dm[i] * A.u[i];
    du[i] = dm[i] * A.s[i];
  }
  orc_silu_bwd(A.g, ds, dg, N * I);
  /* gate/up projections: dh2 = dg Wg + du Wu */
  orc_matmul(dg, w[ORC_W_GATE], dh2, N, d, I, 0, 0, 0.0);
  orc_matmul(du, w[ORC_W_UP], dh2, N, d, I, 0, 0, 1.0);
  orc_matmul(dg, A.h2, dw[ORC_W_GATE], I, d, N, 1, 0, 0.0);
  orc_matmul(du, A.h2, dw[ORC_W_UP], I, d, N, 1, 0, 0.0);
  orc_rmsnorm_bwd(dh2, A.h, w[ORC_W_POST_NORM], tmp, dw[ORC_W_POST_NORM], N, d, c->eps);
  for (int64_t i = 0; i < N * d; ++i) dh[i] += tmp[i];
  /* o_proj */
  orc_matmul(dh, w[ORC_W_O], dattn, N, H * D, d, 0, 0, 0.0);
  orc_matmul(dh, A.attn, dw[ORC_W_O], d, H * D, N, 1, 0, 0.0);
  orc_attention_bwd(A.qr, A.kr, A.v, dattn, dqr, dkr, dv, B, T, H, Hk, D,
                    1.0 / sqrt((double)D));
  orc_rope(dqr, dqn, B, T, H, D, 0, c->theta, -1.0, c->rope_factor, c->rope_low_freq,
           c->rope_high_freq, c->rope_orig_max_pos);
  orc_rope(dkr, dkn, B, T, Hk, D, 0, c->theta, -1.0, c->rope_factor, c->rope_low_freq,
           c->rope_high_freq, c->rope_orig_max_pos);
  if (c->qk_norm) {
    orc_rmsnorm_bwd(dqn, A.q, w[ORC_W_Q_NORM], dq, dw[ORC_W_Q_NORM], N * H, D, c->eps);
    orc_rmsnorm_bwd(dkn, A.k, w[ORC_W_K_NORM], dk, dw[ORC_W_K_NORM], N * Hk, D, c->eps);
  } else {
    memcpy(dq, dqn, (size_t)(N * H * D) * sizeof(double));
    memcpy(dk, dkn, (size_t)(N * Hk * D) * sizeof(double));
  }
  orc_matmul(dq, w[ORC_W_Q], dh1, N, d, H * D, 0, 0, 0.0);
  orc_matmul(dk, w[ORC_W_K], dh1, N, d, Hk * D, 0, 0, 1.0);
  orc_matmul(dv, w[ORC_W_V], dh1, N, d, Hk * D, 0, 0, 1.0);
  orc_matmul(dq, A.h1, dw[ORC_W_Q], H * D, d, N, 1, 0, 0.0);
  orc_matmul(dk, A.h1, dw[ORC_W_K], Hk * D, d, N, 1, 0, 0.0);
  orc_matmul(dv, A.h1, dw[ORC_W_V], Hk * D, d, N, 1, 0, 0.0);
  orc_rmsnorm_bwd(dh1, x, w[ORC_W_IN_NORM], tmp, dw[ORC_W_IN_NORM], N, d, c->eps);
  for (int64_t i = 0; i < N * d; ++i) dx[i] = dh[i] + tmp[i];

  block_free_acts(&A);
  free(dh); free(dm); free(dg); free(du); free(ds); free(dh2); free(tmp); free(dattn);
  free(dqr); free(dkr); free(dv); free(dqn); free(dkn); free(dq); free(dk); free(dh1);
}

/* Scores over all L keys, the mask applied as a -FLT_MAX fill (which
 * underflows to probability 0), then softmax and P V. */
void orc_attention_offset(const double* q, const double* k, const double* v, double* o,
                          int64_t B, int64_t T, int64_t L, int64_t H, int64_t Hk, int64_t D,
                          int64_t pos, double scale) {
  const int64_t group = H / Hk;
  double* p = DALLOC(L);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t kvh = h / group;
      for (int64_t t = 0; t < T; ++t) {
        const double* qt = q + ((b * T + t) * H + h) * D;
        double m = -DBL_MAX;
        for (int64_t j = 0; j < L; ++j) {
          double s = 0.0;
          const double* kj = k + ((b * L + j) * Hk + kvh) * D;
          for (int64_t d = 0; d < D; ++d) s += qt[d] * kj[d];
          s *= scale;
          if (j > pos + t) s = -FLT_MAX;
          p[j] = s;
          m = s > m ? s : m;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < L; ++j) {
          p[j] = exp(p[j] - m);
          sum += p[j];
        }
        double* ot = o + ((b * T + t) * H + h) * D;
        for (int64_t d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t j = 0; j < L; ++j) acc += p[j] * v[((b * L + j) * Hk + kvh) * D + d];
          ot[d] = acc / sum;
        }
      }
    }
  free(p);
}

/* -------------------------------------------------------------- Model */
static int64_t per_layer(const orc_cfg* c) { return c->qk_norm ? 11 : 9; }

int64_t orc_model_num_params(const orc_cfg* c) { return 2 + c->layers * per_layer(c); }

/* Map a layer's slice of the collect_parameters list (model.cpp:81-94) to ORC_W_*. */
static void layer_slots(const orc_cfg* c, int64_t base, int64_t slot[ORC_W_COUNT]) {
  int64_t j = base;
  for (int i = 0; i < ORC_W_COUNT; ++i) slot[i] = -1;
  slot[ORC_W_IN_NORM] = j++;
  slot[ORC_W_Q] = j++;
  slot[ORC_W_K] = j++;
  slot[ORC_W_V] = j++;
  slot[ORC_W_O] = j++;
  if (c->qk_norm) {
    slot[ORC_W_Q_NORM] = j++;
    slot[ORC_W_K_NORM] = j++;
  }
  slot[ORC_W_POST_NORM] = j++;
  slot[ORC_W_GATE] = j++;
  slot[ORC_W_UP] = j++;
  slot[ORC_W_DOWN] = j++;
}

/* Model::forward_train_logits + forward_train_masked (include/ctd/nn/model.h:170-206):
 * embedding, blocks, final RMSNorm, tied head logits = h E^T, masked CE. */
double orc_model_loss(const orc_cfg* c, const double* const* params, double* const* grads,
                      const int64_t* ids, const int64_t* targets, const double* mask,
                      int64_t B, int64_t T) {
  const int64_t N = B * T, d = c->hidden, V = c->vocab, L = c->layers;
  const int64_t np = orc_model_num_params(c);
  double** xs = (double**)xcalloc((size_t)(L + 1), sizeof(double*));
  for (int64_t l = 0; l <= L; ++l) xs[l] = DALLOC(N * d);
  orc_embedding_fwd(ids, params[0], xs[0], N, d);
  for (int64_t l = 0; l < L; ++l) {
    int64_t slot[ORC_W_COUNT];
    const double* w[ORC_W_COUNT];
    layer_slots(c, 1 + l * per_layer(c), slot);
    for (int i = 0; i < ORC_W_COUNT; ++i) w[i] = slot[i] >= 0 ? params[slot[i]] : NULL;
    orc_block_fwd(c, w, xs[l], xs[l + 1], B, T);
  }
  double* hn = DALLOC(N * d);
  orc_rmsnorm_fwd(xs[L], params[np - 1], hn, N, d, c->eps);
  double* logits = DALLOC(N * V);
  orc_matmul(hn, params[0], logits, N, V, d, 0, 1, 0.0);
  const double loss = orc_ce_masked_fwd(logits, targets, mask, N, V, NULL, NULL);

  if (grads) {
    double* dlogits = DALLOC(N * V);
    orc_ce_masked_bwd(logits, targets, mask, N, V, 1.0, dlogits);
    double* dhn = DALLOC(N * d);
    double* dx = DALLOC(N * d);
    double* dcur = DALLOC(N * d);
    double* demb = DALLOC(V * d);
    orc_matmul(dlogits, params[0], dhn, N, d, V, 0, 0, 0.0);      /* dX = dY E */
    orc_matmul(dlogits, hn, grads[0], V, d, N, 1, 0, 0.0);        /* dE = dY^T X */
    orc_rmsnorm_bwd(dhn, xs[L], params[np - 1], dcur, grads[np - 1], N, d, c->eps);
    for (int64_t l = L - 1; l >= 0; --l) {
      int64_t slot[ORC_W_COUNT];
      const double* w[ORC_W_COUNT];
      double* dw[ORC_W_COUNT];
      double* scratch[ORC_W_COUNT] = {0};
      layer_slots(c, 1 + l * per_layer(c), slot);
      for (int i = 0; i < ORC_W_COUNT; ++i) {
        w[i] = slot[i] >= 0 ? params[slot[i]] : NULL;
        if (slot[i] >= 0) {
          dw[i] = grads[slot[i]];
        } else {
          scratch[i] = DALLOC(c->head_dim);
          dw[i] = scratch[i];
        }
      }
      orc_block_bwd(c, w, xs[l], dcur, dx, dw, B, T);
      memcpy(dcur, dx, (size_t)(N * d) * sizeof(double));
      for (int i = 0; i < ORC_W_COUNT; ++i) free(scratch[i]);
    }
    orc_embedding_bwd(ids, dcur, demb, N, d, V);
    for (int64_t i = 0; i < V * d; ++i) grads[0][i] += demb[i]; /* tied weight: two contributions */
    free(dlogits); free(dhn); free(dx); free(dcur); free(demb);
  }
  for (int64_t l = 0; l <= L; ++l) free(xs[l]);
  free(xs); free(hn); free(logits);
  return loss;
}

void orc_model_logits(const orc_cfg* c, const double* const* params, const int64_t* ids,
                      double* logits, int64_t B, int64_t T) {
  const int64_t N = B * T, d = c->hidden, L = c->layers;
  const int64_t np = orc_model_num_params(c);
  double* x = DALLOC(N * d);
  double* y = DALLOC(N * d);
  orc_embedding_fwd(ids, params[0], x, N, d);
  for (int64_t l = 0; l < L; ++l) {
    int64_t slot[ORC_W_COUNT];
    const double* w[ORC_W_COUNT];
    layer_slots(c, 1 + l * per_layer(c), slot);
    for (int i = 0; i < ORC_W_COUNT; ++i) w[i] = slot[i] >= 0 ? params[slot[i]] : NULL;
    orc_block_fwd(c, w, x, y, B, T);
    double* tmp = x;
    x = y;
    y = tmp;
  }
  orc_rmsnorm_fwd(x, params[np - 1], y, N, d, c->eps);
  orc_matmul(y, params[0], logits, N, c->vocab, d, 0, 1, 0.0);
  free(x);
  free(y);
}
