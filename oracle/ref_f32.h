/* ref_f32.h -- the reference's scalar fp32 CPU test ops and their composition
 * (ref_f32.c).  TEST INFRASTRUCTURE ONLY: bench.py's CPU baseline and its
 * check in tests/. */
#ifndef REF_F32_H
#define REF_F32_H
#include <stdint.h>

typedef struct {
  int d, H, Hk, Dh, I; /* hidden, query heads, KV heads, head dim, MLP width */
  float eps, theta;
} rf_block_cfg;

/* Block weights in the reference's layouts (Linear weights [out, in]); qn/kn
 * are the QK-Norm weights [Dh], NULL without QK-Norm. */
typedef struct {
  const float *ln1, *wq, *wk, *wv, *wo, *qn, *kn, *ln2, *wg, *wu, *wd;
} rf_block_w;
/* Gradient buffers of the same shapes; the backward adds into them. */
typedef struct {
  float *ln1, *wq, *wk, *wv, *wo, *qn, *kn, *ln2, *wg, *wu, *wd;
} rf_block_g;

void rf_mm(const float* a, const float* b, float* c, int M, int K, int N, int ta, int tb);
void rf_rms_norm(const float* x, const float* w, float* y, int rows, int H, float eps);
void rf_softmax(const float* x, float* y, int rows, int N);
void rf_rope(float* x, int B, int T, int H, int D, int pos_start, float theta);
void rf_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float b1,
              float b2, float eps, float wd, int step);

/* One block over T tokens (batch 1): x, y, dy, dx [T, d]. */
void rf_block_forward(const rf_block_cfg* c, const rf_block_w* w, const float* x, float* y, int T);
void rf_block_fwd_bwd(const rf_block_cfg* c, const rf_block_w* w, const float* x, const float* dy,
                      float* y, float* dx, rf_block_g* g, int T, int checkpoint);
/* One causal attention head over q/k/v/dout [T, D]: o, and with dout non-NULL
 * dq, dk, dv. */
void rf_attention_head(const float* q, const float* k, const float* v, const float* dout,
                       float* o, float* dq, float* dk, float* dv, int T, int D);
float rf_lm_head_ce(const float* h, const float* E, const int64_t* tgt, const float* mask,
                    float* dh, float* dE, int n, int d, int V);
#endif
