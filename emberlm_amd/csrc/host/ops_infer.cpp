// Inference-only ops: KV-cache writes/reads and attention with a position
// offset (reference src/ops/kv_cache.cu:50-108, include/ctd/nn/attention.h:43-97).
// None of these record autograd history.
#include <cmath>

#include "ctd/ops/attention.h"
#include "ctd/ops/decode.h"
#include "ctd/ops/kv_cache.h"
#include "ember_hip.h"
#include "op_util.h"

namespace ctd::ops {

using namespace detail;

void write_kv_inplace(Tensor& cache, const Tensor& src, int pos) {
  check_f32(cache, "write_kv", "cache");
  check_f32(src, "write_kv", "src");
  require(cache.dim() == 4 && src.dim() == 4, "write_kv: expected 4D inputs");
  const int64_t B = src.shape()[0], T = src.shape()[1], Hk = src.shape()[2], D = src.shape()[3];
  const int64_t max_seq = cache.shape()[2];
  require(cache.shape()[0] == B && cache.shape()[1] == Hk && cache.shape()[3] == D,
          "write_kv: cache / src dim mismatch");
  require(pos >= 0 && pos + T <= max_seq, "write_kv: write range out of cache bounds");
  CTD_CHECK(ember_kv_write(cfp(src), fp(cache), B, T, Hk, D, max_seq, pos, S()));
}

Tensor read_kv_expanded(const Tensor& cache, int valid_len, int group) {
  check_f32(cache, "read_kv_expanded", "cache");
  require(cache.dim() == 4, "read_kv_expanded: 4D cache required");
  const int64_t B = cache.shape()[0], Hk = cache.shape()[1], max_seq = cache.shape()[2],
                D = cache.shape()[3];
  require(valid_len >= 0 && valid_len <= max_seq, "read_kv_expanded: valid_len out of range");
  require(group > 0, "read_kv_expanded: group must be > 0");
  Tensor out = Tensor::empty({B, Hk * group, valid_len, D}, DType::kFloat32, cache.device());
  CTD_CHECK(
      ember_kv_read_expanded(cfp(cache), fp(out), B, Hk, group, valid_len, D, max_seq, S()));
  return out;
}

namespace {

Tensor decode_attention(const Tensor& q, const Tensor& k, const Tensor& v, int64_t Hk,
                        int64_t L, int position_start, int64_t sb, int64_t sh, int64_t st,
                        float scale, const char* op) {
  const int64_t B = q.shape()[0], T = q.shape()[1], H = q.shape()[2], D = q.shape()[3];
  require(Hk > 0 && H % Hk == 0, std::string(op) + ": num_heads % num_kv_heads != 0");
  require(D == 64 || D == 128, std::string(op) + ": head_dim must be 64 or 128");
  require(position_start >= 0, std::string(op) + ": position_start must be >= 0");
  Tensor o = empty_like(q);
  if (B == 0 || T == 0) return o;
  require(L >= 1, std::string(op) + ": no keys to attend to");
  const size_t wsb = ember_attn_decode_workspace_bytes(B, T, H, Hk, D, L);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  CTD_CHECK(ember_attn_decode(cfp(q), cfp(k), cfp(v), fp(o), B, T, H, Hk, D, L, position_start,
                              sb, sh, st, scale, wsb ? ws.data_ptr() : nullptr, wsb, S()));
  return o;
}

}  // namespace

Tensor cached_attention(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache,
                        int64_t valid_len, int position_start, float scale) {
  check_f32(q, "cached_attention", "q");
  check_f32(k_cache, "cached_attention", "k cache");
  check_f32(v_cache, "cached_attention", "v cache");
  require(q.dim() == 4 && k_cache.dim() == 4, "cached_attention: expected q [B,T,H,D] and "
                                              "cache [B,Hk,S,D]");
  require(k_cache.shape() == v_cache.shape(), "cached_attention: k and v caches differ");
  const int64_t Hk = k_cache.shape()[1], max_seq = k_cache.shape()[2], D = k_cache.shape()[3];
  require(k_cache.shape()[0] == q.shape()[0] && D == q.shape()[3],
          "cached_attention: q / cache shape mismatch");
  require(valid_len >= 0 && valid_len <= max_seq, "cached_attention: valid_len out of range");
  return decode_attention(q, k_cache, v_cache, Hk, valid_len, position_start, Hk * max_seq * D,
                          max_seq * D, D, scale, "cached_attention");
}

Tensor offset_attention(const Tensor& q, const Tensor& k, const Tensor& v, int position_start,
                        float scale) {
  check_f32(q, "offset_attention", "q");
  check_f32(k, "offset_attention", "k");
  check_f32(v, "offset_attention", "v");
  require(q.dim() == 4 && k.dim() == 4, "offset_attention: expected [B,T,H,D]");
  require(k.shape() == v.shape(), "offset_attention: k and v shapes differ");
  const int64_t T = k.shape()[1], Hk = k.shape()[2], D = k.shape()[3];
  require(k.shape()[0] == q.shape()[0] && T == q.shape()[1] && D == q.shape()[3],
          "offset_attention: q/k shape mismatch");
  return decode_attention(q, k, v, Hk, T, position_start, T * Hk * D, D, Hk * D, scale,
                          "offset_attention");
}

namespace {

int64_t rows_of(const Tensor& x, int64_t K, const char* op) {
  require(x.dim() >= 1 && x.shape().back() == K, std::string(op) + ": in_features mismatch");
  const int64_t M = x.numel() / K;
  require(M <= kDecodeMaxRows, std::string(op) + ": more than 8 token rows");
  return M;
}

std::vector<int64_t> with_last(const Tensor& x, int64_t n) {
  std::vector<int64_t> sh = x.shape();
  sh.back() = n;
  return sh;
}

}  // namespace

std::vector<Tensor> decode_linear(const Tensor& x, const Tensor& norm_w, float eps,
                                  const std::vector<Tensor>& weights,
                                  const std::vector<Tensor>& residuals) {
  check_f32(x, "decode_linear", "x");
  require(!weights.empty() && weights.size() <= 3, "decode_linear: 1 to 3 weights");
  require(residuals.empty() || residuals.size() == weights.size(),
          "decode_linear: one residual per weight");
  const int64_t K = weights[0].shape().at(1);
  const int64_t M = rows_of(x, K, "decode_linear");
  if (norm_w.defined()) {
    check_f32(norm_w, "decode_linear", "norm weight");
    require(norm_w.numel() == K, "decode_linear: norm weight size != in_features");
  }
  std::vector<Tensor> out;
  const float* W[3] = {};
  int64_t N[3] = {};
  float* y[3] = {};
  const float* res[3] = {};
  for (size_t i = 0; i < weights.size(); ++i) {
    check_f32(weights[i], "decode_linear", "weight");
    require(weights[i].dim() == 2 && weights[i].shape()[1] == K,
            "decode_linear: weights must be [N, K] with one K");
    N[i] = weights[i].shape()[0];
    out.push_back(Tensor::empty(with_last(x, N[i]), DType::kFloat32, x.device()));
    W[i] = cfp(weights[i]);
    y[i] = fp(out.back());
    if (!residuals.empty()) {
      check_f32(residuals[i], "decode_linear", "residual");
      require(residuals[i].shape() == out.back().shape(), "decode_linear: residual shape");
      res[i] = cfp(residuals[i]);
    }
  }
  CTD_CHECK(ember_decode_gemv(cfp(x), M, K, norm_w.defined() ? cfp(norm_w) : nullptr, eps,
                              static_cast<int>(weights.size()), W, N, y,
                              residuals.empty() ? nullptr : res, S()));
  return out;
}

Tensor decode_gate_up(const Tensor& x, const Tensor& norm_w, float eps, const Tensor& w_gate,
                      const Tensor& w_up) {
  check_f32(x, "decode_gate_up", "x");
  check_f32(w_gate, "decode_gate_up", "gate weight");
  check_f32(w_up, "decode_gate_up", "up weight");
  require(w_gate.dim() == 2 && w_gate.shape() == w_up.shape(),
          "decode_gate_up: gate and up weights differ");
  const int64_t I = w_gate.shape()[0], K = w_gate.shape()[1];
  const int64_t M = rows_of(x, K, "decode_gate_up");
  if (norm_w.defined()) {
    check_f32(norm_w, "decode_gate_up", "norm weight");
    require(norm_w.numel() == K, "decode_gate_up: norm weight size != in_features");
  }
  Tensor out = Tensor::empty(with_last(x, I), DType::kFloat32, x.device());
  CTD_CHECK(ember_decode_gateup(cfp(x), M, K, norm_w.defined() ? cfp(norm_w) : nullptr, eps,
                                cfp(w_gate), cfp(w_up), I, fp(out), S()));
  return out;
}

namespace {

// Checks shared by decode_qkv_post and decode_qkv_attention; returns the
// RoPE frequencies of head_dim under theta / scaling.
std::vector<float> check_qkv_post(const char* op, const Tensor& q, const Tensor& k,
                                  const Tensor& v, int64_t H, int64_t Hk, int64_t D,
                                  const Tensor& q_norm_w, const Tensor& k_norm_w, float theta,
                                  const RopeScaling& scaling, int position_start,
                                  const Tensor& k_cache, const Tensor& v_cache) {
  const std::string o(op);
  check_f32(q, op, "q");
  check_f32(k, op, "k");
  check_f32(v, op, "v");
  check_f32(k_cache, op, "k cache");
  check_f32(v_cache, op, "v cache");
  require(q.dim() == 3 && k.dim() == 3 && k.shape() == v.shape(),
          o + ": expected q [B,T,H*D], k/v [B,T,Hk*D]");
  const int64_t B = q.shape()[0], T = q.shape()[1];
  require(q.shape()[2] == H * D && k.shape()[0] == B && k.shape()[1] == T &&
              k.shape()[2] == Hk * D,
          o + ": q/k/v widths != heads * head_dim");
  require(k_cache.dim() == 4 && k_cache.shape() == v_cache.shape() && k_cache.shape()[0] == B &&
              k_cache.shape()[1] == Hk && k_cache.shape()[3] == D,
          o + ": cache / src dim mismatch");
  require(position_start >= 0 && position_start + T <= k_cache.shape()[2],
          "write_kv: write range out of cache bounds");
  for (const Tensor* w : {&q_norm_w, &k_norm_w})
    if (w->defined()) {
      check_f32(*w, op, "norm weight");
      require(w->numel() == D, o + ": QK-Norm weight size != head_dim");
    }
  std::vector<float> freqs(static_cast<size_t>(D / 2));
  CTD_CHECK(ember_rope_freqs_host(freqs.data(), static_cast<int>(D), theta, scaling.factor,
                                  scaling.low_freq_factor, scaling.high_freq_factor,
                                  scaling.original_max_pos));
  return freqs;
}

}  // namespace

Tensor decode_qkv_post(const Tensor& q, const Tensor& k, const Tensor& v, int num_heads,
                       int num_kv_heads, int head_dim, const Tensor& q_norm_w,
                       const Tensor& k_norm_w, float eps, float theta, const RopeScaling& scaling,
                       int position_start, Tensor& k_cache, Tensor& v_cache) {
  const int64_t H = num_heads, Hk = num_kv_heads, D = head_dim;
  const std::vector<float> freqs =
      check_qkv_post("decode_qkv_post", q, k, v, H, Hk, D, q_norm_w, k_norm_w, theta, scaling,
                     position_start, k_cache, v_cache);
  const int64_t B = q.shape()[0], T = q.shape()[1], max_seq = k_cache.shape()[2];
  Tensor qo = Tensor::empty({B, T, H, D}, DType::kFloat32, q.device());
  CTD_CHECK(ember_decode_qkv_post(cfp(q), cfp(k), cfp(v), B, T, H, Hk, D,
                                  q_norm_w.defined() ? cfp(q_norm_w) : nullptr,
                                  k_norm_w.defined() ? cfp(k_norm_w) : nullptr, eps, freqs.data(),
                                  position_start, fp(qo), fp(k_cache), fp(v_cache), max_seq, S()));
  return qo;
}

Tensor decode_qkv_attention(const Tensor& q, const Tensor& k, const Tensor& v, int num_heads,
                            int num_kv_heads, int head_dim, const Tensor& q_norm_w,
                            const Tensor& k_norm_w, float eps, float theta,
                            const RopeScaling& scaling, int position_start, Tensor& k_cache,
                            Tensor& v_cache, float scale) {
  const int64_t H = num_heads, Hk = num_kv_heads, D = head_dim;
  const std::vector<float> freqs =
      check_qkv_post("decode_qkv_attention", q, k, v, H, Hk, D, q_norm_w, k_norm_w, theta,
                     scaling, position_start, k_cache, v_cache);
  require(Hk > 0 && H % Hk == 0, "decode_qkv_attention: num_heads % num_kv_heads != 0");
  require(D == 64 || D == 128, "decode_qkv_attention: head_dim must be 64 or 128");
  const int64_t B = q.shape()[0], T = q.shape()[1], max_seq = k_cache.shape()[2];
  require(T <= kDecodeMaxRows, "decode_qkv_attention: more than 8 new rows per call");
  Tensor o = Tensor::empty({B, T, H, D}, DType::kFloat32, q.device());
  if (B == 0 || T == 0) return o;
  const size_t wsb = ember_attn_decode_workspace_bytes(B, T, H, Hk, D, position_start + T);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  CTD_CHECK(ember_attn_decode_qkv(cfp(q), cfp(k), cfp(v), B, T, H, Hk, D,
                                  q_norm_w.defined() ? cfp(q_norm_w) : nullptr,
                                  k_norm_w.defined() ? cfp(k_norm_w) : nullptr, eps, freqs.data(),
                                  position_start, fp(k_cache), fp(v_cache), max_seq, scale, fp(o),
                                  wsb ? ws.data_ptr() : nullptr, wsb, S()));
  return o;
}

}  // namespace ctd::ops
