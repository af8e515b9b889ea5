// Inference-only ops: KV-cache writes/reads and attention with a position
// offset (reference src/ops/kv_cache.cu:50-108, include/ctd/nn/attention.h:43-97).
// None of these record autograd history.
#include <cmath>

#include "ctd/ops/attention.h"
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

}  // namespace ctd::ops
