// The reference's unfused attention-chain ops (softmax, causal mask,
// repeat_kv, mul_scalar, permute), kept so its ops:: API is complete.
// Backward formulas: src/ops/softmax.cu:54-80, mask.cu:41-52,
// repeat_kv.cu:29-43 and 125-165, permute.cu:102-127.
#include <vector>

#include "ctd/ops/mask.h"
#include "ctd/ops/permute.h"
#include "ctd/ops/repeat_kv.h"
#include "ctd/ops/softmax.h"
#include "op_util.h"

namespace ctd::ops {

using namespace detail;

// ================================================================= softmax
namespace {
struct SoftmaxBackward : autograd::Node {
  Tensor y;
  const char* name() const override { return "SoftmaxBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    Tensor dx = softmax_backward_impl(y, go.at(0));
    release_saved(y);
    return {dx};
  }
};
}  // namespace

Tensor softmax_impl(const Tensor& x) {
  check_f32(x, "softmax");
  require(x.dim() >= 1 && x.shape().back() > 0, "softmax: empty last dim");
  Tensor y = empty_like(x);
  const int64_t N = x.shape().back();
  CTD_CHECK(ember_softmax_fwd(cfp(x), fp(y), x.numel() / N, N, S()));
  return y;
}

Tensor softmax_backward_impl(const Tensor& y, const Tensor& g) {
  check_f32(y, "softmax_backward", "y");
  check_f32(g, "softmax_backward", "g");
  require(y.shape() == g.shape(), "softmax_backward: shape mismatch");
  Tensor dx = empty_like(y);
  const int64_t N = y.shape().back();
  CTD_CHECK(ember_softmax_bwd(cfp(y), cfp(g), fp(dx), y.numel() / N, N, S()));
  return dx;
}

Tensor softmax(const Tensor& x) {
  Tensor y = softmax_impl(x);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<SoftmaxBackward>();
    node->y = y.detach();
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

// ============================================================ causal mask
namespace {
constexpr float kMaskFill = -3.40282346638528859812e+38F;  // -FLT_MAX (mask.cu:37)

void mask_dims(const Tensor& s, int64_t& rows, int64_t& Tq, int64_t& Tk) {
  check_f32(s, "apply_causal_mask", "scores");
  require(s.dim() >= 2, "apply_causal_mask: expected [..., Tq, Tk]");
  Tk = s.shape()[s.dim() - 1];
  Tq = s.shape()[s.dim() - 2];
  rows = Tk ? s.numel() / Tk : 0;
}

struct CausalMaskBackward : autograd::Node {
  int q0 = 0;
  const char* name() const override { return "CausalMaskBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    return {causal_mask_backward_impl(go.at(0), q0)};
  }
};
}  // namespace

void apply_causal_mask_inplace(Tensor& scores, int q_pos_start) {
  int64_t rows, Tq, Tk;
  mask_dims(scores, rows, Tq, Tk);
  CTD_CHECK(ember_causal_mask(cfp(scores), fp(scores), rows, Tq, Tk, q_pos_start, kMaskFill, S()));
}

Tensor apply_causal_mask_impl(const Tensor& scores, int q_pos_start) {
  int64_t rows, Tq, Tk;
  mask_dims(scores, rows, Tq, Tk);
  Tensor out = empty_like(scores);
  CTD_CHECK(ember_causal_mask(cfp(scores), fp(out), rows, Tq, Tk, q_pos_start, kMaskFill, S()));
  return out;
}

Tensor causal_mask_backward_impl(const Tensor& g, int q_pos_start) {
  int64_t rows, Tq, Tk;
  mask_dims(g, rows, Tq, Tk);
  Tensor out = empty_like(g);
  CTD_CHECK(ember_causal_mask(cfp(g), fp(out), rows, Tq, Tk, q_pos_start, 0.0f, S()));
  return out;
}

Tensor apply_causal_mask(const Tensor& scores, int q_pos_start) {
  Tensor y = apply_causal_mask_impl(scores, q_pos_start);
  if (autograd::any_requires_grad({scores})) {
    auto node = std::make_shared<CausalMaskBackward>();
    node->q0 = q_pos_start;
    node->next_edges = autograd::collect_next_edges({scores});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

// ============================================================== repeat_kv
namespace {
struct RepeatKvBackward : autograd::Node {
  int group = 1;
  const char* name() const override { return "RepeatKvBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    return {repeat_kv_sum_impl(go.at(0), group)};
  }
};

struct MulScalarBackward : autograd::Node {
  float c = 1.0f;
  const char* name() const override { return "MulScalarBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    return {mul_scalar_impl(go.at(0), c)};
  }
};
}  // namespace

Tensor repeat_kv_heads_impl(const Tensor& x, int group) {
  check_f32(x, "repeat_kv_heads");
  require(x.dim() == 4 && group >= 1, "repeat_kv_heads: expected [B,T,H_kv,D] and group >= 1");
  const auto& s = x.shape();
  Tensor y = Tensor::empty({s[0], s[1], s[2] * group, s[3]}, x.dtype(), x.device());
  CTD_CHECK(ember_repeat_kv(cfp(x), fp(y), s[0] * s[1], s[2], group, s[3], S()));
  return y;
}

Tensor repeat_kv_sum_impl(const Tensor& y, int group) {
  check_f32(y, "repeat_kv_sum");
  require(y.dim() == 4 && group >= 1 && y.shape()[2] % group == 0,
          "repeat_kv_sum: expected [B,T,H_kv*group,D]");
  const auto& s = y.shape();
  Tensor x = Tensor::empty({s[0], s[1], s[2] / group, s[3]}, y.dtype(), y.device());
  CTD_CHECK(ember_repeat_kv_sum(cfp(y), fp(x), s[0] * s[1], s[2] / group, group, s[3], S()));
  return x;
}

Tensor repeat_kv_heads(const Tensor& x, int group) {
  Tensor y = repeat_kv_heads_impl(x, group);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<RepeatKvBackward>();
    node->group = group;
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor mul_scalar_impl(const Tensor& x, float c) {
  check_f32(x, "mul_scalar");
  Tensor y = empty_like(x);
  CTD_CHECK(ember_scale(cfp(x), c, fp(y), x.numel(), S()));
  return y;
}

Tensor mul_scalar(const Tensor& x, float c) {
  Tensor y = mul_scalar_impl(x, c);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<MulScalarBackward>();
    node->c = c;
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

// ================================================================ permute
namespace {
struct PermuteBackward : autograd::Node {
  std::vector<int> inverse;
  const char* name() const override { return "PermuteBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    return {permute_impl(go.at(0), inverse)};
  }
};
}  // namespace

Tensor permute_impl(const Tensor& x, const std::vector<int>& perm) {
  check_f32(x, "permute");
  const int nd = static_cast<int>(x.dim());
  require(static_cast<int>(perm.size()) == nd && nd >= 1 && nd <= 6,
          "permute: perm must match rank (1..6)");
  std::vector<int64_t> out_shape(nd);
  for (int i = 0; i < nd; ++i) {
    require(perm[i] >= 0 && perm[i] < nd, "permute: bad axis");
    out_shape[i] = x.shape()[perm[i]];
  }
  Tensor y = Tensor::empty(out_shape, x.dtype(), x.device());
  CTD_CHECK(ember_permute(cfp(x), fp(y), nd, x.shape().data(), perm.data(), S()));
  return y;
}

Tensor permute(const Tensor& x, const std::vector<int>& perm) {
  Tensor y = permute_impl(x, perm);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<PermuteBackward>();
    node->inverse.resize(perm.size());
    for (size_t i = 0; i < perm.size(); ++i) node->inverse[perm[i]] = static_cast<int>(i);
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

}  // namespace ctd::ops
