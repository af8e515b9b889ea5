// Ops on the training block's path: matmul/bmm, RMSNorm, RoPE, elementwise,
// fused SwiGLU and fused causal attention.  Each public op launches through
// the C ABI and, when an input requires grad, records a backward node with
// the reference's gradient formulas (src/ops/*.cu, src/ops/matmul.cpp).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <utility>

#include "ctd/ops/attention.h"
#include "ctd/ops/elementwise.h"
#include "ctd/ops/matmul.h"
#include "ctd/ops/norm.h"
#include "ctd/ops/rope.h"
#include "op_util.h"

namespace ctd::ops {

using namespace detail;

// ================================================================== matmul
namespace {

struct MM {
  int64_t M, N, K, lda, ldb;
};

MM mm_dims(const Tensor& a, const Tensor& b, bool ta, bool tb, const char* op) {
  check_f32(a, op, "a");
  check_f32(b, op, "b");
  require(a.dim() == 2 && b.dim() == 2, std::string(op) + ": expected 2-D operands");
  MM d;
  d.M = ta ? a.shape()[1] : a.shape()[0];
  d.K = ta ? a.shape()[0] : a.shape()[1];
  const int64_t kb = tb ? b.shape()[1] : b.shape()[0];
  d.N = tb ? b.shape()[0] : b.shape()[1];
  require(d.K == kb, std::string(op) + ": inner dimension mismatch (" + std::to_string(d.K) +
                         " vs " + std::to_string(kb) + ")");
  d.lda = a.shape()[1];
  d.ldb = b.shape()[1];
  return d;
}

// Forward y = op(a) op(b); backward table of src/ops/matmul.cpp:99-118, one
// operand at a time: each gradient is op(x) op(y) of dy and the other operand,
// dy first or second.
struct GradForm {
  bool dy_first, tx, ty;
};
GradForm grad_a_form(bool ta, bool tb) {
  if (!ta && !tb) return {true, false, true};   // dy b^T
  if (ta && !tb) return {false, false, true};   // b dy^T
  if (!ta && tb) return {true, false, false};   // dy b
  return {false, true, true};                   // b^T dy^T
}
GradForm grad_b_form(bool ta, bool tb) {
  if (!ta && !tb) return {false, true, false};  // a^T dy
  if (ta && !tb) return {false, false, false};  // a dy
  if (!ta && tb) return {true, true, false};    // dy^T a
  return {true, true, true};                    // dy^T a^T
}

template <typename F>
Tensor grad_product(const GradForm& f, const Tensor& dy, const Tensor& other, F mm) {
  return f.dy_first ? mm(dy, other, f.tx, f.ty) : mm(other, dy, f.tx, f.ty);
}

template <typename F>
std::pair<Tensor, Tensor> matmul_like_backward(const Tensor& dy, const Tensor& a,
                                               const Tensor& b, bool ta, bool tb, bool need_a,
                                               bool need_b, F mm) {
  Tensor dA, dB;
  if (need_a) dA = grad_product(grad_a_form(ta, tb), dy, b, mm);
  if (need_b) dB = grad_product(grad_b_form(ta, tb), dy, a, mm);
  return {dA, dB};
}

// c += op(x) op(y) on the GEMM (beta = 1): the same float additions as the
// product stored and then accumulated into c.
void matmul_accumulate(const Tensor& x, const Tensor& y, bool tx, bool ty, Tensor& c) {
  const MM d = mm_dims(x, y, tx, ty, "matmul");
  const size_t wsb = ember_gemm_f32_workspace_bytes(d.M, d.N, d.K, 1);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32_ws(tx, ty, d.M, d.N, d.K, 1.0f, cfp(x), d.lda, 0, cfp(y), d.ldb, 0,
                              1.0f, fp(c), d.N, 0, 1, wsb ? ws.data_ptr() : nullptr, wsb, S()));
  runtime::gemm_profile_end(ev, 2.0 * d.M * d.N * d.K, 2 * tx + ty);
}

struct MatmulBackward : autograd::Node {
  Tensor a, b;
  bool ta = false, tb = false;
  const char* name() const override { return "MatmulBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    return backward_with_partials(go, {});
  }
  // dA goes straight into a partial sum the engine already holds for a
  // (another consumer's gradient), by a beta = 1 GEMM: the fan-in add of
  // src/core/autograd.cu:86-118 done where dA is stored.
  bool accepts_partials() const override { return true; }
  std::vector<Tensor> backward_with_partials(const std::vector<Tensor>& go,
                                             const std::vector<Tensor>& partials) override {
    autograd::NoGradGuard ng;
    const bool na = next_edges.at(0).node != nullptr, nb = next_edges.at(1).node != nullptr;
    const Tensor& dy = go.at(0);
    const Tensor* into = partials.empty() ? nullptr : &partials[0];
    const bool fold = na && into && into->storage() && into->dtype() == DType::kFloat32 &&
                      into->device() == a.device() && into->is_contiguous() &&
                      into->shape() == a.shape();
    // dB first: it is a's last reader, so a's memory goes back to the
    // allocator before dA is allocated (when this node held a alone, as the
    // MLP's down projection holds the [tokens, intermediate] activation, the
    // same block can hold the gradient of that activation).
    Tensor dB;
    if (nb) dB = grad_product(grad_b_form(ta, tb), dy, a, matmul_impl);
    release_saved(a);
    Tensor dA;
    if (na) {
      const GradForm f = grad_a_form(ta, tb);
      if (fold) {
        Tensor acc = *into;
        if (f.dy_first) matmul_accumulate(dy, b, f.tx, f.ty, acc);
        else matmul_accumulate(b, dy, f.tx, f.ty, acc);
        dA = acc;
      } else {
        dA = grad_product(f, dy, b, matmul_impl);
      }
    }
    release_saved(b);
    return {dA, dB};
  }
};

struct BmmBackward : autograd::Node {
  Tensor a, b;
  bool ta = false, tb = false;
  const char* name() const override { return "BmmBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    const bool na = next_edges.at(0).node != nullptr, nb = next_edges.at(1).node != nullptr;
    auto [dA, dB] = matmul_like_backward(go.at(0), a, b, ta, tb, na, nb, bmm_impl);
    release_saved(a, b);
    return {dA, dB};
  }
};

}  // namespace

Tensor matmul_impl(const Tensor& a, const Tensor& b, bool transa, bool transb) {
  const MM d = mm_dims(a, b, transa, transb, "matmul");
  Tensor c = Tensor::empty({d.M, d.N}, DType::kFloat32, a.device());
  // Weight-gradient shapes (few output tiles, K = tokens) split K into partials.
  const size_t wsb = ember_gemm_f32_workspace_bytes(d.M, d.N, d.K, 1);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32_ws(transa, transb, d.M, d.N, d.K, 1.0f, cfp(a), d.lda, 0, cfp(b),
                              d.ldb, 0, 0.0f, fp(c), d.N, 0, 1, wsb ? ws.data_ptr() : nullptr,
                              wsb, S()));
  runtime::gemm_profile_end(ev, 2.0 * d.M * d.N * d.K, 2 * transa + transb);
  return c;
}

Tensor matmul(const Tensor& a, const Tensor& b, bool transa, bool transb) {
  Tensor y = matmul_impl(a, b, transa, transb);
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<MatmulBackward>();
    node->a = a.detach();
    node->b = b.detach();
    node->ta = transa;
    node->tb = transb;
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor matmul_graph_only(const Tensor& a, const Tensor& b, bool transa, bool transb,
                         const Tensor& values) {
  const MM d = mm_dims(a, b, transa, transb, "matmul_graph_only");
  require(values.is_contiguous() && values.numel() == d.M * d.N,
          "matmul_graph_only: values must be M*N contiguous elements");
  Tensor y = values.detach().reshape({d.M, d.N});
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<MatmulBackward>();
    node->a = a.detach();
    node->b = b.detach();
    node->ta = transa;
    node->tb = transb;
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y.mark_placeholder();  // its elements are `values`, not the product
}

Tensor matmul_add(const Tensor& a, const Tensor& b, bool transa, bool transb, const Tensor& d) {
  const MM dm = mm_dims(a, b, transa, transb, "matmul_add");
  check_f32(d, "matmul_add", "d");
  require(d.device() == a.device() && d.is_contiguous() && d.dim() == 2 &&
              d.shape()[0] == dm.M && d.shape()[1] == dm.N,
          "matmul_add: d must be a contiguous [M, N] tensor on the operands' device");
  Tensor y = Tensor::empty({dm.M, dm.N}, DType::kFloat32, a.device());
  const size_t wsb = ember_gemm_f32_workspace_bytes(dm.M, dm.N, dm.K, 1);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32_add(transa, transb, dm.M, dm.N, dm.K, 1.0f, cfp(a), dm.lda, cfp(b),
                               dm.ldb, cfp(d), dm.N, fp(y), dm.N, wsb ? ws.data_ptr() : nullptr,
                               wsb, S()));
  runtime::gemm_profile_end(ev, 2.0 * dm.M * dm.N * dm.K, 2 * transa + transb);
  if (!autograd::any_requires_grad({a, b, d})) return y;
  // The graph of add(d, matmul(a, b)) over the fused values.
  Tensor m = matmul_graph_only(a, b, transa, transb, y);
  return add_graph_only(d, m, y);
}

Tensor bmm_impl(const Tensor& a, const Tensor& b, bool transa, bool transb) {
  check_f32(a, "bmm", "a");
  check_f32(b, "bmm", "b");
  require(a.dim() == 3 && b.dim() == 3 && a.shape()[0] == b.shape()[0],
          "bmm: expected [B,*,*] operands with equal batch");
  const int64_t Bt = a.shape()[0];
  const int64_t M = transa ? a.shape()[2] : a.shape()[1];
  const int64_t K = transa ? a.shape()[1] : a.shape()[2];
  const int64_t kb = transb ? b.shape()[2] : b.shape()[1];
  const int64_t N = transb ? b.shape()[1] : b.shape()[2];
  require(K == kb, "bmm: inner dimension mismatch");
  Tensor c = Tensor::empty({Bt, M, N}, DType::kFloat32, a.device());
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32(transa, transb, M, N, K, 1.0f, cfp(a), a.shape()[2],
                           a.shape()[1] * a.shape()[2], cfp(b), b.shape()[2],
                           b.shape()[1] * b.shape()[2], 0.0f, fp(c), N, M * N, Bt, S()));
  runtime::gemm_profile_end(ev, 2.0 * Bt * M * N * K, 2 * transa + transb);
  return c;
}

Tensor bmm(const Tensor& a, const Tensor& b, bool transa, bool transb) {
  Tensor y = bmm_impl(a, b, transa, transb);
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<BmmBackward>();
    node->a = a.detach();
    node->b = b.detach();
    node->ta = transa;
    node->tb = transb;
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

// ================================================================= RMSNorm
namespace {

void check_norm(const Tensor& x, const Tensor& w) {
  check_f32(x, "rms_norm", "x");
  check_f32(w, "rms_norm", "weight");
  require(x.dim() >= 1, "rms_norm: x must have >= 1 dim");
  require(w.dim() == 1 && w.shape()[0] == x.shape().back(), "rms_norm: weight shape mismatch");
}

// dx and dw; with `into`, dx is added into that tensor (which is returned).
std::pair<Tensor, Tensor> rms_bwd(const Tensor& dy, const Tensor& x, const Tensor& w,
                                  const Tensor* rstd, float eps, bool need_dx, bool need_dw,
                                  const Tensor* into = nullptr) {
  const int64_t H = x.shape().back();
  const int64_t rows = x.numel() / H;
  Tensor dx = into ? *into : need_dx ? empty_like(x) : Tensor{};
  Tensor dw = need_dw ? empty_like(w) : Tensor{};
  const size_t wsb = need_dw ? ember_rmsnorm_bwd_workspace_bytes(rows, H) : 0;
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  auto fn = into ? ember_rmsnorm_bwd_accumulate : ember_rmsnorm_bwd;
  CTD_CHECK(fn(cfp(dy), cfp(x), cfp(w), rstd ? cfp(*rstd) : nullptr,
               dx.storage() ? fp(dx) : nullptr, need_dw ? fp(dw) : nullptr, rows, H, eps,
               wsb ? ws.data_ptr() : nullptr, wsb, S()));
  return {dx, dw};
}

struct RmsNormBackward : autograd::Node {
  Tensor x, w, rstd;
  float eps = 1e-5f;
  const char* name() const override { return "RmsNormBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    return backward_with_partials(go, {});
  }
  // dx goes straight into the running sum the engine already holds for x
  // (the residual stream's other gradient), as MatmulBackward does for dA.
  bool accepts_partials() const override { return true; }
  std::vector<Tensor> backward_with_partials(const std::vector<Tensor>& go,
                                             const std::vector<Tensor>& partials) override {
    autograd::NoGradGuard ng;
    check_f32(go.at(0), "rms_norm backward", "grad");
    const bool need_dx = next_edges.at(0).node != nullptr;
    const Tensor* into = partials.empty() ? nullptr : &partials[0];
    const bool fold = need_dx && into && into->storage() && into->dtype() == DType::kFloat32 &&
                      into->device() == x.device() && into->is_contiguous() &&
                      into->shape() == x.shape();
    auto r = rms_bwd(go[0], x, w, &rstd, eps, need_dx, next_edges.at(1).node != nullptr,
                     fold ? into : nullptr);
    release_saved(x, w, rstd);
    return {r.first, r.second};
  }
};

}  // namespace

Tensor rms_norm_impl(const Tensor& x, const Tensor& weight, float eps) {
  check_norm(x, weight);
  const int64_t H = x.shape().back();
  Tensor y = empty_like(x);
  CTD_CHECK(ember_rmsnorm_fwd(cfp(x), cfp(weight), fp(y), nullptr, x.numel() / H, H, eps, S()));
  return y;
}

std::pair<Tensor, Tensor> rms_norm_backward_impl(const Tensor& dy, const Tensor& x,
                                                 const Tensor& w, float eps) {
  check_norm(x, w);
  check_f32(dy, "rms_norm backward", "dy");
  require(dy.shape() == x.shape(), "rms_norm backward: dy shape mismatch");
  return rms_bwd(dy, x, w, nullptr, eps, true, true);
}

Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps) {
  check_norm(x, weight);
  if (!autograd::any_requires_grad({x, weight})) return rms_norm_impl(x, weight, eps);
  const int64_t H = x.shape().back();
  const int64_t rows = x.numel() / H;
  Tensor y = empty_like(x);
  Tensor rstd = Tensor::empty({rows}, DType::kFloat32, x.device());
  CTD_CHECK(ember_rmsnorm_fwd(cfp(x), cfp(weight), fp(y), fp(rstd), rows, H, eps, S()));
  auto node = std::make_shared<RmsNormBackward>();
  node->x = x.detach();
  node->w = weight.detach();
  node->rstd = rstd;
  node->eps = eps;
  node->next_edges = autograd::collect_next_edges({x, weight});
  autograd::set_history(y, std::move(node));
  return y;
}

// ==================================================================== RoPE
namespace {

struct RopeArgs {
  int64_t B, T, H, D;
  float freqs[128];
};

RopeArgs rope_args(const Tensor& x, float theta, const RopeScaling& sc) {
  check_f32(x, "rope");
  require(x.dim() == 4, "rope: expected [B, T, H, D]");
  RopeArgs a{x.shape()[0], x.shape()[1], x.shape()[2], x.shape()[3], {}};
  require(a.D % 2 == 0, "rope: head_dim must be even");
  require(a.D <= 256, "rope: head_dim must be <= 256");
  CTD_CHECK(ember_rope_freqs_host(a.freqs, static_cast<int>(a.D), theta, sc.factor,
                                  sc.low_freq_factor, sc.high_freq_factor, sc.original_max_pos));
  return a;
}

void launch_rope(const Tensor& x, Tensor& y, int pos0, float theta, const RopeScaling& sc,
                 float sign) {
  RopeArgs a = rope_args(x, theta, sc);
  CTD_CHECK(ember_rope(cfp(x), fp(y), a.B, a.T, a.H, a.D, pos0, a.freqs, sign, S()));
}

struct RopeBackward : autograd::Node {
  int position_start = 0;
  float theta = 10000.0f;
  RopeScaling scaling;
  const char* name() const override { return "RopeBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    return {rope_transpose_impl(go.at(0), position_start, theta, scaling)};
  }
};

}  // namespace

void apply_rope_inplace(Tensor& x, int position_start, float theta, const RopeScaling& scaling) {
  launch_rope(x, x, position_start, theta, scaling, 1.0f);
}

Tensor rope_impl(const Tensor& x, int position_start, float theta, const RopeScaling& scaling) {
  Tensor y = Tensor::empty(x.shape(), x.dtype(), x.device());
  launch_rope(x, y, position_start, theta, scaling, 1.0f);
  return y;
}

Tensor rope_transpose_impl(const Tensor& x, int position_start, float theta,
                           const RopeScaling& scaling) {
  Tensor y = Tensor::empty(x.shape(), x.dtype(), x.device());
  launch_rope(x, y, position_start, theta, scaling, -1.0f);
  return y;
}

namespace {

struct QkNormRopeBackward : autograd::Node {
  Tensor x, w, rstd;
  float eps = 1e-6f;
  int position_start = 0;
  RopeArgs args{};
  const char* name() const override { return "QkNormRopeBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    check_f32(go.at(0), "qk_norm_rope backward", "grad");
    const bool need_dx = next_edges.at(0).node != nullptr;
    const bool need_dw = next_edges.at(1).node != nullptr;
    const int64_t rows = args.B * args.T * args.H;
    Tensor dx = need_dx ? empty_like(x) : Tensor{};
    Tensor dw = need_dw ? empty_like(w) : Tensor{};
    const size_t wsb = need_dw ? ember_rmsnorm_bwd_workspace_bytes(rows, args.D) : 0;
    Tensor ws = wsb ? workspace(wsb) : Tensor{};
    CTD_CHECK(ember_qknorm_rope_bwd(cfp(go[0]), cfp(x), cfp(w), cfp(rstd),
                                    need_dx ? fp(dx) : nullptr, need_dw ? fp(dw) : nullptr, rows,
                                    args.H, args.T, args.D, eps, position_start, args.freqs,
                                    wsb ? ws.data_ptr() : nullptr, wsb, S()));
    release_saved(x, w, rstd);
    return {dx, dw};
  }
};

}  // namespace

Tensor qk_norm_rope(const Tensor& x, const Tensor& weight, float eps, int position_start,
                    float theta, const RopeScaling& scaling) {
  check_norm(x, weight);
  const RopeArgs a = rope_args(x, theta, scaling);
  if ((a.D != 64 && a.D != 128) || !x.is_contiguous())
    return rope(rms_norm(x, weight, eps), position_start, theta, scaling);
  const int64_t rows = a.B * a.T * a.H;
  const bool grad = autograd::any_requires_grad({x, weight});
  Tensor y = empty_like(x);
  Tensor rstd = grad ? Tensor::empty({rows}, DType::kFloat32, x.device()) : Tensor{};
  CTD_CHECK(ember_qknorm_rope_fwd(cfp(x), cfp(weight), fp(y), grad ? fp(rstd) : nullptr, rows,
                                  a.H, a.T, a.D, eps, position_start, a.freqs, S()));
  if (grad) {
    auto node = std::make_shared<QkNormRopeBackward>();
    node->x = x.detach();
    node->w = weight.detach();
    node->rstd = rstd;
    node->eps = eps;
    node->position_start = position_start;
    node->args = a;
    node->next_edges = autograd::collect_next_edges({x, weight});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor rope(const Tensor& x, int position_start, float theta, const RopeScaling& scaling) {
  Tensor y = rope_impl(x, position_start, theta, scaling);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<RopeBackward>();
    node->position_start = position_start;
    node->theta = theta;
    node->scaling = scaling;
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

// ============================================================= elementwise
namespace {

void check_binary(const Tensor& a, const Tensor& b, const char* op) {
  check_f32(a, op, "a");
  check_f32(b, op, "b");
  require(a.shape() == b.shape(), std::string(op) + ": shape mismatch");
}

struct AddBackward : autograd::Node {
  const char* name() const override { return "AddBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    // Both inputs receive dy; the engine copies on write if a slot is later
    // accumulated into (src/ops/elementwise.cu:177-184 made two copies up front).
    return {go.at(0), go.at(0)};
  }
};

struct MulBackward : autograd::Node {
  Tensor a, b;
  const char* name() const override { return "MulBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    Tensor da, db;
    if (next_edges.at(0).node) da = mul_impl(go.at(0), b);
    if (next_edges.at(1).node) db = mul_impl(go.at(0), a);
    release_saved(a, b);
    return {da, db};
  }
};

struct SiluBackward : autograd::Node {
  Tensor x;
  const char* name() const override { return "SiluBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    Tensor dx = silu_backward_impl(x, go.at(0));
    release_saved(x);
    return {dx};
  }
};

struct SwigluBackward : autograd::Node {
  Tensor g, u;
  const char* name() const override { return "SwigluBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    check_f32(go.at(0), "swiglu backward", "grad");
    // The gradients overwrite gate and up when this node is their only
    // holder and will not run again (the kernel reads each element before it
    // writes it): two [tokens, intermediate] buffers fewer in the MLP's
    // backward.
    const bool reuse = !autograd::graph_retained();
    Tensor dg = reuse && g.storage().use_count() == 1 ? g : empty_like(g);
    Tensor du = reuse && u.storage().use_count() == 1 && u.storage() != g.storage()
                    ? u
                    : empty_like(u);
    CTD_CHECK(ember_swiglu_bwd(cfp(g), cfp(u), cfp(go[0]), fp(dg), fp(du), g.numel(), S()));
    release_saved(g, u);
    return {dg, du};
  }
};

}  // namespace

Tensor add_impl(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "add");
  Tensor y = empty_like(a);
  CTD_CHECK(ember_add(cfp(a), cfp(b), fp(y), a.numel(), S()));
  return y;
}

Tensor add(const Tensor& a, const Tensor& b) {
  Tensor y = add_impl(a, b);
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<AddBackward>();
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor add_graph_only(const Tensor& a, const Tensor& b, const Tensor& values) {
  check_binary(a, b, "add_graph_only");
  require(values.shape() == a.shape(), "add_graph_only: values must have the operands' shape");
  Tensor y = values.detach();
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<AddBackward>();
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor mul_impl(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "mul");
  Tensor y = empty_like(a);
  CTD_CHECK(ember_mul(cfp(a), cfp(b), fp(y), a.numel(), S()));
  return y;
}

Tensor mul(const Tensor& a, const Tensor& b) {
  Tensor y = mul_impl(a, b);
  if (autograd::any_requires_grad({a, b})) {
    auto node = std::make_shared<MulBackward>();
    node->a = a.detach();
    node->b = b.detach();
    node->next_edges = autograd::collect_next_edges({a, b});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor silu_impl(const Tensor& x) {
  check_f32(x, "silu");
  Tensor y = empty_like(x);
  CTD_CHECK(ember_silu(cfp(x), fp(y), x.numel(), S()));
  return y;
}

Tensor silu(const Tensor& x) {
  Tensor y = silu_impl(x);
  if (autograd::any_requires_grad({x})) {
    auto node = std::make_shared<SiluBackward>();
    node->x = x.detach();
    node->next_edges = autograd::collect_next_edges({x});
    autograd::set_history(y, std::move(node));
  }
  return y;
}

Tensor sub_impl(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "sub");
  Tensor y = empty_like(a);
  CTD_CHECK(ember_sub(cfp(a), cfp(b), fp(y), a.numel(), S()));
  return y;
}

Tensor scale_impl(const Tensor& x, float alpha) {
  check_f32(x, "scale");
  Tensor y = empty_like(x);
  CTD_CHECK(ember_scale(cfp(x), alpha, fp(y), x.numel(), S()));
  return y;
}

Tensor silu_backward_impl(const Tensor& x, const Tensor& g) {
  check_binary(x, g, "silu_backward");
  Tensor y = empty_like(x);
  CTD_CHECK(ember_silu_bwd(cfp(x), cfp(g), fp(y), x.numel(), S()));
  return y;
}

Tensor swiglu_impl(const Tensor& g, const Tensor& u) {
  check_binary(g, u, "swiglu");
  Tensor h = empty_like(g);
  CTD_CHECK(ember_swiglu_fwd(cfp(g), cfp(u), fp(h), g.numel(), S()));
  return h;
}

Tensor swiglu_(Tensor& g, const Tensor& u) {
  check_binary(g, u, "swiglu_");
  require(!autograd::any_requires_grad({g, u}),
          "swiglu_: in place on tensors that require grad would lose the saved gate");
  require(g.storage() != u.storage(), "swiglu_: g and u share storage");
  CTD_CHECK(ember_swiglu_fwd(cfp(g), cfp(u), fp(g), g.numel(), S()));
  return g;
}

Tensor swiglu(const Tensor& g, const Tensor& u) {
  Tensor h = swiglu_impl(g, u);
  if (autograd::any_requires_grad({g, u})) {
    auto node = std::make_shared<SwigluBackward>();
    node->g = g.detach();
    node->u = u.detach();
    node->next_edges = autograd::collect_next_edges({g, u});
    autograd::set_history(h, std::move(node));
  }
  return h;
}

// =============================================================== attention
namespace {

struct AttnDims {
  int64_t B, T, H, Hk, D;
};

AttnDims attn_dims(const Tensor& q, const Tensor& k, const Tensor& v) {
  check_f32(q, "causal_attention", "q");
  check_f32(k, "causal_attention", "k");
  check_f32(v, "causal_attention", "v");
  require(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "causal_attention: expected [B,T,H,D]");
  AttnDims d{q.shape()[0], q.shape()[1], q.shape()[2], k.shape()[2], q.shape()[3]};
  require(k.shape() == v.shape(), "causal_attention: k and v shapes differ");
  require(k.shape()[0] == d.B && k.shape()[1] == d.T && k.shape()[3] == d.D,
          "causal_attention: q/k shape mismatch");
  require(d.Hk > 0 && d.H % d.Hk == 0, "causal_attention: num_heads % num_kv_heads != 0");
  require(d.D == 64 || d.D == 128, "causal_attention: head_dim must be 64 or 128");
  return d;
}

// Algorithmic FLOPs of the causal forward: S = Q K^T and O = P V over the
// T(T+1)/2 visible (query, key) pairs.  The backward's four products (dV,
// dP, dQ, dK) are twice this; the kernels execute 2.5x with dS kept (S is
// recomputed), 3.5x without (S and dP recomputed in both passes).
double attn_fwd_flops(const AttnDims& d) {
  return 4.0 * static_cast<double>(d.B) * d.H * d.D * (static_cast<double>(d.T) * (d.T + 1) / 2);
}

std::atomic<int64_t> g_attn_ds_bytes{kAttentionBackwardDsBytes};

constexpr size_t kAttnDsMaxPieces = 16;

// Buffers for the dS that ember_attn_bwd_scattered keeps, whole KV rows
// (one (batch, KV head) pair's strips) each: as many rows as the budget
// holds, in multiples of 8.  They are placed in free blocks the allocator
// already holds, several if need be, so that the 2.2 GB of dS a Qwen3-1.7B
// layer keeps per chunk at B=8, T=4096 needs no contiguous block; the memory held grows
// only when the free blocks hold fewer than 16 rows, and then to 16.  dQ, dK
// and dV are bitwise the same for any rows per chunk; fewer rows leave the
// dK/dV launch too few workgroups to balance the causal triangle's heavy key
// blocks: with 8-row chunks it took 13.2 ms per Qwen3-1.7B layer against
// 8.8 ms with 32-row chunks.
std::vector<Tensor> attn_bwd_ds_buffers(const AttnDims& d) {
  const int64_t budget = g_attn_ds_bytes.load();
  const size_t row = ember_attn_bwd_ds_row_bytes(d.T, d.H, d.Hk);
  const size_t kv_rows = static_cast<size_t>(d.B * d.Hk);
  std::vector<Tensor> bufs;
  if (budget <= 0 || row == 0) return bufs;
  size_t want = std::min(kv_rows, static_cast<size_t>(budget) / row);
  if (want < kv_rows && want >= 8) want -= want % 8;
  if (want == 0) return bufs;
  for (size_t bytes : device_scatter_plan(row, want, std::min<size_t>(want, 16), 8,
                                          kAttnDsMaxPieces))
    bufs.push_back(workspace(bytes));
  return bufs;
}

std::atomic<bool> g_attn_keep_scores{false};

// Buffers for every KV row's scores (ember_attn_fwd_scores), from the free
// blocks first.
std::vector<Tensor> attn_scores_buffers(const AttnDims& d) {
  const size_t row = ember_attn_bwd_ds_row_bytes(d.T, d.H, d.Hk);
  const size_t kv_rows = static_cast<size_t>(d.B * d.Hk);
  std::vector<Tensor> bufs;
  for (size_t bytes : device_scatter_plan(row, kv_rows, kv_rows, 1, kAttnDsMaxPieces))
    bufs.push_back(workspace(bytes));
  return bufs;
}

void buffer_list(std::vector<Tensor>& bufs, std::vector<float*>& ptr, std::vector<size_t>& bytes) {
  for (Tensor& t : bufs) {
    ptr.push_back(fp(t));
    bytes.push_back(static_cast<size_t>(t.numel()) * sizeof(float));
  }
}

struct CausalAttentionBackward : autograd::Node {
  Tensor q, k, v, o, lse;
  std::vector<Tensor> scores;  // the forward's S (set_attention_keep_scores)
  float scale = 1.0f;
  const char* name() const override { return "CausalAttentionBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    const Tensor& dout = go.at(0);
    check_f32(dout, "causal_attention backward", "grad");
    const AttnDims d = attn_dims(q, k, v);
    Tensor dq = empty_like(q), dk = empty_like(k), dv = empty_like(v);
    const size_t wsb = ember_attn_bwd_workspace_bytes_min(d.B, d.T, d.H);
    Tensor ws = workspace(wsb);
    if (!scores.empty() && !autograd::graph_retained()) {
      // dS is written over the scores, so a retained graph takes the path below
      std::vector<float*> s_ptr;
      std::vector<size_t> s_bytes;
      buffer_list(scores, s_ptr, s_bytes);
      void* ev = runtime::gemm_profile_begin();
      CTD_CHECK(ember_attn_bwd_from_scores(cfp(q), cfp(k), cfp(v), cfp(o), cfp(lse), cfp(dout),
                                           fp(dq), fp(dk), fp(dv), d.B, d.T, d.H, d.Hk, d.D,
                                           scale, ws.data_ptr(), wsb, s_ptr.data(),
                                           s_bytes.data(), static_cast<int>(s_ptr.size()), S()));
      runtime::gemm_profile_end(ev, 2.0 * attn_fwd_flops(d), runtime::kProfileAttnBwd);
      scores.clear();
      release_saved(q, k, v, o, lse);
      return {dq, dk, dv};
    }
    std::vector<Tensor> ds = attn_bwd_ds_buffers(d);
    std::vector<float*> ds_ptr;
    std::vector<size_t> ds_bytes;
    for (Tensor& t : ds) {
      ds_ptr.push_back(fp(t));
      ds_bytes.push_back(static_cast<size_t>(t.numel()) * sizeof(float));
    }
    void* ev = runtime::gemm_profile_begin();
    CTD_CHECK(ember_attn_bwd_scattered(cfp(q), cfp(k), cfp(v), cfp(o), cfp(lse), cfp(dout),
                                       fp(dq), fp(dk), fp(dv), d.B, d.T, d.H, d.Hk, d.D, scale,
                                       ws.data_ptr(), wsb, ds_ptr.data(), ds_bytes.data(),
                                       static_cast<int>(ds_ptr.size()), S()));
    runtime::gemm_profile_end(ev, 2.0 * attn_fwd_flops(d), runtime::kProfileAttnBwd);
    release_saved(q, k, v, o, lse);
    if (!autograd::graph_retained()) scores.clear();
    return {dq, dk, dv};
  }
};

}  // namespace

void set_attention_backward_ds_bytes(int64_t bytes) {
  g_attn_ds_bytes.store(bytes < 0 ? kAttentionBackwardDsBytes : bytes);
}

void set_attention_keep_scores(bool on) { g_attn_keep_scores.store(on); }

Tensor causal_attention_impl(const Tensor& q, const Tensor& k, const Tensor& v, float scale,
                             Tensor* lse_out) {
  const AttnDims d = attn_dims(q, k, v);
  Tensor o = empty_like(q);
  Tensor lse = Tensor::empty({d.B, d.H, d.T}, DType::kFloat32, q.device());
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_attn_fwd(cfp(q), cfp(k), cfp(v), fp(o), fp(lse), d.B, d.T, d.H, d.Hk, d.D,
                           scale, S()));
  runtime::gemm_profile_end(ev, attn_fwd_flops(d), runtime::kProfileAttnFwd);
  if (lse_out) *lse_out = lse;
  return o;
}

Tensor causal_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale) {
  const bool grad = autograd::any_requires_grad({q, k, v});
  Tensor lse, o;
  std::vector<Tensor> scores;
  if (grad && g_attn_keep_scores.load()) {
    const AttnDims d = attn_dims(q, k, v);
    o = empty_like(q);
    lse = Tensor::empty({d.B, d.H, d.T}, DType::kFloat32, q.device());
    scores = attn_scores_buffers(d);
    std::vector<float*> s_ptr;
    std::vector<size_t> s_bytes;
    buffer_list(scores, s_ptr, s_bytes);
    const size_t tb = ember_attn_scores_workspace_bytes(d.B, d.H);
    Tensor table = workspace(tb);
    void* ev = runtime::gemm_profile_begin();
    CTD_CHECK(ember_attn_fwd_scores(cfp(q), cfp(k), cfp(v), fp(o), fp(lse), d.B, d.T, d.H, d.Hk,
                                    d.D, scale, s_ptr.data(), s_bytes.data(),
                                    static_cast<int>(s_ptr.size()), table.data_ptr(), tb, S()));
    runtime::gemm_profile_end(ev, attn_fwd_flops(d), runtime::kProfileAttnFwd);
  } else {
    o = causal_attention_impl(q, k, v, scale, &lse);
  }
  if (grad) {
    auto node = std::make_shared<CausalAttentionBackward>();
    node->scores = std::move(scores);
    node->q = q.detach();
    node->k = k.detach();
    node->v = v.detach();
    node->o = o.detach();
    node->lse = lse;
    node->scale = scale;
    node->next_edges = autograd::collect_next_edges({q, k, v});
    autograd::set_history(o, std::move(node));
  }
  return o;
}

}  // namespace ctd::ops
