// Masked cross-entropy and embedding ops.
// Reference: src/ops/loss.cu:104-429 and src/ops/embedding.cu.  The loss keeps
// only lse[N] from the forward (no [N,V] probabilities) and, when its saved
// logits are not shared with anyone else, writes dlogits over them.
#include "ctd/ops/embedding.h"
#include "ctd/ops/loss.h"
#include "op_util.h"

namespace ctd::ops {

using namespace detail;

namespace {

void check_ce(const Tensor& logits, const Tensor& targets, const Tensor& mask) {
  check_f32(logits, "cross_entropy_masked", "logits");
  check_f32(mask, "cross_entropy_masked", "loss_mask");
  require(targets.dtype() == DType::kInt64 && targets.device().is_hip() && targets.is_contiguous(),
          "cross_entropy_masked: targets must be contiguous int64 on the HIP device");
  require(logits.dim() == 2, "cross_entropy_masked: logits must be [N, V]");
  require(targets.dim() == 1 && targets.shape()[0] == logits.shape()[0],
          "cross_entropy_masked: targets shape mismatch");
  require(mask.dim() == 1 && mask.shape()[0] == logits.shape()[0],
          "cross_entropy_masked: loss_mask shape mismatch");
}

struct CeOut {
  Tensor loss, lse, mask_sum;
};

CeOut ce_fwd(const Tensor& logits, const Tensor& targets, const Tensor& mask) {
  check_ce(logits, targets, mask);
  const int64_t N = logits.shape()[0], V = logits.shape()[1];
  CeOut o;
  o.loss = Tensor::empty({1}, DType::kFloat32, logits.device());
  o.mask_sum = Tensor::empty({1}, DType::kFloat32, logits.device());
  o.lse = Tensor::empty({N}, DType::kFloat32, logits.device());
  const size_t wsb = ember_ce_masked_fwd_workspace_bytes(N);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  CTD_CHECK(ember_ce_masked_fwd(cfp(logits), static_cast<const int64_t*>(targets.data_ptr()),
                                cfp(mask), N, V, fp(o.lse), fp(o.loss), fp(o.mask_sum),
                                wsb ? ws.data_ptr() : nullptr, wsb, S()));
  return o;
}

struct CrossEntropyMaskedBackward : autograd::Node {
  Tensor logits, targets, mask, lse, mask_sum;
  const char* name() const override { return "CrossEntropyMaskedBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    const Tensor& dy = go.at(0);
    check_f32(dy, "cross_entropy_masked backward", "grad");
    float ms = 0.0f;
    mask_sum.copy_to_host(&ms);  // the reference also reads it back (loss.cu:392-396)
    if (!(ms > 0.0f))
      throw std::runtime_error("cross_entropy_masked: sum(loss_mask) == 0 in backward");
    const int64_t N = logits.shape()[0], V = logits.shape()[1];
    // Overwrite the logits when this node is their only holder (saves a full [N,V] buffer).
    Tensor dlogits = logits.storage().use_count() == 1 ? logits : empty_like(logits);
    CTD_CHECK(ember_ce_masked_bwd(cfp(logits), static_cast<const int64_t*>(targets.data_ptr()),
                                  cfp(mask), cfp(lse), cfp(dy), cfp(mask_sum), N, V, fp(dlogits),
                                  S()));
    logits = targets = mask = lse = mask_sum = Tensor{};
    return {dlogits, Tensor{}, Tensor{}};
  }
};

Tensor ones_mask(int64_t n, Device dev) {
  Tensor m = Tensor::empty({n}, DType::kFloat32, dev);
  if (n) CTD_CHECK(ember_fill(fp(m), n, 1.0f, S()));
  return m;
}

}  // namespace

Tensor cross_entropy_masked_impl(const Tensor& logits, const Tensor& targets,
                                 const Tensor& loss_mask) {
  return ce_fwd(logits, targets, loss_mask).loss;
}

Tensor cross_entropy_masked(const Tensor& logits, const Tensor& targets,
                            const Tensor& loss_mask) {
  CeOut o = ce_fwd(logits, targets, loss_mask);
  if (autograd::any_requires_grad({logits, targets, loss_mask})) {
    auto node = std::make_shared<CrossEntropyMaskedBackward>();
    node->logits = logits.detach();
    node->targets = targets.detach();
    node->mask = loss_mask.detach();
    node->lse = o.lse;
    node->mask_sum = o.mask_sum;
    node->next_edges = autograd::collect_next_edges({logits, targets, loss_mask});
    autograd::set_history(o.loss, std::move(node));
  }
  return o.loss;
}

// Plain mean cross-entropy = the masked loss with an all-ones mask
// (test_autograd.cpp:397-414 of the reference checks exactly this identity).
Tensor cross_entropy_impl(const Tensor& logits, const Tensor& targets) {
  require(logits.dim() == 2, "cross_entropy: logits must be [N, V]");
  return cross_entropy_masked_impl(logits, targets, ones_mask(logits.shape()[0], logits.device()));
}

Tensor cross_entropy(const Tensor& logits, const Tensor& targets) {
  require(logits.dim() == 2, "cross_entropy: logits must be [N, V]");
  return cross_entropy_masked(logits, targets, ones_mask(logits.shape()[0], logits.device()));
}

// =============================================================== embedding
namespace {

void check_emb(const Tensor& ids, const Tensor& w) {
  require(ids.dtype() == DType::kInt64, "embedding: ids must be int64");
  require(ids.device().is_hip() && ids.is_contiguous(), "embedding: ids must be on the HIP device");
  check_f32(w, "embedding", "weight");
  require(w.dim() == 2, "embedding: weight must be [vocab, hidden]");
}

struct EmbeddingBackward : autograd::Node {
  Tensor ids;
  int64_t vocab = 0;
  const char* name() const override { return "EmbeddingBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    Tensor dw = embedding_backward_impl(ids, go.at(0), vocab);
    ids = Tensor{};
    return {Tensor{}, dw};
  }
};

}  // namespace

Tensor embedding_impl(const Tensor& ids, const Tensor& weight) {
  check_emb(ids, weight);
  const int64_t V = weight.shape()[0], H = weight.shape()[1];
  std::vector<int64_t> shape = ids.shape();
  shape.push_back(H);
  Tensor out = Tensor::empty(shape, DType::kFloat32, weight.device());
  CTD_CHECK(ember_embedding_fwd(static_cast<const int64_t*>(ids.data_ptr()), cfp(weight), fp(out),
                                ids.numel(), H, V, S()));
  return out;
}

Tensor embedding_backward_impl(const Tensor& ids, const Tensor& dy, int64_t vocab) {
  require(ids.dtype() == DType::kInt64 && ids.device().is_hip(), "embedding_backward: bad ids");
  check_f32(dy, "embedding_backward", "dy");
  const int64_t n = ids.numel();
  require(n > 0 ? dy.numel() % n == 0 : true, "embedding_backward: dy shape mismatch");
  const int64_t H = n ? dy.numel() / n : dy.shape().back();
  Tensor dw = Tensor::empty({vocab, H}, DType::kFloat32, dy.device());
  const size_t wsb = ember_embedding_bwd_workspace_bytes(n, vocab);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  CTD_CHECK(ember_embedding_bwd(static_cast<const int64_t*>(ids.data_ptr()), cfp(dy), fp(dw), n, H,
                                vocab, /*accumulate=*/0, wsb ? ws.data_ptr() : nullptr, wsb, S()));
  return dw;
}

Tensor embedding(const Tensor& ids, const Tensor& weight) {
  Tensor out = embedding_impl(ids, weight);
  if (autograd::any_requires_grad({ids, weight})) {
    auto node = std::make_shared<EmbeddingBackward>();
    node->ids = ids.detach();
    node->vocab = weight.shape()[0];
    node->next_edges = autograd::collect_next_edges({ids, weight});
    autograd::set_history(out, std::move(node));
  }
  return out;
}

}  // namespace ctd::ops
