// Masked cross-entropy and embedding ops.
// Reference: src/ops/loss.cu:104-429 and src/ops/embedding.cu.  The loss keeps
// only lse[N] from the forward (no [N,V] probabilities) and, when its saved
// logits are not shared with anyone else, writes dlogits over them.
#include <algorithm>
#include <atomic>

#include "ctd/ops/embedding.h"
#include "ctd/ops/loss.h"
#include "ember_hip.h"
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
    // Overwrite the logits when this node is their only holder and will not
    // run again (saves a full [N,V] buffer).
    Tensor dlogits = logits.storage().use_count() == 1 && !autograd::graph_retained()
                         ? logits
                         : empty_like(logits);
    CTD_CHECK(ember_ce_masked_bwd(cfp(logits), static_cast<const int64_t*>(targets.data_ptr()),
                                  cfp(mask), cfp(lse), cfp(dy), cfp(mask_sum), N, V, fp(dlogits),
                                  S()));
    release_saved(logits, targets, mask, lse, mask_sum);
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

namespace {

std::atomic<int64_t> g_head_chunk_rows{0};
std::atomic<bool> g_head_active_rows{true};

// Rows per chunk: at most ~0.64 GB of logits (1024 rows at V = 151936), a
// multiple of 256, at least 256.  The chunk is the LM head's largest buffer;
// at this size it fits the holes the layers' activations leave in the
// device allocator's cache, where 4096-row chunks (2.5 GB) made the allocator
// hold ~1.4x the live bytes at Qwen3-0.6B.  The head's GEMMs run at the same
// rate on 1024 rows; dE is read and written once more per chunk.
int64_t head_chunk_rows(int64_t N, int64_t V) {
  if (const int64_t fixed = g_head_chunk_rows.load()) return std::min(N, fixed);
  const int64_t budget = static_cast<int64_t>(0.64e9) / (V * static_cast<int64_t>(sizeof(float)));
  int64_t r = std::max<int64_t>(256, budget / 256 * 256);
  return std::min(N, r);
}

// C = op(A) op(B) (+ C when accumulate) through the C ABI with its split-K workspace.
void head_gemm(bool ta, bool tb, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
               const float* B, int64_t ldb, float* C, int64_t ldc, bool accumulate) {
  const size_t wsb = ember_gemm_f32_workspace_bytes(M, N, K, 1);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32_ws(ta, tb, M, N, K, 1.0f, A, lda, 0, B, ldb, 0,
                              accumulate ? 1.0f : 0.0f, C, ldc, 0, 1,
                              wsb ? ws.data_ptr() : nullptr, wsb, S()));
  runtime::gemm_profile_end(ev, 2.0 * M * N * K, 2 * ta + tb);
}

// head_gemm with M (dim 0) or K (dim 1) cut on the device to the chunk's
// active rows, count[0] - base.
void head_gemm_dyn(bool ta, bool tb, int64_t M, int64_t N, int64_t K, const float* A,
                   int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                   bool accumulate, const int64_t* count, int64_t base, int dim) {
  const size_t wsb = dim == 0 ? ember_gemm_f32_workspace_bytes(M, N, K, 1) : 0;
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  void* ev = runtime::gemm_profile_begin();
  CTD_CHECK(ember_gemm_f32_dyn(ta, tb, M, N, K, 1.0f, A, lda, B, ldb, accumulate ? 1.0f : 0.0f,
                               C, ldc, count, base, dim, wsb ? ws.data_ptr() : nullptr, wsb, S()));
  // Algorithmic flops: the chunk's active rows only.
  const int64_t ext = dim == 0 ? M : K;
  runtime::gemm_profile_end_rows(ev, 2.0 * M * N * K / static_cast<double>(ext), count, base,
                                 ext, 2 * ta + tb);
}

int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }

// The LM head + loss over only the rows whose mask value is nonzero: they are
// listed on the device (ember_mask_rows) and taken `rows` at a time, so the
// three GEMMs run on those rows only, sized on the device.  Row losses land
// at their batch rows (zeros elsewhere), so the loss is the one-pass-per-row
// result bit for bit; dh rows of masked-out tokens are 0, as they are when
// computed.
void head_loss_active_rows(const Tensor& h, const Tensor& w, const int64_t* tg,
                           const Tensor& loss_mask, int64_t rows, Tensor& lse,
                           Tensor& row_loss, const Tensor& one, const Tensor& mask_sum,
                           Tensor& dh, Tensor& dw) {
  const int64_t N = h.shape()[0], H = h.shape()[1], V = w.shape()[0];
  const Device dev = h.device();
  const bool grad = one.defined();
  Tensor list = Tensor::empty({N + 1}, DType::kInt64, dev);
  int64_t* idx = static_cast<int64_t*>(list.data_ptr());
  const int64_t* count = idx + N;
  CTD_CHECK(ember_mask_rows(cfp(loss_mask), N, idx, idx + N, S()));
  CTD_CHECK(ember_fill(fp(row_loss), N, 0.0f, S()));
  if (dh.defined()) CTD_CHECK(ember_fill(fp(dh), N * H, 0.0f, S()));
  // Chunks of whole 16-row stages, so that only the last one is ragged and the
  // device-side row counts, clamped to a chunk, never run into the next one.
  rows = round16(rows);
  const int64_t cap = rows;
  Tensor logits = Tensor::empty({cap, V}, DType::kFloat32, dev);
  Tensor hc = Tensor::empty({cap, H}, DType::kFloat32, dev);
  Tensor dhc = dh.defined() ? Tensor::empty({cap, H}, DType::kFloat32, dev) : Tensor{};
  for (int64_t r0 = 0; r0 < N; r0 += rows) {
    const int64_t n = std::min(rows, N - r0);  // the chunk's capacity; active rows on the device
    CTD_CHECK(ember_rows_gather(cfp(h), H, H, idx, count, r0, cap, fp(hc), S()));
    head_gemm_dyn(false, true, round16(n), V, H, cfp(hc), H, cfp(w), H, fp(logits), V, false,
                  count, r0, 0);
    CTD_CHECK(ember_ce_masked_rows_idx(cfp(logits), tg, cfp(loss_mask), idx, count, r0, n, V,
                                       fp(lse) + r0, fp(row_loss), S()));
    if (!grad) continue;
    CTD_CHECK(ember_ce_masked_bwd_idx(cfp(logits), tg, cfp(loss_mask), cfp(lse) + r0, idx, count,
                                      r0, n, V, cfp(one), cfp(mask_sum), fp(logits), S()));
    if (dh.defined()) {
      head_gemm_dyn(false, false, n, H, V, cfp(logits), V, cfp(w), H, fp(dhc), H, false, count,
                    r0, 0);
      CTD_CHECK(ember_rows_scatter(cfp(dhc), H, idx, count, r0, n, fp(dh), H, S()));
    }
    if (dw.defined())
      head_gemm_dyn(true, false, V, H, round16(n), cfp(logits), V, cfp(hc), H, fp(dw), H, r0 > 0,
                    count, r0, 1);
  }
}

struct LinearCrossEntropyBackward : autograd::Node {
  Tensor dh, dw, mask_sum;  // gradients for an upstream gradient of 1
  bool want_h = false, want_w = false;
  const char* name() const override { return "LinearCrossEntropyBackward"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& go) override {
    autograd::NoGradGuard ng;
    const Tensor& dy = go.at(0);
    check_f32(dy, "linear_cross_entropy_masked backward", "grad");
    float ms = 0.0f, g = 0.0f;
    mask_sum.copy_to_host(&ms);
    if (!(ms > 0.0f))
      throw std::runtime_error("cross_entropy_masked: sum(loss_mask) == 0 in backward");
    dy.copy_to_host(&g);
    // Scaled in place, unless the graph is kept for another pass, which needs
    // the gradients for an upstream gradient of 1 again.
    const bool keep = autograd::graph_retained();
    Tensor gh = want_h ? dh : Tensor{}, gw = want_w ? dw : Tensor{};
    if (g != 1.0f) {
      if (want_h) {
        if (keep) gh = empty_like(dh);
        CTD_CHECK(ember_scale(cfp(dh), g, fp(gh), dh.numel(), S()));
      }
      if (want_w) {
        if (keep) gw = empty_like(dw);
        CTD_CHECK(ember_scale(cfp(dw), g, fp(gw), dw.numel(), S()));
      }
    }
    release_saved(dh, dw, mask_sum);
    return {gh, gw, Tensor{}, Tensor{}};
  }
};

}  // namespace

void set_linear_cross_entropy_chunk_rows(int64_t rows) {
  require(rows >= 0, "set_linear_cross_entropy_chunk_rows: rows must be >= 0");
  g_head_chunk_rows.store(rows);
}

void set_linear_cross_entropy_active_rows(bool on) { g_head_active_rows.store(on); }

Tensor linear_cross_entropy_masked(const Tensor& h, const Tensor& w, const Tensor& targets,
                                   const Tensor& loss_mask) {
  check_f32(h, "linear_cross_entropy_masked", "h");
  check_f32(w, "linear_cross_entropy_masked", "weight");
  check_f32(loss_mask, "linear_cross_entropy_masked", "loss_mask");
  require(h.dim() == 2 && w.dim() == 2 && h.shape()[1] == w.shape()[1],
          "linear_cross_entropy_masked: expected h [N, H] and weight [V, H]");
  const int64_t N = h.shape()[0], H = h.shape()[1], V = w.shape()[0];
  require(targets.dtype() == DType::kInt64 && targets.device().is_hip() &&
              targets.is_contiguous() && targets.dim() == 1 && targets.shape()[0] == N,
          "linear_cross_entropy_masked: targets must be contiguous int64 [N] on the HIP device");
  require(loss_mask.dim() == 1 && loss_mask.shape()[0] == N,
          "linear_cross_entropy_masked: loss_mask shape mismatch");
  const bool want_h = autograd::any_requires_grad({h});
  const bool want_w = autograd::any_requires_grad({w});
  const bool grad = want_h || want_w;
  const Device dev = h.device();
  Tensor loss = Tensor::empty({1}, DType::kFloat32, dev);
  Tensor mask_sum = Tensor::empty({1}, DType::kFloat32, dev);
  Tensor lse = Tensor::empty({N}, DType::kFloat32, dev);
  Tensor row_loss = Tensor::empty({N}, DType::kFloat32, dev);
  const int64_t* tg = static_cast<const int64_t*>(targets.data_ptr());
  Tensor dh, dw, one;
  if (grad) {
    // sum(mask) first: each chunk's dlogits needs it.
    CTD_CHECK(ember_ce_masked_reduce(nullptr, cfp(loss_mask), N, fp(loss), fp(mask_sum), S()));
    one = Tensor::empty({1}, DType::kFloat32, dev);
    CTD_CHECK(ember_fill(fp(one), 1, 1.0f, S()));
    if (want_h) dh = Tensor::empty({N, H}, DType::kFloat32, dev);
    if (want_w) dw = Tensor::empty({V, H}, DType::kFloat32, dev);  // running dlogits^T h
  }
  // The active-row form needs the LDS-DMA GEMM's shapes: H, V in whole
  // 16-k stages, 16-byte aligned operands.
  const bool active_rows = g_head_active_rows.load() && N > 0 && H % 16 == 0 && V % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(h.data_ptr()) % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(w.data_ptr()) % 16 == 0;
  if (active_rows) {
    head_loss_active_rows(h, w, tg, loss_mask, head_chunk_rows(N, V), lse, row_loss, one,
                          mask_sum, dh, dw);
  } else if (N > 0) {
    const int64_t rows = head_chunk_rows(N, V);
    Tensor logits = Tensor::empty({rows, V}, DType::kFloat32, dev);
    for (int64_t r0 = 0; r0 < N; r0 += rows) {
      const int64_t n = std::min(rows, N - r0);
      const float* hc = cfp(h) + r0 * H;
      head_gemm(false, true, n, V, H, hc, H, cfp(w), H, fp(logits), V, false);
      CTD_CHECK(ember_ce_masked_rows(cfp(logits), tg + r0, cfp(loss_mask) + r0, n, V,
                                     fp(lse) + r0, fp(row_loss) + r0, S()));
      if (!grad) continue;
      CTD_CHECK(ember_ce_masked_bwd(cfp(logits), tg + r0, cfp(loss_mask) + r0, cfp(lse) + r0,
                                    cfp(one), cfp(mask_sum), n, V, fp(logits), S()));
      if (want_h) head_gemm(false, false, n, H, V, cfp(logits), V, cfp(w), H, fp(dh) + r0 * H, H,
                            false);
      if (want_w) head_gemm(true, false, V, H, n, cfp(logits), V, hc, H, fp(dw), H, r0 > 0);
    }
  }
  CTD_CHECK(ember_ce_masked_reduce(cfp(row_loss), cfp(loss_mask), N, fp(loss), fp(mask_sum),
                                   S()));
  if (grad) {
    auto node = std::make_shared<LinearCrossEntropyBackward>();
    node->dh = dh;
    node->dw = dw;
    node->mask_sum = mask_sum;
    node->want_h = want_h;
    node->want_w = want_w;
    node->next_edges = autograd::collect_next_edges({h, w, targets, loss_mask});
    autograd::set_history(loss, std::move(node));
  }
  return loss;
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
    return backward_with_partials(go, {});
  }
  // A tied embedding's weight already holds the LM head's dE when this runs:
  // the rows' sums are added into it (each touched row gets dE + its total,
  // the same rounding as a separate dW and add), so no [V, H] dW is
  // allocated, zeroed and added.
  bool accepts_partials() const override { return true; }
  std::vector<Tensor> backward_with_partials(const std::vector<Tensor>& go,
                                             const std::vector<Tensor>& partials) override {
    autograd::NoGradGuard ng;
    const Tensor* into = partials.size() > 1 && partials[1].defined() ? &partials[1] : nullptr;
    Tensor dw;
    if (into && into->dtype() == DType::kFloat32 && into->is_contiguous() &&
        into->device().is_hip() && into->dim() == 2 && into->shape()[0] == vocab) {
      dw = *into;
      embedding_backward_into(ids, go.at(0), dw);
    } else {
      dw = embedding_backward_impl(ids, go.at(0), vocab);
    }
    release_saved(ids);
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

namespace {
// dw (= 0 first unless accumulate) += the rows of dy summed per id.
void embedding_backward_launch(const Tensor& ids, const Tensor& dy, Tensor& dw, bool accumulate) {
  require(ids.dtype() == DType::kInt64 && ids.device().is_hip(), "embedding_backward: bad ids");
  check_f32(dy, "embedding_backward", "dy");
  const int64_t n = ids.numel(), vocab = dw.shape()[0];
  require(n > 0 ? dy.numel() % n == 0 : true, "embedding_backward: dy shape mismatch");
  const int64_t H = n ? dy.numel() / n : dy.shape().back();
  require(dw.dim() == 2 && dw.shape()[1] == H, "embedding_backward: dw shape mismatch");
  const size_t wsb = ember_embedding_bwd_workspace_bytes(n, H, vocab);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  CTD_CHECK(ember_embedding_bwd(static_cast<const int64_t*>(ids.data_ptr()), cfp(dy), fp(dw), n, H,
                                vocab, accumulate ? 1 : 0, wsb ? ws.data_ptr() : nullptr, wsb,
                                S()));
}
}  // namespace

Tensor embedding_backward_impl(const Tensor& ids, const Tensor& dy, int64_t vocab) {
  check_f32(dy, "embedding_backward", "dy");
  const int64_t n = ids.numel();
  const int64_t H = n && dy.numel() % n == 0 ? dy.numel() / n : dy.shape().back();
  Tensor dw = Tensor::empty({vocab, H}, DType::kFloat32, dy.device());
  embedding_backward_launch(ids, dy, dw, false);
  return dw;
}

void embedding_backward_into(const Tensor& ids, const Tensor& dy, Tensor& dw) {
  check_f32(dw, "embedding_backward", "dw");
  embedding_backward_launch(ids, dy, dw, true);
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
