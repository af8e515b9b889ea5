// Autograd engine and activation checkpointing.
//
// Reference: src/core/autograd.cu.  Same semantics: thread-local grad mode,
// AccumulateGrad leaf sinks (a leaf's first grad is aliased, later ones are
// added), dependency counting then a FIFO (Kahn) walk, in-place fan-in
// accumulation, and checkpoint() that runs fn under no-grad and re-runs it with
// a nested backward.  Two deliberate differences, both about memory:
//   - a node is released as soon as it has run (its saved tensors with it)
//     instead of being kept alive until backward returns
//     (keep_alive, autograd.cu:170, 251); the walked graph is consumed, and a
//     second backward through it throws, unless the backward was asked to
//     retain the graph (then nodes keep their saved tensors, a leaf's first
//     gradient is copied rather than aliased so later passes add into
//     storage only the leaf holds, and the graph can be walked again);
//   - fan-in accumulation is done out of place when the slot's storage is
//     shared (e.g. AddBackward hands the same grad to both inputs without
//     copying it), in place otherwise.
#include <queue>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "ctd/autograd.h"
#include "ctd/runtime.h"
#include "ember_hip.h"

namespace ctd::autograd {

namespace {
thread_local bool g_grad_enabled = true;
thread_local bool g_retain_graph = false;

Tensor copy_of(const Tensor& t) {
  Tensor c = Tensor::empty(t.shape(), t.dtype(), t.device());
  if (t.nbytes())
    CTD_CHECK(ember_memcpy_async(c.data_ptr(), t.data_ptr(), t.nbytes(), 2,
                                 runtime::compute_stream()));
  return c;
}

struct AccumulateGrad : public Node {
  std::weak_ptr<AutogradMeta> leaf_meta;
  const char* name() const override { return "AccumulateGrad"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) override {
    if (grads_out.size() != 1) throw std::runtime_error("AccumulateGrad: expected 1 grad");
    auto meta = leaf_meta.lock();
    if (!meta) return {};
    const Tensor& g = grads_out[0];
    if (!meta->grad.storage()) {
      // With the graph retained, g may be a node's saved tensor that a later
      // pass returns again: the leaf gets its own copy to add into.
      meta->grad = g_retain_graph ? copy_of(g) : g;
    } else {
      accumulate_inplace(meta->grad, g);
    }
    return {};
  }
};

}  // namespace

bool is_grad_enabled() { return g_grad_enabled; }
bool graph_retained() { return g_retain_graph; }
NoGradGuard::NoGradGuard() : prev_(g_grad_enabled) { g_grad_enabled = false; }
NoGradGuard::~NoGradGuard() { g_grad_enabled = prev_; }

bool any_requires_grad(const std::vector<Tensor>& inputs) {
  if (!is_grad_enabled()) return false;
  for (const auto& t : inputs)
    if (t.requires_grad()) return true;
  return false;
}

std::vector<Edge> collect_next_edges(const std::vector<Tensor>& inputs) {
  std::vector<Edge> edges;
  edges.reserve(inputs.size());
  for (const auto& t : inputs) {
    const auto& meta = t.autograd_meta();
    if (meta && meta->grad_fn) {
      edges.push_back(Edge{meta->grad_fn, meta->output_nr});
    } else if (meta && meta->requires_grad) {
      if (!meta->grad_accumulator) {
        auto node = std::make_shared<AccumulateGrad>();
        node->leaf_meta = meta;
        meta->grad_accumulator = node;
      }
      edges.push_back(Edge{meta->grad_accumulator, 0});
    } else {
      edges.push_back(Edge{nullptr, 0});
    }
  }
  return edges;
}

void set_history(Tensor& out, std::shared_ptr<Node> node, uint32_t output_nr) {
  auto& meta = out.mutable_autograd_meta();
  // A fresh meta: a view must not share (and overwrite) its source's history.
  meta = std::make_shared<AutogradMeta>();
  meta->requires_grad = true;
  meta->grad_fn = std::move(node);
  meta->output_nr = output_nr;
}

void accumulate_inplace(Tensor& dst, const Tensor& src) {
  if (dst.shape() != src.shape()) {
    std::string m = "accumulate: shape mismatch: dst=[";
    for (auto d : dst.shape()) m += std::to_string(d) + ",";
    m += "] src=[";
    for (auto d : src.shape()) m += std::to_string(d) + ",";
    throw std::runtime_error(m + "]");
  }
  if (dst.dtype() != DType::kFloat32 || src.dtype() != DType::kFloat32)
    throw std::runtime_error("accumulate: only fp32");
  if (!dst.device().is_hip() || !src.device().is_hip())
    throw std::runtime_error("accumulate: only HIP device tensors");
  const int64_t n = dst.numel();
  if (n == 0) return;
  CTD_CHECK(ember_accumulate(static_cast<float*>(dst.data_ptr()),
                             static_cast<const float*>(src.data_ptr()), n,
                             runtime::compute_stream()));
}

namespace {

// dst += src without writing through storage that someone else also holds.
void accumulate_slot(Tensor& slot, const Tensor& incoming) {
  if (slot.storage().use_count() > 1 || slot.storage() == incoming.storage()) {
    Tensor sum = Tensor::empty(slot.shape(), slot.dtype(), slot.device());
    CTD_CHECK(ember_add(static_cast<const float*>(slot.data_ptr()),
                        static_cast<const float*>(incoming.data_ptr()),
                        static_cast<float*>(sum.data_ptr()), slot.numel(),
                        runtime::compute_stream()));
    slot = sum;
  } else {
    accumulate_inplace(slot, incoming);
  }
}

// For each edge of n: the gradient its input already holds, when nothing but
// the engine holds that storage and no earlier edge of n targets the same
// slot (so a node may add into it in place); else an empty tensor.
std::vector<Tensor> partial_sums(const Node& n,
                                 std::unordered_map<Node*, std::vector<Tensor>>& grads_in) {
  std::vector<Tensor> out(n.next_edges.size());
  for (size_t i = 0; i < n.next_edges.size(); ++i) {
    const Edge& e = n.next_edges[i];
    if (!e.node) continue;
    bool repeated = false;
    for (size_t j = 0; j < i; ++j)
      repeated = repeated || (n.next_edges[j].node == e.node &&
                              n.next_edges[j].input_nr == e.input_nr);
    if (repeated) continue;
    auto it = grads_in.find(e.node.get());
    if (it == grads_in.end() || it->second.size() <= e.input_nr) continue;
    const Tensor& slot = it->second[e.input_nr];
    if (slot.storage() && slot.storage().use_count() == 1) out[i] = slot;
  }
  return out;
}

Tensor ones_like_scalar(const Tensor& t) {
  if (t.dtype() != DType::kFloat32) throw std::runtime_error("backward: fp32 only");
  if (t.numel() != 1) throw std::runtime_error("backward: only scalar loss is supported");
  const float one = 1.0f;
  return Tensor::from_host(&one, t.shape(), t.dtype(), t.device());
}

struct RetainScope {
  bool prev;
  explicit RetainScope(bool on) : prev(g_retain_graph) { g_retain_graph = on; }
  ~RetainScope() { g_retain_graph = prev; }
};

void run_backward(const std::shared_ptr<AutogradMeta>& root_meta, Tensor root_grad,
                  bool retain) {
  if (!root_meta || !root_meta->grad_fn)
    throw std::runtime_error("backward: this tensor has no grad_fn");
  const RetainScope scope(retain);
  Node* const root = root_meta->grad_fn.get();
  const uint32_t root_nr = root_meta->output_nr;
  if (root->consumed)
    throw std::runtime_error("backward: this graph was already consumed by a backward pass; "
                             "run the forward again");

  std::unordered_map<Node*, int> indeg;
  std::unordered_map<Node*, std::shared_ptr<Node>> alive;
  {
    std::vector<Node*> stack{root};
    indeg[root] = 0;
    alive[root] = root_meta->grad_fn;
    while (!stack.empty()) {
      Node* cur = stack.back();
      stack.pop_back();
      for (const Edge& e : cur->next_edges) {
        if (!e.node) continue;
        Node* p = e.node.get();
        auto it = indeg.find(p);
        if (it == indeg.end()) {
          indeg[p] = 1;
          alive[p] = e.node;
          stack.push_back(p);
        } else {
          it->second += 1;
        }
      }
    }
  }
  std::unordered_map<Node*, std::vector<Tensor>> grads_in;
  grads_in[root].resize(root_nr + 1);
  grads_in[root][root_nr] = std::move(root_grad);

  std::queue<Node*> ready;
  ready.push(root);
  while (!ready.empty()) {
    Node* n = ready.front();
    ready.pop();
    std::vector<Tensor> out_grads;
    std::vector<Tensor> partials;
    {
      std::vector<Tensor> grads = std::move(grads_in[n]);
      grads_in.erase(n);
      if (n->accepts_partials()) {
        partials = partial_sums(*n, grads_in);
        out_grads = n->backward_with_partials(grads, partials);
      } else {
        out_grads = n->backward(grads);
      }
    }
    if (out_grads.size() != n->next_edges.size())
      throw std::runtime_error(std::string("backward: node ") + n->name() +
                               " returned wrong number of grads");
    for (size_t i = 0; i < out_grads.size(); ++i) {
      const Edge& e = n->next_edges[i];
      if (!e.node) continue;
      Tensor& incoming = out_grads[i];
      Node* p = e.node.get();
      const bool added = i < partials.size() && partials[i].storage() &&
                         incoming.storage() == partials[i].storage();
      if (i < partials.size()) partials[i] = Tensor{};  // the slot's storage is exclusive again
      if (incoming.storage() && !added) {  // (added: the node summed into the slot)
        auto& slots = grads_in[p];
        if (slots.size() <= e.input_nr) slots.resize(e.input_nr + 1);
        if (!slots[e.input_nr].storage()) {
          slots[e.input_nr] = std::move(incoming);
        } else {
          accumulate_slot(slots[e.input_nr], incoming);
        }
      }
      auto it = indeg.find(p);
      if (it != indeg.end() && --it->second == 0) ready.push(p);
    }
    out_grads.clear();
    if (retain) continue;
    // Consume the node: its edges and (when no tensor still refers to it) the
    // node itself with its saved tensors.
    if (!n->next_edges.empty()) n->consumed = true;
    n->next_edges.clear();
    alive.erase(n);
  }
}

}  // namespace

// ------------------------------------------------------------ checkpoint
namespace {
class CheckpointNode : public Node {
 public:
  std::function<Tensor(const Tensor&)> fn;
  Tensor saved_input;
  const char* name() const override { return "CheckpointNode"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) override {
    Tensor inp = saved_input.detach();
    inp.requires_grad_(true);
    Tensor output = fn(inp);
    output.backward(grads_out.at(0));
    return {inp.grad()};
  }
};
}  // namespace

Tensor checkpoint(std::function<Tensor(const Tensor&)> fn, const Tensor& input) {
  if (!is_grad_enabled()) return fn(input);
  Tensor output;
  {
    NoGradGuard no_grad;
    output = fn(input);
  }
  auto node = std::make_shared<CheckpointNode>();
  node->fn = std::move(fn);
  node->saved_input = input.detach();
  node->next_edges = collect_next_edges({input});
  set_history(output, std::move(node));
  return output;
}

}  // namespace ctd::autograd

namespace ctd {

Tensor& Tensor::requires_grad_(bool v) {
  if (!autograd_meta_) autograd_meta_ = std::make_shared<autograd::AutogradMeta>();
  if (v && autograd_meta_->grad_fn)
    throw std::runtime_error("requires_grad_: cannot mark a non-leaf as requires_grad");
  autograd_meta_->requires_grad = v;
  return *this;
}

bool Tensor::requires_grad() const { return autograd_meta_ && autograd_meta_->requires_grad; }

Tensor Tensor::grad() const {
  if (!autograd_meta_) return Tensor{};
  return autograd_meta_->grad;
}

void Tensor::zero_grad_() {
  if (autograd_meta_) autograd_meta_->grad = Tensor{};
}

void Tensor::backward() { backward(false); }

void Tensor::backward(bool retain_graph) {
  if (!autograd_meta_ || !autograd_meta_->grad_fn)
    throw std::runtime_error("backward: this tensor has no grad_fn");
  autograd::run_backward(autograd_meta_, autograd::ones_like_scalar(*this), retain_graph);
}

void Tensor::backward(const Tensor& grad_output) { backward(grad_output, false); }

void Tensor::backward(const Tensor& grad_output, bool retain_graph) {
  autograd::run_backward(autograd_meta_, grad_output, retain_graph);
}

Tensor Tensor::detach() const {
  Tensor t = *this;
  t.autograd_meta_.reset();
  return t;
}

}  // namespace ctd
