// Reverse-mode engine and activation checkpointing.
//
// Semantics follow src/core/autograd.cu of the reference (thread-local grad
// mode, leaf sinks that alias a leaf's first gradient and add the later ones,
// fan-in sums, checkpoint() re-running its function under a nested backward);
// the engine itself is this build's own design:
//
//  * A backward pass is a BackwardPass object.  A depth-first walk from the
//    root gives every reachable node a frame (its index in the walk) holding
//    the node, its count of producer edges still to arrive, and its inbox: one
//    gradient slot per output of the node.
//  * Ready nodes (every producer delivered) run in priority order: leaf sinks
//    first, then the most recently created node.  Nodes are numbered when they
//    are constructed, so the pass follows the forward in reverse wherever the
//    dependencies allow; a gradient is consumed soon after it is produced and
//    saved activations are released in the reverse order of their creation.
//  * Delivering into an occupied slot adds; the add is done in place unless
//    another tensor shares the slot's storage (AddBackward hands one gradient
//    to both of its inputs without copying it).  A node that accepts partials
//    is offered the slots its edges point at, when the engine alone holds
//    them, and may add its own contribution there inside its kernel.
//  * A node runs once per pass and, unless the pass retains the graph, is
//    released right after it has run (with its saved tensors and its edges).
//    The reference keeps every node alive until backward returns
//    (autograd.cu:170, 251); with retain_graph the nodes and saved tensors are
//    kept, a leaf's first gradient is copied instead of aliased, and the same
//    graph can be walked again.
#include <atomic>
#include <queue>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "ctd/autograd.h"
#include "ctd/runtime.h"
#include "ember_hip.h"

namespace ctd::autograd {

namespace {
thread_local bool t_grad_mode = true;
thread_local bool t_keep_graph = false;
std::atomic<uint64_t> g_node_counter{0};

struct GradModeScope {
  bool saved;
  explicit GradModeScope(bool on) : saved(t_grad_mode) { t_grad_mode = on; }
  ~GradModeScope() { t_grad_mode = saved; }
};

struct KeepGraphScope {
  bool saved;
  explicit KeepGraphScope(bool on) : saved(t_keep_graph) { t_keep_graph = on; }
  ~KeepGraphScope() { t_keep_graph = saved; }
};

Tensor duplicate(const Tensor& t) {
  Tensor c = Tensor::empty(t.shape(), t.dtype(), t.device());
  if (t.nbytes())
    CTD_CHECK(ember_memcpy_async(c.data_ptr(), t.data_ptr(), t.nbytes(), 2,
                                 runtime::compute_stream()));
  return c;
}

void require_same_layout(const Tensor& dst, const Tensor& src, const char* who) {
  if (dst.shape() != src.shape()) {
    std::string msg = std::string(who) + ": shape mismatch: dst=[";
    for (int64_t d : dst.shape()) msg += std::to_string(d) + ",";
    msg += "] src=[";
    for (int64_t d : src.shape()) msg += std::to_string(d) + ",";
    throw std::runtime_error(msg + "]");
  }
  if (dst.dtype() != DType::kFloat32 || src.dtype() != DType::kFloat32)
    throw std::runtime_error(std::string(who) + ": only fp32");
  if (!dst.device().is_hip() || !src.device().is_hip())
    throw std::runtime_error(std::string(who) + ": only HIP device tensors");
}

// The sink of a leaf tensor: it owns no saved state, only a weak link to the
// leaf's metadata (the leaf may be gone by the time the pass reaches it).
class LeafSink final : public Node {
 public:
  explicit LeafSink(const std::shared_ptr<AutogradMeta>& meta) : meta_(meta) {}
  const char* name() const override { return "AccumulateGrad"; }
  std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) override {
    if (grads_out.size() != 1) throw std::runtime_error("AccumulateGrad: expected 1 grad");
    std::shared_ptr<AutogradMeta> meta = meta_.lock();
    const Tensor& g = grads_out[0];
    if (!meta || !g.defined()) return {};
    if (meta->grad.defined()) {
      accumulate_inplace(meta->grad, g);
    } else {
      // A retained graph may hand the same saved tensor over again in a later
      // pass; the leaf then needs storage of its own to add into.
      meta->grad = t_keep_graph ? duplicate(g) : g;
    }
    return {};
  }

 private:
  std::weak_ptr<AutogradMeta> meta_;
};

// dst (a slot the engine holds) += src.  In place only when nothing else can
// observe dst's storage.
void fold_into_slot(Tensor& slot, const Tensor& incoming) {
  const bool shared =
      slot.storage().use_count() > 1 || slot.storage() == incoming.storage();
  if (!shared) {
    accumulate_inplace(slot, incoming);
    return;
  }
  require_same_layout(slot, incoming, "accumulate");
  Tensor sum = Tensor::empty(slot.shape(), slot.dtype(), slot.device());
  if (slot.numel())
    CTD_CHECK(ember_add(static_cast<const float*>(slot.data_ptr()),
                        static_cast<const float*>(incoming.data_ptr()),
                        static_cast<float*>(sum.data_ptr()), slot.numel(),
                        runtime::compute_stream()));
  slot = std::move(sum);
}

Tensor scalar_seed(const Tensor& loss) {
  if (loss.dtype() != DType::kFloat32) throw std::runtime_error("backward: fp32 only");
  if (loss.numel() != 1) throw std::runtime_error("backward: only scalar loss is supported");
  const float one = 1.0f;
  return Tensor::from_host(&one, loss.shape(), loss.dtype(), loss.device());
}

class BackwardPass {
 public:
  BackwardPass(std::shared_ptr<Node> root, uint32_t root_output, bool keep)
      : keep_(keep) {
    index_graph(std::move(root));
    Frame& r = frames_[0];
    r.inbox.resize(root_output + 1);
    root_output_ = root_output;
  }

  void run(Tensor seed) {
    frames_[0].inbox[root_output_] = std::move(seed);
    push_ready(0);
    while (!ready_.empty()) {
      const uint32_t f = ready_.top().second;
      ready_.pop();
      step(f);
    }
  }

 private:
  struct Frame {
    std::shared_ptr<Node> node;
    uint32_t waiting = 0;       // producer edges that have not delivered yet
    std::vector<Tensor> inbox;  // gradient per output of the node
  };

  // Frames in depth-first discovery order; counts each edge into a node.
  void index_graph(std::shared_ptr<Node> root) {
    frame_of_[root.get()] = 0;
    frames_.push_back(Frame{std::move(root), 0, {}});
    std::vector<uint32_t> todo{0};
    while (!todo.empty()) {
      const uint32_t f = todo.back();
      todo.pop_back();
      Node* n = frames_[f].node.get();
      for (const Edge& e : n->next_edges) {
        if (!e.node) continue;
        auto [it, fresh] = frame_of_.try_emplace(e.node.get(), static_cast<uint32_t>(frames_.size()));
        if (fresh) {
          frames_.push_back(Frame{e.node, 0, {}});
          todo.push_back(it->second);
        }
        frames_[it->second].waiting += 1;
      }
    }
  }

  void push_ready(uint32_t f) {
    const Node* n = frames_[f].node.get();
    // Sinks first (they only fold a gradient into a leaf and free the slot),
    // then the most recently created node.
    const uint64_t rank = dynamic_cast<const LeafSink*>(n) ? UINT64_MAX : n->sequence_nr;
    ready_.emplace(rank, f);
  }

  // The slots a partial-accepting node may add into: for each edge, the
  // target's slot when it already holds a gradient nothing else refers to,
  // and no earlier edge of the same node targets that slot.
  std::vector<Tensor> offers_for(const Node& n) {
    std::vector<Tensor> offers(n.next_edges.size());
    for (size_t i = 0; i < n.next_edges.size(); ++i) {
      const Edge& e = n.next_edges[i];
      if (!e.node) continue;
      bool seen = false;
      for (size_t j = 0; j < i && !seen; ++j)
        seen = n.next_edges[j].node == e.node && n.next_edges[j].input_nr == e.input_nr;
      if (seen) continue;
      const Frame& t = frames_[frame_of_.at(e.node.get())];
      if (e.input_nr >= t.inbox.size()) continue;
      const Tensor& slot = t.inbox[e.input_nr];
      if (slot.defined() && slot.storage().use_count() == 1) offers[i] = slot;
    }
    return offers;
  }

  void step(uint32_t f) {
    std::shared_ptr<Node> node = frames_[f].node;
    std::vector<Tensor> incoming = std::move(frames_[f].inbox);
    frames_[f].inbox.clear();

    std::vector<Tensor> offers;
    std::vector<Tensor> outputs;
    if (node->accepts_partials()) {
      offers = offers_for(*node);
      outputs = node->backward_with_partials(incoming, offers);
    } else {
      outputs = node->backward(incoming);
    }
    incoming.clear();
    if (outputs.size() != node->next_edges.size())
      throw std::runtime_error(std::string("backward: node ") + node->name() +
                               " returned wrong number of grads");

    for (size_t i = 0; i < outputs.size(); ++i) {
      const Edge& e = node->next_edges[i];
      if (!e.node) continue;
      const uint32_t t = frame_of_.at(e.node.get());
      const bool summed_in_place = i < offers.size() && offers[i].defined() &&
                                   outputs[i].defined() &&
                                   outputs[i].storage() == offers[i].storage();
      if (i < offers.size()) offers[i] = Tensor{};  // the slot is the engine's alone again
      if (outputs[i].defined() && !summed_in_place) deliver(t, e.input_nr, std::move(outputs[i]));
      if (--frames_[t].waiting == 0) push_ready(t);
    }
    outputs.clear();

    if (keep_) return;
    if (!node->next_edges.empty()) node->consumed = true;
    node->next_edges.clear();
    frames_[f].node.reset();  // releases the node unless a tensor still refers to it
  }

  void deliver(uint32_t t, uint32_t slot_nr, Tensor g) {
    std::vector<Tensor>& inbox = frames_[t].inbox;
    if (inbox.size() <= slot_nr) inbox.resize(slot_nr + 1);
    if (!inbox[slot_nr].defined())
      inbox[slot_nr] = std::move(g);
    else
      fold_into_slot(inbox[slot_nr], g);
  }

  const bool keep_;
  uint32_t root_output_ = 0;
  std::vector<Frame> frames_;
  std::unordered_map<const Node*, uint32_t> frame_of_;
  std::priority_queue<std::pair<uint64_t, uint32_t>> ready_;
};

void backward_from(const std::shared_ptr<AutogradMeta>& meta, Tensor seed, bool keep) {
  if (!meta || !meta->grad_fn) throw std::runtime_error("backward: this tensor has no grad_fn");
  if (meta->grad_fn->consumed)
    throw std::runtime_error("backward: this graph was already consumed by a backward pass; "
                             "run the forward again");
  const KeepGraphScope scope(keep);
  BackwardPass pass(meta->grad_fn, meta->output_nr, keep);
  pass.run(std::move(seed));
}

}  // namespace

Node::Node() : sequence_nr(g_node_counter.fetch_add(1, std::memory_order_relaxed)) {}

bool is_grad_enabled() { return t_grad_mode; }
bool graph_retained() { return t_keep_graph; }
NoGradGuard::NoGradGuard() : prev_(t_grad_mode) { t_grad_mode = false; }
NoGradGuard::~NoGradGuard() { t_grad_mode = prev_; }

bool any_requires_grad(const std::vector<Tensor>& inputs) {
  if (!t_grad_mode) return false;
  for (const Tensor& t : inputs)
    if (t.requires_grad()) return true;
  return false;
}

std::vector<Edge> collect_next_edges(const std::vector<Tensor>& inputs) {
  std::vector<Edge> edges(inputs.size());
  for (size_t i = 0; i < inputs.size(); ++i) {
    const std::shared_ptr<AutogradMeta>& meta = inputs[i].autograd_meta();
    if (!meta) continue;                     // a constant: no edge
    if (meta->grad_fn) {                     // produced by a recorded op
      edges[i] = Edge{meta->grad_fn, meta->output_nr};
    } else if (meta->requires_grad) {        // a leaf: its (shared) sink
      if (!meta->grad_accumulator) meta->grad_accumulator = std::make_shared<LeafSink>(meta);
      edges[i] = Edge{meta->grad_accumulator, 0};
    }
  }
  return edges;
}

void set_history(Tensor& out, std::shared_ptr<Node> node, uint32_t output_nr) {
  // The output gets metadata of its own: a view must not rewrite the history
  // of the tensor it views.
  auto meta = std::make_shared<AutogradMeta>();
  meta->requires_grad = true;
  meta->grad_fn = std::move(node);
  meta->output_nr = output_nr;
  out.mutable_autograd_meta() = std::move(meta);
}

void accumulate_inplace(Tensor& dst, const Tensor& src) {
  require_same_layout(dst, src, "accumulate");
  if (dst.numel() == 0) return;
  CTD_CHECK(ember_accumulate(static_cast<float*>(dst.data_ptr()),
                             static_cast<const float*>(src.data_ptr()), dst.numel(),
                             runtime::compute_stream()));
}

// ------------------------------------------------------------ checkpoint
namespace {

// Keeps the block's input and function; its backward replays the function on
// a fresh leaf copy of the input with the tape on, back-propagates the
// incoming gradient through the replay (parameters accumulate their
// gradients there), and hands the leaf's gradient on.
class RecomputeNode final : public Node {
 public:
  RecomputeNode(std::function<Tensor(const Tensor&)> block, Tensor input)
      : block_(std::move(block)), input_(std::move(input)) {}
  const char* name() const override { return "CheckpointNode"; }

  std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) override {
    if (grads_out.empty() || !grads_out[0].defined()) return {Tensor{}};
    Tensor leaf = input_.detach();
    leaf.requires_grad_(true);
    Tensor replay;
    {
      const GradModeScope tape_on(true);  // the replay must record, whatever the caller's mode
      replay = block_(leaf);
    }
    // The replay's graph is built afresh on every call, so its own pass never
    // needs to keep it; the outer pass's setting decides whether the saved
    // input stays for another recompute.
    replay.backward(grads_out[0], false);
    Tensor g = leaf.grad();
    if (!graph_retained()) input_ = Tensor{};  // the saved activation is not needed again
    return {g};
  }

 private:
  std::function<Tensor(const Tensor&)> block_;
  Tensor input_;
};

}  // namespace

Tensor checkpoint(std::function<Tensor(const Tensor&)> fn, const Tensor& input) {
  if (!t_grad_mode) return fn(input);
  Tensor out;
  {
    const GradModeScope tape_off(false);
    out = fn(input);
  }
  auto node = std::make_shared<RecomputeNode>(std::move(fn), input.detach());
  node->next_edges = collect_next_edges({input});
  set_history(out, std::move(node));
  return out;
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

Tensor Tensor::grad() const { return autograd_meta_ ? autograd_meta_->grad : Tensor{}; }

void Tensor::zero_grad_() {
  if (autograd_meta_) autograd_meta_->grad = Tensor{};
}

void Tensor::backward() { backward(false); }

void Tensor::backward(bool retain_graph) {
  if (!autograd_meta_ || !autograd_meta_->grad_fn)
    throw std::runtime_error("backward: this tensor has no grad_fn");
  autograd::backward_from(autograd_meta_, autograd::scalar_seed(*this), retain_graph);
}

void Tensor::backward(const Tensor& grad_output) { backward(grad_output, false); }

void Tensor::backward(const Tensor& grad_output, bool retain_graph) {
  autograd::backward_from(autograd_meta_, grad_output, retain_graph);
}

Tensor Tensor::detach() const {
  Tensor t = *this;
  t.autograd_meta_.reset();
  return t;
}

}  // namespace ctd
