#pragma once
// Autograd engine: graph nodes, backward pass, activation checkpointing
// (mirrors include/ctd/autograd.h of the reference).

#include <functional>
#include <memory>
#include <vector>

#include "ctd/tensor.h"

namespace ctd::autograd {

class Node;

struct Edge {
  std::shared_ptr<Node> node;
  uint32_t input_nr = 0;
};

class Node {
 public:
  Node();
  virtual ~Node() = default;
  virtual std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) = 0;
  // A node that accepts partials is run through backward_with_partials: for
  // each edge whose input already holds a gradient from an earlier node, in
  // storage nothing else holds, partials[edge] is that running sum (else
  // empty).  The node may add its own gradient for the edge into it in place
  // and return that same tensor for the edge; the engine then adds nothing.
  // Added in this build (the reference always returns a new gradient).
  virtual bool accepts_partials() const { return false; }
  virtual std::vector<Tensor> backward_with_partials(const std::vector<Tensor>& grads_out,
                                                     const std::vector<Tensor>& partials) {
    (void)partials;
    return backward(grads_out);
  }
  virtual const char* name() const { return "Node"; }
  std::vector<Edge> next_edges;
  // Set once a backward pass that does not retain the graph has run this
  // node and released its edges.
  bool consumed = false;
  // Creation order (process-wide counter).  Among the nodes whose inputs are
  // complete, the engine runs the most recently created one first (leaf
  // gradient sinks before any), i.e. the forward in reverse.  Added in this
  // build.
  const uint64_t sequence_nr;
};

struct AutogradMeta {
  bool requires_grad = false;
  Tensor grad;
  std::shared_ptr<Node> grad_fn;
  uint32_t output_nr = 0;
  std::shared_ptr<Node> grad_accumulator;
};

bool is_grad_enabled();

// True while a backward pass runs that keeps its graph for another pass
// (Tensor::backward(..., retain_graph = true)).  Nodes then keep their saved
// tensors and never overwrite them; otherwise each node drops them once it
// has run.  A nested backward (the recompute inside checkpoint) has its own
// setting.
bool graph_retained();

class NoGradGuard {
 public:
  NoGradGuard();
  ~NoGradGuard();
  NoGradGuard(const NoGradGuard&) = delete;
  NoGradGuard& operator=(const NoGradGuard&) = delete;

 private:
  bool prev_;
};

std::vector<Edge> collect_next_edges(const std::vector<Tensor>& inputs);
void set_history(Tensor& out, std::shared_ptr<Node> node, uint32_t output_nr = 0);
bool any_requires_grad(const std::vector<Tensor>& inputs);
void accumulate_inplace(Tensor& dst, const Tensor& src);

// Runs fn(input) without recording the tape and re-runs it with autograd
// during backward.  fn must be a pure function of input and parameter leaves.
Tensor checkpoint(std::function<Tensor(const Tensor&)> fn, const Tensor& input);

}  // namespace ctd::autograd
