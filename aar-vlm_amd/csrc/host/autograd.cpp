// Reverse-mode sweep over the recorded graph (the behaviour of the reference's
// run_backward / add_grads, cppsrc/autograd/backward.cpp:17-113).
//
// Two phases:
//  1. `schedule`: the nodes reachable from the root in reverse DFS post-order,
//     where a node's inputs are explored last input first.  Each node is
//     entered once, the first time the walk reaches it.
//  2. `sweep`: nodes run in that order.  Every node owns one pending-gradient
//     slot (indexed by its position in the schedule); a gradient arriving at a
//     slot that already holds one is added to it (held + new, on the GPU), so
//     fan-in sums accumulate in the order the consumers run.  Gradients for
//     leaves go straight into the leaf's grad slot the same way.  A node that
//     fuses fan-ins (Function::fuses_fan_in) is handed the held gradients of
//     its inputs and may return held + new computed by its own kernel, the
//     same sum in the same order without a separate add pass.
// This fixes the summation order of every fan-in to the reference's: its
// stack walk pushes a node's inputs in order and pops the last one first,
// which is the same post-order.  Error messages match the reference's.
#include <algorithm>
#include <optional>
#include <unordered_map>
#include <unordered_set>

#include "aar_hip.h"
#include "ops.hpp"
#include "tensor.hpp"

namespace aar {

namespace {
// The tensor itself when it is dense row-major, else a dense copy.
Tensor dense(const Tensor& t) { return t.is_contiguous() ? t : contiguous(t); }
}  // namespace

Tensor add_grads(const Tensor& a, const Tensor& b) {
  if (a.shape != b.shape) throw std::runtime_error("autograd: grad shape mismatch");
  if (a.device != b.device) throw std::runtime_error("autograd: grad device mismatch");
  if (a.device == Device::CPU) throw_cpu_compute("add_grads");
  if (a.dtype != DType::Fp32 || b.dtype != DType::Fp32)
    throw std::runtime_error("autograd: only Fp32 gradients are supported");
  const Tensor lhs = dense(a);
  const Tensor rhs = dense(b);
  Tensor sum = Tensor::empty(lhs.shape, lhs.dtype, lhs.device);
  check_status(aar_add_f32(static_cast<const float*>(lhs.data()), static_cast<const float*>(rhs.data()),
                           static_cast<float*>(sum.data()), static_cast<int64_t>(lhs.numel()), current_stream()),
               "add_grads");
  return sum;
}

namespace {

using FnPtr = std::shared_ptr<Function>;

// Reverse post-order of the graph below `root`.  An explicit cursor per open
// node walks its inputs from the last to the first; a node is marked when it
// is opened, so a node reachable along several paths is opened once, from
// the first path the walk takes.
std::vector<FnPtr> schedule(const FnPtr& root) {
  struct Open {
    Function* fn;
    size_t remaining;  // inputs not yet looked at: inputs[0, remaining)
  };
  std::vector<FnPtr> post;
  std::unordered_map<Function*, FnPtr> owner;  // keeps each opened node alive and marks it
  std::vector<Open> path;
  auto open = [&](const FnPtr& fn) {
    owner.emplace(fn.get(), fn);
    path.push_back({fn.get(), fn->inputs.size()});
  };
  open(root);
  while (!path.empty()) {
    Open& cur = path.back();
    if (cur.remaining == 0) {
      post.push_back(owner.at(cur.fn));
      path.pop_back();
      continue;
    }
    const FnPtr& next = cur.fn->inputs[--cur.remaining].grad_fn;
    if (next && owner.find(next.get()) == owner.end()) open(next);  // may reallocate `path`
  }
  std::reverse(post.begin(), post.end());
  return post;
}

// Adds `g` into a pending-gradient slot (first arrival is stored as is).
void deposit(std::optional<Tensor>& slot, const Tensor& g) {
  if (slot) {
    slot = add_grads(*slot, g);
  } else {
    slot = g;
  }
}

// Leaf accumulation: the first gradient is stored contiguous, later ones are
// added to the stored one.  Leaves that do not track a gradient are skipped.
void deposit_leaf(Tensor& leaf, const Tensor& g) {
  if (!leaf.grad_slot) return;
  std::shared_ptr<Tensor>& held = *leaf.grad_slot;
  held = std::make_shared<Tensor>(held ? add_grads(*held, g) : dense(g));
}

void sweep(const std::vector<FnPtr>& nodes, const Tensor& seed) {
  std::unordered_map<const Function*, size_t> position;
  position.reserve(nodes.size());
  for (size_t i = 0; i < nodes.size(); ++i) position.emplace(nodes[i].get(), i);
  std::vector<std::optional<Tensor>> pending(nodes.size());
  pending[0] = seed;
  for (size_t i = 0; i < nodes.size(); ++i) {
    if (!pending[i]) continue;  // nothing flowed into this node
    const Tensor upstream = std::move(*pending[i]);
    pending[i].reset();
    Function& fn = *nodes[i];
    std::vector<bool> summed(fn.inputs.size(), false);
    std::vector<Tensor> outs;
    if (fn.fuses_fan_in()) {
      // the gradients already held for this node's inputs, for it to add onto
      std::vector<const Tensor*> held(fn.inputs.size(), nullptr);
      for (size_t k = 0; k < fn.inputs.size(); ++k) {
        Function::Input& in = fn.inputs[k];
        if (!in.needs_grad) continue;
        if (in.grad_fn) {
          std::optional<Tensor>& slot = pending[position.at(in.grad_fn.get())];
          if (slot) held[k] = &*slot;
        } else if (in.leaf.grad_slot && *in.leaf.grad_slot) {
          held[k] = in.leaf.grad_slot->get();
        }
      }
      outs = fn.backward_into(upstream, held, summed);
      summed.resize(fn.inputs.size(), false);
    } else {
      outs = fn.backward(upstream);
    }
    if (outs.size() != fn.inputs.size()) {
      throw std::runtime_error("autograd: backward returned wrong number of grads");
    }
    for (size_t k = 0; k < outs.size(); ++k) {
      Function::Input& in = fn.inputs[k];
      if (!in.needs_grad) continue;
      if (in.grad_fn) {
        std::optional<Tensor>& slot = pending[position.at(in.grad_fn.get())];
        if (summed[k]) {
          slot = outs[k];  // held + new, summed by the producing kernel
        } else {
          deposit(slot, outs[k]);
        }
      } else if (summed[k]) {
        if (in.leaf.grad_slot) *in.leaf.grad_slot = std::make_shared<Tensor>(outs[k]);
      } else {
        deposit_leaf(in.leaf, outs[k]);
      }
    }
  }
}

}  // namespace

void run_backward(const Tensor& root, const Tensor& grad_output) {
  if (!root.grad_fn) return;
  sweep(schedule(root.grad_fn), grad_output);
}

}  // namespace aar
