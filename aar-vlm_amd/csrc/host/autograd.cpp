// Backward engine: iterative DFS topological sort, reverse sweep, gradient
// fan-in through add_grads.  Follows run_backward / add_grads /
// accumulate_into_leaf (cppsrc/autograd/backward.cpp:17-113): same order of
// node visits, same fan-in summation order and the same error messages.  The
// fan-in sum runs on the GPU through aar_add_f32 (the reference's add_cuda).
#include <algorithm>
#include <unordered_map>
#include <unordered_set>

#include "aar_hip.h"
#include "ops.hpp"
#include "tensor.hpp"

namespace aar {

Tensor add_grads(const Tensor& a, const Tensor& b) {
  if (a.shape != b.shape) throw std::runtime_error("autograd: grad shape mismatch");
  if (a.device != b.device) throw std::runtime_error("autograd: grad device mismatch");
  if (a.device == Device::CPU) throw_cpu_compute("add_grads");
  if (a.dtype != DType::Fp32 || b.dtype != DType::Fp32)
    throw std::runtime_error("autograd: only Fp32 gradients are supported");
  Tensor ac = a.is_contiguous() ? a : contiguous(a);
  Tensor bc = b.is_contiguous() ? b : contiguous(b);
  Tensor out = Tensor::empty(ac.shape, ac.dtype, ac.device);
  check_status(aar_add_f32(static_cast<const float*>(ac.data()), static_cast<const float*>(bc.data()),
                           static_cast<float*>(out.data()), (int64_t)ac.numel(), current_stream()),
               "add_grads");
  return out;
}

namespace {

void accumulate_into_leaf(Tensor& leaf, const Tensor& grad) {
  if (!leaf.grad_slot) return;
  auto& slot = *leaf.grad_slot;
  if (slot) {
    slot = std::make_shared<Tensor>(add_grads(*slot, grad));
  } else {
    slot = std::make_shared<Tensor>(grad.is_contiguous() ? grad : contiguous(grad));
  }
}

}  // namespace

void run_backward(const Tensor& root, const Tensor& grad_output) {
  if (!root.grad_fn) return;

  struct Frame {
    std::shared_ptr<Function> fn;
    bool expanded;
  };
  std::vector<Frame> stack;
  std::vector<std::shared_ptr<Function>> order;
  std::unordered_set<Function*> visited;

  stack.push_back({root.grad_fn, false});
  while (!stack.empty()) {
    Frame& top = stack.back();
    if (!top.expanded) {
      if (visited.count(top.fn.get())) {
        stack.pop_back();
        continue;
      }
      visited.insert(top.fn.get());
      top.expanded = true;
      // Copy before pushing: push_back may reallocate and invalidate `top`.
      std::vector<std::shared_ptr<Function>> next;
      for (const auto& edge : top.fn->inputs)
        if (edge.grad_fn && !visited.count(edge.grad_fn.get())) next.push_back(edge.grad_fn);
      for (auto& n : next) stack.push_back({std::move(n), false});
    } else {
      order.push_back(std::move(top.fn));
      stack.pop_back();
    }
  }
  std::reverse(order.begin(), order.end());

  std::unordered_map<Function*, Tensor> grads;
  grads[root.grad_fn.get()] = grad_output;

  for (auto& fn : order) {
    auto it = grads.find(fn.get());
    if (it == grads.end()) continue;
    Tensor grad_at = std::move(it->second);
    grads.erase(it);

    std::vector<Tensor> input_grads = fn->backward(grad_at);
    if (input_grads.size() != fn->inputs.size()) {
      throw std::runtime_error("autograd: backward returned wrong number of grads");
    }
    for (size_t i = 0; i < fn->inputs.size(); ++i) {
      auto& edge = fn->inputs[i];
      if (!edge.needs_grad) continue;
      const Tensor& g = input_grads[i];
      if (edge.grad_fn) {
        auto it2 = grads.find(edge.grad_fn.get());
        if (it2 == grads.end()) {
          grads[edge.grad_fn.get()] = g;
        } else {
          it2->second = add_grads(it2->second, g);
        }
      } else {
        accumulate_into_leaf(edge.leaf, g);
      }
    }
  }
}

}  // namespace aar
