// pybind11 module aargrad._core for the MI355X backend.  Same module name,
// classes, properties, function names, argument names and defaults as the
// reference binding (cppsrc/python/binding.cpp:84-185); every op releases the
// GIL.  Ops of the reference API that this build does not run on the GPU yet
// are still bound and raise RuntimeError when called.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <atomic>
#include <cstring>
#include <sstream>

#include "aar_hip.h"
#include "ops.hpp"
#include "tensor.hpp"

namespace py = pybind11;
using namespace aar;
using gil_release = py::call_guard<py::gil_scoped_release>;

namespace {

DType numpy_to_dtype(const py::dtype& dt) {
  if (dt.is(py::dtype::of<float>())) return DType::Fp32;
  if (dt.is(py::dtype::of<int64_t>())) return DType::Int64;
  if (dt.kind() == 'f' && dt.itemsize() == 2) return DType::Fp16;
  throw std::runtime_error("unsupported numpy dtype; expected float32, float16, or int64");
}

py::dtype dtype_to_numpy(DType d) {
  switch (d) {
    case DType::Fp32: return py::dtype::of<float>();
    case DType::Fp16: return py::dtype("float16");
    case DType::Int64: return py::dtype::of<int64_t>();
    case DType::Bf16: throw std::runtime_error("bf16 has no numpy equivalent");
  }
  throw std::runtime_error("unknown dtype");
}

std::shared_ptr<Tensor> from_numpy(py::array arr, bool requires_grad) {
  auto dt = numpy_to_dtype(arr.dtype());
  py::array contig = py::array::ensure(arr, py::array::c_style);
  std::vector<int64_t> shape(contig.shape(), contig.shape() + contig.ndim());
  auto t = std::make_shared<Tensor>(Tensor::empty(shape, dt, Device::CPU));
  t->set_requires_grad(requires_grad);
  if (t->nbytes()) std::memcpy(t->data(), contig.data(), t->nbytes());
  return t;
}

py::array to_numpy(const Tensor& t) {
  if (t.device != Device::CPU) {
    throw std::runtime_error("to_numpy requires CPU tensor; call .to(Device.CPU) first");
  }
  Tensor src = t.is_contiguous() ? t : contiguous(t);
  std::vector<py::ssize_t> shape(src.shape.begin(), src.shape.end());
  py::array out(dtype_to_numpy(src.dtype), shape);
  if (src.nbytes()) std::memcpy(out.mutable_data(), src.data(), src.nbytes());
  return out;
}

int device_count() {
  int n = 0;
  if (aar_device_count(&n) != AAR_OK) return 0;
  return n;
}

}  // namespace

PYBIND11_MODULE(_core, m) {
  m.doc() = "aargrad core: fp32 tensors with autograd; compute on the MI355X (gfx950) GPU";

  py::enum_<DType>(m, "DType")
      .value("Fp32", DType::Fp32)
      .value("Fp16", DType::Fp16)
      .value("Bf16", DType::Bf16)
      .value("Int64", DType::Int64);

  py::enum_<Device>(m, "Device").value("CPU", Device::CPU).value("CUDA", Device::CUDA);

  py::class_<Tensor, std::shared_ptr<Tensor>>(m, "Tensor")
      .def_static("empty", &Tensor::empty, py::arg("shape"), py::arg("dtype"),
                  py::arg("device") = Device::CPU, gil_release())
      .def_static("zeros", &Tensor::zeros, py::arg("shape"), py::arg("dtype"),
                  py::arg("device") = Device::CPU, gil_release())
      .def_static("ones", &Tensor::ones, py::arg("shape"), py::arg("dtype"),
                  py::arg("device") = Device::CPU, gil_release())
      .def_readonly("shape", &Tensor::shape)
      .def_readonly("strides", &Tensor::strides)
      .def_readonly("storage_offset", &Tensor::storage_offset)
      .def_readonly("dtype", &Tensor::dtype)
      .def_readonly("device", &Tensor::device)
      .def_property("requires_grad", [](const Tensor& t) { return t.requires_grad; },
                    [](Tensor& t, bool r) { t.set_requires_grad(r); })
      .def_property_readonly("is_leaf", &Tensor::is_leaf)
      .def_property_readonly("numel", &Tensor::numel)
      .def("is_contiguous", &Tensor::is_contiguous)
      .def_property_readonly("grad", &Tensor::grad)
      .def("to", &Tensor::to, py::arg("device"), gil_release())
      .def("zero_grad", &Tensor::zero_grad, gil_release())
      .def("backward", py::overload_cast<>(&Tensor::backward), gil_release())
      .def("backward", py::overload_cast<const Tensor&>(&Tensor::backward), py::arg("grad_output"),
           gil_release())
      .def("__repr__", [](const Tensor& t) {
        std::ostringstream s;
        s << "Tensor(shape=[";
        for (size_t i = 0; i < t.shape.size(); ++i) {
          if (i) s << ", ";
          s << t.shape[i];
        }
        s << "], dtype=" << dtype_name(t.dtype) << ", device=" << (t.device == Device::CPU ? "CPU" : "CUDA")
          << ")";
        return s.str();
      });

  m.def("from_numpy", &from_numpy, py::arg("array"), py::arg("requires_grad") = false);
  m.def("to_numpy", &to_numpy, py::arg("tensor"));
  m.def("cuda_synchronize", &device_synchronize, gil_release());

  // Ops on the MI355X path.
  m.def("add", &add, gil_release());
  m.def("matmul", &matmul, gil_release());
  m.def("matmul_a_bt", &matmul_a_bt, gil_release());
  m.def("matmul_at_b", &matmul_at_b, gil_release());
  m.def("softmax", &softmax, gil_release());
  m.def("layernorm", &layernorm, py::arg("x"), py::arg("weight"), py::arg("bias"), py::arg("eps") = 1e-5f,
        gil_release());
  m.def("flash_attention", &flash_attention, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal"),
        gil_release());
  m.def("reshape", &reshape, py::arg("x"), py::arg("shape"), gil_release());
  m.def("transpose", &transpose, py::arg("x"), py::arg("dim_a"), py::arg("dim_b"), gil_release());
  m.def("slice", &slice, py::arg("x"), py::arg("dim"), py::arg("start"), py::arg("end"), gil_release());
  m.def("squeeze", &squeeze, py::arg("x"), py::arg("dim"), gil_release());
  m.def("unsqueeze", &unsqueeze, py::arg("x"), py::arg("dim"), gil_release());
  m.def("contiguous", &contiguous, py::arg("x"), gil_release());

  // Ops of the GPT training step around the path.
  m.def("sub", &sub, gil_release());
  m.def("mul", &mul, gil_release());
  m.def("relu", &relu, gil_release());
  m.def("gelu", &gelu, gil_release());
  m.def("sum_all", &sum_all, gil_release());
  m.def("add_bias", &add_bias, gil_release());
  m.def("scale", &scale, py::arg("x"), py::arg("alpha"), gil_release());
  m.def("scaled_add_inplace", &scaled_add_inplace, py::arg("dst"), py::arg("src"), py::arg("alpha"),
        gil_release());
  m.def("embedding", &embedding, py::arg("weight"), py::arg("ids"), gil_release());
  m.def("cross_entropy", &cross_entropy, py::arg("logits"), py::arg("targets"), py::arg("ignore_index") = -100,
        gil_release());
  m.def("adamw_step", &adamw_step, py::arg("param"), py::arg("grad"), py::arg("m"), py::arg("v"), py::arg("lr"),
        py::arg("beta1"), py::arg("beta2"), py::arg("eps"), py::arg("weight_decay"),
        py::arg("bias_correction1"), py::arg("bias_correction2"), gil_release());
  m.def("manual_seed", &manual_seed, py::arg("seed"));
  m.def("apply_causal_mask", &apply_causal_mask, gil_release());
  m.def("bmm", &bmm, gil_release());
  m.def("bmm_a_bt", &bmm_a_bt, gil_release());
  m.def("bmm_at_b", &bmm_at_b, gil_release());
  m.def("dropout", &dropout, py::arg("x"), py::arg("p"), gil_release());

  // Extensions of this build (not in the reference API).
  m.def("_flash_attention_fwd", &flash_attention_fwd_lse, py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("causal"), gil_release(),
        "Forward flash attention returning (O, lse); lse = m + ln(l) per query row.");
  m.def("_flash_attention_qkv", &flash_attention_qkv, py::arg("qkv"), py::arg("n_heads"), py::arg("causal"),
        gil_release(),
        "Attention over a packed projection [..., T, 3*D] -> [..., T, D]: the MultiHeadAttention "
        "composition (per-head views of q, k, v, flash attention, heads merged back) in one op.");
  m.def("_scaled_add_inplace_multi", &scaled_add_inplace_multi, py::arg("dsts"), py::arg("srcs"), py::arg("alpha"),
        gil_release(), "scaled_add_inplace over lists of tensors, up to 48 per launch (bit-identical).");
  m.def("_adamw_step_multi", &adamw_step_multi, py::arg("params"), py::arg("grads"), py::arg("m"), py::arg("v"),
        py::arg("lr"), py::arg("beta1"), py::arg("beta2"), py::arg("eps"), py::arg("weight_decay"),
        py::arg("bias_correction1"), py::arg("bias_correction2"), gil_release(),
        "adamw_step over lists of tensors, up to 48 per launch (bit-identical).");
  m.def("_linear", &linear, py::arg("x"), py::arg("weight"), py::arg("bias"), gil_release(),
        "x W^T + b as one GEMM with the bias added in its epilogue: the values and gradients of "
        "add_bias(matmul_a_bt(x, W), b).");
  m.def("_mlp_relu", &mlp_relu, py::arg("x"), py::arg("w1"), py::arg("b1"), py::arg("w2"), py::arg("b2"),
        gil_release(),
        "linear(relu(linear(x, w1, b1)), w2, b2) with bias + relu in the first GEMM's epilogue: the "
        "values and gradients of the composition.");
  m.def("_linear_residual", &linear_residual, py::arg("r"), py::arg("a"), py::arg("weight"), gil_release(),
        "r + a W^T as one GEMM with the residual added in its epilogue: the values and gradients of "
        "add(r, matmul_a_bt(a, W)).");
  m.def("_embedding_add", &embedding_add, py::arg("w1"), py::arg("ids1"), py::arg("w2"), py::arg("ids2"),
        gil_release(),
        "add(embedding(w1, ids1), embedding(w2, ids2)) in one lookup-and-add pass: the values and gradients of "
        "the composition.");
  m.def("_mlp_relu_residual", &mlp_relu_residual, py::arg("r"), py::arg("x"), py::arg("w1"), py::arg("b1"),
        py::arg("w2"), py::arg("b2"), gil_release(),
        "r + _mlp_relu(x, w1, b1, w2, b2) with the residual added in the second GEMM's epilogue: the values "
        "and gradients of the composition.");
  m.def("_token_windows", &token_windows, py::arg("tokens"), py::arg("starts"), py::arg("seq_len"),
        gil_release(),
        "(x, y) int64 [len(starts), seq_len] with x[b] = tokens[s:s+T], y[b] = tokens[s+1:s+T+1], "
        "s = starts[b], gathered on the device from a token stream resident there.");
  m.def("_device_count", &device_count);
  m.def("_empty_cache", &device_empty_cache, gil_release());
  m.def("_memory_in_use", &device_bytes_in_use);
  m.def("_memory_cached", &device_bytes_cached);
}
