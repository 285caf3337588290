// Direct Python bindings of the hot ops (module _fp8_fast), for eager calls.
//
// A torch.ops call parses its arguments against the schema, boxes them and
// goes through the dispatcher: ~2 us of host time per call on the MI355X
// boxes' hosts, more than a small GEMM or act-quant kernel runs. These
// bindings call the same C++ op functions (torch_ops.h) without it. Each
// returns None, so that the Python wrapper takes the torch.ops route, unless
// the call is a plain eager one: every tensor argument exactly a
// torch.Tensor (no subclass such as FakeTensor), none requiring grad, and no
// TorchDispatchMode, torch-function mode or functorch transform active.
// Results and errors are those of the torch.ops route (same functions).
#include <torch/extension.h>

#include <ATen/PythonTorchFunctionTLS.h>
#include <c10/core/impl/LocalDispatchKeySet.h>
#include <c10/core/impl/TorchDispatchModeTLS.h>
#include <torch/csrc/autograd/python_variable.h>

#include "torch_ops.h"

namespace py = pybind11;

namespace {

bool plain_eager_tls() {
  return c10::impl::TorchDispatchModeTLS::stack_len() == 0 &&
         !at::impl::torch_function_mode_enabled() &&
         !c10::impl::tls_is_dispatch_key_included(c10::DispatchKey::FuncTorchDynamicLayerFrontMode);
}

bool plain_tensor(py::handle h) {
  return THPVariable_CheckExact(h.ptr()) && !THPVariable_Unpack(h.ptr()).requires_grad();
}

const at::Tensor& T(py::handle h) { return THPVariable_Unpack(h.ptr()); }

py::object matmul(py::handle A, py::handle B, py::handle As, py::handle Bs, int64_t block_n,
                  int64_t block_k, at::ScalarType out_dtype) {
  if (!(plain_eager_tls() && plain_tensor(A) && plain_tensor(B) && plain_tensor(As) &&
        plain_tensor(Bs)))
    return py::none();
  return py::cast(
      fp8b_torch::w8a8_block_fp8_matmul_dtype(T(A), T(B), T(As), T(Bs), block_n, block_k,
                                              out_dtype));
}

py::object act_quant(py::handle x, int64_t block_size) {
  if (!(plain_eager_tls() && plain_tensor(x))) return py::none();
  return py::cast(fp8b_torch::act_quant(T(x), block_size));
}

py::object silu_and_mul(py::handle out, py::handle x) {
  if (!(plain_eager_tls() && plain_tensor(out) && plain_tensor(x))) return py::none();
  at::Tensor o = T(out);
  fp8b_torch::silu_and_mul(o, T(x));
  return py::reinterpret_borrow<py::object>(out);
}

py::object silu_and_mul_quant(py::handle x, int64_t block_size) {
  if (!(plain_eager_tls() && plain_tensor(x))) return py::none();
  return py::cast(fp8b_torch::silu_and_mul_quant(T(x), block_size));
}

py::object act_quant_matmul(py::handle x, py::handle B, py::handle Bs, int64_t block_n,
                            int64_t block_k, at::ScalarType out_dtype) {
  if (!(plain_eager_tls() && plain_tensor(x) && plain_tensor(B) && plain_tensor(Bs)))
    return py::none();
  return py::cast(
      fp8b_torch::act_quant_matmul(T(x), T(B), T(Bs), block_n, block_k, out_dtype));
}

py::object gemm_nt(py::handle A, py::handle B, py::handle As, py::handle Bs, int64_t block_k) {
  if (!(plain_eager_tls() && plain_tensor(A) && plain_tensor(B) && plain_tensor(As) &&
        plain_tensor(Bs)))
    return py::none();
  return py::cast(fp8b_torch::gemm_fp8_fp8_bf16_nt(T(A), T(B), T(As), T(Bs), block_k));
}

}  // namespace

PYBIND11_MODULE(_fp8_fast, m) {
  m.def("w8a8_block_fp8_matmul_dtype", &matmul);
  m.def("act_quant", &act_quant);
  m.def("silu_and_mul", &silu_and_mul);
  m.def("silu_and_mul_quant", &silu_and_mul_quant);
  m.def("act_quant_matmul", &act_quant_matmul);
  m.def("gemm_fp8_fp8_bf16_nt", &gemm_nt);
}
