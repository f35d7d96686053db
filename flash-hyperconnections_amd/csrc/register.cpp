// PyTorch-ROCm operator registration for flash_hypercons (the counterpart of
// the reference's csrc/register.cpp and the ATen half of csrc/matrix_exp.cu).
//
// Schemas are the reference's (csrc/register.cpp:10-13) plus two debug ops and
// the hyper-connection stream mixing (_hc_mix, its backward and a debug
// variant, fused with exp(h) for 2 <= n <= 4; _hc_apply and its backward with
// exp(h) supplied, for 5 <= n <= 8), which has no counterpart in the reference.
// The implementations sit on the CUDA dispatch key, which ROCm tensors use.
// Each one checks its inputs with the reference's messages
// (csrc/matrix_exp.cu:52-59), allocates the contiguous output in the input
// dtype, and hands raw device pointers, element strides and the lazy-negation
// bit to the C ABI of libflash_hypercons_hip.so on the current HIP stream.
// No staging copies are made (the reference materialises FP32 contiguous
// copies in prepare_matrix, csrc/matrix_exp.cu:35-44).
//
// The autograd kernel of _matrix_exp is registered here as well, so that an
// eager forward + backward never enters Python below the call itself (the
// reference registers it from Python, ops/matrix_exp/__init__.py:61-77).
#include <Python.h>

#include <ATen/ATen.h>
#include <ATen/PythonTorchFunctionTLS.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <torch/autograd.h>
#include <torch/csrc/Exceptions.h>
#include <torch/csrc/autograd/python_variable.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <optional>
#include <tuple>

#include "flash_hypercons.h"

namespace flash_hypercons {
namespace {

int dtype_code(at::ScalarType t) {
  return t == at::kFloat ? FH_DTYPE_F32 : t == at::kBFloat16 ? FH_DTYPE_BF16 : FH_DTYPE_F16;
}

void check_input(const at::Tensor& a) {
  TORCH_CHECK(a.is_cuda() && a.layout() == at::kStrided && a.dim() == 3 && a.size(-1) == a.size(-2) &&
                  a.size(-1) > 1 && a.size(-1) <= 32 &&
                  (a.scalar_type() == at::kFloat || a.scalar_type() == at::kHalf ||
                   a.scalar_type() == at::kBFloat16),
              "expected a strided CUDA [B, N, N] tensor, 2 <= N <= 32, in float32, float16, or bfloat16");
}

void check_direction(const at::Tensor& a, const at::Tensor& d) {
  TORCH_CHECK(d.sizes() == a.sizes() && d.device() == a.device() && d.scalar_type() == a.scalar_type() &&
                  d.layout() == at::kStrided,
              "matrix exponential direction must match the input");
}

struct View {
  const void* data;
  int64_t strides[3];
  int neg;
};

View view_of(const at::Tensor& t) {
  View v;
  v.data = t.const_data_ptr();
  v.strides[0] = t.stride(0);
  v.strides[1] = t.stride(1);
  v.strides[2] = t.stride(2);
  v.neg = t.is_neg() ? 1 : 0;
  return v;
}

hipStream_t current_stream() { return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

void check_status(int rc) { TORCH_CHECK(rc == FH_OK, "flash_hypercons: ", fh_last_error()); }

at::Tensor run(const at::Tensor& a, const std::optional<at::Tensor>& direction, int variant, int32_t* s_out) {
  check_input(a);
  if (direction) check_direction(a, *direction);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  at::Tensor out = at::empty(a.sizes(), a.options());
  if (a.numel() == 0) return out;
  const View x = view_of(a);
  const int n = static_cast<int>(a.size(-1));
  if (direction) {
    const View g = view_of(*direction);
    check_status(fh_expm_launch(x.data, x.strides, x.neg, g.data, g.strides, g.neg, out.mutable_data_ptr(),
                                dtype_code(a.scalar_type()), a.size(0), n, variant, s_out, current_stream()));
  } else {
    check_status(fh_expm_launch(x.data, x.strides, x.neg, nullptr, nullptr, 0, out.mutable_data_ptr(),
                                dtype_code(a.scalar_type()), a.size(0), n, variant, s_out, current_stream()));
  }
  return out;
}

at::Tensor matrix_exp_hip(const at::Tensor& a) { return run(a, std::nullopt, FH_VARIANT_AUTO, nullptr); }

at::Tensor frechet_hip(const at::Tensor& a, const at::Tensor& direction) {
  return run(a, direction, FH_VARIANT_AUTO, nullptr);
}

// Debug: result of the chosen kernel family plus its per-matrix s.
std::tuple<at::Tensor, at::Tensor> expm_debug_hip(const at::Tensor& a, const std::optional<at::Tensor>& direction,
                                                  int64_t variant) {
  check_input(a);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  at::Tensor s = at::empty({a.size(0)}, a.options().dtype(at::kInt));
  at::Tensor out = run(a, direction, static_cast<int>(variant), s.mutable_data_ptr<int32_t>());
  return {out, s};
}

// Debug: (degree, s) int32 [B, 2] and the FP64 norm [B] behind s.
std::tuple<at::Tensor, at::Tensor> expm_params_hip(const at::Tensor& a, const std::optional<at::Tensor>& direction) {
  check_input(a);
  if (direction) check_direction(a, *direction);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  at::Tensor params = at::empty({a.size(0), 2}, a.options().dtype(at::kInt));
  at::Tensor norms = at::empty({a.size(0)}, a.options().dtype(at::kDouble));
  if (a.size(0) == 0) return {params, norms};
  const View x = view_of(a);
  const int n = static_cast<int>(a.size(-1));
  View g{};
  if (direction) g = view_of(*direction);
  check_status(fh_expm_params(x.data, x.strides, x.neg, direction ? g.data : nullptr, direction ? g.strides : nullptr,
                              g.neg, dtype_code(a.scalar_type()), a.size(0), n, params.mutable_data_ptr<int32_t>(),
                              norms.mutable_data_ptr<double>(), current_stream()));
  return {params, norms};
}

// ---- fused hyper-connection stream mixing ---------------------------------

void check_mix(const at::Tensor& h, const at::Tensor& x) {
  TORCH_CHECK(h.is_cuda() && h.layout() == at::kStrided && h.dim() == 3 && h.size(-1) == h.size(-2) &&
                  h.size(-1) >= 2 && h.size(-1) <= 4 &&
                  (h.scalar_type() == at::kFloat || h.scalar_type() == at::kHalf ||
                   h.scalar_type() == at::kBFloat16),
              "mix_streams: expected a strided CUDA [B, n, n] tensor h, 2 <= n <= 4, in float32, float16, or "
              "bfloat16");
  TORCH_CHECK(x.device() == h.device() && x.scalar_type() == h.scalar_type() && x.layout() == at::kStrided &&
                  x.dim() == 3 && x.size(0) == h.size(0) && x.size(1) == h.size(1) && x.size(2) >= 1,
              "mix_streams: expected x [B, n, C] of h's dtype and device, C >= 1");
}

// Rows contiguous, 16-byte aligned, strides and C in whole 16-byte vectors,
// one token's rows spanning < 2 GiB (the kernels' 32-bit buffer offsets):
// what the kernel reads in place; anything else is copied once (the copy's
// token spans n * C elements, which the Python routing keeps < 2 GiB).
at::Tensor streamable(const at::Tensor& x) {
  const int64_t es = static_cast<int64_t>(x.element_size());
  const int64_t v = 16 / es;
  constexpr int64_t kSpan = int64_t{1} << 31;
  const bool ok = !x.is_neg() && x.stride(2) == 1 && x.stride(1) % v == 0 && x.stride(0) % v == 0 &&
                  x.stride(0) >= 0 && x.stride(1) >= 0 && x.size(2) % v == 0 &&
                  reinterpret_cast<uintptr_t>(x.const_data_ptr()) % 16 == 0 && x.stride(1) < kSpan &&
                  ((x.size(1) - 1) * x.stride(1) + x.size(2)) * es < kSpan;
  if (ok) return x;
  at::Tensor c = x.resolve_neg().contiguous();
  if (x.size(2) % v == 0 && reinterpret_cast<uintptr_t>(c.const_data_ptr()) % 16 == 0) return c;
  // C not a whole number of vectors: pad the rows (the padding is never read back).
  const int64_t padded = (x.size(2) + v - 1) / v * v;
  at::Tensor p = at::zeros({x.size(0), x.size(1), padded}, x.options());
  p.narrow(2, 0, x.size(2)).copy_(c);
  return p;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> mix_run(const at::Tensor& h, const at::Tensor& x,
                                                       const std::optional<at::Tensor>& grad, bool want_aux) {
  check_mix(h, x);
  if (grad) TORCH_CHECK(grad->sizes() == x.sizes() && grad->device() == x.device() &&
                            grad->scalar_type() == x.scalar_type(),
                        "mix_streams: grad must match x");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
  const int64_t B = h.size(0), n = h.size(1), C = x.size(2);
  const at::Tensor xs = streamable(x);
  const int64_t Cp = xs.size(2);
  at::Tensor out = at::empty({B, n, Cp}, x.options());
  at::Tensor dh = grad ? at::empty({B, n, n}, h.options()) : at::Tensor();
  at::Tensor aux = want_aux ? at::empty({B, n, n}, h.options().dtype(at::kFloat)) : at::Tensor();
  if (B > 0) {
    const View hv = view_of(h);
    const int64_t x_strides[3] = {xs.stride(0), xs.stride(1), xs.stride(2)};
    float* aux_ptr = want_aux ? aux.mutable_data_ptr<float>() : nullptr;
    if (grad) {
      at::Tensor gs = streamable(*grad);
      if (gs.size(2) != Cp) {  // x needed padding that grad did not: pad grad alike
        at::Tensor p = at::zeros({B, n, Cp}, gs.options());
        p.narrow(2, 0, C).copy_(gs.narrow(2, 0, C));
        gs = p;
      }
      const int64_t g_strides[3] = {gs.stride(0), gs.stride(1), gs.stride(2)};
      check_status(fh_hc_mix_backward(hv.data, hv.strides, hv.neg, xs.const_data_ptr(), x_strides,
                                      gs.const_data_ptr(), g_strides, dh.mutable_data_ptr(), out.mutable_data_ptr(),
                                      aux_ptr, dtype_code(h.scalar_type()), B, static_cast<int>(n), Cp,
                                      current_stream()));
    } else {
      check_status(fh_hc_mix(hv.data, hv.strides, hv.neg, xs.const_data_ptr(), x_strides, out.mutable_data_ptr(),
                             aux_ptr, dtype_code(h.scalar_type()), B, static_cast<int>(n), Cp, current_stream()));
    }
  }
  if (Cp != C) out = out.narrow(2, 0, C).contiguous();
  return {out, dh, aux};
}

at::Tensor hc_mix_hip(const at::Tensor& h, const at::Tensor& x) {
  return std::get<0>(mix_run(h, x, std::nullopt, false));
}

std::tuple<at::Tensor, at::Tensor> hc_mix_backward_hip(const at::Tensor& h, const at::Tensor& x,
                                                       const at::Tensor& grad) {
  auto r = mix_run(h, x, grad, false);
  return {std::get<1>(r), std::get<0>(r)};
}

// Debug: (y or dx, dh or empty, FP32 exp(h) or dE) -- the values the fused
// kernels keep on chip, for checking against the restatement.
std::tuple<at::Tensor, at::Tensor, at::Tensor> hc_mix_aux_hip(const at::Tensor& h, const at::Tensor& x,
                                                              const std::optional<at::Tensor>& grad) {
  auto r = mix_run(h, x, grad, true);
  if (!grad) std::get<1>(r) = at::empty({0}, h.options());
  return r;
}

// ---- stream mixing with exp(h) supplied, 5 <= n <= 8 ------------------------

void check_apply(const at::Tensor& e, const at::Tensor& x) {
  TORCH_CHECK(e.is_cuda() && e.layout() == at::kStrided && e.dim() == 3 && e.size(-1) == e.size(-2) &&
                  e.size(-1) >= 5 && e.size(-1) <= 8 && e.scalar_type() == at::kFloat,
              "hc_apply: expected a strided CUDA float32 [B, n, n] tensor e, 5 <= n <= 8");
  TORCH_CHECK(x.device() == e.device() && x.layout() == at::kStrided && x.dim() == 3 && x.size(0) == e.size(0) &&
                  x.size(1) == e.size(1) && x.size(2) >= 1 &&
                  (x.scalar_type() == at::kFloat || x.scalar_type() == at::kHalf ||
                   x.scalar_type() == at::kBFloat16),
              "hc_apply: expected x [B, n, C] on e's device, C >= 1, in float32, float16, or bfloat16");
}

// (y, empty) forward; (dx, dE) backward.
std::tuple<at::Tensor, at::Tensor> apply_run(const at::Tensor& e, const at::Tensor& x,
                                             const std::optional<at::Tensor>& grad) {
  check_apply(e, x);
  if (grad) TORCH_CHECK(grad->sizes() == x.sizes() && grad->device() == x.device() &&
                            grad->scalar_type() == x.scalar_type(),
                        "hc_apply: grad must match x");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(e.device());
  const int64_t B = e.size(0), n = e.size(1), C = x.size(2);
  const at::Tensor ec = e.resolve_neg().contiguous();
  const at::Tensor xs = streamable(x);
  const int64_t Cp = xs.size(2);
  at::Tensor out = at::empty({B, n, Cp}, x.options());
  at::Tensor de = grad ? at::empty({B, n, n}, e.options()) : at::empty({0}, e.options());
  if (B > 0) {
    const int64_t x_strides[3] = {xs.stride(0), xs.stride(1), xs.stride(2)};
    if (grad) {
      at::Tensor gs = streamable(*grad);
      if (gs.size(2) != Cp) {
        at::Tensor p = at::zeros({B, n, Cp}, gs.options());
        p.narrow(2, 0, C).copy_(gs.narrow(2, 0, C));
        gs = p;
      }
      const int64_t g_strides[3] = {gs.stride(0), gs.stride(1), gs.stride(2)};
      check_status(fh_hc_apply_backward(ec.const_data_ptr<float>(), xs.const_data_ptr(), x_strides,
                                        gs.const_data_ptr(), g_strides, out.mutable_data_ptr(),
                                        de.mutable_data_ptr<float>(), dtype_code(x.scalar_type()), B,
                                        static_cast<int>(n), Cp, current_stream()));
    } else {
      check_status(fh_hc_apply(ec.const_data_ptr<float>(), xs.const_data_ptr(), x_strides, out.mutable_data_ptr(),
                               dtype_code(x.scalar_type()), B, static_cast<int>(n), Cp, current_stream()));
    }
  }
  if (Cp != C) out = out.narrow(2, 0, C).contiguous();
  return {out, de};
}

at::Tensor hc_apply_hip(const at::Tensor& e, const at::Tensor& x) { return std::get<0>(apply_run(e, x, std::nullopt)); }

std::tuple<at::Tensor, at::Tensor> hc_apply_backward_hip(const at::Tensor& e, const at::Tensor& x,
                                                         const at::Tensor& grad) {
  return apply_run(e, x, grad);
}

using MatrixExpOp = c10::TypedOperatorHandle<at::Tensor(const at::Tensor&)>;
using FrechetOp = c10::TypedOperatorHandle<at::Tensor(const at::Tensor&, const at::Tensor&)>;

const MatrixExpOp& matrix_exp_op() {
  static const MatrixExpOp op =
      c10::Dispatcher::singleton().findSchemaOrThrow("flash_hypercons::_matrix_exp", "").typed<at::Tensor(const at::Tensor&)>();
  return op;
}

const FrechetOp& frechet_op() {
  static const FrechetOp op = c10::Dispatcher::singleton()
                                  .findSchemaOrThrow("flash_hypercons::_frechet", "")
                                  .typed<at::Tensor(const at::Tensor&, const at::Tensor&)>();
  return op;
}

// [[A, G], [0, A]] in FP32; exp of it holds L(A, G) in its top-right block.
at::Tensor frechet_block(const at::Tensor& input, const at::Tensor& direction) {
  const at::Tensor a = input.to(at::kFloat);
  const at::Tensor g = direction.to(at::kFloat);
  return at::cat({at::cat({a, g}, -1), at::cat({at::zeros_like(a), a}, -1)}, -2);
}

at::Tensor top_right(const at::Tensor& e, int64_t n, at::ScalarType dtype) {
  return e.narrow(-2, 0, n).narrow(-1, n, n).to(dtype);
}

// Reference ops/matrix_exp/__init__.py:32-37: the native block exponential.
at::Tensor frechet_reference(const at::Tensor& input, const at::Tensor& direction) {
  return top_right(at::linalg_matrix_exp(frechet_block(input, direction)), input.size(-1), input.scalar_type());
}

// The same block through this operator (2N <= 32): differentiable, and its
// own gradient is again the Frechet kernel.
at::Tensor frechet_differentiable(const at::Tensor& input, const at::Tensor& direction) {
  return top_right(matrix_exp_op().call(frechet_block(input, direction)), input.size(-1), input.scalar_type());
}

// Whether a tensor's Python object (if Python ever saw it) is of a type other
// than torch.Tensor, i.e. may override __torch_function__.  Decided without the
// interpreter: the object stays alive while the tensor does, and its type
// pointer is fixed.
bool python_type_may_override(const at::Tensor& t) {
  PyObject* obj = t.unsafeGetTensorImpl()->pyobj_slot()->load_pyobj();
  return obj != nullptr && Py_TYPE(obj) != reinterpret_cast<PyTypeObject*>(THPVariableClass);
}

// The reference's first backward branch (ops/matrix_exp/__init__.py:67-73):
// when has_torch_function((input, grad_output)) holds -- a __torch_function__
// mode is active where the engine runs (the engine carries the caller's mode
// stack into the backward; torch.autograd.grad and Tensor.backward themselves
// dispatch through an active mode, which is popped while its handler runs) or
// an argument's Python type overrides __torch_function__ -- the gradient is
// the native block exponential computed in Python, so that subclasses see (and
// wrap) every call as they do in the reference.  The
// check and that computation are the Python module's
// (_torch_function_backward), called under the GIL only when the mode stack
// or an argument's type can make the answer yes; otherwise returns an
// undefined tensor at the cost of three loads.
at::Tensor torch_function_gradient(const at::Tensor& input, const at::Tensor& grad) {
  if (!at::impl::torch_function_mode_enabled() && !python_type_may_override(input) &&
      !python_type_may_override(grad))
    return {};
  pybind11::gil_scoped_acquire gil;
  at::Tensor out;
  PyObject* module = PyImport_ImportModule("flash_hypercons.ops.matrix_exp");
  PyObject* py_input = module ? THPVariable_Wrap(input) : nullptr;
  PyObject* py_grad = py_input ? THPVariable_Wrap(grad) : nullptr;
  PyObject* result =
      py_grad ? PyObject_CallMethod(module, "_torch_function_backward", "OO", py_input, py_grad) : nullptr;
  if (result != nullptr && result != Py_None) {
    if (THPVariable_Check(result)) out = THPVariable_Unpack(result);
    else PyErr_SetString(PyExc_TypeError, "_torch_function_backward must return a Tensor or None");
  }
  Py_XDECREF(result);
  Py_XDECREF(py_grad);
  Py_XDECREF(py_input);
  Py_XDECREF(module);
  if (PyErr_Occurred()) {
    python_error err;  // holds the Python exception; the engine re-raises it in the caller
    err.persist();
    throw std::move(err);
  }
  return out;
}

// Gradient of exp at A against G, L(A^T, G) (reference :65-74).  The
// __torch_function__ branch first (above); forward-mode tangents take the
// native block exponential, as the reference does; a backward that builds a
// graph (create_graph=True) takes the differentiable block through this
// operator; otherwise the Frechet kernel.  Tensors with a __torch_dispatch__
// (fake, functional, user subclasses) take the same branches and reach their
// handlers through the dispatcher.
at::Tensor exp_gradient(const at::Tensor& input, const at::Tensor& grad) {
  if (at::Tensor via_python = torch_function_gradient(input, grad); via_python.defined()) return via_python;
  const at::Tensor a = input.mT();
  if (input._fw_grad(0).defined() || grad._fw_grad(0).defined()) return frechet_reference(a, grad);
  if (at::GradMode::is_enabled()) {
    return 2 * input.size(-1) <= 32 ? frechet_differentiable(a, grad) : frechet_reference(a, grad);
  }
  return frechet_op().call(a, grad);
}

class MatrixExpFunction : public torch::autograd::Function<MatrixExpFunction> {
 public:
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& input) {
    ctx->save_for_backward({input});
    at::AutoDispatchBelowADInplaceOrView below;
    return matrix_exp_op().call(input);
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const at::Tensor input = ctx->get_saved_variables()[0];
    if (!grads[0].defined()) return {at::Tensor()};
    return {exp_gradient(input, grads[0])};
  }
};

at::Tensor matrix_exp_autograd(const at::Tensor& input) { return MatrixExpFunction::apply(input); }

}  // namespace
}  // namespace flash_hypercons

TORCH_LIBRARY(flash_hypercons, m) {
  m.def("_matrix_exp(Tensor input) -> Tensor");
  m.def("_frechet(Tensor input, Tensor direction) -> Tensor");
  m.def("_expm_debug(Tensor input, Tensor? direction, int variant) -> (Tensor, Tensor)");
  m.def("_expm_params(Tensor input, Tensor? direction=None) -> (Tensor, Tensor)");
  m.def("_hc_mix(Tensor h, Tensor x) -> Tensor");
  m.def("_hc_mix_backward(Tensor h, Tensor x, Tensor grad) -> (Tensor, Tensor)");
  m.def("_hc_mix_aux(Tensor h, Tensor x, Tensor? grad) -> (Tensor, Tensor, Tensor)");
  m.def("_hc_apply(Tensor e, Tensor x) -> Tensor");
  m.def("_hc_apply_backward(Tensor e, Tensor x, Tensor grad) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(flash_hypercons, CUDA, m) {
  m.impl("_matrix_exp", &flash_hypercons::matrix_exp_hip);
  m.impl("_frechet", &flash_hypercons::frechet_hip);
  m.impl("_expm_debug", &flash_hypercons::expm_debug_hip);
  m.impl("_expm_params", &flash_hypercons::expm_params_hip);
  m.impl("_hc_mix", &flash_hypercons::hc_mix_hip);
  m.impl("_hc_mix_backward", &flash_hypercons::hc_mix_backward_hip);
  m.impl("_hc_mix_aux", &flash_hypercons::hc_mix_aux_hip);
  m.impl("_hc_apply", &flash_hypercons::hc_apply_hip);
  m.impl("_hc_apply_backward", &flash_hypercons::hc_apply_backward_hip);
}

TORCH_LIBRARY_IMPL(flash_hypercons, Autograd, m) { m.impl("_matrix_exp", &flash_hypercons::matrix_exp_autograd); }

static PyModuleDef module = {PyModuleDef_HEAD_INIT, "_C", nullptr, -1, nullptr};

PyMODINIT_FUNC PyInit__C() { return PyModule_Create(&module); }
