"""Differentiation and PyTorch-integration contract on the GPU.

What a caller of the reference can rely on (ops/matrix_exp/__init__.py:32-97,
register.cpp:10-24), checked against FP64 references and closed forms:

* the operator contract itself (``torch.library.opcheck``: schema, fake
  kernels, autograd registration, dynamic shapes) for every operand layout the
  kernels read in place;
* reverse mode of any order, forward mode, and their mixtures;
* ``torch.func`` transforms, which take the native exponential;
* ``torch.compile``: the scoped or direct call is captured as the custom op,
  transforms compile to native graphs;
* autocast leaves the operator's dtype alone, Parameters are routed.

The backward's __torch_function__ branch (a subclass gradient, or a mode active during the
backward, sends it to the native block exponential) is pinned as the reference has it.
Two deliberate differences from the reference are pinned here as well: an
input carrying a forward-mode tangent gets its tangent from the Frechet kernel
(row f1), and a backward that builds a graph differentiates this operator's own
block exponential when 2N <= 32 (row f2).
"""

import math

import pytest
import torch
from torch.profiler import ProfilerActivity, profile

import flash_hypercons as fh
from tests.reference import check_error, check_north_star, reference

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
FRECHET = "flash_hypercons::_frechet"
FORWARD = "flash_hypercons::_matrix_exp"
NATIVE = "aten::linalg_matrix_exp"


def profiled(fn):
    """(result, set of operator names) over fn, autograd threads included."""
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        out = fn()
    return out, {event.key for event in prof.key_averages()}


def operand(values, layout):
    if layout == "contiguous":
        return values.contiguous()
    if layout == "transposed":
        return values.mT.contiguous().mT
    if layout == "negated":
        return torch._neg_view((-values).contiguous())
    if layout == "expanded":
        return values[:1].expand_as(values)
    raise ValueError(layout)


def fp64_grads(a, g, h=None):
    """FP64 first derivative <exp'(A), G> and, with h, the second derivative along h."""
    ref_a = a.detach().double().requires_grad_()
    (first,) = torch.autograd.grad(reference(ref_a), ref_a, g.double(), create_graph=h is not None)
    if h is None:
        return first, None
    (second,) = torch.autograd.grad(first, ref_a, h.double())
    return first, second


@pytest.mark.parametrize("layout", ["contiguous", "transposed", "expanded"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [3, 9, 32])
def test_operator_contract_opcheck(n, dtype, layout):
    values = (torch.randn(3, n, n, device="cuda") * 0.05).to(dtype)
    x = operand(values, layout).detach().requires_grad_()
    torch.library.opcheck(torch.ops.flash_hypercons._matrix_exp.default, (x,))
    d = operand(torch.randn(3, n, n, device="cuda").to(dtype), "transposed")
    torch.library.opcheck(torch.ops.flash_hypercons._frechet.default, (x.detach(), d))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 8, 9, 16, 17, 32])
def test_second_order_reverse_mode(n, dtype):
    """create_graph=True: first and second derivatives against FP64 autograd.  For 2N <= 32 the
    first derivative is this operator's block exponential, so the second one runs the Frechet
    kernel again and no native exponential is involved; beyond, the native block is used."""
    a = (torch.randn(3, n, n, device="cuda") * 0.5).to(dtype).requires_grad_()
    g, h = torch.randn_like(a), torch.randn_like(a)

    def both():
        (first,) = torch.autograd.grad(fh.matrix_exp(a), a, g, create_graph=True)
        (second,) = torch.autograd.grad(first, a, h)
        return first, second

    (first, second), names = profiled(both)
    ref_first, ref_second = fp64_grads(a, g, h)
    check_error(first, ref_first, backward=True)
    check_error(second, ref_second, backward=True)
    assert (FRECHET in names) == (2 * n <= 32)
    assert (NATIVE in names) == (2 * n > 32)


@pytest.mark.parametrize("grad_mode", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 8, 9, 16, 17, 32])
def test_forward_mode_tangent_is_the_frechet_kernel(n, dtype, grad_mode):
    """A dual input: the primal is the forward kernel and the tangent L(A, H) the Frechet kernel
    without the backward's transpose, bit-identical to the operators called directly and within
    the north-star tolerances of FP64; scoped torch.linalg.matrix_exp behaves the same."""
    a = (torch.randn(5, n, n, device="cuda") * 0.7).to(dtype)
    h = torch.randn_like(a)
    for call in (fh.matrix_exp, torch.linalg.matrix_exp):
        with torch.set_grad_enabled(grad_mode), torch.autograd.forward_ad.dual_level(), fh.use_backend():
            dual = torch.autograd.forward_ad.make_dual(a, h)
            out, names = profiled(lambda dual=dual, call=call: call(dual))
            primal, tangent = torch.autograd.forward_ad.unpack_dual(out)
        assert {FORWARD, FRECHET} <= names and NATIVE not in names
        assert torch.equal(primal, torch.ops.flash_hypercons._matrix_exp(a))
        assert torch.equal(tangent, torch.ops.flash_hypercons._frechet(a, h))
        check_north_star(primal, reference(a))
        check_north_star(tangent, reference(a, h), backward=True)


class _LoggingTensor(torch.Tensor):
    """A __torch_function__ subclass that records the functions called on it."""

    calls = []

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        cls.calls.append(getattr(func, "__name__", str(func)))
        return super().__torch_function__(func, types, args, kwargs or {})


@pytest.mark.parametrize("n", [4, 9])
def test_backward_with_a_torch_function_subclass_gradient(n):
    """Reference :67-73: when the upstream gradient's type overrides __torch_function__, the
    backward is the native block exponential computed through that type -- its result is the
    subclass, its calls reach the subclass's handler, no Frechet kernel runs.  A plain gradient
    on the same graph takes the kernel."""
    a = (torch.randn(3, n, n, device="cuda") * 0.3).requires_grad_()
    g_plain = torch.randn(3, n, n, device="cuda")
    g = g_plain.as_subclass(_LoggingTensor)
    _LoggingTensor.calls.clear()
    y = fh.matrix_exp(a)
    (grad,), names = profiled(lambda: torch.autograd.grad(y, a, g))
    assert type(grad) is _LoggingTensor
    assert FRECHET not in names and NATIVE in names
    assert _LoggingTensor.calls, "the subclass saw no call"
    check_error(grad.as_subclass(torch.Tensor), reference(a.detach().mT, g_plain), backward=True)
    y = fh.matrix_exp(a)
    (grad,), names = profiled(lambda: torch.autograd.grad(y, a, g_plain))
    assert type(grad) is torch.Tensor and FRECHET in names and NATIVE not in names


def test_backward_under_a_torch_function_mode():
    """Reference :67-73 as well: has_torch_function is also true while a __torch_function__ mode
    is active during the backward.  torch.autograd.grad and Tensor.backward dispatch through an
    active mode, which is popped while its handler runs, so a backward started inside
    use_backend() still finds no mode and takes the Frechet kernel (in the reference too).  A
    mode that is active when the engine itself runs (entered below the Python entry points) sends
    the backward to the native block exponential.  Parameters (whose type disables
    __torch_function__) take the kernel."""
    from torch.autograd.graph import _engine_run_backward
    from torch.overrides import TorchFunctionMode

    class Passthrough(TorchFunctionMode):
        def __torch_function__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    a = (torch.randn(3, 4, 4, device="cuda") * 0.3).requires_grad_()
    g = torch.randn(3, 4, 4, device="cuda")
    with fh.use_backend():
        y = torch.linalg.matrix_exp(a)
        (scoped,), names = profiled(lambda: torch.autograd.grad(y, a, g))
    assert FRECHET in names and NATIVE not in names
    y = fh.matrix_exp(a)
    with Passthrough():
        (inside,), names = profiled(lambda: _engine_run_backward((y,), (g,), False, False, (a,), True, False))
    assert FRECHET not in names and NATIVE in names
    check_error(inside, reference(a.detach().mT, g), backward=True)
    torch.testing.assert_close(inside, scoped, rtol=1e-5, atol=1e-6)
    p = torch.nn.Parameter(a.detach().clone())
    (grad,), names = profiled(lambda: torch.autograd.grad(fh.matrix_exp(p), p, g))
    assert FRECHET in names and type(grad) is torch.Tensor
    assert torch.equal(grad, scoped)


def test_backward_python_errors_reach_the_caller():
    """An exception raised by a subclass's handler inside the backward's native branch comes back
    to the caller as that exception."""

    class Failing(torch.Tensor):
        @classmethod
        def __torch_function__(cls, func, types, args=(), kwargs=None):
            if getattr(func, "__name__", "") == "cat":
                raise KeyError("from the subclass")
            return super().__torch_function__(func, types, args, kwargs or {})

    a = (torch.randn(2, 4, 4, device="cuda") * 0.3).requires_grad_()
    g = torch.randn(2, 4, 4, device="cuda").as_subclass(Failing)
    y = fh.matrix_exp(a)
    with pytest.raises(KeyError, match="from the subclass"):
        torch.autograd.grad(y, a, g)


@pytest.mark.parametrize("layout", ["transposed", "expanded", "float64"])
def test_forward_mode_tangent_layouts(layout):
    """Tangents the operator cannot take as they are (another dtype) use the native block
    exponential; strided ones (a transposed view, a broadcast with stride 0) go to the kernel."""
    a = torch.randn(4, 4, 4, device="cuda") * 0.5
    if layout == "transposed":
        h = torch.randn(4, 4, 4, device="cuda").mT
    elif layout == "expanded":
        h = torch.randn(1, 4, 4, device="cuda").expand(4, 4, 4)
    else:
        a = a.double()
        h = torch.randn(4, 4, 4, device="cuda", dtype=torch.float64)
    with torch.autograd.forward_ad.dual_level():
        dual = torch.autograd.forward_ad.make_dual(a, h)
        output, names = profiled(lambda: fh.matrix_exp(dual))
        primal, tangent = torch.autograd.forward_ad.unpack_dual(output)
    if layout == "float64":
        assert FORWARD not in names  # float64 is not eligible at all
    else:
        assert FRECHET in names
    check_error(primal, reference(a))
    check_error(tangent, reference(a, h), backward=True)


@pytest.mark.parametrize("n", [4, 9, 16])
def test_reverse_over_forward(n):
    """The tangent built with grad enabled is differentiable: d/dA <L(A, H), W> matches FP64."""
    a = (torch.randn(3, n, n, device="cuda") * 0.5).requires_grad_()
    h, w = torch.randn_like(a), torch.randn_like(a)
    with torch.autograd.forward_ad.dual_level():
        dual = torch.autograd.forward_ad.make_dual(a, h)
        tangent = torch.autograd.forward_ad.unpack_dual(fh.matrix_exp(dual)).tangent
        (grad,) = torch.autograd.grad(tangent, a, w)
    ref_a = a.detach().double().requires_grad_()
    (ref_grad,) = torch.autograd.grad(reference(ref_a, h.double()), ref_a, w.double())
    check_error(tangent, reference(a.detach(), h), backward=True)
    check_error(grad, ref_grad, backward=True)


@pytest.mark.parametrize("dual_input,dual_grad", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("n", [4, 16, 32])
def test_forward_over_reverse_closed_form(n, dual_input, dual_grad):
    """A = a*I commutes with everything, so L(A^T, G) = e^a G exactly.  With a forward tangent I
    on A the gradient's tangent is d/da (e^a G) = e^a G; with a tangent T on G it is e^a T; with
    both, their sum.  a = 0, G = T = I recovers the textbook case L(0, I) = I."""
    for a_val in (0.0, 0.3):
        x = torch.full((2, n, n), 0.0, device="cuda")
        x.diagonal(dim1=-2, dim2=-1).fill_(a_val)
        x.requires_grad_()
        eye = torch.eye(n, device="cuda").expand(2, n, n)
        gval = eye.clone() if a_val == 0.0 else torch.randn(2, n, n, device="cuda")
        tval = eye.clone() if a_val == 0.0 else torch.randn(2, n, n, device="cuda")
        with torch.autograd.forward_ad.dual_level():
            xin = torch.autograd.forward_ad.make_dual(x, eye) if dual_input else x
            g = torch.autograd.forward_ad.make_dual(gval, tval) if dual_grad else gval
            (grad,) = torch.autograd.grad(fh.matrix_exp(xin), xin, g)
            primal, tangent = torch.autograd.forward_ad.unpack_dual(grad)
        scale = math.exp(a_val)
        expected_tangent = (scale * gval if dual_input else 0) + (scale * tval if dual_grad else 0)
        torch.testing.assert_close(primal, scale * gval, rtol=1e-5, atol=1e-5)
        assert tangent is not None
        torch.testing.assert_close(tangent, expected_tangent, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", DTYPES)
def test_function_transforms_take_the_native_path(dtype):
    """jvp, grad and vmap of the exponential: native results (the reference's rule), checked
    against FP64 with the reference's tolerance."""
    a = (torch.randn(2, 4, 4, device="cuda") * 0.05).to(dtype)
    t = torch.randn_like(a) * 0.1
    with fh.use_backend():
        (y, tangent), names = profiled(lambda: torch.func.jvp(torch.linalg.matrix_exp, (a,), (t,)))
        grad = torch.func.grad(lambda x: torch.linalg.matrix_exp(x).sum())(a)
    assert FORWARD not in names
    check_error(y, reference(a))
    check_error(tangent, reference(a, t), backward=True)
    check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
    stacked = torch.stack([a, 2 * a, -a])
    out, names = profiled(lambda: torch.vmap(fh.matrix_exp)(stacked))
    assert FORWARD not in names
    check_error(out, reference(stacked))


@pytest.mark.parametrize("dtype", DTYPES)
def test_nested_transforms_on_diagonal_matrices(dtype):
    """For diagonal D = diag(d): exp(D) = diag(e^d), and the gradient of sum_i w_i exp(D)_ii is
    diag(w e^d), whose jvp along the identity is again diag(w e^d).  grad inside jvp, with and
    without vmap over a batch of such matrices."""
    n = 4
    d = torch.tensor([-0.2, -0.05, 0.1, 0.2], device="cuda", dtype=dtype)
    w = torch.tensor([1.0, 0.5, -2.0, 3.0], device="cuda", dtype=dtype)
    a = d.diag().expand(3, n, n)
    eye = torch.eye(n, device="cuda", dtype=dtype).expand_as(a)
    expected = (w.double() * d.double().exp()).diag().expand_as(a)
    gradient = torch.func.grad(lambda x: (fh.matrix_exp(x).diagonal(dim1=-2, dim2=-1) * w).sum())
    for fn in (gradient, torch.vmap(gradient)):
        primal, tangent = torch.func.jvp(fn, (a,), (eye,))
        check_error(primal, expected, backward=True)
        check_error(tangent, expected, backward=True)


class Captured:
    """torch.compile with a backend that keeps every FX graph it is handed."""

    def __init__(self, fn):
        self.graphs = []

        def backend(gm, inputs):
            self.graphs.append(gm)
            return gm.forward

        self.fn = torch.compile(fn, backend=backend, fullgraph=True)

    def __call__(self, *args):
        return self.fn(*args)

    def targets(self):
        return {node.target for gm in self.graphs for node in gm.graph.nodes}


def _is_custom(target):
    return target in (torch.ops.flash_hypercons._matrix_exp.default, torch.ops.flash_hypercons._matrix_exp)


@pytest.mark.compile
@pytest.mark.parametrize("scoped", [False, True])
def test_compile_captures_the_operator(scoped):
    """Dynamo captures the call (direct, or torch.linalg.matrix_exp inside the scope) as the
    custom op; the compiled function's gradient runs the Frechet kernel; called again outside
    the scope, the scoped function's guards send it back to native."""
    fn = torch.linalg.matrix_exp if scoped else fh.matrix_exp
    a = (torch.randn(3, 9, 9, device="cuda") * 0.03).requires_grad_()
    captured = Captured(fn)
    with fh.use_backend():
        y = captured(a)
        y_inductor = torch.compile(fn, fullgraph=True)(a)
    assert any(_is_custom(t) for t in captured.targets())
    assert torch.equal(y.detach(), torch.ops.flash_hypercons._matrix_exp(a.detach()))
    check_north_star(y_inductor.detach(), reference(a.detach()))
    (grad,), names = profiled(lambda: torch.autograd.grad(y_inductor.sum(), a))
    assert FRECHET in names
    check_north_star(grad, reference(a.detach().mT, torch.ones_like(a)), backward=True)
    if scoped:
        _, names = profiled(lambda: captured(a))
        assert FORWARD not in names


@pytest.mark.compile
@pytest.mark.parametrize("transform", ["grad", "jvp", "vmap"])
def test_compiled_transforms_stay_native(transform):
    a = torch.zeros(2, 4, 4, device="cuda")
    eye = torch.eye(4, device="cuda").expand_as(a)
    fns = {
        "grad": torch.func.grad(lambda x: fh.matrix_exp(x).diagonal(dim1=-2, dim2=-1).sum()),
        "jvp": lambda x: torch.func.jvp(fh.matrix_exp, (x,), (eye,))[1],
        "vmap": torch.vmap(fh.matrix_exp),
    }
    captured = Captured(fns[transform])
    out = captured(a)
    torch.testing.assert_close(out, eye)  # exp(0) = I; d/dA tr exp(A) at 0 = I; L(0, I) = I
    assert not any("flash_hypercons" in str(t) for t in captured.targets())


def test_autocast_leaves_the_operator_dtype():
    p = torch.nn.Parameter(torch.randn(2, 8, 8, device="cuda") * 0.03)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, names = profiled(lambda: fh.matrix_exp(p))
    assert y.dtype == torch.float32 and FORWARD in names
    check_north_star(y.detach(), reference(p.detach()))
    (grad,) = torch.autograd.grad(y.sum(), p)
    check_north_star(grad, reference(p.detach().mT, torch.ones_like(p)), backward=True)
