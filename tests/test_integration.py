"""PyTorch integration on the GPU: opcheck, higher-order and forward-mode AD,
function transforms, torch.compile, autocast and parameters.

Cases follow the reference suite (tests/test_integration.py there).
"""

import pytest
import torch

import flash_hypercons as fh
from tests.reference import check_error, check_north_star, reference
from tests.test_routing import op_names

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("n", [4, 9, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_opcheck(dtype, n):
    a = (torch.randn(3, n, n, device="cuda") * 0.03).to(dtype).mT.detach().requires_grad_()
    torch.library.opcheck(torch.ops.flash_hypercons._matrix_exp.default, (a,))
    torch.library.opcheck(torch.ops.flash_hypercons._frechet.default, (a.detach(), torch.randn_like(a)))


@pytest.mark.parametrize("n", [4, 16, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_double_backward_and_forward_ad(dtype, n):
    a = (torch.randn(2, n, n, device="cuda") * 0.03).to(dtype).requires_grad_()
    g, h = torch.randn_like(a) * 0.1, torch.randn_like(a) * 0.1
    y = fh.matrix_exp(a)
    (first,) = torch.autograd.grad(y, a, g, create_graph=True)
    (second,) = torch.autograd.grad(first, a, h)
    ref_a = a.detach().double().requires_grad_()
    (ref_first,) = torch.autograd.grad(reference(ref_a), ref_a, g.double(), create_graph=True)
    (ref_second,) = torch.autograd.grad(ref_first, ref_a, h.double())
    check_error(first, ref_first, backward=True)
    check_error(second, ref_second, backward=True)
    for grad_enabled in (False, True):
        with torch.set_grad_enabled(grad_enabled), torch.autograd.forward_ad.dual_level(), fh.use_backend():
            dual = torch.autograd.forward_ad.make_dual(a, g)
            output, names = op_names(lambda dual=dual: torch.linalg.matrix_exp(dual))
            primal, tangent = torch.autograd.forward_ad.unpack_dual(output)
            # The reference sends forward-mode inputs to the native exponential; here the
            # primal runs the forward kernel and the tangent the Frechet kernel.
            assert "flash_hypercons::_matrix_exp" in names
            check_error(primal, reference(a))
            check_error(tangent, reference(a, g), backward=True)


@pytest.mark.parametrize("n", [2, 4, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_forward_ad_tangent_from_frechet_kernel(dtype, n):
    """A dual input: the primal is this operator's forward and the tangent L(A, H) its Frechet
    kernel (no transpose), both to the north-star tolerances."""
    a = (torch.randn(5, n, n, device="cuda") * 0.7).to(dtype)
    h = torch.randn_like(a)
    with torch.autograd.forward_ad.dual_level():
        dual = torch.autograd.forward_ad.make_dual(a, h)
        output, names = op_names(lambda: fh.matrix_exp(dual))
        primal, tangent = torch.autograd.forward_ad.unpack_dual(output)
    assert "flash_hypercons::_matrix_exp" in names
    assert "flash_hypercons::_frechet" in names
    assert "aten::linalg_matrix_exp" not in names
    check_north_star(primal, reference(a))
    check_north_star(tangent, reference(a, h), backward=True)
    # Bit-identical to the operators called directly.
    assert torch.equal(primal, torch.ops.flash_hypercons._matrix_exp(a))
    assert torch.equal(tangent, torch.ops.flash_hypercons._frechet(a, h))


@pytest.mark.parametrize("layout", ["transposed", "expanded", "float64"])
def test_forward_ad_tangent_layouts(layout):
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
        output, names = op_names(lambda: fh.matrix_exp(dual))
        primal, tangent = torch.autograd.forward_ad.unpack_dual(output)
    if layout == "float64":
        assert "flash_hypercons::_matrix_exp" not in names  # float64 is not eligible at all
    else:
        assert "flash_hypercons::_frechet" in names
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


@pytest.mark.parametrize("n", [2, 4, 8, 9, 16, 17])
@pytest.mark.parametrize("dtype", DTYPES)
def test_double_backward_stays_on_device(dtype, n):
    """create_graph=True: the first-order gradient is the top-right block of this operator on
    [[A^T, G], [0, A^T]] (2N <= 32), so the second derivative runs the Frechet kernel again;
    beyond 2N = 32 the native block exponential is used as in the reference."""
    a = (torch.randn(3, n, n, device="cuda") * 0.5).to(dtype).requires_grad_()
    g, h = torch.randn_like(a), torch.randn_like(a)

    def second_order():
        (first,) = torch.autograd.grad(fh.matrix_exp(a), a, g, create_graph=True)
        (second,) = torch.autograd.grad(first, a, h)
        return first, second

    (first, second), names = op_names(second_order)
    ref_a = a.detach().double().requires_grad_()
    (ref_first,) = torch.autograd.grad(reference(ref_a), ref_a, g.double(), create_graph=True)
    (ref_second,) = torch.autograd.grad(ref_first, ref_a, h.double())
    check_error(first, ref_first, backward=True)
    check_error(second, ref_second, backward=True)
    if 2 * n <= 32:
        assert "flash_hypercons::_frechet" in names
        assert "aten::linalg_matrix_exp" not in names
    else:
        assert "aten::linalg_matrix_exp" in names


@pytest.mark.parametrize("dtype", DTYPES)
def test_function_transforms_use_native(dtype):
    a = (torch.randn(2, 4, 4, device="cuda") * 0.03).to(dtype)
    g = torch.randn_like(a) * 0.1
    with fh.use_backend():
        y, tangent = torch.func.jvp(torch.linalg.matrix_exp, (a,), (g,))
        grad = torch.func.grad(lambda x: torch.linalg.matrix_exp(x).sum())(a)
    check_error(y, reference(a))
    check_error(tangent, reference(a, g), backward=True)
    check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
    batched = a.unsqueeze(0).expand(3, *a.shape)
    check_error(torch.vmap(fh.matrix_exp)(batched), reference(batched))


@pytest.mark.parametrize("tangent_arg", ["input", "grad", "both"])
@pytest.mark.parametrize("n", [4, 16, 32])
def test_forward_over_reverse_at_zero(n, tangent_arg):
    a = torch.zeros(1, n, n, device="cuda", requires_grad=True)
    identity = torch.eye(n, device="cuda").unsqueeze(0)
    with torch.autograd.forward_ad.dual_level():
        x = torch.autograd.forward_ad.make_dual(a, identity) if tangent_arg in ("input", "both") else a
        g = torch.autograd.forward_ad.make_dual(identity, identity) if tangent_arg in ("grad", "both") else identity
        (gradient,) = torch.autograd.grad(fh.matrix_exp(x), x, g)
        primal, tangent = torch.autograd.forward_ad.unpack_dual(gradient)
        assert tangent is not None
        torch.testing.assert_close(primal, identity)
        torch.testing.assert_close(tangent, (2 if tangent_arg == "both" else 1) * identity)


@pytest.mark.parametrize("dtype", DTYPES)
def test_nested_transforms_on_diagonal_matrices(dtype):
    n = 4
    diagonal = torch.linspace(-0.2, 0.2, n, device="cuda", dtype=dtype)
    a = diagonal.diag().expand(3, n, n)
    identity = torch.eye(n, device="cuda", dtype=dtype).expand_as(a)
    expected = diagonal.double().exp().diag().expand_as(a)
    gradient = torch.func.grad(lambda x: fh.matrix_exp(x).diagonal(dim1=-2, dim2=-1).sum())
    for fn in (gradient, torch.vmap(gradient)):
        primal, tangent = torch.func.jvp(fn, (a,), (identity,))
        check_error(primal, expected, backward=True)
        check_error(tangent, expected, backward=True)


@pytest.mark.compile
@pytest.mark.parametrize("transform", ["grad", "jvp", "vmap"])
def test_compiled_transforms_stay_native(transform):
    a = torch.zeros(2, 4, 4, device="cuda")
    identity = torch.eye(4, device="cuda").expand_as(a)
    if transform == "grad":
        fn = torch.func.grad(lambda x: fh.matrix_exp(x).diagonal(dim1=-2, dim2=-1).sum())
    elif transform == "jvp":

        def fn(x):
            return torch.func.jvp(fh.matrix_exp, (x,), (identity,))[1]

    else:
        fn = torch.vmap(fh.matrix_exp)
    graphs = []

    def capture(gm, inputs):
        graphs.append(gm)
        return gm.forward

    actual = torch.compile(fn, backend=capture, fullgraph=True)(a)
    torch.testing.assert_close(actual, identity)
    assert not any("flash_hypercons" in str(node.target) for gm in graphs for node in gm.graph.nodes)


@pytest.mark.compile
@pytest.mark.parametrize("scoped", [False, True])
def test_compile_captures_custom_op(scoped):
    graphs = []

    def capture(gm, inputs):
        graphs.append(gm)
        return gm.forward

    fn = torch.linalg.matrix_exp if scoped else fh.matrix_exp
    a = (torch.randn(3, 9, 9, device="cuda") * 0.03).requires_grad_()
    captured = torch.compile(fn, backend=capture, fullgraph=True)
    compiled = torch.compile(fn, fullgraph=True)
    with fh.use_backend():
        captured(a)
        y = compiled(a)
    assert any(
        node.target in (torch.ops.flash_hypercons._matrix_exp.default, torch.ops.flash_hypercons._matrix_exp)
        for gm in graphs
        for node in gm.graph.nodes
    )
    grad, names = op_names(lambda: torch.autograd.grad(y.sum(), a)[0])
    assert "flash_hypercons::_frechet" in names
    check_error(y, reference(a))
    check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
    if scoped:
        _, names = op_names(lambda: captured(a))
        assert "flash_hypercons::_matrix_exp" not in names


def test_autocast_and_parameter():
    a = torch.nn.Parameter(torch.randn(2, 8, 8, device="cuda") * 0.03)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = fh.matrix_exp(a)
    assert y.dtype == a.dtype
    check_error(y, reference(a))
    (grad,) = torch.autograd.grad(y.sum(), a)
    check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
