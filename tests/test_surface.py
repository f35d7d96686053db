"""Routing surface of flash_hypercons: which implementation runs for which input and entry point.

The reference's contract (ops/matrix_exp/__init__.py:13-29, :80-118): eligible
inputs -- strided [B, N, N] device tensors, 2 <= N <= 32, float32 / float16 /
bfloat16 (here: on a ROCm gfx950 device) -- run the flash_hypercons operators;
everything else, CPU tensors included, falls through to native
``linalg_matrix_exp`` with native results and native errors.  ``use_backend()``
reroutes ``torch.linalg.matrix_exp``, ``torch.matrix_exp`` and
``Tensor.matrix_exp`` inside a thread-local, nestable scope and nothing else.

How the route is observed here:
* forward -- ``OpLog``, a TorchDispatchMode that records every operator that
  reaches the dispatcher below autograd;
* backward -- by the bits: the Frechet kernel's result for random inputs is
  bit-identical to ``flash_hypercons::_frechet`` on the same operands and (with
  overwhelming probability) differs from the native block exponential's;
* profiler names -- one test checks that both operators appear under their
  schema names, as profiler-based callers expect.

The table-driven cases run every input class through every entry point.
"""

from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import pytest
import torch
from torch.overrides import _get_current_function_mode
from torch.utils._python_dispatch import TorchDispatchMode

import flash_hypercons as fh
from tests.reference import check_north_star, reference

GPU = torch.cuda.is_available() and torch.version.hip is not None
KERNEL_FWD = "flash_hypercons._matrix_exp"
NATIVE_FWD = "aten.linalg_matrix_exp"


class OpLog(TorchDispatchMode):
    """Records the operators dispatched while active (below autograd)."""

    def __init__(self):
        super().__init__()
        self.ops = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops.append(str(func))
        return func(*args, **(kwargs or {}))

    def saw(self, prefix: str) -> bool:
        return any(op.startswith(prefix) for op in self.ops)


def traced(fn):
    log = OpLog()
    with log:
        out = fn()
    return out, log


# Every way a caller reaches the exponential.  Scoped entry points only route inside use_backend().
ENTRY_POINTS = {
    "fh.matrix_exp": (lambda x: fh.matrix_exp(x), False),
    "torch.linalg.matrix_exp": (lambda x: torch.linalg.matrix_exp(x), True),
    "torch.linalg.matrix_exp(input=)": (lambda x: torch.linalg.matrix_exp(input=x), True),
    "torch.matrix_exp": (lambda x: torch.matrix_exp(x), True),
    "Tensor.matrix_exp": (lambda x: x.matrix_exp(), True),
}

# (label, shape, dtype, routed to the kernel when on the GPU)
INPUTS = [
    ("batched n=4 f32", (3, 4, 4), torch.float32, True),
    ("batched n=9 bf16", (3, 9, 9), torch.bfloat16, True),
    ("batched n=32 f16", (2, 32, 32), torch.float16, True),
    ("batched n=2 f32", (5, 2, 2), torch.float32, True),
    ("empty batch n=4", (0, 4, 4), torch.float32, True),
    ("single matrix (ndim 2)", (4, 4), torch.float32, False),
    ("extra batch dim (ndim 4)", (1, 2, 4, 4), torch.float32, False),
    ("n=33 beyond range", (2, 33, 33), torch.float32, False),
    ("n=1", (2, 1, 1), torch.float32, False),
    ("empty matrices", (2, 0, 0), torch.float32, False),
    ("float64", (2, 4, 4), torch.float64, False),
    ("complex64", (2, 4, 4), torch.complex64, False),
]


def _make(shape, dtype, device, scale=0.1):
    return (torch.randn(shape, device=device, dtype=torch.float64) * scale).to(dtype)


def _assert_native_result(actual, x):
    expected = torch.linalg.matrix_exp(x)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)


@pytest.mark.parametrize("entry", list(ENTRY_POINTS))
@pytest.mark.parametrize("label,shape,dtype,_", INPUTS, ids=[row[0] for row in INPUTS])
def test_cpu_inputs_fall_through_to_native(label, shape, dtype, _, entry):
    """On the CPU every input class, through every entry point, inside nested scopes, is native:
    same bits as torch, no flash_hypercons operator dispatched, the torch functions untouched."""
    fn, _scoped = ENTRY_POINTS[entry]
    x = _make(shape, dtype, "cpu")
    before = (torch.linalg.matrix_exp, torch.matrix_exp, torch.Tensor.matrix_exp)
    with fh.use_backend(), fh.use_backend():
        y, log = traced(lambda: fn(x))
    assert not log.saw("flash_hypercons")
    _assert_native_result(y, x)
    assert (torch.linalg.matrix_exp, torch.matrix_exp, torch.Tensor.matrix_exp) == before


def test_config1_cpu_plumbing_against_fixture():
    """BASELINE config 1 on the CPU: fh.matrix_exp + backward of y.sum() falls through to native
    torch; outputs and gradients match the committed FP64 fixture (relative Frobenius <= 1e-5 /
    1e-4) and no flash_hypercons operator runs."""
    d = np.load(Path(__file__).resolve().parent / "golden" / "c1_cpu_plumbing.npz")
    x = torch.from_numpy(d["x"]).requires_grad_()
    y, log = traced(lambda: fh.matrix_exp(x))
    (grad,) = torch.autograd.grad(y.sum(), x)
    assert not log.saw("flash_hypercons") and log.saw(NATIVE_FWD)
    check_north_star(y.detach(), torch.from_numpy(d["y"]))
    check_north_star(grad, torch.from_numpy(d["grad"]), backward=True)
    torch.manual_seed(0)
    assert torch.equal(x.detach(), torch.randn(128, 4, 4))  # the fixture holds config 1's seeded inputs


@pytest.mark.parametrize(
    "make",
    [lambda: torch.ones(2, 3), lambda: torch.ones(2, 2, dtype=torch.int64), lambda: torch.ones(2),
     lambda: torch.ones(3, 2, 5)],
    ids=["non-square", "int64", "vector", "batched non-square"],
)
def test_invalid_inputs_raise_the_native_error(make):
    value = make()
    try:
        torch.linalg.matrix_exp(value)
    except (RuntimeError, TypeError) as exc:
        native = type(exc)
    else:
        pytest.fail("native torch accepted an invalid input")
    for entry in ("torch.linalg.matrix_exp", "torch.matrix_exp", "Tensor.matrix_exp"):
        with fh.use_backend(), pytest.raises(native):
            ENTRY_POINTS[entry][0](value)


def test_unsupported_keyword_is_a_type_error_inside_the_scope():
    with fh.use_backend(), pytest.raises(TypeError):
        torch.linalg.matrix_exp(torch.eye(2), out=torch.empty(2, 2))


def test_scope_restores_on_exit_and_on_exception():
    assert _get_current_function_mode() is None
    with fh.use_backend() as outer:
        assert _get_current_function_mode() is outer
        with pytest.raises(KeyError), fh.use_backend():
            raise KeyError("inner scope fails")
        assert _get_current_function_mode() is outer
    assert _get_current_function_mode() is None


def test_scope_does_not_leak_into_other_threads():
    with fh.use_backend(), ThreadPoolExecutor(max_workers=2) as pool:
        assert pool.submit(_get_current_function_mode).result() is None
        assert _get_current_function_mode() is not None


def test_cpu_gradient_through_scope_is_native():
    a = _make((3, 4, 4), torch.float64, "cpu").requires_grad_()
    g = torch.randn(3, 4, 4, dtype=torch.float64)
    with fh.use_backend():
        y = torch.matrix_exp(a)
    (grad,) = torch.autograd.grad(y, a, g)
    ref = a.detach().clone().requires_grad_()
    (expected,) = torch.autograd.grad(torch.linalg.matrix_exp(ref), ref, g)
    assert torch.equal(grad, expected)


# ---- GPU ------------------------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("entry", list(ENTRY_POINTS))
@pytest.mark.parametrize("label,shape,dtype,routed", INPUTS, ids=[row[0] for row in INPUTS])
def test_gpu_routing_table(label, shape, dtype, routed, entry):
    """Each input class through each entry point: eligible inputs reach the kernel (the scoped
    entry points only inside use_backend()); the rest produce native results bit for bit."""
    fn, scoped = ENTRY_POINTS[entry]
    x = _make(shape, dtype, "cuda")
    _, outside = traced(lambda: fn(x))
    with fh.use_backend():
        y, inside = traced(lambda: fn(x))
    expect_kernel = routed
    assert inside.saw(KERNEL_FWD) == expect_kernel
    assert outside.saw(KERNEL_FWD) == (routed and not scoped)
    if expect_kernel:
        assert torch.equal(y, torch.ops.flash_hypercons._matrix_exp(x))
        if y.numel():
            check_north_star(y, reference(x))
    else:
        _assert_native_result(y, x)


@pytest.mark.gpu
@pytest.mark.parametrize("n,dtype", [(4, torch.float32), (9, torch.float32), (16, torch.bfloat16),
                                     (32, torch.float16)])
def test_gpu_backward_runs_the_frechet_kernel(n, dtype):
    """The gradient of a routed call is L(A^T, G) from the Frechet kernel: bit-identical to the
    operator on the same operands, and not the native block exponential's bits."""
    a = _make((6, n, n), dtype, "cuda", scale=0.4).requires_grad_()
    g = torch.randn(6, n, n, device="cuda").to(dtype)
    for entry, (fn, scoped) in ENTRY_POINTS.items():
        with fh.use_backend():
            y = fn(a)
        (grad,) = torch.autograd.grad(y, a, g)
        assert torch.equal(grad, torch.ops.flash_hypercons._frechet(a.detach().mT, g)), entry
        check_north_star(grad, reference(a.detach().mT, g), backward=True)
    if dtype == torch.float32:
        # The native block exponential's FP32 bits differ (low-precision outputs may round alike).
        native = torch.autograd.grad(torch.ops.aten.linalg_matrix_exp.default(a), a, g)[0]
        assert not torch.equal(native, grad)


@pytest.mark.gpu
def test_profiler_shows_operator_schema_names():
    from torch.profiler import ProfilerActivity, profile

    a = _make((3, 9, 9), torch.float32, "cuda").requires_grad_()
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        y = fh.matrix_exp(a)
        torch.autograd.grad(y.sum(), a)
    names = {event.key for event in prof.key_averages()}
    assert {"flash_hypercons::_matrix_exp", "flash_hypercons::_frechet"} <= names


@pytest.mark.gpu
def test_direct_aten_calls_are_not_rerouted():
    a = _make((3, 9, 9), torch.float32, "cuda")
    with fh.use_backend():
        y, log = traced(lambda: torch.ops.aten.linalg_matrix_exp.default(a))
    assert not log.saw(KERNEL_FWD)
    _assert_native_result(y, a)


@pytest.mark.gpu
def test_tensor_subclasses_keep_their_type_and_go_native():
    class Tagged(torch.Tensor):
        pass

    a = _make((2, 4, 4), torch.float32, "cuda", scale=0.05).as_subclass(Tagged)
    y, log = traced(lambda: fh.matrix_exp(a))
    assert isinstance(y, Tagged)
    assert not log.saw(KERNEL_FWD)
    torch.testing.assert_close(y.as_subclass(torch.Tensor), torch.linalg.matrix_exp(a.as_subclass(torch.Tensor)))


@pytest.mark.gpu
def test_parameters_are_routed_like_tensors():
    p = torch.nn.Parameter(_make((2, 8, 8), torch.float32, "cuda", scale=0.05))
    y, log = traced(lambda: fh.matrix_exp(p))
    assert log.saw(KERNEL_FWD)
    check_north_star(y.detach(), reference(p.detach()))
