"""Routing surface: use_backend() scopes, aliases, native fallback.

Cases follow the reference suite (tests/test_routing.py there).  The CPU cases
run everywhere; the GPU cases prove dispatch through profiler event names.
"""

from concurrent.futures import ThreadPoolExecutor

import pytest
import torch
from torch.profiler import ProfilerActivity, profile

import flash_hypercons as fh
from tests.reference import check_error, reference

ALIAS = torch.linalg.matrix_exp


def op_names(fn):
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        result = fn()
    return result, {event.key for event in prof.key_averages()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64])
@pytest.mark.parametrize("shape", [(2, 4, 4), (4, 4), (1, 2, 4, 4), (2, 33, 33), (2, 0, 0), (2, 1, 1), (0, 3, 3)])
def test_cpu_tensors_use_native(shape, dtype):
    a = torch.randn(shape, dtype=dtype) * 0.1
    expected = torch.linalg.matrix_exp(a)
    with fh.use_backend(), fh.use_backend():
        actual, names = op_names(lambda: fh.matrix_exp(a))
        torch.testing.assert_close(actual, expected)
        torch.testing.assert_close(ALIAS(input=a), expected)
        torch.testing.assert_close(a.matrix_exp(), expected)
        torch.testing.assert_close(torch.matrix_exp(a), expected)
    assert not any(name.startswith("flash_hypercons::") for name in names)
    assert torch.linalg.matrix_exp is ALIAS


@pytest.mark.parametrize("value", [torch.ones(2, 3), torch.ones(2, 2, dtype=torch.int64), torch.ones(2)])
def test_native_errors_preserved(value):
    with pytest.raises((RuntimeError, TypeError)) as native:
        torch.linalg.matrix_exp(value)
    with fh.use_backend(), pytest.raises(type(native.value)):
        torch.linalg.matrix_exp(value)


def test_unsupported_signature_raises():
    with fh.use_backend(), pytest.raises(TypeError):
        torch.linalg.matrix_exp(torch.eye(2), out=torch.empty(2, 2))


def test_cpu_backward_and_scope_restoration():
    a = (torch.randn(3, 4, 4, dtype=torch.float64) * 0.1).requires_grad_()
    with fh.use_backend():
        y = torch.linalg.matrix_exp(a)
    (grad,) = torch.autograd.grad(y.sum(), a)
    torch.testing.assert_close(grad, reference(a.mT, torch.ones_like(a)))
    with pytest.raises(ValueError, match="inside"), fh.use_backend():
        raise ValueError("inside")
    from torch.overrides import _get_current_function_mode

    assert _get_current_function_mode() is None


def test_scope_is_thread_local():
    from torch.overrides import _get_current_function_mode

    with fh.use_backend(), ThreadPoolExecutor(max_workers=1) as pool:
        assert pool.submit(_get_current_function_mode).result() is None


@pytest.mark.gpu
def test_scopes_aliases_and_backward_on_gpu():
    a = (torch.randn(3, 9, 9, device="cuda") * 0.03).requires_grad_()
    original = (torch.linalg.matrix_exp, torch.matrix_exp, torch.Tensor.matrix_exp)
    for call in (
        lambda: torch.linalg.matrix_exp(a),
        lambda: ALIAS(input=a),
        lambda: torch.matrix_exp(a),
        lambda: a.matrix_exp(),
    ):
        with fh.use_backend(), fh.use_backend():
            y, names = op_names(call)
        assert "flash_hypercons::_matrix_exp" in names
        grad, names = op_names(lambda y=y: torch.autograd.grad(y.sum(), a)[0])
        assert "flash_hypercons::_frechet" in names
        check_error(y, reference(a))
        check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
    with pytest.raises(ValueError, match="scope"), fh.use_backend():
        raise ValueError("scope")
    _, names = op_names(lambda: torch.linalg.matrix_exp(a))
    assert "flash_hypercons::_matrix_exp" not in names
    assert original == (torch.linalg.matrix_exp, torch.matrix_exp, torch.Tensor.matrix_exp)
    with fh.use_backend():
        _, names = op_names(lambda: torch.ops.aten.linalg_matrix_exp.default(a))
    assert "flash_hypercons::_matrix_exp" not in names


@pytest.mark.gpu
@pytest.mark.parametrize(
    "shape,dtype",
    [((4, 4), torch.float32), ((1, 2, 4, 4), torch.float32), ((2, 33, 33), torch.float32),
     ((2, 4, 4), torch.float64), ((2, 4, 4), torch.complex64), ((2, 1, 1), torch.float32)],
)
def test_gpu_ineligible_inputs_use_native(shape, dtype):
    a = torch.randn(shape, device="cuda", dtype=dtype) * 0.1
    expected = torch.linalg.matrix_exp(a)
    with fh.use_backend():
        actual, names = op_names(lambda: torch.linalg.matrix_exp(a))
    torch.testing.assert_close(actual, expected)
    assert "flash_hypercons::_matrix_exp" not in names


@pytest.mark.gpu
def test_tensor_subclass_uses_native():
    class SubTensor(torch.Tensor):
        pass

    a = (torch.randn(2, 4, 4, device="cuda") * 0.03).as_subclass(SubTensor)
    y, names = op_names(lambda: fh.matrix_exp(a))
    assert isinstance(y, SubTensor)
    assert "flash_hypercons::_matrix_exp" not in names
    torch.testing.assert_close(y, torch.linalg.matrix_exp(a))
