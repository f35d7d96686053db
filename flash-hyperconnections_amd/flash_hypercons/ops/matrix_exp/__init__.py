"""Adaptive small-matrix exponentials and scoped PyTorch routing (MI355X / gfx950).

Python surface of the reference's ``flash_hypercons/ops/matrix_exp/__init__.py``
(same names, routing rules and error behaviour).  Eligible tensors -- strided
``[B, N, N]`` ROCm tensors on a gfx950 device with 2 <= N <= 32 in float32,
float16 or bfloat16 -- go to the ``flash_hypercons::_matrix_exp`` operator,
whose backward is ``flash_hypercons::_frechet``; both run the HIP kernels of
``libflash_hypercons_hip.so``.  Everything else uses native PyTorch, as in the
reference.  Importing this module fails if the compiled extension is missing:
there is no Python or CPU stand-in for the kernels.
"""

import functools

import torch
from torch.overrides import TorchFunctionMode, has_torch_function

from flash_hypercons import _C  # noqa: F401  (registers the flash_hypercons::* operators)

_NATIVE = torch.ops.aten.linalg_matrix_exp.default
_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_FUNCTIONS = (torch.linalg.matrix_exp, torch.matrix_exp, torch.Tensor.matrix_exp)
_ARCH = "gfx950"  # the only code object the extension carries


@functools.lru_cache(maxsize=None)
def _device_supported(index: int) -> bool:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0] == _ARCH


def _eligible(input: torch.Tensor) -> bool:
    """Reference ops/matrix_exp/__init__.py:13-23, with the platform test flipped to ROCm/gfx950."""
    return (
        isinstance(input, torch.Tensor)
        and input.device.type == "cuda"
        and torch.version.hip is not None
        and input.layout == torch.strided
        and input.ndim == 3
        and input.shape[-1] == input.shape[-2]
        and 1 < input.shape[-1] <= 32
        and input.dtype in _DTYPES
        and _device_supported(input.device.index)
    )


def _native(input: torch.Tensor, *, promote: bool = False) -> torch.Tensor:
    """Reference :26-29: native exponential, FP32-promoted for GPU low precision when asked."""
    if promote and input.is_cuda and input.dtype in (torch.float16, torch.bfloat16):
        return _NATIVE(input.float()).to(input.dtype)
    return _NATIVE(input)


def _frechet_reference(input: torch.Tensor, direction: torch.Tensor) -> torch.Tensor:
    """Reference :32-37: differentiable Frechet derivative via the 2N x 2N block exponential."""
    n = input.shape[-1]
    a, g = input.float(), direction.float()
    zero = torch.zeros_like(a)
    block = torch.cat((torch.cat((a, g), -1), torch.cat((zero, a), -1)), -2)
    return _NATIVE(block)[..., :n, n:].to(input.dtype)


@torch.library.register_fake("flash_hypercons::_matrix_exp")
def _matrix_exp_fake(input):
    """Reference :40-49."""
    torch._check(input.device.type == "cuda")
    torch._check(input.layout == torch.strided)
    torch._check(input.ndim == 3)
    torch._check(input.dtype in _DTYPES)
    torch._check(input.shape[-1] == input.shape[-2])
    torch._check(input.shape[-1] > 1)
    torch._check(input.shape[-1] <= 32)
    return input.new_empty(input.shape)


@torch.library.register_fake("flash_hypercons::_frechet")
def _frechet_fake(input, direction):
    """Reference :52-58."""
    torch._check(direction.shape == input.shape)
    torch._check(direction.device == input.device)
    torch._check(direction.dtype == input.dtype)
    torch._check(direction.layout == torch.strided)
    return _matrix_exp_fake(input)


@torch.library.register_fake("flash_hypercons::_expm_params")
def _expm_params_fake(input, direction=None):
    _matrix_exp_fake(input)
    return input.new_empty((input.shape[0], 2), dtype=torch.int32), input.new_empty((input.shape[0],), dtype=torch.float64)


@torch.library.register_fake("flash_hypercons::_expm_debug")
def _expm_debug_fake(input, direction, variant):
    return _matrix_exp_fake(input), input.new_empty((input.shape[0],), dtype=torch.int32)


def _frechet_differentiable(input: torch.Tensor, direction: torch.Tensor) -> torch.Tensor:
    """Differentiable L(input, direction) for a backward that builds a graph.

    The same 2N x 2N block exponential as ``_frechet_reference``, but taken with
    this build's own operator whenever the block is itself eligible (2N <= 32):
    its gradient is then again the HIP Frechet kernel, so second derivatives
    stay on the device.  Larger blocks use the reference's native path.
    """
    n = input.shape[-1]
    if 2 * n > 32 or not _eligible(input):
        return _frechet_reference(input, direction)
    a, g = input.float(), direction.float()
    zero = torch.zeros_like(a)
    block = torch.cat((torch.cat((a, g), -1), torch.cat((zero, a), -1)), -2)
    return torch.ops.flash_hypercons._matrix_exp(block)[..., :n, n:].to(input.dtype)


def _backward(ctx, grad_output):
    """Reference :65-74: the gradient of exp at A against G is L(A^T, G).

    Tensor subclasses, modes and forward-mode tangents take the reference's
    native block exponential as in the reference; a backward that builds a
    graph (``create_graph=True``) takes the block exponential through this
    operator (``_frechet_differentiable``) instead of the native one.  The
    operator's own autograd kernel is the C++ restatement of this function
    (``csrc/register.cpp``, ``exp_gradient``); this one serves
    ``_DualMatrixExp``.
    """
    (input,) = ctx.saved_tensors
    if (
        has_torch_function((input, grad_output))
        or torch.autograd.forward_ad.unpack_dual(input).tangent is not None
        or torch.autograd.forward_ad.unpack_dual(grad_output).tangent is not None
    ):
        return _frechet_reference(input.mT, grad_output)
    if torch.is_grad_enabled():
        return _frechet_differentiable(input.mT, grad_output)
    return torch.ops.flash_hypercons._frechet(input.mT, grad_output)




def _torch_function_backward(input: torch.Tensor, grad_output: torch.Tensor):
    """Reference :67-73, the backward's first branch, for the C++ autograd kernel of
    ``_matrix_exp``: with a ``__torch_function__`` mode active or an argument whose type
    overrides ``__torch_function__``, the gradient is the native block exponential computed
    here (so subclasses see and wrap every call); otherwise None, and the kernel goes on."""
    if has_torch_function((input, grad_output)):
        return _frechet_reference(input.mT, grad_output)
    return None


def _tangent(input: torch.Tensor, tangent: torch.Tensor) -> torch.Tensor:
    """L(input, tangent), the forward-mode derivative of exp at input along tangent.

    The Frechet kernel without the backward's transpose.  A computation that
    builds a graph takes the differentiable block exponential
    (``_frechet_differentiable``); a tangent the operator cannot take (another
    dtype, device or layout) takes the reference's native block exponential.
    """
    if (
        not isinstance(tangent, torch.Tensor)
        or type(tangent) is not torch.Tensor
        or tangent.layout != torch.strided
        or tangent.shape != input.shape
        or tangent.dtype != input.dtype
        or tangent.device != input.device
        or torch.autograd.forward_ad.unpack_dual(tangent).tangent is not None
    ):
        return _frechet_reference(input, tangent)
    if torch.is_grad_enabled() and (input.requires_grad or tangent.requires_grad):
        return _frechet_differentiable(input, tangent)
    return torch.ops.flash_hypercons._frechet(input, tangent)


class _DualMatrixExp(torch.autograd.Function):
    """exp(A) for an input that carries a forward-mode tangent H.

    The reference sends such inputs to the native exponential
    (ops/matrix_exp/__init__.py:89-94); here the primal runs the forward kernel
    and the tangent is L(A, H) from the Frechet kernel.  Reverse mode is the
    operator's own backward (``_backward``), which sees the saved input with its
    tangent, so forward-over-reverse keeps working through the native block
    exponential as in the reference.
    """

    @staticmethod
    def forward(input):
        return torch.ops.flash_hypercons._matrix_exp(input)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(inputs[0])
        ctx.save_for_forward(inputs[0])

    @staticmethod
    def backward(ctx, grad_output):
        return _backward(ctx, grad_output)

    @staticmethod
    def jvp(ctx, tangent):
        (input,) = ctx.saved_tensors
        return _tangent(input, tangent)


def matrix_exp(input: torch.Tensor) -> torch.Tensor:
    """exp(input) for batched square matrices; [B, N, N] (2 <= N <= 32) float32 / float16 /
    bfloat16 tensors on a gfx950 device run the HIP kernels, anything else native PyTorch.

    Differentiable: the gradient is the structured Frechet derivative L(A^T, G) from the Frechet
    kernel; a forward-mode tangent H on an eligible input is carried as L(A, H) from the same
    kernel.  Inputs under functorch transforms, tensor subclasses, and dual inputs that are not
    eligible take the native exponential; on the GPU their float16 / bfloat16 values are
    evaluated in float32 and cast back.
    """
    # Check transforms before shape eligibility: vmap can hide batch dimensions.
    if isinstance(input, torch.Tensor) and (
        type(input) not in (torch.Tensor, torch.nn.Parameter) or torch._C._are_functorch_transforms_active()
    ):
        return _native(input, promote=True)
    dual = isinstance(input, torch.Tensor) and torch.autograd.forward_ad.unpack_dual(input).tangent is not None
    if not _eligible(input):
        return _native(input, promote=dual)
    if dual:
        return _DualMatrixExp.apply(input)
    return torch.ops.flash_hypercons._matrix_exp(input)


class _MatrixExpMode(TorchFunctionMode):
    """Reference :100-108: reroutes the three matrix-exp entry points, nothing else."""

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func in _FUNCTIONS:
            if len(args) == 1 and not kwargs:
                return matrix_exp(args[0])
            if not args and set(kwargs) == {"input"}:
                return matrix_exp(kwargs["input"])
        return func(*args, **kwargs)


def use_backend() -> TorchFunctionMode:
    """Context manager: inside it, torch.linalg.matrix_exp, torch.matrix_exp and
    Tensor.matrix_exp called from Python go through ``matrix_exp`` above.

    The mode is per thread and may be nested; leaving the block, normally or by an exception,
    restores the previous routing.  Calls that Dynamo traces inside the block are captured as the
    custom operator.  ATen or C++ callers of linalg_matrix_exp are not affected.
    """
    return _MatrixExpMode()


__all__ = ["matrix_exp", "use_backend"]
