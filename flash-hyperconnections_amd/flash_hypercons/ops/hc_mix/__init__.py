"""Hyper-connection stream mixing with the matrix exponential fused in.

``mix_streams(h, x)`` returns ``matrix_exp(h) @ x`` for ``h`` of shape
``[B, n, n]`` (the per-token mixing generator) and ``x`` of shape ``[B, n, C]``
(the n residual streams of each token).  The reference stops at
``matrix_exp(h)`` (ops/matrix_exp/__init__.py:80-97) and leaves the product to
the caller; on a gfx950 device with float32 / float16 / bfloat16 operands of
one dtype this build streams x once per direction:

* 2 <= n <= 4: the product is computed in the same kernel that computes
  exp(h), so exp(h) never goes through memory, and the backward is one kernel
  as well (dX = exp(h)^T dY, dE = dY X^T reduced on chip, dH = L(h^T, dE));
* 5 <= n <= 8: exp(h) is computed in FP32 by ``matrix_exp`` (a few bytes per
  token next to x's n*C elements) and applied by a streaming kernel; the
  backward is one streaming kernel for dX and dE followed by the Frechet
  kernel for dH.

Everything else -- other n, CPU tensors, function transforms, forward-mode
tangents, a backward that builds a graph -- is the composition
``matrix_exp(h) @ x`` with this package's ``matrix_exp``.
"""

import torch

from flash_hypercons import _C  # noqa: F401  (registers the flash_hypercons::* operators)
from flash_hypercons.ops.matrix_exp import _device_supported, _frechet_differentiable, matrix_exp

_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _streamed(h: torch.Tensor, x: torch.Tensor) -> bool:
    """Operands the streaming kernels take (any n; the callers pick the n range)."""
    return (
        isinstance(h, torch.Tensor)
        and isinstance(x, torch.Tensor)
        and type(h) in (torch.Tensor, torch.nn.Parameter)
        and type(x) in (torch.Tensor, torch.nn.Parameter)
        and not torch._C._are_functorch_transforms_active()
        and h.device.type == "cuda"
        and torch.version.hip is not None
        and x.device == h.device
        and h.layout == torch.strided
        and x.layout == torch.strided
        and h.ndim == 3
        and x.ndim == 3
        and h.shape[-1] == h.shape[-2]
        and x.shape[0] == h.shape[0]
        and x.shape[1] == h.shape[1]
        and x.shape[2] >= 1
        and h.dtype in _DTYPES
        and x.dtype == h.dtype
        and torch.autograd.forward_ad.unpack_dual(h).tangent is None
        and torch.autograd.forward_ad.unpack_dual(x).tangent is None
        and _token_span(x) < 2**31
        and _device_supported(h.device.index)
    )


def _token_span(x: torch.Tensor) -> int:
    """Bytes of one token's n contiguous rows, C rounded up to whole 16-byte vectors: the span the
    streaming kernels address with 32-bit offsets (inputs read in place span no more, or are copied
    to this layout first)."""
    es = x.element_size()
    v = 16 // es
    return x.shape[1] * (-(-x.shape[2] // v) * v) * es


@torch.library.register_fake("flash_hypercons::_hc_mix")
def _hc_mix_fake(h, x):
    torch._check(h.ndim == 3 and x.ndim == 3)
    torch._check(x.shape[0] == h.shape[0] and x.shape[1] == h.shape[1])
    return x.new_empty(x.shape)


@torch.library.register_fake("flash_hypercons::_hc_mix_backward")
def _hc_mix_backward_fake(h, x, grad):
    torch._check(grad.shape == x.shape)
    return h.new_empty(h.shape), x.new_empty(x.shape)


@torch.library.register_fake("flash_hypercons::_hc_mix_aux")
def _hc_mix_aux_fake(h, x, grad):
    second = h.new_empty(h.shape) if grad is not None else h.new_empty((0,))
    return x.new_empty(x.shape), second, h.new_empty(h.shape, dtype=torch.float32)


def _fused(h: torch.Tensor, x: torch.Tensor) -> bool:
    return _streamed(h, x) and 2 <= h.shape[-1] <= 4


def _applied(h: torch.Tensor, x: torch.Tensor) -> bool:
    return _streamed(h, x) and 5 <= h.shape[-1] <= 8


@torch.library.register_fake("flash_hypercons::_hc_apply")
def _hc_apply_fake(e, x):
    torch._check(e.ndim == 3 and x.ndim == 3)
    torch._check(x.shape[0] == e.shape[0] and x.shape[1] == e.shape[1])
    return x.new_empty(x.shape)


@torch.library.register_fake("flash_hypercons::_hc_apply_backward")
def _hc_apply_backward_fake(e, x, grad):
    torch._check(grad.shape == x.shape)
    return x.new_empty(x.shape), e.new_empty(e.shape)


class _MixStreams(torch.autograd.Function):
    @staticmethod
    def forward(h, x):
        return torch.ops.flash_hypercons._hc_mix(h, x)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    @staticmethod
    def backward(ctx, grad):
        h, x = ctx.saved_tensors
        if torch.is_grad_enabled():
            # A backward that builds a graph: the same gradients from differentiable pieces.
            return _frechet_differentiable(h.mT, grad @ x.mT), matrix_exp(h).mT @ grad
        dh, dx = torch.ops.flash_hypercons._hc_mix_backward(h, x, grad.contiguous())
        return dh, dx


class _MixStreamsApplied(torch.autograd.Function):
    """5 <= n <= 8: E = exp(h) in FP32 (the P = 8 kernel), then y = E x streamed;
    backward: (dX, dE) in one streaming pass, dH = L(h^T, dE) in FP32, rounded to h's dtype."""

    @staticmethod
    def forward(ctx, h, x):
        hf = h.float()
        e = torch.ops.flash_hypercons._matrix_exp(hf)
        ctx.save_for_backward(h, x, e, hf)
        return torch.ops.flash_hypercons._hc_apply(e, x)

    @staticmethod
    def backward(ctx, grad):
        h, x, e, hf = ctx.saved_tensors
        if torch.is_grad_enabled():
            return _frechet_differentiable(h.mT, grad @ x.mT), matrix_exp(h).mT @ grad
        dx, de = torch.ops.flash_hypercons._hc_apply_backward(e, x, grad.contiguous())
        dh = torch.ops.flash_hypercons._frechet(hf.mT, de).to(h.dtype) if ctx.needs_input_grad[0] else None
        return dh, dx


def mix_streams(h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """exp(h) @ x per token: h [B, n, n], x [B, n, C] -> [B, n, C] (hyper-connection stream mixing).

    Differentiable in both arguments.  On gfx950: fused into one HIP kernel per
    direction for 2 <= n <= 4; for 5 <= n <= 8, exp(h) from ``matrix_exp`` in FP32
    and one streaming kernel per direction.  Otherwise composed from
    ``matrix_exp`` and a batched product.
    """
    if _fused(h, x):
        return _MixStreams.apply(h, x)
    if _applied(h, x):
        return _MixStreamsApplied.apply(h, x)
    return matrix_exp(h) @ x


__all__ = ["mix_streams"]
