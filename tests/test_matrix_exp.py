"""Behavioural and numerical contract of fh.matrix_exp on the GPU.

Case list follows the reference suite (tests/test_matrix_exp.py there):
sizes 2..32 x dtypes x batch {0, 1, 35} on transposed inputs; bit-identical
results across launch-boundary batch sizes; the squaring-count boundaries and
the non-finite rule; negated / transposed / expanded views; a finite-difference
check of the VJP; large rotations with closed forms; a non-default stream.
"""

import math

import pytest
import torch

import flash_hypercons as fh
from tests.reference import check_error, check_north_star, reference

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
THETA = 3.010066362817634


def op_names(fn):
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CPU]) as prof:
        result = fn()
    return result, {event.key for event in prof.key_averages()}


@pytest.mark.parametrize("batch", [0, 1, 35])
@pytest.mark.parametrize("n", range(2, 33))
@pytest.mark.parametrize("dtype", DTYPES)
def test_sizes_dtypes_and_empty_batches(dtype, n, batch):
    base = torch.randn(batch, n, n, device="cuda") * 0.1
    a = base.to(dtype).mT.detach().requires_grad_()
    g = torch.randn_like(a) * 0.2
    y = fh.matrix_exp(a)
    (grad,) = torch.autograd.grad(y, a, g)
    assert y.dtype == dtype and grad.dtype == dtype
    assert y.device == a.device and grad.device == a.device
    assert y.shape == a.shape and grad.shape == a.shape
    check_error(y, reference(a))
    check_error(grad, reference(a.mT, g), backward=True)
    if batch:
        check_north_star(y, reference(a))
        check_north_star(grad, reference(a.mT, g), backward=True)


@pytest.mark.parametrize("n", [2, 4, 5, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_bitwise_identical_across_batch_sizes(dtype, n):
    one = (torch.randn(1, n, n, device="cuda") * 0.1).to(dtype)
    g1 = torch.randn_like(one) * 0.2
    first = None
    for batch in (1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257):
        x = one.repeat(batch, 1, 1).requires_grad_()
        y = fh.matrix_exp(x)
        (grad,) = torch.autograd.grad(y, x, g1.repeat(batch, 1, 1))
        check_error(y, reference(one).expand_as(y))
        check_error(grad, reference(one.mT, g1).expand_as(grad), backward=True)
        if first is None:
            first = (y.detach()[:1].clone(), grad[:1].clone())
        assert torch.equal(y.detach(), first[0].expand_as(y))
        assert torch.equal(grad, first[1].expand_as(grad))


@pytest.mark.parametrize("n", [2, 4, 8, 16, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_squaring_boundaries_and_nonfinite(dtype, n):
    norms = torch.tensor(
        [0, 0.1, THETA * (1 - 1e-5), THETA * (1 + 1e-5), 2 * THETA * (1 - 1e-5), 2 * THETA * (1 + 1e-5),
         12.04028, 24.08056],
        device="cuda",
    )
    m = torch.randn(len(norms), n, n, device="cuda")
    m = m - m.mT  # skew-symmetric: orthogonal exponential, no FP16 overflow
    scale = norms / torch.linalg.matrix_norm(m, ord=1)
    a = (m * scale[:, None, None]).to(dtype).requires_grad_()
    g = torch.randn_like(a) * 0.2
    y = fh.matrix_exp(a)
    (grad,) = torch.autograd.grad(y, a, g)
    check_error(y, reference(a))
    check_error(grad, reference(a.mT, g), backward=True)
    params, _ = torch.ops.flash_hypercons._expm_params(a.detach())
    import oracle

    expected_s, _ = oracle.torch_params(a.detach().cpu())
    assert torch.equal(params[:, 1].cpu(), expected_s)
    if dtype == torch.float32:
        assert params[:, 1].tolist()[:7] == [0, 0, 0, 1, 1, 2, 3]

    z = torch.zeros(4, n, n, device="cuda", dtype=dtype)
    z[0, 0, 0], z[1, 0, 0], z[2, 0, 0] = float("nan"), float("inf"), -float("inf")
    z.requires_grad_()
    y = fh.matrix_exp(z)
    (grad,) = torch.autograd.grad(y, z, torch.ones_like(z))
    assert y[:3].isnan().all() and grad[:3].isnan().all()
    torch.testing.assert_close(y[3], torch.eye(n, device="cuda", dtype=dtype))
    torch.testing.assert_close(grad[3], torch.ones_like(grad[3]))


@pytest.mark.parametrize("n", [3, 4, 8, 16, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_negated_transposed_expanded_views(dtype, n):
    for transpose in (False, True):
        base = (torch.randn(1, n, n, device="cuda") * 0.03).to(dtype)
        a = torch._neg_view(base.mT if transpose else base).expand(3, n, n).requires_grad_()
        g = torch._neg_view(torch.randn(3, n, n, device="cuda", dtype=dtype))
        y = fh.matrix_exp(a)
        (grad,) = torch.autograd.grad(y, a, g)
        check_error(y, reference(a))
        check_error(grad, reference(a.mT, g), backward=True)
        check_north_star(y, reference(a))


@pytest.mark.parametrize("n", [4, 8, 9, 16, 32])
def test_operand_spanning_more_than_2gib(n):
    """A view whose single matrix spans > 2 GiB of storage (row stride 2^27 elements): the
    P = 16/32 kernels' 32-bit buffer offsets cannot reach it, so the launcher takes the
    64-bit-indexed kernel; N <= 8 kernels index in 64 bits themselves.  Results must match
    the same matrices passed contiguously, to the north-star tolerance."""
    row_stride = 1 << 27
    batch = 3
    storage = torch.zeros((n - 1) * row_stride + batch * n + n, device="cuda")
    a = storage.as_strided((batch, n, n), (n, row_stride, 1))
    a.copy_(torch.randn(batch, n, n, device="cuda") * 0.5)
    g = torch.randn(batch, n, n, device="cuda")
    dense = a.contiguous()
    y = torch.ops.flash_hypercons._matrix_exp(a)
    frechet = torch.ops.flash_hypercons._frechet(a, g)
    check_north_star(y, reference(dense))
    check_north_star(frechet, reference(dense, g), backward=True)
    check_north_star(torch.ops.flash_hypercons._frechet(g, a), reference(g, dense), backward=True)
    del storage, a


def test_vjp_matches_central_difference():
    for n in (3, 4, 8, 16, 32):
        a = (torch.randn(2, n, n, device="cuda") * 0.03).requires_grad_()
        h = torch.randn_like(a) * 0.1
        g = torch.randn_like(a) * 0.2
        (gradient,) = torch.autograd.grad(fh.matrix_exp(a), a, g)
        step = 0.005
        with torch.no_grad():
            diff = ((fh.matrix_exp(a + step * h) - fh.matrix_exp(a - step * h)) * g).sum() / (2 * step)
        torch.testing.assert_close((gradient * h).sum(), diff, atol=0.001, rtol=0.005)


@pytest.mark.parametrize("n", [4, 8, 16, 32])
@pytest.mark.parametrize("dtype", DTYPES)
def test_large_rotations(dtype, n):
    for batch in (1, 129):
        for angle in (25, 100, 1000):
            a = torch.zeros(batch, n, n, device="cuda", dtype=dtype)
            a[:, 0, 1], a[:, 1, 0] = -angle, angle
            a.requires_grad_()
            expected = torch.eye(n, device="cuda", dtype=torch.float64).expand(batch, n, n).clone()
            expected[:, 0, 0] = expected[:, 1, 1] = math.cos(angle)
            expected[:, 0, 1], expected[:, 1, 0] = -math.sin(angle), math.sin(angle)
            y = fh.matrix_exp(a)
            g = (0.125 * torch.eye(n, device="cuda", dtype=dtype)).expand_as(a)
            (grad,) = torch.autograd.grad(y, a, g)
            check_error(y, expected)
            check_error(grad, 0.125 * expected.mT, backward=True)
            tol = 0.002 if dtype == torch.float32 else 0.1
            yy = y.detach().double()
            torch.testing.assert_close(yy.mT @ yy, torch.eye(n, device="cuda", dtype=torch.float64).expand_as(yy),
                                       atol=tol, rtol=0)


def test_honours_current_stream():
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        a = (torch.randn(3, 9, 9, device="cuda") * 0.1).requires_grad_()
        b = (torch.randn(5, 4, 4, device="cuda") * 0.1).requires_grad_()
        y = fh.matrix_exp(a)
        z = fh.matrix_exp(b)
        (grad,) = torch.autograd.grad(y.sum(), a)
        (grad_b,) = torch.autograd.grad(z.sum(), b)
    stream.synchronize()
    check_error(y, reference(a))
    check_error(grad, reference(a.mT, torch.ones_like(a)), backward=True)
    check_error(z, reference(b))
    check_error(grad_b, reference(b.mT, torch.ones_like(b)), backward=True)


def test_custom_ops_dispatch():
    a = (torch.randn(3, 4, 4, device="cuda") * 0.03).requires_grad_()
    y, names = op_names(lambda: fh.matrix_exp(a))
    assert "flash_hypercons::_matrix_exp" in names
    _, names = op_names(lambda: torch.autograd.grad(y.sum(), a))
    assert "flash_hypercons::_frechet" in names


def test_invalid_direct_calls_raise_reference_messages():
    with pytest.raises(RuntimeError, match="expected a strided CUDA"):
        torch.ops.flash_hypercons._matrix_exp(torch.randn(2, 33, 33, device="cuda"))
    with pytest.raises(RuntimeError, match="expected a strided CUDA"):
        torch.ops.flash_hypercons._matrix_exp(torch.randn(2, 4, 4, device="cuda", dtype=torch.float64))
    with pytest.raises(RuntimeError, match="direction must match"):
        torch.ops.flash_hypercons._frechet(torch.randn(2, 4, 4, device="cuda"), torch.randn(2, 5, 5, device="cuda"))


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_graph_capture_replays_match_eager(n):
    """The launches allocate nothing and issue no memsets, so forward + Frechet can be captured
    in a HIP graph; every replay (with eager work in between) equals the eager result bit for bit."""
    torch.manual_seed(n)
    x = torch.randn(300, n, n, device="cuda") * 0.4
    g = torch.randn(300, n, n, device="cuda")
    eager_y = torch.ops.flash_hypercons._matrix_exp(x)
    eager_d = torch.ops.flash_hypercons._frechet(x.mT, g)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):  # warm-up on the capture stream
            torch.ops.flash_hypercons._matrix_exp(x)
            torch.ops.flash_hypercons._frechet(x.mT, g)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = torch.ops.flash_hypercons._matrix_exp(x)
        d = torch.ops.flash_hypercons._frechet(x.mT, g)
    for replay in range(3):
        y.zero_()
        d.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager_y), f"replay {replay}"
        assert torch.equal(d, eager_d), f"replay {replay}"
        torch.ops.flash_hypercons._matrix_exp(g)  # unrelated eager work between replays


@pytest.mark.skipif(torch.cuda.device_count() < 2, reason="needs a second GPU (these boxes have one)")
def test_input_on_noncurrent_device():
    """The launch runs on the input's device under a device guard and restores the current one
    (reference tests/test_matrix_exp.py:143-149)."""
    torch.cuda.set_device(0)
    a = torch.randn(2, 4, 4, device="cuda:1") * 0.1
    y = fh.matrix_exp(a)
    assert torch.cuda.current_device() == 0
    assert y.device == a.device
    check_north_star(y, reference(a))
