"""Numerical and behavioural contract of the operators on the GPU.

* every size 2..32, dtype and batch (empty included) meets the north-star
  tolerances against FP64, with contiguous outputs in the input dtype;
* results do not depend on how an operand is laid out (transposed, negated,
  expanded, padded rows) -- bit for bit against the materialised operand --
  nor on the batch around a matrix or its position in it;
* the squaring count steps exactly where ||A||_1 crosses theta18 * 2^k (exact
  rational arithmetic decides), non-finite matrices give NaN matrices without
  touching their neighbours;
* closed forms: rotations, diagonal matrices (the Frechet derivative's divided
  differences), nilpotent matrices, scalar-plus-nilpotent;
* the backward kernel is the adjoint of the forward-mode kernel, and the
  forward-mode kernel is the derivative of the forward one;
* streams, HIP-graph capture, > 2 GiB strides, error messages, device guard.
"""

import math
from fractions import Fraction

import pytest
import torch

import flash_hypercons as fh
import oracle
from tests.fullsize import error_ratio, excess_over_reference
from tests.reference import check_north_star, reference

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
THETA = 3.010066362817634
EXP = torch.ops.flash_hypercons._matrix_exp
FRECHET = torch.ops.flash_hypercons._frechet


def rand(shape, dtype=torch.float32, scale=0.3, seed=0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=gen, dtype=torch.float64) * scale).to(dtype).cuda()


def step(x, g):
    """Forward and autograd backward through the public entry point."""
    xin = x.detach().requires_grad_()
    y = fh.matrix_exp(xin)
    (grad,) = torch.autograd.grad(y, xin, g)
    return y.detach(), grad


@pytest.mark.parametrize("batch", [0, 1, 35, 300])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", range(2, 33))
def test_every_size_dtype_and_batch(n, dtype, batch):
    x = rand((batch, n, n), dtype, scale=1.0 / n**0.5, seed=n).mT  # noncontiguous input
    g = rand((batch, n, n), dtype, scale=1.0, seed=1000 + n)
    y, grad = step(x, g)
    for out in (y, grad):
        assert out.dtype == dtype and out.device == x.device and out.shape == x.shape
        assert out.is_contiguous()
    if batch:
        check_north_star(y, reference(x))
        check_north_star(grad, reference(x.mT, g), backward=True)


def _layout(values, kind):
    """The same logical values stored in another way."""
    if kind == "contiguous":
        return values.contiguous()
    if kind == "transposed":
        return values.mT.contiguous().mT
    if kind == "negated":
        return torch._neg_view((-values).contiguous())
    if kind == "negated transposed":
        return torch._neg_view((-values).mT.contiguous().mT)
    if kind == "padded rows":
        b, n, _ = values.shape
        buf = torch.zeros(b, n, n + 3, dtype=values.dtype, device=values.device)
        buf[..., :n] = values
        return buf[..., :n]
    if kind == "batch stride 0":
        return values[:1].expand_as(values)
    raise ValueError(kind)


LAYOUTS = ["transposed", "negated", "negated transposed", "padded rows", "batch stride 0"]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 3, 4, 5, 8, 9, 16, 17, 32])
def test_layouts_are_read_in_place_bit_for_bit(n, dtype):
    """The kernels read strided, negated and broadcast operands in place; the numbers they
    produce must be the bits they produce for the materialised contiguous operand."""
    values = rand((67, n, n), dtype, scale=1.5 / n**0.5, seed=3 * n)
    gvals = rand((67, n, n), dtype, scale=1.0, seed=7 * n)
    for kind in LAYOUTS:
        x = _layout(values, kind)
        dense = x.contiguous() if not x.is_neg() else x.resolve_neg().contiguous()
        assert torch.equal(EXP(x), EXP(dense)), kind
        for gkind in ("contiguous", kind):
            d = _layout(gvals, gkind)
            dd = d.resolve_neg().contiguous()
            assert torch.equal(FRECHET(x, d), FRECHET(dense, dd)), (kind, gkind)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 5, 8, 9, 16, 17, 32])
def test_result_independent_of_batch_and_position(n, dtype):
    """One probe matrix planted at the first, group-boundary and last positions of batches of
    many sizes: its forward and Frechet results are always the same bits."""
    probe = rand((1, n, n), dtype, scale=2.0 / n**0.5, seed=11)
    gprobe = rand((1, n, n), dtype, scale=1.0, seed=12)
    seen_y = seen_d = None
    for batch in (1, 2, 15, 63, 64, 65, 129, 257, 1000):
        x = rand((batch, n, n), dtype, scale=2.0 / n**0.5, seed=batch)
        g = rand((batch, n, n), dtype, scale=1.0, seed=batch + 1)
        spots = sorted({0, min(63, batch - 1), min(64, batch - 1), batch - 1})
        for i in spots:
            x[i], g[i] = probe[0], gprobe[0]
        y, d = EXP(x), FRECHET(x, g)
        for i in spots:
            if seen_y is None:
                seen_y, seen_d = y[i].clone(), d[i].clone()
            assert torch.equal(y[i], seen_y) and torch.equal(d[i], seen_d), (batch, i)


def _exact_squarings(m):
    """Smallest s >= 0 with ||m||_1 <= theta18 * 2^s, in exact rational arithmetic."""
    rows = m.double().cpu().tolist()
    norm = max(sum(Fraction(abs(r[j])) for r in rows) for j in range(len(rows)))
    s = 0
    while norm > Fraction(THETA) * 2**s:
        s += 1
    return s


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 8, 16, 32])
def test_squaring_count_steps_at_theta_boundaries(n, dtype):
    """Matrices scaled to 1-norms a hair below and above theta18 * 2^k (k = 0..5): the kernels'
    squaring count is the exact rational one and the restatement's, forward and backward."""
    targets = [0.0, 1e-3]
    for k in range(6):
        for rel in (-3e-5, 3e-5):
            targets.append(THETA * 2**k * (1 + rel))
    m = rand((len(targets), n, n), torch.float64, scale=1.0, seed=n)
    m = m - m.mT  # skew-symmetric: exp is orthogonal, so large norms do not overflow FP16
    m = m / torch.linalg.matrix_norm(m, ord=1)[:, None, None]
    a = (m * torch.tensor(targets, dtype=torch.float64, device="cuda")[:, None, None]).to(dtype)
    params, _ = torch.ops.flash_hypercons._expm_params(a)
    _, s_kernel = torch.ops.flash_hypercons._expm_debug(a, None, 0)
    exact = [_exact_squarings(a[i]) for i in range(len(targets))]
    assert params[:, 1].cpu().tolist() == exact
    assert s_kernel.cpu().tolist() == exact
    assert exact == oracle.torch_params(a.cpu())[0].tolist()
    g = rand(a.shape, dtype, scale=0.01, seed=5)
    pb, _ = torch.ops.flash_hypercons._expm_params(a.mT, g)
    assert torch.equal(pb[:, 1].cpu(), oracle.torch_params(a.mT.cpu(), g.cpu())[0])
    y, grad = step(a, g)
    # Accuracy: within the north-star bound, or -- where scaling and squaring at s = 5, 6 takes the
    # reference's own FP32 arithmetic beyond it -- no worse than that arithmetic (the restatement).
    for out, x, d, backward in ((y, a, None, False), (grad, a.mT, g, True)):
        ora = (oracle.torch_matrix_exp(x.cpu()) if d is None else oracle.torch_frechet(x.cpu(), d.cpu()))[0]
        ref64 = reference(x, d)
        excess = excess_over_reference(error_ratio(out, ref64, backward=backward),
                                       error_ratio(ora.cuda(), ref64, backward=backward), dtype)
        limit = 1.5 if dtype == torch.float32 else 1.0
        assert float(excess.max()) <= limit, excess.tolist()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [3, 4, 8, 13, 32])
def test_nonfinite_matrices_become_nan_without_touching_neighbours(n, dtype):
    x = rand((7, n, n), dtype, scale=0.2, seed=2)
    g = rand((7, n, n), dtype, scale=1.0, seed=3)
    clean_y, clean_d = EXP(x), FRECHET(x, g)
    x[1, 0, 0] = float("nan")
    x[2, n - 1, n - 1] = float("inf")
    x[3, 0, n - 1] = -float("inf")
    g[4, n // 2, 0] = float("nan")  # only the Frechet direction is bad
    y, d = EXP(x), FRECHET(x, g)
    for i in (1, 2, 3):
        assert bool(y[i].isnan().all()) and bool(d[i].isnan().all())
    assert bool(d[4].isnan().all()) and torch.equal(y[4], clean_y[4])
    for i in (0, 5, 6):
        assert torch.equal(y[i], clean_y[i]) and torch.equal(d[i], clean_d[i])
    params, _ = torch.ops.flash_hypercons._expm_params(x)
    assert params[1:4].cpu().tolist() == [[-1, -1]] * 3


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 8, 16, 32])
def test_zero_matrix_gives_identity_and_direction(n, dtype):
    """exp(0) = I exactly (the polynomial's constant term (b3_0 + b4_0) * b4_0 rounds to 1.0f), and
    L(0, G) = G up to the rounding of the polynomial's linear coefficient chain: a few FP32 ulps,
    exact after rounding to FP16/BF16; the same bits as the restatement at n <= 8."""
    z = torch.zeros(3, n, n, dtype=dtype, device="cuda")
    g = rand((3, n, n), dtype, scale=1.0, seed=9)
    assert torch.equal(EXP(z), torch.eye(n, dtype=dtype, device="cuda").expand(3, n, n))
    d = FRECHET(z, g)
    if dtype == torch.float32:
        torch.testing.assert_close(d, g, rtol=4 * 2.0**-24, atol=0)
    else:
        assert torch.equal(d, g)
    if n <= 8:
        assert torch.equal(d.cpu(), oracle.torch_frechet(z.cpu(), g.cpu())[0])


def _rotation(batch, n, angles, dtype):
    a = torch.zeros(batch, n, n, dtype=torch.float64, device="cuda")
    ang = torch.tensor(angles, dtype=torch.float64, device="cuda").repeat(batch // len(angles) + 1)[:batch]
    ang = ang.to(dtype).double()  # the angle the kernel sees (1500 is not a BF16 value)
    a[:, 0, 1], a[:, 1, 0] = -ang, ang
    exact = torch.eye(n, dtype=torch.float64, device="cuda").repeat(batch, 1, 1)
    exact[:, 0, 0] = exact[:, 1, 1] = torch.cos(ang)
    exact[:, 0, 1], exact[:, 1, 0] = -torch.sin(ang), torch.sin(ang)
    return a.to(dtype), exact


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 4, 8, 16, 32])
def test_closed_form_rotations(n, dtype):
    """exp of a plane-rotation generator with angles up to 1500 rad (s up to 9): cosine/sine
    entries, orthogonality, and L(A^T, c I) = c exp(A^T) since I commutes with A."""
    a, exact = _rotation(130, n, [0.75, 6.0, 37.5, 250.0, 1500.0], dtype)
    y, grad = step(a, (0.25 * torch.eye(n, device="cuda")).to(dtype).expand(130, n, n))
    tol = 3e-3 if dtype == torch.float32 else 6e-2
    torch.testing.assert_close(y.double(), exact, atol=tol, rtol=0)
    torch.testing.assert_close(grad.double(), 0.25 * exact.mT, atol=tol, rtol=0)
    yy = y.double()
    torch.testing.assert_close(yy.mT @ yy, torch.eye(n, dtype=torch.float64, device="cuda").expand_as(yy),
                               atol=2 * tol, rtol=0)


@pytest.mark.parametrize("n", [3, 4, 7, 8, 12, 16, 32])
def test_closed_form_diagonal_divided_differences(n):
    """For D = diag(d): exp(D) = diag(e^d) and L(D, E)_ij = E_ij (e^d_i - e^d_j) / (d_i - d_j)
    (e^d_i on the diagonal), the Frechet derivative's divided-difference form."""
    gen = torch.Generator().manual_seed(n)
    d = (torch.rand(4, n, generator=gen, dtype=torch.float64) * 6 - 3)
    e = torch.randn(4, n, n, generator=gen, dtype=torch.float64)
    ed = d.exp()
    num = ed[:, :, None] - ed[:, None, :]
    den = d[:, :, None] - d[:, None, :]
    dd = torch.where(den == 0, ed[:, :, None].expand_as(num), num / torch.where(den == 0, 1.0, den))
    a = torch.diag_embed(d).float().cuda()
    check_north_star(EXP(a), torch.diag_embed(ed).cuda())
    check_north_star(FRECHET(a, e.float().cuda()), (e * dd).cuda(), backward=True)


@pytest.mark.parametrize("n", [2, 4, 6, 8, 16, 32])
def test_closed_form_scalar_plus_nilpotent(n):
    """A = c I + N with N strictly upper triangular: exp(A) = e^c (I + N + N^2/2! + ...), a finite
    sum; the Frechet derivative in direction N is exp(A) N (N commutes with A)."""
    gen = torch.Generator().manual_seed(n)
    nil = torch.triu(torch.randn(3, n, n, generator=gen, dtype=torch.float64) / n**0.5, diagonal=1)
    c = torch.tensor([-1.0, 0.0, 1.5], dtype=torch.float64)
    a = nil + c[:, None, None] * torch.eye(n, dtype=torch.float64)
    series = torch.eye(n, dtype=torch.float64).expand(3, n, n).clone()
    term = series.clone()
    for k in range(1, n):
        term = term @ nil / k
        series = series + term
    exact = c.exp()[:, None, None] * series
    check_north_star(EXP(a.float().cuda()), exact.cuda())
    check_north_star(FRECHET(a.float().cuda(), nil.float().cuda()), (exact @ nil).cuda(), backward=True)


@pytest.mark.parametrize("n", [3, 4, 8, 9, 16, 32])
def test_backward_is_adjoint_of_forward_mode(n):
    """<L(A^T, G), H> = <G, L(A, H)>: the reverse-mode (gradient) kernel is the adjoint of the
    forward-mode kernel, and the forward-mode kernel is the derivative of the forward kernel
    (fourth-order central difference of exp in FP64 direction)."""
    a = rand((6, n, n), scale=1.2 / n**0.5, seed=n)
    g = rand((6, n, n), scale=1.0, seed=n + 1)
    h = rand((6, n, n), scale=1.0, seed=n + 2)
    vjp = FRECHET(a.mT, g).double()
    jvp = FRECHET(a, h).double()
    lhs = (vjp * h.double()).sum((-2, -1))
    rhs = (g.double() * jvp).sum((-2, -1))
    fro = lambda t: t.flatten(1).norm(dim=1)  # noqa: E731
    scale = fro(vjp) * fro(h.double()) + fro(g.double()) * fro(jvp)
    assert bool(((lhs - rhs).abs() <= 2e-5 * scale).all())
    step_h = 1e-2
    ad = a.double()

    def e64(t):
        return torch.linalg.matrix_exp(ad + t * h.double())

    fd = (8 * (e64(step_h) - e64(-step_h)) - (e64(2 * step_h) - e64(-2 * step_h))) / (12 * step_h)
    check_north_star(FRECHET(a, h), fd, backward=True)


def test_side_stream_results_equal_default_stream():
    x = rand((300, 9, 9), scale=0.5, seed=1)
    g = rand((300, 9, 9), scale=1.0, seed=2)
    x4 = rand((300, 4, 4), scale=0.5, seed=3)
    expect = (EXP(x), FRECHET(x.mT, g), EXP(x4))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        y, grad = step(x, g)
        y4 = fh.matrix_exp(x4)
    stream.synchronize()
    assert torch.equal(y, expect[0]) and torch.equal(grad, expect[1]) and torch.equal(y4, expect[2])


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_graph_capture_replays_match_eager(n):
    """The launches allocate nothing and issue no memsets, so forward + Frechet can be captured
    in a HIP graph; every replay (with eager work in between) equals the eager result bit for bit."""
    x = rand((300, n, n), scale=0.4, seed=n)
    g = rand((300, n, n), scale=1.0, seed=n + 1)
    eager_y = EXP(x)
    eager_d = FRECHET(x.mT, g)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):  # warm-up on the capture stream
            EXP(x)
            FRECHET(x.mT, g)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = EXP(x)
        d = FRECHET(x.mT, g)
    for replay in range(3):
        y.zero_()
        d.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager_y), f"replay {replay}"
        assert torch.equal(d, eager_d), f"replay {replay}"
        EXP(g)  # unrelated eager work between replays


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
    check_north_star(EXP(a), reference(dense))
    check_north_star(FRECHET(a, g), reference(dense, g), backward=True)
    check_north_star(FRECHET(g, a), reference(g, dense), backward=True)
    del storage, a


@pytest.mark.parametrize("n", [4, 8])
def test_dense_batch_larger_than_2gib(n):
    """A packed batch of more than 2 GiB: the buffer-to-LDS (P = 4) and count-ordered (P = 8)
    kernels address it with 32-bit offsets, so the launcher takes the 64-bit-indexed kernels.
    Sampled matrices (the first, those around byte 2^31, the last, and random ones) must be
    the bits the same matrices give in a small batch and the oracle's, forward and Frechet."""
    batch = (1 << 31) // (4 * n * n) + 3
    gen = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(batch, n, n, device="cuda", generator=gen) * 0.3
    g = torch.randn(batch, n, n, device="cuda", generator=gen)
    edge = (1 << 31) // (4 * n * n)
    idx = torch.cat((torch.tensor([0, edge - 2, edge - 1, edge, edge + 1, batch - 1]),
                     torch.randint(0, batch, (250,), generator=torch.Generator().manual_seed(n)))).unique().cuda()
    for y, small, direction in ((EXP(x), EXP(x[idx]), None), (FRECHET(x.mT, g), FRECHET(x[idx].mT, g[idx]), g)):
        assert torch.equal(y[idx], small)
        if direction is None:
            want, _ = oracle.torch_matrix_exp(x[idx].cpu())
        else:
            want, _ = oracle.torch_frechet(x[idx].mT.cpu(), direction[idx].cpu())
        assert torch.equal(small.cpu(), want)
        del y
    del x, g
    torch.cuda.empty_cache()


def test_invalid_direct_calls_raise_reference_messages():
    with pytest.raises(RuntimeError, match="expected a strided CUDA"):
        EXP(torch.randn(2, 33, 33, device="cuda"))
    with pytest.raises(RuntimeError, match="expected a strided CUDA"):
        EXP(torch.randn(2, 4, 4, device="cuda", dtype=torch.float64))
    with pytest.raises(NotImplementedError):
        EXP(torch.randn(2, 4, 4))  # registered for the device dispatch key only, as in the reference
    with pytest.raises(RuntimeError, match="direction must match"):
        FRECHET(torch.randn(2, 4, 4, device="cuda"), torch.randn(2, 5, 5, device="cuda"))


@pytest.mark.skipif(torch.cuda.device_count() < 2, reason="needs a second GPU (these boxes have one)")
def test_input_on_noncurrent_device():
    """The launch runs on the input's device under a device guard and restores the current one."""
    torch.cuda.set_device(0)
    a = torch.randn(2, 4, 4, device="cuda:1") * 0.1
    y = fh.matrix_exp(a)
    assert torch.cuda.current_device() == 0
    assert y.device == a.device
    check_north_star(y, reference(a))


def test_rotation_angles_reach_large_squaring_counts():
    """The rotation case above really exercises deep squaring: s grows like log2(angle)."""
    a, _ = _rotation(5, 4, [0.75, 6.0, 37.5, 250.0, 1500.0], torch.float32)
    params, _ = torch.ops.flash_hypercons._expm_params(a)
    s = params[:, 1].cpu().tolist()
    assert s == sorted(s) and s[-1] >= 9 and s[0] == 0
    assert s[-1] == math.ceil(math.log2(1500.0 / THETA))
