"""Stream mixing for 5 <= n <= 8 streams: ``fh.mix_streams(h, x) = exp(h) @ x``
with exp(h) computed by ``matrix_exp`` in FP32 and applied by the streaming
kernels behind ``_hc_apply`` / ``_hc_apply_backward``.  Checks, on the GPU:

* E = ``_matrix_exp(h.float())`` is bit-identical to the CPU restatement's FP32
  exponential (the P = 8 kernel), so the path starts from the same bits the
  2 <= n <= 4 fusion keeps on chip;
* y = E x and dx = E^T dY agree with FP64 products of the same operands,
  element by element, within the bound of an n-term FMA chain in FP32 plus the
  rounding to the storage dtype; dE = dY x^T within the bound of its summation
  (per-lane chains of about C/64 terms, then a 6-level tree);
* dh through autograd is bit-identical to the restatement's L(h^T, dE) on the
  kernel's own dE, rounded to h's dtype; both gradients agree with FP64
  autograd of ``linalg.matrix_exp(h) @ x`` normwise;
* views of x and dY, C not a multiple of the vector width, batches larger
  than the grid and token slices give the same bits; non-finite h gives NaN
  for that token only; dE does not change from run to run;
* a mistake planted in the FP64 reference (transposed E, dropped term, dE
  transposed) fails the bounds, so the bounds can see one.
"""

import pytest
import torch

import flash_hypercons as fh
import oracle

from tests.mixcheck import bound_violations, dE_terms, oracle_exp, oracle_frechet

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
OPS = torch.ops.flash_hypercons
THREADS = oracle.default_threads()


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view({4: torch.int32, 2: torch.int16}[t.element_size()])


def same_bits(a, b):
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(_bits(a), _bits(b))


def _inputs(b, n, c, dtype, scale=0.5, device="cuda"):
    h = (torch.randn(b, n, n, device=device) * scale).to(dtype)
    x = torch.randn(b, n, c, device=device).to(dtype)
    return h, x


def _exp(h):
    return OPS._matrix_exp(h.float())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("n", [5, 6, 7, 8])
@pytest.mark.parametrize("c", [8, 40, 2056, 5000])
def test_forward_and_backward_against_restatement_and_fp64(n, c, dtype):
    h, x = _inputs(33, n, c, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    e = _exp(h)
    e_ref = oracle_exp(h, THREADS)
    assert same_bits(e.cpu(), e_ref), "exp(h) differs from the restatement"
    y = OPS._hc_apply(e, x)
    assert same_bits(y, fh.mix_streams(h, x))
    e64, x64, g64 = e_ref.double(), x.double().cpu(), g.double().cpu()
    assert bound_violations(y, e64 @ x64, e64.abs() @ x64.abs(), n, dtype) == 0
    dx, de = OPS._hc_apply_backward(e, x, g)
    assert de.dtype == torch.float32 and de.shape == (33, n, n)
    assert bound_violations(dx, e64.mT @ g64, e64.abs().mT @ g64.abs(), n, dtype) == 0
    assert bound_violations(de, g64 @ x64.mT, g64.abs() @ x64.abs().mT, dE_terms(c), torch.float32) == 0
    _, de2 = OPS._hc_apply_backward(e, x, g)
    assert same_bits(de2, de), "dE must not change from run to run"
    hr, xr = h.clone().requires_grad_(), x.clone().requires_grad_()
    fh.mix_streams(hr, xr).backward(g)
    assert same_bits(xr.grad, dx)
    dh_ref = oracle.round_to_dtype(oracle_frechet(h.mT, de, THREADS), dtype)
    assert same_bits(hr.grad, dh_ref), "dh differs from the restatement's L(h^T, dE)"


@pytest.mark.gpu
def test_planted_mistakes_fail_the_bounds():
    h, x = _inputs(16, 8, 512, torch.float32)
    g = torch.randn_like(x)
    e = _exp(h)
    e64, x64, g64 = oracle_exp(h, THREADS).double(), x.double().cpu(), g.double().cpu()
    y = OPS._hc_apply(e, x)
    dx, de = OPS._hc_apply_backward(e, x, g)
    scale = e64.abs() @ x64.abs()
    assert bound_violations(y, e64 @ x64, scale, 8, torch.float32) == 0
    assert bound_violations(y, e64.mT @ x64, scale, 8, torch.float32) > 0
    dropped = e64.clone()
    dropped[:, :, 7] = 0
    assert bound_violations(y, dropped @ x64, scale, 8, torch.float32) > 0
    assert bound_violations(dx, e64 @ g64, e64.abs().mT @ g64.abs(), 8, torch.float32) > 0
    de_scale = g64.abs() @ x64.abs().mT
    assert bound_violations(de, x64 @ g64.mT, de_scale, dE_terms(512), torch.float32) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_autograd_against_fp64(dtype):
    h0, x0 = _inputs(24, 6, 264, dtype)
    g = torch.randn_like(x0, dtype=torch.float32).to(dtype)
    h, x = h0.clone().requires_grad_(), x0.clone().requires_grad_()
    fh.mix_streams(h, x).backward(g)
    h64 = h0.double().cpu().requires_grad_()
    x64 = x0.double().cpu().requires_grad_()
    (torch.linalg.matrix_exp(h64) @ x64).backward(g.double().cpu())
    tol = {torch.float32: 1e-5, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}[dtype]
    for got, ref in ((h.grad, h64.grad), (x.grad, x64.grad)):
        assert got.dtype == dtype
        err = (got.double().cpu() - ref).flatten(1).norm(dim=1) / ref.flatten(1).norm(dim=1)
        assert err.max().item() < tol, err.max().item()


@pytest.mark.gpu
def test_graph_building_backward():
    h0, x0 = _inputs(6, 7, 64, torch.float32)
    g = torch.randn_like(x0)
    h, x = h0.clone().requires_grad_(), x0.clone().requires_grad_()
    dh, dx = torch.autograd.grad(fh.mix_streams(h, x), (h, x), g, create_graph=True)
    hk, xk = h0.clone().requires_grad_(), x0.clone().requires_grad_()
    fh.mix_streams(hk, xk).backward(g)
    torch.testing.assert_close(dh, hk.grad, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(dx, xk.grad, rtol=1e-5, atol=1e-5)
    (second,) = torch.autograd.grad((dh * dh).sum() + (dx * dx).sum(), x)
    h64, x64 = h0.double().requires_grad_(), x0.double().requires_grad_()
    dh64, dx64 = torch.autograd.grad(torch.linalg.matrix_exp(h64) @ x64, (h64, x64), g.double(), create_graph=True)
    (second64,) = torch.autograd.grad((dh64 * dh64).sum() + (dx64 * dx64).sum(), x64)
    err = (second.double() - second64).flatten(1).norm(dim=1) / second64.flatten(1).norm(dim=1)
    assert err.max().item() < 1e-4, err


@pytest.mark.gpu
def test_gradient_of_one_operand():
    h, x = _inputs(9, 6, 72, torch.bfloat16)
    g = torch.randn_like(x, dtype=torch.float32).to(torch.bfloat16)
    xr = x.clone().requires_grad_()
    fh.mix_streams(h, xr).backward(g)
    hr = h.clone().requires_grad_()
    fh.mix_streams(hr, x).backward(g)
    dx, de = OPS._hc_apply_backward(_exp(h), x, g)
    assert same_bits(xr.grad, dx)
    assert same_bits(hr.grad, OPS._frechet(h.float().mT, de).to(torch.bfloat16))


@pytest.mark.gpu
@pytest.mark.compile
def test_compile_keeps_the_apply_operators():
    h, x = _inputs(16, 8, 128, torch.bfloat16)
    g = torch.randn_like(x, dtype=torch.float32).to(torch.bfloat16)
    compiled = torch.compile(lambda a, b: fh.mix_streams(a, b), fullgraph=True)
    hr, xr = h.clone().requires_grad_(), x.clone().requires_grad_()
    y = compiled(hr, xr)
    y.backward(g)
    assert same_bits(y, fh.mix_streams(h, x))
    he, xe = h.clone().requires_grad_(), x.clone().requires_grad_()
    fh.mix_streams(he, xe).backward(g)
    assert same_bits(hr.grad, he.grad) and same_bits(xr.grad, xe.grad)


def _x_view(x, layout):
    b, n, c = x.shape
    if layout == "contiguous":
        return x
    if layout == "wide_rows":
        wide = torch.zeros(b, n, c + 64, dtype=x.dtype, device=x.device)
        wide[..., :c] = x
        return wide[..., :c]
    if layout == "token_major":
        return x.transpose(0, 1).contiguous().transpose(0, 1)
    if layout == "negated":
        return torch._neg_view((-x).contiguous())
    if layout == "column_strided":
        wide = torch.zeros(b, n, 2 * c, dtype=x.dtype, device=x.device)
        wide[..., ::2] = x
        return wide[..., ::2]
    raise ValueError(layout)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("xl", ["contiguous", "wide_rows", "token_major", "negated", "column_strided"])
@pytest.mark.parametrize("c", [96, 100])
def test_layouts_give_the_same_bits(xl, c, dtype):
    h, x = _inputs(11, 8, c, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    e = _exp(h)
    xv, gv = _x_view(x, xl), _x_view(g, xl)
    assert same_bits(OPS._hc_apply(e, xv), OPS._hc_apply(e, x))
    assert same_bits(OPS._hc_apply(e.mT.contiguous().mT, xv), OPS._hc_apply(e, x))
    dx, de = OPS._hc_apply_backward(e, xv, gv)
    dx_c, de_c = OPS._hc_apply_backward(e, x, g)
    assert same_bits(dx, dx_c) and same_bits(de, de_c)
    assert same_bits(fh.mix_streams(h, xv), fh.mix_streams(h, x))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=str)
def test_tokens_do_not_depend_on_the_batch(dtype):
    # 40,000 tokens: more token sets than the grid holds, so the grid-stride loop is used.
    h, x = _inputs(40000, 5, 16, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    e = _exp(h)
    y = OPS._hc_apply(e, x)
    dx, de = OPS._hc_apply_backward(e, x, g)
    for lo, hi in ((0, 1), (5, 14), (39991, 40000), (17, 4113)):
        assert same_bits(OPS._hc_apply(e[lo:hi], x[lo:hi]), y[lo:hi])
        dx_s, de_s = OPS._hc_apply_backward(e[lo:hi], x[lo:hi], g[lo:hi])
        assert same_bits(dx_s, dx[lo:hi]) and same_bits(de_s, de[lo:hi])


@pytest.mark.gpu
def test_empty_batch():
    h, x = _inputs(0, 6, 64, torch.float32)
    assert fh.mix_streams(h, x).shape == (0, 6, 64)
    dx, de = OPS._hc_apply_backward(_exp(h), x, x)
    assert dx.shape == (0, 6, 64) and de.shape == (0, 6, 6)


@pytest.mark.gpu
@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_nonfinite_h_poisons_only_its_token(bad):
    h, x = _inputs(20, 8, 64, torch.float32)
    g = torch.randn_like(x)

    def run(hh):
        hr, xr = hh.clone().requires_grad_(), x.clone().requires_grad_()
        y = fh.mix_streams(hr, xr)
        y.backward(g)
        return y.detach(), hr.grad, xr.grad

    clean = run(h)
    h[9, 1, 2] = bad
    poisoned = run(h)
    keep = torch.arange(20) != 9
    for a, b in zip(poisoned, clean):
        assert torch.isnan(a[9]).all()
        assert same_bits(a[keep], b[keep])


@pytest.mark.gpu
def test_operator_checks():
    e = torch.zeros(2, 4, 4, device="cuda")
    x = torch.zeros(2, 4, 8, device="cuda")
    with pytest.raises(RuntimeError, match="5 <= n <= 8"):
        OPS._hc_apply(e, x)
    e8 = torch.zeros(2, 8, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="float32"):
        OPS._hc_apply(e8, torch.zeros(2, 8, 8, device="cuda"))
    with pytest.raises(RuntimeError, match="grad must match"):
        OPS._hc_apply_backward(e8.float(), torch.zeros(2, 8, 8, device="cuda"), torch.zeros(2, 8, 16, device="cuda"))


def test_cpu_and_other_n_are_the_composition():
    h, x = _inputs(4, 6, 10, torch.float32, device="cpu")
    assert torch.equal(fh.mix_streams(h, x), torch.linalg.matrix_exp(h) @ x)


def test_operator_schemas():
    assert str(OPS._hc_apply.default._schema) == "flash_hypercons::_hc_apply(Tensor e, Tensor x) -> Tensor"
    assert (
        str(OPS._hc_apply_backward.default._schema)
        == "flash_hypercons::_hc_apply_backward(Tensor e, Tensor x, Tensor grad) -> (Tensor, Tensor)"
    )


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        e = torch.empty(8, 6, 6, device="cuda")
        x = torch.empty(8, 6, 100, device="cuda", dtype=torch.bfloat16)
        assert OPS._hc_apply(e, x).shape == (8, 6, 100)
        dx, de = OPS._hc_apply_backward(e, x, x)
        assert dx.shape == (8, 6, 100) and de.shape == (8, 6, 6) and de.dtype == torch.float32
