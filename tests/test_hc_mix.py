"""Fused hyper-connection stream mixing, ``fh.mix_streams(h, x) = exp(h) @ x``.

The reference returns exp(h) (ops/matrix_exp/__init__.py:80-97) and the caller
multiplies; this build fuses the product (and its backward) into one kernel per
direction for 2 <= n <= 4.  Checks, on the GPU:

* exp(h) inside the kernel (read back through the debug operator
  ``_hc_mix_aux``) is bit-identical to the CPU restatement's FP32 exponential,
  and rounds to exactly what ``fh.matrix_exp`` returns;
* y = exp(h) x agrees with the restatement's exp composed with an FP64 product,
  element by element, within the error bound of an n-term FMA chain in FP32
  plus the final rounding to the storage dtype;
* the backward's dE = dY x^T agrees with the FP64 product within the bound of
  its summation (per-lane chains of about C/64 terms, then a 6-level tree);
  dh is bit-identical to the restatement's Frechet derivative L(h^T, dE) on the
  kernel's own dE; dx = exp(h)^T dY agrees with FP64 like y;
* gradients through autograd equal the backward kernel's, and agree with FP64
  autograd of the composed ``linalg.matrix_exp(h) @ x`` normwise;
* views of h and x (transposed, negated, expanded, strided tokens and rows,
  non-unit column stride, C not a multiple of the 16-byte vector) give the same
  bits as contiguous operands; results do not depend on the batch around a
  token; non-finite h gives NaN for that token only;
* everything the streaming kernels do not cover (n = 9, CPU, forward-mode
  tangents, function transforms) is the composed ``matrix_exp(h) @ x``
  (5 <= n <= 8 has its own kernels, tested in tests/test_hc_apply.py).
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


def _inputs(b, n, c, dtype, scale=0.7, device="cuda"):
    h = (torch.randn(b, n, n, device=device) * scale).to(dtype)
    x = torch.randn(b, n, c, device=device).to(dtype)
    return h, x


def _oracle_exp(h):
    return oracle_exp(h, THREADS)


def _oracle_frechet(a, d):
    return oracle_frechet(a, d, THREADS)


# --- forward ---------------------------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("n", [2, 3, 4])
@pytest.mark.parametrize("c", [8, 36, 2048, 5000])
def test_forward_against_restatement_and_fp64(n, c, dtype):
    h, x = _inputs(37, n, c, dtype)
    y, empty, e = OPS._hc_mix_aux(h, x, None)
    assert empty.numel() == 0 and e.dtype == torch.float32
    e_ref = _oracle_exp(h)
    assert same_bits(e.cpu(), e_ref), "exp(h) differs from the restatement"
    assert same_bits(oracle.round_to_dtype(e_ref.numpy(), dtype), fh.matrix_exp(h).cpu())
    assert same_bits(y, fh.mix_streams(h, x))
    e64, x64 = e_ref.double(), x.double().cpu()
    assert bound_violations(y, e64 @ x64, e64.abs() @ x64.abs(), n, dtype) == 0


@pytest.mark.gpu
def test_forward_mistakes_fail_the_bound():
    """The FP64 bound is tight enough to see a transposed exp(h) or a dropped term."""
    h, x = _inputs(16, 4, 256, torch.float32)
    e64, x64 = _oracle_exp(h).double(), x.double().cpu()
    scale = e64.abs() @ x64.abs()
    y = fh.mix_streams(h, x)
    assert bound_violations(y, e64 @ x64, scale, 4, torch.float32) == 0
    assert bound_violations(y, e64.mT @ x64, scale, 4, torch.float32) > 0
    dropped = e64.clone()
    dropped[:, :, 3] = 0
    assert bound_violations(y, dropped @ x64, scale, 4, torch.float32) > 0


# --- backward --------------------------------------------------------------------------------------------


def _backward_checks(h, x, g, dtype):
    n, c = x.shape[1], x.shape[2]
    dx, dh, de = OPS._hc_mix_aux(h, x, g)
    e64 = _oracle_exp(h).double()
    x64, g64 = x.double().cpu(), g.double().cpu()
    assert bound_violations(de, g64 @ x64.mT, g64.abs() @ x64.abs().mT, dE_terms(c), torch.float32) == 0
    dh_ref = oracle.round_to_dtype(_oracle_frechet(h.mT, de), dtype)
    assert same_bits(dh.cpu(), dh_ref), "dh differs from the restatement's L(h^T, dE)"
    assert bound_violations(dx, e64.mT @ g64, e64.abs().mT @ g64.abs(), n, dtype) == 0
    dh2, dx2 = OPS._hc_mix_backward(h, x, g)
    assert same_bits(dh2, dh) and same_bits(dx2, dx)
    _, _, de2 = OPS._hc_mix_aux(h, x, g)
    assert same_bits(de2, de), "dE must not change from run to run"
    return dh, dx


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("n", [2, 3, 4])
@pytest.mark.parametrize("c", [8, 36, 2048, 5000])
def test_backward_against_restatement_and_fp64(n, c, dtype):
    h, x = _inputs(37, n, c, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    _backward_checks(h, x, g, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_autograd_equals_kernels_and_fp64(dtype):
    h0, x0 = _inputs(24, 4, 512, dtype)
    g = torch.randn_like(x0, dtype=torch.float32).to(dtype)
    h, x = h0.clone().requires_grad_(), x0.clone().requires_grad_()
    y = fh.mix_streams(h, x)
    y.backward(g)
    dh, dx = OPS._hc_mix_backward(h0, x0, g)
    assert same_bits(h.grad, dh) and same_bits(x.grad, dx)
    # FP64 autograd of the composed expression, per token, normwise.
    h64 = h0.double().cpu().requires_grad_()
    x64 = x0.double().cpu().requires_grad_()
    (torch.linalg.matrix_exp(h64) @ x64).backward(g.double().cpu())
    tol = {torch.float32: 1e-5, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}[dtype]
    for got, ref in ((h.grad, h64.grad), (x.grad, x64.grad)):
        err = (got.double().cpu() - ref).flatten(1).norm(dim=1) / ref.flatten(1).norm(dim=1)
        assert err.max().item() < tol, err.max().item()


@pytest.mark.gpu
def test_graph_building_backward_and_second_order():
    h0, x0 = _inputs(6, 3, 64, torch.float32)
    g = torch.randn_like(x0)
    h, x = h0.clone().requires_grad_(), x0.clone().requires_grad_()
    dh, dx = torch.autograd.grad(fh.mix_streams(h, x), (h, x), g, create_graph=True)
    dh_k, dx_k = OPS._hc_mix_backward(h0, x0, g)
    torch.testing.assert_close(dh, dh_k, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(dx, dx_k, rtol=1e-5, atol=1e-5)
    (second,) = torch.autograd.grad((dh * dh).sum() + (dx * dx).sum(), x)
    h64, x64 = h0.double().requires_grad_(), x0.double().requires_grad_()
    dh64, dx64 = torch.autograd.grad(torch.linalg.matrix_exp(h64) @ x64, (h64, x64), g.double(), create_graph=True)
    (second64,) = torch.autograd.grad((dh64 * dh64).sum() + (dx64 * dx64).sum(), x64)
    # FP32 second derivatives cancel in places: compare normwise per token.
    err = (second.double() - second64).flatten(1).norm(dim=1) / second64.flatten(1).norm(dim=1)
    assert err.max().item() < 1e-4, err


# --- layouts, batches, edge values -----------------------------------------------------------------------


def _h_view(h, layout):
    if layout == "contiguous":
        return h
    if layout == "transposed":
        return h.mT.contiguous().mT
    if layout == "negated":
        return torch._neg_view((-h).contiguous())
    if layout == "expanded":
        return h[:1].expand_as(h)
    raise ValueError(layout)


def _x_view(x, layout):
    b, n, c = x.shape
    if layout == "contiguous":
        return x
    if layout == "wide_rows":  # rows inside wider rows: streamed in place
        wide = torch.zeros(b, n, c + 64, dtype=x.dtype, device=x.device)
        wide[..., :c] = x
        return wide[..., :c]
    if layout == "token_major":  # [n, B, C] storage: token stride C, row stride B*C
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
@pytest.mark.parametrize("hl", ["contiguous", "transposed", "negated", "expanded"])
@pytest.mark.parametrize("xl", ["contiguous", "wide_rows", "token_major", "negated", "column_strided"])
def test_layouts_give_the_same_bits(hl, xl, dtype):
    h, x = _inputs(11, 4, 96, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    hv, xv, gv = _h_view(h, hl), _x_view(x, xl), _x_view(g, xl)
    hc = hv.resolve_neg().contiguous()
    assert same_bits(fh.mix_streams(hv, xv), fh.mix_streams(hc, x))
    dh, dx = OPS._hc_mix_backward(hv, xv, gv)
    dh_c, dx_c = OPS._hc_mix_backward(hc, x, g)
    assert same_bits(dh, dh_c) and same_bits(dx, dx_c)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [4, 8])
def test_token_rows_spanning_2gib_are_copied_not_rejected(n):
    """Token-major storage [n, B, C] viewed as [B, n, C]: a token's rows lie B*C elements apart.
    With B large enough, one token's rows span more than the streaming kernels' 32-bit buffer
    offsets reach; such operands (x and the upstream gradient) are copied to contiguous rows
    first, so the results are the contiguous operands' bit for bit (n = 4: fused kernels; n = 8:
    exp then the apply kernels)."""
    dtype, c, tokens = torch.bfloat16, 4096, 16
    b_total = 2**31 // ((n - 1) * c * 2) + 1
    store_x = torch.empty(n, b_total, c, dtype=dtype, device="cuda")
    store_g = torch.empty(n, b_total, c, dtype=dtype, device="cuda")
    x = store_x.permute(1, 0, 2)[:tokens]
    g = store_g.permute(1, 0, 2)[:tokens]
    x.copy_(torch.randn(tokens, n, c, device="cuda").to(dtype))
    g.copy_(torch.randn(tokens, n, c, device="cuda").to(dtype))
    assert ((n - 1) * x.stride(1) + c) * x.element_size() >= 2**31
    h = (torch.randn(tokens, n, n, device="cuda") * 0.5).to(dtype)
    xc, gc = x.contiguous(), g.contiguous()
    y = fh.mix_streams(h, x)
    assert same_bits(y, fh.mix_streams(h, xc))
    e64, x64 = torch.linalg.matrix_exp(h.double()), x.double()
    assert bool(((y.double() - e64 @ x64).abs() <= 2.0**-7 * (e64.abs() @ x64.abs()) + 1e-30).all())
    hr, xr = h.clone().requires_grad_(), x.detach().requires_grad_()
    dh, dx = torch.autograd.grad(fh.mix_streams(hr, xr), (hr, xr), g)
    hr2, xr2 = h.clone().requires_grad_(), xc.clone().requires_grad_()
    dh_c, dx_c = torch.autograd.grad(fh.mix_streams(hr2, xr2), (hr2, xr2), gc)
    assert same_bits(dh, dh_c) and same_bits(dx, dx_c)
    del store_x, store_g, x, g


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=str)
def test_tokens_do_not_depend_on_the_batch(dtype):
    # 40,000 tokens: more token blocks than the grid holds, so the grid-stride loop is used.
    h, x = _inputs(40000, 4, 16, dtype)
    g = torch.randn_like(x, dtype=torch.float32).to(dtype)
    y = fh.mix_streams(h, x)
    dh, dx = OPS._hc_mix_backward(h, x, g)
    for lo, hi in ((0, 1), (5, 14), (39991, 40000), (17, 4113)):
        assert same_bits(fh.mix_streams(h[lo:hi], x[lo:hi]), y[lo:hi])
        dh_s, dx_s = OPS._hc_mix_backward(h[lo:hi], x[lo:hi], g[lo:hi])
        assert same_bits(dh_s, dh[lo:hi]) and same_bits(dx_s, dx[lo:hi])


@pytest.mark.gpu
def test_empty_batch():
    h, x = _inputs(0, 4, 64, torch.float32)
    assert fh.mix_streams(h, x).shape == (0, 4, 64)
    dh, dx = OPS._hc_mix_backward(h, x, x)
    assert dh.shape == (0, 4, 4) and dx.shape == (0, 4, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_nonfinite_h_poisons_only_its_token(bad):
    h, x = _inputs(20, 4, 64, torch.float32)
    g = torch.randn_like(x)
    clean_y = fh.mix_streams(h, x)
    clean_dh, clean_dx = OPS._hc_mix_backward(h, x, g)
    h[9, 1, 2] = bad
    y = fh.mix_streams(h, x)
    dh, dx = OPS._hc_mix_backward(h, x, g)
    assert torch.isnan(y[9]).all() and torch.isnan(dx[9]).all() and torch.isnan(dh[9]).all()
    keep = torch.arange(20) != 9
    assert same_bits(y[keep], clean_y[keep])
    assert same_bits(dh[keep], clean_dh[keep]) and same_bits(dx[keep], clean_dx[keep])


@pytest.mark.gpu
def test_nonfinite_x_stays_in_its_column():
    h, x = _inputs(3, 4, 64, torch.float32)
    clean = fh.mix_streams(h, x)
    x[1, 2, 7] = float("inf")
    y = fh.mix_streams(h, x)
    assert not torch.isfinite(y[1, :, 7]).any()
    other = torch.ones_like(y, dtype=torch.bool)
    other[1, :, 7] = False
    assert same_bits(y[other], clean[other])


# --- what the fusion does not cover -----------------------------------------------------------------------


@pytest.mark.gpu
def test_outside_the_fusion_is_the_composition():
    h, x = _inputs(5, 9, 40, torch.float32)
    assert same_bits(fh.mix_streams(h, x), fh.matrix_exp(h) @ x)
    h4, x4 = _inputs(5, 4, 40, torch.float32)
    # Forward-mode tangents and function transforms take the composed path.
    import torch.autograd.forward_ad as fwAD

    t = torch.randn_like(h4)
    with fwAD.dual_level():
        y = fwAD.unpack_dual(fh.mix_streams(fwAD.make_dual(h4, t), x4))
        y_ref = fwAD.unpack_dual(fh.matrix_exp(fwAD.make_dual(h4, t)) @ x4)
    assert same_bits(y.primal, y_ref.primal) and same_bits(y.tangent, y_ref.tangent)
    vm = torch.func.vmap(lambda a, b: fh.mix_streams(a[None], b[None])[0])(h4, x4)
    vm_ref = torch.func.vmap(lambda a, b: (fh.matrix_exp(a[None]) @ b[None])[0])(h4, x4)
    assert same_bits(vm, vm_ref)


@pytest.mark.gpu
@pytest.mark.compile
def test_compile_keeps_the_fused_operator():
    h, x = _inputs(16, 4, 128, torch.bfloat16)
    g = torch.randn_like(x, dtype=torch.float32).to(torch.bfloat16)

    def step(a, b):
        return fh.mix_streams(a, b)

    compiled = torch.compile(step, fullgraph=True)
    hr, xr = h.clone().requires_grad_(), x.clone().requires_grad_()
    y = compiled(hr, xr)
    y.backward(g)
    assert same_bits(y, fh.mix_streams(h, x))
    dh, dx = OPS._hc_mix_backward(h, x, g)
    assert same_bits(hr.grad, dh) and same_bits(xr.grad, dx)


def test_cpu_is_the_composition():
    h, x = _inputs(4, 4, 10, torch.float32, device="cpu")
    assert torch.equal(fh.mix_streams(h, x), torch.linalg.matrix_exp(h) @ x)
    hr = h.clone().requires_grad_()
    fh.mix_streams(hr, x).sum().backward()
    assert hr.grad is not None and torch.isfinite(hr.grad).all()


def test_operator_schemas():
    assert str(OPS._hc_mix.default._schema) == "flash_hypercons::_hc_mix(Tensor h, Tensor x) -> Tensor"
    assert (
        str(OPS._hc_mix_backward.default._schema)
        == "flash_hypercons::_hc_mix_backward(Tensor h, Tensor x, Tensor grad) -> (Tensor, Tensor)"
    )


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        h = torch.empty(8, 4, 4, device="cuda")
        x = torch.empty(8, 4, 100, device="cuda")
        assert OPS._hc_mix(h, x).shape == (8, 4, 100)
        dh, dx = OPS._hc_mix_backward(h, x, x)
        assert dh.shape == (8, 4, 4) and dx.shape == (8, 4, 100)
