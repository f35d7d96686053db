"""The C ABI launched on the GPU the way a caller of include/flash_hypercons.h binds it.

ctypes loads libflash_hypercons_hip.so directly (no torch extension in the
path), passes device pointers, element strides, the negation flag, the dtype
code and the current HIP stream.  Each launch is compared bit for bit with the
torch operator on the same logical operands (both run the same kernels), and,
for n <= 8, with the CPU restatement; squaring counts from ``fh_expm_launch``
and ``fh_expm_params`` with the restatement's; ``fh_hc_mix`` and
``fh_hc_mix_backward`` (exp(h) x and its gradients) with the mixing operators,
and their exp(h) / dE side outputs with the restatement; ``fh_hc_apply`` and
``fh_hc_apply_backward`` (5 <= n <= 8, exp(h) supplied) with the apply
operators and their dE with the restatement's dh.  Operands: contiguous,
transposed views, lazily negated storage and expanded (stride-0) batches.
"""

import ctypes
from pathlib import Path

import pytest
import torch

import flash_hypercons
import oracle

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = Path(flash_hypercons.__file__).resolve().parent / "libflash_hypercons_hip.so"
CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
I64x3 = ctypes.c_int64 * 3


def _lib():
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.fh_matrix_exp.argtypes = [vp, vp, i32, vp, i32, i64, i32, vp]
    lib.fh_frechet.argtypes = [vp, vp, i32, vp, vp, i32, vp, i32, i64, i32, vp]
    lib.fh_expm_launch.argtypes = [vp, vp, i32, vp, vp, i32, vp, i32, i64, i32, i32, vp, vp]
    lib.fh_expm_params.argtypes = [vp, vp, i32, vp, vp, i32, i32, i64, i32, vp, vp, vp]
    lib.fh_hc_mix.argtypes = [vp, vp, i32, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    lib.fh_hc_mix_backward.argtypes = [vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    lib.fh_hc_apply.argtypes = [vp, vp, vp, vp, i32, i64, i32, i64, vp]
    lib.fh_hc_apply_backward.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    for f in (lib.fh_matrix_exp, lib.fh_frechet, lib.fh_expm_launch, lib.fh_expm_params, lib.fh_hc_mix,
              lib.fh_hc_mix_backward, lib.fh_hc_apply, lib.fh_hc_apply_backward):
        f.restype = ctypes.c_int
    lib.fh_last_error.restype = ctypes.c_char_p
    return lib


LIB = None


def lib():
    global LIB
    if LIB is None:
        LIB = _lib()
    return LIB


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Operand:
    """A logical [B, n, n] operand and how the C ABI receives it: storage pointer, strides,
    negation flag."""

    def __init__(self, values, layout):
        self.layout = layout
        if layout == "contiguous":
            self.storage = values.contiguous()
            self.logical, self.neg = self.storage, 0
        elif layout == "transposed":
            self.storage = values.mT.contiguous()  # logical values read through swapped strides
            self.logical, self.neg = self.storage.mT, 0
        elif layout == "negated":
            self.storage = (-values).contiguous()  # the flag negates exactly
            self.logical, self.neg = torch._neg_view(self.storage), 1
        elif layout == "expanded":
            self.storage = values[:1].contiguous()
            self.logical, self.neg = self.storage.expand_as(values), 0
        else:
            raise ValueError(layout)
        self.strides = I64x3(*self.logical.stride())

    @property
    def ptr(self):
        return self.storage.data_ptr()


def c_matrix_exp(x: Operand, dtype, batch, n):
    out = torch.empty(batch, n, n, dtype=dtype, device="cuda")
    rc = lib().fh_matrix_exp(x.ptr, x.strides, x.neg, out.data_ptr(), CODES[dtype], batch, n, _stream())
    assert rc == 0, lib().fh_last_error()
    return out


def c_frechet(x: Operand, g: Operand, dtype, batch, n):
    out = torch.empty(batch, n, n, dtype=dtype, device="cuda")
    rc = lib().fh_frechet(x.ptr, x.strides, x.neg, g.ptr, g.strides, g.neg, out.data_ptr(), CODES[dtype], batch, n,
                          _stream())
    assert rc == 0, lib().fh_last_error()
    return out


def _values(batch, n, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    base = torch.randn(batch, n, n, generator=gen, dtype=torch.float64)
    base = base / torch.linalg.matrix_norm(base, ord=1)[:, None, None]
    scale = 10 ** torch.empty(batch, dtype=torch.float64).uniform_(-2.0, 1.0, generator=gen)
    x = (base * scale[:, None, None]).to(dtype).cuda()
    g = torch.randn(batch, n, n, generator=gen).to(dtype).cuda()
    return x, g


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [3, 4, 8, 16, 32])
@pytest.mark.parametrize("layout", ["contiguous", "transposed", "negated", "expanded"])
def test_entry_points_match_operator_and_oracle(layout, n, dtype):
    import flash_hypercons  # noqa: F401

    batch = 131 if n <= 8 else 37
    xv, gv = _values(batch, n, dtype, seed=17 * n + CODES[dtype])
    x = Operand(xv, layout)
    g = Operand(gv, "transposed" if layout == "contiguous" else "contiguous")
    y = c_matrix_exp(x, dtype, batch, n)
    d = c_frechet(x, g, dtype, batch, n)
    torch.cuda.synchronize()
    assert torch.equal(y, torch.ops.flash_hypercons._matrix_exp(x.logical))
    assert torch.equal(d, torch.ops.flash_hypercons._frechet(x.logical, g.logical))
    if n <= 8:
        exp_y, _ = oracle.torch_matrix_exp(x.logical.cpu())
        exp_d, _ = oracle.torch_frechet(x.logical.cpu(), g.logical.cpu())
        for got, want in ((y, exp_y), (d, exp_d)):
            a, e = got.cpu().double(), want.double()
            assert bool(((a == e) | (a.isnan() & e.isnan())).all())


@pytest.mark.parametrize("n", [2, 4, 7, 12, 32])
def test_launch_and_params_report_oracle_squarings(n):
    batch = 200
    xv, gv = _values(batch, n, torch.float32, seed=5 * n)
    xv[3, 0, 0] = float("nan")  # non-finite rule: s = -1, NaN output
    x, g = Operand(xv, "transposed"), Operand(gv, "contiguous")
    out = torch.empty(batch, n, n, device="cuda")
    s = torch.empty(batch, dtype=torch.int32, device="cuda")
    for direction in (None, g):
        dptr = None if direction is None else direction.ptr
        dstr = None if direction is None else direction.strides
        dneg = 0 if direction is None else direction.neg
        rc = lib().fh_expm_launch(x.ptr, x.strides, x.neg, dptr, dstr, dneg, out.data_ptr(), 0, batch, n, 0,
                                  s.data_ptr(), _stream())
        assert rc == 0, lib().fh_last_error()
        params = torch.empty(batch, 2, dtype=torch.int32, device="cuda")
        norms = torch.empty(batch, dtype=torch.float64, device="cuda")
        rc = lib().fh_expm_params(x.ptr, x.strides, x.neg, dptr, dstr, dneg, 0, batch, n, params.data_ptr(),
                                  norms.data_ptr(), _stream())
        assert rc == 0, lib().fh_last_error()
        torch.cuda.synchronize()
        exp_s, exp_norm = oracle.torch_params(x.logical.cpu(), None if direction is None else direction.logical.cpu())
        assert torch.equal(s.cpu(), exp_s)
        assert torch.equal(params[:, 1].cpu(), exp_s)
        assert params[:, 0].cpu().tolist() == [18 if v >= 0 else -1 for v in exp_s.tolist()]
        got_norm = norms.cpu()
        assert torch.equal(got_norm.isnan(), exp_norm.isnan())
        assert torch.equal(got_norm[~got_norm.isnan()], exp_norm[~exp_norm.isnan()])
        assert bool(out[3].isnan().all())


def test_errors_do_not_launch():
    x = torch.zeros(2, 4, 4, dtype=torch.float64, device="cuda")
    out = torch.empty_like(x)
    strides = I64x3(*x.stride())
    # float64 has no dtype code: any unknown code is rejected with the reference's message
    rc = lib().fh_matrix_exp(x.data_ptr(), strides, 0, out.data_ptr(), 3, 2, 4, _stream())
    assert rc == 1 and b"2 <= N <= 32" in lib().fh_last_error()
    rc = lib().fh_frechet(x.data_ptr(), strides, 0, None, strides, 0, out.data_ptr(), 0, 2, 4, _stream())
    assert rc == 1 and b"direction must match" in lib().fh_last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["contiguous", "transposed", "negated", "expanded"])
def test_hc_mix_entry_points(layout, dtype):
    import flash_hypercons  # noqa: F401

    batch, n, cols = 29, 4, 264
    hv, _ = _values(batch, n, dtype, seed=3 + CODES[dtype])
    h = Operand(hv, layout)
    x = torch.randn(batch, n, cols, device="cuda").to(dtype)
    gy = torch.randn(batch, n, cols, device="cuda").to(dtype)
    xs, gs = I64x3(*x.stride()), I64x3(*gy.stride())
    y = torch.empty_like(x)
    e = torch.empty(batch, n, n, device="cuda")
    rc = lib().fh_hc_mix(h.ptr, h.strides, h.neg, x.data_ptr(), xs, y.data_ptr(), e.data_ptr(), CODES[dtype], batch,
                         n, cols, _stream())
    assert rc == 0, lib().fh_last_error()
    dh = torch.empty(batch, n, n, dtype=dtype, device="cuda")
    dx = torch.empty_like(x)
    de = torch.empty(batch, n, n, device="cuda")
    rc = lib().fh_hc_mix_backward(h.ptr, h.strides, h.neg, x.data_ptr(), xs, gy.data_ptr(), gs, dh.data_ptr(),
                                  dx.data_ptr(), de.data_ptr(), CODES[dtype], batch, n, cols, _stream())
    assert rc == 0, lib().fh_last_error()
    torch.cuda.synchronize()
    ops = torch.ops.flash_hypercons
    assert torch.equal(y, ops._hc_mix(h.logical, x))
    dh_op, dx_op = ops._hc_mix_backward(h.logical, x, gy)
    assert torch.equal(dh, dh_op) and torch.equal(dx, dx_op)
    exp_e, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(h.logical))
    assert torch.equal(e.cpu(), torch.from_numpy(exp_e))
    exp_dh, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(h.logical.mT), de.cpu().numpy())
    assert torch.equal(dh.cpu(), oracle.round_to_dtype(exp_dh, dtype))


def test_hc_mix_rejects_unstreamable_rows():
    x = torch.zeros(2, 4, 10, device="cuda")  # 10 columns: not whole 16-byte vectors
    h = torch.zeros(2, 4, 4, device="cuda")
    out = torch.empty_like(x)
    hs, xs = I64x3(*h.stride()), I64x3(*x.stride())
    rc = lib().fh_hc_mix(h.data_ptr(), hs, 0, x.data_ptr(), xs, out.data_ptr(), None, 0, 2, 4, 10, _stream())
    assert rc == 1 and b"multiples of 4 elements" in lib().fh_last_error()
    x8 = torch.zeros(2, 4, 8, device="cuda")
    x8s = I64x3(*x8.stride())
    rc = lib().fh_hc_mix_backward(h.data_ptr(), hs, 0, x8.data_ptr(), x8s, None, x8s, h.data_ptr(), x8.data_ptr(),
                                  None, 0, 2, 4, 8, _stream())
    assert rc == 1 and b"null grad" in lib().fh_last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [5, 8])
def test_hc_apply_entry_points(n, dtype):
    import flash_hypercons  # noqa: F401

    batch, cols = 21, 136
    hv, _ = _values(batch, n, dtype, seed=41 + n + CODES[dtype])
    ops = torch.ops.flash_hypercons
    e = ops._matrix_exp(hv.float())
    # x and dY as row views inside wider rows (token-major storage), streamed in place.
    x = torch.randn(n, batch, cols + 24, device="cuda").to(dtype).transpose(0, 1)[..., :cols]
    gy = torch.randn(batch, n, cols, device="cuda").to(dtype)
    xs, gs = I64x3(*x.stride()), I64x3(*gy.stride())
    y = torch.empty(batch, n, cols, dtype=dtype, device="cuda")
    rc = lib().fh_hc_apply(e.data_ptr(), x.data_ptr(), xs, y.data_ptr(), CODES[dtype], batch, n, cols, _stream())
    assert rc == 0, lib().fh_last_error()
    dx = torch.empty_like(y)
    de = torch.empty(batch, n, n, device="cuda")
    rc = lib().fh_hc_apply_backward(e.data_ptr(), x.data_ptr(), xs, gy.data_ptr(), gs, dx.data_ptr(), de.data_ptr(),
                                    CODES[dtype], batch, n, cols, _stream())
    assert rc == 0, lib().fh_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y, ops._hc_apply(e, x))
    dx_op, de_op = ops._hc_apply_backward(e, x, gy)
    assert torch.equal(dx, dx_op) and torch.equal(de, de_op)
    exp_e, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(hv))
    assert torch.equal(e.cpu(), torch.from_numpy(exp_e))
    # The public op's dh is the restatement's L(h^T, dE) on this dE, rounded to the dtype.
    hr = hv.clone().requires_grad_()
    flash_hypercons.mix_streams(hr, x).backward(gy)
    exp_dh, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(hv.mT), de.cpu().numpy())
    assert torch.equal(hr.grad.cpu(), oracle.round_to_dtype(exp_dh, dtype))
