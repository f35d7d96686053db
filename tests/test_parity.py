"""HIP kernels against the CPU oracle (oracle/fh_oracle.c) and FP64 torch.

* The squaring count s and the degree (always 18) must be bit-identical to the
  oracle for every matrix, in both directions, for every size class and dtype.
* The generic kernel (FH_VARIANT_GENERIC) evaluates in the reference's exact
  order and must match the oracle bit for bit.
* The tuned P == 4 kernel (one matrix per lane, plain FP32 FMAs) and the P == 8
  kernel (2 x 2 blocks of exact 4x4x1 MFMA steps) keep the reference's
  evaluation order and must also match the oracle bit for bit.
* Every kernel must meet the FP32 / FP16 / BF16 tolerances against FP64.
Inputs are seeded; GPU results are compared through the C ABI that the
``flash_hypercons::_expm_debug`` / ``_expm_params`` operators wrap.
"""

import pytest
import torch

import oracle
from tests.reference import check_north_star, reference

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SIZES = [2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 31, 32]
GENERIC, AUTO = 1, 0


def scaled_inputs(batch, n, dtype, seed, low=-3.0, high=1.0):
    """Gaussian matrices with unit 1-norm times 10^U(low, high): s spans 0..~5."""
    gen = torch.Generator().manual_seed(seed)
    base = torch.randn(batch, n, n, generator=gen, dtype=torch.float64)
    base = base / torch.linalg.matrix_norm(base, ord=1)[:, None, None]
    scale = 10 ** torch.empty(batch, dtype=torch.float64).uniform_(low, high, generator=gen)
    a = (base * scale[:, None, None]).to(dtype)
    g = torch.randn(batch, n, n, generator=gen).to(dtype)
    return a, g


def run_kernel(x, g, variant):
    import flash_hypercons  # noqa: F401

    return torch.ops.flash_hypercons._expm_debug(x, g, variant)


def oracle_result(x, g):
    if g is None:
        return oracle.torch_matrix_exp(x.cpu())
    return oracle.torch_frechet(x.cpu(), g.cpu())


def same_values(actual, expected):
    """Bitwise equality up to the sign of zero, with NaN matching NaN."""
    a = actual.cpu().double()
    e = expected.double()
    both_nan = a.isnan() & e.isnan()
    equal = (a == e) | both_nan
    return bool(equal.all()), int((~equal).sum())


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", SIZES)
def test_generic_bitwise_and_squarings(n, dtype, backward):
    a, g = scaled_inputs(67, n, dtype, seed=1000 * n + 7 * backward + DTYPES.index(dtype))
    a, g = a.cuda(), g.cuda()
    x = a.mT if backward else a
    direction = g if backward else None
    out, s = run_kernel(x, direction, GENERIC)
    exp_out, exp_s = oracle_result(x, direction)
    assert torch.equal(s.cpu(), exp_s)
    ok, bad = same_values(out, exp_out)
    assert ok, f"{bad} elements differ from the oracle"


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", SIZES)
def test_tuned_squarings_and_tolerance(n, dtype, backward):
    a, g = scaled_inputs(259, n, dtype, seed=2000 * n + 7 * backward + DTYPES.index(dtype))
    a, g = a.cuda(), g.cuda()
    x = a.mT if backward else a
    direction = g if backward else None
    out, s = run_kernel(x, direction, AUTO)
    _, exp_s = oracle_result(x, direction)
    assert torch.equal(s.cpu(), exp_s), "squaring counts differ from the oracle"
    params, norms = torch.ops.flash_hypercons._expm_params(x, direction)
    exp_s2, exp_norm = oracle.torch_params(x.cpu(), None if direction is None else direction.cpu())
    assert torch.equal(params[:, 1].cpu(), exp_s2)
    assert bool((params[:, 0] == 18).all())
    assert torch.equal(norms.cpu(), exp_norm)
    check_north_star(out, reference(x, direction), backward=backward)


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 3, 4, 5, 6, 7, 8])
def test_small_kernels_bitwise(n, dtype, backward):
    """The P = 4 (one matrix per lane) and P = 8 (4x4x1 MFMA blocks) kernels keep the
    reference's evaluation order and match the oracle bit for bit."""
    a, g = scaled_inputs(1000, n, dtype, seed=3000 * n + 7 * backward + DTYPES.index(dtype))
    a, g = a.cuda(), g.cuda()
    x = a.mT if backward else a
    direction = g if backward else None
    out, s = run_kernel(x, direction, AUTO)
    exp_out, exp_s = oracle_result(x, direction)
    assert torch.equal(s.cpu(), exp_s)
    ok, bad = same_values(out, exp_out)
    assert ok, f"{bad} elements differ from the oracle"


def _laid_out(m, layout):
    """The same logical [B, n, n] values stored row-major ("rows": every row one aligned
    vector), column-major ("cols": a transposed view) or with a padded row stride that no
    vector class accepts ("none")."""
    if layout == "rows":
        return m.contiguous()
    if layout == "cols":
        return m.mT.contiguous().mT
    b, n, _ = m.shape
    padded = torch.zeros(b, n, n + 1, dtype=m.dtype, device=m.device)
    padded[:, :, :n] = m
    return padded[:, :, :n]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [4, 8])
def test_small_kernels_bitwise_all_layouts(n, dtype):
    """Every load path of the P = 4 and P = 8 kernels (row vectors, column vectors,
    element-wise; X and G classified independently, dense or not) gives the oracle's
    values bit for bit, forward and Frechet, over a batch with a partial last group."""
    a, g = scaled_inputs(300, n, dtype, seed=577 * n + DTYPES.index(dtype))
    a, g = a.cuda(), g.cuda()
    for xl in ("rows", "cols", "none"):
        x = _laid_out(a, xl)
        out, s = run_kernel(x, None, AUTO)
        exp_out, exp_s = oracle_result(x, None)
        assert torch.equal(s.cpu(), exp_s), xl
        ok, bad = same_values(out, exp_out)
        assert ok, f"forward, x {xl}: {bad} elements differ from the oracle"
        for gl in ("rows", "cols", "none"):
            d = _laid_out(g, gl)
            out, s = run_kernel(x, d, AUTO)
            exp_out, exp_s = oracle_result(x, d)
            assert torch.equal(s.cpu(), exp_s), (xl, gl)
            ok, bad = same_values(out, exp_out)
            assert ok, f"Frechet, x {xl}, g {gl}: {bad} elements differ from the oracle"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [3, 4])
def test_p4_frechet_large_batch_bitwise(n, dtype):
    """The persistent P = 4 Frechet kernel over half a million matrices: several groups
    per wavefront (prefetch of the next group, staged stores, a partial last group) with
    squaring counts spread over 0..7 inside every wavefront.  Each matrix must match the
    oracle bit for bit."""
    batch = (1 << 19) + 37
    a, g = scaled_inputs(batch, n, dtype, seed=91 * n + DTYPES.index(dtype), low=-3.0, high=2.0)
    x = a.cuda().mT
    out, s = run_kernel(x, g.cuda(), AUTO)
    exp_out, exp_s = oracle_result(x, g)
    assert torch.equal(s.cpu(), exp_s)
    assert int(exp_s.max()) >= 6 and int((exp_s == 0).sum()) > 0
    ok, bad = same_values(out, exp_out)
    assert ok, f"{bad} elements differ from the oracle"


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_nonfinite_rule_matches_oracle(n):
    a = torch.zeros(5, n, n, device="cuda")
    a[0, 0, 0] = float("nan")
    a[1, n - 1, 0] = float("inf")
    a[2, 0, n - 1] = -float("inf")
    a[3] = torch.randn(n, n) * 0.1
    g = torch.randn(5, n, n, device="cuda")
    g[4, 1, 1] = float("nan")
    for direction in (None, g):
        for variant in (GENERIC, AUTO):
            out, s = run_kernel(a, direction, variant)
            exp_out, exp_s = oracle_result(a, direction)
            assert torch.equal(s.cpu(), exp_s)
            ok, bad = same_values(out, exp_out) if variant == GENERIC else (True, 0)
            assert ok, f"{bad} elements differ"
            assert torch.equal(out.isnan().cpu(), exp_out.isnan())


def test_config1_golden_fixture_on_gpu():
    """BASELINE config 1 inputs on the GPU path against the committed FP64 fixture."""
    from pathlib import Path

    import numpy as np

    import flash_hypercons as fh
    from tests.reference import rel_frobenius

    d = np.load(Path(__file__).resolve().parent / "golden" / "c1_cpu_plumbing.npz")
    x = torch.from_numpy(d["x"]).cuda().requires_grad_()
    y = fh.matrix_exp(x)
    (grad,) = torch.autograd.grad(y.sum(), x)
    assert rel_frobenius(y.detach().cpu(), torch.from_numpy(d["y"])).max() <= 1e-5
    assert rel_frobenius(grad.cpu(), torch.from_numpy(d["grad"])).max() <= 1e-4
    exp_out, _ = oracle.torch_matrix_exp(x.detach().cpu())
    ok, bad = same_values(y.detach(), exp_out)
    assert ok, f"{bad} elements differ from the oracle"


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_squaring_boundary_fixture_on_gpu(n):
    from pathlib import Path

    import numpy as np

    d = np.load(Path(__file__).resolve().parent / "golden" / "s_boundaries.npz")
    x = torch.from_numpy(d[f"x{n}"]).cuda()
    params, _ = torch.ops.flash_hypercons._expm_params(x)
    assert params[:, 1].cpu().tolist() == d[f"s{n}"].tolist()
    _, s = run_kernel(x, None, AUTO)
    assert s.cpu().tolist() == d[f"s{n}"].tolist()


def _baseline_inputs(name):
    """BASELINE configs 2-5 at their full shapes (bench.py's seeded generators)."""
    import bench

    x, g, _ = bench.make_inputs(name, torch, "cuda")
    return x, g


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "c5f32"])
def test_full_size_configs_sampled(name):
    """Size-independent properties at BASELINE sizes: a matrix's result does not depend on
    the batch around it (bit for bit, forward and Frechet), its squaring count matches the
    oracle's, and the sampled results meet the north-star tolerances against FP64."""
    x, g = _baseline_inputs(name)
    b = x.shape[0]
    xt = x.mT
    y, s_fwd = run_kernel(x, None, AUTO)
    d, s_bwd = run_kernel(xt, g, AUTO)
    gen = torch.Generator().manual_seed(7)
    idx = torch.cat((torch.randint(0, b, (192,), generator=gen), torch.arange(b - 64, b))).unique()
    idx_dev = idx.to(x.device)
    xs, gs, xts = x[idx_dev], g[idx_dev], xt[idx_dev]
    y_small, _ = run_kernel(xs, None, AUTO)
    d_small, _ = run_kernel(xts, gs, AUTO)
    assert torch.equal(y[idx_dev], y_small)
    assert torch.equal(d[idx_dev], d_small)
    o_fwd, s_ref = oracle_result(xs, None)
    o_bwd, s_ref_b = oracle_result(xts, gs)
    assert torch.equal(s_fwd[idx_dev].cpu().to(s_ref.dtype), s_ref)
    assert torch.equal(s_bwd[idx_dev].cpu().to(s_ref_b.dtype), s_ref_b)
    finite = s_ref >= 0
    finite_b = s_ref_b >= 0
    f, fb = finite.to(x.device), finite_b.to(x.device)
    check_north_star(y_small[f], reference(xs[f]), squarings=s_ref[finite])
    check_north_star(d_small[fb], reference(xts[fb], gs[fb]), backward=True, squarings=s_ref_b[finite_b])
    # The tile kernels' FP32 error matches the reference arithmetic's: compare means.
    if x.dtype == torch.float32:
        for out, ora, ref in ((y_small[f], o_fwd[finite], reference(xs[f])),
                              (d_small[fb], o_bwd[finite_b], reference(xts[fb], gs[fb]))):
            from tests.reference import rel_frobenius

            ratio = rel_frobenius(out, ref).mean() / rel_frobenius(ora.to(out.device), ref).mean()
            assert ratio <= 1.25, f"mean FP32 error {ratio:.2f}x the reference arithmetic's"
