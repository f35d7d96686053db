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


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch", [128, 7 * 64, 6 * 64 + 5, 64 * 64 + 63])
def test_p4_count_ordered_batches_bitwise(batch, dtype, backward):
    """Dense n = 4 batches: FP16/BF16 run in pairs of groups ordered by squaring count, FP32
    one group at a time through the buffer-to-LDS ring.  Whole pairs, an odd last group, a
    partial group, and inside the full groups non-finite matrices (s = -1, NaN rows), counts
    above 127 (entries near the dtype's maximum) and counts from 0 to ~7.  Every matrix must
    match the oracle bit for bit and report the oracle's count."""
    a, g = scaled_inputs(batch, 4, dtype, seed=batch + 13 * backward + DTYPES.index(dtype), low=-4.0, high=2.0)
    a[5, 1, 2] = float("nan")
    a[70, 3, 3] = float("inf")
    a[100, 0, 0] = -float("inf")
    big = 6.0e4 if dtype == torch.float16 else 3.0e38
    a[9] = torch.full((4, 4), big).to(dtype)
    a[33, :, 1] = -big
    g[11, 2, 0] = float("nan")
    x = a.cuda().mT if backward else a.cuda()
    direction = g.cuda() if backward else None
    out, s = run_kernel(x, direction, AUTO)
    exp_out, exp_s = oracle_result(x, direction)
    assert torch.equal(s.cpu(), exp_s)
    if dtype != torch.float16:
        assert int(exp_s.max()) > 127
    assert int((exp_s < 0).sum()) >= 3
    ok, bad = same_values(out, exp_out)
    assert ok, f"{bad} elements differ from the oracle"
    if dtype == torch.bfloat16:  # NaN results are stored as the reference's 0x7FC0 (c10 rounding)
        nan = out.isnan()
        assert int(nan.sum()) > 0
        assert bool((out.view(torch.int16)[nan] == 0x7FC0).all())


@pytest.mark.parametrize("layout", ["rows", "cols"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch", [32, 3 * 32, 5 * 32 + 17, 4096 + 21])
def test_p8_count_ordered_batches_bitwise(batch, dtype, layout):
    """Dense n = 8 forward batches run in pairs of 16-matrix units ordered by squaring count,
    with the count taken from the row layout for row-major operands.  Cases: whole pairs, a
    partial last pair (one full and one partial unit), both dense layouts, and inside the full
    pairs non-finite matrices (s = -1), counts above 127 (entries near the dtype's maximum),
    counts from 0 to ~7, and the squaring-boundary fixture's matrices, whose counts only the
    exact FP64 norm decides.  Every matrix must match the oracle bit for bit and report the
    oracle's count."""
    from pathlib import Path

    import numpy as np

    fixture = np.load(Path(__file__).resolve().parent / "golden" / "s_boundaries.npz")
    a, _ = scaled_inputs(batch, 8, torch.float32, seed=batch + 31 * DTYPES.index(dtype), low=-4.0, high=2.0)
    at = torch.arange(fixture["x8"].shape[0]) * 3 + 1
    a[at] = torch.from_numpy(fixture["x8"])
    a[2, 1, 6] = float("nan")
    a[6, 7, 7] = float("inf")
    a[batch - 40 if batch > 64 else 12, 0, 3] = -float("inf")
    big = {torch.float32: 3.0e38, torch.bfloat16: 3.0e38, torch.float16: 6.0e4}[dtype]
    a[9] = torch.full((8, 8), big)
    a[17, :, 5] = -big
    x = _laid_out(a.to(dtype).cuda(), layout)
    out, s = run_kernel(x, None, AUTO)
    exp_out, exp_s = oracle_result(x, None)
    assert torch.equal(s.cpu(), exp_s)
    if dtype == torch.float32:  # the boundary matrices keep their counts only in FP32
        assert exp_s[at].tolist() == fixture["s8"].tolist()
    if dtype != torch.float16:
        assert int(exp_s.max()) > 127
    assert int((exp_s < 0).sum()) >= 3
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


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_full_size_results_do_not_depend_on_the_batch(name):
    """A size-independent property at BASELINE sizes: a matrix's result is the same bits whether
    it is computed inside the full batch or alone in a small one (forward and Frechet), for a
    sample that includes the partial last group.  (Every matrix against the oracle:
    tests/test_full_parity.py.)"""
    x, g = _baseline_inputs(name)
    b = x.shape[0]
    xt = x.mT
    y, _ = run_kernel(x, None, AUTO)
    d, _ = run_kernel(xt, g, AUTO)
    gen = torch.Generator().manual_seed(7)
    idx = torch.cat((torch.randint(0, b, (192,), generator=gen), torch.arange(b - 64, b))).unique()
    idx_dev = idx.to(x.device)
    y_small, _ = run_kernel(x[idx_dev], None, AUTO)
    d_small, _ = run_kernel(xt[idx_dev], g[idx_dev], AUTO)
    assert torch.equal(y[idx_dev], y_small)
    assert torch.equal(d[idx_dev], d_small)


@pytest.mark.parametrize("n", [4, 8])
def test_subnormal_intermediates_bitwise(n):
    """Strictly upper-triangular matrices with 1e-20 on the superdiagonal: A^2 and the (0, 2)
    entry of exp(A) are FP32 subnormals (1e-40).  The P = 4 kernel (VALU FMAs) and the P = 8
    kernel (4x4x1 MFMA steps) must keep them exactly as the oracle's fmaf chain does, forward
    and Frechet; a flush to zero anywhere would change these bits."""
    a = torch.zeros(3, n, n)
    for i in range(n - 1):
        a[:, i, i + 1] = 1e-20
    a[1] *= -1.0
    a[2, 0, n - 1] = 3e-21
    g = torch.zeros(3, n, n)
    for i in range(n - 1):
        g[:, i, i + 1] = 2e-20
    g[2] += torch.eye(n) * 1e-19
    a, g = a.cuda(), g.cuda()
    for x, direction in ((a, None), (a.mT, g), (a, g)):
        out, s = run_kernel(x, direction, AUTO)
        exp_out, exp_s = oracle_result(x, direction)
        assert torch.equal(s.cpu(), exp_s)
        ok, bad = same_values(out, exp_out)
        assert ok, f"{bad} elements differ from the oracle"
    # The case exercises what it claims: the oracle's result has subnormal entries.
    exp_out, _ = oracle_result(a, None)
    tiny = exp_out[exp_out != 0].abs()
    assert bool((tiny < torch.finfo(torch.float32).tiny).any())
