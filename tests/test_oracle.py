"""Pins the CPU oracle (oracle/fh_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible slip in the restatement -- a wrong
coefficient or sign, a transposed operand, a dropped term, a row sum in place
of a column sum, the wrong summation association, >= for > -- fails at least
one of them:

* golden fixtures (tests/golden/): BASELINE config 1 against FP64 PyTorch, and
  the reference's squaring-boundary matrices against exact rational counts;
* FP64 ``torch.linalg.matrix_exp`` (the reference tests' oracle,
  tests/reference.py:4-11 there) over every size class, dtype and scale;
* closed forms: zero, rotations (cos/sin), diagonal (elementwise exp),
  nilpotent (finite series), L(A, I) = e^A, L(A, A) = A e^A, L(0, G) = G;
* structure: exp(A^T) = exp(A)^T; L(X, G) equals the U block of the oracle's
  own forward on [[X, G], [0, X]];
* the squaring count against brute-force rational arithmetic, and the
  per-size summation association on inputs where it changes the FP64 sum;
* output rounding against torch's own conversions.
"""

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.reference import rel_frobenius

GOLDEN = Path(__file__).resolve().parent / "golden"
THETA = oracle.THETA18


def fp64_exp(a):
    return torch.linalg.matrix_exp(a.double())


def fp64_frechet(x, g):
    x, g = x.double(), g.double()
    n = x.shape[-1]
    block = torch.cat((torch.cat((x, g), -1), torch.cat((torch.zeros_like(x), x), -1)), -2)
    return torch.linalg.matrix_exp(block)[..., :n, n:]


def ora_exp(x):
    out, s, _ = oracle.matrix_exp_f32(x.float().contiguous().numpy())
    return torch.from_numpy(out), torch.from_numpy(s)


def ora_frechet(x, g):
    out, s, _ = oracle.matrix_exp_f32(x.float().contiguous().numpy(), g.float().contiguous().numpy())
    return torch.from_numpy(out), torch.from_numpy(s)


def scaled(batch, n, seed, low, high):
    gen = torch.Generator().manual_seed(seed)
    base = torch.randn(batch, n, n, generator=gen, dtype=torch.float64)
    base = base / torch.linalg.matrix_norm(base, ord=1)[:, None, None]
    scale = 10 ** torch.empty(batch, dtype=torch.float64).uniform_(low, high, generator=gen)
    return (base * scale[:, None, None]).float(), torch.randn(batch, n, n, generator=gen)


# ---- golden fixtures -------------------------------------------------------

def test_config1_fixture():
    d = np.load(GOLDEN / "c1_cpu_plumbing.npz")
    x = torch.from_numpy(d["x"])
    y, _ = ora_exp(x)
    assert rel_frobenius(y, torch.from_numpy(d["y"])).max() <= 1e-5
    g, _ = ora_frechet(x.mT, torch.ones_like(x))
    assert rel_frobenius(g, torch.from_numpy(d["grad"])).max() <= 1e-4


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_squaring_boundary_fixture(n):
    d = np.load(GOLDEN / "s_boundaries.npz")
    s, _ = oracle.params_f32(d[f"x{n}"])
    assert s.tolist() == d[f"s{n}"].tolist() == [0, 0, 0, 1, 1, 2, 3, 4]


# ---- FP64 reference --------------------------------------------------------

@pytest.mark.parametrize("n", [2, 3, 4, 5, 7, 8, 9, 13, 16, 17, 25, 32])
def test_forward_and_frechet_against_fp64(n):
    x, g = scaled(40, n, seed=n, low=-3, high=1.2)
    y, s = ora_exp(x)
    assert rel_frobenius(y, fp64_exp(x)).max() <= 1e-5
    assert s.max() >= 1  # the sample exercises squaring
    l, _ = ora_frechet(x.mT, g)
    assert rel_frobenius(l, fp64_frechet(x.mT, g)).max() <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_rounding_is_faithful(dtype):
    x, g = scaled(64, 8, seed=11, low=-2, high=0.8)
    x = x.to(dtype)
    y, _ = oracle.torch_matrix_exp(x)
    assert y.dtype == dtype
    from tests.reference import check_north_star

    check_north_star(y, fp64_exp(x.float()))
    l, _ = oracle.torch_frechet(x.mT, g.to(dtype))
    check_north_star(l, fp64_frechet(x.float().mT, g.to(dtype).float()), backward=True)


# ---- closed forms ----------------------------------------------------------

@pytest.mark.parametrize("n", [2, 4, 8, 16, 32])
def test_zero_matrix(n):
    z = torch.zeros(3, n, n)
    y, s = ora_exp(z)
    assert torch.equal(y, torch.eye(n).expand(3, n, n))
    assert s.tolist() == [0, 0, 0]
    g = torch.randn(3, n, n)
    l, _ = ora_frechet(z, g)
    # L(0, G) = G; the polynomial's linear coefficient is 1 only to FP32 rounding
    assert rel_frobenius(l, g.double()).max() <= 1e-6


@pytest.mark.parametrize("angle", [0.3, 25.0, 100.0, 1000.0])
@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_rotation_closed_form(n, angle):
    a = torch.zeros(1, n, n)
    a[0, 0, 1], a[0, 1, 0] = -angle, angle
    y, _ = ora_exp(a)
    expected = torch.eye(n, dtype=torch.float64)
    expected[0, 0] = expected[1, 1] = math.cos(angle)
    expected[0, 1], expected[1, 0] = -math.sin(angle), math.sin(angle)
    assert (y[0].double() - expected).abs().max() <= 2e-3  # reference tolerance, s up to 9
    # gradient of <G, exp(A)> with G = 0.125 I is 0.125 exp(A)^T
    l, _ = ora_frechet(a.mT, 0.125 * torch.eye(n).expand(1, n, n))
    assert (l[0].double() - 0.125 * expected.T).abs().max() <= 2e-3


@pytest.mark.parametrize("n", [3, 4, 8, 16, 32])
def test_diagonal_is_elementwise_exp(n):
    d = torch.linspace(-3.0, 2.0, n)
    y, _ = ora_exp(torch.diag(d)[None])
    expected = torch.diag(d.double().exp())
    assert ((y[0].double() - expected).abs() / expected.abs().max()).max() <= 2e-6


@pytest.mark.parametrize("n", [4, 8])
def test_nilpotent_finite_series(n):
    gen = torch.Generator().manual_seed(n)
    a = torch.triu(torch.randn(n, n, generator=gen, dtype=torch.float64), diagonal=1) * 0.5
    series = torch.eye(n, dtype=torch.float64)
    term = torch.eye(n, dtype=torch.float64)
    for k in range(1, n):
        term = term @ a / k
        series = series + term
    y, _ = ora_exp(a.float()[None])
    assert rel_frobenius(y[0], series) <= 1e-5


@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_frechet_identities(n):
    x, _ = scaled(6, n, seed=100 + n, low=-1, high=1)
    eye = torch.eye(n).expand(6, n, n).contiguous()
    y, _ = ora_exp(x)
    l_i, _ = ora_frechet(x, eye)  # L(A, I) = e^A
    assert rel_frobenius(l_i, y.double()).max() <= 1e-5
    l_a, _ = ora_frechet(x, x)  # L(A, A) = A e^A
    assert rel_frobenius(l_a, x.double() @ fp64_exp(x)).max() <= 1e-4


# ---- structure ---------------------------------------------------------------

@pytest.mark.parametrize("n", [4, 8, 16, 32])
def test_transpose_symmetry(n):
    x, _ = scaled(20, n, seed=200 + n, low=-2, high=1)
    y, s = ora_exp(x)
    yt, st = ora_exp(x.mT.contiguous())
    assert rel_frobenius(yt, y.mT.double()).max() <= 1e-5


@pytest.mark.parametrize("n", [2, 4, 8, 16])
def test_frechet_is_block_of_augmented_forward(n):
    x, g = scaled(10, n, seed=300 + n, low=-2, high=0.5)
    l, _ = ora_frechet(x, g)
    block = torch.cat((torch.cat((x, g), -1), torch.cat((torch.zeros_like(x), x), -1)), -2)
    big, _ = ora_exp(block)
    assert rel_frobenius(l, big[..., :n, n:].double()).max() <= 1e-4


# ---- squaring count ---------------------------------------------------------

def exact_s(x: np.ndarray, g: np.ndarray | None = None):
    """min s >= 0 with norm <= theta 2^s, norm the exact 1-norm (|x| + |g| per entry)."""
    cols = []
    for j in range(x.shape[1]):
        c = Fraction(0)
        for r in range(x.shape[0]):
            c += Fraction(abs(float(x[r, j])))
            if g is not None:
                c += Fraction(abs(float(g[r, j])))
        cols.append(c)
    norm = max(cols)
    theta = Fraction(THETA)
    s = 0
    while norm > theta * 2**s:
        s += 1
    # distance of norm/theta from the nearest power of two, relative
    q = norm / theta
    rel = min(abs(q / 2**k - 1) for k in range(0, 140))
    return s, float(rel)


@pytest.mark.parametrize("pair", [False, True])
@pytest.mark.parametrize("n", [3, 4, 6, 8, 12, 16, 24, 32])
def test_squaring_count_brute_force(n, pair):
    x, g = scaled(64, n, seed=400 + n + 50 * pair, low=-2, high=2.5)
    # non-symmetric on purpose: row sums and column sums differ
    xs = x.numpy()
    gs = g.numpy() if pair else None
    s, _ = oracle.params_f32(xs, gs)
    for b in range(len(xs)):
        es, rel = exact_s(xs[b], None if gs is None else gs[b])
        assert rel > 1e-12  # no sample sits on a rounding boundary
        assert s[b] == es


def test_row_sum_would_differ():
    # A matrix whose largest column sum is below theta but largest row sum above:
    # the 1-norm must use columns (s = 0), the infinity norm would give s = 1.
    a = np.zeros((4, 4), np.float32)
    a[0, :] = 1.0  # row sum 4 > theta, column sums 1
    s, norm = oracle.params_f32(a[None])
    assert norm[0] == 1.0 and s[0] == 0


def test_summation_association_per_padded_size():
    big = np.float32(2.0**53)
    col = np.zeros((4, 4), np.float32)
    col[:, 0] = [big, 1.0, 1.0, 1.0]
    # P = 4: ((x0 + x2) + (x1 + x3)) = (2^53 + 1) + 2 -> 2^53 + 2 (exact in double)
    assert oracle.norm1(col) == 2.0**53 + 2.0
    # P = 16 (same column, zero padded): sequential ((x0 + x1) + x2) + x3 -> 2^53
    pad = np.zeros((16, 16), np.float32)
    pad[:4, :4] = col
    assert oracle.norm1(pad) == 2.0**53
    # P = 8 butterfly ((x0+x4)+(x2+x6))+((x1+x5)+(x3+x7)): (2^53 + 1) + 2 -> 2^53 + 2
    p8 = np.zeros((8, 8), np.float32)
    p8[:4, :4] = col
    assert oracle.norm1(p8) == 2.0**53 + 2.0


def test_nonfinite_rule():
    for bad in (float("nan"), float("inf"), -float("inf")):
        x = torch.zeros(1, 4, 4)
        x[0, 2, 1] = bad
        y, s = ora_exp(x)
        assert y.isnan().all() and s.item() == -1
        l, s2 = ora_frechet(torch.zeros(1, 4, 4), x)
        assert l.isnan().all() and s2.item() == -1


def test_degree_is_always_18():
    assert oracle.DEGREE == 18
    c = oracle.coefficients()
    # the constant term of the evaluation, (b3_0 + b4_0) * b4_0, is 1 to FP32 accuracy
    assert abs((float(c[2, 0]) + float(c[3, 0])) * float(c[3, 0]) - 1.0) < 1e-6


# ---- output rounding ---------------------------------------------------------

def test_bf16_rounding_matches_torch():
    vals = np.array([1.0, 1.00390625, 1.01171875, 3.0e38, -2.5e-40, 65504.0, 1e-45, float("inf"), -0.0],
                    np.float32)
    rnd = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 1e3
    x = np.concatenate([vals, rnd, np.nextafter(vals[:3], np.float32(2))])
    mine = oracle.round_to_dtype(x, torch.bfloat16)
    theirs = torch.from_numpy(x).to(torch.bfloat16)
    assert torch.equal(mine.view(torch.int16), theirs.view(torch.int16))
    nan = oracle.round_to_dtype(np.array([float("nan")], np.float32), torch.bfloat16)
    assert nan.isnan().all()


def test_f16_rounding_matches_torch():
    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 3e4
    mine = oracle.round_to_dtype(x, torch.float16)
    theirs = torch.from_numpy(x).to(torch.float16)
    assert torch.equal(mine.view(torch.int16), theirs.view(torch.int16))


def test_combine_contraction_choice_is_bounded():
    """The restatement's one unpinned choice: the reference's combine c0*I + c1*A + ... is
    contracted as fmaf(c1, A, c0*I); a compiler may instead form fmaf(c0, I, c1*A), which
    rounds c1*A first (only D's diagonal can change).  No reference fixture separates the two.
    Over seeded matrices of every padded size and both directions, the other choice changes
    the results of some matrices (the knob is live) by at most 4 * 2^s FP32 units relative,
    i.e. by the order of one rounding, amplified by the squarings like any other."""
    rng = np.random.default_rng(5)
    for n in (4, 8, 16, 32):
        b = 600 if n <= 8 else 120
        base = rng.standard_normal((b, n, n))
        base /= np.abs(base).sum(1).max(1)[:, None, None]
        x = (base * 10 ** rng.uniform(-2, 1.5, b)[:, None, None]).astype(np.float32)
        g = rng.standard_normal((b, n, n)).astype(np.float32)
        ref = [oracle.matrix_exp_f32(x, threads=4), oracle.matrix_exp_f32(x, g, threads=4)]
        oracle.set_combine_contraction(True)
        try:
            alt = [oracle.matrix_exp_f32(x, threads=4), oracle.matrix_exp_f32(x, g, threads=4)]
        finally:
            oracle.set_combine_contraction(False)
        changed = 0
        for (r, s, _), (a, s_alt, _) in zip(ref, alt):
            assert np.array_equal(s, s_alt)  # the count does not depend on the polynomial
            diff = (a.astype(np.float64) - r).reshape(b, -1)
            rel = np.linalg.norm(diff, axis=1) / np.linalg.norm(r.reshape(b, -1).astype(np.float64), axis=1)
            changed += int((diff != 0).any(1).sum())
            assert (rel <= 4 * 2.0 ** s.clip(0) * 2.0**-24).all(), (n, rel.max())
        assert changed > 0, n
