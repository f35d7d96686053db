"""The full-size parity harness (tests/fullsize.py) on the CPU.

The GPU parity test and bench.py's parity block trust these counts, so the
counting itself is checked here with a stand-in "kernel" made from the oracle:
an exact copy must count zero everywhere, and mistakes planted in the stand-in
(a wrong squaring count, a flipped bit, an error above the north-star bound)
must be counted where they were planted.
"""

import pytest
import torch

import oracle
from tests.fullsize import (direction_parity, error_ratio, excess_over_reference, strict_failure_allowance,
                            strict_failures)
from tests.reference import reference


def _inputs(batch, n, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    base = torch.randn(batch, n, n, generator=gen, dtype=torch.float64)
    base = base / torch.linalg.matrix_norm(base, ord=1)[:, None, None]
    scale = 10 ** torch.empty(batch, dtype=torch.float64).uniform_(-2, 1.5, generator=gen)
    return (base * scale[:, None, None]).to(dtype), torch.randn(batch, n, n, generator=gen).to(dtype)


def _oracle_launch(x, g):
    return oracle.torch_matrix_exp(x) if g is None else oracle.torch_frechet(x, g)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("backward", [False, True])
def test_exact_copy_counts_nothing(backward, dtype):
    x, g = _inputs(300, 4, dtype, seed=3 + backward)
    xs = x.mT if backward else x
    gs = g if backward else None
    out, _ = _oracle_launch(xs, gs)
    r = direction_parity(xs, gs, out, threads=2, launch=_oracle_launch)
    assert r["s_mismatches"] == 0 and r["bitwise_mismatches_vs_oracle"] == 0
    assert r["strict_failures_kernel"] == r["strict_failures_oracle"]
    assert r["matrices_worse_than_reference"] == 0 and r["debug_launch_matches_op"]
    assert r["max_excess_over_reference"] <= (1.0 if dtype == torch.float32 else 0.0)


def test_planted_mistakes_are_counted():
    x, g = _inputs(200, 4, torch.float32, seed=11)
    out, s = _oracle_launch(x, None)
    bad = out.clone()
    bad[5, 1, 2] = torch.nextafter(bad[5, 1, 2], torch.tensor(float("inf")))  # one ulp: bitwise only
    bad[9] *= 1.001  # 1e-3 relative: breaks the 1e-5 bound

    def wrong_s(xx, gg):
        o, ss = _oracle_launch(xx, gg)
        ss = ss.clone()
        ss[17] += 1
        return bad, ss

    r = direction_parity(x, None, bad, threads=1, launch=wrong_s)
    assert r["s_mismatches"] == 1
    assert r["bitwise_mismatches_vs_oracle"] == 2
    assert r["strict_failures_kernel"] == r["strict_failures_oracle"] + 1
    assert r["matrices_worse_than_reference"] == 1
    assert r["max_excess_over_reference"] > 10


def test_low_precision_rule_counts_ulps_and_infinities():
    ref = reference(torch.zeros(3, 4, 4))  # identity
    act = ref.to(torch.float16).clone()
    assert not strict_failures(act, ref, backward=False).any()
    act[1, 0, 0] = torch.nextafter(act[1, 0, 0], torch.tensor(2.0, dtype=torch.float16))  # one ulp: allowed
    act[2, 3, 3] = float("inf")
    assert strict_failures(act, ref, backward=False).tolist() == [False, False, True]
    act[1, 0, 0] = 1.0 + 3 * 2.0**-10  # three ulps
    assert strict_failures(act, ref, backward=False).tolist() == [False, True, True]
    k = error_ratio(act, ref, backward=False)
    assert k[1].item() == 3.0 and k[2].isinf()
    # against a reference arithmetic two ulps off on matrix 1 and broken on matrix 2: one ulp more
    o = torch.tensor([0.0, 2.0, float("inf")], dtype=torch.float64)
    assert excess_over_reference(k, o, torch.float16).tolist() == [-1.0, 1.0, 0.0]


def test_overflow_band_and_gate():
    from tests.fullsize import check

    ref = torch.full((3, 4, 4), 1.0, dtype=torch.float64)
    ref[0, 0, 0] = 65519.0  # a hair below the FP16 overflow threshold 65520
    ref[1, 0, 0] = 60000.0
    ref[2, 0, 0] = -65530.0  # a hair above (rounds to -inf)
    act = ref.to(torch.float16).clone()
    assert error_ratio(act, ref, backward=False).tolist()[0] <= 1.0
    act[0, 0, 0] = float("inf")  # inside the band: either rounding is the same evaluation
    act[2, 0, 0] = -65504.0
    act[1, 0, 0] = float("inf")  # far from the threshold: broken
    assert error_ratio(act, ref, backward=False)[:, None].isinf().flatten().tolist() == [False, True, False]
    act[2, 0, 0] = float("inf")  # wrong sign
    assert error_ratio(act, ref, backward=False)[2].isinf()

    good = {"s_mismatches": 0, "bitwise_mismatches_vs_oracle": 0, "strict_failures_kernel": 3,
            "strict_failures_oracle": 3, "mean_rel_frobenius": 1.0e-6, "oracle_mean_rel_frobenius": 1.0e-6,
            "max_excess_over_reference": 1.2, "excess_unit": "ratio", "debug_launch_matches_op": True}
    assert check(good, 32) == [] and check(good, 4) == []
    for key, value, n in (("s_mismatches", 1, 32), ("bitwise_mismatches_vs_oracle", 5, 4),
                          ("strict_failures_kernel", 4, 4), ("strict_failures_kernel", 12, 32),
                          ("mean_rel_frobenius", 1.2e-6, 32), ("max_excess_over_reference", 5.0, 32),
                          ("debug_launch_matches_op", False, 32)):
        assert check({**good, key: value}, n), key
    assert check({**good, "bitwise_mismatches_vs_oracle": 7}, 32) == []  # n >= 16 need not match in bits
    # Tiles: binomial noise on the count is allowed (3 + 3 sqrt(3) + 3 = 11), none at n <= 8.
    assert strict_failure_allowance(3) == 8 and strict_failure_allowance(500) == 70
    assert check({**good, "strict_failures_kernel": 11}, 32) == []
    # FP16/BF16: the mean normwise error, in output ulps, against the restatement's.
    low = {**good, "excess_unit": "output ulps", "max_excess_over_reference": -1.0, "mean_normwise_ulps": 1.0e-4,
           "oracle_mean_normwise_ulps": 1.0e-4}
    del low["mean_rel_frobenius"], low["oracle_mean_rel_frobenius"]
    assert check(low, 32) == []
    assert check({**low, "mean_normwise_ulps": 1.1e-4}, 32)
    assert check({**low, "max_excess_over_reference": 2.5}, 32)


def test_normwise_floor_uses_overflowed_scale():
    """A small entry next to one that overflows FP16: its error is measured at the scale of the
    largest entry (normwise), not in its own ulps."""
    ref = torch.zeros(1, 4, 4, dtype=torch.float64)
    ref[0, 0, 0] = 1.0e6  # overflows FP16
    ref[0, 1, 1] = 3.0
    act = ref.to(torch.float16).clone()
    act[0, 1, 1] = 3.0 + 40 * 2.0**-9  # 40 ulps of 3.0, far below one "ulp" at 1e6
    assert error_ratio(act, ref, backward=False).item() > 30
    assert error_ratio(act, ref, backward=False, normwise=True).item() < 1e-3


def test_normwise_reads_infinity_as_an_interval():
    ref = torch.zeros(2, 4, 4, dtype=torch.float64)
    ref[:, 0, 0] = 1.0e7  # the matrix scale: one FP16-style ulp there is 2^(23 - 10) = 8192
    ref[0, 1, 1] = 65000.0  # below the FP16 overflow threshold 65520
    ref[1, 1, 1] = -65000.0
    act = ref.to(torch.float16).clone()
    act[0, 1, 1] = float("inf")  # 520 below the interval [65520, inf): 520 / 8192 ulps
    act[1, 1, 1] = float("inf")  # wrong sign: 130520 away
    r = error_ratio(act, ref, backward=False, normwise=True)
    assert abs(r[0].item() - 520 / 8192) < 1e-9
    assert abs(r[1].item() - 130520 / 8192) < 1e-9


def test_sweep_overflow_rule_on_planted_results():
    """The seeded sweep's rule for n >= 9 results the reference arithmetic overflows
    (tests/test_parity_sweep.py::_mismatches), on a stand-in result made from the oracle and
    judged against the FP64 exact result: where the exact value lies beyond the output range, a
    non-finite value of either kind or a finite one at the top of the range passes and an ordinary
    finite value fails; where it lies within the range, a non-finite value or one within the
    tolerance passes and one far off fails; a NaN where the oracle's result is finite fails."""
    from tests.reference import reference
    from tests.test_parity_sweep import _mismatches

    n, dtype = 10, torch.bfloat16
    # exp(89 I) = e^89 I: its diagonal (4.5e38) lies just beyond the BF16/FP32 range, its zeros inside.
    x = torch.eye(n, dtype=torch.float64).repeat(2, 1, 1) * torch.tensor([0.1, 89.0])[:, None, None]
    x = x.to(dtype)
    want, want_s = oracle.torch_matrix_exp(x)
    assert bool(torch.isfinite(want[0]).all()) and not bool(torch.isfinite(want[1]).all())
    exact = lambda rows: reference(x[rows])  # noqa: E731
    ex1 = reference(x[1:2])[0]
    top = torch.finfo(dtype).max
    bad = ((~torch.isfinite(want[1])) & (ex1.abs() > top)).nonzero()[0].tolist()
    inside = (ex1.abs() < top).nonzero()[0].tolist()

    def planted(value, at):
        out = want.clone()
        out[1, at[0], at[1]] = value
        return out

    def rule(out):
        return _mismatches(out, want_s, want, want_s, n, dtype, exact)

    assert rule(want) == []
    other = float("nan") if not bool(want[1, bad[0], bad[1]].isnan()) else float("inf")
    assert rule(planted(other, bad)) == []
    assert rule(planted(0.99 * top, bad)) == []
    assert rule(planted(1.0, bad))
    assert rule(planted(-0.5 * top, bad))
    assert rule(planted(float("inf"), inside)) == []  # the kernel's own order may overflow
    assert rule(planted(0.0, inside)) == []
    assert rule(planted(0.9 * top, inside))
    out = want.clone()
    out[0, 2, 3] = float("nan")
    assert rule(out)
