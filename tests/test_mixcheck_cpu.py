"""The fused-mixing parity checks (tests/mixcheck.py) on the CPU, with the CPU restatement's
exp(h) and FP32 torch products standing in for the kernels: a faithful computation passes, and
planted mistakes -- a transposed exp(h), a dropped term, a lost column chunk in dE, dh taken
at h instead of h^T, a perturbed last bit of exp(h) -- each fail."""

import pytest
import torch

import oracle
from tests.mixcheck import check_mix, mix_parity, oracle_exp, oracle_frechet


def _standin(h, x, g):
    """What the kernels compute, with the restatement's exp and FP32 products."""
    e = oracle_exp(h)
    y = (e @ x.float()).to(x.dtype)
    dx = (e.mT @ g.float()).to(x.dtype)
    de = g.float() @ x.float().mT
    dh = oracle.round_to_dtype(oracle_frechet(h.mT, de), x.dtype)
    return y, e, dx, dh, de


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_faithful_standin_passes(dtype):
    torch.manual_seed(3)
    h = (torch.randn(40, 4, 4) * 0.7).to(dtype)
    x = torch.randn(40, 4, 256).to(dtype)
    g = torch.randn(40, 4, 256).to(dtype)
    y, e, dx, dh, de = _standin(h, x, g)
    report = mix_parity(h, x, g, y, e, dx, dh, de, chunk=16)
    assert check_mix(report) == [], report


def test_planted_mistakes_fail():
    torch.manual_seed(4)
    h = torch.randn(24, 4, 4) * 0.7
    x = torch.randn(24, 4, 128)
    g = torch.randn(24, 4, 128)
    y, e, dx, dh, de = _standin(h, x, g)
    planted = {
        "y_bound_violations": dict(y=e.mT @ x),
        "dx_bound_violations": dict(dx=e @ g),
        "de_bound_violations": dict(de=g[..., 8:] @ x[..., 8:].mT),
        "dh_bitwise_mismatches": dict(dh=oracle.round_to_dtype(oracle_frechet(h, de), torch.float32)),
        "exp_bitwise_mismatches": dict(e=(e.view(torch.int32) ^ 1).view(torch.float32)),
    }
    dropped = e.clone()
    dropped[:, :, 3] = 0
    planted_y2 = dropped @ x
    for key, change in planted.items():
        args = dict(y=y, e=e, dx=dx, dh=dh, de=de)
        args.update(change)
        report = mix_parity(h, x, g, args["y"], args["e"], args["dx"], args["dh"], args["de"], chunk=8)
        assert report[key] > 0, (key, report)
    report = mix_parity(h, x, g, planted_y2, e, dx, dh, de)
    assert report["y_bound_violations"] > 0
