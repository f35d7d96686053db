"""Parity checks of the fused stream mixing (``fh.mix_streams``) against the CPU
restatement and FP64 products -- test infrastructure, shared by
tests/test_hc_mix.py and bench.py's CPU leg.

``bound_violations`` counts entries of a computed product outside the
elementwise error bound of an FP32 summation with a stated number of roundings
(plus the final rounding to the storage dtype), around the FP64 product of the
same operands.  ``mix_parity`` applies it, and the bitwise checks of exp(h) and
dh against the restatement, to a whole workload in chunks of tokens, so that
the FP64 copies stay small.
"""

from __future__ import annotations

import numpy as np

import oracle

U32 = 2.0**-24


def _torch():
    import torch

    return torch


def half_ulp(dtype) -> float:
    torch = _torch()
    return {torch.float32: 0.0, torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8}[dtype]


def floor(dtype) -> float:
    """Half the smallest subnormal spacing of dtype (absolute slack for results that underflow)."""
    torch = _torch()
    return {torch.float32: 2.0**-150, torch.float16: 2.0**-25, torch.bfloat16: 2.0**-134}[dtype]


def bound_violations(actual, ref64, scale64, terms: int, dtype) -> int:
    """Entries with |actual - ref| > u |ref| + terms 2^-24 (1 + u) scale + floor.

    ``scale`` is |A| @ |B| of the product A @ B, so the middle term bounds a
    summation with ``terms`` FP32 roundings; u is the relative half-ulp of the
    storage dtype (0 for a result that stays FP32).
    """
    a = actual.detach().double().cpu()
    u = half_ulp(dtype)
    bound = u * ref64.abs() + terms * U32 * (1 + u) * scale64 + floor(dtype)
    return int(((a - ref64).abs() > bound).sum())


def oracle_exp(h, threads: int = 1):
    """The restatement's FP32 exp(h) as a torch tensor on the CPU."""
    torch = _torch()
    out, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(h), threads=threads)
    return torch.from_numpy(out)


def oracle_frechet(a, d, threads: int = 1) -> np.ndarray:
    """The restatement's FP32 L(a, d)."""
    out, _, _ = oracle.matrix_exp_f32(oracle.tensor_to_f32(a), oracle.tensor_to_f32(d), threads=threads)
    return out


def dE_terms(cols: int) -> int:
    """Roundings of one dE entry: a per-lane chain over about C/64 columns (at most 16 more, the
    chunk rounding), then a 6-level tree over the wavefront; with margin."""
    return cols // 64 + 24


def mix_parity(h, x, g, y, e, dx, dh, de, *, chunk: int = 1024, threads: int = 1) -> dict:
    """Parity of one forward (y, and e = exp(h) read back from the kernel) and one backward (dx,
    dh, and de = the kernel's dE) of the fused mixing, over every token.

    * e bit-identical to the restatement's exp(h); dh bit-identical to the restatement's
      L(h^T, de) rounded to the dtype;
    * y, dx within the n-term FMA-chain bound of the FP64 products e @ x and e^T @ g;
    * de within the summation bound of the FP64 product g @ x^T.
    """
    torch = _torch()
    dtype = x.dtype
    n, cols = x.shape[1], x.shape[2]
    e_ref = oracle_exp(h, threads)
    e_cpu = e.detach().cpu()
    report = {"tokens": int(x.shape[0]), "n": int(n), "cols": int(cols), "dtype": str(dtype).replace("torch.", "")}
    report["exp_bitwise_mismatches"] = int((e_cpu.view(torch.int32) != e_ref.view(torch.int32)).any(-1).any(-1).sum())
    dh_ref = oracle.round_to_dtype(oracle_frechet(h.mT, de, threads), dtype)
    dh_cpu = dh.detach().cpu()
    ibits = {4: torch.int32, 2: torch.int16}[dh_cpu.element_size()]
    report["dh_bitwise_mismatches"] = int((dh_cpu.view(ibits) != dh_ref.view(ibits)).any(-1).any(-1).sum())
    y_bad = dx_bad = de_bad = 0
    e64_all = e_ref.double()
    for lo in range(0, x.shape[0], chunk):
        hi = min(lo + chunk, x.shape[0])
        e64 = e64_all[lo:hi]
        x64 = x[lo:hi].double().cpu()
        g64 = g[lo:hi].double().cpu()
        y_bad += bound_violations(y[lo:hi], e64 @ x64, e64.abs() @ x64.abs(), n, dtype)
        dx_bad += bound_violations(dx[lo:hi], e64.mT @ g64, e64.abs().mT @ g64.abs(), n, dtype)
        de_bad += bound_violations(de[lo:hi], g64 @ x64.mT, g64.abs() @ x64.abs().mT, dE_terms(cols),
                                   torch.float32)
    report["y_bound_violations"] = y_bad
    report["dx_bound_violations"] = dx_bad
    report["de_bound_violations"] = de_bad
    return report


def check_mix(report: dict) -> list[str]:
    """Reasons a mix_parity report fails (empty when it passes)."""
    keys = ("exp_bitwise_mismatches", "dh_bitwise_mismatches", "y_bound_violations", "dx_bound_violations",
            "de_bound_violations")
    return [f"{k} = {report[k]}" for k in keys if report[k] != 0]
