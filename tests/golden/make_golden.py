"""Writes the committed golden fixtures under tests/golden/.

Run: python tests/golden/make_golden.py

Fixtures are data only (inputs and expected outputs); none of them is
produced by running reference code.  Expected values come from native
PyTorch in FP64 -- the oracle the reference's own tests use
(tests/reference.py:4-11 there: linalg_matrix_exp of the matrix, and of the
block matrix [[A, G], [0, A]] for the Frechet derivative) -- and from exact
rational arithmetic for the squaring counts.

* c1_cpu_plumbing.npz: x = [128, 4, 4] FP32 entries
  N(0, 1) from torch.manual_seed(0); loss = y.sum(), i.e. upstream gradient
  all ones.  Stores x, exp(x) and the gradient exp-Frechet L(x^T, 1) in FP64.
* s_boundaries.npz -- skew-symmetric 4x4, 8x8, 16x16, 32x32 FP32 matrices
  scaled to the 1-norms of the reference's boundary test
  (tests/test_matrix_exp.py:51-63 there) and their exact squaring counts.
"""

from fractions import Fraction
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
THETA = 3.010066362817634
NORMS = [0.0, 0.1, THETA * (1 - 1e-5), THETA * (1 + 1e-5), 2 * THETA * (1 - 1e-5), 2 * THETA * (1 + 1e-5),
         12.04028, 24.08056]


def exact_squarings(m: np.ndarray) -> int:
    """Smallest s >= 0 with ||m||_1 <= theta * 2^s, in exact rational arithmetic."""
    norm = max(sum(Fraction(abs(float(v))) for v in m[:, j]) for j in range(m.shape[1]))
    theta = Fraction(THETA)
    s = 0
    while norm > theta * 2**s:
        s += 1
    return s


def fp64_exp(a: torch.Tensor) -> torch.Tensor:
    return torch.linalg.matrix_exp(a.double())


def fp64_frechet(a: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    a, g = a.double(), g.double()
    n = a.shape[-1]
    block = torch.cat((torch.cat((a, g), -1), torch.cat((torch.zeros_like(a), a), -1)), -2)
    return torch.linalg.matrix_exp(block)[..., :n, n:]


def c1_fixture() -> None:
    torch.manual_seed(0)
    x = torch.randn(128, 4, 4)
    y = fp64_exp(x)
    ones = torch.ones_like(x)
    grad = fp64_frechet(x.mT, ones)
    np.savez_compressed(HERE / "c1_cpu_plumbing.npz", x=x.numpy(), y=y.numpy(), grad=grad.numpy())


def boundary_fixture() -> None:
    gen = torch.Generator().manual_seed(5)
    out = {}
    for n in (4, 8, 16, 32):
        m = torch.randn(len(NORMS), n, n, generator=gen, dtype=torch.float64)
        m = m - m.mT
        m = m * (torch.tensor(NORMS, dtype=torch.float64) / torch.linalg.matrix_norm(m, ord=1).clamp_min(1e-300))[:, None, None]
        m32 = m.float().numpy()
        out[f"x{n}"] = m32
        out[f"s{n}"] = np.array([exact_squarings(mm) for mm in m32], dtype=np.int32)
    np.savez_compressed(HERE / "s_boundaries.npz", **out)


if __name__ == "__main__":
    c1_fixture()
    boundary_fixture()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
