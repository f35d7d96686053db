"""CPU oracle for the batched small-matrix exponential -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker.  The shipped package
(``flash_hypercons``) never imports it and has no CPU fallback of its own.

The arithmetic lives in ``fh_oracle.c`` (a plain-C restatement of
``csrc/MatrixExpSmall.cuh`` of the reference; each step cites its file:line
there).  This module converts tensors exactly to FP32, calls the C code through
ctypes, and rounds results to the output dtype the way the reference stores them
(``MatrixExpSmall.cuh:108-112``: round-to-nearest-even).

Every function here is pinned by ``tests/test_oracle.py`` against the FP64
``torch.linalg.matrix_exp`` oracle the reference's tests use
(``tests/reference.py:4-11``), the reference's known-answer tests
(``tests/test_matrix_exp.py:47-129``, ``tests/test_integration.py:57-83``),
closed forms, and a brute-force rational check of the squaring count.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libfh_oracle.so"
THETA18 = 3.010066362817634  # csrc/MatrixExpSmall.cuh:14
DEGREE = 18  # csrc/MatrixExpSmall.cuh:163, :368 -- every finite matrix uses t18

_lib = None


def build(force: bool = False) -> Path:
    """Compile fh_oracle.c with gcc (``make -C oracle``)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "fh_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        f64p = ctypes.POINTER(ctypes.c_double)
        _lib.fho_matrix_exp.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int, f32p, i32p, f64p]
        _lib.fho_matrix_exp.restype = ctypes.c_int
        _lib.fho_expm_params.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int, i32p, f64p]
        _lib.fho_expm_params.restype = ctypes.c_int
        _lib.fho_norm1.argtypes = [f32p, f32p, ctypes.c_int]
        _lib.fho_norm1.restype = ctypes.c_double
        _lib.fho_squarings.argtypes = [ctypes.c_double]
        _lib.fho_squarings.restype = ctypes.c_int
        _lib.fho_padded_size.argtypes = [ctypes.c_int]
        _lib.fho_padded_size.restype = ctypes.c_int
        _lib.fho_f32_to_bf16.argtypes = [f32p, ctypes.POINTER(ctypes.c_uint16), ctypes.c_int64]
        _lib.fho_f32_to_bf16.restype = None
        _lib.fho_coefficients.argtypes = []
        _lib.fho_set_combine_contraction.argtypes = [ctypes.c_int]
        _lib.fho_set_combine_contraction.restype = None
        _lib.fho_coefficients.restype = f32p
    return _lib


def _ptr(a: np.ndarray | None, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _as_f32(a: np.ndarray) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.float32:
        raise TypeError(f"oracle expects FP32 arrays (exact conversion is the caller's job), got {a.dtype}")
    return np.ascontiguousarray(a)


def default_threads() -> int:
    """Host threads the checker may use: the process's CPU affinity, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _chunks(batch: int, threads: int):
    threads = max(1, min(threads, batch // 4096 or 1))
    step = -(-batch // threads)
    return [(lo, min(batch, lo + step)) for lo in range(0, batch, step)]


def matrix_exp_f32(x: np.ndarray, g: np.ndarray | None = None, threads: int = 1):
    """exp(x) (g None) or the U block of exp([[x, g], [0, x]]) for FP32 [B, n, n].

    Returns (FP32 result before output rounding, int32 s per matrix, FP64 norm).
    s is -1 where the non-finite rule fired.  ``threads`` > 1 splits the batch
    into contiguous chunks run concurrently (the C code keeps no shared state
    and ctypes releases the GIL); every matrix is computed independently, so
    the result does not depend on the split.
    """
    x = _as_f32(x)
    if x.ndim != 3 or x.shape[-1] != x.shape[-2]:
        raise ValueError("expected [B, n, n]")
    batch, n = x.shape[0], x.shape[-1]
    if g is not None:
        g = _as_f32(g)
        if g.shape != x.shape:
            raise ValueError("direction must match the input")
    out = np.empty_like(x)
    s = np.empty(batch, np.int32)
    norm = np.empty(batch, np.float64)

    def run(lo_hi):
        lo, hi = lo_hi
        rc = lib().fho_matrix_exp(
            _ptr(x[lo:hi], ctypes.c_float), None if g is None else _ptr(g[lo:hi], ctypes.c_float), hi - lo, n,
            _ptr(out[lo:hi], ctypes.c_float), _ptr(s[lo:hi], ctypes.c_int32), _ptr(norm[lo:hi], ctypes.c_double),
        )
        if rc != 0:
            raise RuntimeError("fho_matrix_exp failed")

    if batch:
        _run_chunks(run, batch, threads)
    return out, s, norm


def _run_chunks(run, batch: int, threads: int) -> None:
    parts = _chunks(batch, threads)
    if len(parts) == 1:
        run(parts[0])
        return
    with ThreadPoolExecutor(max_workers=len(parts)) as pool:
        for f in [pool.submit(run, p) for p in parts]:
            f.result()


def params_f32(x: np.ndarray, g: np.ndarray | None = None, threads: int = 1):
    """(s, FP64 norm) per matrix; the degree is always 18 for finite matrices."""
    x = _as_f32(x)
    batch, n = x.shape[0], x.shape[-1]
    if g is not None:
        g = _as_f32(g)
    s = np.empty(batch, np.int32)
    norm = np.empty(batch, np.float64)

    def run(lo_hi):
        lo, hi = lo_hi
        rc = lib().fho_expm_params(_ptr(x[lo:hi], ctypes.c_float), None if g is None else _ptr(g[lo:hi], ctypes.c_float),
                                   hi - lo, n, _ptr(s[lo:hi], ctypes.c_int32), _ptr(norm[lo:hi], ctypes.c_double))
        if rc != 0:
            raise RuntimeError("fho_expm_params failed")

    if batch:
        _run_chunks(run, batch, threads)
    return s, norm


def norm1(tile: np.ndarray, g: np.ndarray | None = None) -> float:
    """FP64 1-norm of one padded P x P FP32 tile with the reference's association."""
    tile = _as_f32(tile)
    P = tile.shape[-1]
    return lib().fho_norm1(_ptr(tile, ctypes.c_float), _ptr(None if g is None else _as_f32(g), ctypes.c_float), P)


def squarings(norm: float) -> int:
    return lib().fho_squarings(float(norm))


def padded_size(n: int) -> int:
    return lib().fho_padded_size(n)


def coefficients() -> np.ndarray:
    p = lib().fho_coefficients()
    return np.ctypeslib.as_array(p, shape=(25,)).reshape(5, 5).copy()


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = _as_f32(a)
    out = np.empty(a.shape, np.uint16)
    if a.size:
        lib().fho_f32_to_bf16(_ptr(a, ctypes.c_float), _ptr(out, ctypes.c_uint16), a.size)
    return out


# ---- torch convenience (tests and bench hand torch tensors around) ---------

def _torch():
    import torch

    return torch


def set_combine_contraction(diag_first: bool) -> None:
    """Test knob: contract each combine's first two terms as fmaf(c0, I, c1*A) (True) instead of
    the restatement's fmaf(c1, A, c0*I) (False, the default).  Global; not for concurrent use."""
    lib().fho_set_combine_contraction(1 if diag_first else 0)


def tensor_to_f32(t) -> np.ndarray:
    """Exact FP32 copy of a (possibly strided / negated / low-precision) tensor."""
    torch = _torch()
    t = t.detach().resolve_neg().resolve_conj().cpu()
    if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError(f"unsupported dtype {t.dtype}")
    return t.float().contiguous().numpy()  # f16/bf16 -> f32 is exact


def round_to_dtype(out_f32: np.ndarray, dtype):
    """Round FP32 results to ``dtype`` (RNE, as the reference's store_value)."""
    torch = _torch()
    if dtype == torch.float32:
        return torch.from_numpy(out_f32.copy())
    if dtype == torch.float16:
        return torch.from_numpy(out_f32.astype(np.float16))  # numpy casts RNE, overflow -> inf
    if dtype == torch.bfloat16:
        bits = f32_to_bf16_bits(out_f32)
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    raise TypeError(dtype)


def torch_matrix_exp(x, threads: int = 1):
    """Oracle forward on a torch tensor: (result in x.dtype on CPU, s int32 tensor)."""
    torch = _torch()
    out, s, _ = matrix_exp_f32(tensor_to_f32(x), threads=threads)
    return round_to_dtype(out, x.dtype), torch.from_numpy(s)


def torch_frechet(x, g, threads: int = 1):
    """Oracle of the op ``_frechet(x, g)``: U block of exp([[x, g],[0, x]])."""
    torch = _torch()
    out, s, _ = matrix_exp_f32(tensor_to_f32(x), tensor_to_f32(g), threads=threads)
    return round_to_dtype(out, x.dtype), torch.from_numpy(s)


def torch_params(x, g=None, threads: int = 1):
    torch = _torch()
    s, norm = params_f32(tensor_to_f32(x), None if g is None else tensor_to_f32(g), threads=threads)
    return torch.from_numpy(s), torch.from_numpy(norm)




__all__ = [
    "THETA18", "DEGREE", "build", "matrix_exp_f32", "params_f32", "norm1", "squarings", "padded_size",
    "coefficients", "f32_to_bf16_bits", "tensor_to_f32", "round_to_dtype", "torch_matrix_exp",
    "torch_frechet", "torch_params", "default_threads", "set_combine_contraction",
]

if os.environ.get("FHO_BUILD_ON_IMPORT"):
    build()
