"""The C-ABI library loads and exports every function include/*.h declares.

CPU only: nothing here launches a kernel.  Argument validation paths that
return before any HIP call are exercised through ctypes as well.
"""

import ctypes
import re
from pathlib import Path

import pytest

import flash_hypercons

ROOT = Path(__file__).resolve().parents[1]
LIB = Path(flash_hypercons.__file__).resolve().parent / "libflash_hypercons_hip.so"


def declared_functions():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = header.read_text()
        names += re.findall(r"FH_API\s+[\w\s\*]+?\b(fh_\w+)\s*\(", text)
    return names


def load():
    return ctypes.CDLL(str(LIB))


def test_headers_declare_entry_points():
    names = declared_functions()
    assert {"fh_matrix_exp", "fh_frechet", "fh_expm_launch", "fh_expm_params", "fh_hc_mix", "fh_hc_mix_backward",
            "fh_hc_apply", "fh_hc_apply_backward", "fh_last_error", "fh_version"} <= set(names)


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports(name):
    assert hasattr(load(), name)


def test_version_and_validation_without_gpu():
    lib = load()
    lib.fh_version.restype = ctypes.c_char_p
    lib.fh_last_error.restype = ctypes.c_char_p
    assert lib.fh_version() == b"0.1.0"
    strides = (ctypes.c_int64 * 3)(16, 4, 1)
    lib.fh_matrix_exp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    # n out of range: rejected with the reference's message before any HIP call.
    rc = lib.fh_matrix_exp(None, strides, 0, None, 0, 4, 33, None)
    assert rc == 1
    assert b"2 <= N <= 32" in lib.fh_last_error()
    # Unknown dtype.
    assert lib.fh_matrix_exp(None, strides, 0, None, 7, 4, 4, None) == 1
    # Empty batch is a no-op and succeeds without touching the device.
    assert lib.fh_matrix_exp(None, strides, 0, None, 0, 0, 4, None) == 0
    # Non-empty batch with null pointers is rejected.
    assert lib.fh_matrix_exp(None, strides, 0, None, 0, 2, 4, None) == 1
    lib.fh_frechet.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                               ctypes.c_void_p]
    assert lib.fh_frechet(None, strides, 0, None, strides, 0, None, 0, 3, 4, None) == 1
    assert b"direction" in lib.fh_last_error()


def test_hc_mix_validation_without_gpu():
    lib = load()
    lib.fh_last_error.restype = ctypes.c_char_p
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.fh_hc_mix.argtypes = [vp, vp, i32, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    lib.fh_hc_mix_backward.argtypes = [vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    hs = (ctypes.c_int64 * 3)(16, 4, 1)
    xs = (ctypes.c_int64 * 3)(4 * 64, 64, 1)
    fake = 1 << 20  # never dereferenced: every call below returns before a HIP call
    # n outside [2, 4], unknown dtype, C < 1.
    for n, dtype, cols in ((5, 0, 64), (1, 0, 64), (4, 3, 64), (4, 0, 0)):
        assert lib.fh_hc_mix(fake, hs, 0, fake, xs, fake, None, dtype, 2, n, cols, None) == 1
        assert b"2 <= n <= 4" in lib.fh_last_error()
    # Empty batch: no-op.
    assert lib.fh_hc_mix(None, hs, 0, None, xs, None, None, 0, 0, 4, 64, None) == 0
    # Null pointers.
    assert lib.fh_hc_mix(None, hs, 0, fake, xs, fake, None, 0, 2, 4, 64, None) == 1
    assert b"null pointer" in lib.fh_last_error()
    # Rows: C and strides in whole 16-byte vectors, unit column stride, aligned base.
    bad_rows = (
        ((ctypes.c_int64 * 3)(4 * 64, 64, 2), fake, 64),
        ((ctypes.c_int64 * 3)(4 * 64, 66, 1), fake, 64),
        (xs, fake, 62),
        (xs, fake + 4, 64),
        ((ctypes.c_int64 * 3)(4 * 64, -64, 1), fake, 64),
    )
    for strides, ptr, cols in bad_rows:
        assert lib.fh_hc_mix(fake, hs, 0, ptr, strides, fake, None, 0, 2, 4, cols, None) == 1
        assert b"16-byte aligned rows" in lib.fh_last_error()
    # Span: one token's input rows, or its contiguous output (n * C elements), at 2 GiB or more.
    # Rows that overlap (row stride 0) keep the input's span small while the output's is not.
    for strides, cols in (((ctypes.c_int64 * 3)(0, 1 << 29, 1), 64),
                          ((ctypes.c_int64 * 3)(0, 0, 1), 1 << 27)):
        assert lib.fh_hc_mix(fake, hs, 0, fake, strides, fake, None, 0, 2, 4, cols, None) == 1
        assert b"span less than 2 GiB" in lib.fh_last_error()
        assert lib.fh_hc_mix_backward(fake, hs, 0, fake, xs if cols == 64 else strides, fake, strides, fake, fake,
                                      None, 0, 2, 4, cols, None) == 1
        assert b"span less than 2 GiB" in lib.fh_last_error()
    # Backward: grad rows follow the same rule; grad and dh must be given.
    bad = (ctypes.c_int64 * 3)(4 * 64, 64, 2)
    assert lib.fh_hc_mix_backward(fake, hs, 0, fake, xs, fake, bad, fake, fake, None, 0, 2, 4, 64, None) == 1
    assert b"16-byte aligned rows" in lib.fh_last_error()
    assert lib.fh_hc_mix_backward(fake, hs, 0, fake, xs, None, xs, fake, fake, None, 0, 2, 4, 64, None) == 1
    assert lib.fh_hc_mix_backward(fake, hs, 0, fake, xs, fake, xs, None, fake, None, 0, 2, 4, 64, None) == 1
    assert b"null grad or dh" in lib.fh_last_error()


def test_hc_apply_validation_without_gpu():
    lib = load()
    lib.fh_last_error.restype = ctypes.c_char_p
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.fh_hc_apply.argtypes = [vp, vp, vp, vp, i32, i64, i32, i64, vp]
    lib.fh_hc_apply_backward.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i64, i32, i64, vp]
    xs = (ctypes.c_int64 * 3)(8 * 64, 64, 1)
    fake = 1 << 20  # never dereferenced: every call below returns before a HIP call
    # n outside [5, 8], unknown dtype, C < 1.
    for n, dtype, cols in ((4, 0, 64), (9, 0, 64), (6, 3, 64), (6, 0, 0)):
        assert lib.fh_hc_apply(fake, fake, xs, fake, dtype, 2, n, cols, None) == 1
        assert b"5 <= n <= 8" in lib.fh_last_error()
    assert lib.fh_hc_apply(None, None, xs, None, 0, 0, 8, 64, None) == 0
    assert lib.fh_hc_apply(None, fake, xs, fake, 0, 2, 8, 64, None) == 1
    assert b"null pointer" in lib.fh_last_error()
    assert lib.fh_hc_apply(fake + 2, fake, xs, fake, 0, 2, 8, 64, None) == 1
    assert b"4-byte aligned" in lib.fh_last_error()
    # Rows: the rule of fh_hc_mix (BF16: C and strides in multiples of 8 elements).
    for strides, ptr, cols in (
        ((ctypes.c_int64 * 3)(8 * 64, 64, 2), fake, 64),
        ((ctypes.c_int64 * 3)(8 * 64, 68, 1), fake, 64),
        (xs, fake, 60),
        (xs, fake + 8, 64),
    ):
        assert lib.fh_hc_apply(fake, ptr, strides, fake, 1, 2, 8, cols, None) == 1
        assert b"16-byte aligned rows" in lib.fh_last_error() and b"multiples of 8" in lib.fh_last_error()
    for strides, cols in (((ctypes.c_int64 * 3)(0, 1 << 28, 1), 64),  # input rows span more than 2 GiB
                          ((ctypes.c_int64 * 3)(0, 0, 1), 1 << 27)):  # output token spans 2 GiB (8 x 2^27 BF16)
        assert lib.fh_hc_apply(fake, fake, strides, fake, 1, 2, 8, cols, None) == 1
        assert b"span less than 2 GiB" in lib.fh_last_error()
    bad = (ctypes.c_int64 * 3)(8 * 64, 64, 2)
    assert lib.fh_hc_apply_backward(fake, fake, xs, fake, bad, fake, fake, 0, 2, 8, 64, None) == 1
    assert b"16-byte aligned rows" in lib.fh_last_error()
    assert lib.fh_hc_apply_backward(fake, fake, xs, None, xs, fake, fake, 0, 2, 8, 64, None) == 1
    assert lib.fh_hc_apply_backward(fake, fake, xs, fake, xs, fake, None, 0, 2, 8, 64, None) == 1
    assert b"null grad or de" in lib.fh_last_error()
    assert lib.fh_hc_apply_backward(fake, fake, xs, fake, xs, fake, fake + 1, 0, 2, 8, 64, None) == 1
    assert b"dE must be 4-byte aligned" in lib.fh_last_error()


def test_extension_registers_operators():
    import torch

    import flash_hypercons  # noqa: F401

    for name in ("_matrix_exp", "_frechet", "_expm_params", "_expm_debug", "_hc_mix", "_hc_mix_backward",
                 "_hc_mix_aux", "_hc_apply", "_hc_apply_backward"):
        assert hasattr(torch.ops.flash_hypercons, name)
    schema = str(torch.ops.flash_hypercons._matrix_exp.default._schema)
    assert schema == "flash_hypercons::_matrix_exp(Tensor input) -> Tensor"
    schema = str(torch.ops.flash_hypercons._frechet.default._schema)
    assert schema == "flash_hypercons::_frechet(Tensor input, Tensor direction) -> Tensor"


def test_package_under_test():
    """The package these tests import: the source tree, or with FH_TEST_INSTALLED set, an
    installed copy (``pip install --no-build-isolation --target DIR .``) that carries both
    libraries."""
    import os

    pkg = Path(flash_hypercons.__file__).resolve().parent
    in_tree = pkg == (ROOT / "flash-hyperconnections_amd" / "flash_hypercons").resolve()
    assert in_tree != (os.environ.get("FH_TEST_INSTALLED", "") not in ("", "0"))
    assert (pkg / "libflash_hypercons_hip.so").is_file() and (pkg / "_C.so").is_file()
    assert Path(flash_hypercons._C.__file__).resolve().parent == pkg


def test_last_error_is_per_thread():
    """fh_last_error() reports the last failing call of the calling thread only."""
    import threading

    lib = load()
    lib.fh_last_error.restype = ctypes.c_char_p
    lib.fh_matrix_exp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    strides = (ctypes.c_int64 * 3)(16, 4, 1)
    failed = threading.Event()
    seen = {}

    def failing():
        seen["rc"] = lib.fh_matrix_exp(None, strides, 0, None, 0, 4, 33, None)
        seen["failing"] = lib.fh_last_error()
        failed.set()

    def clean():
        failed.wait(10)
        seen["ok_rc"] = lib.fh_matrix_exp(None, strides, 0, None, 0, 0, 4, None)  # empty batch: succeeds
        seen["clean"] = lib.fh_last_error()

    threads = [threading.Thread(target=failing), threading.Thread(target=clean)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(10)
    assert seen["rc"] == 1 and b"2 <= N <= 32" in seen["failing"]
    assert seen["ok_rc"] == 0 and seen["clean"] == b""
