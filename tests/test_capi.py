"""The C-ABI library loads and exports every function include/*.h declares.

CPU only: nothing here launches a kernel.  Argument validation paths that
return before any HIP call are exercised through ctypes as well.
"""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "flash-hyperconnections_amd" / "flash_hypercons" / "libflash_hypercons_hip.so"


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
    assert {"fh_matrix_exp", "fh_frechet", "fh_expm_launch", "fh_expm_params", "fh_last_error",
            "fh_version"} <= set(names)


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


def test_extension_registers_operators():
    import torch

    import flash_hypercons  # noqa: F401

    for name in ("_matrix_exp", "_frechet", "_expm_params", "_expm_debug"):
        assert hasattr(torch.ops.flash_hypercons, name)
    schema = str(torch.ops.flash_hypercons._matrix_exp.default._schema)
    assert schema == "flash_hypercons::_matrix_exp(Tensor input) -> Tensor"
    schema = str(torch.ops.flash_hypercons._frechet.default._schema)
    assert schema == "flash_hypercons::_frechet(Tensor input, Tensor direction) -> Tensor"
