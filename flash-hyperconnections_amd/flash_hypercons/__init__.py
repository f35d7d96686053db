"""Small batched matrix exponentials for PyTorch on AMD Instinct MI355X (gfx950)."""

import torch  # noqa: F401  (loads libc10/libtorch before the extension module)

from .ops.hc_mix import mix_streams
from .ops.matrix_exp import matrix_exp, use_backend

__version__ = "0.1.0"
__all__ = ["matrix_exp", "mix_streams", "use_backend"]
