"""CPU checks of bench.py's contract: the one-GPU rule and the seeded workloads.

No GPU is touched: ``--gpus`` above 1 must exit before torch is imported, and the
synthetic inputs of every config must be reproducible (their hashes are what
the JSON line reports).
"""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused(gpus):
    proc = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", gpus],
        capture_output=True, text=True, timeout=120, cwd=ROOT, env={**os.environ, "HIP_VISIBLE_DEVICES": ""},
    )
    assert proc.returncode == 2
    assert "measures one GPU" in proc.stderr
    assert proc.stdout == ""


def test_config_inputs_are_seeded_and_shaped():
    import torch

    sys.path.insert(0, str(ROOT))
    import bench

    shapes = {"c2": (1 << 20, 4, 4), "c3": (1 << 20, 4, 4), "c4": (65536, 16, 16), "p8": (262144, 8, 8)}
    dtypes = {"c2": torch.float32, "c3": torch.bfloat16, "c4": torch.float32, "p8": torch.float32}
    for name, shape in shapes.items():
        x1, g1, _ = bench.make_inputs(name, torch, "cpu")
        x2, g2, _ = bench.make_inputs(name, torch, "cpu")
        assert tuple(x1.shape) == shape and x1.dtype == dtypes[name]
        assert torch.equal(x1, x2) and torch.equal(g1, g2)
        assert bench.sha256(x1) == bench.sha256(x2)
    x, _, layout = bench.make_inputs("c4", torch, "cpu")
    assert layout == "transposed view" and x.stride(-2) == 1  # BASELINE config 4 is a transposed view
