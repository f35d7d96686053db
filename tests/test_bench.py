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


def _canned_full():
    """A full report shaped as bench.py builds it, with every optional block present and long."""
    sys.path.insert(0, str(ROOT))
    import bench

    class Args:
        steps, warmup, settle = 20, 5, 0.3

    def cfg(n):
        return {"shape": [1 << 20, n, n], "dtype": "float32", "layout": "contiguous",
                "matrices_per_s_fwd_bwd": 1.4e10, "ms_step": 0.0742, "ms_step_trials": [0.0742] * 50,
                "ms_step_graph": 0.09, "ms_fwd_kernel": 0.0236, "ms_bwd_kernel": 0.0515,
                "ms_fwd_trials": [0.0236] * 50, "ms_bwd_trials": [0.0515] * 50, "mean_s_fwd": 0.0,
                "mean_s_bwd": 1.23, "bound": "hbm", "roofline_frac_step": 0.566,
                "fwd_kernel": {"bound": "hbm", "achieved_gbs": 5700.0, "achieved_tflops": 1.0, "frac": 0.71},
                "bwd_kernel": {"bound": "hbm", "achieved_gbs": 3909.2, "achieved_tflops": 2.0, "frac": 0.49},
                "input_sha256": "0" * 16, "grad_sha256": "1" * 16}

    mix = {"workload": "w" * 100, "path": "fused", "shape": [16384, 4, 4096], "dtype": "bfloat16",
           "tokens_per_s_fwd_bwd": 3.4e7, "ms_step": 0.482, "ms_step_trials": [0.48] * 50, "ms_fwd_kernel": 0.184,
           "ms_bwd_kernel": 0.297, "ms_fwd_trials": [0.18] * 50, "ms_bwd_trials": [0.3] * 50,
           "composed_ms_fwd": 4.0, "composed_ms_step": 9.3, "composed_ms_step_trials": [9.3] * 50,
           "speedup_fwd_vs_composed": 20.0, "speedup_step_vs_composed": 19.0, "fwd_kernel": {}, "bwd_kernel": {},
           "roofline_frac_step": 0.696}
    results = {name: cfg(4) for name in ("c2", "c3", "c4", "c5", "c5f32", "p8", "c2s8")}
    results.update({"hc": mix, "hc8": dict(mix)})
    cold = {"sets": 4, "input_mib": 512.0, "ms_step": 0.0877, "ms_step_trials": [0.0877] * 5,
            "matrices_per_s_fwd_bwd": 1.2e10}
    rows = [{"n": n, "batch": b, "dtype": d, "mode": m, "seed": 1, "input_sha256": "a" * 64, "grad_sha256": "b" * 64,
             "median_us": 20.0, "matrices_per_s": 1e9, "stock_gpu_us": 3000.0, "speedup_vs_stock": 150.0,
             "trials_us": [20.0] * 3, "stock_trials_us": [3000.0] * 3, "reference_a100_us": 22.83}
            for n in (4, 8, 16, 32) for b in (1, 128, 1024, 65536) for d in ("f32", "f16", "bf16")
            for m in ("forward", "forward_backward")]
    table = {"dtypes": ["f32"], "batches": [65536], "sizes": [4, 8, 16, 32], "method": "m", "reference_source": "r",
             "rows": rows}
    latency = {"unit": "us", "fh_forward": 7.3, "fh_forward_backward": 50.8, "native_forward": 500.0,
               "native_forward_backward": 1200.0, "trivial_op_forward_backward": 48.0, "shape": "[1,4,4] float32"}
    full = bench.full_report(Args, results, cold, table, latency, [{"n": 4}] * 40)
    rep = {"matrices": 1 << 20, "s_mismatches": 0, "s_max": 7, "nonfinite_matrices": 0,
           "bitwise_mismatches_vs_oracle": 0, "strict_failures_kernel": 0, "strict_failures_oracle": 0,
           "matrices_worse_than_reference": 0, "max_excess_over_reference": 0.0, "excess_unit": "ratio",
           "debug_launch_matches_op": True, "max_rel_frobenius": 1e-6, "mean_rel_frobenius": 1e-7,
           "oracle_mean_rel_frobenius": 1e-7}
    mixrep = {"tokens": 16384, "n": 4, "cols": 4096, "dtype": "bfloat16", "exp_bitwise_mismatches": 0,
              "dh_bitwise_mismatches": 0, "y_bound_violations": 0, "dx_bound_violations": 0,
              "de_bound_violations": 0}
    parity = {name: {"forward": dict(rep), "backward": dict(rep)} for name in ("c2", "c3", "c4", "c5", "c5f32", "p8")}
    parity.update({"hc": mixrep, "hc8": mixrep})
    full.update({
        "cpu_baseline": {"value": 2.18e6, "unit": "matrices/s", "cores": 16, "kind": "reference", "sample": "s" * 300,
                         "forward_value": 1e7, "trials_s": [0.5] * 3, "torch_threads": 16, "cpu_count": 256,
                         "affinity_cpus": 16, "physical_cores_host": 128, "cpu_model": "AMD EPYC"},
        "cpu_oracle_port": {"value": 3.05e5, "unit": "matrices/s", "cores": 1, "kind": "port", "sample": "p"},
        "parity": {"pass": True, "failures": {}, "configs": parity, "rule": "r" * 500},
    })
    return bench, full


def test_stdout_line_is_compact_and_carries_the_required_keys():
    """The driver parses the last stdout line from a bounded tail: the line must stay far below
    that (8 KB) with every optional block present, and keep the required keys, the roofline and
    the CPU baseline."""
    import json

    bench, full = _canned_full()
    assert len(json.dumps(full)) > 20000  # the full report alone would not fit
    line = bench.compact_line(full)
    text = json.dumps(line)
    assert len(text) < 8000, len(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype", "config",
                "roofline", "cpu_baseline", "higher_is_better", "scaling", "vs_baseline", "data"):
        assert key in line, key
    assert line["steps"] == 20 and line["warmup"] == 5 and line["n_gpus"] == 1
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in line["roofline"], key
    assert line["roofline"]["frac"] == pytest.approx(3909.2 / 8000, rel=1e-3)
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in line["cpu_baseline"], key
    assert line["cold_step"]["step_roofline_frac"] == pytest.approx(0.566 * 0.0742 / 0.0877, rel=1e-3)
    assert line["parity"]["pass"] is True and set(line["parity"]["configs"]) >= {"c2", "c3", "c4", "c5", "hc"}
    assert set(line["configs"]) >= {"c2", "c3", "c4", "c5", "c5f32", "p8", "hc", "hc8"}
    assert json.loads(text) == line


def test_stdout_line_drops_optional_blocks_rather_than_outgrow_the_limit():
    import json

    bench, full = _canned_full()
    full["parity"]["failures"] = {f"c{i}.forward": "x" * 1000 for i in range(50)}
    full["configs"].update({f"extra{i}": full["configs"]["c2"] for i in range(200)})
    line = bench.compact_line(full)
    assert len(json.dumps(line)) <= bench.LINE_LIMIT
    assert "roofline" in line and "cpu_baseline" in line and line["parity"]["pass"] is True
