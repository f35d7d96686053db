"""Throughput of the batched small-matrix exponential (forward + Frechet backward) on one MI355X.

Headline (``value``): BASELINE config 2 -- [1048576, 4, 4] FP32, entries N(0, 0.25^2),
upstream gradient N(0, 1); one step = ``fh.matrix_exp`` forward plus
``torch.autograd.grad`` backward over the whole batch, inputs resident in HBM.
Metric: matrices per second of forward + backward.

Also reported in the same JSON line:
* ``roofline`` -- the dominant kernel of that step (the P = 4 Frechet kernel),
  algorithmic bytes per launch / its mean launch time from HIP events on the
  stream it runs on, against MI355X's 8 TB/s;
* ``cpu_baseline`` -- the CPU restatement (oracle/, scalar C, one thread) over
  the same workload; ``cpu_native_torch`` -- native torch.linalg.matrix_exp +
  autograd on the host cores (the reference's own CPU path), on a sample;
* ``configs`` -- configs 3-5 (BF16 N=4 sweep, strided FP32 N=16, FP16 N=32 and
  the same shape in FP32) with their own rooflines (HBM for N=4, FP32 MFMA for
  N>=16, where the flop count uses each matrix's own squaring count);
* ``reference_table`` -- the reference's own benchmark (N = 4, 8, 16, 32 at
  B = 65,536 FP32, wall time per direct-API call) beside its published A100
  figures; ``small_batch_latency`` -- B = 1 wall time per call.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--only c2]
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "flash-hyperconnections_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
METRIC = "matrices/sec fwd+bwd (N=4 B=2^20, N=32 B=32768); % HBM/MFMA roofline"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_inputs(name: str, torch, device):
    """Seeded synthetic inputs per BASELINE configs 2-5 (seed 0; base, then per-matrix scale, then grad)."""
    torch.manual_seed(0)
    if name == "c2":
        b, n = 1 << 20, 4
        x = torch.randn(b, n, n) * 0.25
        g = torch.randn(b, n, n)
        dtype, layout = torch.float32, "contiguous"
    elif name == "c3":
        b, n = 1 << 20, 4
        base = torch.randn(b, n, n)
        base = base / torch.linalg.matrix_norm(base, ord=1)[:, None, None]
        x = base * (10 ** torch.empty(b).uniform_(-3, 2))[:, None, None]
        g = torch.randn(b, n, n)
        dtype, layout = torch.bfloat16, "contiguous"
    elif name == "c4":
        b, n = 65536, 16
        base = torch.randn(b, n, n) / 4 * (10 ** torch.empty(b).uniform_(-1, 1))[:, None, None]
        x = base
        g = torch.randn(b, n, n)
        dtype, layout = torch.float32, "transposed view"
    elif name == "c2s8":
        # Not a BASELINE config: one GPU's share of config 2 sharded over 8 GPUs (B / 8).
        b, n = 1 << 17, 4
        x = torch.randn(b, n, n) * 0.25
        g = torch.randn(b, n, n)
        dtype, layout = torch.float32, "contiguous"
    elif name == "p8":
        # Not a BASELINE config: the P = 8 kernel (n = 5..8) at [262144, 8, 8] FP32, same
        # per-matrix scale law as config 5.
        b, n = 1 << 18, 8
        x = torch.randn(b, n, n) / n**0.5 * (10 ** torch.empty(b).uniform_(-1, 1))[:, None, None]
        g = torch.randn(b, n, n)
        dtype, layout = torch.float32, "contiguous"
    elif name in ("c5", "c5f32"):
        b, n = 32768, 32
        x = torch.randn(b, n, n) / n**0.5 * (10 ** torch.empty(b).uniform_(-1, 1.5))[:, None, None]
        g = torch.randn(b, n, n)
        dtype, layout = (torch.float16 if name == "c5" else torch.float32), "contiguous"
    else:
        raise ValueError(name)
    x = x.to(dtype).to(device)
    g = g.to(dtype).to(device)
    if layout == "transposed view":
        x = x.transpose(-1, -2)  # noncontiguous input, as BASELINE config 4 specifies
    return x, g, layout


def sha256(t) -> str:
    import torch

    return hashlib.sha256(t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes()).hexdigest()


def time_loop(torch, fn, iters: int, warmup: int) -> float:
    """Mean ms per call of fn(), HIP events on the current stream (where the kernels launch)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def measure_config(name: str, torch, fh, steps: int, warmup: int, device) -> dict:
    x, g, layout = make_inputs(name, torch, device)
    b, n = x.shape[0], x.shape[-1]
    e = x.element_size()
    xin = x.detach().requires_grad_()

    def step():
        y = fh.matrix_exp(xin)
        return torch.autograd.grad(y, xin, g)[0]

    fwd = torch.ops.flash_hypercons._matrix_exp
    bwd = torch.ops.flash_hypercons._frechet
    xt = x.detach().mT
    ms_step = time_loop(torch, step, steps, warmup)
    ms_fwd = time_loop(torch, lambda: fwd(x), steps, warmup)
    ms_bwd = time_loop(torch, lambda: bwd(xt, g), steps, warmup)

    # Graph-captured step (launch overhead removed): same kernels, replayed.
    ms_graph = None
    try:
        gstream = torch.cuda.Stream()
        gstream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(gstream):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(gstream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        ms_graph = time_loop(torch, graph.replay, steps, 2)
    except Exception as exc:  # pragma: no cover - reported, not fatal
        log(f"[bench] graph capture of {name} failed: {exc}")

    params_f, _ = torch.ops.flash_hypercons._expm_params(x)
    params_b, _ = torch.ops.flash_hypercons._expm_params(xt, g)
    s_f = params_f[:, 1].clamp_min(0).double()
    s_b = params_b[:, 1].clamp_min(0).double()
    bytes_fwd = b * n * n * 2 * e
    bytes_bwd = b * n * n * 3 * e
    flops_fwd = float(((5 + s_f) * 2 * n**3).sum())
    flops_bwd = float(((5 + s_b) * 3 * 2 * n**3).sum())
    # Roofline time = max(bytes / HBM peak, flops / FP32 matrix peak), per kernel and per step.
    def ideal(nbytes, nflops):
        t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e9), nflops / (MFMA_F32_PEAK_TFLOPS * 1e12)
        return ("hbm", t_hbm) if t_hbm >= t_mfma else ("mfma", t_mfma)

    bound, t_ideal = ideal(bytes_fwd + bytes_bwd, flops_fwd + flops_bwd)
    bound_fwd, t_fwd = ideal(bytes_fwd, flops_fwd)
    bound_bwd, t_bwd = ideal(bytes_bwd, flops_bwd)
    out = {
        "shape": [b, n, n],
        "dtype": str(x.dtype).replace("torch.", ""),
        "layout": layout,
        "matrices_per_s_fwd_bwd": b / (ms_step * 1e-3),
        "ms_step": ms_step,
        "ms_step_graph": ms_graph,
        "ms_fwd_kernel": ms_fwd,
        "ms_bwd_kernel": ms_bwd,
        "mean_s_fwd": float(s_f.mean()),
        "mean_s_bwd": float(s_b.mean()),
        "bound": bound,
        "roofline_frac_step": t_ideal / (ms_step * 1e-3),
        "fwd_kernel": {
            "bound": bound_fwd,
            "achieved_gbs": bytes_fwd / (ms_fwd * 1e-3) / 1e9,
            "achieved_tflops": flops_fwd / (ms_fwd * 1e-3) / 1e12,
            "frac": t_fwd / (ms_fwd * 1e-3),
        },
        "bwd_kernel": {
            "bound": bound_bwd,
            "achieved_gbs": bytes_bwd / (ms_bwd * 1e-3) / 1e9,
            "achieved_tflops": flops_bwd / (ms_bwd * 1e-3) / 1e12,
            "frac": t_bwd / (ms_bwd * 1e-3),
        },
        "input_sha256": sha256(x)[:16],
        "grad_sha256": sha256(g)[:16],
    }
    del xin, x, g, xt
    return out


def profiled_traffic(key: str):
    """HBM bytes per launch of a kernel from a committed rocprofv3 counter summary (or None)."""
    path = ROOT / "profiles" / "expm_p4_c2_hbm_traffic.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch " + key + " = "):
                return int(line.rsplit("=", 1)[1])
    except OSError:
        pass
    return None


def cpu_oracle_baseline(torch) -> dict:
    """The CPU restatement (scalar C, 1 thread) over the full config-2 workload."""
    import numpy as np

    import oracle

    x, g, _ = make_inputs("c2", torch, "cpu")
    xf = oracle.tensor_to_f32(x)
    gf = oracle.tensor_to_f32(g)
    xt = np.ascontiguousarray(xf.transpose(0, 2, 1))
    t0 = time.perf_counter()
    oracle.matrix_exp_f32(xf)
    oracle.matrix_exp_f32(xt, gf)
    dt = time.perf_counter() - t0
    return {
        "value": x.shape[0] / dt,
        "unit": "matrices/s",
        "cores": 1,
        "kind": "port",
        "sample": f"all {x.shape[0]} config-2 matrices, forward + Frechet backward, oracle/fh_oracle.c "
        f"(scalar C restatement, one thread), {dt:.2f} s",
    }


def cpu_native_torch(torch, sample: int = 1 << 18) -> dict:
    """Native torch.linalg.matrix_exp + autograd on host cores (the reference's CPU path)."""
    x, g, _ = make_inputs("c2", torch, "cpu")
    x = x[:sample].clone().requires_grad_()
    g = g[:sample].clone()
    threads = torch.get_num_threads()
    y = torch.linalg.matrix_exp(x[:1024])  # warm
    torch.autograd.grad(y.sum(), x)
    times, fwd_times = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        with torch.no_grad():
            torch.linalg.matrix_exp(x)
        fwd_times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        y = torch.linalg.matrix_exp(x)
        torch.autograd.grad(y, x, g)
        times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": sample / dt,
        "forward_value": sample / statistics.median(fwd_times),
        "unit": "matrices/s",
        "cores": threads,
        "cpu_count": os.cpu_count(),
        "cpu_model": model,
        "sample": f"first {sample} config-2 matrices, torch.linalg.matrix_exp + autograd.grad "
        f"(value) and forward alone (forward_value), median of 3",
    }


def small_batch_latency(torch, fh, device, iters: int = 400) -> dict:
    """Host-bound latency at B=1, N=4 FP32 (the reference's small-batch comparison): wall time
    per call, including launch and the autograd engine, averaged over back-to-back calls."""
    x = torch.randn(1, 4, 4, device=device) * 0.25
    g = torch.randn(1, 4, 4, device=device)
    xg = x.clone().requires_grad_()

    def per_call(fn):
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / iters * 1e6

    return {
        "unit": "us",
        "fh_forward": per_call(lambda: fh.matrix_exp(x)),
        "fh_forward_backward": per_call(lambda: torch.autograd.grad(fh.matrix_exp(xg), xg, g)),
        "native_forward": per_call(lambda: torch.linalg.matrix_exp(x)),
        "native_forward_backward": per_call(lambda: torch.autograd.grad(torch.linalg.matrix_exp(xg), xg, g)),
        "trivial_op_forward_backward": per_call(lambda: torch.autograd.grad(xg * 2.0, xg, g)),
        "shape": "[1,4,4] float32",
    }


# The reference's published table (VALIDATION.md:84-95): A100 80GB PCIe, FP32, B = 65,536,
# median wall time per direct-API call in microseconds.
REFERENCE_A100_US = {
    (4, "forward"): 22.83, (4, "forward_backward"): 164.22,
    (8, "forward"): 58.21, (8, "forward_backward"): 208.52,
    (16, "forward"): 370.30, (16, "forward_backward"): 1208.46,
    (32, "forward"): 1948.02, (32, "forward_backward"): 8723.40,
}


def reference_table(torch, fh, device, batch: int = 65536, warmup: int = 5, repeat: int = 10, trials: int = 3) -> dict:
    """The reference's own benchmark on this GPU (its benchmarks/matrix_exp.py:75-105 method):
    seeded inputs randn*0.1 and grads randn*0.2, FP32, B = 65,536; per mode, warmup calls, then
    trials of back-to-back direct-API calls with synchronization at trial boundaries only; median
    of the per-call trial means.  Wall time includes Python selection, allocation and autograd."""
    rows = []
    for n in (4, 8, 16, 32):
        seed = 9041 + n * 1000003 + batch * 3
        torch.manual_seed(seed)
        a = torch.randn(batch, n, n, device=device) * 0.1
        g = torch.randn_like(a) * 0.2
        for mode in ("forward", "forward_backward"):
            x = a.detach().requires_grad_(mode == "forward_backward")

            def call(x=x, mode=mode):
                y = fh.matrix_exp(x)
                if mode == "forward_backward":
                    return torch.autograd.grad(y, x, g)[0]
                return y

            for _ in range(warmup):
                call()
            times = []
            for _ in range(trials):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(repeat):
                    call()
                torch.cuda.synchronize()
                times.append((time.perf_counter() - t0) * 1e6 / repeat)
            us = statistics.median(times)
            ref = REFERENCE_A100_US[(n, mode)]
            rows.append({"n": n, "mode": mode, "median_us": us, "matrices_per_s": batch / us * 1e6,
                         "reference_a100_us": ref, "reference_time_over_ours": ref / us})
    return {"batch": batch, "dtype": "f32", "method": f"{warmup} warmup, {trials} trials x {repeat} calls, median",
            "reference_source": "reference VALIDATION.md:84-95 (A100 80GB PCIe)", "rows": rows}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baselines")
    ap.add_argument("--only", default=None, help="comma list of configs (c2,c3,c4,c5,c5f32,p8,c2s8)")
    ap.add_argument("--extras", action="store_true",
                    help="with --only: also run the reference table and the small-batch latency")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one device copy of exactly 64 MiB (profiler counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: the operator has no cross-GPU step (every matrix is independent; "
            f"B shards contiguously with no exchange), and this build runs on single-GPU boxes. "
            f"--gpus {args.gpus} is not supported.",
            file=sys.stderr,
        )
        return 2
    import torch

    import flash_hypercons as fh

    device = torch.device("cuda:0")
    if args.calibrate_copy:
        # A plain copy of known size: reads and writes exactly 64 MiB.
        src = torch.ones(16 << 20, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    configs = (args.only or "c2,c3,c4,c5,c5f32,p8,c2s8").split(",")
    results = {}
    for name in configs:
        log(f"[bench] {name} ...")
        results[name] = measure_config(name, torch, fh, args.steps, args.warmup, device)
        log(f"[bench] {name}: {json.dumps(results[name])}")
        torch.cuda.empty_cache()

    head = results.get("c2")
    table = latency = None
    if args.only is None or args.extras:
        # Not part of --only runs, so that a profile of one config holds only its own launches.
        log("[bench] reference table ...")
        table = reference_table(torch, fh, device)
        for row in table["rows"]:
            log(f"[bench] reference table: n={row['n']:2} {row['mode']:16} {row['median_us']:9.1f} us "
                f"(A100 {row['reference_a100_us']:8.1f} us, x{row['reference_time_over_ours']:.2f})")
        log("[bench] small-batch latency ...")
        latency = small_batch_latency(torch, fh, device)
        log(f"[bench] small-batch latency: {json.dumps(latency)}")
    line = {
        "metric": METRIC,
        "value": head["matrices_per_s_fwd_bwd"] if head else None,
        "unit": "matrices/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_step"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, BASELINE config 2 distribution)",
        "config": {
            "workload": "BASELINE config 2: fh.matrix_exp forward + autograd backward on [1048576,4,4] FP32, "
            "x ~ N(0,0.25^2), grad ~ N(0,1)",
            "global_batch": 1 << 20,
            "n": 4,
            "parallelism": "single GPU",
        },
    }
    if head:
        b = 1 << 20
        bytes_bwd = b * 16 * 3 * 4
        achieved = head["bwd_kernel"]["achieved_gbs"]
        line["roofline"] = {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic("expm_p4_frechet_c2_f32"),
            "traffic_source": "profiles/expm_p4_c2_hbm_traffic.md (FETCH_SIZE, WRITE_SIZE; copy-calibrated)",
            "kernel": "expm_p4_kernel<F32, Pair=true> (Frechet backward, P=4)",
            "algorithmic_bytes_per_launch": bytes_bwd,
            "mean_launch_ms": head["ms_bwd_kernel"],
        }
        line["step_roofline_frac"] = head["roofline_frac_step"]
    if not args.skip_cpu:
        log("[bench] cpu baselines ...")
        line["cpu_baseline"] = cpu_oracle_baseline(torch)
        line["cpu_native_torch"] = cpu_native_torch(torch)
    if latency is not None:
        line["small_batch_latency"] = latency
        line["reference_table"] = table
    line["configs"] = results
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
