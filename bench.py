"""Throughput of the batched small-matrix exponential (forward + Frechet backward) on one MI355X.

Headline (``value``): BASELINE config 2 -- [1048576, 4, 4] FP32, entries N(0, 0.25^2),
upstream gradient N(0, 1); one step = ``fh.matrix_exp`` forward plus
``torch.autograd.grad`` backward over the whole batch, inputs resident in HBM.
Metric: matrices per second of forward + backward.  The K timed steps run as one
sequence bracketed by device synchronisations, split into >= 5 consecutive trials
by HIP events on the stream the kernels run on; ``ms_per_step`` is the median over
the trials of the per-step time (every trial's time is kept in ``trials_ms``).  Before
its W warmup steps each config runs its step untimed for ``--settle`` seconds
(default 0.3 s), so that the device has left its idle clocks when timing starts.

stdout carries ONE compact JSON line (well under 8 KB: the required keys, ``roofline``,
``cpu_baseline``, ``cold_step`` and one short summary per config and per parity gate); the
full report -- every field below with every trial -- goes to stderr and to ``--report``
(default gpurun_out/bench_report.json), as the reference's benchmark writes its report to a
file (benchmarks/matrix_exp.py:119-125).

Reported (in full in the report, summarised in the line):
* ``roofline`` -- the dominant kernel of that step (the P = 4 Frechet kernel):
  algorithmic bytes per launch / its median launch time (HIP events around
  back-to-back launches, same trial split) against MI355X's 8 TB/s;
* ``cold_step`` -- the same step cycling through 4 input/gradient sets
  (512 MiB of inputs, more than the 256 MB Infinity Cache), so that no launch
  finds its operands in the last-level cache;
* ``cpu_baseline`` -- the reference's CPU path (its ``matrix_exp`` falls through
  to native ``torch.linalg.matrix_exp`` on CPU tensors, backward by autograd)
  over ALL config-2 matrices on the host threads this process may use;
  ``cpu_oracle_port`` -- the C restatement (oracle/, one thread) over the same
  workload, whose results feed ``parity``;
* ``parity`` -- per config, over every matrix: squaring counts against the
  restatement, bitwise mismatches, strict north-star failures of the kernels
  and of the restatement, the kernels' error relative to the restatement's
  (tests/fullsize.py), all computed after the timed region;
* ``configs`` -- configs 3-5 (BF16 N=4 sweep, strided FP32 N=16, FP16 N=32 and
  the same shape in FP32) plus ``p8`` / ``c2s8`` with their own rooflines (HBM
  bytes at 8 TB/s, product flops from each matrix's own squaring count at the
  FP32 matrix peak), and ``hc`` -- the fused stream mixing ``fh.mix_streams``
  (y = exp(h) x, 16,384 tokens x 4 streams x 4,096 columns, BF16) forward and
  forward + backward, each fused kernel against the HBM roofline, beside the
  composed ``fh.matrix_exp(h) @ x`` on the same inputs;
* ``reference_table`` -- the reference's own benchmark (N = 4, 8, 16, 32 at
  B = 65,536 FP32, wall time per direct-API call; with ``--sweep`` its whole
  grid, B in {1, 128, 1024, 65536} x FP32/FP16/BF16, with seeds and input
  hashes per row) beside its published A100 figures; ``stock_gpu`` -- native
  torch.linalg.matrix_exp + autograd on this GPU in the same sweep;
  ``small_batch_latency`` -- B = 1 wall time per call.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--trials T] [--settle S] [--skip-cpu]
                       [--only c2,...] [--extras] [--sweep] [--report PATH]
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "flash-hyperconnections_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
VALU_F32_UNPACKED_TFLOPS = 78.6  # 256 CUs x 4 SIMDs x 16 lanes x 2 flops x 2.4 GHz (packed FP32 is not used)
METRIC = "matrices/sec fwd+bwd (N=4 B=2^20, N=32 B=32768); % HBM/MFMA roofline"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_inputs(name: str, torch, device, seed: int = 0):
    """Seeded synthetic inputs per BASELINE configs 2-5 (seed 0 unless given; base, then per-matrix
    scale, then grad)."""
    torch.manual_seed(seed)
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


def split_trials(total: int, trials: int) -> list[int]:
    """Sizes of `trials` consecutive trials covering exactly `total` steps (>= 1 each)."""
    trials = max(1, min(trials, total))
    base, extra = divmod(total, trials)
    return [base + (1 if i < extra else 0) for i in range(trials)]


def time_trials(torch, fn, steps: int, warmup: int, trials: int) -> dict:
    """`warmup` untimed calls, then exactly `steps` timed calls bracketed by
    torch.cuda.synchronize(), split into trials that are consecutive segments of that one run: a
    HIP event on the current stream (the one the kernels launch on) between segments, no
    synchronisation inside.  A trial thus measures the device time of its calls with the host
    queueing ahead, as in a training loop, rather than the host's latency to the first launch on
    an idle queue, which a synchronise per trial would add to every trial (~25 us on a slow host,
    a quarter of a config-2 step over 4-step trials).  Returns the median and every trial's ms per
    call; `mean_ms` is the whole run's."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    sizes = split_trials(steps, trials)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(len(sizes) + 1)]
    torch.cuda.synchronize()
    events[0].record(stream)
    for i, size in enumerate(sizes):
        for _ in range(size):
            fn()
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    per_call = [events[i].elapsed_time(events[i + 1]) / size for i, size in enumerate(sizes)]
    return {"median_ms": statistics.median(per_call), "trials_ms": per_call,
            "mean_ms": events[0].elapsed_time(events[-1]) / steps}


def settle(torch, fn, seconds: float) -> int:
    """Run fn back to back for about `seconds` of wall time, untimed, then synchronise: brings
    the device from idle to the clocks it holds under sustained load before anything is timed
    (measured: the first ~0.1 s of a config's steps ran 5-25% slower than the rest).  Returns the
    number of calls."""
    if seconds <= 0:
        return 0
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        calls += 8
        torch.cuda.synchronize()
    return calls


SETTLE_S = 0.3  # set from --settle in main()


def kernel_launches(steps: int, trials: int) -> int:
    """Launches of a single-kernel loop: at least 25 per trial, so that the queue runs ahead of the
    host and a trial's time is the kernels' own (its first launch's latency amortised)."""
    return max(steps, 25 * max(1, trials))


def roofline_times(nbytes: float, nflops: float, compute_peak_tflops: float):
    """(bound, seconds) of max(bytes / HBM peak, flops / compute peak)."""
    t_hbm, t_cmp = nbytes / (HBM_PEAK_GBS * 1e9), nflops / (compute_peak_tflops * 1e12)
    return ("hbm", t_hbm) if t_hbm >= t_cmp else ("mfma", t_cmp)


def measure_config(name: str, torch, fh, steps: int, warmup: int, trials: int, device, keep: bool) -> tuple[dict, dict]:
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
    settle(torch, step, SETTLE_S)
    t_step = time_trials(torch, step, steps, warmup, trials)
    t_fwd = time_trials(torch, lambda: fwd(x), kernel_launches(steps, trials), warmup, trials)
    t_bwd = time_trials(torch, lambda: bwd(xt, g), kernel_launches(steps, trials), warmup, trials)
    ms_step, ms_fwd, ms_bwd = t_step["median_ms"], t_fwd["median_ms"], t_bwd["median_ms"]

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
        ms_graph = time_trials(torch, graph.replay, steps, 2, trials)["median_ms"]
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
    peak = MFMA_F32_PEAK_TFLOPS
    bound, t_ideal = roofline_times(bytes_fwd + bytes_bwd, flops_fwd + flops_bwd, peak)
    bound_fwd, t_f = roofline_times(bytes_fwd, flops_fwd, peak)
    bound_bwd, t_b = roofline_times(bytes_bwd, flops_bwd, peak)
    out = {
        "shape": [b, n, n],
        "dtype": str(x.dtype).replace("torch.", ""),
        "layout": layout,
        "matrices_per_s_fwd_bwd": b / (ms_step * 1e-3),
        "ms_step": ms_step,
        "ms_step_trials": t_step["trials_ms"],
        "ms_step_graph": ms_graph,
        "ms_fwd_kernel": ms_fwd,
        "ms_bwd_kernel": ms_bwd,
        "ms_fwd_trials": t_fwd["trials_ms"],
        "ms_bwd_trials": t_bwd["trials_ms"],
        "mean_s_fwd": float(s_f.mean()),
        "mean_s_bwd": float(s_b.mean()),
        "bound": bound,
        "roofline_frac_step": t_ideal / (ms_step * 1e-3),
        "fwd_kernel": {
            "bound": bound_fwd,
            "achieved_gbs": bytes_fwd / (ms_fwd * 1e-3) / 1e9,
            "achieved_tflops": flops_fwd / (ms_fwd * 1e-3) / 1e12,
            "frac": t_f / (ms_fwd * 1e-3),
        },
        "bwd_kernel": {
            "bound": bound_bwd,
            "achieved_gbs": bytes_bwd / (ms_bwd * 1e-3) / 1e9,
            "achieved_tflops": flops_bwd / (ms_bwd * 1e-3) / 1e12,
            "frac": t_b / (ms_bwd * 1e-3),
        },
        "input_sha256": sha256(x)[:16],
        "grad_sha256": sha256(g)[:16],
    }
    if n <= 4:
        # P = 4 runs on the (unpacked) FP32 VALU: report against that peak as well.
        _, t_valu = roofline_times(bytes_fwd + bytes_bwd, flops_fwd + flops_bwd, VALU_F32_UNPACKED_TFLOPS)
        out["roofline_frac_step_unpacked_valu_peak"] = t_valu / (ms_step * 1e-3)
    kept = {}
    if keep:
        y = fh.matrix_exp(xin)
        (grad,) = torch.autograd.grad(y, xin, g)
        kept = {"x": x.detach(), "g": g, "y": y.detach(), "grad": grad}
    del xin
    return out, kept


MIX_SHAPE = (16384, 4, 4096)  # tokens, streams, columns


def make_mix_inputs(torch, device, shape=MIX_SHAPE, dtype=None, seed: int = 0):
    """Seeded inputs of the fused stream mixing: per token an n x n generator h ~ N(0, 0.25^2)
    (config 2's law) and n residual streams x ~ N(0, 1) of width C; upstream gradient N(0, 1)."""
    dtype = dtype or torch.bfloat16
    tokens, n, cols = shape
    gen = torch.Generator(device=device).manual_seed(seed)
    h = (torch.randn(tokens, n, n, device=device, generator=gen) * 0.25).to(dtype)
    x = torch.randn(tokens, n, cols, device=device, generator=gen).to(dtype)
    g = torch.randn(tokens, n, cols, device=device, generator=gen).to(dtype)
    return h, x, g


MIX_WIDE_SHAPE = (16384, 8, 4096)  # the 8-stream case: exp(h) from the P = 8 kernel, then apply


def measure_mix(torch, fh, steps: int, warmup: int, trials: int, device, keep: bool,
                shape=MIX_SHAPE) -> tuple[dict, dict]:
    """``fh.mix_streams`` against the composed ``fh.matrix_exp(h) @ x`` (exp kernel, then torch's
    batched product) on the same inputs: the forward alone, and forward + autograd backward of
    both operands.  n <= 4: y = exp(h) x fused, one kernel per direction; HBM roofline of each
    from its algorithmic bytes (forward reads h and x and writes y; backward reads h, x and dy and
    writes dh and dx).  5 <= n <= 8: the streaming apply kernels (forward reads E in FP32 and x,
    writes y; backward reads E, x and dy, writes dx and dE in FP32), with the exponential and
    Frechet launches of the step on top."""
    h, x, g = make_mix_inputs(torch, device, shape=shape)
    tokens, n, cols = x.shape
    es = x.element_size()
    ops = torch.ops.flash_hypercons
    hr, xr = h.clone().requires_grad_(), x.clone().requires_grad_()
    wide = n > 4
    if wide:
        e = ops._matrix_exp(h.float())
        fwd_kernel, bwd_kernel = (lambda: ops._hc_apply(e, x)), (lambda: ops._hc_apply_backward(e, x, g))
        bytes_fwd = tokens * (4 * n * n + 2 * n * cols * es)
        bytes_bwd = tokens * (8 * n * n + 3 * n * cols * es)
        short = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[x.dtype]
        key = f"hc_apply_{{}}_{short}_n{n}"
        summary = "hc_apply_hbm_traffic.md"
    else:
        fwd_kernel, bwd_kernel = (lambda: ops._hc_mix(h, x)), (lambda: ops._hc_mix_backward(h, x, g))
        bytes_fwd = tokens * (n * n + 2 * n * cols) * es
        bytes_bwd = tokens * (2 * n * n + 3 * n * cols) * es
        key = "hc_mix_{}_bf16_n4"
        summary = "hc_mix_hbm_traffic.md"

    def fused_step():
        return torch.autograd.grad(fh.mix_streams(hr, xr), (hr, xr), g)

    def composed_step():
        return torch.autograd.grad(fh.matrix_exp(hr) @ xr, (hr, xr), g)

    settle(torch, fused_step, SETTLE_S)
    t_fwd = time_trials(torch, fwd_kernel, kernel_launches(steps, trials), warmup, trials)
    t_bwd = time_trials(torch, bwd_kernel, kernel_launches(steps, trials), warmup, trials)
    t_step = time_trials(torch, fused_step, steps, warmup, trials)
    t_cfwd = time_trials(torch, lambda: fh.matrix_exp(h) @ x, steps, warmup, trials)
    t_cstep = time_trials(torch, composed_step, steps, warmup, trials)
    ms_f, ms_b = t_fwd["median_ms"], t_bwd["median_ms"]
    out = {
        "workload": "fh.mix_streams: y = exp(h) @ x per token, h [T, n, n], x [T, n, C]",
        "path": "exp (P = 8 kernel) + streaming apply" if wide else "fused",
        "shape": [tokens, n, cols],
        "dtype": str(x.dtype).replace("torch.", ""),
        "tokens_per_s_fwd_bwd": tokens / (t_step["median_ms"] * 1e-3),
        "ms_step": t_step["median_ms"],
        "ms_step_trials": t_step["trials_ms"],
        "ms_fwd_kernel": ms_f,
        "ms_bwd_kernel": ms_b,
        "ms_fwd_trials": t_fwd["trials_ms"],
        "ms_bwd_trials": t_bwd["trials_ms"],
        "composed_ms_fwd": t_cfwd["median_ms"],
        "composed_ms_step": t_cstep["median_ms"],
        "composed_ms_step_trials": t_cstep["trials_ms"],
        "speedup_fwd_vs_composed": t_cfwd["median_ms"] / ms_f,
        "speedup_step_vs_composed": t_cstep["median_ms"] / t_step["median_ms"],
        "fwd_kernel": {"bound": "hbm", "algorithmic_bytes": bytes_fwd, "achieved_gbs": bytes_fwd / (ms_f * 1e-3) / 1e9,
                       "frac": bytes_fwd / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "traffic": profiled_traffic(key.format("fwd"), summary)},
        "bwd_kernel": {"bound": "hbm", "algorithmic_bytes": bytes_bwd, "achieved_gbs": bytes_bwd / (ms_b * 1e-3) / 1e9,
                       "frac": bytes_bwd / (ms_b * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "traffic": profiled_traffic(key.format("bwd"), summary)},
        "roofline_frac_step": (bytes_fwd + bytes_bwd) / (HBM_PEAK_GBS * 1e9) / (t_step["median_ms"] * 1e-3),
    }
    kept = {}
    if keep and wide:
        y = fh.mix_streams(h, x)
        dx, de = ops._hc_apply_backward(e, x, g)
        dh = torch.autograd.grad(fh.mix_streams(hr, xr), hr, g)[0]
        kept = {"h": h, "x": x, "g": g, "y": y, "e": e, "dx": dx, "dh": dh, "de": de}
    elif keep:
        y, _, e = ops._hc_mix_aux(h, x, None)
        dx, dh, de = ops._hc_mix_aux(h, x, g)
        kept = {"h": h, "x": x, "g": g, "y": y, "e": e, "dx": dx, "dh": dh, "de": de}
    del hr, xr
    return out, kept


def mix_sweep(torch, fh, device, steps: int = 20, warmup: int = 3, trials: int = 5) -> list:
    """``fh.mix_streams`` (fused for n <= 4, exp(h) then one streaming kernel per direction for
    5 <= n <= 8) against the composed ``fh.matrix_exp(h) @ x`` over stream counts, widths and
    dtypes (forward and forward + backward, HIP-event medians)."""
    rows = []
    for dtype in (torch.bfloat16, torch.float32):
        for n in (2, 3, 4, 6, 8):
            for cols in (256, 1024, 4096, 7168):
                if dtype == torch.float32 and cols != 4096:
                    continue
                tokens = 16384
                h, x, g = make_mix_inputs(torch, device, shape=(tokens, n, cols), dtype=dtype)
                hr, xr = h.clone().requires_grad_(), x.clone().requires_grad_()
                fused_f = time_trials(torch, lambda: fh.mix_streams(h, x), steps, warmup, trials)["median_ms"]
                comp_f = time_trials(torch, lambda: fh.matrix_exp(h) @ x, steps, warmup, trials)["median_ms"]
                fused_s = time_trials(torch, lambda: torch.autograd.grad(fh.mix_streams(hr, xr), (hr, xr), g), steps,
                                      warmup, trials)["median_ms"]
                comp_s = time_trials(torch, lambda: torch.autograd.grad(fh.matrix_exp(hr) @ xr, (hr, xr), g), steps,
                                     warmup, trials)["median_ms"]
                es = x.element_size()
                fwd_bytes = tokens * (n * n + 2 * n * cols) * es
                rows.append({"tokens": tokens, "n": n, "cols": cols, "dtype": str(dtype).replace("torch.", ""),
                             "path": "fused" if n <= 4 else "exp + apply",
                             "fused_fwd_ms": fused_f, "composed_fwd_ms": comp_f, "fused_step_ms": fused_s,
                             "composed_step_ms": comp_s, "fused_fwd_gbs": fwd_bytes / (fused_f * 1e-3) / 1e9,
                             "step_speedup": comp_s / fused_s})
                log(f"[bench] mix sweep n={n} C={cols} {rows[-1]['dtype']}: fused {fused_f * 1e3:.1f} / "
                    f"{fused_s * 1e3:.1f} us, composed {comp_f * 1e3:.1f} / {comp_s * 1e3:.1f} us")
                del h, x, g, hr, xr
    return rows


def cold_step(torch, fh, steps: int, warmup: int, trials: int, device, sets: int = 4) -> dict:
    """Config 2's step cycling through `sets` distinct input/gradient sets (each 128 MiB), so the
    working set of consecutive steps exceeds the 256 MB last-level cache."""
    pairs = []
    for k in range(sets):
        if k == 0:
            x, g, _ = make_inputs("c2", torch, device)
        else:
            gen = torch.Generator(device=device).manual_seed(1000 + k)
            x = torch.randn(1 << 20, 4, 4, device=device, generator=gen) * 0.25
            g = torch.randn(1 << 20, 4, 4, device=device, generator=gen)
        pairs.append((x.detach().requires_grad_(), g))
    state = {"i": 0}

    def step():
        x, g = pairs[state["i"] % sets]
        state["i"] += 1
        y = fh.matrix_exp(x)
        return torch.autograd.grad(y, x, g)[0]

    t = time_trials(torch, step, steps, warmup, trials)
    b = pairs[0][0].shape[0]
    return {"sets": sets, "input_mib": sets * 2 * b * 16 * 4 / 2**20, "ms_step": t["median_ms"],
            "ms_step_trials": t["trials_ms"], "matrices_per_s_fwd_bwd": b / (t["median_ms"] * 1e-3)}


def profiled_traffic(key: str, summary: str = "expm_p4_c2_hbm_traffic.md"):
    """HBM bytes per launch of a kernel from a committed rocprofv3 counter summary (or None)."""
    path = ROOT / "profiles" / summary
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch " + key + " = "):
                return int(line.rsplit("=", 1)[1])
    except OSError:
        pass
    return None


def _cpu_model() -> tuple[str, int | None]:
    """lscpu model name and physical core count of the whole host (sockets x cores per socket)."""
    model, cores, sockets = "", None, None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            val = val.strip()
            if key.strip() == "Model name":
                model = val
            elif key.strip() == "Core(s) per socket":
                cores = int(val)
            elif key.strip() == "Socket(s)":
                sockets = int(val)
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    return model, (cores * sockets if cores and sockets else None)


def cpu_leg(torch, kept: dict, mix_kept: dict | None = None) -> dict:
    """The CPU side of the run, after every GPU timing: the reference's CPU path timed over all of
    config 2, the C restatement timed over the same workload, and the parity block built from the
    restatement's results (the restatement is the checker here, never the thing measured on the
    GPU)."""
    import numpy as np

    import oracle
    from tests.fullsize import check, direction_parity

    try:
        threads = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        threads = os.cpu_count() or 1
    threads = max(1, min(threads, 16))
    model, physical = _cpu_model()
    result = {}

    # 1. The reference's CPU path: native matrix_exp + autograd on every config-2 matrix.
    x, g, _ = make_inputs("c2", torch, "cpu")
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    xr = x.clone().requires_grad_()
    y = torch.linalg.matrix_exp(xr)  # warm-up call, full batch
    torch.autograd.grad(y, xr, g)
    times, fwd_times = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        with torch.no_grad():
            torch.linalg.matrix_exp(x)
        fwd_times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        y = torch.linalg.matrix_exp(xr)
        torch.autograd.grad(y, xr, g)
        times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    result["cpu_baseline"] = {
        "value": x.shape[0] / dt,
        "unit": "matrices/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": f"all {x.shape[0]} config-2 matrices: native torch.linalg.matrix_exp + torch.autograd.grad (the "
        f"reference's matrix_exp falls through to these on CPU tensors), 1 warm-up call, median of 3 trials "
        f"({dt:.2f} s per trial); forward alone {statistics.median(fwd_times):.3f} s",
        "forward_value": x.shape[0] / statistics.median(fwd_times),
        "trials_s": times,
        "torch_threads": torch.get_num_threads(),
        "cpu_count": os.cpu_count(),
        "affinity_cpus": threads,
        "physical_cores_host": physical,
        "cpu_model": model,
    }
    torch.set_num_threads(prev_threads)
    del xr, y

    # 2. The C restatement, one thread, same workload (forward + Frechet of x^T).
    xf = oracle.tensor_to_f32(x)
    gf = oracle.tensor_to_f32(g)
    xt = np.ascontiguousarray(xf.transpose(0, 2, 1))
    t0 = time.perf_counter()
    oracle.matrix_exp_f32(xf)
    oracle.matrix_exp_f32(xt, gf)
    dt = time.perf_counter() - t0
    result["cpu_oracle_port"] = {
        "value": x.shape[0] / dt, "unit": "matrices/s", "cores": 1, "kind": "port",
        "sample": f"all {x.shape[0]} config-2 matrices, forward + Frechet backward, oracle/fh_oracle.c (scalar C "
        f"restatement, one thread), {dt:.2f} s",
    }

    # 3. Parity over every matrix of every measured config.
    parity = {}
    for name, k in kept.items():
        t0 = time.perf_counter()
        parity[name] = {"forward": direction_parity(k["x"], None, k["y"], threads=threads),
                        "backward": direction_parity(k["x"].mT, k["g"], k["grad"], threads=threads)}
        log(f"[bench] parity {name} ({time.perf_counter() - t0:.1f} s): {json.dumps(parity[name])}")
    failures = {f"{name}.{d}": why for name, rep in parity.items() for d, r in rep.items()
                if (why := check(r, kept[name]["x"].shape[-1]))}
    for name, k in (mix_kept or {}).items():
        if not k:
            continue
        from tests.mixcheck import check_mix, mix_parity

        t0 = time.perf_counter()
        parity[name] = mix_parity(k["h"], k["x"], k["g"], k["y"], k["e"], k["dx"], k["dh"], k["de"], threads=threads)
        log(f"[bench] parity {name} ({time.perf_counter() - t0:.1f} s): {json.dumps(parity[name])}")
        if why := check_mix(parity[name]):
            failures[name] = why
    result["parity"] = {"pass": not failures, "failures": failures, "configs": parity,
                        "rule": "tests/fullsize.py check(): s == oracle for every matrix; n <= 8 bit-identical "
                        "to the oracle; n >= 9: strict north-star failures <= the oracle's + 3 sqrt(oracle's) "
                        "+ 3 and mean error <= 1.05x the oracle's; per-matrix excess over the oracle's error "
                        "under a sanity cap. hc, hc8 "
                        "(tests/mixcheck.py): exp(h) and dh bit-identical to the oracle, y / dx / dE within "
                        "the FP32 summation bound of the FP64 products, every token"}
    return result


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


def reference_table(torch, fh, device, sizes=(4, 8, 16, 32), batches=(65536,), dtypes=("f32",), warmup: int = 5,
                    repeat: int = 10, trials: int = 3) -> dict:
    """The reference's own benchmark on this GPU (its benchmarks/matrix_exp.py:75-105 method):
    seeded inputs randn*0.1 and grads randn*0.2; per (n, B, dtype, mode) and per implementation
    (this operator, and native torch.linalg.matrix_exp on the same GPU -- the reference's "stock"
    column, with FP16/BF16 promoted to FP32 and cast back as its benchmark does), warmup calls,
    then trials of back-to-back direct-API calls with synchronisation at trial boundaries only; the
    implementations alternate order per trial; median of the per-call trial means.  Wall time
    includes Python selection, allocation and autograd."""
    dt_map = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    rows = []

    def native(x):
        if x.dtype in (torch.float16, torch.bfloat16):
            return torch.linalg.matrix_exp(x.float()).to(x.dtype)
        return torch.linalg.matrix_exp(x)

    for dname in dtypes:
        dtype = dt_map[dname]
        for batch in batches:
            for n in sizes:
                seed = 9041 + n * 1000003 + batch * 3
                torch.manual_seed(seed)
                a = (torch.randn(batch, n, n, device=device) * 0.1).to(dtype)
                g = (torch.randn(batch, n, n, device=device) * 0.2).to(dtype)
                a_hash, g_hash = sha256(a), sha256(g)  # the whole tensors, as the reference records
                for mode in ("forward", "forward_backward"):
                    x = a.detach().requires_grad_(mode == "forward_backward")
                    impls = {"flash_hypercons": fh.matrix_exp, "stock": native}

                    def call(fn, x=x, mode=mode, g=g):
                        y = fn(x)
                        if mode == "forward_backward":
                            return torch.autograd.grad(y, x, g)[0]
                        return y

                    times = {k: [] for k in impls}
                    for k, fn in impls.items():
                        for _ in range(warmup):
                            call(fn)
                    order = list(impls)
                    for t in range(trials):
                        for k in (order if t % 2 == 0 else order[::-1]):
                            torch.cuda.synchronize()
                            t0 = time.perf_counter()
                            for _ in range(repeat):
                                call(impls[k])
                            torch.cuda.synchronize()
                            times[k].append((time.perf_counter() - t0) * 1e6 / repeat)
                    us = statistics.median(times["flash_hypercons"])
                    stock = statistics.median(times["stock"])
                    row = {"n": n, "batch": batch, "dtype": dname, "mode": mode, "seed": seed,
                           "input_sha256": a_hash, "grad_sha256": g_hash, "median_us": us,
                           "matrices_per_s": batch / us * 1e6, "stock_gpu_us": stock, "speedup_vs_stock": stock / us,
                           "trials_us": times["flash_hypercons"], "stock_trials_us": times["stock"]}
                    ref = REFERENCE_A100_US.get((n, mode)) if (dname == "f32" and batch == 65536) else None
                    if ref is not None:
                        row["reference_a100_us"] = ref
                        row["reference_time_over_ours"] = ref / us
                    rows.append(row)
                del a, g
    return {"dtypes": list(dtypes), "batches": list(batches), "sizes": list(sizes),
            "method": f"{warmup} warmup, {trials} trials x {repeat} calls, median, implementations alternating",
            "reference_source": "reference VALIDATION.md:84-95 (A100 80GB PCIe) and benchmarks/matrix_exp.py",
            "rows": rows}


HEADLINE_KERNEL = "expm_p4_dma_kernel<F32, true, 2, 1> (Frechet backward, P=4, buffer-to-LDS loads)"
LINE_LIMIT = 8000  # bytes: the stdout line must sit wholly inside a driver's captured tail


def full_report(args, results: dict, cold, table, latency, mix_rows) -> dict:
    """Everything the run measured, keyed as the compact line's fields plus the detail (every
    trial, every config's kernels, the reference table, the stream-mixing sweep)."""
    head = results.get("c2")
    full = {
        "metric": METRIC,
        "value": head["matrices_per_s_fwd_bwd"] if head else None,
        "unit": "matrices/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": args.settle,
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
        full["trials"] = len(head["ms_step_trials"])
        full["trials_ms"] = head["ms_step_trials"]
        full["roofline"] = {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic("expm_p4_frechet_c2_f32"),
            "traffic_source": "profiles/expm_p4_c2_hbm_traffic.md (FETCH_SIZE, WRITE_SIZE; copy-calibrated)",
            "kernel": HEADLINE_KERNEL,
            "algorithmic_bytes_per_launch": bytes_bwd,
            "median_launch_ms": head["ms_bwd_kernel"],
            "launch_trials_ms": head["ms_bwd_trials"],
        }
        full["step_roofline_frac"] = head["roofline_frac_step"]
        if cold is not None:
            full["cold_step"] = cold
            full["cold_over_warm"] = cold["ms_step"] / head["ms_step"]
            # Same algorithmic bytes, the step's time with no operand in the last-level cache.
            full["cold_step_roofline_frac"] = head["roofline_frac_step"] * head["ms_step"] / cold["ms_step"]
    if latency is not None:
        full["small_batch_latency"] = latency
        full["reference_table"] = table
    if mix_rows is not None:
        full["mix_sweep"] = mix_rows
    full["configs"] = results
    return full


def _r(v, digits: int = 4):
    """v rounded to `digits` significant digits (None and non-floats pass through)."""
    if isinstance(v, float) and v == v and v not in (float("inf"), float("-inf")) and v != 0.0:
        return float(f"{v:.{digits}g}")
    return v


def compact_line(full: dict) -> dict:
    """The stdout JSON line: the driver's required keys, the roofline and CPU baseline, and one
    short summary per config (step / forward / backward microseconds, roofline fraction) and per
    parity gate (counts only).  Bounded well under LINE_LIMIT bytes whatever the configs hold."""
    keys = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config")
    line = {k: full.get(k) for k in keys}
    line["value"], line["ms_per_step"] = _r(line["value"], 6), _r(line["ms_per_step"], 6)
    line["timing"] = (f"median of {full.get('trials', 0)} consecutive trials of the K timed steps (HIP events, "
                      f"one sync each side); each config first runs {full.get('settle_s')} s of untimed steps, "
                      f"then the W warmup steps")
    if "trials_ms" in full:
        line["trials_ms"] = [_r(t) for t in full["trials_ms"]]
    if "roofline" in full:
        rf = full["roofline"]
        line["roofline"] = {k: _r(rf[k]) for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")}
        line["roofline"]["traffic"] = rf["traffic"]  # bytes per launch, an integer
        line["roofline"]["kernel"] = rf["kernel"]
        line["roofline"]["algorithmic_bytes_per_launch"] = rf["algorithmic_bytes_per_launch"]
        line["roofline"]["median_launch_ms"] = _r(rf["median_launch_ms"])
        line["step_roofline_frac"] = _r(full.get("step_roofline_frac"), 3)
    if "cold_step" in full:
        line["cold_step"] = {"ms": _r(full["cold_step"]["ms_step"]), "sets": full["cold_step"]["sets"],
                             "step_roofline_frac": _r(full["cold_step_roofline_frac"], 3)}
    if "cpu_baseline" in full:
        cb = full["cpu_baseline"]
        line["cpu_baseline"] = {"value": _r(cb["value"]), "unit": cb["unit"], "cores": cb["cores"],
                                "kind": cb["kind"], "sample": cb["sample"][:400],
                                "cpu_model": (cb.get("cpu_model") or "")[:80]}
    if "cpu_oracle_port" in full:
        line["cpu_oracle_port"] = {"value": _r(full["cpu_oracle_port"]["value"]), "cores": 1, "kind": "port"}
    summary = {}
    for name, res in (full.get("configs") or {}).items():
        if "matrices_per_s_fwd_bwd" in res:
            summary[name] = {"us": [_r(res["ms_step"] * 1e3), _r(res["ms_fwd_kernel"] * 1e3),
                                    _r(res["ms_bwd_kernel"] * 1e3)],
                             "frac": _r(res["roofline_frac_step"], 3), "bound": res["bound"],
                             "rate": _r(res["matrices_per_s_fwd_bwd"], 3)}
        elif "tokens_per_s_fwd_bwd" in res:
            summary[name] = {"us": [_r(res["ms_step"] * 1e3), _r(res["ms_fwd_kernel"] * 1e3),
                                    _r(res["ms_bwd_kernel"] * 1e3)],
                             "frac": _r(res["roofline_frac_step"], 3), "bound": "hbm",
                             "rate": _r(res["tokens_per_s_fwd_bwd"], 3),
                             "composed_us": _r(res["composed_ms_step"] * 1e3)}
    if summary:
        line["configs"] = summary
        line["configs_fields"] = "us = [step, forward kernel, backward kernel]; frac = step roofline fraction"
    if "parity" in full:
        par = full["parity"]
        comp = {}
        for name, rep in par["configs"].items():
            if "forward" in rep:
                comp[name] = {d: [r["s_mismatches"], r["bitwise_mismatches_vs_oracle"], r["strict_failures_kernel"],
                                  r["strict_failures_oracle"], _r(r["max_excess_over_reference"], 3)]
                              for d, r in rep.items()}
            else:
                comp[name] = [rep.get(k) for k in ("exp_bitwise_mismatches", "dh_bitwise_mismatches",
                                                    "y_bound_violations", "dx_bound_violations", "de_bound_violations")]
        line["parity"] = {
            "pass": par["pass"],
            "failures": {k: str(v)[:200] for k, v in list(par["failures"].items())[:8]},
            "configs": comp,
            "fields": "matrices: [s mismatches, bitwise mismatches vs oracle, strict failures kernel, strict "
                      "failures oracle, max excess over the oracle's error]; mixing: [exp(h) bit mismatches, dh "
                      "bit mismatches, y / dx / dE bound violations]",
        }
    if full.get("small_batch_latency"):
        lat = full["small_batch_latency"]
        line["small_batch_latency_us"] = {k: _r(lat[k], 3) for k in (
            "fh_forward", "fh_forward_backward", "trivial_op_forward_backward", "native_forward_backward")}
    if full.get("reference_table"):
        rows = full["reference_table"]["rows"]
        line["reference_table_us"] = [[r["n"], r["batch"], r["dtype"], r["mode"][:3] if r["mode"] == "forward"
                                       else "f+b", _r(r["median_us"], 3), r.get("reference_a100_us")]
                                      for r in rows][:64]
    size = len(json.dumps(line))
    if size > LINE_LIMIT:  # never let the line outgrow the limit: drop the optional summaries
        for k in ("reference_table_us", "configs", "small_batch_latency_us", "trials_ms"):
            line.pop(k, None)
            if len(json.dumps(line)) <= LINE_LIMIT:
                break
    return line


def main() -> int:
    global SETTLE_S
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--trials", type=int, default=5, help="the K timed steps are split into this many trials")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="seconds of untimed steps per config before its W warmup steps (device clocks settle)")
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU leg (CPU baselines and parity)")
    ap.add_argument("--only", default=None, help="comma list of configs (c2,c3,c4,c5,c5f32,p8,c2s8,hc,hc8)")
    ap.add_argument("--extras", action="store_true",
                    help="with --only: also run the reference table and the small-batch latency")
    ap.add_argument("--sweep", action="store_true",
                    help="reference table over B in {1,128,1024,65536} x {f32,f16,bf16} (the reference's sweep), "
                    "and fused vs composed stream mixing over n and C")
    ap.add_argument("--report", default="gpurun_out/bench_report.json",
                    help="file (relative to the repo root) for the full JSON report; '' to skip")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one device copy of exactly 64 MiB (profiler counter calibration)")
    args = ap.parse_args()
    SETTLE_S = args.settle
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
    configs = (args.only or "c2,c3,c4,c5,c5f32,p8,c2s8,hc,hc8").split(",")
    results, kept, mix_kept = {}, {}, {}
    for name in configs:
        log(f"[bench] {name} ...")
        if name in ("hc", "hc8"):
            results[name], mix_kept[name] = measure_mix(torch, fh, args.steps, args.warmup, args.trials, device,
                                                        keep=not args.skip_cpu,
                                                        shape=MIX_SHAPE if name == "hc" else MIX_WIDE_SHAPE)
            log(f"[bench] {name}: {json.dumps(results[name])}")
            continue
        results[name], k = measure_config(name, torch, fh, args.steps, args.warmup, args.trials, device,
                                          keep=not args.skip_cpu and name != "c2s8")
        if k:
            kept[name] = k
        log(f"[bench] {name}: {json.dumps(results[name])}")

    head = results.get("c2")
    cold = None
    if head is not None:
        log("[bench] cold c2 step ...")
        cold = cold_step(torch, fh, args.steps, args.warmup, args.trials, device)
        log(f"[bench] cold c2 step: {json.dumps(cold)}")
    table = latency = mix_rows = None
    if args.only is None or args.extras or args.sweep:
        # Not part of --only runs, so that a profile of one config holds only its own launches.
        log("[bench] reference table ...")
        if args.sweep:
            table = reference_table(torch, fh, device, batches=(1, 128, 1024, 65536), dtypes=("f32", "f16", "bf16"))
        else:
            # Longer trials than the reference's 10 calls: at N <= 8 a call is host-bound and 10
            # calls leave the median at the mercy of one slow launch.
            table = reference_table(torch, fh, device, repeat=40, trials=5)
        for row in table["rows"]:
            log(f"[bench] reference table: n={row['n']:2} B={row['batch']:6} {row['dtype']:4} {row['mode']:16} "
                f"{row['median_us']:9.1f} us (stock GPU {row['stock_gpu_us']:9.1f} us)")
        if args.sweep:
            log("[bench] stream-mixing sweep ...")
            mix_rows = mix_sweep(torch, fh, device)
        log("[bench] small-batch latency ...")
        latency = small_batch_latency(torch, fh, device)
        log(f"[bench] small-batch latency: {json.dumps(latency)}")
    full = full_report(args, results, cold, table, latency, mix_rows)
    if not args.skip_cpu:
        log("[bench] cpu leg ...")
        leg = cpu_leg(torch, kept, mix_kept)
        full.update(leg)
    line = compact_line(full)
    # The whole report (every trial, every config's kernels, full parity reports, the reference
    # table) goes to a file and to stderr; stdout carries one compact line.
    text = json.dumps(full)
    log("[bench] full report: " + text)
    if args.report:
        report = Path(args.report) if Path(args.report).is_absolute() else ROOT / args.report
        try:
            report.parent.mkdir(parents=True, exist_ok=True)
            report.write_text(text + "\n")
            line["report"] = args.report
        except OSError as exc:
            log(f"[bench] could not write {args.report}: {exc}")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
