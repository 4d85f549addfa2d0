#!/usr/bin/env python3
"""Benchmark of the fused kernel library on one MI355X. It reports:
  * HBM GB/s of RMSNorm and GEGLU fwd+bwd;
  * TFLOP/s of relative-position flash attention fwd+bwd.
Each is also given as a fraction of the MI355X roofline. The reference's eager torch path is
timed on the host CPU beside it.

    python bench.py [--steps K] [--warmup W] [--only LIST] [--no-cpu] [--cpu-seconds S]

LIST is comma-separated from: relpos, relpos_fwd, relpos_fp16, relpos_fp32, relpos_long, rmsnorm,
geglu, geglu_linear, selftest_shapes, config1, bucket (default: all).

A "step" is one forward + backward pass of a kernel over one batch of synthetic input that is
already resident in HBM (3 and 5; config 4 is the forward-only attention
line). Prints ONE JSON line. `value` is the relpos attention fwd+bwd TFLOP/s (the dominant
kernel); `components` holds every workload's own figure and roofline.

Cache-cold protocol: every workload rotates through independent input sets. Their total
exceeds 3 x (L2 + MALL) = 3 x (32 MB + 256 MB) on an MI355X. Step k runs the forward of set
k mod n and the backward of set (k - lag) mod n. So between a set's forward and its backward,
`lag` forwards and backwards of other sets stream several hundred MB through the caches, and
consecutive steps never touch the same set. This is how a training step sees these kernels:
the rest of the model runs between a layer's forward and its backward. The per-kernel figures
rotate the same sets. The old back-to-back figure (forward and backward of one set, over and
over) is kept as `mall_warm`: it is partly served by the 256 MB MALL and is not the headline.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "kernel-rsi_amd" / "library"), str(ROOT / "kernel-rsi_amd"), str(ROOT / "oracle")]

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, published
PEAK_FP32_TFLOPS = 157.3       # MI355X fp32 MFMA, published
METRIC = "HBM GB/s (RMSNorm/GEGLU) + TFLOP/s relpos attn fwd+bwd, 1 MI355X"
CACHE_BYTES = (32 + 256) << 20  # L2 (8 XCDs x 4 MB) + MALL
# The reference kernels' own fwd+bwd times at its selftest shapes on one H20-3e
# (library/replay/nvidia_h20_3e.json of the reference), for the selftest-shape lines.
H20_SELFTEST_US = {"rmsnorm": 39.6, "geglu": 43.7, "relpos_attention": 415.9}


def cpu_model() -> dict:
    """What the host CPU says it is: lscpu's model name plus /proc/cpuinfo's family, model and
    stepping numbers (some VMs report only a generic name such as 'AMD EPYC')."""
    info = {"model": platform.processor() or "unknown"}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "Model name":
                info["model"] = val
            elif key in ("Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)"):
                info[key] = val
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("cpu family", "model", "stepping", "vendor_id") and key not in info:
                info[key] = val.strip()
            if key == "flags":
                info["avx512f"] = "avx512f" in val.split()
                break
    except OSError:
        pass
    return info


def _gen(shape, seed, std=1.0, mean=0.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


_PAD: list = []


def _queue_head_start() -> None:
    """Put ~1.5 ms of unrelated GPU work (fills of a 1 GiB buffer) in the stream. The host's
    per-step launch cost (~25-30 us through the Python binding) exceeds the run time of the
    smallest workloads, so without this head start the GPU would wait for the host. With it,
    the host enqueues the timed steps before the GPU reaches them, and the events see them back
    to back. The fills run before the first event."""
    if not _PAD:
        _PAD.append(torch.empty(1 << 28, dtype=torch.float32, device="cuda"))
    for _ in range(10):
        _PAD[0].fill_(0.0)


SETTLE_MS = 30.0  # untimed GPU work queued right before each timed region
SETTLE_MAX_STEPS = 400


def _time_steps(step, steps: int, warmup: int, stream: torch.cuda.Stream) -> dict:
    """Warm up, then time exactly `steps` back-to-back calls of step(), bracketed by synchronize.
    One pair of HIP events on the kernels' stream goes around all of them. Returns the mean GPU
    ms per step (from the events) and the host's ms per step to enqueue them.

    One pair, not one per step: event records between steps leave the GPU idle for ~10 us each
    (kernel trace: 10-11 us gaps before every step's first kernel).

    Settle run: the synchronize between warm-up and timing leaves the GPU idle while the host
    sets up, and its clocks then take ~20-30 ms of sustained load to come back. Measured on
    config 5's step after a 30 ms idle gap: the first 20 steps average 1.533 ms, steps 40-60
    1.421 ms, so timing from an idle start reported 1.51-1.52 ms per step where a continuous
    training loop runs at 1.42. So after the synchronize the GPU first gets untimed settle
    steps totalling about SETTLE_MS of its time (sized from the warm-up, at most
    SETTLE_MAX_STEPS), then the head-start fills, then the timed steps."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record(stream)
    step()
    w1.record(stream)
    torch.cuda.synchronize()
    one = max(w0.elapsed_time(w1), 1e-3)
    settle = min(SETTLE_MAX_STEPS, math.ceil(SETTLE_MS / one))
    for _ in range(settle):
        step()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _queue_head_start()
    a.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    host = (time.perf_counter() - t0) * 1e3 / steps
    b.record(stream)
    torch.cuda.synchronize()
    return {"ms_mean": a.elapsed_time(b) / steps, "host_ms": host, "settle_steps": settle}


def _rotating(fn, nset: int):
    """step() calling fn(k mod nset) on its k-th call."""
    k = [0]

    def step():
        fn(k[0] % nset)
        k[0] += 1
    return step


def _pipelined(fwd, bwd, nset: int, lag: int):
    """step(): the forward of set k mod nset and the backward of set (k - lag) mod nset."""
    k = [0]

    def step():
        fwd(k[0] % nset)
        bwd((k[0] - lag) % nset)
        k[0] += 1
    return step


def _rate(work: float, ms: float, scale: float) -> float:
    return work / (ms * 1e-3) / scale


def _kernel_line(ms: float, work: int, unit: str) -> dict:
    key = "bytes" if unit == "GB/s" else "flops"
    return {"ms": round(ms, 4), key: work, unit: round(_rate(work, ms, 1e9 if unit == "GB/s" else 1e12), 1)}


def _roofline(value: float, unit: str, peak_tflops: float = PEAK_BF16_TFLOPS) -> dict:
    peak, bound = (PEAK_HBM_GBS, "hbm") if unit == "GB/s" else (peak_tflops, "mfma")
    return {"bound": bound, "achieved": round(value, 2), "peak": peak, "unit": unit,
            "frac": round(value / peak, 4), "traffic": None}


# ------------------------------------------------------------------ CPU baseline
def _cpu_seconds(fn, budget: float, max_reps: int = 50) -> tuple[float, int]:
    """Median seconds of fn() after one warm-up, repeating until ~budget seconds of work
    (at least 3 repetitions)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start < budget or len(times) < 3):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    times.sort()
    return times[len(times) // 2], len(times)


def _cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return min(n, 16)  # the box's CPU share for one GPU


def cpu_legs(kind: str, inputs: dict, work_fwd: int, work_fb: int, unit: str, sample: str,
             budget: float) -> dict:
    """The reference's eager torch path on the host CPU (the oracle's restatement of its
    reference() formulas + autograd): forward and forward+backward, in bf16 (as the eager model
    runs) and fp32. Rates are the sample's algorithmic work over its median time; the work is
    linear in the sampled rows or (batch, head) pairs, so the full workload's CPU time is its
    work over the same rate. The headline leg is forward+backward in bf16."""
    import krsi_oracle as O
    scale = 1e9 if unit == "GB/s" else 1e12
    legs = {}
    for dname, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        cast = {k: (v.to(dt) if isinstance(v, torch.Tensor) and v.is_floating_point() and k != "pd" else v)
                for k, v in inputs.items()}
        for mode, work in (("fwd", work_fwd), ("fwd_bwd", work_fb)):
            args = {**cast, "fwd_only": mode == "fwd"}
            sec, reps = _cpu_seconds(lambda: O.cpu_eager_step(kind, args), budget)
            legs[f"{mode}_{dname}"] = {"value": round(work / sec / scale, 4), "unit": unit,
                                       "median_s": round(sec, 5), "reps": reps}
    head = legs["fwd_bwd_bf16"]
    return {"value": head["value"], "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{sample}; fwd+bwd bf16, median of {head['reps']} reps",
            "extrapolation": "rate = the sample's algorithmic work / its median time; work is linear "
                             "in the sampled rows or (batch, head) pairs",
            "legs": legs}


# ------------------------------------------------------------------- workloads
def bench_rmsnorm(args) -> dict:
    import _hip
    rows, n, eps = 32768, 4096, 1e-6
    nset, lag = 4, 2  # 4 x (x + g) = 2.1 GB of inputs
    xs = [_gen((rows, n), 0 if i == 0 else 100 + i) for i in range(nset)]
    gs = [_gen((rows, n), 2 if i == 0 else 200 + i) for i in range(nset)]
    x_dev = [x.cuda() for x in xs]
    g_dev = [g.cuda() for g in gs]
    w = _gen((n,), 1, std=0.02, mean=1.0).cuda()
    st = torch.cuda.current_stream()
    rstd = [_hip.rmsnorm_fwd(x, w, eps)[1] for x in x_dev]

    def fwd(i):
        rstd[i] = _hip.rmsnorm_fwd(x_dev[i], w, eps)[1]

    def bwd(i):
        _hip.rmsnorm_bwd(g_dev[i], x_dev[i], w, rstd[i])

    t = _time_steps(_pipelined(fwd, bwd, nset, lag), args.steps, args.warmup, st)
    tf = _time_steps(_rotating(fwd, nset), args.steps, args.warmup, st)
    tb = _time_steps(_rotating(bwd, nset), args.steps, args.warmup, st)
    warm = _time_steps(lambda: (fwd(0), bwd(0)), args.steps, args.warmup, st)
    fwd_b = 4 * rows * n + 4 * rows + 2 * n          # x in, y out, rstd out, w in
    bwd_b = 6 * rows * n + 4 * rows + 4 * n          # g, x in, dx out, rstd in, w in, dw out
    total = fwd_b + bwd_b
    gbs = _rate(total, t["ms_mean"], 1e9)
    res = {"workload": "rmsnorm fwd+bwd x[8,4096,4096] bf16 (BASELINE config 2)", "value": round(gbs, 1),
           "unit": "GB/s", "ms_per_step": round(t["ms_mean"], 4), "host_enqueue_ms_per_step": round(t["host_ms"], 4),
           "algorithmic_bytes": total,
           "rotation": f"{nset} input sets (x, g: {nset * 4 * rows * n / 1e9:.2f} GB), backward lags forward by {lag}",
           "kernels": {"rmsnorm_fwd": _kernel_line(tf["ms_mean"], fwd_b, "GB/s"),
                       "rmsnorm_bwd": _kernel_line(tb["ms_mean"], bwd_b, "GB/s")},
           "mall_warm": {"ms_per_step": round(warm["ms_mean"], 4),
                         "GB/s": round(_rate(total, warm["ms_mean"], 1e9), 1),
                         "note": "forward and backward of one set back to back: x partly MALL-resident"},
           "roofline": _roofline(gbs, "GB/s")}
    if not args.no_cpu:
        sr = 1024  # bounded sample: 1024 of the 32768 rows
        res["cpu_baseline"] = cpu_legs(
            "rmsnorm", {"x": xs[0][:sr], "w": w.cpu(), "g": gs[0][:sr], "eps": eps},
            4 * sr * n + 4 * sr + 2 * n, 10 * sr * n + 8 * sr + 6 * n, "GB/s",
            f"{sr} of {rows} rows", args.cpu_seconds)
    return res


def bench_geglu(args, approximate="none") -> dict:
    import _hip
    rows, f = 8192, 4096
    nset, lag = 6, 3  # 6 x (u + g) = 1.2 GB of inputs
    us = [_gen((rows, 2 * f), 0 if i == 0 else 100 + i) for i in range(nset)]
    gs = [_gen((rows, f), 2 if i == 0 else 200 + i) for i in range(nset)]
    u_dev = [u.cuda() for u in us]
    g_dev = [g.cuda() for g in gs]
    st = torch.cuda.current_stream()

    def fwd(i):
        _hip.geglu_fwd(u_dev[i], approximate)

    def bwd(i):
        _hip.geglu_bwd(g_dev[i], u_dev[i], approximate)

    t = _time_steps(_pipelined(fwd, bwd, nset, lag), args.steps, args.warmup, st)
    tf = _time_steps(_rotating(fwd, nset), args.steps, args.warmup, st)
    tb = _time_steps(_rotating(bwd, nset), args.steps, args.warmup, st)
    warm = _time_steps(lambda: (fwd(0), bwd(0)), args.steps, args.warmup, st)
    fwd_b, bwd_b = 6 * rows * f, 10 * rows * f
    total = fwd_b + bwd_b
    gbs = _rate(total, t["ms_mean"], 1e9)
    form = "erf" if approximate == "none" else "tanh"
    res = {"workload": f"geglu fwd+bwd u[4,2048,8192] bf16, gelu {form} (BASELINE config 3)",
           "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(t["ms_mean"], 4),
           "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_bytes": total,
           "rotation": f"{nset} input sets (u, g: {nset * 6 * rows * f / 1e9:.2f} GB), backward lags forward by {lag}",
           "kernels": {"geglu_fwd": _kernel_line(tf["ms_mean"], fwd_b, "GB/s"),
                       "geglu_bwd": _kernel_line(tb["ms_mean"], bwd_b, "GB/s")},
           "mall_warm": {"ms_per_step": round(warm["ms_mean"], 4),
                         "GB/s": round(_rate(total, warm["ms_mean"], 1e9), 1),
                         "note": "forward and backward of one set back to back: u partly MALL-resident"},
           "roofline": _roofline(gbs, "GB/s")}
    if not args.no_cpu:
        sr = 512
        res["cpu_baseline"] = cpu_legs(
            "geglu", {"u": us[0][:sr], "g": gs[0][:sr], "approximate": approximate},
            6 * sr * f, 16 * sr * f, "GB/s", f"{sr} of {rows} rows", args.cpu_seconds)
    return res


def bench_relpos(args, B=4, S=4096, H=16, D=64, dtype=torch.bfloat16) -> dict:
    import _hip
    scale = 1.0 / math.sqrt(D)
    nset, lag = 4, 2  # 4 x (qkv + dout) = 0.54 GB of inputs, plus per-set out32 and lse
    dname = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
    peak = PEAK_FP32_TFLOPS if dtype == torch.float32 else PEAK_BF16_TFLOPS
    qkvs = [_gen((B * S, 3 * H * D), 0 if i == 0 else 100 + i, dtype=dtype) for i in range(nset)]
    douts = [_gen((B * S, H * D), 2 if i == 0 else 200 + i, dtype=dtype) for i in range(nset)]
    qkv_dev = [q.cuda() for q in qkvs]
    dout_dev = [d.cuda() for d in douts]
    pd = _gen((H, 2 * S - 1), 1, std=0.02, dtype=torch.float32).cuda()
    st = torch.cuda.current_stream()
    saved = [_hip.relpos_fwd(q, pd, B, S, H, D, scale)[1:] for q in qkv_dev]

    def fwd(i):
        saved[i] = _hip.relpos_fwd(qkv_dev[i], pd, B, S, H, D, scale)[1:]

    def bwd(i):
        _hip.relpos_bwd(dout_dev[i], qkv_dev[i], pd, *saved[i], B, S, H, D, scale)

    fl_fwd = 4 * B * H * S * S * D
    fl_bwd = 10 * B * H * S * S * D
    total = fl_fwd + fl_bwd
    t = _time_steps(_pipelined(fwd, bwd, nset, lag), args.steps, args.warmup, st)
    tf = _time_steps(_rotating(fwd, nset), args.steps, args.warmup, st)
    tb = _time_steps(_rotating(bwd, nset), args.steps, args.warmup, st)
    warm = _time_steps(lambda: (fwd(0), bwd(0)), args.steps, args.warmup, st)
    tfl = _rate(total, t["ms_mean"], 1e12)
    cfg = "BASELINE config 5" if (B, S, H, D) == (4, 4096, 16, 64) else "BASELINE config 4 shape, fwd+bwd"
    suffix = ")" if dname == "bf16" else f" shape, {dname} activations)" if "5" in cfg else f", {dname} activations)"
    res = {"workload": f"relpos attention fwd+bwd B{B} H{H} L{S} D{D} {dname}, pd fp32 [H,2L-1] "
                       f"({cfg}{suffix}",
           "value": round(tfl, 2), "unit": "TFLOP/s", "ms_per_step": round(t["ms_mean"], 4),
           "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_flops": total,
           "matrix_dtype": dname,
           "rotation": f"{nset} input sets (qkv, dout), backward lags forward by {lag}",
           "kernels": {"relpos_fwd": _kernel_line(tf["ms_mean"], fl_fwd, "TFLOP/s"),
                       "relpos_bwd (dq+delta+dpd, dkdv, dpd reduce)": _kernel_line(tb["ms_mean"], fl_bwd, "TFLOP/s")},
           "mall_warm": {"ms_per_step": round(warm["ms_mean"], 4),
                         "TFLOP/s": round(_rate(total, warm["ms_mean"], 1e12), 1)},
           "roofline": {**_roofline(tfl, "TFLOP/s", peak),
                        "scope": "one fwd+bwd step = forward + dQ + dK/dV + dpd reduce kernels, "
                                 "14*B*H*L^2*D flops" + (" on fp32 MFMA" if dname == "fp32" else "")}}
    if not args.no_cpu and dname == "bf16":
        nb = 2  # bounded sample: 2 of the B*H = 64 (batch, head) pairs, full L
        q0, d0 = qkvs[0], douts[0]
        sample = {"qkv": q0.view(B, S, 3, H, D)[0, :, :, :nb].reshape(S, 3 * nb * D).clone(),
                  "pd": pd[:nb].cpu(), "dout": d0.view(B, S, H, D)[0, :, :nb].reshape(S, nb * D).clone(),
                  "dims": (1, S, nb, D), "scale": scale}
        res["cpu_baseline"] = cpu_legs("relpos", sample, 4 * nb * S * S * D, 14 * nb * S * S * D, "TFLOP/s",
                                       f"SDPA-MATH on {nb} of {B * H} (batch, head) pairs at L={S}",
                                       args.cpu_seconds)
    return res


def bench_relpos_long(args) -> dict:
    """Long context, B1 H8 L16384 D64 bf16 fwd+bwd (not a BASELINE config; parity-tested at this
    S): the dpd diagonal sums are formed inside the dK/dV kernel, so the backward's workspace is
    B*H*ceil(L/128)*(L+128) fp32 partial rows instead of the reference's [B, H, L, L] fp32 dbias.
    Two input sets (0.2 GB with their outputs), backward lagging the forward by one. (H = 8 keeps
    every grid of this leg distinct from config 5's, whose kernel traces are selected by grid.)"""
    import _hip
    B, S, H, D = 1, 16384, 8, 64
    scale = 1.0 / math.sqrt(D)
    nset, lag = 2, 1
    qkv_dev = [_gen((B * S, 3 * H * D), 300 + i).cuda() for i in range(nset)]
    dout_dev = [_gen((B * S, H * D), 400 + i).cuda() for i in range(nset)]
    pd = _gen((H, 2 * S - 1), 1, std=0.02, dtype=torch.float32).cuda()
    st = torch.cuda.current_stream()
    saved = [_hip.relpos_fwd(q, pd, B, S, H, D, scale)[1:] for q in qkv_dev]

    def fwd(i):
        saved[i] = _hip.relpos_fwd(qkv_dev[i], pd, B, S, H, D, scale)[1:]

    def bwd(i):
        _hip.relpos_bwd(dout_dev[i], qkv_dev[i], pd, *saved[i], B, S, H, D, scale)

    total = 14 * B * H * S * S * D
    t = _time_steps(_pipelined(fwd, bwd, nset, lag), args.steps, args.warmup, st)
    tfl = _rate(total, t["ms_mean"], 1e12)
    return {"workload": f"relpos attention fwd+bwd B{B} H{H} L{S} D{D} bf16 (long context)",
            "value": round(tfl, 2), "unit": "TFLOP/s", "ms_per_step": round(t["ms_mean"], 4),
            "algorithmic_flops": total, "matrix_dtype": "bf16",
            "rotation": f"{nset} input sets (qkv, dout), backward lags forward by {lag}",
            "bwd_workspace_bytes": int(_hip.lib().krsi_relpos_bwd_workspace_bytes(B, S, H, D)),
            "reference_dbias_bytes": 4 * B * H * S * S,
            "roofline": _roofline(tfl, "TFLOP/s")}


def bench_relpos_fwd_config4(args) -> dict:
    import _hip
    B, S, H, D = 2, 1024, 16, 72
    scale = 1.0 / math.sqrt(D)
    nset = 16  # 16 x 14.2 MB of qkv, 16 x 21 MB of outputs
    qkv_dev = [_gen((B * S, 3 * H * D), 0 if i == 0 else 100 + i).cuda() for i in range(nset)]
    pd = _gen((H, 2 * S - 1), 1, std=0.02, dtype=torch.float32).cuda()
    st = torch.cuda.current_stream()
    t = _time_steps(_rotating(lambda i: _hip.relpos_fwd(qkv_dev[i], pd, B, S, H, D, scale), nset),
                    args.steps, args.warmup, st)
    warm = _time_steps(lambda: _hip.relpos_fwd(qkv_dev[0], pd, B, S, H, D, scale), args.steps, args.warmup, st)
    # The same forward when no backward follows (relpos_attention under no_grad): out only.
    tn = _time_steps(_rotating(lambda i: _hip.relpos_fwd(qkv_dev[i], pd, B, S, H, D, scale, stats=False), nset),
                     args.steps, args.warmup, st)
    fl = 4 * B * H * S * S * D
    tfl = _rate(fl, t["ms_mean"], 1e12)
    return {"workload": f"relpos attention fwd B{B} H{H} L{S} D{D} bf16 (BASELINE config 4)",
            "value": round(tfl, 1), "unit": "TFLOP/s", "ms_per_step": round(t["ms_mean"], 4),
            "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_flops": fl,
            "matrix_dtype": "bf16", "rotation": f"{nset} input sets",
            "mall_warm": {"ms_per_step": round(warm["ms_mean"], 4), "TFLOP/s": round(_rate(fl, warm["ms_mean"], 1e12), 1),
                          "note": "one set, forward after forward: its 14 MB qkv stays in the caches"},
            "no_grad": {"ms_per_step": round(tn["ms_mean"], 4), "TFLOP/s": round(_rate(fl, tn["ms_mean"], 1e12), 1),
                        "note": "out only (no out32 or lse: nothing for a backward), what relpos_attention "
                                "runs when no input requires grad; same rotation"},
            "roofline": _roofline(tfl, "TFLOP/s")}


def bench_geglu_linear(args) -> dict:
    """The merged gate|up projection feeding GEGLU at config 3's u [8192, 8192] (K = 4096): the
    fused kernel (geglu_linear, u never written) against the unfused pair (hipBLASLt GEMM via
    torch, then the GEGLU forward kernel). Forward only: the fused op exists for the forward."""
    import _hip
    rows, K, F = 8192, 4096, 4096
    nset = 2
    xs = [_gen((rows, K), 30 + i).cuda() for i in range(nset)]
    ws = [(_gen((2 * F, K), 40 + i, dtype=torch.float32) / K ** 0.5).to(torch.bfloat16).cuda() for i in range(nset)]
    st = torch.cuda.current_stream()
    tf = _time_steps(_rotating(lambda i: _hip.geglu_linear_fwd(xs[i], ws[i], "tanh"), nset), args.steps, args.warmup, st)
    tu = _time_steps(_rotating(lambda i: _hip.geglu_fwd(torch.nn.functional.linear(xs[i], ws[i]), "tanh"), nset),
                     args.steps, args.warmup, st)
    tg = _time_steps(_rotating(lambda i: torch.nn.functional.linear(xs[i], ws[i]), nset), args.steps, args.warmup, st)
    fl = 2 * rows * 2 * F * K
    tfl = _rate(fl, tf["ms_mean"], 1e12)
    return {"workload": f"merged projection + GEGLU forward, x [{rows},{K}] bf16, w [{2 * F},{K}], gelu tanh",
            "value": round(tfl, 1), "unit": "TFLOP/s", "ms_per_step": round(tf["ms_mean"], 4),
            "matrix_dtype": "bf16",
            "algorithmic_flops": fl, "roofline": _roofline(tfl, "TFLOP/s"),
            "unfused": {"ms": round(tu["ms_mean"], 4), "gemm_ms": round(tg["ms_mean"], 4),
                        "gemm_TFLOP/s": round(_rate(fl, tg["ms_mean"], 1e12), 1),
                        "note": "hipBLASLt GEMM (torch) writes u, then the GEGLU forward kernel reads it"},
            "fused_vs_unfused": round(tu["ms_mean"] / tf["ms_mean"], 3)}


def bench_selftest_shapes(args) -> dict:
    """The reference's selftest() shapes (its only published timings, on an H20-3e), timed as
    that selftest times them: one input set, forward + backward back to back. These working
    sets (8-40 MB) fit the MALL, so the rates are cache-assisted by construction."""
    import _hip
    st = torch.cuda.current_stream()
    out = {}
    rows, n = 4096, 1024
    x, g = _gen((rows, n), 0).cuda(), _gen((rows, n), 2).cuda()
    w = _gen((n,), 1, std=0.1, mean=1.0).cuda()
    t = _time_steps(lambda: _hip.rmsnorm_bwd(g, x, w, _hip.rmsnorm_fwd(x, w, 1e-6)[1]), args.steps, args.warmup, st)
    work = 10 * rows * n + 8 * rows + 6 * n
    out["rmsnorm"] = (f"rmsnorm fwd+bwd x[{rows},{n}] bf16", t, work, "GB/s")
    rows, f = 2048, 2816
    u, gg = _gen((rows, 2 * f), 0).cuda(), _gen((rows, f), 2).cuda()
    t = _time_steps(lambda: (_hip.geglu_fwd(u, "tanh"), _hip.geglu_bwd(gg, u, "tanh")), args.steps, args.warmup, st)
    out["geglu"] = (f"geglu fwd+bwd u[{rows},{2 * f}] bf16, gelu tanh", t, 16 * rows * f, "GB/s")
    B, S, H, D = 4, 512, 16, 64
    qkv = (0.6 * _gen((B * S, 3 * H * D), 0, dtype=torch.float32)).to(torch.bfloat16).cuda()
    pd = _gen((H, 2 * S - 1), 1, dtype=torch.float32).cuda()
    dout = _gen((B * S, H * D), 2).cuda()

    def attn():
        _, o32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 1.0)
        _hip.relpos_bwd(dout, qkv, pd, o32, lse, B, S, H, D, 1.0)
    t = _time_steps(attn, args.steps, args.warmup, st)
    out["relpos_attention"] = (f"relpos attention fwd+bwd B{B} S{S} H{H} D{D} bf16, scale 1", t,
                               14 * B * H * S * S * D, "TFLOP/s")
    res = {}
    for name, (wl, t, work, unit) in out.items():
        v = _rate(work, t["ms_mean"], 1e9 if unit == "GB/s" else 1e12)
        us = t["ms_mean"] * 1e3
        res[name] = {"workload": wl, "us_per_step": round(us, 1), "value": round(v, 1), "unit": unit,
                     "roofline": _roofline(v, unit), "h20_reference_kernel_us": H20_SELFTEST_US[name],
                     "vs_h20_reference_kernel": round(H20_SELFTEST_US[name] / us, 2),
                     "host_enqueue_us_per_step": round(t["host_ms"] * 1e3, 1)}
    return res


def bench_bucket(args) -> dict:
    """The T5 bucketed table step either side of the attention at config 5's S and H: the gather
    (table [32, H] -> pd [H, 2S-1]) and the bucket sum of dpd (dpd [H, 2S-1] -> dtable [32, H],
    fixed order, no scatter), each against the torch ops that do the same step on the same GPU
    (index_select, and index_add_, whose atomics make it non-deterministic). Launch-latency bound:
    the bytes are a few MB."""
    import _hip
    import relpos_attention as A
    S, H, nb = 4096, 16, 32
    st = torch.cuda.current_stream()
    table = _gen((nb, H), 1, dtype=torch.float32).cuda()
    dpd = _gen((H, 2 * S - 1), 2, dtype=torch.float32).cuda()
    bucket = A.t5_relative_position_bucket(S, True, nb, 128, table.device)
    bl = bucket.long()
    npd = H * (2 * S - 1)
    work = {"gather": 4 * (2 * S - 1) + 4 * nb * H + 4 * npd, "sum": 4 * npd + 4 * (2 * S - 1) + 4 * nb * H}
    legs = {
        "gather": (lambda: _hip.relpos_bucket_gather(table, bucket, S),
                   lambda: table.index_select(0, bl).t().contiguous()),
        "sum": (lambda: _hip.relpos_bucket_sum(dpd, bucket, S, nb),
                lambda: torch.zeros(nb, H, device=dpd.device).index_add_(0, bl, dpd.t())),
    }
    out = {}
    for name, (ours, ref) in legs.items():
        t = _time_steps(ours, args.steps, args.warmup, st)
        r = _time_steps(ref, args.steps, args.warmup, st)
        out[name] = {"us": round(t["ms_mean"] * 1e3, 2), "algorithmic_bytes": work[name],
                     "GB/s": round(_rate(work[name], t["ms_mean"], 1e9), 1),
                     "torch_ops_us": round(r["ms_mean"] * 1e3, 2)}
    g = _hip.relpos_bucket_sum(dpd, bucket, S, nb)
    ref = torch.zeros(nb, H, device=dpd.device, dtype=torch.float64).index_add_(0, bl, dpd.t().double())
    out["sum_max_rel_err_vs_fp64"] = float(((g.double() - ref).abs().max() / ref.abs().max()).item())
    return {"workload": f"T5 bucketed relative-position table, S {S}, H {H}, {nb} buckets (config 5's table step)",
            "legs": out}


def bench_config1(args) -> dict:
    """the RMSNorm forward the reference runs on its CPU path, x [2,1024,1152]
    and the ragged [1,300,1152]. The CPU figure (full size, no sampling) is the headline here;
    the GPU forward is timed beside it (launch-latency bound at this size)."""
    import _hip
    n, eps = 1152, 1e-6
    st = torch.cuda.current_stream()
    w = _gen((n,), 1, std=0.02, mean=1.0)
    res = {}
    for name, rows in (("x[2,1024,1152]", 2048), ("x[1,300,1152]", 300)):
        x = _gen((rows, n), 0)
        work = 4 * rows * n + 4 * rows + 2 * n
        xd, wd = x.cuda(), w.cuda()
        t = _time_steps(lambda: _hip.rmsnorm_fwd(xd, wd, eps), args.steps, args.warmup, st)
        entry = {"gpu_fwd_us": round(t["ms_mean"] * 1e3, 2),
                 "gpu_fwd_GB/s": round(_rate(work, t["ms_mean"], 1e9), 1), "algorithmic_bytes": work}
        if not args.no_cpu:
            import krsi_oracle as O
            for dname, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
                inp = {"x": x.to(dt), "w": w.to(dt), "eps": eps, "fwd_only": True}
                sec, reps = _cpu_seconds(lambda: O.cpu_eager_step("rmsnorm", inp), min(args.cpu_seconds, 2.0), 200)
                entry[f"cpu_fwd_{dname}"] = {"us": round(sec * 1e6, 1), "GB/s": round(work / sec / 1e9, 2),
                                             "reps": reps, "cores": torch.get_num_threads()}
        res[name] = entry
    return {"workload": "rmsnorm fwd on the reference's CPU path, eps 1e-6 (BASELINE config 1)", "shapes": res}


# ------------------------------------------------------- measured HBM ceiling
# The row-pattern probe of hw.py that moves each bandwidth-bound kernel's bytes.
KERNEL_PATTERN = {"rmsnorm_fwd": "rms_fwd", "rmsnorm_bwd": "rms_bwd", "geglu_fwd": "geglu_fwd",
                  "geglu_bwd": "geglu_bwd"}


def attach_stream_ceiling(comps: dict) -> dict:
    """The cache-cold rate of each bandwidth-bound kernel's own access pattern with trivial
    arithmetic on this box (hw.py's row-pattern probes: same arrays, row layout and read:write
    bytes, best of a sweep over chunks per thread and non-temporal loads and stores). Each
    bandwidth component gets the ceiling of its fwd+bwd step (the probes' time for the same
    bytes) and its fraction of it, beside the roofline against the published 8 TB/s."""
    import hw
    if not any(k in KERNEL_PATTERN for c in comps.values() for k in c.get("kernels", {})):
        return {}
    probe = hw.probe_patterns(hw.Clock(samples=3), quick=True)
    if "error" in probe:
        return probe
    for comp in comps.values():
        ks = {k: v for k, v in comp.get("kernels", {}).items() if k in KERNEL_PATTERN}
        if not ks:
            continue
        t = sum(v["bytes"] / (probe[KERNEL_PATTERN[k]]["gbs"] * 1e9) for k, v in ks.items())
        ceil = sum(v["bytes"] for v in ks.values()) / t / 1e9
        comp["stream_ceiling"] = {"GB/s": round(ceil, 1), "frac": round(comp["value"] / ceil, 4),
                                  "source": "hw.py row-pattern probes of each kernel's traffic, this run"}
    return {f"pattern_{k}_GB/s": v["gbs"] for k, v in probe.items()}


def attach_gemm_ceiling(comps: dict) -> dict:
    """The vendor library's dense GEMM rate on this box (hw.py's probe: hipBLASLt through
    torch.mm at 8192^3, per dtype), beside the published MFMA peak. It runs under the same
    clock and power limits as the attention kernels, so each matrix component also gets its
    fraction of it."""
    import hw
    if not any(c.get("matrix_dtype") for c in comps.values()):
        return {}
    rates = hw.probe_gemm(hw.Clock(samples=3), 8192)
    for comp in comps.values():
        rate = rates.get(comp.get("matrix_dtype"))
        if rate:
            comp["gemm_ceiling"] = {"TFLOP/s": rate, "frac": round(comp["value"] / rate, 4),
                                    "source": f"hipBLASLt {comp['matrix_dtype']} GEMM 8192^3 (torch.mm), this run"}
    return {f"gemm_{k}_TFLOP/s": v for k, v in rates.items() if isinstance(v, (int, float))}


# ------------------------------------------------------------------- traffic
def _csrc_sha256() -> str:
    import hashlib
    h = hashlib.sha256()
    for f in sorted((ROOT / "kernel-rsi_amd" / "csrc").glob("*")) + [ROOT / "kernel-rsi_amd" / "build.py"]:
        h.update(f.read_bytes())
    return h.hexdigest()


def attach_traffic(comps: dict) -> None:
    """roofline.traffic = HBM bytes per step from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (profiles/traffic.json, scaled by a 2 GiB copy). Counters cannot be read inside this
    process, so the figure is taken from those runs, and only while the kernel sources and the
    build script (its flags) still hash to what was profiled; otherwise it is null."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return
    fresh = rec.get("csrc_sha256") == _csrc_sha256()
    for name, comp in comps.items():
        t = rec.get("components", {}).get(name)
        if t is None or "roofline" not in comp:
            continue
        comp["roofline"]["traffic"] = t["bytes_per_step"] if fresh else None
        comp["roofline"]["traffic_unit"] = "bytes per step (HBM read + write)"
        comp["roofline"]["traffic_source"] = t["summary"] if fresh else f"stale: {t['summary']} profiled other sources"
        if fresh and comp.get("algorithmic_bytes"):
            comp["roofline"]["traffic_vs_algorithmic"] = round(t["bytes_per_step"] / comp["algorithmic_bytes"], 3)


def measured_copy_gbs() -> float:
    """Achievable HBM rate on this box: a 2 GiB device-to-device copy (read + write bytes)."""
    n = 1 << 30
    a = torch.empty(n, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    del a, b
    return round(2 * 2 * n / (ms * 1e-3) / 1e9, 1)


ALL = ("relpos,relpos_fwd,relpos_fp16,relpos_fp32,relpos_long,rmsnorm,geglu,geglu_linear,selftest_shapes,config1,"
       "bucket")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default=ALL)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU time budget per CPU-baseline leg")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's kernels run on one MI355X and no "
              "multi-GPU figure is produced; run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    torch.set_num_threads(_cpu_threads())
    only = set(args.only.split(","))
    comps = {}
    if "relpos" in only:
        comps["relpos_attention"] = bench_relpos(args)
    if "relpos_fwd" in only:
        comps["relpos_attention_fwd_config4"] = bench_relpos_fwd_config4(args)
    if "relpos_fp16" in only:
        comps["relpos_attention_fp16"] = bench_relpos(args, dtype=torch.float16)
    if "relpos_fp32" in only:
        comps["relpos_attention_fp32"] = bench_relpos(args, B=2, S=1024, H=16, D=72, dtype=torch.float32)
    if "relpos_long" in only:
        comps["relpos_attention_long"] = bench_relpos_long(args)
    if "rmsnorm" in only:
        comps["rmsnorm"] = bench_rmsnorm(args)
    if "geglu" in only:
        comps["geglu"] = bench_geglu(args, "none")
    if "geglu_linear" in only:
        comps["geglu_linear"] = bench_geglu_linear(args)
    if "selftest_shapes" in only:
        comps["selftest_shapes"] = bench_selftest_shapes(args)
    if "config1" in only:
        comps["rmsnorm_config1"] = bench_config1(args)
    if "bucket" in only:
        comps["relpos_bucket_table"] = bench_bucket(args)
    attach_traffic(comps)
    ceilings = {**attach_stream_ceiling(comps), **attach_gemm_ceiling(comps)}
    # The headline is config 5's attention; a run limited by --only to components without a
    # single figure of their own (the selftest shapes, config 1) prints value null.
    head = comps.get("relpos_attention") or next((c for c in comps.values() if "value" in c), None)
    if head is None:
        head = {"value": None, "unit": None, "ms_per_step": None, "roofline": None,
                "workload": "no headline component in --only " + args.only}
    cpu = cpu_model()
    line = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "timing": (f"per leg: {args.warmup} warm-up steps, synchronize, untimed settle steps worth ~{SETTLE_MS:g} ms "
                   f"of GPU time (clocks back at steady state), head-start fills, then {args.steps} timed steps "
                   "between one pair of HIP events"),
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded CPU randn, BASELINE shapes)",
        "config": {"workload": head["workload"], "device": torch.cuda.get_device_name(0)},
        "roofline": head["roofline"],
        "cpu_baseline": {**head["cpu_baseline"], "cpu": cpu["model"]} if "cpu_baseline" in head else None,
        "components": comps,
        "host_cpu": cpu,
        "measured_peaks": {"hbm_copy_GB/s (torch copy)": measured_copy_gbs(), **ceilings},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
