#!/usr/bin/env python3
"""Benchmark of the fused kernel library on one MI355X: HBM GB/s of RMSNorm and GEGLU
fwd+bwd and TFLOP/s of relative-position flash attention fwd+bwd, each as a fraction of the
MI355X roofline, with the reference's eager torch path timed on the host CPU beside it.

    python bench.py [--steps K] [--warmup W] [--only relpos,rmsnorm,geglu,relpos_fwd,relpos_fp16] [--no-cpu]

A "step" is one forward + backward pass of a kernel over one batch of synthetic input that
is already resident in HBM (3 and 5; config 4 is the forward-only
attention line). Prints ONE JSON line; `value` is the relpos attention fwd+bwd TFLOP/s (the
dominant kernel), and `components` holds every workload's own figure and roofline.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "kernel-rsi_amd" / "library"), str(ROOT / "oracle")]

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, published
METRIC = "HBM GB/s (RMSNorm/GEGLU) + TFLOP/s relpos attn fwd+bwd, 1 MI355X"


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _gen(shape, seed, std=1.0, mean=0.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


_PAD: list = []


def _queue_head_start() -> None:
    """Put ~1.5 ms of unrelated GPU work (fills of a 1 GiB buffer) in the stream, so that the
    host, whose per-step launch cost (~25-30 us through the Python binding) exceeds the run
    time of the smallest workload (config 4, ~25 us), enqueues the timed steps before the GPU
    reaches them and the events see them back to back. The fills run before the first event."""
    if not _PAD:
        _PAD.append(torch.empty(1 << 28, dtype=torch.float32, device="cuda"))
    for _ in range(10):
        _PAD[0].fill_(0.0)


def _time_steps(step, steps: int, warmup: int, stream: torch.cuda.Stream) -> dict:
    """Warm up, then time exactly `steps` back-to-back steps bracketed by synchronize, with
    one pair of HIP events on the stream the kernels launch on around all of them. Returns
    the mean GPU ms per step (events) and the host's ms per step to enqueue them.

    One pair, not one per step: event records between steps leave the GPU idle for ~10 us
    each (kernel trace: 10-11 us gaps before every step's first kernel, none inside a step
    or in the untimed warm-up). A/B on one box: the same attention and RMSNorm step times
    either way (within 1 %), but the 25 us config 4 forward read 27.2 us with a pair per step."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _queue_head_start()
    a.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    host = (time.perf_counter() - t0) * 1e3 / steps
    b.record(stream)
    torch.cuda.synchronize()
    return {"ms_mean": a.elapsed_time(b) / steps, "host_ms": host}


def _cpu_time(fn, min_s: float = 10.0, max_reps: int = 50) -> tuple[float, int]:
    """Median seconds of fn() after one warm-up, repeating until ~min_s of CPU work."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start < min_s or len(times) < 3):
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


# ------------------------------------------------------------------- workloads
def bench_rmsnorm(args) -> dict:
    import _hip
    rows, n, eps = 32768, 4096, 1e-6
    x = _gen((rows, n), 0).cuda()
    w = _gen((n,), 1, std=0.02, mean=1.0).cuda()
    g = _gen((rows, n), 2).cuda()
    st = torch.cuda.current_stream()
    state = {}

    def step():
        y, rstd = _hip.rmsnorm_fwd(x, w, eps)
        state["r"] = _hip.rmsnorm_bwd(g, x, w, rstd)

    t = _time_steps(step, args.steps, args.warmup, st)
    # Per-kernel: forward and backward timed separately with the same protocol.
    _, rstd = _hip.rmsnorm_fwd(x, w, eps)
    tf = _time_steps(lambda: _hip.rmsnorm_fwd(x, w, eps), args.steps, args.warmup, st)
    tb = _time_steps(lambda: _hip.rmsnorm_bwd(g, x, w, rstd), args.steps, args.warmup, st)
    fwd_b = 4 * rows * n + 4 * rows + 2 * n          # x in, y out, rstd out, w in
    bwd_b = 6 * rows * n + 4 * rows + 4 * n          # g, x in, dx out, rstd in, w in, dw out
    total = fwd_b + bwd_b
    gbs = total / (t["ms_mean"] * 1e-3) / 1e9
    res = {"workload": "rmsnorm fwd+bwd x[8,4096,4096] bf16 (BASELINE config 2)", "value": round(gbs, 1),
           "unit": "GB/s", "ms_per_step": round(t["ms_mean"], 4), "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_bytes": total,
           "kernels": {"rmsnorm_fwd": {"ms": round(tf["ms_mean"], 4), "bytes": fwd_b,
                                       "GB/s": round(fwd_b / tf["ms_mean"] / 1e6, 1)},
                       "rmsnorm_bwd": {"ms": round(tb["ms_mean"], 4), "bytes": bwd_b,
                                       "GB/s": round(bwd_b / tb["ms_mean"] / 1e6, 1)}},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}}
    if not args.no_cpu:
        import krsi_oracle as O
        sr = 1024  # bounded sample: 1024 of the 32768 rows
        xs, gs, ws = x[:sr].cpu(), g[:sr].cpu(), w.cpu()
        sec, reps = _cpu_time(lambda: O.cpu_eager_step("rmsnorm", {"x": xs, "w": ws, "g": gs, "eps": eps}))
        sb = 10 * sr * n + 8 * sr + 6 * n
        res["cpu_baseline"] = {"value": round(sb / sec / 1e9, 2), "unit": "GB/s", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": f"reference eager torch fwd+bwd (bf16) on {sr} of {rows} rows, "
                                                         f"median of {reps} reps"}
    return res


def bench_geglu(args, approximate="none") -> dict:
    import _hip
    rows, f = 8192, 4096
    ncopy = 2  # rotate two input sets (working set 2 x 402 MB > 256 MB MALL)
    us = [_gen((rows, 2 * f), 10 * i).cuda() for i in range(ncopy)]
    gs = [_gen((rows, f), 10 * i + 2).cuda() for i in range(ncopy)]
    st = torch.cuda.current_stream()
    it = [0]

    def step():
        i = it[0] % ncopy
        it[0] += 1
        _hip.geglu_fwd(us[i], approximate)
        _hip.geglu_bwd(gs[i], us[i], approximate)

    t = _time_steps(step, args.steps, args.warmup, st)
    tf = _time_steps(lambda: _hip.geglu_fwd(us[it[0] % ncopy], approximate), args.steps, args.warmup, st)
    tb = _time_steps(lambda: _hip.geglu_bwd(gs[0], us[0], approximate), args.steps, args.warmup, st)
    fwd_b, bwd_b = 6 * rows * f, 10 * rows * f
    total = fwd_b + bwd_b
    gbs = total / (t["ms_mean"] * 1e-3) / 1e9
    res = {"workload": f"geglu fwd+bwd u[4,2048,8192] bf16, gelu {'erf' if approximate == 'none' else 'tanh'} "
                       "(BASELINE config 3)", "value": round(gbs, 1), "unit": "GB/s",
           "ms_per_step": round(t["ms_mean"], 4), "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_bytes": total,
           "kernels": {"geglu_fwd": {"ms": round(tf["ms_mean"], 4), "bytes": fwd_b,
                                     "GB/s": round(fwd_b / tf["ms_mean"] / 1e6, 1)},
                       "geglu_bwd": {"ms": round(tb["ms_mean"], 4), "bytes": bwd_b,
                                     "GB/s": round(bwd_b / tb["ms_mean"] / 1e6, 1)}},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}}
    if not args.no_cpu:
        import krsi_oracle as O
        sr = 512
        u_s, g_s = us[0][:sr].cpu(), gs[0][:sr].cpu()
        sec, reps = _cpu_time(lambda: O.cpu_eager_step("geglu", {"u": u_s, "g": g_s, "approximate": approximate}))
        res["cpu_baseline"] = {"value": round(16 * sr * f / sec / 1e9, 2), "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"reference eager torch fwd+bwd (bf16) on {sr} of {rows} rows, "
                                         f"median of {reps} reps"}
    return res


def bench_relpos(args, B=4, S=4096, H=16, D=64, fwd_only=False, dtype=torch.bfloat16) -> dict:
    import _hip
    scale = 1.0 / math.sqrt(D)
    qkv = _gen((B * S, 3 * H * D), 0, dtype=dtype).cuda()
    pd = _gen((H, 2 * S - 1), 1, std=0.02, dtype=torch.float32).cuda()
    dout = _gen((B * S, H * D), 2, dtype=dtype).cuda()
    dname = "bf16" if dtype == torch.bfloat16 else "fp16"
    st = torch.cuda.current_stream()
    fl_fwd = 4 * B * H * S * S * D
    fl_bwd = 10 * B * H * S * S * D
    _, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
    tf = _time_steps(lambda: _hip.relpos_fwd(qkv, pd, B, S, H, D, scale), args.steps, args.warmup, st)
    if fwd_only:
        tfl = fl_fwd / (tf["ms_mean"] * 1e-3) / 1e12
        return {"workload": f"relpos attention fwd B{B} H{H} L{S} D{D} bf16 (BASELINE config 4)",
                "value": round(tfl, 1), "unit": "TFLOP/s", "ms_per_step": round(tf["ms_mean"], 4), "host_enqueue_ms_per_step": round(tf["host_ms"], 4),
                "algorithmic_flops": fl_fwd,
                "roofline": {"bound": "mfma", "achieved": round(tfl, 1), "peak": PEAK_BF16_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(tfl / PEAK_BF16_TFLOPS, 4), "traffic": None}}

    def step():
        o, o32, l = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
        _hip.relpos_bwd(dout, qkv, pd, o32, l, B, S, H, D, scale)

    t = _time_steps(step, args.steps, args.warmup, st)
    tb = _time_steps(lambda: _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, scale),
                     args.steps, args.warmup, st)
    total = fl_fwd + fl_bwd
    tfl = total / (t["ms_mean"] * 1e-3) / 1e12
    res = {"workload": f"relpos attention fwd+bwd B{B} H{H} L{S} D{D} {dname}, pd fp32 [H,2L-1] "
                       "(BASELINE config 5" + (")" if dname == "bf16" else " shape, fp16 activations)"),
           "value": round(tfl, 2), "unit": "TFLOP/s",
           "ms_per_step": round(t["ms_mean"], 4), "host_enqueue_ms_per_step": round(t["host_ms"], 4), "algorithmic_flops": total,
           "kernels": {"relpos_fwd": {"ms": round(tf["ms_mean"], 4), "flops": fl_fwd,
                                      "TFLOP/s": round(fl_fwd / tf["ms_mean"] / 1e9, 1)},
                       "relpos_bwd (dq+delta+dpd, dkdv, dpd reduce)": {
                           "ms": round(tb["ms_mean"], 4), "flops": fl_bwd,
                           "TFLOP/s": round(fl_bwd / tb["ms_mean"] / 1e9, 1)}},
           "roofline": {"bound": "mfma", "achieved": round(tfl, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tfl / PEAK_BF16_TFLOPS, 4), "traffic": None,
                        "scope": "one fwd+bwd step = relpos_fwd_kernel + relpos_bwd_dq_kernel + "
                                 "relpos_bwd_dkdv_kernel + relpos_dpd_reduce4, 14*B*H*L^2*D flops"}}
    if not args.no_cpu and dname == "bf16":
        import krsi_oracle as O
        nb = 2  # bounded sample: 2 of the B*H = 64 (batch, head) pairs, full L
        qs = qkv.view(B, S, 3, H, D)[0, :, :, :nb].reshape(S, 3 * nb * D).cpu()
        ps, ds_ = pd[:nb].cpu(), dout.view(B, S, H, D)[0, :, :nb].reshape(S, nb * D).cpu()
        sec, reps = _cpu_time(lambda: O.cpu_eager_step("relpos", {"qkv": qs, "pd": ps, "dout": ds_,
                                                                  "dims": (1, S, nb, D), "scale": scale}),
                              min_s=10.0, max_reps=10)
        res["cpu_baseline"] = {"value": round(14 * nb * S * S * D / sec / 1e12, 4), "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"reference eager torch SDPA-MATH fwd+bwd (bf16 in, fp32 math) on "
                                         f"{nb} of {B * H} (batch, head) pairs at L={S}, median of {reps} reps"}
    return res


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
        if t is None:
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


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="relpos,relpos_fwd,rmsnorm,geglu,relpos_fp16")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's kernels run on one MI355X and no "
              "multi-GPU figure is produced (see DESIGN.md for how the path would shard).", file=sys.stderr)
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
        comps["relpos_attention_fwd_config4"] = bench_relpos(args, B=2, S=1024, H=16, D=72, fwd_only=True)
    if "relpos_fp16" in only:
        comps["relpos_attention_fp16"] = bench_relpos(args, dtype=torch.float16)
    if "rmsnorm" in only:
        comps["rmsnorm"] = bench_rmsnorm(args)
    if "geglu" in only:
        comps["geglu"] = bench_geglu(args, "none")
    attach_traffic(comps)
    head = comps.get("relpos_attention") or next(iter(comps.values()))
    line = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded CPU randn, BASELINE shapes)",
        "config": {"workload": head["workload"], "device": torch.cuda.get_device_name(0)},
        "roofline": head["roofline"],
        "cpu_baseline": {**head.get("cpu_baseline", {}), "cpu": _cpu_model()} if "cpu_baseline" in head else None,
        "components": comps,
        "measured_peaks": {"hbm_copy_GB/s": measured_copy_gbs()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
