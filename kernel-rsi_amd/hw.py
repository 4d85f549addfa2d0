#!/usr/bin/env python3
"""Measure this GPU's achievable peaks and write them to hardware/<device slug>.json.

  python kernel-rsi_amd/hw.py

Mirrors the reference's tools/hw.py (:90-178) for an MI355X: dense GEMM TFLOP/s per dtype as
the vendor library (hipBLASLt through torch.matmul) reaches them, skinny-GEMM rates, copy / read
/ write GB/s, launch costs (one torch op, one graph replay), and the derived ridge points. The
roofline fractions elsewhere in this package use the published peaks (HBM 8.0 TB/s, bf16 dense
2.5 PFLOP/s); these measured ceilings are reported beside them. NVIDIA-only probes of the
reference (Triton launch probe, ncu availability) have no counterpart here.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent


def slug(text: str) -> str:
    return "".join(c if c.isalnum() else "_" for c in text).strip("_").lower()


def best_ms(fn, iters: int = 10, reps: int = 5) -> float:
    """Best over reps of the mean event time of iters back-to-back calls, after a warm-up."""
    fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / iters)
    return best


def main() -> int:
    if not torch.cuda.is_available():
        raise SystemExit("no GPU")
    props = torch.cuda.get_device_properties(0)
    n = 8192

    def gemm_tflops(dtype, iters=10):
        a = torch.randn(n, n, device="cuda", dtype=dtype)
        b = torch.randn(n, n, device="cuda", dtype=dtype)
        t = 2 * n ** 3 / best_ms(lambda: a @ b, iters=iters) / 1e9
        del a, b
        return round(t, 1)

    tflops = {"fp16": gemm_tflops(torch.float16), "bf16": gemm_tflops(torch.bfloat16)}
    old_tf32 = torch.backends.cuda.matmul.allow_tf32
    try:
        torch.backends.cuda.matmul.allow_tf32 = False
        tflops["fp32"] = gemm_tflops(torch.float32, iters=3)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old_tf32
    try:
        a = torch.randn(n, n, device="cuda").to(torch.float8_e4m3fn)
        b = torch.randn(n, n, device="cuda").to(torch.float8_e4m3fn).t().contiguous().t()
        one = torch.ones((), device="cuda")
        tflops["fp8"] = round(2 * n ** 3 / best_ms(
            lambda: torch._scaled_mm(a, b, one, one, out_dtype=torch.bfloat16)) / 1e9, 1)
        del a, b
    except Exception as e:  # noqa: BLE001 - the fp8 GEMM entry point differs across builds
        tflops["fp8_error"] = f"{type(e).__name__}: {str(e).splitlines()[0][:160]}"
    skinny = {}
    for m_ in (16, 64, 256, 1024):
        a = torch.randn(m_, 4096, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
        skinny[f"M{m_}xN4096xK4096"] = round(2 * m_ * 4096 * 4096 / best_ms(lambda: a @ b, iters=50) / 1e9, 1)
    tflops["skinny_bf16"] = skinny
    torch.cuda.empty_cache()

    numel = 512 << 20  # 1 GiB per fp16 buffer: far beyond L2 and the 256 MB MALL
    src = torch.randn(numel, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    copy = 4 * numel / best_ms(lambda: dst.copy_(src)) / 1e6
    read = 2 * numel / best_ms(lambda: src.sum(dtype=torch.float32)) / 1e6
    write = 2 * numel / best_ms(lambda: dst.fill_(1.0)) / 1e6
    del src, dst
    torch.cuda.empty_cache()

    x = torch.zeros(1, device="cuda")
    launch_torch = best_ms(lambda: x.add_(1.0), iters=200) * 1000
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        x.add_(1.0)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        x.add_(1.0)
    launch_graph = best_ms(g.replay, iters=200) * 1000

    bw = max(copy, read)
    info = {
        "device": props.name, "arch": props.gcnArchName, "cus": props.multi_processor_count,
        "l2_mb": round(getattr(props, "L2_cache_size", 0) / 2 ** 20, 1),
        "memory_gb": round(props.total_memory / 2 ** 30, 1), "tflops": tflops,
        "bw_copy_gbs": round(copy), "bw_read_gbs": round(read), "bw_write_gbs": round(write),
        "ridge_flop_per_byte": {k: round(v * 1e12 / (bw * 1e9), 1) for k, v in tflops.items()
                                if isinstance(v, (int, float))},
        "published_peaks": {"hbm_gbs": 8000, "bf16_dense_tflops": 2500, "fp8_dense_tflops": 5000,
                            "fp32_tflops": 157.3},
        "default_half_dtype": "bf16", "features": {"bf16_mfma": True, "fp8": True},
        "launch_us_torch": round(launch_torch, 1), "launch_us_graph_replay": round(launch_graph, 1),
        "torch": torch.__version__, "hip": torch.version.hip,
    }
    path = HERE / "hardware" / f"{slug(props.name)}.json"
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(info, indent=2) + "\n")
    for k, v in info.items():
        print(f"{k:>24}: {v}")
    print(f"saved {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
