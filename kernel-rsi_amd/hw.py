#!/usr/bin/env python3
"""Measured ceilings of this GPU, written to hardware/<gpu>.json.

  python kernel-rsi_amd/hw.py [--quick] [--stream-only] [--lds-only] [--lds-banks]

The reference's tools read two things from such a record: `tflops[dtype]` and
`bw_copy_gbs` / `bw_read_gbs` (tools/common.py:56-64; its own probe is tools/hw.py). They use
them as roofline denominators. This module fills those keys for an MI355X and adds what this
package's roofline discussion uses:
  * the published peaks;
  * the rate of a hand-written streaming kernel at each read:write mix (libkrsi_probe.so), the
    practical HBM ceiling for bandwidth-bound kernels, which torch's copy does not reach;
  * the rate of each bandwidth-bound kernel's own access pattern with trivial arithmetic
    (the row-pattern probes of libkrsi_probe.so), the ceiling that kernel is measured against;
  * LDS bytes per clock per CU of each access form the attention kernels use (the LDS probes
    of libkrsi_probe.so; `--lds-banks` runs the bank-pattern probe that
    probe/lds_banks.py fits under a counter run);
  * launch costs;
  * the ridge points.
The probes are a table of small functions. Each runs under `Clock`, which reports the median
of per-call HIP event times after a warm-up. The bandwidth probes use 1 GiB buffers, far
beyond the 4 MB L2 of each XCD and the 256 MB MALL, so every call streams HBM.

The record is named after the product (AMD Instinct MI355X for gfx950 with 256 CUs), because
torch reports a generic name on boxes without the marketing-name table. A copy is also kept
under the slug of torch's device name, which is the file the reference's tools open on this
machine.
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
PUBLISHED = {"hbm_gbs": 8000, "bf16_dense_tflops": 2500, "fp16_dense_tflops": 2500,
             "fp8_dense_tflops": 5000, "fp32_tflops": 157.3}


def slug(text: str) -> str:
    return "".join(c if c.isalnum() else "_" for c in text).strip("_").lower()


def product_name(props) -> str:
    """The marketing name of the part (torch says 'AMD Radeon Graphics' when the driver's name
    table is absent, as on these boxes)."""
    arch = props.gcnArchName.split(":")[0]
    if arch == "gfx950" and props.multi_processor_count == 256:
        return "AMD Instinct MI355X"
    return props.name


class Clock:
    """Median device milliseconds of one call of fn (HIP events around `inner` calls)."""

    def __init__(self, samples: int = 7):
        self.samples = samples

    def ms(self, fn, inner: int = 10) -> float:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(self.samples):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(inner):
                fn()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b) / inner)
        return statistics.median(times)


def _square(n, dtype):
    return torch.randn(n, n, device="cuda").to(dtype)


def probe_gemm(clock: Clock, n: int) -> dict:
    """Dense n^3 GEMM rate of the vendor library (hipBLASLt via torch.matmul) per dtype."""
    out = {}
    for key, dtype, inner in (("bf16", torch.bfloat16, 10), ("fp16", torch.float16, 10),
                              ("fp32", torch.float32, 3)):
        a, b = _square(n, dtype), _square(n, dtype)
        prev = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = False  # fp32 means fp32 here (gfx950 has no TF32)
        try:
            out[key] = round(2 * n ** 3 / clock.ms(lambda: torch.mm(a, b), inner) / 1e9, 1)
        finally:
            torch.backends.cuda.matmul.allow_tf32 = prev
        del a, b
    try:
        a = _square(n, torch.float8_e4m3fn)
        bt = _square(n, torch.float8_e4m3fn).t()  # column-major right operand
        one = torch.ones((), device="cuda")
        out["fp8"] = round(2 * n ** 3 / clock.ms(
            lambda: torch._scaled_mm(a, bt, one, one, out_dtype=torch.bfloat16)) / 1e9, 1)
    except Exception as e:  # noqa: BLE001 - the fp8 GEMM entry point differs across torch builds
        out["fp8_error"] = f"{type(e).__name__}: {str(e).splitlines()[0][:160]}"
    return out


def probe_skinny(clock: Clock) -> dict:
    """bf16 GEMM rate with few rows (decode-like shapes), K = N = 4096."""
    w = _square(4096, torch.bfloat16)
    rates = {}
    for m in (16, 64, 256, 1024):
        x = torch.randn(m, 4096, device="cuda").to(torch.bfloat16)
        rates[f"M{m}xN4096xK4096"] = round(2 * m * 4096 * 4096 / clock.ms(lambda: x @ w, 50) / 1e9, 1)
    return rates


def probe_bandwidth(clock: Clock) -> dict:
    """GB/s of a device copy (read + write), a reduction (read) and a fill (write) of 1 GiB."""
    nbytes = 1 << 30
    src = torch.empty(nbytes // 2, device="cuda", dtype=torch.float16).normal_()
    dst = torch.empty_like(src)
    res = {
        "bw_copy_gbs": 2 * nbytes / clock.ms(lambda: dst.copy_(src)) / 1e6,
        "bw_read_gbs": nbytes / clock.ms(lambda: torch.sum(src, dtype=torch.float32)) / 1e6,
        "bw_write_gbs": nbytes / clock.ms(lambda: dst.fill_(0.5)) / 1e6,
    }
    del src, dst
    torch.cuda.empty_cache()
    return {k: round(v) for k, v in res.items()}


STREAM_MIXES = ((1, 0), (0, 1), (1, 1), (2, 1), (3, 1), (3, 2))


def probe_stream(clock: Clock, quick: bool = False, mixes=STREAM_MIXES) -> dict:
    """GB/s of a hand-written streaming kernel (libkrsi_probe.so, built with the library) at each
    read:write mix, cache-cold. This is the practical HBM ceiling for bandwidth-bound kernels
    moving bytes in that proportion (RMSNorm forward is 1:1, its backward and the GEGLU forward
    2:1, the GEGLU backward 3:2). Best over a small sweep of grid size, chunks in flight and
    non-temporal stores. Each array is 512 MiB; two sets alternate, so no call finds its data in
    the 256 MB MALL."""
    import ctypes

    path = HERE / "libkrsi_probe.so"
    if not path.is_file():
        return {"error": f"{path.name} not built"}
    lib = ctypes.CDLL(str(path))
    lib.krsi_probe_stream.restype = ctypes.c_int
    lib.krsi_probe_stream.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                                           ctypes.c_void_p]
    nbytes = 512 << 20
    n = nbytes // 16
    sets = [[torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 256) for _ in range(5)]
            for _ in range(2)]
    ptrs = [(ctypes.c_void_p * 3)(*[t.data_ptr() for t in s[:3]]) for s in sets]
    outs = [(ctypes.c_void_p * 2)(*[t.data_ptr() for t in s[3:]]) for s in sets]
    stream = torch.cuda.current_stream().cuda_stream
    sweep = [(u, nt, b) for u in (1, 4) for nt in (0, 1) for b in ((1024, 32768) if quick else (1024, 4096, 32768))]
    res = {}
    for r, w in mixes:
        best = (0.0, None)
        for u, nt, blocks in sweep:
            if w == 0 and nt:
                continue
            k = [0]

            def call():
                i = k[0] % 2
                k[0] += 1
                rc = lib.krsi_probe_stream(r, w, u, nt, blocks, ptrs[i], outs[i], n, stream)
                if rc:
                    raise RuntimeError(f"krsi_probe_stream({r}, {w}, {u}, {nt}, {blocks}) returned {rc}")
            gbs = (r + w) * nbytes / clock.ms(call, 4) / 1e6
            if gbs > best[0]:
                best = (gbs, {"unroll": u, "nontemporal": nt, "blocks": blocks})
        res[f"r{r}w{w}"] = {"gbs": round(best[0]), **best[1]}
    del sets
    torch.cuda.empty_cache()
    return res


# The library's bandwidth-bound kernels at their BASELINE shapes: (pattern, rows, chunks of 16
# bytes in the narrow row, bytes per call, rotating sets).
PATTERNS = {
    "rms_fwd": (0, 32768, 512, 32768 * 512 * 16 * 2, 4),
    "rms_bwd": (1, 32768, 512, 32768 * 512 * 16 * 3, 4),
    "geglu_fwd": (2, 8192, 512, 8192 * 512 * 16 * 3, 6),
    "geglu_bwd": (3, 8192, 512, 8192 * 512 * 16 * 5, 6),
}


def probe_patterns(clock: Clock, quick: bool = False) -> dict:
    """GB/s of the row-pattern probes (libkrsi_probe.so krsi_probe_rows): each bandwidth-bound
    kernel's exact HBM traffic (same arrays, row layout and read:write bytes) with trivial
    arithmetic, best over chunks per thread, rows per workgroup and non-temporal loads / stores.
    Cache-cold: sets of arrays rotate, several hundred MB each, past the 256 MB MALL."""
    import ctypes

    path = HERE / "libkrsi_probe.so"
    if not path.is_file():
        return {"error": f"{path.name} not built"}
    lib = ctypes.CDLL(str(path))
    lib.krsi_probe_rows.restype = ctypes.c_int
    lib.krsi_probe_rows.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                                        ctypes.c_int, ctypes.c_void_p]
    stream = torch.cuda.current_stream().cuda_stream
    shapes = ((1, 1), (2, 1), (4, 1), (1, 2), (2, 2), (1, 4))
    if quick:
        shapes = ((1, 1), (2, 1))
    res = {}
    for name, (pat, rows, n, nbytes, nsets) in PATTERNS.items():
        chunk = rows * n * 16
        sizes = {0: ([chunk], [chunk]), 1: ([chunk, chunk], [chunk]), 2: ([2 * chunk], [chunk]),
                 3: ([chunk, 2 * chunk], [2 * chunk])}[pat]
        sets = [([torch.empty(b, dtype=torch.uint8, device="cuda").random_(0, 256) for b in sizes[0]],
                 [torch.empty(b, dtype=torch.uint8, device="cuda") for b in sizes[1]]) for _ in range(nsets)]
        ins = [(ctypes.c_void_p * 2)(*([t.data_ptr() for t in i] + [0] * (2 - len(i)))) for i, _ in sets]
        outs = [(ctypes.c_void_p * 1)(o[0].data_ptr()) for _, o in sets]
        best = (0.0, None)
        for vpt, rpb in shapes:
            for ntl in (0, 1):
                for nts in (0, 1):
                    k = [0]

                    def call():
                        i = k[0] % nsets
                        k[0] += 1
                        rc = lib.krsi_probe_rows(pat, vpt, rpb, ntl, nts, ins[i], outs[i], rows, n, stream)
                        if rc:
                            raise RuntimeError(f"krsi_probe_rows({pat}, {vpt}, {rpb}, {ntl}, {nts}) returned {rc}")
                    gbs = nbytes / clock.ms(call, 2 * nsets) / 1e6
                    if gbs > best[0]:
                        best = (gbs, {"vpt": vpt, "rows_per_block": rpb, "nt_load": ntl, "nt_store": nts})
        res[name] = {"gbs": round(best[0]), **best[1]}
        del sets, ins, outs
        torch.cuda.empty_cache()
    return res


LDS_FORMS = ("ds_read_b128", "ds_read_b64", "ds_read_b64_tr_b16", "ds_read_b32", "ds_write_b32",
             "ds_write_b64", "ds_write_b128", "ds_add_f32", "ds_read_b128 half-wave broadcast")


def _probe_lib():
    import ctypes  # noqa: PLC0415

    path = HERE / "libkrsi_probe.so"
    if not path.exists():
        raise RuntimeError(f"{path} is missing: run kernel-rsi_amd/build.py first")
    lib = ctypes.CDLL(str(path))
    lib.krsi_probe_lds_rate.restype = ctypes.c_int
    lib.krsi_probe_lds_rate.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 3
    lib.krsi_probe_lds_form_bytes.restype = ctypes.c_int
    lib.krsi_probe_lds_form_bytes.argtypes = [ctypes.c_int]
    lib.krsi_probe_lds_banks.restype = ctypes.c_int
    lib.krsi_probe_lds_banks.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p]
    return lib


def probe_lds(quick: bool = False) -> dict:
    """LDS bytes per clock per CU of each access form (libkrsi_probe.so krsi_probe_lds_rate): one
    workgroup per CU, 8 and 16 waves, each wave 8 independent accesses per wait; clocks are each
    workgroup's s_memtime cycles over its loop, averaged over the CUs."""
    lib = _probe_lib()
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    cycles = torch.zeros(ncu, dtype=torch.int64, device="cuda")
    out = {}
    for threads in (512, 1024):
        sink = torch.empty(ncu * threads, dtype=torch.int32, device="cuda")
        for form, name in enumerate(LDS_FORMS):
            iters = 128 if form == 7 else (1024 if quick else 4096)
            for it in (8, iters):  # a short warm-up launch, then the timed one
                if lib.krsi_probe_lds_rate(form, ncu, threads, it, sink.data_ptr(), cycles.data_ptr(), stream) != 0:
                    raise RuntimeError(f"krsi_probe_lds_rate({form}, {ncu}, {threads}, {it}) failed")
            torch.cuda.synchronize()
            mean_cyc = cycles.double().mean().item()
            nbytes = iters * 8 * lib.krsi_probe_lds_form_bytes(form) * (threads // 64)
            out.setdefault(name, {})[f"{threads // 64} waves/CU"] = round(nbytes / mean_cyc, 1)
    return out


def lds_bank_patterns_run(iters: int = 100) -> int:
    """Launch the bank-pattern probe once per pattern of probe/lds_banks.py (one wave each), for a
    counter run: rocprofv3 --kernel-trace --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS -- python3
    kernel-rsi_amd/hw.py --lds-banks. Returns the number of patterns."""
    sys.path.insert(0, str(HERE / "probe"))
    import lds_banks  # noqa: PLC0415

    pats = lds_banks.patterns()
    for p in pats:
        assert len(p) == 64 and all(a % 16 == 0 and 0 <= a < 32768 - 16 for a in p), "pattern out of range"
    lib = _probe_lib()
    addr = torch.tensor([a for p in pats for a in p], dtype=torch.int32, device="cuda")
    sink = torch.empty(64, dtype=torch.int32, device="cuda")
    if lib.krsi_probe_lds_banks(addr.data_ptr(), len(pats), iters, sink.data_ptr(),
                                torch.cuda.current_stream().cuda_stream) != 0:
        raise RuntimeError("krsi_probe_lds_banks failed")
    torch.cuda.synchronize()
    return len(pats)


def probe_launch(clock: Clock) -> dict:
    """Microseconds per tiny kernel: one stream launch of a torch op, one graph replay."""
    x = torch.zeros(1, device="cuda")
    per_launch = clock.ms(lambda: x.add_(1.0), 200) * 1e3
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        x.add_(1.0)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        x.add_(1.0)
    per_replay = clock.ms(g.replay, 200) * 1e3
    return {"launch_us_torch": round(per_launch, 1), "launch_us_graph_replay": round(per_replay, 1)}


def collect(quick: bool = False) -> dict:
    props = torch.cuda.get_device_properties(0)
    clock = Clock(samples=3 if quick else 7)
    tflops = probe_gemm(clock, 4096 if quick else 8192)
    tflops["skinny_bf16"] = probe_skinny(clock)
    torch.cuda.empty_cache()
    rec = {"device": product_name(props), "torch_device_name": props.name,
           "arch": props.gcnArchName, "cus": props.multi_processor_count,
           "l2_mb": round(getattr(props, "L2_cache_size", 0) / 2 ** 20, 1),
           "memory_gb": round(props.total_memory / 2 ** 30, 1), "tflops": tflops}
    rec.update(probe_bandwidth(clock))
    rec["stream_kernel_gbs"] = probe_stream(clock, quick)
    rec["pattern_probe_gbs"] = probe_patterns(clock, quick)
    rec["lds_bytes_per_clk_per_cu"] = probe_lds(quick)
    stream_bw = max(rec["bw_copy_gbs"], rec["bw_read_gbs"])
    rec["ridge_flop_per_byte"] = {k: round(v * 1e3 / stream_bw, 1) for k, v in tflops.items()
                                  if isinstance(v, (int, float))}
    rec["published_peaks"] = dict(PUBLISHED)
    rec["default_half_dtype"] = "bf16"
    rec["features"] = {"bf16_mfma": True, "fp8": True, "tf32": False}
    rec.update(probe_launch(clock))
    rec.update({"torch": torch.__version__, "hip": torch.version.hip})
    return rec


def write(rec: dict, root: Path = HERE / "hardware") -> list[Path]:
    """The record under the product's name and, if it differs, under torch's device name."""
    root.mkdir(parents=True, exist_ok=True)
    paths = [root / f"{slug(rec['device'])}.json"]
    alias = root / f"{slug(rec['torch_device_name'])}.json"
    if alias != paths[0]:
        paths.append(alias)
    text = json.dumps(rec, indent=2) + "\n"
    for p in paths:
        p.write_text(text)
    return paths


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--quick", action="store_true", help="smaller GEMM and fewer samples")
    ap.add_argument("--out-dir", type=Path, default=HERE / "hardware", help="where the record goes")
    ap.add_argument("--stream-only", action="store_true",
                    help="only the streaming-kernel ceilings, printed, no record written")
    ap.add_argument("--lds-only", action="store_true", help="only the LDS rates, printed, no record written")
    ap.add_argument("--lds-banks", action="store_true",
                    help="only the bank-pattern probe's launches (for a counter run), no record written")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("hw.py measures a GPU; none is visible")
    if args.lds_banks:
        print(f"launched {lds_bank_patterns_run()} bank patterns", flush=True)
        return 0
    if args.lds_only:
        for name, v in probe_lds(args.quick).items():
            print(f"{name}: {v}", flush=True)
        return 0
    if args.stream_only:
        for mix, v in probe_stream(Clock(samples=5), args.quick).items():
            print(f"{mix}: {v}", flush=True)
        for name, v in probe_patterns(Clock(samples=5), args.quick).items():
            print(f"{name}: {v}", flush=True)
        return 0
    rec = collect(args.quick)
    width = max(map(len, rec))
    for k, v in rec.items():
        print(f"{k:>{width}}  {v}")
    for p in write(rec, args.out_dir):
        print(f"wrote {p}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
