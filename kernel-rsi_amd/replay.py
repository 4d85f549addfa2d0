#!/usr/bin/env python3
"""Re-run the library's self-tests on this GPU and keep the results as a record.

  python kernel-rsi_amd/replay.py [module ...]

The record's schema is what the reference's tooling reads (tools/replay.py:35-42, written by
library/replay/<gpu>.json). The schema is:
  * {"versions": {...}, "library": {module: selftest() minus "checks"}, "regions": {}}
The self-tests are those of the public kernel modules in library/. The private ones start with
an underscore. Beside the schema, "host_costs" gives per module the host's time to enqueue one
eager fwd+bwd at the selftest shape and the device's time for one, which shows where a
training step of those sizes is bound by the host. Each self-test checks three things against the fp32 reference and the eager
original: the eager kernel, the kernel under torch.compile(fullgraph=True), and their timings.

A module that raises is recorded as failed with its error, and the others still run. The exit
status is 1 if any module failed. The record is written under the product's name (see hw.py)
and, if torch reports another device name, under that name's slug too. The second copy is the
file the reference's tooling opens on this machine.
"""
from __future__ import annotations

import argparse
import importlib
import json
import sys
import traceback
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "library"
for _p in (HERE, LIBRARY):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

import hw  # noqa: E402  (kernel-rsi_amd/hw.py: product name and slug)
from _harness import versions  # noqa: E402


def kernel_modules() -> list[str]:
    return sorted(p.stem for p in LIBRARY.glob("*.py") if not p.stem.startswith("_"))


def run_one(name: str) -> dict:
    """selftest() of library/<name>.py; its result without the per-tensor reports, or the error."""
    try:
        result = importlib.import_module(name).selftest()
    except Exception as e:  # noqa: BLE001 - a broken module is a recorded failure
        traceback.print_exc(limit=2)
        return {"pass": False, "error": f"{type(e).__name__}: {e}"}
    return {k: v for k, v in result.items() if k != "checks"}


def _selftest_step(name: str):
    """(leaves, fn, cotangent) of the module's selftest shape, for the host-cost probe."""
    import geglu
    import relpos_attention
    import rmsnorm
    g = torch.Generator(device="cuda").manual_seed(0)

    def rnd(*shape, dtype=torch.bfloat16, scale=1.0):
        return (scale * torch.randn(*shape, device="cuda", generator=g)).to(dtype)
    if name == "rmsnorm":
        x, w = rnd(4096, 1024), (1 + rnd(1024, scale=0.02, dtype=torch.float32)).to(torch.bfloat16)
        return [x, w], lambda a, b: rmsnorm.rmsnorm(a, b, 1e-6), rnd(4096, 1024)
    if name == "geglu":
        return [rnd(2048, 5632)], geglu.geglu, rnd(2048, 2816)
    if name == "relpos_attention":
        B, S, H, D = 4, 512, 16, 64
        return ([rnd(B * S, 3 * H * D, scale=0.6), rnd(H, 2 * S - 1, dtype=torch.float32)],
                lambda q, p: relpos_attention.relpos_attention(q, p, B, S, H, D, 1.0), rnd(B * S, H * D))
    return None


def host_cost(name: str, calls: int = 50) -> dict:
    """Per eager fwd+bwd (the module function, then torch.autograd.grad) at the selftest shape:
    the host's time to enqueue one (measured on the CPU while the GPU is held busy, so nothing
    waits on the device) and the device's time for one when the queue is full. When host_us is
    the larger, a training step of these sizes is bound by the host, whatever the kernels do."""
    import time
    spec = _selftest_step(name)
    if spec is None:
        return {}
    leaves, fn, cot = spec
    xs = [t.detach().requires_grad_(True) for t in leaves]

    def step():
        torch.autograd.grad(fn(*xs), xs, cot)
    for _ in range(5):
        step()
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))  # ~0.1 s of device time ahead of the calls
    t0 = time.perf_counter()
    for _ in range(calls):
        step()
    host = (time.perf_counter() - t0) / calls
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2e8))
    a.record()
    for _ in range(calls):
        step()
    b.record()
    b.synchronize()
    dev = a.elapsed_time(b) / calls * 1e-3
    return {"host_us_per_fwd_bwd": round(host * 1e6, 1), "device_us_per_fwd_bwd": round(dev * 1e6, 1),
            "host_bound": host > dev}


def summary(name: str, r: dict) -> str:
    if "error" in r and "kernel_us" not in r:
        return f"{name:<18} ERROR  {r['error'][:200]}"
    parts = [f"{name:<18} {'PASS' if r['pass'] else 'FAIL'}",
             f"eager {r['kernel_us']:.1f} us (reference {r['reference_us']:.1f} us, "
             f"{r['speedup']:.2f}x, {r['significance']})"]
    c = r.get("compiled", {})
    if "kernel_us" in c:
        parts.append(f"compiled {c['kernel_us']:.1f} us (reference {c['reference_us']:.1f} us, "
                     f"{c['speedup']:.2f}x, {c['significance']})"
                     + ("" if c.get("pass") else " NOT EQUIVALENT"))
    else:
        parts.append(f"compiled: {c.get('error', 'not run')}")
    return " | ".join(parts)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("modules", nargs="*", help="library modules to run (default: all)")
    ap.add_argument("--out-dir", type=Path, default=LIBRARY / "replay", help="where the record goes")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("replay.py runs the kernels; no GPU is visible")
    props = torch.cuda.get_device_properties(0)
    info = {**versions(), "arch": props.gcnArchName, "product": hw.product_name(props)}
    record = {"versions": info, "library": {}, "regions": {}, "host_costs": {}}
    for name in args.modules or kernel_modules():
        record["library"][name] = run_one(name)
        print(summary(name, record["library"][name]), flush=True)
        try:
            record["host_costs"][name] = host_cost(name)
        except Exception as e:  # noqa: BLE001 - the cost probe is informative only
            record["host_costs"][name] = {"error": f"{type(e).__name__}: {e}"}
        print(f"{'':<18} host cost per eager fwd+bwd: {record['host_costs'][name]}", flush=True)
    text = json.dumps(record, indent=2, default=str) + "\n"
    out_dir = args.out_dir
    out_dir.mkdir(parents=True, exist_ok=True)
    targets = {out_dir / f"{hw.slug(info['product'])}.json", out_dir / f"{hw.slug(info['device'])}.json"}
    for p in sorted(targets):
        p.write_text(text)
        print(f"wrote {p}")
    failed = [n for n, r in record["library"].items() if not r["pass"]]
    if failed:
        print(f"failed: {', '.join(failed)}")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
