#!/usr/bin/env python3
"""Re-run the library's self-tests on this GPU and keep the results as a record.

  python kernel-rsi_amd/replay.py [module ...]

The record's schema is what the reference's tooling reads (tools/replay.py:35-42, written by
library/replay/<gpu>.json). The schema is:
  * {"versions": {...}, "library": {module: selftest() minus "checks"}, "regions": {}}
The self-tests are those of the public kernel modules in library/. The private ones start with
an underscore. Each self-test checks three things against the fp32 reference and the eager
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
    record = {"versions": info, "library": {}, "regions": {}}
    for name in args.modules or kernel_modules():
        record["library"][name] = run_one(name)
        print(summary(name, record["library"][name]), flush=True)
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
