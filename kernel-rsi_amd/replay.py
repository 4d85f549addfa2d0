#!/usr/bin/env python3
"""Run every library module's selftest() on this GPU and record the results.

  python kernel-rsi_amd/replay.py

Mirrors the reference's tools/replay.py (library part, :25-50): each non-underscore module in
library/ is loaded, its selftest() (fp32 reference vs eager original vs kernel, then the kernel
under torch.compile(fullgraph=True), and timing) is run, and the dicts minus "checks" go to
library/replay/<device slug>.json, one line per module on stdout. Exit status 1 if any fails.
The file name is the slug of torch's device name, as the reference's tools compute it, so they
find this file on the same machine.
"""
from __future__ import annotations

import importlib.util
import json
import sys
import traceback
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "library"
sys.path.insert(0, str(LIB))

import torch  # noqa: E402

from _harness import versions  # noqa: E402


def slug(text: str) -> str:
    return "".join(c if c.isalnum() else "_" for c in text).strip("_").lower()


def main() -> int:
    if not torch.cuda.is_available():
        raise SystemExit("no GPU")
    info = versions()
    info["arch"] = torch.cuda.get_device_properties(0).gcnArchName
    out = {"versions": info, "library": {}, "regions": {}}
    for f in sorted(p for p in LIB.glob("*.py") if not p.name.startswith("_")):
        try:
            spec = importlib.util.spec_from_file_location(f"krsi_lib_{f.stem}", f)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            r = mod.selftest()
            out["library"][f.stem] = {k: v for k, v in r.items() if k != "checks"}
            c = r.get("compiled", {})
            ctxt = (f" | compile(fullgraph): {'ok' if c.get('pass') else 'FAIL'}"
                    + (f" {c['kernel_us']:.1f} us vs compiled ref {c['reference_us']:.1f} us "
                       f"{c['speedup']:.2f}x ({c['significance']})" if "kernel_us" in c else f" {c.get('error', '')}"))
            print(f"{f.stem:<18} {'PASS' if r['pass'] else 'FAIL'}  eager: {r['kernel_us']:.1f} us vs "
                  f"{r['reference_us']:.1f} us {r['speedup']:.2f}x ({r['significance']}){ctxt}", flush=True)
        except Exception as e:  # noqa: BLE001 - one broken module must not hide the others
            out["library"][f.stem] = {"pass": False, "error": f"{type(e).__name__}: {e}"}
            print(f"{f.stem:<18} ERROR {type(e).__name__}: {str(e)[:200]}", flush=True)
            traceback.print_exc(limit=1)
    path = LIB / "replay" / f"{slug(info['device'])}.json"
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(out, indent=2, default=str) + "\n")
    bad = [k for k, v in out["library"].items() if not v["pass"]]
    print(f"\nsaved {path}" + (f"\nFAILED: {bad}" if bad else ""))
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
