"""Build libkrsi_hip.so, the gfx950 kernel library, from csrc/ with hipcc.

    python kernel-rsi_amd/build.py          # or __graft_entry__.build()

Every HIP source is compiled for gfx950 only (no CUDA/HIP dual path), in
parallel, and linked into kernel-rsi_amd/libkrsi_hip.so, which the ctypes
binding in library/_hip.py loads. The library links libamdhip64.so.7 by soname
and is loaded after torch, so it binds to the HIP runtime torch already loaded.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
OBJDIR = HERE / "_build"
LIB = HERE / "libkrsi_hip.so"
# The streaming-bandwidth probe of hw.py: its own library, not part of the kernel library.
PROBE_SRCS = [HERE / "probe" / "stream_probe.hip", HERE / "probe" / "lds_probe.hip"]
PROBE_LIB = HERE / "libkrsi_probe.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for all device code (they are not
# needed: the kernels are HBM- or MFMA-bound).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source extra flags. The attention kernels are scheduled by LLVM's max-ILP strategy: with
# the default one the backward kernels left more of their LDS and MFMA latency exposed (A/B at
# B4 H16 S4096 D64: backward 1.082 -> 1.064 ms; S = 512 and 2048: -4 % and -7 %; D = 72 at
# S = 1024: +2 %; forward unchanged; outputs bitwise the same).
EXTRA_FLAGS = {"relpos_attn.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).is_file():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libkrsi_hip.so)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that
    # note is expected and filtered out.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in p.stderr.splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"build step failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    OBJDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    cmds = []
    objs = []
    for src in srcs:
        obj = OBJDIR / (src.stem + ".o")
        objs.append(obj)
        if src.suffix == ".hip":
            cmds.append([hipcc, *HIP_FLAGS, *EXTRA_FLAGS.get(src.name, []), f"-I{INCLUDE}", f"-I{CSRC}",
                         "-c", str(src), "-o", str(obj)])
        else:
            cmds.append(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([hipcc, *HIP_FLAGS, "-shared", "-o", str(tmp), *map(str, PROBE_SRCS)], verbose)
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
