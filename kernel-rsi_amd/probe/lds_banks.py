#!/usr/bin/env python3
"""Bank-conflict model of ds_read_b128 on gfx950, fitted to counter readings.

  rocprofv3 --kernel-trace --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS --output-format csv -d <dir> -o run -- \\
      python3 kernel-rsi_amd/hw.py --lds-banks
  python3 kernel-rsi_amd/probe/lds_banks.py <dir>/run_counter_collection.csv

hw.py --lds-banks launches the probe (libkrsi_probe.so krsi_probe_lds_banks) once per pattern
below: one wave reading 128 bits per lane at the pattern's byte addresses, 800 times. This
script turns each dispatch's counters into conflict cycles per read and scores candidate
models of how the LDS serves a wave's 64 lanes. A model splits the lanes into 4 groups of 16,
each served in one pass over 64 banks of 4 bytes, where lanes on the same address share a
read (broadcast) and every further distinct address on a bank costs one cycle. Candidates:
groups by any 2 lane-index bits, and groups by lane bit 5 with the parity of any subset of the
other bits. The patterns: 10 random ones (8 rows x 16 bank quads), 15 that put 4 lanes
differing in 2 chosen bits on one quad, and the attention kernels' bias-window reads (forward
and dK/dV lane orders).
"""
from __future__ import annotations

import collections
import csv
import itertools
import random
import sys

READS_PER_DISPATCH = 100 * 8
INIT_WRITES = 8192 // 64  # the kernel's LDS fill, per wave


def _bias_addr(x0: int, wld: int = 208, b0: int = 4) -> int:
    """Byte address of read_bias16's first 128-bit read for window entry x0 (4 copies, copy cc
    at cc*WLD, copy 0 at 4, the read taken from the copy that 16-byte-aligns x0)."""
    cc = (-x0) & 3
    return ((b0 if cc == 0 else cc * wld) + x0 + cc) * 4


def _kperm(l: int) -> int:
    return 2 * (l & 15) + (l >> 4)


def patterns() -> list[list[int]]:
    rnd = random.Random(1)
    pats = [[rnd.randrange(8) * 256 + rnd.randrange(16) * 16 for _ in range(64)] for _ in range(10)]
    for b1, b2 in itertools.combinations(range(6), 2):
        others = [b for b in range(6) if b not in (b1, b2)]
        pats.append([(((l >> b1) & 1) | (((l >> b2) & 1) << 1)) * 256
                     + sum(((l >> b) & 1) << i for i, b in enumerate(others)) * 16 for l in range(64)])
    # 128-query forward block, wave 0, key block 0: x0 = 4g + 127 - l % 32
    pats.append([_bias_addr(4 * (l >> 5) + 127 - (l & 31)) for l in range(64)])
    # 128-key dK/dV block, wave 0, query block 0: x0 = 127 - kperm(l % 32) + 4g
    pats.append([_bias_addr(127 - _kperm(l & 31) + 4 * (l >> 5)) for l in range(64)])
    return pats


def names() -> list[str]:
    return ([f"random {k}" for k in range(10)]
            + [f"4 lanes per quad differing in bits {b1},{b2}" for b1, b2 in itertools.combinations(range(6), 2)]
            + ["forward bias read", "dK/dV bias read"])


def model_cycles(addrs: list[int], groups: list[list[int]]) -> int:
    total = 0
    for grp in groups:
        banks = collections.defaultdict(set)
        for lane in grp:
            for w in range(4):
                dw = addrs[lane] // 4 + w
                banks[dw % 64].add(dw)
        total += max(len(s) for s in banks.values()) - 1
    return total


def candidate_models() -> dict[str, list[list[int]]]:
    out = {}
    for b1, b2 in itertools.combinations(range(6), 2):
        key = lambda l, b1=b1, b2=b2: ((l >> b1) & 1) | (((l >> b2) & 1) << 1)  # noqa: E731
        out[f"groups by lane bits {b1},{b2}"] = [[l for l in range(64) if key(l) == k] for k in range(4)]
    for mask in range(1, 32):
        bits = [b for b in range(5) if mask >> b & 1]
        key = lambda l, mask=mask: ((l >> 5) & 1) * 2 + (bin(l & mask).count("1") & 1)  # noqa: E731
        out[f"lane bit 5 and parity of bits {','.join(map(str, bits))}"] = [
            [l for l in range(64) if key(l) == k] for k in range(4)]
    return out


def measured(csv_path: str) -> list[float]:
    per = collections.defaultdict(dict)
    for row in csv.DictReader(open(csv_path)):
        if "lds_bank_kernel" in row["Kernel_Name"]:
            per[int(row["Dispatch_Id"])][row["Counter_Name"]] = float(row["Counter_Value"])
    out = []
    for d in sorted(per):
        reads = per[d]["SQ_INSTS_LDS"] - INIT_WRITES
        assert reads == READS_PER_DISPATCH, f"dispatch {d}: {reads} reads"
        out.append(per[d]["SQ_LDS_BANK_CONFLICT"] / reads)
    return out


def main(argv: list[str]) -> int:
    meas = measured(argv[1])
    pats = patterns()
    assert len(meas) == len(pats), f"{len(meas)} dispatches for {len(pats)} patterns"
    scored = []
    for name, groups in candidate_models().items():
        pred = [model_cycles(p, groups) for p in pats]
        scored.append((sum(abs(a - b) for a, b in zip(pred, meas)), name, pred))
    scored.sort(key=lambda s: s[0])
    best = scored[0]
    naive = next(s for s in scored if s[1] == "groups by lane bits 4,5")
    print(f"best model: {best[1]} (total |error| {best[0]:g} cycles over {len(pats)} patterns)")
    print(f"next best: {scored[1][1]} ({scored[1][0]:g}); 16 consecutive lanes per group: {naive[0]:g}")
    print("| pattern | measured cycles/read | best model | 16 consecutive lanes |")
    print("|---|---:|---:|---:|")
    for n, m, b, c in zip(names(), meas, best[2], naive[2]):
        print(f"| {n} | {m:g} | {b} | {c} |")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
