"""Shared helpers of the test suite: seeded inputs, the parity assertion and case logging."""
from __future__ import annotations

import sys

import torch

import krsi_oracle as O
from _harness import compare


def log(msg: str) -> None:
    """Name the case before a GPU step, so a run that dies mid-way still says where."""
    print(f"[krsi] {msg}", file=sys.stderr, flush=True)


def assert_parity(names, ref32, orig, cand, slack: float = 2.0, row_slack: float = 3.0,
                  extra_msg: str = "") -> dict:
    """The reference's acceptance criterion (tools/common.py:322-392) with slack 2: every
    output within 2x the eager bf16 original's worst error and rel-L2, per-row check at 3x."""
    res = compare(ref32, orig, cand, slack=slack, row_slack=row_slack)
    lines = []
    for name, o in zip(names, res.get("outputs", [])):
        if "rel_l2" in o:
            ratio = o["rel_l2"] / max(o["orig_rel_l2"], 1e-12)
            lines.append(f"{name}: rel_l2 {o['rel_l2']:.3e} (orig {o['orig_rel_l2']:.3e}, x{ratio:.2f}) "
                         f"max_err {o['max_err']:.3e} (orig {o['orig_max_err']:.3e}) "
                         f"bad_rows {o.get('bad_rows', 0)} pass {o['pass']}")
        else:
            lines.append(f"{name}: {o}")
    log("; ".join(lines))
    assert res["pass"], "parity failed " + extra_msg + "\n" + "\n".join(lines) + f"\n{res}"
    return res


def seeded(shape, seed, std=1.0, mean=0.0, dtype=torch.bfloat16, device="cuda"):
    return O.randn(shape, seed, std=std, mean=mean, dtype=dtype).to(device)
