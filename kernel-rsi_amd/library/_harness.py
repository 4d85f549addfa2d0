"""Parity and timing harness of the library self-tests.

Restates the acceptance criterion and timing protocol of the reference's
tools/common.py so that `selftest()` results mean the same thing:
  * compare()            - tools/common.py:322-392: an output passes if no element is
                           further from the fp32 reference than `slack` x the eager
                           original's worst error (+ 1e-3 x max|ref| + 1e-6), its
                           relative L2 error is within `slack` x the original's
                           (+ 1e-5), and no row (last dim >= 64) has a relative error
                           above `row_slack` x the original's on the same row.
  * pure_fp32            - tools/common.py:154-163 (TF32 off for the fp32 reference).
  * time_calls/time_ab   - tools/common.py:238-298, 433-464: graph replay, median of
                           reps, eager fallback on a host sync; interleaved rounds.
  * significance         - tools/common.py:467-473.
  * selftest_autograd    - tools/common.py:476-518: fp32 reference vs eager original vs
                           candidate, output and every float input's gradient under one
                           random cotangent (randn * 1e-2), torch.compile(fullgraph=True)
                           check, and timing; same return keys (tools/replay.py:35-42).
"""
from __future__ import annotations

import torch
from torch.utils._pytree import tree_flatten


def tensors(x) -> list[torch.Tensor]:
    return [t for t in tree_flatten(x)[0] if isinstance(t, torch.Tensor)]


class pure_fp32:
    """Context manager: matmul and cuDNN/MIOpen convolutions in true fp32."""

    def __enter__(self):
        self._saved = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32)
        torch.backends.cuda.matmul.allow_tf32 = False
        torch.backends.cudnn.allow_tf32 = False
        return self

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = self._saved
        return False


def versions() -> dict:
    dev = torch.cuda.get_device_name(torch.cuda.current_device()) if torch.cuda.is_available() else "cpu"
    return {"device": dev, "torch": torch.__version__, "cuda": torch.version.cuda,
            "hip": getattr(torch.version, "hip", None), "triton": None}


# ------------------------------------------------------------------ numerics
def _bad_dims(bad: torch.Tensor) -> list[str]:
    """For each dim, which indices hold failing elements (the bug's footprint)."""
    notes = []
    for d in range(bad.dim()):
        rest = tuple(i for i in range(bad.dim()) if i != d)
        hit = (bad.any(dim=rest) if rest else bad).nonzero().flatten()
        if hit.numel() == 0:
            continue
        n = bad.shape[d]
        s = f"dim{d} (size {n}): {hit.numel()} bad"
        if hit.numel() < n:
            s += f", first {int(hit[0])}, last {int(hit[-1])}"
            if hit.numel() <= 8:
                s += f", at {hit.tolist()}"
        notes.append(s)
    return notes


def _unravel(flat: int, shape) -> list[int]:
    idx = []
    for size in reversed(shape):
        idx.append(flat % size)
        flat //= size
    return idx[::-1]


def _judge(r: torch.Tensor, o: torch.Tensor, c: torch.Tensor, slack: float, row_slack: float) -> dict:
    r, o, c = r.float(), o.float(), c.float()
    peak = r.abs().max().item() or 1.0
    eo, ec = (o - r).abs(), (c - r).abs()
    rnorm = r.norm() + 1e-12
    budget = slack * eo.max() + 1e-3 * peak + 1e-6
    bad = (ec > budget) | ~torch.isfinite(c)
    res = {"max_err": ec.max().item(), "orig_max_err": eo.max().item(),
           "rel_l2": (ec.norm() / rnorm).item(), "orig_rel_l2": (eo.norm() / rnorm).item(),
           "nonfinite": int((~torch.isfinite(c)).sum()), "bad_fraction": bad.float().mean().item()}
    ok = not bool(bad.any()) and res["rel_l2"] <= slack * res["orig_rel_l2"] + 1e-5
    # Per-row check against the original's error on the same row: a bug confined to
    # a few rows (one head, one token) hardly moves the tensor-wide numbers.
    if r.dim() >= 2 and r.shape[-1] >= 64 and r.numel() // r.shape[-1] >= 2:
        rr = r.reshape(-1, r.shape[-1])
        rn = rr.norm(dim=1)
        live = rn > 1e-6 * (rn.max() + 1e-30)
        if bool(live.any()):
            row_c = ((c - r).reshape(rr.shape).norm(dim=1) / (rn + 1e-30))[live]
            row_o = ((o - r).reshape(rr.shape).norm(dim=1) / (rn + 1e-30))[live]
            ref_row = torch.maximum(row_o, row_o.median() + 1e-5)
            over = row_c > row_slack * ref_row
            res["bad_rows"] = int(over.sum())
            if res["bad_rows"]:
                ok = False
                w = int((row_c / ref_row).argmax())
                res["worst_row"] = {"row": int(live.nonzero().flatten()[w]), "rel": row_c[w].item(),
                                    "orig_rel": row_o[w].item()}
    if not ok and bool(bad.any()):
        flat = int(ec.flatten().nan_to_num(float("inf")).argmax())
        res["worst"] = {"index": _unravel(flat, r.shape), "ref": r.flatten()[flat].item(),
                        "got": c.flatten()[flat].item()}
        res["where"] = _bad_dims(bad)
    res["pass"] = ok
    return res


def compare(ref32, orig, cand, *, slack: float = 2.0, row_slack: float = 3.0) -> dict:
    """Judge `cand` against an fp32 run `ref32`, with the eager original `orig` as the
    noise yardstick. Returns {"pass": bool, "outputs": [per-tensor report]}."""
    rs, os_, cs = tensors(ref32), tensors(orig), tensors(cand)
    if len(rs) != len(cs):
        return {"pass": False, "reason": f"output count {len(cs)} != {len(rs)}"}
    outs, ok = [], True
    for i, (r, o, c) in enumerate(zip(rs, os_, cs)):
        item = {"output": i, "shape": list(r.shape), "dtype": str(c.dtype)}
        if tuple(c.shape) != tuple(r.shape):
            item.update({"pass": False, "reason": f"shape {list(c.shape)} != {list(r.shape)}"})
        elif not r.is_floating_point():
            item.update({"pass": bool(torch.equal(c.to(r.dtype), r)), "exact": True})
        else:
            item.update(_judge(r, o, c, slack, row_slack))
        ok = ok and item["pass"]
        outs.append(item)
    return {"pass": ok, "outputs": outs}


# -------------------------------------------------------------------- timing
def _sync_probe(fns) -> str | None:
    """Run the first callable with sync debugging set to error; describe the first host sync."""
    prev = torch.cuda.get_sync_debug_mode()
    try:
        torch.cuda.set_sync_debug_mode("error")
        for f in fns[:1]:
            f()
        return None
    except RuntimeError as e:
        return str(e).splitlines()[0][:120]
    finally:
        torch.cuda.set_sync_debug_mode(prev)
        torch.cuda.synchronize()


def _event_ms(run, reps: int, per: int) -> list[float]:
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = []
    for _ in range(reps):
        start.record()
        run()
        end.record()
        end.synchronize()
        out.append(start.elapsed_time(end) / per)
    return sorted(out)


def time_calls(fns: list, warmup: int = 5, reps: int = 20, graph: bool = True) -> dict:
    """Median device time per call of fns (each a zero-arg callable). Graph replay first;
    eager events if the callables sync with the host or cannot be captured."""
    torch.cuda.synchronize()
    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()

    def eager():
        for f in fns:
            f()

    host = _event_ms(eager, reps, len(fns))
    res = {"host_ms": host[len(host) // 2], "copies": len(fns)}
    if not graph:
        res.update(device_ms=res["host_ms"], mode="eager")
        return res
    why = _sync_probe(fns)
    if why:
        res.update(device_ms=res["host_ms"], mode="eager", note=f"not graph-capturable: host sync ({why})")
        return res
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            eager()
        g.replay()
        torch.cuda.synchronize()
        samples = _event_ms(g.replay, reps, len(fns))
        med = samples[len(samples) // 2]
        res.update(device_ms=med, mode="graph", spread=(samples[-1] - samples[0]) / max(med, 1e-9))
        del g
    except Exception as e:  # noqa: BLE001 - capture is best effort
        torch.cuda.synchronize()
        res.update(device_ms=res["host_ms"], mode="eager", note=f"graph capture failed: {str(e)[:200]}")
    return res


def time_ab(variants: dict, rounds: int = 5, reps: int = 10) -> dict:
    """Time variants (name -> list of callables) in interleaved rounds, all in one mode."""
    probe = {name: time_calls(fns, warmup=3, reps=3) for name, fns in variants.items()}
    use_graph = all(p["mode"] == "graph" for p in probe.values())
    eager_only = [n for n, p in probe.items() if p["mode"] != "graph"]
    dev = {n: [] for n in variants}
    host = {n: [] for n in variants}
    first = {}
    for k in range(rounds):
        order = list(variants) if k % 2 == 0 else list(reversed(list(variants)))
        for name in order:
            t = time_calls(variants[name], warmup=3 if k else 5, reps=reps, graph=use_graph)
            if eager_only:
                t["note"] = (f"all variants timed eagerly: {eager_only} could not be graph-captured "
                             f"({probe[eager_only[0]].get('note', '')[:120]})")
            dev[name].append(t["device_ms"])
            host[name].append(t["host_ms"])
            first.setdefault(name, t)
    out = {}
    for name in variants:
        d, hs = sorted(dev[name]), sorted(host[name])
        dm, hm = d[len(d) // 2], hs[len(hs) // 2]
        out[name] = {**first[name], "device_ms": dm, "rounds": d, "noise": (d[-1] - d[0]) / max(dm, 1e-12),
                     "host_ms": hm, "host_rounds": hs, "host_noise": (hs[-1] - hs[0]) / max(hm, 1e-12)}
    return out


def significance(base: dict, cand: dict) -> str:
    """'faster' / 'slower' only when the round ranges do not overlap."""
    if max(cand["rounds"]) < min(base["rounds"]):
        return "faster"
    if min(cand["rounds"]) > max(base["rounds"]):
        return "slower"
    return "within noise"


def selftest_autograd(fn, ref, inputs: list, slack: float = 2.0, time: bool = True) -> dict:
    """Check fn against ref (output and the gradient of every float input) under one
    random cotangent, then under torch.compile(fullgraph=True), and time both."""
    def run(f, xs, dtype=None, cot=None):
        xs = [x.detach().to(dtype or x.dtype).requires_grad_(x.is_floating_point()) for x in xs]
        out = f(*xs)
        cot = torch.randn_like(out.float()).mul_(1e-2) if cot is None else cot
        grads = torch.autograd.grad(out, [x for x in xs if x.requires_grad], cot.to(out.dtype))
        return [out.detach()] + [g.detach() for g in grads], cot

    with pure_fp32():
        ref32, cot = run(ref, inputs, torch.float32)
    orig, _ = run(ref, inputs, cot=cot)
    cand, _ = run(fn, inputs, cot=cot)
    checks = compare(ref32, orig, cand, slack=slack)
    leaves = [x.detach().requires_grad_(x.is_floating_point()) for x in inputs]
    gout = cot.to(inputs[0].dtype)

    def step(f):
        return lambda: torch.autograd.grad(f(*leaves), [x for x in leaves if x.requires_grad], gout)

    variants = {"reference": [step(ref)], "kernel": [step(fn)]}
    compiled: dict = {}
    try:
        torch._dynamo.reset()
        cfn, cref = torch.compile(fn, fullgraph=True), torch.compile(ref)
        cand_c, _ = run(cfn, inputs, cot=cot)
        compiled = {"pass": compare(ref32, orig, cand_c, slack=slack)["pass"]}
        variants.update(compiled_reference=[step(cref)], compiled_kernel=[step(cfn)])
    except Exception as e:  # noqa: BLE001
        compiled = {"pass": False, "error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}
    res = {"pass": checks["pass"] and compiled.get("pass", False), "checks": checks, **versions()}
    if not time:
        return {**res, "compiled": compiled}
    t = time_ab(variants, rounds=3)
    us = {k: round(v["device_ms"] * 1000, 1) for k, v in t.items()}
    if "compiled_kernel" in t:
        compiled.update(kernel_us=us["compiled_kernel"], reference_us=us["compiled_reference"],
                        speedup=round(us["compiled_reference"] / us["compiled_kernel"], 2),
                        significance=significance(t["compiled_reference"], t["compiled_kernel"]))
    return {**res, "reference_us": us["reference"], "kernel_us": us["kernel"],
            "speedup": round(us["reference"] / us["kernel"], 2),
            "significance": significance(t["reference"], t["kernel"]), "compiled": compiled}
