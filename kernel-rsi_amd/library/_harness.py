"""Acceptance rule and timing used by every library module's selftest().

Two things are contract with the reference's tooling. Everything else here is this package's own.
  * The acceptance rule (tools/common.py:322-392). A candidate is measured against an fp32
    run, in units of the eager original's error against that same run. Each output passes if:
      - every element is within 2x the original's worst element error, plus
        1e-3 * max|ref| + 1e-6;
      - its relative L2 error is within 2x the original's, plus 1e-5;
      - on every row of length >= 64, its relative error is within 3x the original's on that
        row. The original's row error is floored at its median row error + 1e-5.
    The pass flag is that verdict, and the report keys are the ones the tooling reads.
  * The selftest() dictionary (tools/common.py:476-518, read by tools/replay.py:35-42).

Structure:
  * `Criterion` holds the constants. `_TensorReport` judges one output; `compare` walks the
    outputs.
  * `Timer` owns the zero-argument callables of one variant (rotated input copies). It
    measures them eagerly with HIP events. Unless one of them synchronises with the host, it
    also captures them once as a HIP graph and measures replays of that graph.
  * `time_ab` interleaves several Timers in alternating order, in one mode for all.
    `significance` names a difference only when the round ranges do not overlap.
  * `selftest_autograd` runs three trials on one shared cotangent: the fp32 reference, the
    eager original and the candidate. It repeats the candidate under
    torch.compile(fullgraph=True), then times forward + backward of each.
"""
from __future__ import annotations

import contextlib
import dataclasses

import torch
from torch.utils._pytree import tree_flatten


def tensors(x) -> list[torch.Tensor]:
    return [leaf for leaf in tree_flatten(x)[0] if isinstance(leaf, torch.Tensor)]


class pure_fp32(contextlib.AbstractContextManager):
    """Reference runs in true fp32: reduced-precision matmul/convolution paths switched off."""

    _FLAGS = ((torch.backends.cuda.matmul, "allow_tf32"), (torch.backends.cudnn, "allow_tf32"))

    def __enter__(self):
        self._was = [getattr(mod, name) for mod, name in self._FLAGS]
        for mod, name in self._FLAGS:
            setattr(mod, name, False)
        return self

    def __exit__(self, *exc):
        for (mod, name), value in zip(self._FLAGS, self._was):
            setattr(mod, name, value)
        return False


def versions() -> dict:
    if torch.cuda.is_available():
        device = torch.cuda.get_device_name(torch.cuda.current_device())
    else:
        device = "cpu"
    return {"device": device, "torch": torch.__version__, "cuda": torch.version.cuda,
            "hip": getattr(torch.version, "hip", None), "triton": None}


# ------------------------------------------------------------------ acceptance
@dataclasses.dataclass(frozen=True)
class Criterion:
    slack: float = 2.0        # element-wise and rel-L2 multiple of the original's error
    row_slack: float = 3.0    # per-row multiple (correct kernels' row ratios reach ~2x)
    peak_frac: float = 1e-3   # element budget floor, relative to max |ref|
    abs_floor: float = 1e-6
    rel_floor: float = 1e-5   # rel-L2 floor, and the floor added to the median row error
    min_row: int = 64         # rows shorter than this are too noisy to judge one by one


def _failure_map(bad: torch.Tensor) -> list[str]:
    """Per dimension, the indices that hold failing elements, read from their coordinates."""
    coords = bad.nonzero()
    lines = []
    for d, size in enumerate(bad.shape):
        hit = torch.unique(coords[:, d]).tolist()
        if not hit:
            continue
        text = f"dim {d}: {len(hit)} of {size} indices fail"
        if len(hit) < size:
            text += f", span {hit[0]}..{hit[-1]}"
            if len(hit) <= 8:
                text += f", {hit}"
        lines.append(text)
    return lines


class _TensorReport:
    """The verdict on one output, built from the candidate's and the original's errors."""

    def __init__(self, ref: torch.Tensor, orig: torch.Tensor, cand: torch.Tensor, crit: Criterion):
        self.ref = ref.float()
        self.d_orig = orig.float() - self.ref
        self.d_cand = cand.float() - self.ref
        self.cand = cand
        self.crit = crit
        self.finite = torch.isfinite(cand)

    def _elementwise(self, out: dict) -> torch.Tensor:
        crit = self.crit
        e_orig, e_cand = self.d_orig.abs(), self.d_cand.abs()
        peak = float(self.ref.abs().max()) or 1.0
        limit = crit.slack * e_orig.max() + crit.peak_frac * peak + crit.abs_floor
        bad = ~self.finite | (e_cand > limit)
        ref_norm = torch.linalg.vector_norm(self.ref) + 1e-12
        out["max_err"] = float(e_cand.max())
        out["orig_max_err"] = float(e_orig.max())
        out["rel_l2"] = float(torch.linalg.vector_norm(self.d_cand) / ref_norm)
        out["orig_rel_l2"] = float(torch.linalg.vector_norm(self.d_orig) / ref_norm)
        out["nonfinite"] = int((~self.finite).sum())
        out["bad_fraction"] = float(bad.float().mean())
        return bad

    def _rows(self, out: dict) -> bool:
        """False if some row's error is more than row_slack x the original's on that row."""
        width = self.ref.shape[-1] if self.ref.dim() >= 2 else 0
        if width < self.crit.min_row or self.ref.numel() // width < 2:
            return True
        ref_rows = torch.linalg.vector_norm(self.ref.reshape(-1, width), dim=1)
        keep = ref_rows > 1e-6 * (ref_rows.max() + 1e-30)
        if not bool(keep.any()):
            return True
        scale = ref_rows[keep] + 1e-30
        cand_rows = torch.linalg.vector_norm(self.d_cand.reshape(-1, width), dim=1)[keep] / scale
        orig_rows = torch.linalg.vector_norm(self.d_orig.reshape(-1, width), dim=1)[keep] / scale
        yardstick = orig_rows.clamp(min=float(orig_rows.median()) + self.crit.rel_floor)
        ratio = cand_rows / yardstick
        failing = ratio > self.crit.row_slack
        out["bad_rows"] = int(failing.sum())
        if not out["bad_rows"]:
            return True
        k = int(ratio.argmax())
        out["worst_row"] = {"row": int(keep.nonzero()[k, 0]), "rel": float(cand_rows[k]),
                            "orig_rel": float(orig_rows[k])}
        return False

    def verdict(self, out: dict) -> dict:
        bad = self._elementwise(out)
        ok = not bool(bad.any())
        ok = ok and out["rel_l2"] <= self.crit.slack * out["orig_rel_l2"] + self.crit.rel_floor
        ok = self._rows(out) and ok
        if not ok and bool(bad.any()):
            err = self.d_cand.abs().flatten().nan_to_num(nan=float("inf"))
            flat = int(err.argmax())
            idx = [int(i) for i in torch.unravel_index(torch.tensor(flat), self.ref.shape)]
            out["worst"] = {"index": idx, "ref": float(self.ref.flatten()[flat]),
                            "got": float(self.cand.float().flatten()[flat])}
            out["where"] = _failure_map(bad)
        out["pass"] = ok
        return out


def compare(ref32, orig, cand, *, slack: float = 2.0, row_slack: float = 3.0) -> dict:
    """Judge each tensor of `cand` against `ref32` (an fp32 run), with the eager original
    `orig` as the noise yardstick. Returns {"pass": bool, "outputs": [one report each]}."""
    crit = Criterion(slack=slack, row_slack=row_slack)
    refs, origs, cands = tensors(ref32), tensors(orig), tensors(cand)
    if len(cands) != len(refs):
        return {"pass": False, "reason": f"output count {len(cands)} != {len(refs)}"}
    reports = []
    for i, (r, o, c) in enumerate(zip(refs, origs, cands)):
        out = {"output": i, "shape": list(r.shape), "dtype": str(c.dtype)}
        if tuple(c.shape) != tuple(r.shape):
            out.update({"pass": False, "reason": f"shape {list(c.shape)} != {list(r.shape)}"})
        elif not r.is_floating_point():
            out.update({"pass": bool(torch.equal(c.to(r.dtype), r)), "exact": True})
        else:
            _TensorReport(r, o, c, crit).verdict(out)
        reports.append(out)
    return {"pass": all(o["pass"] for o in reports), "outputs": reports}


# ---------------------------------------------------------------------- timing
def _median(xs: list[float]) -> float:
    xs = sorted(xs)
    return xs[len(xs) // 2]


class Timer:
    """Device time per call of a list of zero-argument callables (one variant, its input
    copies rotated): HIP events around eager passes and around replays of one captured graph."""

    def __init__(self, fns):
        self.fns = list(fns)
        self.graph = None
        self.why_eager = None

    def run(self):
        for f in self.fns:
            f()

    def _per_call(self, body, reps: int) -> list[float]:
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(reps)]
        for start, stop in marks:
            start.record()
            body()
            stop.record()
            stop.synchronize()
        return [start.elapsed_time(stop) / len(self.fns) for start, stop in marks]

    def host_sync(self) -> str | None:
        """The first host synchronisation the callables make once warm (None if they make
        none). Found with torch's sync debug mode on the second call: the first, unprobed,
        leaves one-time work out (a torch.compile compilation synchronises), and it comes
        before any capture is attempted, since a capture that fails part-way leaves the
        process's graph state unusable."""
        self.fns[0]()
        torch.cuda.synchronize()
        before = torch.cuda.get_sync_debug_mode()
        torch.cuda.set_sync_debug_mode("error")
        try:
            self.fns[0]()
        except RuntimeError as e:
            return str(e).splitlines()[0][:120]
        finally:
            torch.cuda.set_sync_debug_mode(before)
            torch.cuda.synchronize()
        return None

    def capture(self) -> bool:
        """Record one pass into a HIP graph (warmed up on a side stream, as torch requires)."""
        sync = self.host_sync()
        if sync:
            self.why_eager = f"not graph-capturable: host sync ({sync})"
            return False
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self.run()
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.run()
            g.replay()
            torch.cuda.synchronize()
            self.graph = g
            return True
        except Exception as e:  # noqa: BLE001 - capture is best effort
            torch.cuda.synchronize()
            self.why_eager = f"graph capture failed: {str(e)[:200]}"
            return False

    def measure(self, warmup: int = 5, reps: int = 20, graph: bool = True) -> dict:
        torch.cuda.synchronize()
        for _ in range(warmup):
            self.run()
        torch.cuda.synchronize()
        host = _median(self._per_call(self.run, reps))
        res = {"host_ms": host, "copies": len(self.fns), "device_ms": host, "mode": "eager"}
        if graph and (self.graph is not None or self.capture()):
            samples = self._per_call(self.graph.replay, reps)
            med = _median(samples)
            res.update(device_ms=med, mode="graph", spread=(max(samples) - min(samples)) / max(med, 1e-9))
        elif graph and self.why_eager:
            res["note"] = self.why_eager
        return res


def time_calls(fns: list, warmup: int = 5, reps: int = 20, graph: bool = True) -> dict:
    """Median device ms per call of fns: graph replay when the callables can be captured,
    eager HIP events otherwise (with a note saying why)."""
    return Timer(fns).measure(warmup=warmup, reps=reps, graph=graph)


def time_ab(variants: dict, rounds: int = 5, reps: int = 10) -> dict:
    """Time variants (name -> list of callables) in interleaved rounds of alternating order.
    Every variant is captured up front; if any cannot be, all are timed eagerly."""
    timers = {name: Timer(fns) for name, fns in variants.items()}
    refused = [name for name, t in timers.items() if not t.capture()]
    use_graph = not refused
    note = None
    if refused:
        note = (f"all variants timed eagerly: {refused} could not be graph-captured "
                f"({(timers[refused[0]].why_eager or '')[:120]})")
    rounds_dev = {name: [] for name in timers}
    rounds_host = {name: [] for name in timers}
    first = {}
    names = list(timers)
    for k in range(rounds):
        for name in (names if k % 2 == 0 else names[::-1]):
            t = timers[name].measure(warmup=3 if k else 5, reps=reps, graph=use_graph)
            if note:
                t["note"] = note
            rounds_dev[name].append(t["device_ms"])
            rounds_host[name].append(t["host_ms"])
            first.setdefault(name, t)
    result = {}
    for name in names:
        dev, host = sorted(rounds_dev[name]), sorted(rounds_host[name])
        dm, hm = _median(dev), _median(host)
        result[name] = {**first[name], "device_ms": dm, "rounds": dev,
                        "noise": (dev[-1] - dev[0]) / max(dm, 1e-12), "host_ms": hm,
                        "host_rounds": host, "host_noise": (host[-1] - host[0]) / max(hm, 1e-12)}
    return result


def significance(base: dict, cand: dict) -> str:
    """'faster' or 'slower' only when the two variants' round ranges are disjoint."""
    lo_c, hi_c = min(cand["rounds"]), max(cand["rounds"])
    lo_b, hi_b = min(base["rounds"]), max(base["rounds"])
    if hi_c < lo_b:
        return "faster"
    if lo_c > hi_b:
        return "slower"
    return "within noise"


# -------------------------------------------------------------------- selftest
def _trial(fn, inputs, dtype=None, cot=None):
    """fn on fresh leaves (cast to dtype if given; floating inputs require grad), then the
    gradient of every floating leaf under the cotangent (drawn as randn * 1e-2 if None).
    Returns ([output, *grads] detached, cotangent)."""
    leaves = [x.detach().to(dtype or x.dtype).requires_grad_(x.is_floating_point()) for x in inputs]
    out = fn(*leaves)
    if cot is None:
        cot = torch.randn(out.shape, device=out.device, dtype=torch.float32) * 1e-2
    wrt = [x for x in leaves if x.requires_grad]
    grads = torch.autograd.grad(out, wrt, cot.to(out.dtype))
    return [out.detach(), *(g.detach() for g in grads)], cot


def selftest_autograd(fn, ref, inputs: list, slack: float = 2.0, time: bool = True) -> dict:
    """fn against ref (output and the gradient of every floating input) on one random
    cotangent: fp32 reference, eager original and candidate; then fn under
    torch.compile(fullgraph=True); then forward + backward timings of all of them."""
    with pure_fp32():
        ref32, cot = _trial(ref, inputs, torch.float32)
    orig, _ = _trial(ref, inputs, cot=cot)
    cand, _ = _trial(fn, inputs, cot=cot)
    checks = compare(ref32, orig, cand, slack=slack)

    leaves = [x.detach().requires_grad_(x.is_floating_point()) for x in inputs]
    wrt = [x for x in leaves if x.requires_grad]
    gout = cot.to(inputs[0].dtype)

    def fwd_bwd(f):
        return lambda: torch.autograd.grad(f(*leaves), wrt, gout)

    variants = {"reference": [fwd_bwd(ref)], "kernel": [fwd_bwd(fn)]}
    try:
        torch._dynamo.reset()
        fn_c, ref_c = torch.compile(fn, fullgraph=True), torch.compile(ref)
        cand_c, _ = _trial(fn_c, inputs, cot=cot)
        compiled = {"pass": compare(ref32, orig, cand_c, slack=slack)["pass"]}
        variants["compiled_reference"] = [fwd_bwd(ref_c)]
        variants["compiled_kernel"] = [fwd_bwd(fn_c)]
    except Exception as e:  # noqa: BLE001 - reported, not raised
        compiled = {"pass": False, "error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}
    result = {"pass": checks["pass"] and compiled.get("pass", False), "checks": checks, **versions()}
    if not time:
        return {**result, "compiled": compiled}

    t = time_ab(variants, rounds=3)
    us = {name: round(v["device_ms"] * 1e3, 1) for name, v in t.items()}

    def speed(base, cand):
        return {"speedup": round(us[base] / us[cand], 2), "significance": significance(t[base], t[cand])}

    if "compiled_kernel" in t:
        compiled.update(kernel_us=us["compiled_kernel"], reference_us=us["compiled_reference"],
                        **speed("compiled_reference", "compiled_kernel"))
    return {**result, "reference_us": us["reference"], "kernel_us": us["kernel"],
            **speed("reference", "kernel"), "compiled": compiled}
