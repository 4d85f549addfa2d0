"""bench.py's output contract on the GPU: one JSON line with the keys the driver reads, the
roofline object and the measured ceilings. Short runs with no CPU baseline: BASELINE config 4's
forward, a subset with no headline component, and the long-context attention line."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

from krsi_testutil import log

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]


def test_bench_prints_one_contract_line():
    log("bench: --only relpos_fwd --no-cpu --steps 2 --warmup 1")
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--only", "relpos_fwd", "--no-cpu",
                        "--steps", "2", "--warmup", "1"], capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, p.stdout[-2000:]
    line = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 2 and line["warmup"] == 1
    assert line["value"] > 0 and line["ms_per_step"] > 0 and line["unit"] == "TFLOP/s"
    assert line["cpu_baseline"] is None  # --no-cpu
    roof = line["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in roof, key
    assert roof["bound"] == "mfma" and roof["peak"] == 2500.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    comp = line["components"]["relpos_attention_fwd_config4"]
    assert comp["gemm_ceiling"]["TFLOP/s"] > 0
    assert line["measured_peaks"]["gemm_bf16_TFLOP/s"] > 0


def test_bench_subset_without_a_headline_component():
    """--only config1 (and likewise selftest_shapes) has no single figure to head the line: the
    line still prints, with value null and the component in place."""
    log("bench: --only config1 --no-cpu --steps 2 --warmup 1")
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--only", "config1", "--no-cpu",
                        "--steps", "2", "--warmup", "1"], capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, p.stdout[-2000:]
    line = json.loads(lines[0])
    assert line["value"] is None and line["roofline"] is None
    shapes = line["components"]["rmsnorm_config1"]["shapes"]
    assert all(s["gpu_fwd_us"] > 0 for s in shapes.values())


def test_bench_long_context_leg():
    """--only relpos_long: the long-context attention line, whose backward workspace (dpd partial
    rows) is a small fraction of the reference's [B, H, S, S] fp32 dbias."""
    log("bench: --only relpos_long --no-cpu --steps 2 --warmup 1")
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--only", "relpos_long", "--no-cpu",
                        "--steps", "2", "--warmup", "1"], capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, p.stdout[-2000:]
    comp = json.loads(lines[0])["components"]["relpos_attention_long"]
    assert comp["value"] > 0 and comp["unit"] == "TFLOP/s"
    assert 0 < comp["bwd_workspace_bytes"] < comp["reference_dbias_bytes"] / 100
