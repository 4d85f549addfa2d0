"""bench.py's command-line contract on the CPU: more than one GPU is refused with a message
and exit status 2 before anything touches a device (this build measures one GPU)."""
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(args, env_extra=None):
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, env=env, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    p = _run(["--gpus", "2", "--steps", "1", "--warmup", "0"])
    assert p.returncode == 2, p.stderr
    assert "one GPU" in p.stderr and p.stdout == ""


def test_world_size_above_one_is_refused():
    p = _run(["--steps", "1"], {"WORLD_SIZE": "4", "RANK": "0", "LOCAL_RANK": "0"})
    assert p.returncode == 2, p.stderr
    assert "one GPU" in p.stderr
