"""krsi_rmsnorm_bwd_noalloc, the backward that uses the library's static scratch instead of a
caller workspace, called through the C ABI. Its dx and dw must equal, bitwise, those of
krsi_rmsnorm_bwd with a workspace. The check runs on two calls in a row, the second with a
smaller input (the scratch keeps the first call's partial rows), in each activation dtype,
and once more after an unrelated workspace call in between."""
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

import _hip
from krsi_testutil import log, seeded

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _inputs(rows, n, dt, seed):
    x = seeded((rows, n), seed, dtype=dt)
    w = seeded((n,), seed + 1, std=0.02, mean=1.0, dtype=dt)
    g = seeded((rows, n), seed + 2, dtype=dt)
    _, rstd = _hip.rmsnorm_fwd(x, w, 1e-6)
    return g, x, w, rstd


def _with_workspace(g, x, w, rstd):
    lib = _hip.lib()
    rows, n = x.shape
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    ws = torch.empty(lib.krsi_rmsnorm_bwd_workspace_bytes(rows, n), dtype=torch.uint8, device=x.device)
    rc = lib.krsi_rmsnorm_bwd(g.data_ptr(), x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                              dw.data_ptr(), ws.data_ptr(), ws.numel(), rows, n, _hip.DTYPE_CODES[x.dtype],
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.krsi_error_string(rc)
    return dx, dw


def _noalloc(g, x, w, rstd):
    lib = _hip.lib()
    rows, n = x.shape
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    rc = lib.krsi_rmsnorm_bwd_noalloc(g.data_ptr(), x.data_ptr(), w.data_ptr(), rstd.data_ptr(),
                                      dx.data_ptr(), dw.data_ptr(), rows, n, _hip.DTYPE_CODES[x.dtype],
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.krsi_error_string(rc)
    return dx, dw


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_noalloc_matches_workspace_entry_point(dt):
    # (4096 x 4096): 512 partial rows, 8 MiB of the scratch; then (300 x 1152): 75 rows.
    for rows, n, seed in ((4096, 4096, 10), (300, 1152, 20)):
        log(f"noalloc rmsnorm bwd {dt} [{rows}, {n}]")
        args = _inputs(rows, n, dt, seed)
        want = _with_workspace(*args)
        got = _noalloc(*args)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]), f"dx differs at [{rows}, {n}]"
        assert torch.equal(got[1], want[1]), f"dw differs at [{rows}, {n}]"


def test_noalloc_largest_accepted_and_repeat():
    """The largest problem the 16 MiB scratch holds at n = 16384 (256 rows), then a smaller
    one, then the first again: every result equals the workspace entry point's."""
    cases = ((256, 16384, 30), (64, 512, 40), (256, 16384, 30))
    for rows, n, seed in cases:
        log(f"noalloc rmsnorm bwd bf16 [{rows}, {n}]")
        args = _inputs(rows, n, torch.bfloat16, seed)
        want = _with_workspace(*args)
        got = _noalloc(*args)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), (rows, n)


# Run in a fresh process, so that the call inside the capture is the first noalloc call on the
# device (the one that looks up the device's copy of the scratch array).
_CAPTURE_SCRIPT = textwrap.dedent("""
    import sys
    for p in sys.argv[1:]:
        sys.path.insert(0, p)
    import torch
    import _hip
    from krsi_testutil import seeded
    lib = _hip.lib()
    rows, n = 2048, 4096
    x = seeded((rows, n), 50)
    w = seeded((n,), 51, std=0.02, mean=1.0)
    g = seeded((rows, n), 52)
    _, rstd = _hip.rmsnorm_fwd(x, w, 1e-6)
    want_dx, want_dw = _hip.rmsnorm_bwd(g, x, w, rstd)
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.krsi_rmsnorm_bwd_noalloc(g.data_ptr(), x.data_ptr(), w.data_ptr(), rstd.data_ptr(),
                                          dx.data_ptr(), dw.data_ptr(), rows, n, 0,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.krsi_error_string(rc)
    for i in range(2):
        dx.zero_()
        dw.zero_()
        # unrelated work between the replays, a workspace backward of other sizes among it
        o = seeded((300, 1152), 60 + i)
        _hip.rmsnorm_bwd(o, o, seeded((1152,), 70, std=0.02, mean=1.0), _hip.rmsnorm_fwd(o, o[0], 1e-6)[1])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, want_dx) and torch.equal(dw, want_dw), f"replay {i}"
    print("noalloc capture ok")
""")


def test_noalloc_first_call_inside_graph_capture():
    """The first noalloc call of a fresh process, made inside torch.cuda.graph capture, then
    two replays with other work in between: dx and dw equal the workspace entry point's."""
    log("noalloc rmsnorm bwd: first call inside a graph capture (child process)")
    here = Path(__file__).resolve().parent
    root = here.parent
    paths = [str(here), str(root / "kernel-rsi_amd" / "library"), str(root / "oracle")]
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, *paths], capture_output=True, text=True,
                       timeout=300, env=dict(os.environ))
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout, r.stdout + r.stderr
