"""krsi_rmsnorm_bwd_noalloc, the backward that uses the library's static scratch instead of a
caller workspace, called through the C ABI. Its dx and dw must equal, bitwise, those of
krsi_rmsnorm_bwd with a workspace. The check runs on two calls in a row, the second with a
smaller input (the scratch keeps the first call's partial rows), in each activation dtype,
and once more after an unrelated workspace call in between."""
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
