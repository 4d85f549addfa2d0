"""RMSNorm, GEGLU, the fused projection and the T5 table step captured in HIP graphs: every
entry point of the library allocates, frees and synchronizes nothing, so a captured fwd+bwd
replays to the eager result. Replayed three times with unrelated eager work in between, each
replay checked."""
import pytest
import torch

import geglu as G
import relpos_attention as A
import rmsnorm as R
from krsi_testutil import log, seeded

pytestmark = pytest.mark.gpu


def _replay_matches(fn, inputs, cotangent, other):
    """fn(*inputs) fwd + autograd bwd eagerly, then captured; replays must equal eager bitwise.
    Nothing allocated before the capture is released inside it: the eager run keeps its own
    leaves and its results stay referenced, and the captured outputs get fresh names (the
    relpos graph test's pattern)."""

    def run(leaves):
        out = fn(*leaves)
        return (out.detach(), *torch.autograd.grad(out, leaves, cotangent))

    eager = run([t.detach().requires_grad_(True) for t in inputs])
    xs = [t.detach().requires_grad_(True) for t in inputs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(xs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = run(xs)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(captured, eager))
        other()  # unrelated eager work between replays
        torch.cuda.synchronize()


DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
def test_rmsnorm_graph_replay_matches_eager(dt):
    log(f"rmsnorm graph replay [2048, 4096] {dt}")
    x = seeded((2048, 4096), 0, dtype=dt)
    w = seeded((4096,), 1, std=0.02, mean=1.0, dtype=dt)
    gy = seeded((2048, 4096), 2, dtype=dt)
    other = seeded((512, 1024), 3)
    _replay_matches(lambda a, b: R.rmsnorm(a, b, 1e-6), [x, w], gy,
                    lambda: R.rmsnorm(other, torch.ones(1024, device="cuda", dtype=torch.bfloat16), 1e-6))


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_geglu_graph_replay_matches_eager(approximate, dt):
    log(f"geglu graph replay [1024, 2*2048] {approximate} {dt}")
    u, gy = seeded((1024, 4096), 4, dtype=dt), seeded((1024, 2048), 5, dtype=dt)
    other = seeded((64, 256), 6)
    _replay_matches(lambda a: G.geglu(a, approximate=approximate), [u], gy, lambda: G.geglu(other))


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
def test_t5_table_chain_graph_replay_matches_eager(dt):
    B, S, H, D = 1, 256, 4, 64
    log(f"t5 table + relpos graph replay B{B} S{S} H{H} D{D} {dt}")
    qkv = seeded((B * S, 3 * H * D), 7, dtype=dt)
    table = seeded((32, H), 8, std=0.5, dtype=torch.float32)
    dout = seeded((B * S, H * D), 9, dtype=dt)
    A.t5_relative_position_bucket(S, True, 32, 128, "cuda")  # build the cached map before capture
    _replay_matches(lambda q, t: A.relpos_attention(q, A.t5_relpos_table(t, S), B, S, H, D, 0.125),
                    [qkv, table], dout, lambda: A.t5_relpos_table(table, 64))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=lambda d: str(d).replace("torch.", ""))
def test_geglu_linear_graph_replay_matches_eager(dt):
    # The fused projection's forward kernel and its backward (vendor GEMMs around the GEGLU
    # backward kernel), captured and replayed.
    rows, K, F = 256, 512, 256
    log(f"geglu_linear graph replay x [{rows}, {K}] w [{2 * F}, {K}] {dt}")
    x = seeded((rows, K), 10, dtype=dt)
    w = (seeded((2 * F, K), 11, dtype=torch.float32) / K ** 0.5).to(dt)
    gy = seeded((rows, F), 12, dtype=dt)
    other = seeded((64, 256), 13)
    _replay_matches(lambda a, b: G.geglu_linear(a, b, approximate="tanh"), [x, w], gy, lambda: G.geglu(other))


def test_launches_go_to_torch_current_stream():
    # The binding reads torch's current stream per call (raw handle), so work queued on a side
    # stream runs there, ordered after that stream's earlier work.
    import _hip
    log("current-stream handle on the default and a side stream")
    x = seeded((64, 256), 0)
    w = torch.ones(256, device="cuda", dtype=torch.bfloat16)
    assert _hip._stream(x) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert _hip._stream(x) == side.cuda_stream
        y, _ = _hip.rmsnorm_fwd(x, w, 1e-6)
    torch.cuda.current_stream().wait_stream(side)
    ref, _ = _hip.rmsnorm_fwd(x, w, 1e-6)
    assert torch.equal(y, ref)
