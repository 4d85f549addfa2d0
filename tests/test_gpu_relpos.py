"""Relative-position flash attention HIP kernels vs the fp32 reference (parity tests proper).

The fp32 reference and the eager bf16 yardstick are oracle.relpos_manual: explicit fp32
matmuls on contiguous operands (SDPA-MATH upcasts bf16 to fp32, so this is the eager
original exactly up to fp32 summation order), run on the CPU for small cases and on the
GPU at the BASELINE sizes. No bf16 batched product is formed in any reference.
"""
import math

import pytest
import torch

import _hip
import krsi_oracle as O
import relpos_attention as A
from krsi_testutil import assert_parity, log, seeded

pytestmark = pytest.mark.gpu


def _inputs(B, S, H, D, std=1.0, pd_std=0.02, seed=0, ld_extra=0):
    qkv = seeded((B * S, 3 * H * D + ld_extra), seed, std=std)
    if ld_extra:
        qkv = qkv[:, :3 * H * D]
    pd = seeded((H, 2 * S - 1), seed + 1, std=pd_std, dtype=torch.float32)
    dout = seeded((B * S, H * D), seed + 2)
    return qkv, pd, dout


def _kernel(qkv, pd, dout, B, S, H, D, scale):
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    out = A.relpos_attention(x, p, B, S, H, D, scale)
    dqkv, dpd = torch.autograd.grad(out, [x, p], dout)
    return out.detach(), dqkv, dpd


def _check(B, S, H, D, scale, std=1.0, pd_std=0.02, ref_device="cpu", seed=0, ld_extra=0, pd_fn=None,
           vs_eager=True):
    """Tolerance, stated: with slack 2 (tools/common.py:476-490), every output's max error and
    rel-L2 are within 2x those of the eager bf16 original AND within 2x those of the reference
    Triton kernels' own rounding points (oracle.relpos_kernel_emulated: bf16 p before PV/dV,
    bf16 dS before dK/dQ), and no row (last dim >= 64) exceeds 3x the latter's error on that
    row. The per-row check is taken against the reference kernel's own error: the eager
    original upcasts to fp32 and rounds once, so at small S its per-row error is not a bound
    the reference kernel meets either."""
    qkv, pd, dout = _inputs(B, S, H, D, std, pd_std, seed, ld_extra)
    if pd_fn is not None:
        pd = pd_fn(pd)
    cand = _kernel(qkv, pd, dout, B, S, H, D, scale)
    dev = torch.device(ref_device)
    r = O.relpos_manual(qkv.to(dev), pd.to(dev), B, S, H, D, scale, dout.to(dev))
    o = O.relpos_manual(qkv.to(dev), pd.to(dev), B, S, H, D, scale, dout.to(dev), eager_bf16=True)
    kem = O.relpos_kernel_emulated(qkv.to(dev), pd.to(dev), B, S, H, D, scale, dout.to(dev))
    ref32, orig = (r[0], r[2], r[3]), (o[0], o[2], o[3])
    cand = tuple(t.to(dev) for t in cand)
    tag = f"B{B} S{S} H{H} D{D}"
    if vs_eager:
        assert_parity(["out", "dqkv", "dpd"], ref32, orig, cand, row_slack=float("inf"),
                      extra_msg=tag + " vs eager bf16")
    assert_parity(["out", "dqkv", "dpd"], ref32, kem, cand, extra_msg=tag + " vs reference-kernel rounding")
    # lse (log2 domain) and out32 of the forward, against fp32.
    out, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
    assert torch.allclose(lse.to(dev), r[1], atol=1e-3, rtol=1e-4), (lse.to(dev) - r[1]).abs().max()
    err32 = (out32.to(dev) - r[0]).norm() / r[0].norm()
    eager_out = (o[0].float() - r[0]).norm() / r[0].norm()
    assert err32 < 2 * eager_out + 1e-5, err32
    return qkv, pd, dout, cand


def test_relpos_single_position():
    """S = 1: softmax over one key is 1, so out = v, dv = dout, and dq, dk, dpd are exactly 0
    in exact arithmetic (a relative criterion is undefined there)."""
    B, S, H, D = 2, 1, 3, 64
    qkv, pd, dout = _inputs(B, S, H, D)
    out, dqkv, dpd = _kernel(qkv, pd, dout, B, S, H, D, 0.125)
    q, k, v = O.split_qkv(qkv, B, S, H, D)
    assert torch.equal(out, v.permute(0, 2, 1, 3).reshape(B * S, H * D))
    d = dqkv.view(B * S, 3, H * D)
    assert torch.equal(d[:, 2], dout)
    assert d[:, :2].abs().max().item() < 1e-5 and dpd.abs().max().item() < 1e-5


@pytest.mark.parametrize("mask", ["causal", "band16"])
@pytest.mark.parametrize("B,H,S,D,scale", [(2, 2, 200, 64, 0.125), (2, 2, 97, 72, -0.2), (2, 64, 520, 64, 0.125),
                                           (1, 192, 300, 128, 0.09)])
def test_relpos_masks_through_the_bias(mask, B, H, S, D, scale):
    """-inf entries of the relative-position table mask key offsets (causal: keys after the
    query; band16: more than 16 away). Masked scores give p = 0 and ds = 0, so the masked
    diagonals of dpd are exactly 0 and the rest match the oracle. Bound: the reference kernel's
    rounding points (bf16 p before dV, bf16 dS before dK and dQ). The eager-bf16 bound is left
    out here: under the causal mask the early queries' p reach 1, and the oracle's emulation of
    the reference kernel itself has 2.5x the eager max error on dV of key 0 (2.7e-2 against
    1.1e-2 at S = 200). The last two shapes have 512+ forward workgroups, so they run the 4-wave
    forward instead of the key-split one."""
    log(f"relpos {mask} mask through pd B{B} S{S} H{H} D{D} scale {scale}")

    def masked(pd):
        r = torch.arange(2 * S - 1, device=pd.device) - (S - 1)  # key - query
        keep = r <= 0 if mask == "causal" else r.abs() <= 16
        return pd.masked_fill(~keep, float("-inf"))

    big = B * H * S * S > 10 ** 7
    _, pd, _, cand = _check(B, S, H, D, scale, pd_std=0.5, pd_fn=masked, vs_eager=False,
                            ref_device="cuda" if big else "cpu")
    dpd = cand[2]
    off = ~torch.isfinite(masked(pd.new_zeros(pd.shape)))
    assert torch.isfinite(cand[0]).all() and torch.isfinite(cand[1]).all()
    assert torch.equal(dpd[off.to(dpd.device)], torch.zeros_like(dpd[off.to(dpd.device)]))


CASES = [  # B, S, H, D, scale, qkv std, pd std
    (1, 2, 1, 64, 0.125, 1.0, 0.02),
    (1, 17, 2, 32, 0.2, 1.0, 1.0),
    (2, 64, 2, 64, 1.0, 0.6, 1.0),        # the reference selftest's distribution (scale 1)
    (1, 128, 2, 128, 1 / math.sqrt(128), 1.0, 0.02),
    (2, 300, 2, 72, 1 / math.sqrt(72), 1.0, 0.02),  # ragged L300, D72
    (1, 200, 1, 16, 0.25, 1.0, 0.5),
    (1, 130, 2, 48, 0.3, 1.0, 0.02),
    (1, 100, 1, 80, 0.1, 1.0, 0.02),
    (1, 96, 2, 96, 0.1, 1.0, 0.02),
    (1, 70, 1, 112, 0.1, 1.0, 0.02),
    (1, 257, 1, 8, 0.35, 1.0, 0.3),
    (1, 96, 2, 64, -0.125, 1.0, 0.5),     # negative scale: sign folded into the bf16 operand
    (1, 80, 2, 32, 0.0, 1.0, 1.0),        # scale 0: scores are the bias alone
]


@pytest.mark.parametrize("B,S,H,D,scale,std,pd_std", CASES)
def test_relpos_small_vs_cpu_oracle(B, S, H, D, scale, std, pd_std):
    log(f"relpos small B{B} S{S} H{H} D{D} scale {scale:.4g}")
    _check(B, S, H, D, scale, std, pd_std, ref_device="cpu")


def test_relpos_strided_qkv():
    """qkv with a row stride wider than 3*H*D (a slice of a bigger projection)."""
    log("relpos strided qkv B2 S96 H2 D64")
    _check(2, 96, 2, 64, 0.125, ref_device="cpu", ld_extra=40)


def test_relpos_unaligned_qkv_takes_a_copy():
    """A qkv view the kernels cannot read in place (base 2 bytes past a 16-byte boundary, odd
    row stride) runs through one contiguous copy: outputs and gradients equal, bitwise, those of
    the same values in a contiguous tensor, and the gradient reaches the original view."""
    log("relpos unaligned qkv B2 S96 H2 D64")
    B, S, H, D = 2, 96, 2, 64
    big = seeded((B * S, 3 * H * D + 9), 0)
    view = big[:, 1:1 + 3 * H * D]
    assert view.data_ptr() % 16 == 2 and (view.stride(0) * 2) % 16 != 0
    _, pd, dout = _inputs(B, S, H, D)
    want = _kernel(view.contiguous(), pd, dout, B, S, H, D, 0.125)
    got = _kernel(view, pd, dout, B, S, H, D, 0.125)
    assert all(torch.equal(a, b) for a, b in zip(got, want))


def test_relpos_fwd_config4():
    """B2 H16 L1024 D72, scale 1/sqrt(72) (fwd; bwd checked too)."""
    log("relpos config4 B2 S1024 H16 D72")
    _check(2, 1024, 16, 72, 1 / math.sqrt(72), ref_device="cuda")


def test_relpos_fwd_config4_ragged():
    """BASELINE config 4's ragged case at its full width: B2 H16 L300 D72 (fwd; bwd checked too)."""
    log("relpos config4 ragged B2 S300 H16 D72")
    _check(2, 300, 16, 72, 1 / math.sqrt(72), ref_device="cuda")


def test_relpos_train_config5():
    """B4 H16 L4096 D64 fwd+bwd, dq/dk/dv and the bias-table gradient."""
    log("relpos config5 B4 S4096 H16 D64")
    qkv, pd, dout, cand = _check(4, 4096, 16, 64, 1 / 8, ref_device="cuda")
    # Rows of dS sum to zero, so the bias-table gradient sums to ~0 per head.
    dpd = cand[2]
    assert (dpd.sum(1).abs() <= 1e-3 * dpd.abs().sum(1) + 1e-4).all()


@pytest.mark.parametrize("S", [8191, 16384])
def test_relpos_long_sequence(S):
    """Long context, B1 H2 D64, against the fp32 reference on the GPU ([S, S] fp32 matrices of
    the reference, up to 1 GiB each). The odd S = 8191 takes the scalar dpd reduce (S % 4 != 0),
    S = 16384 the 128-bit one. The kernels' dpd partial rows take B*H*ceil(S/128)*(S+128)*4
    bytes of workspace, quadratic in S but 1/128 of the reference's [B, H, S, S] dbias."""
    log(f"relpos long context B1 S{S} H2 D64")
    qkv, pd, dout, cand = _check(1, S, 2, 64, 0.125, ref_device="cuda")
    dpd = cand[2]
    assert (dpd.sum(1).abs() <= 1e-3 * dpd.abs().sum(1) + 1e-4).all()


@pytest.mark.parametrize("B,S,H,D,dt", [(2, 1024, 16, 72, torch.bfloat16),   # key-split forward
                                        (4, 1024, 16, 64, torch.bfloat16),   # 4-wave forward
                                        (2, 300, 2, 32, torch.float16),      # unstaged store (D <= 32)
                                        (1, 200, 2, 64, torch.float32)])     # fp32 kernels
def test_relpos_forward_without_stats(B, S, H, D, dt):
    """The forward with out32 and lse left out (null, for a forward no backward follows) stores
    bitwise the same output, writes nothing else, and is what relpos_attention runs when no
    input requires grad or grad mode is off."""
    log(f"relpos forward without stats B{B} S{S} H{H} D{D} {dt}")
    qkv = seeded((B * S, 3 * H * D), 3, dtype=dt)
    pd = seeded((H, 2 * S - 1), 4, std=0.02, dtype=torch.float32)
    want, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125)
    got, o32, l2 = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125, stats=False)
    assert o32 is None and l2 is None and torch.equal(got, want)
    assert torch.equal(A.relpos_attention(qkv, pd, B, S, H, D, 0.125), want)
    with torch.no_grad():
        assert torch.equal(A.relpos_attention(qkv.requires_grad_(True), pd, B, S, H, D, 0.125), want)


@pytest.mark.parametrize("B,S,H", [(2, 1024, 16), (1, 1024, 17), (1, 640, 27), (1, 300, 16)])
def test_relpos_backward_grid_paths(B, S, H):
    """D = 64 backward grids around the one-launch pairing of dQ and dK/dV blocks: 256 blocks
    of each kind (the XCD-half pairing, 32 per XCD half), 136 (17 per XCD half), 135 (an odd
    count per XCD, so the two kernels run in separate launches) and 48 (one workgroup per CU)."""
    log(f"relpos backward grid paths B{B} S{S} H{H} D64")
    _check(B, S, H, 64, 0.125, ref_device="cuda")


@pytest.mark.parametrize("B,S,H,D,dt,chunks", [
    (1, 1101, 3, 64, torch.bfloat16, (1, 4)),   # 9 key blocks; S % 4 != 0: the scalar dpd sum
    (2, 520, 2, 80, torch.float16, (2,)),       # 5 key blocks, D 80; the 128-bit dpd sum
    (1, 700, 2, 64, torch.float32, (1, 4)),     # fp32 kernels
    (1, 512, 4, 64, torch.bfloat16, (3,)),      # a grid that pairs dQ and dK/dV when unchunked
    (1, 777, 2, 128, torch.bfloat16, (2,)),     # D 128 (one wave per SIMD); chunks 2, 2, 2, 1
])
def test_relpos_backward_bounded_workspace(B, S, H, D, dt, chunks):
    """A workspace that holds the dpd partial rows of only `c` of the ceil(S/128) key blocks
    (down to krsi_relpos_bwd_workspace_min_bytes, c = 1): the key blocks go in chunks of c,
    one dK/dV launch and one dpd sum each. dqkv is bitwise the full-workspace result (each
    block's dK/dV does not depend on the chunking); dpd is the same terms summed in another
    order, equal to fp32 rounding (rel 1e-5 of its largest entry)."""
    qkv = seeded((B * S, 3 * H * D), 5, dtype=dt)
    pd = seeded((H, 2 * S - 1), 6, std=0.02, dtype=torch.float32)
    dout = seeded((B * S, H * D), 7, dtype=dt)
    out, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125)
    full = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125)
    lo = _hip.lib().krsi_relpos_bwd_workspace_min_bytes(B, S, H, D)
    rows = B * H * (S + 128) * 4
    for c in chunks:
        log(f"relpos bounded workspace B{B} S{S} H{H} D{D} {dt}: {c} key blocks per launch")
        dqkv, dpd = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125,
                                    workspace_max=lo + (c - 1) * rows)
        assert torch.equal(dqkv, full[0]), f"{c} blocks per launch"
        torch.testing.assert_close(dpd, full[1], rtol=0, atol=1e-5 * full[1].abs().max().item())
    # The cap is raised to the minimum, so a cap of 1 byte runs one block per launch.
    dqkv, dpd = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125, workspace_max=1)
    assert torch.equal(dqkv, full[0])


def test_relpos_bounded_workspace_parity(monkeypatch):
    """relpos_attention's backward under the module-wide workspace cap (one key block per
    dK/dV launch) against the fp32 reference, to the parity bar of the unbounded path."""
    monkeypatch.setattr(_hip, "RELPOS_BWD_WORKSPACE_MAX", 1)
    log("relpos bounded workspace parity B2 S700 H2 D64")
    _check(2, 700, 2, 64, 0.125)


def test_relpos_backward_deterministic():
    log("relpos determinism B2 S512 H4 D64")
    B, S, H, D = 2, 512, 4, 64
    qkv, pd, dout = _inputs(B, S, H, D)
    out, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125)
    a = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125)
    b = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    out2, out32_2, lse2 = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125)
    assert torch.equal(out, out2) and torch.equal(out32, out32_2) and torch.equal(lse, lse2)


def test_relpos_deterministic_at_config5_under_interleaved_work():
    # forward and backward repeated with unrelated GPU work of varying
    # size in between, which shifts which workgroups run where and when; every output,
    # dpd's fixed-order diagonal sums included, must come out bitwise the same.
    B, S, H, D = 4, 4096, 16, 64
    log(f"relpos determinism B{B} S{S} H{H} D{D}, 8 runs with interleaved work")
    qkv, pd, dout = _inputs(B, S, H, D)
    first = None
    for i in range(8):
        torch.randn(1 << (16 + i), device="cuda").mul_(2).sum()
        out, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.125)
        dqkv, dpd = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.125)
        got = (out, out32, lse, dqkv, dpd)
        if first is None:
            first = [t.clone() for t in got]
        else:
            assert all(torch.equal(a, b) for a, b in zip(first, got)), f"run {i}"


def test_relpos_graph_replay_matches_eager():
    """fwd+bwd captured in a HIP graph and replayed with eager work in between: every replay
    equals the eager result (the kernels use no memset and keep no state between calls)."""
    log("relpos graph replay B1 S256 H2 D64")
    B, S, H, D = 1, 256, 2, 64
    qkv, pd, dout = _inputs(B, S, H, D)
    eager = _kernel(qkv, pd, dout, B, S, H, D, 0.125)
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            torch.autograd.grad(A.relpos_attention(x, p, B, S, H, D, 0.125), [x, p], dout)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = A.relpos_attention(x, p, B, S, H, D, 0.125)
        dq, dp = torch.autograd.grad(out, [x, p], dout)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]) and torch.equal(dq, eager[1]) and torch.equal(dp, eager[2])
        _kernel(qkv, pd, dout, B, S, H, D, 0.5)   # unrelated eager work between replays
        torch.cuda.synchronize()


def test_relpos_graph_replay_bounded_workspace(monkeypatch):
    """The chunked backward (one dK/dV launch and one accumulating dpd sum per key block)
    captured in a HIP graph: every replay equals the eager result, with eager work between."""
    monkeypatch.setattr(_hip, "RELPOS_BWD_WORKSPACE_MAX", 1)
    log("relpos graph replay, bounded workspace, B1 S600 H2 D64")
    B, S, H, D = 1, 600, 2, 64
    qkv, pd, dout = _inputs(B, S, H, D)
    eager = _kernel(qkv, pd, dout, B, S, H, D, 0.125)
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            torch.autograd.grad(A.relpos_attention(x, p, B, S, H, D, 0.125), [x, p], dout)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = A.relpos_attention(x, p, B, S, H, D, 0.125)
        dq, dp = torch.autograd.grad(out, [x, p], dout)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]) and torch.equal(dq, eager[1]) and torch.equal(dp, eager[2])
        _kernel(qkv, pd, dout, B, S, H, D, 0.5)   # unrelated eager work between replays
        torch.cuda.synchronize()


def test_relpos_rejects_bad_input():
    qkv, pd, _ = _inputs(1, 8, 1, 64)
    with pytest.raises(ValueError):
        A.relpos_attention(qkv, pd[:, :-1], 1, 8, 1, 64, 0.125)   # wrong table size
    with pytest.raises(ValueError):
        A.relpos_attention(qkv.cpu(), pd.cpu(), 1, 8, 1, 64, 0.125)  # CPU tensors
    q2 = seeded((8, 3 * 12), 0)
    with pytest.raises(ValueError):
        A.relpos_attention(q2, seeded((1, 15), 1, dtype=torch.float32), 1, 8, 1, 12, 0.125)  # D % 8


@pytest.mark.parametrize("B,S,H,D", [(4, 2048, 8, 128), (4, 1024, 16, 72), (4, 4096, 4, 32), (2, 300, 128, 64),
                                     (1, 333, 256, 72)])
def test_relpos_large_grid_head_dims(B, S, H, D):
    """Grids of 512+ forward workgroups take the 4-wave forward (smaller grids split keys over
    two wave groups, which the small cases above exercise): head dims other than 64 there, and
    ragged S, whose last query block has waves wholly past S and one partly past it (the
    staged output store skips those rows)."""
    assert (S + 127) // 128 * B * H >= 512
    log(f"relpos large grid B{B} S{S} H{H} D{D}")
    _check(B, S, H, D, 1 / math.sqrt(D), ref_device="cuda")
