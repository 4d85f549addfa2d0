"""fp16 and fp32 activations (the reference's kernels are dtype-generic): the HIP kernels vs
the fp32 reference, with the eager original in the same dtype as the noise yardstick.

Tolerance, stated: the reference's acceptance criterion with slack 2 (tools/common.py:
322-392, 476-490), as for bf16: every output's max error and rel-L2 within 2x those of the
eager original in the same dtype, per-row errors within 3x, with the criterion's absolute
floors (1e-3 of the peak per element, 1e-5 rel-L2), which is what an fp32 run is held to.
Attention in fp16 is additionally held to the reference Triton kernels' own rounding points
(P and dS rounded to fp16), per row at 3x. Attention in fp32 (fp32 MFMA, P and dS unrounded as
the reference keeps them for fp32 inputs) is held to the same criterion against a float64
reference of the same fp32 inputs, with the eager fp32 computation as the yardstick; in practice
that is the floors (1e-5 rel-L2, 1e-3 of the peak per element, per-row 3x the median row error
+ 1e-5), far tighter than the reference's own fp32 path, which runs its products in TF32.
"""
import math

import pytest
import torch

import _hip
import geglu as G
import krsi_oracle as O
import relpos_attention as A
import rmsnorm as R
from krsi_testutil import assert_parity, log, seeded

pytestmark = pytest.mark.gpu
EPS = 1e-6
DTYPES = [torch.float16, torch.float32]


def _name(dt):
    return str(dt).replace("torch.", "")


# ------------------------------------------------------------------- RMSNorm
def _rms(x, w, g, dt):
    ref32 = O.rmsnorm_train(x, w, EPS, g.float(), torch.float32)
    orig = O.rmsnorm_train(x, w, EPS, g, dt)
    xx = x.detach().requires_grad_(True)
    ww = w.detach().requires_grad_(True)
    y = R.rmsnorm(xx, ww, EPS)
    dx, dw = torch.autograd.grad(y, [xx, ww], g)
    assert y.dtype == dt and dx.dtype == dt and dw.dtype == dt
    return ref32, orig, (y.detach(), dx, dw)


@pytest.mark.parametrize("dt", DTYPES, ids=_name)
@pytest.mark.parametrize("rows,n", [(2048, 1152), (300, 4096), (5, 7), (33, 1001), (64, 256),
                                    (9, 8192), (5, 16384), (1000, 512)])
def test_rmsnorm_dtypes(dt, rows, n):
    log(f"rmsnorm {_name(dt)} rows={rows} n={n}")
    x = seeded((rows, n), 30 + n, dtype=dt)
    w = seeded((n,), 31, std=0.1, mean=1.0, dtype=dt)
    g = seeded((rows, n), 32, dtype=dt)
    ref32, orig, cand = _rms(x, w, g, dt)
    assert_parity(["y", "dx", "dw"], ref32, orig, cand, extra_msg=_name(dt))
    # The forward against the eager original of the same dtype: in fp16 bitwise except at
    # rounding ties of x*r (fp32 statistics summed in another order); in fp32, which has no
    # rounding point to absorb that order, within a few fp32 ulps.
    eager = O.rmsnorm(x, w, EPS)
    if dt == torch.float16:
        same = (cand[0] == eager).float().mean().item()
        assert same > 0.999, same
    else:
        assert torch.allclose(cand[0], eager, rtol=4e-7 * 8, atol=1e-7), (cand[0] - eager).abs().max()


@pytest.mark.parametrize("dt", DTYPES, ids=_name)
def test_rmsnorm_dtypes_unaligned_and_deterministic(dt):
    log(f"rmsnorm {_name(dt)} unaligned view + determinism")
    base = seeded((64 * 256 + 1,), 33, dtype=dt)
    x = base[1:].view(64, 256)
    w = seeded((256,), 34, std=0.1, mean=1.0, dtype=dt)
    g = seeded((64, 256), 35, dtype=dt)
    ref32, orig, cand = _rms(x, w, g, dt)
    assert_parity(["y", "dx", "dw"], ref32, orig, cand, extra_msg=_name(dt))
    x = seeded((2048, 4096), 36, dtype=dt)
    w = seeded((4096,), 37, std=0.02, mean=1.0, dtype=dt)
    g = seeded((2048, 4096), 38, dtype=dt)
    _, rstd = _hip.rmsnorm_fwd(x, w, EPS)
    a = _hip.rmsnorm_bwd(g, x, w, rstd)
    b = _hip.rmsnorm_bwd(g, x, w, rstd)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_rmsnorm_mixed_dtypes_rejected():
    x = seeded((4, 64), 1, dtype=torch.float16)
    with pytest.raises(TypeError):
        R.rmsnorm(x, torch.ones(64, device="cuda", dtype=torch.float32), EPS)
    with pytest.raises(TypeError):
        R.rmsnorm(x.double(), torch.ones(64, device="cuda", dtype=torch.float64), EPS)


# --------------------------------------------------------------------- GEGLU
@pytest.mark.parametrize("dt", DTYPES, ids=_name)
@pytest.mark.parametrize("approximate", ["none", "tanh"])
@pytest.mark.parametrize("rows,f", [(1, 8), (7, 1001), (64, 2816), (300, 64), (2, 4100), (512, 4096)])
def test_geglu_dtypes(dt, approximate, rows, f):
    log(f"geglu {_name(dt)} {approximate} rows={rows} f={f}")
    u = seeded((rows, 2 * f), 40 + f, std=2.0, dtype=dt)
    g = seeded((rows, f), 41, dtype=dt)
    ref32 = O.geglu_train(u, g.float(), approximate, torch.float32)
    orig = O.geglu_train(u, g, approximate, dt)
    uu = u.detach().requires_grad_(True)
    out = G.geglu(uu, approximate=approximate)
    (du,) = torch.autograd.grad(out, [uu], g)
    assert out.dtype == dt and du.dtype == dt
    assert_parity(["out", "du"], ref32, orig, (out.detach(), du), extra_msg=_name(dt))


# ------------------------------------------------ relative-position attention
def _relpos_fp16(B, S, H, D, scale, std=1.0, pd_std=0.02, ref_device="cpu", ld_extra=0, seed=50,
                 pd_fn=None, vs_eager=True):
    dt = torch.float16
    qkv = seeded((B * S, 3 * H * D + ld_extra), seed, std=std, dtype=dt)
    if ld_extra:
        qkv = qkv[:, :3 * H * D]
    pd = seeded((H, 2 * S - 1), seed + 1, std=pd_std, dtype=torch.float32)
    if pd_fn is not None:
        pd = pd_fn(pd)
    dout = seeded((B * S, H * D), seed + 2, dtype=dt)
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    out = A.relpos_attention(x, p, B, S, H, D, scale)
    dqkv, dpd = torch.autograd.grad(out, [x, p], dout)
    assert out.dtype == dt and dqkv.dtype == dt and dpd.dtype == torch.float32
    dev = torch.device(ref_device)
    a = (qkv.to(dev), pd.to(dev), B, S, H, D, scale, dout.to(dev))
    r = O.relpos_manual(*a)
    o = O.relpos_manual(*a, eager_dtype=dt)
    kem = O.relpos_kernel_emulated(*a, dtype=dt)
    cand = (out.detach().to(dev), dqkv.to(dev), dpd.to(dev))
    tag = f"fp16 B{B} S{S} H{H} D{D}"
    if vs_eager:
        assert_parity(["out", "dqkv", "dpd"], (r[0], r[2], r[3]), (o[0], o[2], o[3]), cand,
                      row_slack=float("inf"), extra_msg=tag + " vs eager fp16")
    assert_parity(["out", "dqkv", "dpd"], (r[0], r[2], r[3]), kem, cand,
                  extra_msg=tag + " vs reference-kernel rounding")
    _, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
    assert torch.allclose(lse.to(dev), r[1], atol=1e-3, rtol=1e-4)
    assert (out32.to(dev) - r[0]).norm() / r[0].norm() < 1e-3


FP16_CASES = [  # B, S, H, D, scale, qkv std, pd std
    (1, 2, 1, 64, 0.125, 1.0, 0.02),
    (1, 17, 2, 32, 0.2, 1.0, 1.0),
    (2, 64, 2, 64, 1.0, 0.6, 1.0),
    (1, 128, 2, 128, 1 / math.sqrt(128), 1.0, 0.02),
    (2, 300, 2, 72, 1 / math.sqrt(72), 1.0, 0.02),
    (1, 257, 1, 8, 0.35, 1.0, 0.3),
    (1, 96, 2, 64, -0.125, 1.0, 0.5),
    (1, 80, 2, 32, 0.0, 1.0, 1.0),
]


@pytest.mark.parametrize("B,S,H,D,scale,std,pd_std", FP16_CASES)
def test_relpos_fp16(B, S, H, D, scale, std, pd_std):
    log(f"relpos fp16 B{B} S{S} H{H} D{D} scale {scale:.4g}")
    _relpos_fp16(B, S, H, D, scale, std, pd_std)


def test_relpos_fp16_strided_and_large():
    log("relpos fp16 strided qkv B2 S96 H2 D64")
    _relpos_fp16(2, 96, 2, 64, 0.125, ld_extra=40)
    log("relpos fp16 B2 S1024 H16 D72")
    _relpos_fp16(2, 1024, 16, 72, 1 / math.sqrt(72), ref_device="cuda")
    # D 64 with 256 blocks of each backward kind: the one-launch dQ + dK/dV pairing.
    log("relpos fp16 B2 S1024 H16 D64")
    _relpos_fp16(2, 1024, 16, 64, 0.125, ref_device="cuda")


def _relpos_fp32(B, S, H, D, scale, std=1.0, pd_std=0.02, ref_device="cpu", ld_extra=0, seed=70,
                 pd_fn=None):
    dt = torch.float32
    qkv = seeded((B * S, 3 * H * D + ld_extra), seed, std=std, dtype=dt)
    if ld_extra:
        qkv = qkv[:, :3 * H * D]
    pd = seeded((H, 2 * S - 1), seed + 1, std=pd_std, dtype=torch.float32)
    if pd_fn is not None:
        pd = pd_fn(pd)
    dout = seeded((B * S, H * D), seed + 2, dtype=dt)
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    out = A.relpos_attention(x, p, B, S, H, D, scale)
    dqkv, dpd = torch.autograd.grad(out, [x, p], dout)
    assert out.dtype == dt and dqkv.dtype == dt and dpd.dtype == torch.float32
    dev = torch.device(ref_device)
    a = (qkv.to(dev), pd.to(dev), B, S, H, D, scale, dout.to(dev))
    r = O.relpos_manual(*a, compute_dtype=torch.float64)
    o = O.relpos_manual(*a)  # the eager fp32 computation (explicit fp32 matmuls + softmax)
    cand = (out.detach().to(dev), dqkv.to(dev), dpd.to(dev))
    tag = f"fp32 B{B} S{S} H{H} D{D}"
    assert_parity(["out", "dqkv", "dpd"], (r[0], r[2], r[3]), (o[0], o[2], o[3]), cand,
                  extra_msg=tag + " vs eager fp32")
    _, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
    assert torch.equal(out32, out.detach())
    assert torch.allclose(lse.to(dev).double(), r[1], atol=1e-5, rtol=1e-6), (lse.to(dev) - r[1]).abs().max()


FP32_CASES = [  # B, S, H, D, scale, qkv std, pd std
    (1, 2, 1, 64, 0.125, 1.0, 0.02),
    (1, 17, 2, 32, 0.2, 1.0, 1.0),
    (2, 64, 2, 64, 1.0, 0.6, 1.0),
    (1, 128, 2, 128, 1 / math.sqrt(128), 1.0, 0.02),
    (2, 300, 2, 72, 1 / math.sqrt(72), 1.0, 0.02),
    (1, 200, 1, 16, 0.25, 1.0, 0.5),
    (1, 130, 2, 48, 0.3, 1.0, 0.02),
    (1, 100, 1, 80, 0.1, 1.0, 0.02),
    (1, 96, 2, 96, 0.1, 1.0, 0.02),
    (1, 70, 1, 112, 0.1, 1.0, 0.02),
    (1, 257, 1, 8, 0.35, 1.0, 0.3),
    (1, 96, 2, 64, -0.125, 1.0, 0.5),
    (1, 80, 2, 32, 0.0, 1.0, 1.0),
]


@pytest.mark.parametrize("B,S,H,D,scale,std,pd_std", FP32_CASES)
def test_relpos_fp32(B, S, H, D, scale, std, pd_std):
    log(f"relpos fp32 B{B} S{S} H{H} D{D} scale {scale:.4g}")
    _relpos_fp32(B, S, H, D, scale, std, pd_std)


def _mask(kind, S):
    """-inf entries of the table: keys after the query (causal) or more than 16 away (band16)."""
    def fn(pd):
        r = torch.arange(2 * S - 1, device=pd.device) - (S - 1)
        keep = r <= 0 if kind == "causal" else r.abs() <= 16
        return pd.masked_fill(~keep, float("-inf"))
    return fn


@pytest.mark.parametrize("mask", ["causal", "band16"])
def test_relpos_fp16_fp32_masks_through_the_bias(mask):
    """Masked relative positions in fp32 (against float64, with the eager fp32 yardstick) and
    fp16 (against the reference kernel's rounding points, as the bf16 masked cases). band16
    masks whole leading key steps of the later queries."""
    log(f"relpos fp32 {mask} mask B2 S160 H2 D64")
    _relpos_fp32(2, 160, 2, 64, 0.125, pd_std=0.5, pd_fn=_mask(mask, 160))
    log(f"relpos fp16 {mask} mask B2 S160 H2 D64")
    _relpos_fp16(2, 160, 2, 64, 0.125, pd_std=0.5, pd_fn=_mask(mask, 160), vs_eager=False)


def test_relpos_fp32_single_position():
    """S = 1: out = v and dv = dout exactly (p = 1 in both passes); dq, dk and dpd are 0 up to
    the rounding of dp - delta, whose two dot products are summed in different orders."""
    B, S, H, D = 2, 1, 3, 64
    qkv = seeded((B * S, 3 * H * D), 80, dtype=torch.float32)
    pd = seeded((H, 1), 81, dtype=torch.float32)
    dout = seeded((B * S, H * D), 82, dtype=torch.float32)
    x = qkv.detach().requires_grad_(True)
    p = pd.detach().requires_grad_(True)
    out = A.relpos_attention(x, p, B, S, H, D, 0.125)
    dqkv, dpd = torch.autograd.grad(out, [x, p], dout)
    q, k, v = O.split_qkv(qkv, B, S, H, D)
    assert torch.equal(out.detach(), v.permute(0, 2, 1, 3).reshape(B * S, H * D))
    d = dqkv.view(B * S, 3, H * D)
    assert torch.equal(d[:, 2], dout)
    assert d[:, :2].abs().max().item() < 1e-5 and dpd.abs().max().item() < 1e-5


def test_relpos_fp32_strided_and_config4_shape():
    """A qkv row stride wider than 3*H*D, then the BASELINE config 4 shape (B2 H16 L1024 D72)
    forward and backward against the float64 reference on the GPU; the backward is bitwise
    reproducible."""
    log("relpos fp32 strided qkv B2 S96 H2 D64")
    _relpos_fp32(2, 96, 2, 64, 0.125, ld_extra=40)
    log("relpos fp32 B2 S1024 H16 D72 (config 4 shape)")
    _relpos_fp32(2, 1024, 16, 72, 1 / math.sqrt(72), ref_device="cuda")
    B, S, H, D = 2, 1024, 16, 72
    qkv = seeded((B * S, 3 * H * D), 90, dtype=torch.float32)
    pd = seeded((H, 2 * S - 1), 91, std=0.02, dtype=torch.float32)
    dout = seeded((B * S, H * D), 92, dtype=torch.float32)
    _, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, 0.1)
    a = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.1)
    b = _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, 0.1)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_relpos_fp16_config5_shape():
    """The BASELINE config 5 shape in fp16 (B4 H16 L4096 D64), against the fp32 reference on the
    GPU, with the same two criteria as the small cases."""
    log("relpos fp16 B4 S4096 H16 D64")
    _relpos_fp16(4, 4096, 16, 64, 1 / 8, ref_device="cuda")


@pytest.mark.parametrize("S", [8191, 16384])
def test_relpos_fp16_fp32_long_sequence(S):
    """Long context in fp16 and fp32 (B1 H2 D64), against the fp32 reference on the GPU: the odd
    S = 8191 takes the scalar dpd reduce, S = 16384 the 128-bit one, as in bf16."""
    log(f"relpos fp16 long context B1 S{S} H2 D64")
    _relpos_fp16(1, S, 2, 64, 0.125, ref_device="cuda")
    log(f"relpos fp32 long context B1 S{S} H2 D64")
    _relpos_fp32(1, S, 2, 64, 0.125, ref_device="cuda")
