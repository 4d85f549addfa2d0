"""Pin the CPU oracle: golden fixtures, independent float64 closed forms, autograd and
gradcheck, special cases the mathematics fixes, and an integer emulation of bf16 rounding.
A plausible mistake in the oracle (a dropped term, a wrong sign or index, a missing rounding
point) fails at least one of these."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import krsi_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLD / name, allow_pickle=False))


def t64(a):
    return torch.tensor(np.asarray(a), dtype=torch.float64)


# --------------------------------------------------------------- golden vectors
def test_golden_rmsnorm_closed_form_and_torch():
    g = load("rmsnorm.npz")
    y, rstd, dx, dw = O.rmsnorm_np64(g["x"], g["w"], float(g["eps"]), g["g"])
    for a, b in ((y, g["y"]), (rstd, g["rstd"]), (dx, g["dx"]), (dw, g["dw"])):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    # The torch restatement (autograd) agrees with the closed form; the reference's formula
    # computes the normalisation in fp32 (x2d.float(), rmsnorm.py:114-115) even for fp64 input.
    ty, tdx, tdw = O.rmsnorm_train(t64(g["x"]), t64(g["w"]), float(g["eps"]), t64(g["g"]), torch.float64)
    np.testing.assert_allclose(ty.numpy(), g["y"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(tdx.numpy(), g["dx"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(tdw.numpy(), g["dw"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("approx,key", [("tanh", "tanh"), ("none", "erf")])
def test_golden_geglu_closed_form_and_torch(approx, key):
    g = load("geglu.npz")
    out, du = O.geglu_np64(g["u"], g["g"], approx)
    np.testing.assert_allclose(out, g[f"out_{key}"], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(du, g[f"du_{key}"], rtol=1e-12, atol=1e-14)
    tout, tdu = O.geglu_train(t64(g["u"]), t64(g["g"]), approx, torch.float64)
    np.testing.assert_allclose(tout.numpy(), g[f"out_{key}"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(tdu.numpy(), g[f"du_{key}"], rtol=1e-9, atol=1e-12)


def test_golden_relpos_closed_form_and_torch():
    g = load("relpos.npz")
    B, S, H, D = (int(v) for v in g["dims"])
    scale = float(g["scale"])
    out, lse, dqkv, dpd = O.relpos_np64(g["qkv"], g["pd"], B, S, H, D, scale, g["dout"])
    for a, k in ((out, "out"), (lse, "lse"), (dqkv, "dqkv"), (dpd, "dpd")):
        np.testing.assert_allclose(a, g[k], rtol=1e-11, atol=1e-12)
    # Explicit-math restatement and the reference's SDPA-MATH formulation, float64 autograd.
    for sdpa in (False, True):
        tout, tdq, tdp = O.relpos_train(t64(g["qkv"]), t64(g["pd"]), B, S, H, D, scale, t64(g["dout"]),
                                        torch.float64, sdpa=sdpa)
        np.testing.assert_allclose(tout.numpy(), g["out"], rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(tdq.numpy(), g["dqkv"], rtol=1e-8, atol=1e-10)
        np.testing.assert_allclose(tdp.numpy(), g["dpd"], rtol=1e-8, atol=1e-10)
    lse_t = O.relpos_lse(t64(g["qkv"]), t64(g["pd"]), B, S, H, D, scale)
    np.testing.assert_allclose(lse_t.numpy(), g["lse"], rtol=1e-6, atol=1e-6)


def test_relpos_manual_fp32_matches_closed_form():
    g = load("relpos.npz")
    B, S, H, D = (int(v) for v in g["dims"])
    m = O.relpos_manual(t64(g["qkv"]).float(), t64(g["pd"]).float(), B, S, H, D, float(g["scale"]),
                        t64(g["dout"]).float())
    for a, k in ((m[0], "out"), (m[1], "lse"), (m[2], "dqkv"), (m[3], "dpd")):
        np.testing.assert_allclose(a.double().numpy(), g[k], rtol=1e-4, atol=2e-5)


# ---------------------------------------------------------------- gradcheck
def test_relpos_manual_float64_matches_closed_form():
    """The float64 mode of relpos_manual (the reference of fp32 attention inputs) against the
    golden float64 closed form, to float64 precision."""
    g = load("relpos.npz")
    B, S, H, D = (int(v) for v in g["dims"])
    m = O.relpos_manual(t64(g["qkv"]), t64(g["pd"]), B, S, H, D, float(g["scale"]), t64(g["dout"]),
                        compute_dtype=torch.float64)
    assert all(t.dtype == torch.float64 for t in m)
    for a, k in ((m[0], "out"), (m[1], "lse"), (m[2], "dqkv"), (m[3], "dpd")):
        np.testing.assert_allclose(a.numpy(), g[k], rtol=1e-10, atol=1e-12)
    # A planted mistake must fail: a transposed bias (pd indexed by i - j).
    flipped = O.relpos_manual(t64(g["qkv"]), t64(g["pd"]).flip(1), B, S, H, D, float(g["scale"]),
                              t64(g["dout"]), compute_dtype=torch.float64)
    assert not np.allclose(flipped[0].numpy(), g["out"], rtol=1e-6, atol=1e-8)


def test_gradcheck_fp64():
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(3, 10, generator=gen, dtype=torch.float64, requires_grad=True)
    w = (1 + 0.1 * torch.randn(10, generator=gen, dtype=torch.float64)).requires_grad_(True)
    # The reference formula normalises in fp32 (x.float()); its math, in float64:
    assert torch.autograd.gradcheck(lambda a, b: b * a * torch.rsqrt(a.pow(2).mean(-1, keepdim=True) + 1e-6),
                                    (x, w))
    u = torch.randn(2, 12, generator=gen, dtype=torch.float64, requires_grad=True)
    for approx in ("tanh", "none"):
        assert torch.autograd.gradcheck(lambda a: O.geglu(a, approx), (u,))
    B, S, H, D = 1, 5, 2, 4
    qkv = torch.randn(B * S, 3 * H * D, generator=gen, dtype=torch.float64, requires_grad=True)
    pd = torch.randn(H, 2 * S - 1, generator=gen, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: O.relpos(a, b, B, S, H, D, 0.7), (qkv, pd))


# -------------------------------------------------- special cases and invariants
def test_rmsnorm_special_cases():
    x = torch.tensor([[3.0] * 8, [-0.5] * 8], dtype=torch.float64)
    w = torch.arange(1, 9, dtype=torch.float64)
    y = O.rmsnorm(x, w, 0.0)
    assert torch.allclose(y, torch.sign(x) * w, atol=1e-15)          # constant row -> w * sign(x)
    xr = torch.randn(16, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    yr = O.rmsnorm(xr, torch.ones(64, dtype=torch.float64), 0.0)
    assert torch.allclose(yr.pow(2).mean(-1), torch.ones(16, dtype=torch.float64))  # unit RMS rows
    # dx is orthogonal to x per row when w = 1 (rescaling x leaves y unchanged).
    g = torch.randn(16, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    _, _, dx, _ = O.rmsnorm_np64(xr.numpy(), np.ones(64), 0.0, g.numpy())
    assert np.abs((dx * xr.numpy()).sum(-1)).max() < 1e-12


def test_geglu_special_cases():
    a = torch.tensor([-30.0, -1.0, 0.0, 1.0, 30.0], dtype=torch.float64)
    u = torch.cat([a, torch.ones_like(a)])[None]
    for approx in ("tanh", "none"):
        out = O.geglu(u, approx)[0]
        assert out[2] == 0 and abs(out[4] - 30) < 1e-12 and abs(out[0]) < 1e-12
    # The tanh form approximates the erf form to better than 1e-3 everywhere.
    z = torch.linspace(-8, 8, 4001, dtype=torch.float64)
    uu = torch.cat([z, torch.ones_like(z)])[None]
    assert (O.geglu(uu, "tanh") - O.geglu(uu, "none")).abs().max() < 1e-3
    # Derivative of the closed form against a central difference.
    uz = np.concatenate([np.linspace(-4, 4, 9), np.ones(9)])[None]
    _, du = O.geglu_np64(uz, np.ones((1, 9)), "tanh")
    h = 1e-6
    up, um = uz.copy(), uz.copy()
    up[0, :9] += h
    um[0, :9] -= h
    fd = (O.geglu_np64(up, np.ones((1, 9)))[0] - O.geglu_np64(um, np.ones((1, 9)))[0]) / (2 * h)
    np.testing.assert_allclose(du[0, :9], fd[0], rtol=1e-6, atol=1e-8)


def test_relpos_special_cases():
    gen = torch.Generator().manual_seed(3)
    B, S, H, D = 2, 9, 2, 8
    qkv = torch.randn(B * S, 3 * H * D, generator=gen, dtype=torch.float64)
    pd = torch.randn(H, 2 * S - 1, generator=gen, dtype=torch.float64)
    dout = torch.randn(B * S, H * D, generator=gen, dtype=torch.float64)
    q, k, v = O.split_qkv(qkv, B, S, H, D)
    # pd = 0: plain softmax attention.
    o0 = O.relpos(qkv, torch.zeros_like(pd), B, S, H, D, 0.5)
    plain = torch.softmax(q @ k.transpose(-2, -1) * 0.5, -1) @ v
    assert torch.allclose(o0, plain.transpose(1, 2).reshape(B * S, H * D), atol=1e-12)
    # A constant shift of the table does not change the output (softmax shift invariance).
    assert torch.allclose(O.relpos(qkv, pd + 3.0, B, S, H, D, 0.5), O.relpos(qkv, pd, B, S, H, D, 0.5), atol=1e-12)
    # Rows of dS sum to zero, so dpd sums to zero per head.
    _, _, dqkv, dpd = O.relpos_np64(qkv.numpy(), pd.numpy(), B, S, H, D, 0.5, dout.numpy())
    assert np.abs(dpd.sum(1)).max() < 1e-12
    # S = 1: out = v, dv = dout, dq = dk = dpd = 0.
    q1 = qkv[:B].clone()
    out, lse, dq1, dpd1 = O.relpos_np64(q1.numpy(), pd[:, 8:9].numpy(), B, 1, H, D, 0.5, dout[:B].numpy())
    np.testing.assert_allclose(out, q1.numpy().reshape(B, 3, H * D)[:, 2], atol=1e-15)
    assert np.abs(dq1.reshape(B, 3, H * D)[:, :2]).max() < 1e-13 and np.abs(dpd1).max() < 1e-13
    # lse lies between the max logit and max + log2(S) (log2 domain).
    lse = O.relpos_lse(qkv, pd, B, S, H, D, 0.5)
    s = (q @ k.transpose(-2, -1) * 0.5 + O.bias_matrix(pd, S)[None]) * O.LOG2E
    mx = s.amax(-1).reshape(B * H, S)
    assert (lse >= mx - 1e-12).all() and (lse <= mx + math.log2(S) + 1e-12).all()
    # torch diagonal sum equals the explicit double loop.
    ds = torch.randn(3, H, S, S, generator=gen, dtype=torch.float64)
    ref = np.zeros((H, 2 * S - 1))
    for hh in range(H):
        for i in range(S):
            for j in range(S):
                ref[hh, j - i + S - 1] += ds[:, hh, i, j].sum().item()
    np.testing.assert_allclose(O.diag_sum(ds, S).numpy(), ref, atol=1e-12)


# ---------------------------------------------------------- bf16 rounding points
def test_bf16_round_matches_torch_including_ties():
    gen = torch.Generator().manual_seed(4)
    a = (torch.randn(100000, generator=gen) * 10).numpy()
    base = np.float32([1.0, 1.0078125, -3.0, 0.3])
    ties = (base.view(np.uint32) + np.uint32(0x8000)).view(np.float32)   # exactly half-way
    a = np.concatenate([a, ties, np.float32([0.0, -0.0, 1e-40, 3.4e38])])
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(a), ref)


def test_rmsnorm_rounding_points_pinned():
    """The oracle's bf16 run must round x*r to bf16 before * w (rmsnorm.py:31, :115); an
    independent numpy emulation agrees bitwise except at rare fp32-order ties, and a variant
    without the intermediate rounding disagrees often."""
    x = O.randn((256, 1152), 5)
    w = O.randn((1152,), 6, std=0.02, mean=1.0)
    y = O.rmsnorm(x, w, 1e-6).float().numpy()
    emu = O.rmsnorm_eager_bf16_np(x.float().numpy(), w.float().numpy(), 1e-6)
    assert (emu == y).mean() > 0.999
    xf = x.float().numpy()
    r = 1.0 / np.sqrt((xf * xf).mean(-1, keepdims=True, dtype=np.float32) + np.float32(1e-6))
    planted = O.bf16_round(w.float().numpy() * (xf * r))                 # no rounding of x*r
    assert (planted == y).mean() < 0.9


def test_eager_emulation_matches_sdpa_bf16():
    """oracle.relpos_manual(eager_bf16=True) reproduces the reference's eager bf16 run
    (SDPA-MATH upcasts bf16 to fp32): out bitwise, dqkv up to fp32 summation order."""
    B, S, H, D = 2, 33, 2, 16
    qkv = O.randn((B * S, 3 * H * D), 8, std=0.6)
    pd = O.randn((H, 2 * S - 1), 9, dtype=torch.float32)
    dout = O.randn((B * S, H * D), 10)
    ob, dqb, dpb = O.relpos_train(qkv, pd, B, S, H, D, 1.0, dout, torch.bfloat16, sdpa=True)
    e = O.relpos_manual(qkv, pd, B, S, H, D, 1.0, dout, eager_bf16=True)
    assert torch.equal(e[0], ob)
    assert (e[2] == dqb).float().mean() > 0.99
    assert ((e[3] - dpb).norm() / dpb.norm()) < 1e-2


def test_kernel_emulation_is_close_to_fp32():
    B, S, H, D = 1, 40, 2, 16
    qkv = O.randn((B * S, 3 * H * D), 11)
    pd = O.randn((H, 2 * S - 1), 12, std=0.3, dtype=torch.float32)
    dout = O.randn((B * S, H * D), 13)
    r = O.relpos_manual(qkv, pd, B, S, H, D, 0.25, dout)
    k = O.relpos_kernel_emulated(qkv, pd, B, S, H, D, 0.25, dout)
    for a, b in ((k[0], r[0]), (k[1], r[2]), (k[2], r[3])):
        assert ((a.float() - b).norm() / b.norm()) < 2e-2


def test_geglu_erf_approximation_bound():
    """The GEGLU kernels evaluate erf with Abramowitz & Stegun 7.1.26 (constants as in
    kernel-rsi_amd/csrc/geglu.hip `erf_as`). Evaluated in float32, as the kernel does, it must
    stay within 6e-7 of erf everywhere (the published bound is 1.5e-7 in exact arithmetic),
    which is ~1/6500 of a bf16 ulp at 1; a wrong coefficient or sign breaks the bound."""
    f32 = np.float32
    p = f32(0.3275911)
    a1, a2, a3, a4, a5 = (f32(v) for v in (0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429))
    x = np.linspace(-12.0, 12.0, 240001).astype(np.float32)
    ax = np.abs(x)
    t = f32(1) / (f32(1) + p * ax)
    q = ((((a5 * t + a4) * t + a3) * t + a2) * t + a1) * t
    y = np.copysign(f32(1) - q * np.exp(-(ax * ax)).astype(np.float32), x)
    ref = np.array([math.erf(float(v)) for v in x])
    assert np.abs(y.astype(np.float64) - ref).max() < 6e-7
    assert y[0] == -1.0 and y[-1] == 1.0 and y[len(x) // 2] == 0.0


# ---------------------------------------------------------- fp16 rounding points
def test_f16_round_matches_torch_including_ties_and_subnormals():
    """The oracle's fp16 runs round with torch's .to(float16); numpy's binary16 conversion
    (an independent implementation) agrees on normals, exact ties, subnormals and overflow."""
    gen = torch.Generator().manual_seed(14)
    a = (torch.randn(100000, generator=gen) * 300).numpy()
    base = np.float32([1.0, 1.5, -3.0, 0.3, 2.0 ** -20])       # 2^-20 is subnormal in fp16
    ulp = np.float32([2.0 ** -10, 2.0 ** -10, 2.0 ** -9, 2.0 ** -12, 2.0 ** -24])
    ties = base + ulp / 2                                        # exactly half-way
    a = np.concatenate([a, ties, np.float32([0.0, -0.0, 1e-8, 6e-8, 65504.0, 65519.0, 65520.0, 1e6])])
    ref = torch.from_numpy(a).to(torch.float16).float().numpy()
    np.testing.assert_array_equal(O.f16_round(a), ref)
    assert O.f16_round(np.float32([65520.0]))[0] == np.inf


def test_rmsnorm_rounding_points_pinned_fp16():
    """fp16 run of the oracle: x*r rounded to fp16 before * w, as in the bf16 case."""
    x = O.randn((256, 1152), 15, dtype=torch.float16)
    w = O.randn((1152,), 16, std=0.02, mean=1.0, dtype=torch.float16)
    y = O.rmsnorm(x, w, 1e-6).float().numpy()
    emu = O.rmsnorm_eager_np(x.float().numpy(), w.float().numpy(), 1e-6, O.f16_round)
    assert (emu == y).mean() > 0.999
    xf = x.float().numpy()
    r = 1.0 / np.sqrt((xf * xf).mean(-1, keepdims=True, dtype=np.float32) + np.float32(1e-6))
    planted = O.f16_round(w.float().numpy() * (xf * r))
    assert (planted == y).mean() < 0.95


def test_eager_emulation_matches_sdpa_fp16():
    """oracle.relpos_manual(eager_dtype=fp16) reproduces the eager fp16 run of the reference
    (SDPA-MATH): out within one fp16 rounding, dqkv up to fp32 summation order."""
    B, S, H, D = 2, 33, 2, 16
    qkv = O.randn((B * S, 3 * H * D), 8, std=0.6, dtype=torch.float16)
    pd = O.randn((H, 2 * S - 1), 9, dtype=torch.float32)
    dout = O.randn((B * S, H * D), 10, dtype=torch.float16)
    ob, dqb, dpb = O.relpos_train(qkv, pd, B, S, H, D, 1.0, dout, torch.float16, sdpa=True)
    e = O.relpos_manual(qkv, pd, B, S, H, D, 1.0, dout, eager_dtype=torch.float16)
    assert e[0].dtype == torch.float16 and e[2].dtype == torch.float16
    assert (e[0] == ob).float().mean() > 0.99
    assert (e[2] == dqb).float().mean() > 0.98
    assert ((e[3] - dpb).norm() / dpb.norm()) < 1e-2


def test_kernel_emulation_fp16_is_close_to_fp32():
    B, S, H, D = 1, 40, 2, 16
    qkv = O.randn((B * S, 3 * H * D), 11, dtype=torch.float16)
    pd = O.randn((H, 2 * S - 1), 12, std=0.3, dtype=torch.float32)
    dout = O.randn((B * S, H * D), 13, dtype=torch.float16)
    r = O.relpos_manual(qkv, pd, B, S, H, D, 0.25, dout)
    k = O.relpos_kernel_emulated(qkv, pd, B, S, H, D, 0.25, dout, dtype=torch.float16)
    assert k[0].dtype == torch.float16
    for a, b in ((k[0], r[0]), (k[1], r[2]), (k[2], r[3])):
        assert ((a.float() - b).norm() / b.norm()) < 5e-3


# -------------------------------------------------------- T5 bucket map (host side)
@pytest.mark.parametrize("S,bidir,nb,maxd", [(1, True, 32, 128), (2, True, 32, 128), (100, True, 32, 128),
                                             (4096, True, 32, 128), (4096, False, 32, 128),
                                             (1000, True, 64, 256), (300, True, 16, 32)])
def test_t5_bucket_map_matches_transformers(S, bidir, nb, maxd):
    """The library's bucket map (torch ops, any device; here the CPU) equals transformers'
    T5Attention._relative_position_bucket for every distance, boundary distances included."""
    import relpos_attention as A

    ours = A.t5_relative_position_bucket(S, bidir, nb, maxd, "cpu")
    assert ours.dtype == torch.int32
    assert torch.equal(ours.long(), O.t5_bucket(S, bidir, nb, maxd))


def test_t5_bucket_map_against_closed_form():
    """The T5 map from its definition in float64 away from bucket boundaries: distance 0 -> 0,
    |d| < 8 exact, sign split at 16, |d| >= 128 -> last bucket, log spacing in between."""
    b = O.t5_bucket(4096).numpy()
    d = np.arange(-4095, 4096)
    for dist, bk in zip(d, b):
        a = abs(int(dist))
        base = 16 if dist > 0 else 0
        if a < 8:
            want = a
        else:
            x = 8 + math.log(a / 8) / math.log(16) * 8
            if abs(x - round(x)) < 1e-6:       # on a boundary: fp32 rounding decides
                continue
            want = min(int(x), 15)
        assert bk == base + want, (dist, bk, base + want)
