"""CPU oracle of the kernel-rsi fused kernels (RMSNorm, GEGLU, relative-position attention).

TEST INFRASTRUCTURE ONLY. This module is the checker, never the product: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it. The library in
kernel-rsi_amd/ never imports it and has no CPU path.

Three layers, each pinning the next:
  1. numpy float64 closed forms (`*_np64`): the textbook math of each op and its gradient,
     written independently of torch (explicit softmax, explicit diagonal sums for dpd).
  2. torch restatements of the reference's `reference()` formulas and their autograd
     backward (`rmsnorm`, `geglu`, `relpos`), run on the CPU in fp32 ("ref32", TF32 is
     irrelevant on the CPU) or bf16 (the eager "original" the parity criterion is scaled
     by). relpos uses explicit matmul + softmax in fp32 and the reference's SDPA-MATH
     formulation (`relpos_sdpa`) is kept to cross-check it.
  3. `bf16_round` - round-to-nearest-even to bfloat16 emulated with integer arithmetic in
     numpy, used to pin the rounding points of layer 2's bf16 runs; fp16 runs are pinned
     against numpy's own IEEE binary16 conversion (`f16_round`), fp32 runs need none.

Reference files followed (kernel-rsi, read, not run):
  rmsnorm          library/rmsnorm.py:113-115 (reference), :22-51 (kernel math)
  geglu            library/geglu.py:111-113 (reference, tanh), :20-52 (kernel math)
  relpos_attention library/relpos_attention.py:204-212 (reference), :26-59 (lse, log2 domain),
                   :143-157 (delta, dpd as the diagonal sum of dS)
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

LOG2E = 1.4426950408889634


# ---------------------------------------------------------------- bf16 rounding
def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32.
    Integer emulation, independent of torch: add 0x7FFF + lsb of the kept half, truncate."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = a[nan]
    return out


def f16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest IEEE binary16 (ties to even, subnormals kept,
    overflow to inf) with numpy's conversion, independent of torch; returned as float32."""
    with np.errstate(over="ignore"):
        return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def to_bf16_exact(t: torch.Tensor) -> torch.Tensor:
    """bf16 tensor -> float64 numpy (exact)."""
    return t.detach().to(torch.float64).cpu().numpy()


# --------------------------------------------------------------------- RMSNorm
def rmsnorm(x2d: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """The reference's formula (library/rmsnorm.py:113-115), in the inputs' dtype semantics."""
    var = x2d.float().pow(2).mean(-1, keepdim=True)
    return w * (x2d.float() * torch.rsqrt(var + eps)).to(x2d.dtype)


def rmsnorm_train(x2d, w, eps, g, dtype=torch.float32):
    """(y, dx, dw) of rmsnorm with inputs cast to `dtype`, autograd backward under cotangent g."""
    x = x2d.detach().to(dtype).requires_grad_(True)
    ww = w.detach().to(dtype).requires_grad_(True)
    y = rmsnorm(x, ww, eps)
    dx, dw = torch.autograd.grad(y, [x, ww], g.to(y.dtype))
    return y.detach(), dx, dw


def rmsnorm_np64(x: np.ndarray, w: np.ndarray, eps: float, g: np.ndarray):
    """Closed form in float64 without intermediate rounding:
    r = (mean x^2 + eps)^-1/2, y = w x r, dx = r (g w) - x r^3 mean(g w x), dw = sum_rows g x r.
    Returns (y, rstd, dx, dw)."""
    x, w, g = (np.asarray(a, np.float64) for a in (x, w, g))
    n = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / n + eps)
    y = w * x * r
    gw = g * w
    dx = r * gw - x * r ** 3 * (gw * x).sum(-1, keepdims=True) / n
    dw = (g * x * r).sum(0)
    return y, r[:, 0], dx, dw


def rmsnorm_eager_np(x: np.ndarray, w: np.ndarray, eps: float, rnd) -> np.ndarray:
    """rmsnorm_eager_bf16_np with the rounding function `rnd` of the activation dtype."""
    x = np.asarray(x, np.float32)
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True, dtype=np.float32) + np.float32(eps))
    return rnd(np.asarray(w, np.float32) * rnd(x * r))


def rmsnorm_eager_bf16_np(x_bf: np.ndarray, w_bf: np.ndarray, eps: float) -> np.ndarray:
    """Eager bf16 forward with its rounding points made explicit: fp32 statistics,
    bf16(x * r), then bf16(w * that). x_bf, w_bf hold bf16 values (as float32)."""
    x = x_bf.astype(np.float32)
    var = (x * x).astype(np.float32).mean(-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    n = bf16_round(x * r)
    return bf16_round(w_bf.astype(np.float32) * n)


# ----------------------------------------------------------------------- GEGLU
def geglu(u: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    """The reference's formula (library/geglu.py:111-113), with the GELU form selectable."""
    a, b = u.chunk(2, dim=-1)
    return F.gelu(a, approximate=approximate) * b


def geglu_train(u, g, approximate="tanh", dtype=torch.float32):
    uu = u.detach().to(dtype).requires_grad_(True)
    out = geglu(uu, approximate)
    (du,) = torch.autograd.grad(out, [uu], g.to(out.dtype))
    return out.detach(), du


def geglu_np64(u: np.ndarray, g: np.ndarray, approximate: str = "tanh"):
    """Closed form in float64: out = gelu(a) b; da = g b gelu'(a); db = g gelu(a).
    gelu_tanh(a) = a/2 (1 + tanh(c (a + k a^3))), gelu_erf(a) = a/2 (1 + erf(a / sqrt 2))."""
    u, g = np.asarray(u, np.float64), np.asarray(g, np.float64)
    f = u.shape[-1] // 2
    a, b = u[..., :f], u[..., f:]
    if approximate == "tanh":
        c, k = math.sqrt(2.0 / math.pi), 0.044715
        t = np.tanh(c * (a + k * a ** 3))
        gel = 0.5 * a * (1 + t)
        dgel = 0.5 * (1 + t) + 0.5 * a * (1 - t * t) * c * (1 + 3 * k * a * a)
    else:
        erf = np.vectorize(math.erf)(a / math.sqrt(2.0))
        gel = 0.5 * a * (1 + erf)
        dgel = 0.5 * (1 + erf) + a * np.exp(-0.5 * a * a) / math.sqrt(2 * math.pi)
    return gel * b, np.concatenate([g * b * dgel, g * gel], axis=-1)


# ------------------------------------------------ relative-position attention
def split_qkv(qkv: torch.Tensor, B: int, S: int, H: int, D: int):
    """q, k, v as [B, H, S, D] views of the fused [B*S, >=3*H*D] projection."""
    t = qkv[:, :3 * H * D].reshape(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
    return t[0], t[1], t[2]


def bias_matrix(pd: torch.Tensor, S: int) -> torch.Tensor:
    """[H, S, S] Toeplitz bias, bias[h, i, j] = pd[h, j - i + S - 1]."""
    pos = torch.arange(S, device=pd.device)
    return pd[:, pos[None, :] - pos[:, None] + S - 1]


def relpos(qkv, pd, B, S, H, D, scale):
    """Explicit-math restatement of the reference: softmax(q k^T scale + bias) v, in the
    dtype of qkv for the products and fp32 softmax when qkv is fp32. Returns [B*S, H*D]."""
    q, k, v = split_qkv(qkv, B, S, H, D)
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale + bias_matrix(pd, S)[None].to(qkv.dtype)
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, v)
    return o.transpose(1, 2).reshape(B * S, H * D)


def relpos_sdpa(qkv, pd, B, S, H, D, scale):
    """The reference's own formulation (SDPA, MATH backend), CPU only."""
    q, k, v = split_qkv(qkv, B, S, H, D)
    from torch.nn.attention import SDPBackend, sdpa_kernel  # noqa: PLC0415

    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias_matrix(pd, S)[None].to(qkv.dtype),
                                           scale=scale)
    return o.transpose(1, 2).reshape(B * S, H * D)


def relpos_lse(qkv, pd, B, S, H, D, scale) -> torch.Tensor:
    """lse[b*H + h, i] = log2 sum_j exp(q_i . k_j scale + bias_ij) (the kernel's log2 domain)."""
    q, k, v = split_qkv(qkv.float(), B, S, H, D)
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale + bias_matrix(pd.float(), S)[None]
    return (torch.logsumexp(s, dim=-1) * LOG2E).reshape(B * H, S)


def relpos_train(qkv, pd, B, S, H, D, scale, dout, dtype=torch.float32, sdpa=False):
    """(out, dqkv, dpd) with qkv cast to `dtype` (pd stays fp32, as the reference's table)."""
    x = qkv.detach().to(dtype).requires_grad_(True)
    p = pd.detach().to(torch.float64 if dtype == torch.float64 else torch.float32).requires_grad_(True)
    out = (relpos_sdpa if sdpa else relpos)(x, p, B, S, H, D, scale)
    dqkv, dpd = torch.autograd.grad(out, [x, p], dout.to(out.dtype))
    return out.detach(), dqkv, dpd


def diag_sum(ds: torch.Tensor, S: int) -> torch.Tensor:
    """[..., H, S, S] -> [H, 2S-1]: sum over leading dims and along the diagonals j - i."""
    ds = ds.reshape(-1, *ds.shape[-3:]).sum(0)
    H = ds.shape[0]
    pos = torch.arange(S, device=ds.device)
    idx = (pos[None, :] - pos[:, None] + S - 1).reshape(-1)
    out = torch.zeros(H, 2 * S - 1, device=ds.device, dtype=ds.dtype)
    return out.index_add_(1, idx, ds.reshape(H, S * S))


def relpos_manual(qkv, pd, B, S, H, D, scale, dout, eager_bf16=False, eager_dtype=None,
                  compute_dtype=torch.float32):
    """Forward and backward of the reference in explicit math with contiguous matmul operands
    (device-agnostic; no 16-bit batched product is ever formed), in compute_dtype (fp32, or
    float64 for the reference of fp32 inputs).
      no eager dtype : the reference (ref32) of the inputs.
      eager_dtype=T  : the eager original in dtype T (bf16 or fp16) as torch runs it -
                       SDPA-MATH upcasts 16-bit inputs to fp32 internally, so it is this fp32
                       math with the bias rounded to T (relpos_attention.py:207), out and dqkv
                       rounded to T, and dpd the fp32 diagonal sum of T-rounded dS (the
                       gather's backward). eager_bf16=True is eager_dtype=torch.bfloat16.
    Returns (out [B*S, H*D], lse [B*H, S] log2 domain, dqkv [B*S, 3*H*D], dpd [H, 2S-1])."""
    if eager_bf16:
        eager_dtype = torch.bfloat16
    cdt = compute_dtype
    q, k, v = (t.to(cdt).contiguous() for t in split_qkv(qkv, B, S, H, D))
    bias = bias_matrix(pd.to(cdt), S)[None]
    if eager_dtype is not None:
        bias = bias.to(eager_dtype).float()
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale + bias
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    del s
    o = torch.matmul(p, v)
    do = dout.to(cdt).reshape(B, S, H, D).permute(0, 2, 1, 3).contiguous()
    dp = torch.matmul(do, v.transpose(-2, -1).contiguous())
    delta = (do * o).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    del dp
    dv = torch.matmul(p.transpose(-2, -1).contiguous(), do)
    del p
    dq = torch.matmul(ds, k) * scale
    dk = torch.matmul(ds.transpose(-2, -1).contiguous(), q) * scale
    if eager_dtype is not None:
        ds = ds.to(eager_dtype).float()
    dpd = diag_sum(ds, S)
    del ds
    out = o.permute(0, 2, 1, 3).reshape(B * S, H * D)
    dqkv = torch.stack([dq, dk, dv], dim=2).permute(0, 3, 2, 1, 4).reshape(B * S, 3 * H * D)
    if eager_dtype is not None:
        out, dqkv = out.to(eager_dtype), dqkv.to(eager_dtype)
    return out, (lse * LOG2E).reshape(B * H, S), dqkv, dpd


def relpos_kernel_emulated(qkv, pd, B, S, H, D, scale, dout, dtype=torch.bfloat16):
    """The reference Triton kernels' rounding points, in fp32 math with contiguous operands
    (the yardstick "the reference kernel's own error"), for activations of `dtype` (T, the
    dtype of q, k and v: bf16 or fp16):
      forward  acc = T(p_u) v with p_u = exp(s - rowmax), l = sum p_u (fp32), o = acc / l,
               stored as out32 (fp32) and out (T)                    (relpos_attention.py:49-58)
      backward p = exp(s - lse) fp32, dv = T(p)^T dO (:88), dp = dO v^T (:89),
               delta = sum dO * out32 (:144), ds = p (dp - delta) (:90),
               dk = scale T(ds)^T q (:92-93), dq = scale T(ds) k (:125-126),
               dpd = diagonal sums of fp32 ds (:91, :154-156); dqkv rounded to T.
    Returns (out T, dqkv T, dpd fp32)."""
    bf = lambda t: t.to(dtype).float()  # noqa: E731
    q, k, v = (t.float().contiguous() for t in split_qkv(qkv, B, S, H, D))
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale + bias_matrix(pd.float(), S)[None]
    m = s.amax(-1, keepdim=True)
    pu = torch.exp(s - m)
    lsum = pu.sum(-1, keepdim=True)
    o32 = torch.matmul(bf(pu), v) / lsum
    del pu
    lse = m + torch.log(lsum)
    p = torch.exp(s - lse)
    del s
    do = dout.float().reshape(B, S, H, D).permute(0, 2, 1, 3).contiguous()
    dv = torch.matmul(bf(p).transpose(-2, -1).contiguous(), do)
    dp = torch.matmul(do, v.transpose(-2, -1).contiguous())
    delta = (do * o32).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    del dp, p
    dsb = bf(ds)
    dq = torch.matmul(dsb, k) * scale
    dk = torch.matmul(dsb.transpose(-2, -1).contiguous(), q) * scale
    del dsb
    dpd = diag_sum(ds, S)
    out = o32.permute(0, 2, 1, 3).reshape(B * S, H * D).to(dtype)
    dqkv = torch.stack([dq, dk, dv], dim=2).permute(0, 3, 2, 1, 4).reshape(B * S, 3 * H * D)
    return out, dqkv.to(dtype), dpd


def t5_bucket(S: int, bidirectional: bool = True, num_buckets: int = 32, max_distance: int = 128):
    """[2S-1] int64 T5 bucket of every distance j - i = r - (S - 1), by transformers'
    T5Attention._relative_position_bucket itself (the published implementation the T5 bias
    step follows; transformers is installed, this runs it on the CPU as the checker)."""
    from transformers.models.t5.modeling_t5 import T5Attention  # noqa: PLC0415

    d = torch.arange(2 * S - 1, dtype=torch.long) - (S - 1)
    return T5Attention._relative_position_bucket(d, bidirectional, num_buckets, max_distance)


def relpos_np64(qkv: np.ndarray, pd: np.ndarray, B, S, H, D, scale, dout: np.ndarray):
    """Float64 closed form with explicit loops over (b, h):
      s = q k^T scale + T, p = softmax(s), o = p v, lse = log2 sum exp(s)
      dP = dO v^T, delta_i = dO_i . o_i, dS = p (dP - delta)
      dq = scale dS k, dk = scale dS^T q, dv = p^T dO, dpd[h, j - i + S - 1] += dS[i, j].
    Returns (out [B*S, H*D], lse [B*H, S], dqkv [B*S, 3*H*D], dpd [H, 2S-1])."""
    qkv = np.asarray(qkv, np.float64)[:, :3 * H * D].reshape(B, S, 3, H, D)
    pd = np.asarray(pd, np.float64)
    dout = np.asarray(dout, np.float64).reshape(B, S, H, D)
    out = np.zeros((B, S, H, D))
    lse = np.zeros((B, H, S))
    dqkv = np.zeros((B, S, 3, H, D))
    dpd = np.zeros((H, 2 * S - 1))
    ii, jj = np.meshgrid(np.arange(S), np.arange(S), indexing="ij")
    diag = jj - ii + S - 1
    for b in range(B):
        for h in range(H):
            q, k, v = qkv[b, :, 0, h], qkv[b, :, 1, h], qkv[b, :, 2, h]
            s = q @ k.T * scale + pd[h][diag]
            m = s.max(-1, keepdims=True)
            e = np.exp(s - m)
            z = e.sum(-1, keepdims=True)
            p = e / z
            o = p @ v
            out[b, :, h] = o
            lse[b, h] = (np.log(z[:, 0]) + m[:, 0]) / math.log(2.0)
            do = dout[b, :, h]
            dp = do @ v.T
            delta = (do * o).sum(-1, keepdims=True)
            ds = p * (dp - delta)
            dqkv[b, :, 0, h] = scale * ds @ k
            dqkv[b, :, 1, h] = scale * ds.T @ q
            dqkv[b, :, 2, h] = p.T @ do
            for i in range(S):
                for j in range(S):
                    dpd[h, j - i + S - 1] += ds[i, j]
    return (out.reshape(B * S, H * D), lse.reshape(B * H, S), dqkv.reshape(B * S, 3 * H * D), dpd)


# ------------------------------------------------------------ seeded inputs
def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, seed: int, std: float = 1.0, mean: float = 0.0, dtype=torch.bfloat16) -> torch.Tensor:
    """CPU-generated N(mean, std^2) cast to dtype: the same values on every machine."""
    return (torch.randn(shape, generator=gen(seed)) * std + mean).to(dtype)


# ------------------------------------------------- CPU baseline (eager path)
def cpu_eager_step(kind: str, inputs: dict):
    """One fwd+bwd (or, with inputs["fwd_only"], one forward) of the reference's eager torch
    path on the CPU, in the inputs' dtype (the cpu_baseline legs)."""
    fwd_only = inputs.get("fwd_only", False)

    def leaves(*names):
        return [inputs[n].detach().requires_grad_(not fwd_only) for n in names]

    if kind == "rmsnorm":
        x, w = leaves("x", "w")
        y = rmsnorm(x, w, inputs["eps"])
        return y if fwd_only else torch.autograd.grad(y, [x, w], inputs["g"])
    if kind == "geglu":
        (u,) = leaves("u")
        out = geglu(u, inputs.get("approximate", "tanh"))
        return out if fwd_only else torch.autograd.grad(out, [u], inputs["g"])
    if kind == "relpos":
        qkv, pd = leaves("qkv", "pd")
        B, S, H, D = inputs["dims"]
        out = relpos_sdpa(qkv, pd, B, S, H, D, inputs["scale"])
        return out if fwd_only else torch.autograd.grad(out, [qkv, pd], inputs["dout"])
    raise ValueError(kind)
