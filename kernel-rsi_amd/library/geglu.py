"""Gated GELU of a fused gate|up projection, on gfx950 (MI355X) HIP kernels: geglu(u).

u is [rows, 2F]: the gate half a = u[:, :F] and the linear half b = u[:, F:], as one merged GEMM
produces them. The result is gelu(a) * b, with gelu(a) rounded to u's dtype before the
product, as in eager torch. The default is the tanh form. geglu(u, approximate="none") gives
the erf form. The backward writes the gradient of both halves into one [rows, 2F] tensor in
one pass, so the merged GEMM's backward takes a single gradient. Same public functions and
arguments as the reference's library/geglu.py:104-120; usable under torch.compile(fullgraph=True).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
import _hip  # noqa: E402
from _compat import compiling  # noqa: E402


def _ops():
    import _ops as ops  # noqa: PLC0415 - registers the krsi:: ops on first use
    return ops


class GEGLU(torch.autograd.Function):
    """Eager path: launches the kernels directly (reference: geglu.py:71-82)."""

    @staticmethod
    def forward(ctx, u, approximate):
        ctx.save_for_backward(u)
        ctx.approximate = approximate
        return _hip.geglu_fwd(u, approximate)

    @staticmethod
    def backward(ctx, g):
        (u,) = ctx.saved_tensors
        return _hip.geglu_bwd(g.contiguous(), u, ctx.approximate), None


def geglu(u, *, approximate="tanh"):
    """gelu(u[:, :F]) * u[:, F:] for a contiguous [rows, 2F] tensor (tanh GELU by default)."""
    if compiling():
        return _ops().geglu_fwd_op(u, approximate)
    return GEGLU.apply(u, approximate)


class GEGLULinear(torch.autograd.Function):
    """Eager path of geglu_linear: one fused kernel forward; the backward recomputes u with the
    vendor GEMM (the forward never wrote it), runs the GEGLU backward kernel on it, and forms
    dx = du w and dw = du^T x with the vendor GEMM."""

    @staticmethod
    def forward(ctx, x, w, approximate):
        ctx.save_for_backward(x, w)
        ctx.approximate = approximate
        return _hip.geglu_linear_fwd(x, w, approximate)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        u = torch.nn.functional.linear(x, w)
        du = _hip.geglu_bwd(g.contiguous(), u, ctx.approximate)
        dx = du @ w if ctx.needs_input_grad[0] else None
        dw = du.t().contiguous() @ x if ctx.needs_input_grad[1] else None
        return dx, dw, None


def geglu_linear(x, w, *, approximate="tanh"):
    """geglu(x @ w.T) for x [rows, K] and the merged weight w = cat([W_gate, W_up]) [2F, K], with
    the GEGLU forward fused into the projection's epilogue (u is never written). bf16 or fp16;
    K and F multiples of 64. Differentiable in x and w."""
    if compiling():
        return _ops().geglu_linear_fwd_op(x, w, approximate)
    return GEGLULinear.apply(x, w, approximate)


def reference(u, *, approximate="tanh"):
    a, b = u.chunk(2, dim=-1)
    return torch.nn.functional.gelu(a, approximate=approximate) * b


def reference_linear(x, w, *, approximate="tanh"):
    """The unfused pair geglu_linear stands for: the merged projection, then reference()."""
    return reference(torch.nn.functional.linear(x, w), approximate=approximate)


def selftest():
    from _harness import selftest_autograd  # noqa: PLC0415

    u = torch.randn(2048, 2 * 2816, device="cuda", dtype=torch.bfloat16)
    return selftest_autograd(geglu, reference, [u])


if __name__ == "__main__":
    print(selftest())
