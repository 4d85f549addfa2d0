"""RMSNorm with its backward, on gfx950 (MI355X) HIP kernels: rmsnorm(x2d, weight, eps).

Each row is scaled by the reciprocal root of its mean square (fp32 arithmetic). The normalised
row is rounded to the input dtype before it is multiplied by the weight, as the reference
formula below (and the eager models it stands in for) does. The forward keeps one fp32
reciprocal root per row for the backward. The backward writes dx in a single pass over the rows.
The weight gradient is summed into per-workgroup fp32 partial rows, which one small launch
then adds in a fixed order, so dw is bitwise reproducible. Row lengths up to 16384.
Same public functions and arguments as the reference's library/rmsnorm.py:106-123; usable under
torch.compile(fullgraph=True).
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


class RMSNorm(torch.autograd.Function):
    """Eager path: launches the kernels directly (reference: rmsnorm.py:71-83)."""

    @staticmethod
    def forward(ctx, x2d, w, eps):
        y, rstd = _hip.rmsnorm_fwd(x2d, w, eps)
        ctx.save_for_backward(x2d, w, rstd)
        return y

    @staticmethod
    def backward(ctx, g):
        x2d, w, rstd = ctx.saved_tensors
        dx, dw = _hip.rmsnorm_bwd(g.contiguous(), x2d, w, rstd)
        return dx, dw, None


def rmsnorm(x2d, w, eps):
    """y = w * (x * rsqrt(mean(x^2) + eps)).to(x.dtype), rows of a 2D contiguous tensor."""
    if compiling():
        return _ops().rmsnorm_fwd_op(x2d, w, eps)[0]
    return RMSNorm.apply(x2d, w, eps)


def reference(x2d, w, eps):
    var = x2d.float().pow(2).mean(-1, keepdim=True)
    return w * (x2d.float() * torch.rsqrt(var + eps)).to(x2d.dtype)


def selftest():
    from _harness import selftest_autograd  # noqa: PLC0415

    x = torch.randn(4096, 1024, device="cuda", dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1024, device="cuda")).to(torch.bfloat16)
    return selftest_autograd(lambda x, w: rmsnorm(x, w, 1e-6), lambda x, w: reference(x, w, 1e-6), [x, w])


if __name__ == "__main__":
    print(selftest())
