"""torch.library registrations of the kernels (the compile path).

Registered once per process: every public module imports this module by the
same top-level name, so loading a public module twice (for example under
replay.py's per-file module names) does not register the ops twice.

Op names follow the reference (library/rmsnorm.py:86-103, geglu.py:85-101,
relpos_attention.py:175-195): krsi::rmsnorm_fwd/bwd, krsi::geglu_fwd/bwd,
krsi::relpos_attn_fwd/bwd; krsi::relpos_bucket_gather/sum (the T5 table step) and
krsi::geglu_linear_fwd (the merged projection with the GEGLU epilogue) have no counterpart there. Their schemas are internal to this library.
"""
from __future__ import annotations

import torch
from torch import Tensor

import _hip

# ------------------------------------------------------------------- RMSNorm


@torch.library.custom_op("krsi::rmsnorm_fwd", mutates_args=())
def rmsnorm_fwd_op(x2d: Tensor, w: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return _hip.rmsnorm_fwd(x2d, w, eps)


@rmsnorm_fwd_op.register_fake
def _(x2d, w, eps):
    return torch.empty_like(x2d), x2d.new_empty((x2d.shape[0],), dtype=torch.float32)


@torch.library.custom_op("krsi::rmsnorm_bwd", mutates_args=())
def rmsnorm_bwd_op(g: Tensor, x2d: Tensor, w: Tensor, rstd: Tensor) -> tuple[Tensor, Tensor]:
    return _hip.rmsnorm_bwd(g, x2d, w, rstd)


@rmsnorm_bwd_op.register_fake
def _(g, x2d, w, rstd):
    return torch.empty_like(x2d), torch.empty_like(w)


def _rms_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1], output[1])


def _rms_backward(ctx, gy, _grstd):
    x2d, w, rstd = ctx.saved_tensors
    dx, dw = rmsnorm_bwd_op(gy.contiguous(), x2d, w, rstd)
    return dx, dw, None


rmsnorm_fwd_op.register_autograd(_rms_backward, setup_context=_rms_setup)

# --------------------------------------------------------------------- GEGLU


@torch.library.custom_op("krsi::geglu_fwd", mutates_args=())
def geglu_fwd_op(u: Tensor, approximate: str) -> Tensor:
    return _hip.geglu_fwd(u, approximate)


@geglu_fwd_op.register_fake
def _(u, approximate):
    return u.new_empty((u.shape[0], u.shape[1] // 2))


@torch.library.custom_op("krsi::geglu_bwd", mutates_args=())
def geglu_bwd_op(g: Tensor, u: Tensor, approximate: str) -> Tensor:
    return _hip.geglu_bwd(g, u, approximate)


@geglu_bwd_op.register_fake
def _(g, u, approximate):
    return torch.empty_like(u)


def _geglu_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.approximate = inputs[1]


def _geglu_backward(ctx, g):
    (u,) = ctx.saved_tensors
    return geglu_bwd_op(g.contiguous(), u, ctx.approximate), None


geglu_fwd_op.register_autograd(_geglu_backward, setup_context=_geglu_setup)


@torch.library.custom_op("krsi::geglu_linear_fwd", mutates_args=())
def geglu_linear_fwd_op(x: Tensor, w: Tensor, approximate: str) -> Tensor:
    return _hip.geglu_linear_fwd(x, w, approximate)


@geglu_linear_fwd_op.register_fake
def _(x, w, approximate):
    return x.new_empty((x.shape[0], w.shape[0] // 2))


def _geglu_linear_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1])
    ctx.approximate = inputs[2]


def _geglu_linear_backward(ctx, g):
    x, w = ctx.saved_tensors
    u = torch.nn.functional.linear(x, w)  # recomputed: the forward never wrote it
    du = geglu_bwd_op(g.contiguous(), u, ctx.approximate)
    dx = du @ w if ctx.needs_input_grad[0] else None
    dw = du.t().contiguous() @ x if ctx.needs_input_grad[1] else None
    return dx, dw, None


geglu_linear_fwd_op.register_autograd(_geglu_linear_backward, setup_context=_geglu_linear_setup)

# ------------------------------------------------ relative-position attention


@torch.library.custom_op("krsi::relpos_attn_fwd", mutates_args=())
def relpos_fwd_op(qkv: Tensor, pd: Tensor, B: int, S: int, H: int, D: int,
                  scale: float) -> tuple[Tensor, Tensor, Tensor]:
    return _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)


@relpos_fwd_op.register_fake
def _(qkv, pd, B, S, H, D, scale):
    return (qkv.new_empty((B * S, H * D)), qkv.new_empty((B * S, H * D), dtype=torch.float32),
            qkv.new_empty((B * H, S), dtype=torch.float32))


@torch.library.custom_op("krsi::relpos_attn_bwd", mutates_args=())
def relpos_bwd_op(dout: Tensor, qkv: Tensor, pd: Tensor, out32: Tensor, lse: Tensor, B: int, S: int,
                  H: int, D: int, scale: float) -> tuple[Tensor, Tensor]:
    return _hip.relpos_bwd(dout, qkv, pd, out32, lse, B, S, H, D, scale)


@relpos_bwd_op.register_fake
def _(dout, qkv, pd, out32, lse, B, S, H, D, scale):
    return qkv.new_empty(qkv.shape), pd.new_empty((H, 2 * S - 1), dtype=torch.float32)


def _relpos_setup(ctx, inputs, output):
    qkv, pd, B, S, H, D, scale = inputs
    ctx.save_for_backward(qkv, pd, output[1], output[2])
    ctx.dims = (B, S, H, D, scale)


def _relpos_backward(ctx, dout, _d32, _dlse):
    dqkv, dpd = relpos_bwd_op(dout.contiguous(), *ctx.saved_tensors, *ctx.dims)
    return dqkv, dpd, None, None, None, None, None


relpos_fwd_op.register_autograd(_relpos_backward, setup_context=_relpos_setup)

# ------------------------------------------ bucketed relative-position table


@torch.library.custom_op("krsi::relpos_bucket_gather", mutates_args=())
def bucket_gather_op(table: Tensor, bucket: Tensor, S: int) -> Tensor:
    return _hip.relpos_bucket_gather(table, bucket, S)


@bucket_gather_op.register_fake
def _(table, bucket, S):
    return table.new_empty((table.shape[1], 2 * S - 1))


@torch.library.custom_op("krsi::relpos_bucket_sum", mutates_args=())
def bucket_sum_op(dpd: Tensor, bucket: Tensor, S: int, num_buckets: int) -> Tensor:
    return _hip.relpos_bucket_sum(dpd, bucket, S, num_buckets)


@bucket_sum_op.register_fake
def _(dpd, bucket, S, num_buckets):
    return dpd.new_empty((num_buckets, dpd.shape[0]))


def _bucket_setup(ctx, inputs, output):
    table, bucket, S = inputs
    ctx.save_for_backward(bucket)
    ctx.S, ctx.nb = S, table.shape[0]


def _bucket_backward(ctx, dpd):
    (bucket,) = ctx.saved_tensors
    return bucket_sum_op(dpd.contiguous(), bucket, ctx.S, ctx.nb), None, None


bucket_gather_op.register_autograd(_bucket_backward, setup_context=_bucket_setup)
