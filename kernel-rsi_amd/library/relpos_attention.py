"""Non-causal flash attention with a learned bias indexed by key - query distance, forward and
backward, on gfx950 (MI355X) HIP kernels: bf16 or fp16 activations on 16-bit MFMA, fp32
activations on fp32 MFMA, with the softmax in fp32 either way.

relpos_attention(qkv, pd, B, S, H, D, scale) returns [B*S, H*D].
  qkv  [B*S, 3*H*D]: the fused projection output. Token t holds q, k and v of head h at columns
       h*D, H*D + h*D and 2*H*D + h*D. It is read in place when its rows start on 16-byte
       boundaries (base address and row stride a multiple of 16 bytes: a row stride that is a
       multiple of 8 elements for bf16/fp16, of 4 for fp32) with unit column stride. Any other
       layout is accepted as the reference accepts it, through one contiguous copy of its first
       3*H*D columns (the gradient still flows to the original tensor).
  pd   [H, 2S-1] fp32: the bias of query i and key j in head h is pd[h, j - i + S - 1]. This
       covers T5 relative positions, ALiBi and any other Toeplitz bias.
The backward keeps the fp32 output to form delta_i = sum_d dO_id * O_id; a forward that no
backward can follow (grad mode off, or neither input requiring grad) stores O alone. The
backward sums dS along its diagonals inside the kernels to form pd's gradient. No
[B, H, S, S] tensor is ever allocated.
D may be any multiple of 8 up to 128 (D = 72 runs). Same public functions and arguments as the
reference's library/relpos_attention.py:198-222; usable under torch.compile(fullgraph=True).
"""
import math
import sys
from pathlib import Path

import torch
import torch.nn.functional as F

sys.path.insert(0, str(Path(__file__).resolve().parent))
import _hip  # noqa: E402
from _compat import compiling  # noqa: E402

LOG2E = 1.4426950408889634


def _ops():
    import _ops as ops  # noqa: PLC0415 - registers the krsi:: ops on first use
    return ops


class RelPosAttention(torch.autograd.Function):
    """Eager path: launches the kernels directly (reference: relpos_attention.py:160-172)."""

    @staticmethod
    def forward(ctx, qkv, pd, B, S, H, D, scale):
        out, out32, lse = _hip.relpos_fwd(qkv, pd, B, S, H, D, scale)
        ctx.save_for_backward(qkv, pd, out32, lse)
        ctx.dims = (B, S, H, D, scale)
        return out

    @staticmethod
    def backward(ctx, dout):
        dqkv, dpd = _hip.relpos_bwd(dout.contiguous(), *ctx.saved_tensors, *ctx.dims)
        return dqkv, dpd, None, None, None, None, None


def _kernel_layout(qkv, H, D):
    """qkv itself when the kernels can read it in place, else a contiguous copy of its q, k and
    v columns (differentiable, so the gradient of the copy reaches qkv)."""
    if qkv.dim() != 2:
        return qkv  # rejected with its shape by the kernel wrapper
    rows_aligned = qkv.stride(1) == 1 and (qkv.stride(0) * qkv.element_size()) % 16 == 0
    if rows_aligned and (compiling() or qkv.data_ptr() % 16 == 0):
        return qkv
    return qkv[:, :3 * H * D].clone(memory_format=torch.contiguous_format)


def relpos_attention(qkv, pd, B, S, H, D, scale):
    qkv = _kernel_layout(qkv, H, D)
    if compiling():
        return _ops().relpos_fwd_op(qkv, pd, B, S, H, D, scale)[0]
    if not (torch.is_grad_enabled() and (qkv.requires_grad or pd.requires_grad)):
        # No backward can follow: the kernels skip the fp32 output and lse it would need.
        return _hip.relpos_fwd(qkv, pd, B, S, H, D, scale, stats=False)[0]
    return RelPosAttention.apply(qkv, pd, B, S, H, D, scale)


# ------------------------------------------ bucketed relative-position table (T5)
_BUCKETS = {}


def t5_relative_position_bucket(S, bidirectional=True, num_buckets=32, max_distance=128, device="cuda"):
    """[2S-1] int32: the T5 bucket of every distance d = j - i = r - (S - 1) (memory minus query
    position), by the T5 formula (transformers T5Attention._relative_position_bucket) in the
    same fp32 op sequence, so distances on a bucket boundary fall as they do in T5. Index setup
    only (built once per arguments and device, then cached); the table math is in the kernels."""
    if compiling():  # traced into the graph (no cache mutation under torch.compile)
        return _t5_bucket_map(S, bidirectional, num_buckets, max_distance, device)
    key = (S, bool(bidirectional), num_buckets, max_distance, str(device))
    if key not in _BUCKETS:
        _BUCKETS[key] = _t5_bucket_map(S, bidirectional, num_buckets, max_distance, device)
    return _BUCKETS[key]


def _t5_bucket_map(S, bidirectional, num_buckets, max_distance, device):
    d = torch.arange(2 * S - 1, device=device, dtype=torch.long) - (S - 1)
    ret = torch.zeros_like(d)
    n = num_buckets
    if bidirectional:
        n //= 2
        ret = ret + (d > 0).to(torch.long) * n
        a = torch.abs(d)
    else:
        a = -torch.min(d, torch.zeros_like(d))
    max_exact = n // 2
    large = max_exact + (torch.log(a.float() / max_exact) / math.log(max_distance / max_exact)
                         * (n - max_exact)).to(torch.long)
    large = torch.min(large, torch.full_like(large, n - 1))
    return (ret + torch.where(a < max_exact, a, large)).to(torch.int32)


class BucketTable(torch.autograd.Function):
    """pd [H, 2S-1] = table[bucket, :].T by the gather kernel; backward: the bucket-sum kernel
    (the reference's note LESSONS.md:35: diagonals, then buckets, no scatter)."""

    @staticmethod
    def forward(ctx, table, bucket, S):
        ctx.save_for_backward(bucket)
        ctx.S, ctx.nb = S, table.shape[0]
        return _hip.relpos_bucket_gather(table, bucket, S)

    @staticmethod
    def backward(ctx, dpd):
        (bucket,) = ctx.saved_tensors
        return _hip.relpos_bucket_sum(dpd, bucket, ctx.S, ctx.nb), None, None


def t5_relpos_table(table, S, bidirectional=True, max_distance=128):
    """pd [H, 2S-1] fp32 for relpos_attention from a T5 relative_attention_bias weight
    table [num_buckets, H] fp32: pd[h, j - i + S - 1] = table[bucket(j - i), h], the bias
    T5Attention.compute_bias builds as [1, H, S, S]. Differentiable w.r.t. table."""
    bucket = t5_relative_position_bucket(S, bidirectional, table.shape[0], max_distance, table.device)
    if compiling():
        return _ops().bucket_gather_op(table, bucket, S)
    return BucketTable.apply(table, bucket, S)


def reference(qkv, pd, B, S, H, D, scale):
    q, k, v = qkv.view(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
    pos = torch.arange(S, device=qkv.device)
    bias = pd[:, pos[None, :] - pos[:, None] + S - 1][None].to(qkv.dtype)
    from torch.nn.attention import SDPBackend, sdpa_kernel  # noqa: PLC0415

    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias, scale=scale)
    return o.transpose(1, 2).reshape(B * S, H * D)


def selftest():
    from _harness import selftest_autograd  # noqa: PLC0415

    B, S, H, D = 4, 512, 16, 64
    qkv = (0.6 * torch.randn(B * S, 3 * H * D, device="cuda")).to(torch.bfloat16)
    pd = torch.randn(H, 2 * S - 1, device="cuda")
    return selftest_autograd(lambda q, p: relpos_attention(q, p, B, S, H, D, 1.0),
                             lambda q, p: reference(q, p, B, S, H, D, 1.0), [qkv, pd])


if __name__ == "__main__":
    print(selftest())
