"""The bucketed relative-position table step (T5) on the GPU: the gather that builds pd from a
[num_buckets, H] table and the bucket sum that is its backward, against torch indexing and a
float64 index_add, and the whole T5 chain table -> pd -> attention -> dtable.

Tolerance, stated: the gather is bitwise (it copies); the bucket sum within 1e-6 relative of a
float64 sum (fp32 addition of at most 2S-1 terms in a fixed order) and bitwise reproducible;
the chain's dtable within 2x of the eager bf16 original's error, as every other output."""
import pytest
import torch

import _hip
import krsi_oracle as O
import relpos_attention as A
from krsi_testutil import assert_parity, log, seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,H,nb,bidir,maxd", [(1, 4, 32, True, 128), (7, 2, 32, True, 128),
                                              (512, 16, 32, True, 128), (4096, 16, 32, True, 128),
                                              (300, 8, 32, False, 128), (1000, 3, 64, True, 256)])
def test_bucket_map_gather_and_sum(S, H, nb, bidir, maxd):
    log(f"t5 buckets S{S} H{H} nb{nb} bidir {bidir} max_distance {maxd}")
    bucket = A.t5_relative_position_bucket(S, bidir, nb, maxd, "cuda")
    ref_map = O.t5_bucket(S, bidir, nb, maxd)
    assert torch.equal(bucket.cpu().long(), ref_map)
    table = seeded((nb, H), 60, dtype=torch.float32)
    pd = _hip.relpos_bucket_gather(table, bucket, S)
    assert torch.equal(pd, table[bucket.long()].t())
    dpd = seeded((H, 2 * S - 1), 61, dtype=torch.float32)
    dt = _hip.relpos_bucket_sum(dpd, bucket, S, nb)
    ref = torch.zeros(nb, H, dtype=torch.float64).index_add_(0, bucket.cpu().long(), dpd.cpu().double().t())
    err = (dt.cpu().double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)
    assert err < 1e-6, err
    assert torch.equal(dt, _hip.relpos_bucket_sum(dpd, bucket, S, nb))


def test_bucket_map_out_of_range_entries():
    """Gather writes NaN for a bucket outside [0, nb); the sum ignores such entries."""
    S, H, nb = 50, 3, 8
    bucket = torch.randint(0, nb, (2 * S - 1,), generator=torch.Generator().manual_seed(0)).to(torch.int32)
    bucket[[0, 10, 98]] = torch.tensor([-1, nb, 1 << 20], dtype=torch.int32)
    bucket = bucket.cuda()
    table = seeded((nb, H), 62, dtype=torch.float32)
    pd = _hip.relpos_bucket_gather(table, bucket, S)
    bad = torch.zeros(2 * S - 1, dtype=torch.bool)
    bad[[0, 10, 98]] = True
    assert torch.isnan(pd[:, bad.cuda()]).all() and not torch.isnan(pd[:, ~bad.cuda()]).any()
    dpd = seeded((H, 2 * S - 1), 63, dtype=torch.float32)
    ok = ~bad
    ref = torch.zeros(nb, H, dtype=torch.float64).index_add_(0, bucket.cpu().long()[ok], dpd.cpu().double().t()[ok])
    dt = _hip.relpos_bucket_sum(dpd, bucket, S, nb)
    assert (dt.cpu().double() - ref).abs().max() < 1e-6 * ref.abs().max()


def test_t5_chain_table_to_attention_gradient():
    """table [32, H] -> pd -> relpos attention -> dtable, against the fp32 reference chain
    (explicit math, pd gathered in torch, dtable summed in float64) with the eager bf16 original
    (bias rounded to bf16, as the reference's reference() does) as the yardstick."""
    B, S, H, D, scale = 2, 256, 4, 64, 0.125
    log(f"t5 chain B{B} S{S} H{H} D{D}")
    qkv = seeded((B * S, 3 * H * D), 64)
    dout = seeded((B * S, H * D), 65)
    table = seeded((32, H), 66, std=0.5, dtype=torch.float32)
    t = table.detach().requires_grad_(True)
    x = qkv.detach().requires_grad_(True)
    pd = A.t5_relpos_table(t, S)
    out = A.relpos_attention(x, pd, B, S, H, D, scale)
    dqkv, dtable = torch.autograd.grad(out, [x, t], dout)
    bucket = O.t5_bucket(S, True, 32, 128)
    pd_ref = table.cpu()[bucket].t().contiguous()
    r = O.relpos_manual(qkv.cpu(), pd_ref, B, S, H, D, scale, dout.cpu())
    o = O.relpos_manual(qkv.cpu(), pd_ref, B, S, H, D, scale, dout.cpu(), eager_bf16=True)

    def to_table(dpd):
        return torch.zeros(32, H, dtype=torch.float64).index_add_(0, bucket, dpd.double().t()).float()

    assert_parity(["out", "dqkv", "dtable"], (r[0], r[2], to_table(r[3])), (o[0], o[2], to_table(o[3])),
                  (out.detach().cpu(), dqkv.cpu(), dtable.cpu()), row_slack=float("inf"))
