"""The reference's acceptance protocol on the GPU, through the library's own `selftest_autograd`
(fp32 reference vs eager original vs kernel under one random cotangent, then the kernel under
torch.compile(fullgraph=True); tools/common.py:476-518 in the reference), for each op, without
timing. A graph break or a fake-tensor mismatch under compile fails the compiled check."""
import pytest
import torch

import geglu as G
import relpos_attention as A
import rmsnorm as R
from _harness import selftest_autograd
from krsi_testutil import log, seeded

pytestmark = pytest.mark.gpu


def _check(res):
    assert res["pass"], res["checks"]
    assert res["compiled"].get("pass"), res["compiled"]


def test_rmsnorm_selftest_protocol_and_compile():
    log("selftest_autograd rmsnorm [1024, 1152] + torch.compile(fullgraph)")
    torch.manual_seed(0)
    x = seeded((1024, 1152), 0)
    w = (1 + 0.02 * seeded((1152,), 1, dtype=torch.float32)).to(torch.bfloat16)
    _check(selftest_autograd(lambda x, w: R.rmsnorm(x, w, 1e-6), lambda x, w: R.reference(x, w, 1e-6),
                             [x, w], time=False))


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_geglu_selftest_protocol_and_compile(approximate):
    log(f"selftest_autograd geglu [512, 2*1408] {approximate} + torch.compile(fullgraph)")
    torch.manual_seed(0)
    u = seeded((512, 2 * 1408), 0)
    _check(selftest_autograd(lambda u: G.geglu(u, approximate=approximate),
                             lambda u: G.reference(u, approximate=approximate), [u], time=False))


def test_relpos_selftest_protocol_and_compile():
    B, S, H, D = 2, 256, 4, 64
    log(f"selftest_autograd relpos B{B} S{S} H{H} D{D} + torch.compile(fullgraph)")
    torch.manual_seed(0)
    qkv = (0.6 * seeded((B * S, 3 * H * D), 0, dtype=torch.float32)).to(torch.bfloat16)
    pd = seeded((H, 2 * S - 1), 1, dtype=torch.float32)
    _check(selftest_autograd(lambda q, p: A.relpos_attention(q, p, B, S, H, D, 1.0),
                             lambda q, p: A.reference(q, p, B, S, H, D, 1.0), [qkv, pd], time=False))


def test_t5_table_chain_selftest_protocol_and_compile():
    """T5 relative_attention_bias table -> pd (gather kernel) -> attention, gradient to the table
    through the bucket-sum kernel, against the reference with pd gathered by torch indexing."""
    B, S, H, D = 2, 256, 4, 64
    log(f"selftest_autograd t5 table chain B{B} S{S} H{H} D{D} + torch.compile(fullgraph)")
    torch.manual_seed(0)
    qkv = (0.6 * seeded((B * S, 3 * H * D), 0, dtype=torch.float32)).to(torch.bfloat16)
    table = seeded((32, H), 2, std=0.5, dtype=torch.float32)
    bucket = A.t5_relative_position_bucket(S, True, 32, 128, "cuda").long()
    _check(selftest_autograd(lambda q, t: A.relpos_attention(q, A.t5_relpos_table(t, S), B, S, H, D, 0.125),
                             lambda q, t: A.reference(q, t[bucket].t(), B, S, H, D, 0.125),
                             [qkv, table], time=False))


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_rmsnorm_geglu_selftest_other_dtypes(dt):
    log(f"selftest_autograd rmsnorm and geglu in {dt} + torch.compile(fullgraph)")
    torch.manual_seed(0)
    x = seeded((512, 1152), 0, dtype=dt)
    w = (1 + 0.02 * seeded((1152,), 1, dtype=torch.float32)).to(dt)
    _check(selftest_autograd(lambda x, w: R.rmsnorm(x, w, 1e-6), lambda x, w: R.reference(x, w, 1e-6),
                             [x, w], time=False))
    u = seeded((256, 2 * 1408), 3, dtype=dt)
    _check(selftest_autograd(lambda u: G.geglu(u, approximate="tanh"),
                             lambda u: G.reference(u, approximate="tanh"), [u], time=False))


@pytest.mark.parametrize("dt", [torch.float16, torch.float32], ids=["float16", "float32"])
def test_relpos_selftest_other_dtypes(dt):
    """fp16, and fp32 on fp32 MFMA: in fp32 the eager original equals the fp32 reference up to
    summation order, so the criterion is its floors (rel-L2 1e-5, 1e-3 of the peak per element)."""
    B, S, H, D = 2, 256, 4, 64
    log(f"selftest_autograd relpos {dt} B{B} S{S} H{H} D{D} + torch.compile(fullgraph)")
    torch.manual_seed(0)
    qkv = (0.6 * seeded((B * S, 3 * H * D), 0, dtype=torch.float32)).to(dt)
    pd = seeded((H, 2 * S - 1), 1, dtype=torch.float32)
    _check(selftest_autograd(lambda q, p: A.relpos_attention(q, p, B, S, H, D, 1.0),
                             lambda q, p: A.reference(q, p, B, S, H, D, 1.0), [qkv, pd], time=False))
