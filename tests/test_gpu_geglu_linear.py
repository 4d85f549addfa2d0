"""The merged gate|up projection with the GEGLU epilogue fused into it (geglu_linear) against the
unfused pair the reference's geglu takes its input from (geglu.py:3-5): u = x @ w.T, then GEGLU.

Tolerance, stated: the reference's acceptance rule with slack 2 (tools/common.py:322-392,
476-518), as for every op here. Output, dx and dw are checked against the fp32 run of the unfused
pair, with the eager bf16 (or fp16) unfused pair as the yardstick, then again under
torch.compile(fullgraph=True). The fused kernel rounds the projection to the activation dtype
before the GEGLU, as the unfused pair's u tensor holds it."""
import pytest
import torch

import geglu as G
from _harness import selftest_autograd
from krsi_testutil import log, seeded

pytestmark = pytest.mark.gpu

CASES = [  # rows, K, F, approximate, dtype
    (300, 256, 128, "tanh", torch.bfloat16),     # ragged rows: a partial row block
    (1024, 1024, 512, "none", torch.bfloat16),
    (1, 64, 64, "tanh", torch.bfloat16),
    (640, 512, 192, "tanh", torch.float16),
    (2048, 2048, 1024, "none", torch.bfloat16),
]


@pytest.mark.parametrize("rows,K,F,approximate,dt", CASES)
def test_geglu_linear_matches_unfused_pair(rows, K, F, approximate, dt):
    log(f"geglu_linear x[{rows},{K}] w[{2 * F},{K}] {approximate} {dt}")
    torch.manual_seed(0)
    x = seeded((rows, K), 0, dtype=dt)
    w = (seeded((2 * F, K), 1, dtype=torch.float32) / K ** 0.5).to(dt)
    res = selftest_autograd(lambda a, b: G.geglu_linear(a, b, approximate=approximate),
                            lambda a, b: G.reference_linear(a, b, approximate=approximate), [x, w], time=False)
    assert res["pass"], res["checks"]
    assert res["compiled"].get("pass"), res["compiled"]


def test_geglu_linear_is_the_gemm_output_rounded_then_geglu():
    """Same inputs through the fused kernel and through hipBLASLt's GEMM + the GEGLU kernel: the
    two differ only by the GEMM's summation order, so every output is within a few bf16 ulps."""
    rows, K, F = 512, 1024, 256
    x = seeded((rows, K), 3)
    w = (seeded((2 * F, K), 4, dtype=torch.float32) / K ** 0.5).to(torch.bfloat16)
    fused = G.geglu_linear(x, w)
    unfused = G.geglu(torch.nn.functional.linear(x, w))
    rel = ((fused.float() - unfused.float()).abs() / (unfused.float().abs() + 1e-2)).max().item()
    assert rel < 0.05, rel


@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
def test_geglu_linear_frozen_weight_gets_no_gradient(compiled):
    """With the weight frozen the backward forms only dx, which equals the dx of the full
    backward bitwise (the same kernels on the same inputs)."""
    rows, K, F = 256, 512, 128
    log(f"geglu_linear frozen weight, {'compiled' if compiled else 'eager'}")
    x0 = seeded((rows, K), 5)
    w0 = (seeded((2 * F, K), 6, dtype=torch.float32) / K ** 0.5).to(torch.bfloat16)
    gy = seeded((rows, F), 7)
    fn = lambda a, b: G.geglu_linear(a, b)  # noqa: E731
    if compiled:
        torch._dynamo.reset()
        fn = torch.compile(fn, fullgraph=True)
    x, w = x0.clone().requires_grad_(True), w0.clone()
    fn(x, w).backward(gy)
    assert w.grad is None
    xf, wf = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    fn(xf, wf).backward(gy)
    assert torch.equal(x.grad, xf.grad) and wf.grad is not None
