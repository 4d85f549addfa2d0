"""GEGLU HIP kernels vs the fp32 reference on the GPU (parity tests proper)."""
import pytest
import torch

import geglu as G
import krsi_oracle as O
from krsi_testutil import assert_parity, log, seeded

pytestmark = pytest.mark.gpu


def _run(u, g, approximate):
    ref32 = O.geglu_train(u, g.float(), approximate, torch.float32)
    orig = O.geglu_train(u, g, approximate, torch.bfloat16)
    uu = u.detach().requires_grad_(True)
    out = G.geglu(uu, approximate=approximate)
    (du,) = torch.autograd.grad(out, [uu], g)
    return ref32, orig, (out.detach(), du)


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_geglu_train_step_full(approximate):
    """u [4,2048,8192] -> out [4,2048,4096], da and db vs fp32 autograd."""
    log(f"geglu fwd+bwd [8192, 8192] approximate={approximate}")
    u = seeded((8192, 8192), 0)
    g = seeded((8192, 4096), 2)
    ref32, orig, cand = _run(u, g, approximate)
    assert_parity(["out", "du"], ref32, orig, cand)
    # Forward bitwise against eager bf16, except where gelu(a) sits on a bf16 rounding tie.
    same = (cand[0] == orig[0]).float().mean().item()
    assert same > 0.999, same


@pytest.mark.parametrize("approximate", ["none", "tanh"])
@pytest.mark.parametrize("rows,f", [(1, 8), (3, 1), (7, 1001), (64, 2816), (300, 64), (2, 4100)])
def test_geglu_shapes(rows, f, approximate):
    log(f"geglu shapes rows={rows} f={f} {approximate}")
    u = seeded((rows, 2 * f), 20 + f, std=2.0)
    g = seeded((rows, f), 21)
    ref32, orig, cand = _run(u, g, approximate)
    assert_parity(["out", "du"], ref32, orig, cand)


def test_geglu_extreme_inputs_finite():
    """Large |a| saturates tanh (exp overflow path) and erf; results stay finite."""
    a = torch.tensor([-100.0, -20.0, -5.0, 0.0, 5.0, 20.0, 100.0, 3e4], device="cuda")
    u = torch.cat([a, torch.ones_like(a)]).to(torch.bfloat16)[None]
    for approx in ("tanh", "none"):
        uu = u.clone().requires_grad_(True)
        out = G.geglu(uu, approximate=approx)
        (du,) = torch.autograd.grad(out, [uu], torch.ones_like(out))
        ref = O.geglu(u.float(), approx).to(torch.bfloat16)
        assert torch.isfinite(out).all() and torch.isfinite(du).all()
        assert torch.allclose(out.float(), ref.float(), rtol=1e-2, atol=1e-2), (out, ref)


def test_geglu_deterministic():
    u = seeded((512, 4096), 0)
    g = seeded((512, 2048), 2)
    import _hip

    assert torch.equal(_hip.geglu_bwd(g, u), _hip.geglu_bwd(g, u))
    assert torch.equal(_hip.geglu_fwd(u), _hip.geglu_fwd(u))


def test_geglu_rejects_bad_input():
    with pytest.raises(ValueError):
        G.geglu(torch.randn(4, 8, dtype=torch.bfloat16))            # CPU tensor
    with pytest.raises(ValueError):
        G.geglu(torch.randn(4, 7, device="cuda", dtype=torch.bfloat16))  # odd width
    with pytest.raises(ValueError):
        G.geglu(torch.randn(4, 8, device="cuda", dtype=torch.bfloat16), approximate="sigmoid")


@pytest.mark.parametrize("f", [8, 3])
def test_geglu_rows_beyond_grid_y(f):
    """rows > 65535: the grid's row dimension is capped and each block strides over rows."""
    log(f"geglu rows=70000 f={f}")
    u = seeded((70000, 2 * f), 70 + f, std=2.0)
    g = seeded((70000, f), 71)
    ref32, orig, cand = _run(u, g, "tanh")
    assert_parity(["out", "du"], ref32, orig, cand)
