"""Write the golden fixtures of tests/golden/ from the oracle's float64 closed forms.

    python tests/golden/make_golden.py

Inputs are CPU-generator seeded and bf16-representable (stored as float32); expected outputs
are float64 from krsi_oracle.*_np64 (the textbook math, no intermediate rounding). The
reference (kernel-rsi) ships no golden vectors for this path, so these fixtures pin the oracle
against later edits; the math itself is pinned by the closed-form and autograd tests in
tests/test_oracle.py.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "oracle"))
import krsi_oracle as O  # noqa: E402


def f32(t):
    return t.float().numpy()


def main():
    # RMSNorm: ragged row length, eps as the BASELINE configs.
    x, w, g = O.randn((5, 24), 100), O.randn((24,), 101, std=0.1, mean=1.0), O.randn((5, 24), 102)
    y, rstd, dx, dw = O.rmsnorm_np64(f32(x), f32(w), 1e-6, f32(g))
    np.savez(HERE / "rmsnorm.npz", x=f32(x), w=f32(w), g=f32(g), eps=1e-6, y=y, rstd=rstd, dx=dx, dw=dw)
    # GEGLU: both GELU forms.
    u, gg = O.randn((3, 32), 110, std=2.0), O.randn((3, 16), 111)
    out_t, du_t = O.geglu_np64(f32(u), f32(gg), "tanh")
    out_e, du_e = O.geglu_np64(f32(u), f32(gg), "none")
    np.savez(HERE / "geglu.npz", u=f32(u), g=f32(gg), out_tanh=out_t, du_tanh=du_t, out_erf=out_e, du_erf=du_e)
    # Relative-position attention: B2 S7 H2 D8 (ragged S, two heads), scale 0.3.
    B, S, H, D, scale = 2, 7, 2, 8, 0.3
    qkv = O.randn((B * S, 3 * H * D), 120)
    pd = O.randn((H, 2 * S - 1), 121, std=0.5, dtype=O.torch.float32)
    dout = O.randn((B * S, H * D), 122)
    out, lse, dqkv, dpd = O.relpos_np64(f32(qkv), f32(pd), B, S, H, D, scale, f32(dout))
    np.savez(HERE / "relpos.npz", qkv=f32(qkv), pd=f32(pd), dout=f32(dout), dims=np.array([B, S, H, D]),
             scale=scale, out=out, lse=lse, dqkv=dqkv, dpd=dpd)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
