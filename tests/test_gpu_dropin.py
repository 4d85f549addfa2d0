"""The caller flow the reference's tools drive, with these kernels as the drop-in.

The flow (tools/region.py:29-47, tools/swap.py:67-71, and the krsi_patch.apply /
remove that tools/report.py:91-105 generates):
  * each region's impl.py defines forward(mod, ...) on the library functions;
  * apply(model) binds that forward to the module instance with types.MethodType;
  * remove(model) drops the instance attribute again.

The model is a two-block T5-style encoder stack. Each block has:
  * RMSNorm;
  * a fused qkv projection into relative-position attention, whose bias comes from a bucketed
    nn.Embedding exactly as in T5;
  * RMSNorm again;
  * a merged gate|up projection into GEGLU (tanh), then the down projection.
It is checked as swap.py checks a training model:
  * the loss, the output and the gradient of every parameter of the patched bf16 model (on the
    GPU) against a float32 run of the unpatched model;
  * the unpatched bf16 model is the noise yardstick (compare(), slack 2, per-row 3x);
  * the check runs before and after one update of all weights.
The unpatched models run on the CPU: eager bf16 attention there uses batched bf16 products,
which this suite keeps off the GPU. remove() must restore the original forward bitwise.
"""
import copy
import importlib.util
import math
import sys
import textwrap
import types
from pathlib import Path

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

import krsi_oracle as O
from krsi_testutil import assert_parity, log

pytestmark = pytest.mark.gpu

LIBDIR = Path(__file__).resolve().parents[1] / "kernel-rsi_amd" / "library"


# ---------------------------------------------------------------- the model
class T5RMSNorm(nn.Module):
    def __init__(self, n, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.eps = eps

    def forward(self, x):
        var = x.float().pow(2).mean(-1, keepdim=True)
        return self.weight * (x.float() * torch.rsqrt(var + self.eps)).to(x.dtype)


class RelPosSelfAttention(nn.Module):
    def __init__(self, d_model, H, D, num_buckets=32, max_distance=128):
        super().__init__()
        self.H, self.D, self.max_distance, self.scale = H, D, max_distance, 1.0 / math.sqrt(D)
        self.qkv = nn.Linear(d_model, 3 * H * D, bias=False)
        self.o = nn.Linear(H * D, d_model, bias=False)
        self.relative_attention_bias = nn.Embedding(num_buckets, H)

    def forward(self, x):
        B, S, _ = x.shape
        q, k, v = self.qkv(x).view(B, S, 3, self.H, self.D).permute(2, 0, 3, 1, 4)
        bucket = O.t5_bucket(S, True, self.relative_attention_bias.num_embeddings, self.max_distance)
        pos = torch.arange(S)
        rel = bucket.to(x.device)[pos[None, :] - pos[:, None] + S - 1]     # [S, S] bucket of j - i
        bias = self.relative_attention_bias(rel).permute(2, 0, 1)[None]   # [1, H, S, S]
        with sdpa_kernel(SDPBackend.MATH):
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias.to(q.dtype), scale=self.scale)
        return self.o(o.transpose(1, 2).reshape(B, S, self.H * self.D))


class GatedMLP(nn.Module):
    def __init__(self, d_model, d_ff):
        super().__init__()
        self.wi = nn.Linear(d_model, 2 * d_ff, bias=False)  # merged gate | up
        self.wo = nn.Linear(d_ff, d_model, bias=False)

    def forward(self, x):
        a, b = self.wi(x).chunk(2, dim=-1)
        return self.wo(F.gelu(a, approximate="tanh") * b)


class Block(nn.Module):
    def __init__(self, d_model, H, D, d_ff):
        super().__init__()
        self.norm1, self.attn = T5RMSNorm(d_model), RelPosSelfAttention(d_model, H, D)
        self.norm2, self.mlp = T5RMSNorm(d_model), GatedMLP(d_model, d_ff)

    def forward(self, x):
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))


class Encoder(nn.Module):
    def __init__(self, layers=2, d_model=256, H=4, D=64, d_ff=512):
        super().__init__()
        self.blocks = nn.ModuleList(Block(d_model, H, D, d_ff) for _ in range(layers))

    def forward(self, x):
        for blk in self.blocks:
            x = blk(x)
        return x


# ------------------------------------------- regions (impl.py) and the patch
IMPLS = {
    "rmsnorm": f'''
        import sys
        sys.path.insert(0, {str(LIBDIR)!r})
        from rmsnorm import rmsnorm

        def forward(mod, x):
            return rmsnorm(x.reshape(-1, x.shape[-1]), mod.weight, mod.eps).view(x.shape)
    ''',
    "attention": f'''
        import sys
        sys.path.insert(0, {str(LIBDIR)!r})
        from relpos_attention import relpos_attention, t5_relpos_table

        def forward(mod, x):
            B, S, _ = x.shape
            qkv = mod.qkv(x.reshape(B * S, -1))
            pd = t5_relpos_table(mod.relative_attention_bias.weight.float(), S, True, mod.max_distance)
            o = relpos_attention(qkv, pd, B, S, mod.H, mod.D, mod.scale)
            return mod.o(o).view(B, S, -1)
    ''',
    "geglu": f'''
        import sys
        sys.path.insert(0, {str(LIBDIR)!r})
        from geglu import geglu

        def forward(mod, x):
            u = mod.wi(x.reshape(-1, x.shape[-1]))
            return mod.wo(geglu(u, approximate="tanh")).view(*x.shape[:-1], -1)
    ''',
}
REGION_OF = {T5RMSNorm: "rmsnorm", RelPosSelfAttention: "attention", GatedMLP: "geglu"}


def _load(path: Path):
    spec = importlib.util.spec_from_file_location("krsi_impl_" + path.parent.name, path / "impl.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class Patch:
    """What report.py exports as krsi_patch: PATCHES maps module qualnames to region dirs."""

    def __init__(self, model: nn.Module, root: Path):
        self.patches = {}
        for name, impl in IMPLS.items():
            d = root / name
            d.mkdir()
            (d / "impl.py").write_text(textwrap.dedent(impl))
        for q, m in model.named_modules():
            if type(m) in REGION_OF:
                self.patches[q] = root / REGION_OF[type(m)]
        self.impls = {d: _load(d) for d in set(self.patches.values())}

    def apply(self, model):
        named = dict(model.named_modules())
        for q, d in self.patches.items():
            m = named[q]
            m.forward = types.MethodType(lambda self, *a, _i=self.impls[d], **k: _i.forward(self, *a, **k), m)
        return model

    def remove(self, model):
        named = dict(model.named_modules())
        for q in self.patches:
            named[q].__dict__.pop("forward", None)
        return model


# ----------------------------------------------------------------- the check
def _step(model, x, target):
    """Loss, output and the gradient of every parameter (swap.py's training comparison)."""
    model.zero_grad(set_to_none=True)
    out = model(x)
    loss = F.mse_loss(out.float(), target)
    loss.backward()
    grads = [p.grad.detach().float().cpu() for p in model.parameters()]
    return [loss.detach().float().cpu().reshape(1), out.detach().float().cpu(), *grads]


def _randomize(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm1.weight") or name.endswith("norm2.weight"):
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            elif "relative_attention_bias" in name:
                p.copy_(0.5 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[-1]))


def _update(models, seed):
    """One identical weight update of every model (the same step for all of them)."""
    g = torch.Generator().manual_seed(seed)
    deltas = [0.02 * torch.randn(p.shape, generator=g) * p.detach().float().abs().mean().cpu()
              for p in models[0].parameters()]
    with torch.no_grad():
        for m in models:
            for p, d in zip(m.parameters(), deltas):
                p.add_(d.to(p.device, p.dtype))


def test_patched_model_matches_fp32_training_step(tmp_path):
    B, S = 2, 256
    base = Encoder()
    _randomize(base, 0)
    x32 = torch.randn(B, S, 256, generator=torch.Generator().manual_seed(1))
    target = torch.randn(B, S, 256, generator=torch.Generator().manual_seed(2))
    ref32 = copy.deepcopy(base).float()                 # float32 run of the original (CPU)
    orig = copy.deepcopy(base).to(torch.bfloat16)       # the original bf16 model (CPU)
    cand = copy.deepcopy(base).to(torch.bfloat16).cuda()
    patch = Patch(cand, tmp_path)
    assert len(patch.patches) == 8                      # 2 blocks x (2 norms, attention, MLP)
    patch.apply(cand)
    names = ["loss", "out"] + [n for n, _ in base.named_parameters()]
    for rnd in range(2):
        log(f"drop-in: T5-style encoder B{B} S{S}, round {rnd} (after {rnd} weight update)")
        r = _step(ref32, x32, target)
        o = _step(orig, x32.to(torch.bfloat16), target)
        c = _step(cand, x32.to(torch.bfloat16).cuda(), target.cuda())
        assert_parity(names, r, o, c, extra_msg=f"drop-in round {rnd}")
        _update([ref32, orig, cand], 10 + rnd)

    # remove() restores the class forward on every patched module, and the model computes
    # bitwise what the unpatched original computes (both on the CPU, same weights).
    patch.remove(cand)
    named = dict(cand.named_modules())
    assert all("forward" not in named[q].__dict__ for q in patch.patches)
    cand_cpu = cand.cpu()
    with torch.no_grad():
        xb = x32.to(torch.bfloat16)
        assert torch.equal(cand_cpu(xb), orig(xb))
    # apply() again on the CPU model: the library has no CPU path and says so.
    patch.apply(cand_cpu)
    with pytest.raises(ValueError, match="no CPU path"):
        cand_cpu(xb)
