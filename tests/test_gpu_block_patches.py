"""The block-kernel model patches (tsplat.native_block_patches) on the GPU.

Each patched forward must return exactly what the corresponding
tsplat.block_ops kernel returns (those are bit-identical to the reference's
AVX-512 kernels, tests/test_gpu_block_ops.py) and stay within fp32
rounding of the plain torch computation it replaces; strict mode must raise
where the reference raises (grad mode, off-device input, unsupported
module), non-strict mode must fall back and count it.  The upstream model
module and the reference's attention patch are absent here, so the
norm/RoPE and block-elementwise patches are driven with stand-ins that have
the same attribute names.
"""
from __future__ import annotations

import math
import types

import pytest

pytestmark = pytest.mark.gpu


def _close(a, b, tol):
    import torch

    err = float((a - b).abs().max())
    scale = float(b.abs().max()) + 1e-30
    assert err <= tol * scale, (err, scale)
    assert bool(torch.isfinite(a).all())


def test_gelu_silu_patches(cuda):
    import torch
    import torch.nn as nn
    import torch.nn.functional as F
    from tsplat import block_ops
    from tsplat.native_block_patches import (apply_triposplat_native_gelu_avx512_patch,
                                             apply_triposplat_native_silu_avx512_patch)

    torch.manual_seed(0)
    m = nn.Sequential(nn.Linear(64, 96), nn.GELU(approximate="tanh"), nn.Linear(96, 64), nn.SiLU()).to(cuda)
    assert apply_triposplat_native_gelu_avx512_patch(m) == {"enabled": False}
    meta = apply_triposplat_native_gelu_avx512_patch(m, enabled=True)
    assert meta["selected"] == ["1"] and meta["skipped_count"] == 0 and meta["enabled"]
    meta_s = apply_triposplat_native_silu_avx512_patch(m, enabled=True)
    assert meta_s["selected"] == ["3"]
    y = torch.randn(7, 96, device=cuda) * 3
    z = torch.randn(7, 64, device=cuda) * 3
    with torch.no_grad():
        g, s = m[1](y), m[3](z)
        torch.cuda.synchronize(cuda)
        assert torch.equal(g, block_ops.gelu_tanh(y))
        assert torch.equal(s, block_ops.silu(z))
        _close(g, F.gelu(y, approximate="tanh"), 1e-6)
        _close(s, F.silu(z), 1e-6)
        out = m(torch.randn(3, 64, device=cuda))
    assert out.shape == (3, 64)
    assert meta["runtime"]["calls"] == 2 and meta_s["runtime"]["calls"] == 2
    with pytest.raises(RuntimeError, match="grad_enabled"):
        m[1](y)
    with torch.no_grad(), pytest.raises(RuntimeError, match="input_cpu"):
        m[3](z.cpu())
    with pytest.raises(ValueError, match="approximate=tanh"):
        apply_triposplat_native_gelu_avx512_patch(nn.Sequential(nn.GELU()).to(cuda), enabled=True)
    lax = nn.Sequential(nn.SiLU()).to(cuda)
    meta_l = apply_triposplat_native_silu_avx512_patch(lax, enabled=True, strict=False)
    assert torch.equal(lax(z), F.silu(z))  # grad mode: the original forward, counted
    assert meta_l["runtime"]["fallbacks"] == 1


def _rmsnorm_module(torch, heads, dim, device):
    """Stand-in for the upstream MultiHeadRMSNorm (matched by class name):
    x * sqrt(dim) / max(||x||, 1e-12) * gamma over the last dim, per head."""
    import torch.nn as nn

    class MultiHeadRMSNorm(nn.Module):
        def __init__(self):
            super().__init__()
            g = torch.Generator().manual_seed(2)
            self.gamma = nn.Parameter(1 + 0.1 * torch.randn(heads, dim, generator=g))

        def forward(self, x):
            n = x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
            return x * math.sqrt(dim) / n * self.gamma

    return MultiHeadRMSNorm().to(device)


def test_norm_rope_patch(cuda):
    import torch
    import torch.nn as nn
    import torch.nn.functional as F
    from tsplat import block_ops
    from tsplat.native_block_patches import apply_triposplat_native_norm_rope_avx512_patch

    torch.manual_seed(1)

    def torch_rope(h, f):
        return torch.view_as_real(torch.view_as_complex(h.reshape(*h.shape[:-1], -1, 2)) * f).flatten(-2)

    fake_model = types.ModuleType("fake_upstream_model")
    fake_model.apply_rotary_emb = torch_rope
    model = nn.ModuleDict({"ln": nn.LayerNorm(128, eps=1e-6), "ln_plain": nn.LayerNorm(128, elementwise_affine=False),
                           "rms": _rmsnorm_module(torch, 4, 64, cuda)}).to(cuda)
    with torch.no_grad():
        model["ln"].weight.uniform_(0.5, 1.5)
        model["ln"].bias.uniform_(-0.1, 0.1)
    x = torch.randn(2, 37, 128, device=cuda) * 2 + 0.5
    xh = torch.randn(2, 37, 4, 64, device=cuda)
    hidden = torch.randn(2, 4, 37, 64, device=cuda)
    ang = torch.rand(2, 4, 37, 32, device=cuda) * 6.28
    freqs = torch.polar(torch.ones_like(ang), ang)
    with torch.no_grad():
        want = (model["ln"](x), model["ln_plain"](x), model["rms"](xh), torch_rope(hidden, freqs))
    meta = apply_triposplat_native_norm_rope_avx512_patch(model, enabled=True, model_module=fake_model)
    assert meta["layernorm_selected_count"] == 2 and meta["rmsnorm_selected"] == ["rms"] and meta["rope_patched"]
    with torch.no_grad():
        got = (model["ln"](x), model["ln_plain"](x), model["rms"](xh), fake_model.apply_rotary_emb(hidden, freqs),
               model._native_avx512_functional_layernorm(x, eps=1e-5))
        torch.cuda.synchronize(cuda)
        assert torch.equal(got[0], block_ops.layer_norm(x, 1e-6, model["ln"].weight, model["ln"].bias))
        assert torch.equal(got[1], block_ops.layer_norm(x, 1e-5))
        assert torch.equal(got[2], block_ops.head_rmsnorm(xh, model["rms"].gamma, 1, 74, 4, dim=64,
                                                          out_bhld=False).view_as(xh))
        assert torch.equal(got[3], block_ops.rope_complex(hidden, torch.view_as_real(freqs).reshape(2, 4, 37, 64)))
    for g, w in zip(got[:4], want):
        _close(g, w, 2e-6)
    _close(got[4], F.layer_norm(x, (128,), eps=1e-5), 2e-6)
    assert meta["runtime"]["rope"]["calls"] == 1 and meta["runtime"]["layernorm"]["calls"] == 3
    with torch.no_grad(), pytest.raises(RuntimeError, match="shape"):
        fake_model.apply_rotary_emb(hidden, freqs[..., :16])  # frequencies that do not cover every vector


def test_block_elementwise_patch(cuda):
    import torch
    import torch.nn as nn
    from tsplat.native_block_patches import apply_triposplat_native_block_elementwise_avx512_patch

    torch.manual_seed(3)
    C = 96

    def torch_modulate(h, scale, shift):
        return h.mul_(1 + scale[:, None]).add_(shift[:, None])

    def torch_residual(x, h, gate):
        return x.add_(h * gate[:, None])

    tap = types.ModuleType("fake_attention_patch")
    tap._modulate_inplace_preserve_order = torch_modulate
    tap._residual_gate_inplace_preserve_order = torch_residual

    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.proj = nn.Linear(C, C)

        def forward(self, h, rope_emb=None):
            return self.proj(h)

    class UnifiedTransformerBlock(nn.Module):
        def __init__(self, modulation):
            super().__init__()
            self.modulation, self.share_mod = modulation, False
            self.adaLN_modulation = nn.Linear(C, 6 * C)
            self.shift_table = nn.Parameter(torch.randn(1, 6 * C) * 0.1)
            self.norm1 = nn.LayerNorm(C, elementwise_affine=False)
            self.norm2 = nn.LayerNorm(C, elementwise_affine=False)
            self.attn, self.mlp = Attn(), nn.Linear(C, C)

        def forward(self, x, mod=None, rotary_emb=None):
            if not self.modulation:
                x = x + self.attn(self.norm1(x), rope_emb=rotary_emb)
                return x + self.mlp(self.norm2(x))
            mod = self.adaLN_modulation(mod) + self.shift_table
            sh1, sc1, g1, sh2, sc2, g2 = mod.chunk(6, dim=1)
            x = torch_residual(x, self.attn(torch_modulate(self.norm1(x), sc1, sh1)), g1)
            return torch_residual(x, self.mlp(torch_modulate(self.norm2(x), sc2, sh2)), g2)

    model = nn.ModuleDict({"b0": UnifiedTransformerBlock(True), "b1": UnifiedTransformerBlock(False)}).to(cuda)
    x = torch.randn(1, 50, C, device=cuda)
    t = torch.randn(1, C, device=cuda)
    with torch.no_grad():
        want0 = model["b0"](x.clone(), t)
        want1 = model["b1"](x.clone())
    meta = apply_triposplat_native_block_elementwise_avx512_patch(model, enabled=True, attention_module=tap)
    assert sorted(meta["selected"]) == ["b0", "b1"]
    assert tap._modulate_inplace_preserve_order is not torch_modulate
    with torch.no_grad():
        got0 = model["b0"](x.clone(), t)
        got1 = model["b1"](x.clone())
    torch.cuda.synchronize(cuda)
    _close(got0, want0, 1e-5)
    _close(got1, want1, 1e-5)
    rt = meta["runtime"]
    assert rt["modulate"]["calls"] == 2 and rt["residual"]["calls"] == 2 and rt["add"]["calls"] == 3
    with pytest.raises(RuntimeError, match="modulate"):
        tap._modulate_inplace_preserve_order(x.cpu(), t.cpu(), t.cpu())
