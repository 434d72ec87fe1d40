"""The packed attention helpers patch (tsplat.native_qkv_packed_attention_v3),
mirroring scripts/native_qkv_packed_attention_patch_v3.py, on a toy model
with the upstream attention module's interface: module selection, the three
replaced helpers (standard, key-bias, selected rows), strict fall-back
errors, runtime counters.  Outputs are compared with a float64 host
computation of the same attention (qkv Linear on the decoded NF24 weights,
RoPE then RMSNorm, softmax(QK^T/8 + bias) V, out Linear): the device path
differs by fp32 GEMM / SDPA summation order only (relative RMSE <= 1e-5).
"""
from __future__ import annotations

import types

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _toy(torch, C=128, H=2):
    nn = torch.nn

    class Norm(nn.Module):
        def __init__(self):
            super().__init__()
            self.gamma = nn.Parameter(1.0 + 0.05 * torch.randn(H, 64))

    class RopeMultiHeadAttention(nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv = nn.Linear(C, 3 * C)
            self.out = nn.Linear(C, C)
            self.q_norm, self.k_norm = Norm(), Norm()
            self.num_heads, self.head_dim = H, 64
            self._type, self.use_rope, self.qk_rms_norm = "self", True, True

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = RopeMultiHeadAttention()

    class Toy(nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = nn.ModuleList([Block(), Block()])

    return Toy()


def _host_attention(attn, x, freqs, bias=None, rows=None):
    """float64 reference on the decoded weights the device uses."""
    from tsplat.nf24 import decode_nf24_i16_weight_t

    def lin(m, v):
        w = decode_nf24_i16_weight_t(m._native_rnf8_codes0_t, m._native_rnf8_codes1_t,
                                     m._native_rnf8_scales0).double().cpu().numpy()
        return v @ w + m._native_rnf8_bias.double().cpu().numpy()

    xb = x.double().cpu().numpy()[0]
    L, C = xb.shape
    H = attn.num_heads
    qkv = lin(attn.qkv, xb).reshape(L, 3, H, 64)
    f = freqs.double().cpu().numpy()[0]  # [L, H, 64] interleaved (cos, sin)

    def rope_norm(y, gamma):
        c, s = f[..., 0::2], f[..., 1::2]
        re, im = y[..., 0::2], y[..., 1::2]
        r = np.empty_like(y)
        r[..., 0::2], r[..., 1::2] = re * c - im * s, re * s + im * c
        return r * 8.0 / np.maximum(np.linalg.norm(r, axis=-1, keepdims=True), 1e-12) * gamma

    q = rope_norm(qkv[:, 0], attn.q_norm.gamma.detach().double().cpu().numpy())
    k = rope_norm(qkv[:, 1], attn.k_norm.gamma.detach().double().cpu().numpy())
    v = qkv[:, 2]
    if rows is not None:
        q = q[rows]
    s = np.einsum("qhd,khd->hqk", q, k) / 8.0
    if bias is not None:
        s = s + bias.double().cpu().numpy()[None, None, :]
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = np.einsum("hqk,khd->qhd", p, v).reshape(-1, C)
    return lin(attn.out, o)


def _rel(a, b):
    a = a.double().cpu().numpy().reshape(b.shape)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def test_packed_attention_helpers(cuda):
    import torch
    from tsplat.native_linear_rnf8_patch import apply_triposplat_native_rnf8_avx512_patch
    from tsplat.native_qkv_packed_attention_v3 import (
        apply_triposplat_native_qkv_packed_attention_helpers_patch)

    torch.manual_seed(0)
    model = _toy(torch).to(cuda).eval()
    apply_triposplat_native_rnf8_avx512_patch(model, enabled=True, include_regex=r"attn[.](qkv|out)$",
                                             strict=True, stages=3, residual_mode="nf24_i16")
    calls = []
    stub = types.ModuleType("attention_stub")
    stub._rope_self_attention_standard = lambda *a, **k: calls.append("standard")
    stub._rope_self_attention_with_key_bias = lambda *a, **k: calls.append("key_bias")
    stub._rope_self_attention_selected_rows = lambda *a, **k: calls.append("selected")
    meta = apply_triposplat_native_qkv_packed_attention_helpers_patch(model, attention_module=stub)
    assert meta["selected"] == ["blocks.0.attn", "blocks.1.attn"] and meta["enabled"]

    L, C, H = 150, 128, 2
    x = torch.randn(1, L, C, device=cuda)
    ang = torch.randn(1, L, H, 32, device=cuda)
    rope = torch.polar(torch.ones_like(ang), ang)            # complex64 (cos, sin)
    freqs = torch.view_as_real(rope).reshape(1, L, H, 64)
    attn = model.blocks[0].attn
    with torch.inference_mode():
        y = stub._rope_self_attention_standard(attn, x, rope, backend="native_avx512_exact")
        bias = torch.zeros(L, device=cuda)
        bias[L - 1] = float(np.log(40.0))
        yb = stub._rope_self_attention_with_key_bias(attn, x, rope, bias, backend="native_avx512_exact")
        sel = torch.arange(0, L, 3, device=cuda, dtype=torch.int64)
        ys = stub._rope_self_attention_selected_rows(attn, x, sel, rope, backend="native_avx512_exact",
                                                     compute_dtype="model", query_chunk_size=128)
    torch.cuda.synchronize(cuda)
    assert calls == []
    assert _rel(y, _host_attention(attn, x, freqs)) <= 1e-5
    assert _rel(yb, _host_attention(attn, x, freqs, bias=bias)) <= 1e-5
    assert _rel(ys, _host_attention(attn, x, freqs, rows=sel.cpu().numpy())) <= 1e-5
    rt = meta["runtime"]
    assert rt["calls"] == 3 and rt["key_bias_calls"] == 1 and rt["selected_row_calls"] == 1
    assert rt["fallbacks"] == 0
    # strict: a selected module that cannot run on the packed path raises
    with pytest.raises(RuntimeError, match="fell back"):
        stub._rope_self_attention_standard(attn, x.cpu(), rope.cpu(), backend="native_avx512_exact")
    # other backends go to the original helper
    with pytest.raises(RuntimeError, match="fell back"):
        stub._rope_self_attention_standard(attn, x, rope, backend="default")
    assert rt["fallbacks"] == 2
