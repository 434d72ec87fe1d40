"""Synthetic flow transformer (benchmark configs 4 and 5) on the device.

The upstream TripoSplat model is not available offline, so this module
freezes a graph with the block structure of the reference's unified block
(scripts/triposplat_attention_patch.py:4978-5033: shift-table modulation,
LN -> modulate -> attention -> gated residual -> LN -> modulate -> MLP ->
gated residual; attention as in :4323-4437, RoPE before q/k RMSNorm) and the
literal layer list of config 4: NF24 QKV + self SDPA + NF24 out, cross
attention (NF24 q on the latent, NF24 kv on the condition tokens, NF24 out),
NF24 MLP fc1 / GELU(tanh) / fc2.  Every Linear is an NF24 packed weight run
by the gfx950 GEMM; self attention uses the fused NF24 QKV projection +
RoPE/RMSNorm writing q/k/v [B, H, L, 64] and the exact SDPA on that layout
(it runs ~3 % faster than the packed-K/V kernel of the reference's path).  The elementwise work runs in
the block_ops kernels, fused where the data allows: LayerNorm + modulation
in one pass, GELU in the fc1 epilogue, the gated residuals in the out / fc2
epilogues, the cross-attention residual add in the xout epilogue, the
cross q/k RMSNorm with the [B,H,L,64] permute; CFG and the Euler update are
the sampler kernels.  torch only allocates, copies and stacks.

Frozen choices (not pinned by the reference; recorded here):
  * LayerNorm eps 1e-6; norm1/norm3 without affine, the cross-attention
    norm with affine weight/bias; the final LayerNorm eps 1e-5
    (attention_patch.py:59);
  * cross attention has no RoPE; q and k get the per-head RMSNorm
    y * 8 / max(||y||, 1e-12) * gamma;
  * RoPE: interleaved (cos, sin) pairs, position = latent token index,
    freq_i = theta^(-2i/64), theta = 10000;
  * timestep: t * 1000 -> sinusoidal [cos | sin] (256) -> NF24 Linear
    256->C -> SiLU -> NF24 Linear C->C = t_emb; shared modulation
    t_mod = NF24 Linear(SiLU(t_emb)) [6C]; block mod = t_mod + shift_table;
  * input layer NF24 C->C on the latent; output: final LN, modulation with
    (shift_table_final + t_emb), NF24 C->C = velocity;
  * CFG pair (condition, zero condition) in one batch of 2; guidance 3,
    schedule t_i = s*u/(1 + (s-1)*u), u = linspace(1, 0, steps+1), s = 3
    (scripts/triposplat_quantized_sampler.py:398-414); v = g*v_c - (g-1)*v_u,
    x -= dt * v (scripts/native_sampler_avx512.c:41-49, 78-84).
Weights: W ~ N(0, 0.02), bias ~ N(0, 0.01), gammas 1 + N(0, 0.05), shift
tables N(0, 0.02); Linear i uses torch seed 1000 + i.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

from . import block_ops as bo
from .native_sampler_backend import NativeSamplerBackend
from .native_sdpa_ctypes import native_sdpa_f32_ex
from .nf24 import bf16_planes, nf24_linear, precision_id, quantize_nf24_i16_per_output_channel
from .qkv import gemm_nf24_qkv_direct


@dataclass(frozen=True)
class FlowConfig:
    hidden: int = 1024
    heads: int = 16
    head_dim: int = 64
    mlp_ratio: int = 4
    blocks: int = 28
    latent_tokens: int = 16384
    cond_tokens: int = 2048
    freq_dim: int = 256
    ln_eps: float = 1e-6
    final_ln_eps: float = 1e-5
    rope_theta: float = 10000.0
    guidance: float = 3.0
    shift: float = 3.0
    steps: int = 20
    # camera state width (the single-stream graph's camera token; the
    # reference's cam_out_layer is a 1024 x 5 Linear, the N = 5 tail GEMM)
    cam_channels: int = 5

    def __post_init__(self):
        if self.hidden != self.heads * self.head_dim or self.head_dim != 64:
            raise ValueError("hidden must be heads * 64")


# Linear layout: name -> (in, out) per block, in this order.
BLOCK_LINEARS = (("qkv", 1, 3), ("out", 1, 1), ("xq", 1, 1), ("xkv", 1, 2), ("xout", 1, 1),
                 ("fc1", 1, 4), ("fc2", 4, 1))


class PackedLinear:
    """An NF24-packed Linear on the device (code01_t, q2_t, scale, bias)."""

    def __init__(self, code01_t, q2_t, scale, bias):
        self.code01_t, self.q2_t, self.scale, self.bias = code01_t, q2_t, scale, bias
        self.in_features = int(code01_t.shape[0])
        self.out_features = int(code01_t.shape[1])
        self.precision = "fp32"  # GEMM product precision (tsplat.nf24.PRECISIONS)
        self.planes = None       # bf16 weight planes of self.precision (tsplat.nf24.bf16_planes)

    def set_precision(self, precision, planes=True):
        """Product precision of this Linear; with planes, a bf16 mode reads
        the weights from bf16 planes built here once (same results, 2 or 4
        bytes per weight) instead of decoding the codes in every call."""
        precision_id(precision)
        self.precision = precision
        if precision == "fp32" or not planes:
            self.planes = None
        elif self.planes is None or (self.planes[1] is not None) != (precision == "bf16x3"):
            self.planes = bf16_planes(self.code01_t, self.q2_t, self.scale, precision)

    @classmethod
    def random(cls, torch, in_f, out_f, seed, device):
        g = torch.Generator(device=device).manual_seed(int(seed))
        w = torch.randn((out_f, in_f), generator=g, device=device, dtype=torch.float32) * 0.02
        b = torch.randn((out_f,), generator=g, device=device, dtype=torch.float32) * 0.01
        codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
        return cls(codes[0], codes[1], scales[0], b)

    def __call__(self, x2, out=None, output_start=0, output_count=None):
        return nf24_linear(x2, self.code01_t, self.q2_t, self.scale, self.bias, out=out,
                           output_start=output_start, output_count=output_count, precision=self.precision,
                           planes=self.planes)

    def epilogue(self, x2, kind, out=None, gate=None):
        """This Linear with a fused elementwise epilogue (block_ops.EPILOGUE_*)."""
        return bo.nf24_linear_epilogue(x2, self.code01_t, self.q2_t, self.scale, self.bias, kind,
                                       out=out, gate=gate, precision=self.precision, planes=self.planes)

    def qkv_direct(self, x2, freqs, q_gamma, k_gamma, B, L, H, kv_layout="packed"):
        """Fused QKV projection + RoPE/RMSNorm (tsplat.qkv.gemm_nf24_qkv_direct)."""
        return gemm_nf24_qkv_direct(x2, self.code01_t, self.q2_t, self.scale, self.bias, freqs,
                                    q_gamma, k_gamma, B, L, H, precision=self.precision,
                                    kv_layout=kv_layout, planes=self.planes)

    def host(self):
        return {k: getattr(self, k).cpu().numpy() for k in ("code01_t", "q2_t", "scale", "bias")}


def set_model_precision(model, precision, include=("blocks",), planes=True):
    """Product precision of a flow model ("fp32" strict, or the opt-in
    "bf16" / "bf16x3"): "blocks" in include sets the block Linears, "io" the
    timestep / input / output Linears, "attention" the SDPA products (Q K^T
    and P V); what include does not name stays fp32.  planes: the bf16-mode
    Linears build their bf16 weight planes now (PackedLinear.set_precision)."""
    precision_id(precision)
    for blk in model.blocks:
        for lin in blk.lin.values():
            lin.set_precision(precision if "blocks" in include else "fp32", planes)
    for lin in (model.t_fc1, model.t_fc2, model.adaln, model.input_layer, model.out_layer):
        lin.set_precision(precision if "io" in include else "fp32", planes)
    model.precision = precision if "blocks" in include else "fp32"
    model.attention_precision = precision if "attention" in include else "fp32"
    return model


def _randn(torch, shape, seed, device, std, mean=0.0):
    g = torch.Generator(device=device).manual_seed(int(seed))
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std + mean


class FlowBlock:
    def __init__(self, torch, cfg: FlowConfig, index: int, device, seed_base: int):
        C = cfg.hidden
        self.cfg = cfg
        self.lin = {}
        for j, (name, a, b) in enumerate(BLOCK_LINEARS):
            self.lin[name] = PackedLinear.random(torch, a * C, b * C, seed_base + j, device)
        s = 50000 + 16 * index
        H = cfg.heads
        self.shift_table = _randn(torch, (6 * C,), s, device, 0.02)
        self.q_gamma = _randn(torch, (H, 64), s + 1, device, 0.05, 1.0)
        self.k_gamma = _randn(torch, (H, 64), s + 2, device, 0.05, 1.0)
        self.xq_gamma = _randn(torch, (H, 64), s + 3, device, 0.05, 1.0)
        self.xk_gamma = _randn(torch, (H, 64), s + 4, device, 0.05, 1.0)
        self.xnorm_w = _randn(torch, (C,), s + 5, device, 0.05, 1.0)
        self.xnorm_b = _randn(torch, (C,), s + 6, device, 0.02)

    def host(self):
        out = {name: lin.host() for name, lin in self.lin.items()}
        for k in ("shift_table", "q_gamma", "k_gamma", "xq_gamma", "xk_gamma", "xnorm_w", "xnorm_b"):
            out[k] = getattr(self, k).cpu().numpy()
        return out


def rope_frequencies(torch, L, H, theta, device):
    """[1, L, H, 64] interleaved (cos, sin) of position * theta^(-2i/64)."""
    i = torch.arange(32, dtype=torch.float64, device=device)
    pos = torch.arange(L, dtype=torch.float64, device=device)
    ang = pos[:, None] * theta ** (-2.0 * i / 64.0)[None, :]
    f = torch.stack((torch.cos(ang), torch.sin(ang)), dim=-1).reshape(L, 64).to(torch.float32)
    return f[None, :, None, :].expand(1, L, H, 64).contiguous()


def timestep_embedding(torch, t, dim, device):
    """[cos | sin] of t * exp(-ln(1e4) * i / half), i < half (the reference's
    triposplat_timestep_embedding_f32_avx512 layout: cos first)."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float32, device=device) / half)
    args = t.to(torch.float32)[:, None] * freqs[None, :]
    return torch.cat((torch.cos(args), torch.sin(args)), dim=-1)


class FlowModel:
    """The frozen synthetic flow model; forward() is one CFG-paired velocity."""

    def __init__(self, cfg: FlowConfig, device, blocks: int | None = None):
        import torch

        self.torch = torch
        self.cfg = cfg
        self.device = device
        C = cfg.hidden
        nb = cfg.blocks if blocks is None else blocks
        self.t_fc1 = PackedLinear.random(torch, cfg.freq_dim, C, 1000, device)
        self.t_fc2 = PackedLinear.random(torch, C, C, 1001, device)
        self.adaln = PackedLinear.random(torch, C, 6 * C, 1002, device)
        self.input_layer = PackedLinear.random(torch, C, C, 1003, device)
        self.out_layer = PackedLinear.random(torch, C, C, 1004, device)
        self.final_shift_table = _randn(torch, (2, C), 49999, device, 0.02)
        self.blocks = [FlowBlock(torch, cfg, i, device, 1010 + 10 * i) for i in range(nb)]
        self._freqs = {}
        self.sampler = NativeSamplerBackend()
        self.precision = "fp32"
        self.attention_precision = "fp32"

    def set_precision(self, precision, include=("blocks",), planes=True):
        return set_model_precision(self, precision, include, planes)

    def freqs(self, L):
        if L not in self._freqs:
            self._freqs[L] = rope_frequencies(self.torch, L, self.cfg.heads, self.cfg.rope_theta, self.device)
        return self._freqs[L]

    # -------------------------------------------------------------- pieces
    def timestep(self, t):
        torch = self.torch
        emb = timestep_embedding(torch, t, self.cfg.freq_dim, self.device).contiguous()
        t_emb = self.t_fc2(bo.silu(self.t_fc1(emb)))
        t_mod = self.adaln(bo.silu(t_emb))
        return t_emb, t_mod

    def block_forward(self, blk: FlowBlock, x, cond, t_mod):
        """x [B, L, C] (updated in place and returned), cond [B, Lc, C], t_mod [B, 6C]."""
        cfg = self.cfg
        B, L, C = (int(s) for s in x.shape)
        Lc = int(cond.shape[1])
        H = cfg.heads
        mod = t_mod.clone()  # [B, 6C] = t_mod + shift_table, chunks (shift, scale, gate) x 2
        for b in range(B):
            bo.add_inplace(mod[b], blk.shift_table)
        shift_msa, scale_msa, gate_msa = mod[:, 0:C], mod[:, C:2 * C], mod[:, 2 * C:3 * C]
        shift_mlp, scale_mlp, gate_mlp = mod[:, 3 * C:4 * C], mod[:, 4 * C:5 * C], mod[:, 5 * C:]
        x2 = x.view(B * L, C)
        lin = blk.lin

        # self attention: LN + modulate, fused NF24 QKV + RoPE/RMSNorm into
        # [B, H, L, 64], exact SDPA, NF24 out with the gated residual in its epilogue
        h = bo.layer_norm(x, cfg.ln_eps, scale=scale_msa, shift=shift_msa)
        q, k, v = lin["qkv"].qkv_direct(h.view(B * L, C), self.freqs(L), blk.q_gamma, blk.k_gamma,
                                        B, L, H, kv_layout="bhld")
        a = native_sdpa_f32_ex(q, k, v, out_layout="blhd", precision=self.attention_precision)
        lin["out"].epilogue(a.view(B * L, C), bo.EPILOGUE_GATED, out=x2, gate=gate_msa)

        # cross attention to the condition tokens (no RoPE)
        h = bo.layer_norm(x, cfg.ln_eps, blk.xnorm_w, blk.xnorm_b)
        xq = bo.head_rmsnorm(lin["xq"](h.view(B * L, C)), blk.xq_gamma, B, L, H)
        kv = lin["xkv"](cond.reshape(B * Lc, C))  # [B*Lc, 2C] = [k | v]
        xk = bo.head_rmsnorm(kv, blk.xk_gamma, B, Lc, H, token_stride=2 * C)
        xv = bo.head_rmsnorm(kv[:, C:], None, B, Lc, H, token_stride=2 * C, normalize=False)
        a = native_sdpa_f32_ex(xq, xk, xv, out_layout="blhd", precision=self.attention_precision)
        lin["xout"].epilogue(a.view(B * L, C), bo.EPILOGUE_ADD, out=x2)

        # MLP: LN + modulate, fc1 with GELU, fc2 with the gated residual
        h = bo.layer_norm(x, cfg.ln_eps, scale=scale_mlp, shift=shift_mlp)
        h = lin["fc1"].epilogue(h.view(B * L, C), bo.EPILOGUE_GELU)
        lin["fc2"].epilogue(h, bo.EPILOGUE_GATED, out=x2, gate=gate_mlp)
        return x

    def velocity(self, z, cond, t, observe=None):
        """z [B, L, C], cond [B, Lc, C], t [B] (already x1000) -> v [B, L, C].
        observe(i, x), when given, sees the hidden state x entering block i,
        and observe(len(blocks), x) the state the final layer receives (for
        checks that recompute single blocks elsewhere; x is updated in place
        afterwards, so keep a copy)."""
        torch = self.torch
        B, L, C = (int(s) for s in z.shape)
        t_emb, t_mod = self.timestep(t)
        x = self.input_layer(z.reshape(B * L, C)).view(B, L, C)
        for i, blk in enumerate(self.blocks):
            if observe is not None:
                observe(i, x)
            x = self.block_forward(blk, x, cond, t_mod)
        if observe is not None:
            observe(len(self.blocks), x)
        fs = t_emb[:, None, :].expand(B, 2, C).contiguous()  # [B, (shift, scale), C]
        for b in range(B):
            bo.add_inplace(fs[b], self.final_shift_table)
        h = bo.layer_norm(x, self.cfg.final_ln_eps, scale=fs[:, 1], shift=fs[:, 0])
        return self.out_layer(h.view(B * L, C)).view(B, L, C)

    def schedule(self):
        """t_i = s u / (1 + (s - 1) u), u = 1 - i / steps, in float64
        (scripts/triposplat_quantized_sampler.py:398-400)."""
        s = self.cfg.shift
        u = [1.0 - i / self.cfg.steps for i in range(self.cfg.steps + 1)]
        return [s * x / (1.0 + (s - 1.0) * x) for x in u]

    def euler_cfg_step(self, z, cond, step=0, observe=None):
        """One sampler step with CFG: z [L, C], cond [Lc, C] -> (z_next, v).
        observe: as in velocity(), over the CFG batch of 2."""
        torch = self.torch
        ts = self.schedule()
        t = torch.full((2,), ts[step] * 1000.0, dtype=torch.float32, device=self.device)
        dt = float(ts[step] - ts[step + 1])
        zz = torch.stack((z, z))
        cc = torch.stack((cond, torch.zeros_like(cond)))
        v = self.velocity(zz, cc, t, observe=observe)
        v_cfg, z_next = v[0:1].clone(), z[None].clone()
        g = torch.full((1,), self.cfg.guidance, dtype=torch.float32, device=self.device)
        d = torch.full((1,), dt, dtype=torch.float32, device=self.device)
        self.sampler.cfg_combine_inplace({"x": v_cfg}, {"x": v[1:2]}, g)
        self.sampler.euler_update_inplace({"x": z_next}, {"x": v_cfg}, d)
        return z_next[0], v_cfg[0]

    def host(self):
        """All parameters as NumPy arrays (for the CPU restatement)."""
        return {
            "t_fc1": self.t_fc1.host(), "t_fc2": self.t_fc2.host(), "adaln": self.adaln.host(),
            "input_layer": self.input_layer.host(), "out_layer": self.out_layer.host(),
            "final_shift_table": self.final_shift_table.cpu().numpy(),
            "blocks": [b.host() for b in self.blocks],
        }
