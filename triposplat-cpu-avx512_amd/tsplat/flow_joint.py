"""Single-stream flow graph with the reference's exactness-preserving work
reduction: negative-branch log(M) key compression and the selected-rows
final block.

The reference's model attends over one joint sequence [latent ; condition]
(scripts/triposplat_attention_patch.py:4978-5033 block order).  Two
reductions keep its outputs while doing less work:

* negative-branch compression (attention_patch.py:5446-5628,
  ``_cached_key_bias``): the CFG negative branch feeds M identical
  (zero) condition rows.  Identical rows stay identical through every block,
  so the branch carries ONE representative condition row and the SDPA adds
  log(M) to that key's score: exp(s + log M) = M exp(s), i.e. M identical
  keys.  Here the negative sequence is L + 1 tokens instead of L + M.
* selected-rows final block (attention_patch.py:5349-5443): only latent rows
  leave the model, so the last block computes queries, attention output,
  residuals and MLP for the L latent rows only, while K/V still cover every
  row (triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2).

Frozen choices (the upstream model is absent): the latent tokens get RoPE at
positions 0..L-1 (theta 1e4), condition tokens the identity rotation (so
identical condition rows have identical keys, which the compression
requires); the block is LN -> modulate -> fused NF24 QKV (RoPE, RMSNorm) ->
packed exact SDPA over all tokens -> NF24 out + gated residual -> LN ->
modulate -> NF24 fc1 + GELU -> NF24 fc2 + gated residual; timestep path,
final layer, schedule and CFG as tsplat.flow.  Linear seeds 3000 + 10 i + j.
Batch 1 per branch (the two CFG branches have different lengths).
"""
from __future__ import annotations

import math

from . import block_ops as bo
from .flow import FlowConfig, PackedLinear, _randn, set_model_precision, timestep_embedding
from .native_sampler_backend import NativeSamplerBackend
from .native_sdpa_ctypes import native_sdpa_f32_ex
from .qkv import q_kv_selected_rope_rmsnorm_pack

JOINT_LINEARS = (("qkv", 1, 3), ("out", 1, 1), ("fc1", 1, 4), ("fc2", 4, 1))


class JointBlock:
    def __init__(self, torch, cfg: FlowConfig, index: int, device):
        C, H = cfg.hidden, cfg.heads
        self.lin = {name: PackedLinear.random(torch, a * C, b * C, 3000 + 10 * index + j, device)
                    for j, (name, a, b) in enumerate(JOINT_LINEARS)}
        s = 60000 + 16 * index
        self.shift_table = _randn(torch, (6 * C,), s, device, 0.02)
        self.q_gamma = _randn(torch, (H, 64), s + 1, device, 0.05, 1.0)
        self.k_gamma = _randn(torch, (H, 64), s + 2, device, 0.05, 1.0)

    def host(self):
        out = {name: lin.host() for name, lin in self.lin.items()}
        for k in ("shift_table", "q_gamma", "k_gamma"):
            out[k] = getattr(self, k).cpu().numpy()
        return out


def joint_frequencies(torch, L, Lc, H, theta, device):
    """[1, L + Lc, H, 64]: latent rows rotated by position, condition rows (1, 0)."""
    i = torch.arange(32, dtype=torch.float64, device=device)
    ang = torch.arange(L, dtype=torch.float64, device=device)[:, None] * theta ** (-2.0 * i / 64.0)[None, :]
    lat = torch.stack((torch.cos(ang), torch.sin(ang)), dim=-1).reshape(L, 64)
    ident = torch.zeros((Lc, 32, 2), dtype=torch.float64, device=device)
    ident[..., 0] = 1.0
    f = torch.cat((lat, ident.reshape(Lc, 64)), 0).to(torch.float32)
    return f[None, :, None, :].expand(1, L + Lc, H, 64).contiguous()


class JointFlowModel:
    """Single-stream synthetic flow model (batch 1 per call)."""

    def __init__(self, cfg: FlowConfig, device, blocks: int | None = None):
        import torch

        self.torch, self.cfg, self.device = torch, cfg, device
        C = cfg.hidden
        nb = cfg.blocks if blocks is None else blocks
        self.t_fc1 = PackedLinear.random(torch, cfg.freq_dim, C, 2000, device)
        self.t_fc2 = PackedLinear.random(torch, C, C, 2001, device)
        self.adaln = PackedLinear.random(torch, C, 6 * C, 2002, device)
        self.input_layer = PackedLinear.random(torch, C, C, 2003, device)
        self.out_layer = PackedLinear.random(torch, C, C, 2004, device)
        self.final_shift_table = _randn(torch, (2, C), 59999, device, 0.02)
        self.blocks = [JointBlock(torch, cfg, i, device) for i in range(nb)]
        self.sampler = NativeSamplerBackend()
        self._freqs, self._sel, self._bias = {}, {}, {}
        self.precision = "fp32"
        self.attention_precision = "fp32"

    def set_precision(self, precision, include=("blocks",)):
        return set_model_precision(self, precision, include)

    def freqs(self, L, Lc):
        if (L, Lc) not in self._freqs:
            self._freqs[(L, Lc)] = joint_frequencies(self.torch, L, Lc, self.cfg.heads,
                                                     self.cfg.rope_theta, self.device)
        return self._freqs[(L, Lc)]

    def selected(self, L):
        if L not in self._sel:
            self._sel[L] = self.torch.arange(L, dtype=self.torch.int64, device=self.device)
        return self._sel[L]

    def key_bias(self, L, multiplicity):
        """[L + 1]: zeros, log(M) at the representative condition key L
        (the reference's _cached_key_bias, attention_patch.py:5618-5628)."""
        key = (L, multiplicity)
        if key not in self._bias:
            b = self.torch.zeros(L + 1, dtype=self.torch.float32, device=self.device)
            b[L] = math.log(float(multiplicity))
            self._bias[key] = b
        return self._bias[key]

    def timestep(self, t):
        emb = timestep_embedding(self.torch, t, self.cfg.freq_dim, self.device).contiguous()
        t_emb = self.t_fc2(bo.silu(self.t_fc1(emb)))
        return t_emb, self.adaln(bo.silu(t_emb))

    def _mod(self, blk, t_mod):
        mod = t_mod.clone()
        bo.add_inplace(mod[0], blk.shift_table)
        C = self.cfg.hidden
        return [mod[:, i * C:(i + 1) * C] for i in range(6)]  # shift, scale, gate (msa), (mlp)

    def block_forward(self, blk, x, t_mod, L, key_bias=None):
        """x [1, Ltot, C] (all rows updated in place)."""
        cfg = self.cfg
        _, Ltot, C = (int(s) for s in x.shape)
        H = cfg.heads
        sm, cm, gm, s2, c2, g2 = self._mod(blk, t_mod)
        lin = blk.lin
        h = bo.layer_norm(x, cfg.ln_eps, scale=cm, shift=sm)
        q, k, v = lin["qkv"].qkv_direct(h.view(Ltot, C), self.freqs(L, Ltot - L), blk.q_gamma,
                                        blk.k_gamma, 1, Ltot, H, kv_layout="bhld")
        a = native_sdpa_f32_ex(q, k, v, key_bias=key_bias, out_layout="blhd",
                               precision=self.attention_precision)
        x2 = x.view(Ltot, C)
        lin["out"].epilogue(a.view(Ltot, C), bo.EPILOGUE_GATED, out=x2, gate=gm)
        h = bo.layer_norm(x, cfg.ln_eps, scale=c2, shift=s2)
        h = lin["fc1"].epilogue(h.view(Ltot, C), bo.EPILOGUE_GELU)
        lin["fc2"].epilogue(h, bo.EPILOGUE_GATED, out=x2, gate=g2)
        return x

    def block_forward_selected(self, blk, x, t_mod, L, key_bias=None):
        """Final block, latent rows only: returns x_lat [1, L, C].  K/V cover all
        Ltot rows; Q, attention output, residuals and MLP only the first L."""
        torch, cfg = self.torch, self.cfg
        _, Ltot, C = (int(s) for s in x.shape)
        H = cfg.heads
        sm, cm, gm, s2, c2, g2 = self._mod(blk, t_mod)
        lin = blk.lin["qkv"]
        h = bo.layer_norm(x, cfg.ln_eps, scale=cm, shift=sm).view(Ltot, C)
        q = lin(h[:L], output_start=0, output_count=C)
        kv = lin(h, output_start=C, output_count=2 * C)
        qo, pk, pv = q_kv_selected_rope_rmsnorm_pack(q, kv, self.freqs(L, Ltot - L), self.selected(L),
                                                     blk.q_gamma, blk.k_gamma, 1, L, Ltot, H)
        a = native_sdpa_f32_ex(qo, pk, pv, kv_packed=True, key_count=Ltot, key_bias=key_bias,
                               out_layout="blhd", precision=self.attention_precision)
        x_lat = x[:, :L].contiguous()
        x2 = x_lat.view(L, C)
        blk.lin["out"].epilogue(a.view(L, C), bo.EPILOGUE_GATED, out=x2, gate=gm)
        h = bo.layer_norm(x_lat, cfg.ln_eps, scale=c2, shift=s2)
        h = blk.lin["fc1"].epilogue(h.view(L, C), bo.EPILOGUE_GELU)
        blk.lin["fc2"].epilogue(h, bo.EPILOGUE_GATED, out=x2, gate=g2)
        return x_lat

    def velocity(self, z, cond, t, *, compress=False, selected_final=True):
        """z [L, C], cond [Lc, C], t [1] -> v [L, C].  compress=True treats the
        Lc condition rows as identical and carries one row with a log(Lc) key
        bias (valid only when they are identical: the CFG negative branch)."""
        torch = self.torch
        L, C = (int(s) for s in z.shape)
        Lc = int(cond.shape[0])
        t_emb, t_mod = self.timestep(t)
        rows = cond[:1] if compress else cond
        bias = self.key_bias(L, Lc) if compress else None
        x = torch.cat((self.input_layer(z).view(L, C), rows), 0)[None].contiguous()
        last = len(self.blocks) - 1
        for i, blk in enumerate(self.blocks):
            if i == last and selected_final:
                x = self.block_forward_selected(blk, x, t_mod, L, bias)
            else:
                x = self.block_forward(blk, x, t_mod, L, bias)
        x = x[:, :L].contiguous()
        fs = t_emb[:, None, :].expand(1, 2, C).contiguous()
        bo.add_inplace(fs[0], self.final_shift_table)
        h = bo.layer_norm(x, self.cfg.final_ln_eps, scale=fs[:, 1], shift=fs[:, 0])
        return self.out_layer(h.view(L, C))

    def schedule(self):
        s = self.cfg.shift
        u = [1.0 - i / self.cfg.steps for i in range(self.cfg.steps + 1)]
        return [s * x / (1.0 + (s - 1.0) * x) for x in u]

    def euler_cfg_step(self, z, cond, step=0, *, reduce_work=True):
        """One CFG Euler step; with reduce_work the negative branch is
        compressed and both branches use the selected final block."""
        torch = self.torch
        ts = self.schedule()
        t = torch.full((1,), ts[step] * 1000.0, dtype=torch.float32, device=self.device)
        dt = float(ts[step] - ts[step + 1])
        v_pos = self.velocity(z, cond, t, selected_final=reduce_work)
        v_neg = self.velocity(z, torch.zeros_like(cond), t, compress=reduce_work,
                              selected_final=reduce_work)
        v_cfg, z_next = v_pos[None].clone(), z[None].clone()
        g = torch.full((1,), self.cfg.guidance, dtype=torch.float32, device=self.device)
        d = torch.full((1,), dt, dtype=torch.float32, device=self.device)
        self.sampler.cfg_combine_inplace({"x": v_cfg}, {"x": v_neg[None].contiguous()}, g)
        self.sampler.euler_update_inplace({"x": z_next}, {"x": v_cfg}, d)
        return z_next[0], v_cfg[0]

    def host(self):
        return {
            "t_fc1": self.t_fc1.host(), "t_fc2": self.t_fc2.host(), "adaln": self.adaln.host(),
            "input_layer": self.input_layer.host(), "out_layer": self.out_layer.host(),
            "final_shift_table": self.final_shift_table.cpu().numpy(),
            "blocks": [b.host() for b in self.blocks],
        }
