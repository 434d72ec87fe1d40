"""Single-stream flow graph with the reference's exactness-preserving work
reduction: negative-branch log(M) key compression and the selected-rows
final block.

The reference's model attends over one joint sequence [latent ; condition ;
camera] (scripts/triposplat_attention_patch.py:4978-5033 block order; the
sequence and the two output heads: :948-971).  Two reductions keep its
outputs while doing less work:

* negative-branch compression (attention_patch.py:5446-5628,
  ``_cached_key_bias``): the CFG negative branch feeds M identical
  (zero) condition rows.  Identical rows stay identical through every block,
  so the branch carries ONE representative condition row and the SDPA adds
  log(M) to that key's score: exp(s + log M) = M exp(s), i.e. M identical
  keys.  Here the negative sequence is L + 1 tokens instead of L + M.
* selected-rows final block (attention_patch.py:5349-5443): only the latent
  and camera rows leave the model, so the last block computes queries,
  attention output, residuals and MLP for those L + 1 rows only, while K/V
  still cover every row (triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2).

Frozen choices (the upstream model is absent): the latent tokens get RoPE at
positions 0..L-1 (theta 1e4), condition tokens and the camera token the
identity rotation (so identical condition rows have identical keys, which the
compression requires); the camera state [1, cam_channels] enters through an
NF24 Linear (cam_channels -> C, the reference's cam_refiner) and leaves
through the final LN + modulation and an NF24 Linear C -> cam_channels (its
cam_out_layer: with cam_channels = 5 the odd-width tail GEMM); the block is
LN -> modulate -> fused NF24 QKV (RoPE, RMSNorm) ->
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


def camera_state(cfg: FlowConfig, seed: int):
    """A seeded camera state [1, cam_channels] ~ N(0, 1) (NumPy PCG64)."""
    import numpy as np

    return np.random.default_rng(seed).standard_normal((1, cfg.cam_channels), dtype=np.float32)


def joint_frequencies(torch, L, Lc, H, theta, device):
    """[1, L + Lc, H, 64]: latent rows rotated by position, the Lc condition
    and camera rows (1, 0)."""
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
        self.cam_refiner = PackedLinear.random(torch, cfg.cam_channels, C, 2005, device)
        self.cam_out_layer = PackedLinear.random(torch, C, cfg.cam_channels, 2006, device)
        self.final_shift_table = _randn(torch, (2, C), 59999, device, 0.02)
        self.blocks = [JointBlock(torch, cfg, i, device) for i in range(nb)]
        self.sampler = NativeSamplerBackend()
        self._freqs, self._sel, self._bias = {}, {}, {}
        self.precision = "fp32"
        self.attention_precision = "fp32"

    def set_precision(self, precision, include=("blocks",), planes=True):
        return set_model_precision(self, precision, include, planes)

    def freqs(self, L, Lc):
        if (L, Lc) not in self._freqs:
            self._freqs[(L, Lc)] = joint_frequencies(self.torch, L, Lc, self.cfg.heads,
                                                     self.cfg.rope_theta, self.device)
        return self._freqs[(L, Lc)]

    def selected(self, L, Ltot):
        """Rows of the final block's queries: the latent rows and the camera row."""
        if (L, Ltot) not in self._sel:
            torch = self.torch
            self._sel[(L, Ltot)] = torch.cat((torch.arange(L, dtype=torch.int64, device=self.device),
                                              torch.tensor([Ltot - 1], dtype=torch.int64, device=self.device)))
        return self._sel[(L, Ltot)]

    def key_bias(self, L, multiplicity):
        """[L + 2]: zeros, log(M) at the representative condition key L, 0 for
        the camera key (the reference's _cached_key_bias, attention_patch.py:5618-5628)."""
        key = (L, multiplicity)
        if key not in self._bias:
            b = self.torch.zeros(L + 2, dtype=self.torch.float32, device=self.device)
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
        """Final block, latent and camera rows only: returns [1, L + 1, C] (the L
        latent rows, then the camera row).  K/V cover all Ltot rows; Q,
        attention output, residuals and MLP only the selected rows."""
        torch, cfg = self.torch, self.cfg
        _, Ltot, C = (int(s) for s in x.shape)
        H = cfg.heads
        Lq = L + 1
        sm, cm, gm, s2, c2, g2 = self._mod(blk, t_mod)
        lin = blk.lin["qkv"]
        h = bo.layer_norm(x, cfg.ln_eps, scale=cm, shift=sm).view(Ltot, C)
        q = lin(torch.cat((h[:L], h[Ltot - 1:]), 0), output_start=0, output_count=C)
        kv = lin(h, output_start=C, output_count=2 * C)
        qo, pk, pv = q_kv_selected_rope_rmsnorm_pack(q, kv, self.freqs(L, Ltot - L), self.selected(L, Ltot),
                                                     blk.q_gamma, blk.k_gamma, 1, Lq, Ltot, H)
        a = native_sdpa_f32_ex(qo, pk, pv, kv_packed=True, key_count=Ltot, key_bias=key_bias,
                               out_layout="blhd", precision=self.attention_precision)
        x_sel = torch.cat((x[:, :L], x[:, Ltot - 1:]), 1).contiguous()
        x2 = x_sel.view(Lq, C)
        blk.lin["out"].epilogue(a.view(Lq, C), bo.EPILOGUE_GATED, out=x2, gate=gm)
        h = bo.layer_norm(x_sel, cfg.ln_eps, scale=c2, shift=s2)
        h = blk.lin["fc1"].epilogue(h.view(Lq, C), bo.EPILOGUE_GELU)
        blk.lin["fc2"].epilogue(h, bo.EPILOGUE_GATED, out=x2, gate=g2)
        return x_sel

    def velocity(self, z, cond, cam, t, *, compress=False, selected_final=True):
        """z [L, C], cond [Lc, C], cam [1, cam_channels], t [1] -> (v [L, C],
        v_cam [1, cam_channels]).  compress=True treats the Lc condition rows as
        identical and carries one row with a log(Lc) key bias (valid only when
        they are identical: the CFG negative branch)."""
        torch = self.torch
        L, C = (int(s) for s in z.shape)
        Lc = int(cond.shape[0])
        t_emb, t_mod = self.timestep(t)
        rows = cond[:1] if compress else cond
        bias = self.key_bias(L, Lc) if compress else None
        x = torch.cat((self.input_layer(z).view(L, C), rows, self.cam_refiner(cam).view(1, C)),
                      0)[None].contiguous()
        last = len(self.blocks) - 1
        for i, blk in enumerate(self.blocks):
            if i == last and selected_final:
                x = self.block_forward_selected(blk, x, t_mod, L, bias)
            else:
                x = self.block_forward(blk, x, t_mod, L, bias)
        if not (selected_final and self.blocks):
            x = torch.cat((x[:, :L], x[:, -1:]), 1).contiguous()
        fs = t_emb[:, None, :].expand(1, 2, C).contiguous()
        bo.add_inplace(fs[0], self.final_shift_table)
        h = bo.layer_norm(x, self.cfg.final_ln_eps, scale=fs[:, 1], shift=fs[:, 0]).view(L + 1, C)
        return self.out_layer(h[:L]), self.cam_out_layer(h[L:])

    def schedule(self):
        s = self.cfg.shift
        u = [1.0 - i / self.cfg.steps for i in range(self.cfg.steps + 1)]
        return [s * x / (1.0 + (s - 1.0) * x) for x in u]

    def euler_cfg_step(self, z, cond, cam, step=0, *, reduce_work=True):
        """One CFG Euler step of the latent and the camera state:
        (z_next, v_cfg, cam_next, v_cam_cfg).  With reduce_work the negative
        branch is compressed and both branches use the selected final block."""
        torch = self.torch
        ts = self.schedule()
        t = torch.full((1,), ts[step] * 1000.0, dtype=torch.float32, device=self.device)
        dt = float(ts[step] - ts[step + 1])
        v_pos, vc_pos = self.velocity(z, cond, cam, t, selected_final=reduce_work)
        v_neg, vc_neg = self.velocity(z, torch.zeros_like(cond), cam, t, compress=reduce_work,
                                      selected_final=reduce_work)
        g = torch.full((1,), self.cfg.guidance, dtype=torch.float32, device=self.device)
        d = torch.full((1,), dt, dtype=torch.float32, device=self.device)
        out = []
        for vp, vn, state in ((v_pos, v_neg, z), (vc_pos, vc_neg, cam)):
            v_cfg, nxt = vp[None].clone(), state[None].clone()
            self.sampler.cfg_combine_inplace({"x": v_cfg}, {"x": vn[None].contiguous()}, g)
            self.sampler.euler_update_inplace({"x": nxt}, {"x": v_cfg}, d)
            out += [nxt[0], v_cfg[0]]
        return tuple(out)

    def host(self):
        return {
            "t_fc1": self.t_fc1.host(), "t_fc2": self.t_fc2.host(), "adaln": self.adaln.host(),
            "input_layer": self.input_layer.host(), "out_layer": self.out_layer.host(),
            "cam_refiner": self.cam_refiner.host(), "cam_out_layer": self.cam_out_layer.host(),
            "final_shift_table": self.final_shift_table.cpu().numpy(),
            "blocks": [b.host() for b in self.blocks],
        }
