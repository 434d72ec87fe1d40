"""CPU fp32 restatement of the synthetic flow model (benchmark configs 4 and 5).

TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg).  The graph
is the one frozen in triposplat-cpu-avx512_amd/tsplat/flow.py; here every
NF24 Linear, the fused QKV projection and both SDPAs run through the CPU
kernels -- the oracle restatement (`backend="oracle"`) or the reference's own
AVX-512 build in oracle/_ref (`backend="reference"`: its NF24 GEMM,
QKV-direct and SDPA kernels and its LayerNorm / modulate / gated-residual /
GELU / SiLU / RMSNorm / CFG / Euler kernels, i.e. the repository's CPU
pipeline).  The elementwise restatements are bit-identical to the reference
kernels, so the two backends differ only where the GEMM / SDPA do.  Parameters come from
FlowModel.host(), so both sides use bit-identical packed weights.

Model-level parity is "unpinned at the upstream boundary": the upstream
TripoSplat model is absent; this restatement is checked against the device
graph, not against the real model.
"""
from __future__ import annotations

import math

import numpy as np

import oracle as O


class CpuFlow:
    def __init__(self, params, cfg, backend="oracle", threads=0):
        self.p = params
        self.cfg = cfg
        self.backend = backend
        self.threads = threads
        self.progress = None  # optional callable(block index) after each block
        # optional callable(i, x): the hidden state entering block i, and
        # (len(blocks), x) the state the final layer receives
        self.observe = None
        if backend == "reference" and not O.ref_available():
            raise RuntimeError("oracle/_ref not built")

    # ---------------------------------------------------------- kernels
    def linear(self, x2, lin):
        x2 = np.ascontiguousarray(x2, np.float32)
        if self.backend == "reference" and lin["code01_t"].shape[1] % 16 == 0:
            return O.ref_nf24_gemm(x2, lin["code01_t"], lin["q2_t"], lin["scale"], lin["bias"], self.threads)
        return O.nf24_gemm(x2, lin["code01_t"], lin["q2_t"], lin["scale"], lin["bias"])

    def qkv_direct(self, x2, lin, freqs, qg, kg, B, L, H):
        if self.backend == "reference":
            return O.ref_gemm_nf24_qkv_direct(x2, lin["code01_t"], lin["q2_t"], lin["scale"], lin["bias"],
                                              freqs, qg, kg, B, L, H, self.threads)
        return O.gemm_nf24_qkv_direct(x2, lin["code01_t"], lin["q2_t"], lin["scale"], lin["bias"],
                                      freqs, qg, kg, B, L, H)

    def sdpa_packed_blhd(self, q, pk, pv, Lk):
        if self.backend == "reference":
            return O.ref_sdpa_packed_blhd(q, pk, pv, Lk, None, self.threads)
        return O.sdpa_q8t512_packed_blhd(q, pk, pv, Lk)

    def sdpa_bhld(self, q, k, v):
        if self.backend == "reference":
            return O.ref_sdpa_q8t512(q, k, v, None, self.threads)
        return O.sdpa_q8t512(q, k, v)

    # ---------------------------------------------------------- elementwise
    # LayerNorm / modulate / gated residual / add / GELU / SiLU / RMSNorm and
    # the sampler updates: the oracle's C restatements (backend "oracle") or
    # the reference's AVX-512 build (backend "reference") -- bit-identical.
    def _ew(self, op, *args):
        st = O.ew(op, *args, backend=self.backend, threads=self.threads)
        if st != 0:
            raise RuntimeError(f"{op} status {st}")

    def freqs(self, L):
        H = self.cfg.heads
        i = np.arange(32, dtype=np.float64)
        ang = np.arange(L, dtype=np.float64)[:, None] * self.cfg.rope_theta ** (-2.0 * i / 64.0)[None, :]
        f = np.stack((np.cos(ang), np.sin(ang)), -1).reshape(L, 64).astype(np.float32)
        return np.ascontiguousarray(np.broadcast_to(f[None, :, None, :], (1, L, H, 64)))

    def timestep(self, t):
        half = self.cfg.freq_dim // 2
        freqs = np.exp(-math.log(10000.0) * np.arange(half, dtype=np.float32) / np.float32(half)).astype(np.float32)
        args = (np.asarray(t, np.float32)[:, None] * freqs[None, :]).astype(np.float32)
        emb = np.concatenate((np.cos(args), np.sin(args)), -1).astype(np.float32)
        t_emb = self.linear(self._silu(self.linear(emb, self.p["t_fc1"])), self.p["t_fc2"])
        t_mod = self.linear(self._silu(t_emb), self.p["adaln"])
        return t_emb, t_mod

    # ---------------------------------------------------------- graph
    def _ln(self, x, eps, w=None, b=None):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        cols = x.shape[-1]
        self._ew("layernorm", x, None if w is None else np.ascontiguousarray(w, np.float32),
                 None if b is None else np.ascontiguousarray(b, np.float32), out, x.size // cols, cols,
                 np.float32(eps), int(w is not None))
        return out

    def _modulate(self, h, scale, shift):
        B, L, C = h.shape
        self._ew("modulate_inplace", h, np.ascontiguousarray(scale), np.ascontiguousarray(shift), B, L, C)
        return h

    def _gated(self, x, h, gate):
        B, L, C = x.shape
        self._ew("gated_residual_inplace", x, np.ascontiguousarray(h, np.float32),
                 np.ascontiguousarray(gate), B, L, C)
        return x

    def _add(self, x, d):
        self._ew("add_inplace", x, np.ascontiguousarray(d, np.float32), x.size)
        return x

    def _gelu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._ew("gelu_tanh", x, out, x.size)
        return out

    def _silu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._ew("silu", x, out, x.size)
        return out

    def _rmsnorm(self, y, gamma):
        y = np.ascontiguousarray(y, np.float32)
        out = np.empty_like(y)
        H, D = gamma.shape
        self._ew("multihead_rmsnorm", y, np.ascontiguousarray(gamma), out, y.size // (H * D), H, D,
                 np.float32(1e-12))
        return out

    def block(self, bp, x, cond, t_mod):
        cfg = self.cfg
        B, L, C = x.shape
        Lc = cond.shape[1]
        H = cfg.heads
        x = np.array(x, dtype=np.float32, copy=True)
        mod = (t_mod + bp["shift_table"]).astype(np.float32)
        sm, cm, gm, s2, c2, g2 = (np.ascontiguousarray(a) for a in np.split(mod, 6, axis=-1))
        h = self._modulate(self._ln(x, cfg.ln_eps), cm, sm)
        q, pk, pv = self.qkv_direct(h.reshape(B * L, C), bp["qkv"], self.freqs(L), bp["q_gamma"],
                                    bp["k_gamma"], B, L, H)
        a = self.sdpa_packed_blhd(q, pk, pv, L).reshape(B * L, C)
        x = self._gated(x, self.linear(a, bp["out"]).reshape(B, L, C), gm)
        h = self._ln(x, cfg.ln_eps, bp["xnorm_w"], bp["xnorm_b"])
        xq = self._rmsnorm(self.linear(h.reshape(B * L, C), bp["xq"]).reshape(B, L, H, 64), bp["xq_gamma"])
        kv = self.linear(cond.reshape(B * Lc, C), bp["xkv"]).reshape(B, Lc, 2, H, 64)
        xk = self._rmsnorm(np.ascontiguousarray(kv[:, :, 0]), bp["xk_gamma"])
        xv = kv[:, :, 1]
        a = self.sdpa_bhld(np.ascontiguousarray(xq.transpose(0, 2, 1, 3)), np.ascontiguousarray(xk.transpose(0, 2, 1, 3)),
                           np.ascontiguousarray(xv.transpose(0, 2, 1, 3)))
        a = np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(B * L, C)
        x = self._add(x, self.linear(a, bp["xout"]).reshape(B, L, C))
        h = self._modulate(self._ln(x, cfg.ln_eps), c2, s2)
        h = self._gelu(self.linear(h.reshape(B * L, C), bp["fc1"]))
        h = self.linear(h, bp["fc2"]).reshape(B, L, C)
        return self._gated(x, h, g2)

    def velocity(self, z, cond, t):
        B, L, C = z.shape
        t_emb, t_mod = self.timestep(t)
        x = self.linear(z.reshape(B * L, C), self.p["input_layer"]).reshape(B, L, C)
        for i, bp in enumerate(self.p["blocks"]):
            if self.observe is not None:
                self.observe(i, x)
            x = self.block(bp, x, cond, t_mod)
            if self.progress is not None:
                self.progress(i)
        if self.observe is not None:
            self.observe(len(self.p["blocks"]), x)
        return self.final_layer(x, t_emb)

    def final_layer(self, x, t_emb):
        """Final LayerNorm, modulation by (shift table + t_emb), output Linear:
        the hidden state after the last block [B, L, C] -> velocity."""
        B, L, C = x.shape
        fs = (self.p["final_shift_table"][None] + t_emb[:, None, :]).astype(np.float32)
        shift, scale = np.ascontiguousarray(fs[:, 0]), np.ascontiguousarray(fs[:, 1])
        h = self._modulate(self._ln(x, self.cfg.final_ln_eps), scale, shift)
        return self.linear(h.reshape(B * L, C), self.p["out_layer"]).reshape(B, L, C)

    def schedule(self):
        """t_i = s u / (1 + (s - 1) u), u = linspace(1, 0, steps + 1) in float64
        (scripts/triposplat_quantized_sampler.py:398-400)."""
        s = self.cfg.shift
        u = np.linspace(1.0, 0.0, self.cfg.steps + 1, dtype=np.float64)
        return s * u / (1.0 + (s - 1.0) * u)

    def step_times(self, step=0):
        """(t * 1000, dt) of a step as the sampler passes them: float32 of the
        float64 schedule values (sampler.py:413-414)."""
        ts = self.schedule()
        return np.float32(ts[step] * 1000.0), np.float32(ts[step] - ts[step + 1])

    def cfg_euler(self, v_pos, v_neg, z, dt):
        """v = g v_c - (g - 1) v_u, z - dt v (native_sampler_avx512.c:41-49,
        78-84): (z_next, v_cfg)."""
        v_cfg = np.array(v_pos, np.float32, copy=True)
        self._ew("cfg_combine_inplace", v_cfg, np.ascontiguousarray(v_neg, np.float32),
                 np.array([self.cfg.guidance], np.float32), 1, v_cfg.size)
        z_next = np.array(z, np.float32, copy=True)
        self._ew("euler_update_inplace", z_next, v_cfg, np.array([dt], np.float32), 1, z_next.size)
        return z_next, v_cfg

    def euler_cfg_step(self, z, cond, step=0):
        t1000, dt = self.step_times(step)
        t = np.full(2, t1000, np.float32)
        v = self.velocity(np.stack((z, z)), np.stack((cond, np.zeros_like(cond))), t)
        return self.cfg_euler(v[0], v[1], z, dt)


def combined_rmse(a, b):
    """RMSE as scripts/compare_latent_npz.py:22-48 reports it (float64)."""
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    return float(np.sqrt(np.mean(d * d)))


def latent_stats(ref, cand):
    """The per-key statistics of scripts/compare_latent_npz.py:22-48 (float64):
    RMSE, MAE, max-abs, mean relative error against max(|ref|, 1e-8), the
    50/95/99th percentiles of |diff|, and the finite / NaN / +Inf / -Inf counts
    of the difference."""
    ref = np.asarray(ref, np.float64)
    d = np.asarray(cand, np.float64) - ref
    ad = np.abs(d)
    mse = float(np.mean(d * d))
    with np.errstate(invalid="ignore"):  # non-finite differences are counted below
        p50, p95, p99 = (float(np.percentile(ad, q)) for q in (50, 95, 99))
    return {
        "mse": mse,
        "rmse": float(np.sqrt(mse)),
        "mae": float(np.mean(ad)),
        "max_abs": float(np.max(ad)),
        "mean_relative_abs": float(np.mean(ad / np.maximum(np.abs(ref), 1e-8))),
        "p50_abs": p50,
        "p95_abs": p95,
        "p99_abs": p99,
        "finite_count": int(np.isfinite(d).sum()),
        "nan_count": int(np.isnan(d).sum()),
        "posinf_count": int(np.isposinf(d).sum()),
        "neginf_count": int(np.isneginf(d).sum()),
    }


def combined_rmse_from_key_mse(per_key):
    """sqrt of the mean of the per-key MSEs (compare_latent_npz.py:67-71):
    the score that combines e.g. the latent and the camera keys."""
    mses = [v["mse"] for v in per_key.values()]
    return float(np.sqrt(np.mean(mses)))


def non_finite(stats):
    """NaN + Inf count of a latent_stats() record (the reference's promotion
    gates require 0 beside the RMSE)."""
    return stats["nan_count"] + stats["posinf_count"] + stats["neginf_count"]


class CpuJointFlow(CpuFlow):
    """CPU restatement of tsplat/flow_joint.py's single-stream graph, computed
    the long way: the full negative sequence (all condition rows, no key
    bias) and the full final block, batch 1 per branch."""

    def joint_freqs(self, L, Lc):
        H = self.cfg.heads
        i = np.arange(32, dtype=np.float64)
        ang = np.arange(L, dtype=np.float64)[:, None] * self.cfg.rope_theta ** (-2.0 * i / 64.0)[None, :]
        lat = np.stack((np.cos(ang), np.sin(ang)), -1).reshape(L, 64)
        ident = np.zeros((Lc, 32, 2))
        ident[..., 0] = 1.0
        f = np.concatenate((lat, ident.reshape(Lc, 64)), 0).astype(np.float32)
        return np.ascontiguousarray(np.broadcast_to(f[None, :, None, :], (1, L + Lc, H, 64)))

    def joint_block(self, bp, x, t_mod, L):
        cfg = self.cfg
        _, Lt, C = x.shape
        H = cfg.heads
        x = np.array(x, dtype=np.float32, copy=True)
        mod = (t_mod + bp["shift_table"]).astype(np.float32)
        sm, cm, gm, s2, c2, g2 = (np.ascontiguousarray(a) for a in np.split(mod, 6, axis=-1))
        h = self._modulate(self._ln(x, cfg.ln_eps), cm, sm)
        q, pk, pv = self.qkv_direct(h.reshape(Lt, C), bp["qkv"], self.joint_freqs(L, Lt - L),
                                    bp["q_gamma"], bp["k_gamma"], 1, Lt, H)
        a = self.sdpa_packed_blhd(q, pk, pv, Lt).reshape(Lt, C)
        x = self._gated(x, self.linear(a, bp["out"]).reshape(1, Lt, C), gm)
        h = self._modulate(self._ln(x, cfg.ln_eps), c2, s2)
        h = self._gelu(self.linear(h.reshape(Lt, C), bp["fc1"]))
        return self._gated(x, self.linear(h, bp["fc2"]).reshape(1, Lt, C), g2)

    def joint_velocity(self, z, cond, cam, t):
        """(v [L, C], v_cam [1, cam_channels]) over the sequence
        [latent ; condition ; camera]."""
        L, C = z.shape
        t_emb, t_mod = self.timestep(t)
        x = np.concatenate((self.linear(z, self.p["input_layer"]), cond,
                            self.linear(cam, self.p["cam_refiner"])), 0)[None].astype(np.float32)
        for i, bp in enumerate(self.p["blocks"]):
            x = self.joint_block(bp, x, t_mod, L)
            if self.progress is not None:
                self.progress(i)
        fs = (self.p["final_shift_table"][None] + t_emb[:, None, :]).astype(np.float32)
        rows = np.ascontiguousarray(np.concatenate((x[:, :L], x[:, -1:]), 1))
        h = self._modulate(self._ln(rows, self.cfg.final_ln_eps),
                           np.ascontiguousarray(fs[:, 1]), np.ascontiguousarray(fs[:, 0])).reshape(L + 1, C)
        return (self.linear(h[:L], self.p["out_layer"]),
                self.linear(np.ascontiguousarray(h[L:]), self.p["cam_out_layer"]))

    def joint_euler_cfg_step(self, z, cond, cam, step=0):
        """(z_next, v_cfg, cam_next, v_cam_cfg) of one CFG Euler step."""
        t1000, dt = self.step_times(step)
        t = np.full(1, t1000, np.float32)
        v_pos, vc_pos = self.joint_velocity(z, cond, cam, t)
        v_neg, vc_neg = self.joint_velocity(z, np.zeros_like(cond), cam, t)
        out = []
        for vp, vn, state in ((v_pos, v_neg, z), (vc_pos, vc_neg, cam)):
            vp, vn = np.ascontiguousarray(vp), np.ascontiguousarray(vn)
            self._ew("cfg_combine_inplace", vp, vn, np.array([self.cfg.guidance], np.float32), 1, vp.size)
            nxt = np.array(state, np.float32, copy=True)
            self._ew("euler_update_inplace", nxt, vp, np.array([dt], np.float32), 1, nxt.size)
            out += [nxt, vp]
        return tuple(out)
