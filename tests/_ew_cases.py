"""Seeded cases for the flow-block / sampler elementwise ops.

Each case is (op, arrays, args, outputs): `arrays` maps names to fp32 NumPy
inputs, `args` is the reference's C argument list without `threads` (array
names as strings, None for a null pointer, then scalars), `outputs` names
the arrays the op writes.  Shared by the CPU oracle tests, the GPU tests and
tests/golden/make_golden.py.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def _specials(n, rng, scale):
    x = (rng.standard_normal(n) * scale).astype(f32)
    sp = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-8, -1e-8, 3.0, -3.0, 9.5, -9.5, 44.0, -44.0,
                   88.0, -88.0, 100.0, -100.0, 1e4, -1e4], f32)
    x[: sp.size] = sp
    return x


def cases():
    r = np.random.default_rng(2024)
    out = {}

    def ln(name, rows, cols, affine, shift=0.0):
        x = (r.standard_normal((rows, cols)) * 2.0 + shift).astype(f32)
        w = (1.0 + 0.1 * r.standard_normal(cols)).astype(f32)
        b = (0.1 * r.standard_normal(cols)).astype(f32)
        arrays = dict(x=x, out=np.zeros_like(x))
        if affine:
            arrays.update(w=w, b=b)
        out[name] = ("layernorm", arrays,
                     ["x", "w" if affine else None, "b" if affine else None, "out", rows, cols,
                      f32(1e-6), int(affine)], ["out"])

    ln("ln_1024_affine", 6, 1024, True)
    ln("ln_1024_plain_offset", 3, 1024, False, shift=30.0)
    ln("ln_1000_ragged", 4, 1000, True)
    ln("ln_7_short", 5, 7, False)

    def rms(name, outer, heads, dim):
        x = r.standard_normal((outer, heads, dim)).astype(f32)
        x[0, 0] = 0.0  # zero vector: the eps branch
        g = (1.0 + 0.05 * r.standard_normal((heads, dim))).astype(f32)
        out[name] = ("multihead_rmsnorm", dict(x=x, g=g, out=np.zeros_like(x)),
                     ["x", "g", "out", outer, heads, dim, f32(1e-12)], ["out"])

    rms("rmsnorm_64", 6, 4, 64)
    rms("rmsnorm_40_ragged", 3, 2, 40)

    ang = r.standard_normal((10, 32)).astype(f32)
    fr = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(10, 64).astype(f32)
    x = r.standard_normal((10, 64)).astype(f32)
    out["rope_10x64"] = ("rope_complex", dict(x=x, f=fr, out=np.zeros_like(x)),
                         ["x", "f", "out", 10, 64], ["out"])

    h = r.standard_normal((2, 4, 1024)).astype(f32)
    s = (0.3 * r.standard_normal((2, 1024))).astype(f32)
    t = r.standard_normal((2, 1024)).astype(f32)
    out["modulate_2x4x1024"] = ("modulate_inplace", dict(h=h, s=s, t=t),
                                 ["h", "s", "t", 2, 4, 1024], ["h"])
    out["modulate_3x5x37"] = ("modulate_inplace",
                              dict(h=r.standard_normal((3, 5, 37)).astype(f32),
                                   s=r.standard_normal((3, 37)).astype(f32),
                                   t=r.standard_normal((3, 37)).astype(f32)),
                              ["h", "s", "t", 3, 5, 37], ["h"])
    xb = r.standard_normal((2, 4, 1024)).astype(f32)
    hb = r.standard_normal((2, 4, 1024)).astype(f32)
    gb = r.standard_normal((2, 1024)).astype(f32)
    out["gated_2x4x1024"] = ("gated_residual_inplace", dict(x=xb, h=hb, g=gb),
                              ["x", "h", "g", 2, 4, 1024], ["x", "h"])
    a = r.standard_normal(1003).astype(f32)
    d = r.standard_normal(1003).astype(f32)
    out["add_1003"] = ("add_inplace", dict(x=a, d=d), ["x", "d", 1003], ["x"])
    xg = _specials(4099, r, 3.0)
    out["gelu_4099"] = ("gelu_tanh", dict(x=xg, out=np.zeros_like(xg)), ["x", "out", xg.size], ["out"])
    out["silu_4099"] = ("silu", dict(x=xg.copy(), out=np.zeros_like(xg)), ["x", "out", xg.size], ["out"])

    pos = r.standard_normal((2, 501)).astype(f32)
    neg = r.standard_normal((2, 501)).astype(f32)
    g = np.array([3.0, 1.5], f32)
    out["cfg_2x501"] = ("cfg_combine_inplace", dict(p=pos, n=neg, g=g), ["p", "n", "g", 2, 501], ["p"])
    smp = r.standard_normal((2, 501)).astype(f32)
    dt = np.array([0.0476, 0.125], f32)
    out["euler_2x501"] = ("euler_update_inplace", dict(x=smp, v=pos.copy(), dt=dt),
                           ["x", "v", "dt", 2, 501], ["x"])
    prev = r.standard_normal((2, 501)).astype(f32)
    pdt = np.array([0.05, 0.0], f32)  # second batch: the 1e-12 clamp
    out["ab2_2x501"] = ("ab2_update_inplace",
                         dict(x=smp.copy(), v=pos.copy(), pv=prev, dt=dt.copy(), pdt=pdt),
                         ["x", "v", "pv", "dt", "pdt", 2, 501], ["x"])
    return out


def run(O, case, backend="oracle", arrays=None):
    """Run a case through oracle.ew on copies of its arrays; returns the arrays."""
    op, arrays0, args, _ = case
    arrs = {k: v.copy() for k, v in (arrays or arrays0).items()}
    conv = [arrs[a] if isinstance(a, str) else a for a in args]
    st = O.ew(op, *conv, backend=backend)
    assert st == 0, (op, st)
    return arrs
