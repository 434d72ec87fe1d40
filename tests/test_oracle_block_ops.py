"""Pinning the oracle's flow-block / sampler restatements (CPU only).

* bit-exact against the reference's own AVX-512 build (oracle/_ref) on every
  case of _ew_cases, where the reference sources are present;
* bit-exact against the committed fixtures tests/golden/ew_ops.npz that the
  reference build wrote;
* against float64 closed forms of each op, with tolerances stated per test,
  including the reference's LayerNorm variance over padded lanes;
* a planted mistake (the GELU / modulation fma written unfused) must break
  bit-exactness.
"""
from __future__ import annotations

import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

import _ew_cases as EC

GOLDEN = Path(__file__).resolve().parent / "golden" / "ew_ops.npz"
CASES = EC.cases()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_build(oracle, name):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    case = CASES[name]
    got = EC.run(oracle, case)
    ref = EC.run(oracle, case, backend="reference")
    for k in case[3]:
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), (name, k)


def test_oracle_matches_golden(oracle):
    data = np.load(GOLDEN)
    for name, case in CASES.items():
        inputs = {k: data[f"{name}/in/{k}"] for k in case[1]}
        got = EC.run(oracle, case, arrays=inputs)
        for k in case[3]:
            assert np.array_equal(_bits(got[k]), _bits(data[f"{name}/out/{k}"])), (name, k)


def test_layernorm_closed_form(oracle):
    """(x - mean) / sqrt(var + eps) in float64, with var including mean^2 for
    each padded lane of the last 16-column chunk (the reference's masked
    loads); |err| <= 2e-5 relative to the output scale.  Dropping the padded
    term misses by ~1e-2 at cols = 1000 and fails."""
    r = np.random.default_rng(5)
    for cols in (1024, 1000, 7):
        x = (r.standard_normal((6, cols)) + 3.0).astype(np.float32)
        out = np.empty_like(x)
        assert oracle.ew("layernorm", x, None, None, out, 6, cols, np.float32(1e-6), 0) == 0
        xd = x.astype(np.float64)
        mean = xd.mean(1, keepdims=True)
        pad = (-cols) % 16
        var = (((xd - mean) ** 2).sum(1, keepdims=True) + pad * mean ** 2) / cols
        exp = (xd - mean) / np.sqrt(var + 1e-6)
        assert np.abs(out - exp).max() <= 2e-5 * np.abs(exp).max(), cols
        if pad:
            wrong = (xd - mean) / np.sqrt(((xd - mean) ** 2).mean(1, keepdims=True) + 1e-6)
            assert np.abs(out - wrong).max() > 1e-3


def test_rmsnorm_rope_closed_forms(oracle):
    r = np.random.default_rng(6)
    x = r.standard_normal((5, 3, 64)).astype(np.float32)
    g = (1 + 0.05 * r.standard_normal((3, 64))).astype(np.float32)
    out = np.empty_like(x)
    assert oracle.ew("multihead_rmsnorm", x, g, out, 5, 3, 64, np.float32(1e-12)) == 0
    xd = x.astype(np.float64)
    exp = xd * 8.0 / np.linalg.norm(xd, axis=-1, keepdims=True) * g
    assert np.abs(out - exp).max() <= 4e-6 * np.abs(exp).max()
    ang = r.standard_normal((4, 32))
    f = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(4, 64).astype(np.float32)
    x = r.standard_normal((4, 64)).astype(np.float32)
    y = np.empty_like(x)
    assert oracle.ew("rope_complex", x, f, y, 4, 64) == 0
    z = (x[:, 0::2] + 1j * x[:, 1::2]).astype(np.complex128) * (f[:, 0::2] + 1j * f[:, 1::2])
    assert np.abs(y[:, 0::2] - z.real).max() <= 1e-6 and np.abs(y[:, 1::2] - z.imag).max() <= 1e-6
    # rotation preserves the norm of each pair
    assert np.allclose(np.hypot(y[:, 0::2], y[:, 1::2]), np.hypot(x[:, 0::2], x[:, 1::2]), rtol=1e-6)


def test_activations_closed_forms(oracle):
    """GELU-tanh and SiLU against float64 math.tanh / math.exp: |err| <=
    3e-7 * max(1, |x|) (the Cephes exp is accurate to ~2 ulp)."""
    x = np.linspace(-12, 12, 40001, dtype=np.float32)
    y = np.empty_like(x)
    assert oracle.ew("gelu_tanh", x, y, x.size) == 0
    xd = x.astype(np.float64)
    exp = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(y - exp) <= 3e-7 * np.maximum(1.0, np.abs(xd)))
    assert oracle.ew("silu", x, y, x.size) == 0
    exp = xd / (1 + np.exp(-xd))
    assert np.all(np.abs(y - exp) <= 3e-7 * np.maximum(1.0, np.abs(xd)))
    z = np.array([0.0, -0.0], np.float32)
    w = np.empty_like(z)
    assert oracle.ew("gelu_tanh", z, w, 2) == 0 and not w.any()


def test_elementwise_and_sampler_closed_forms(oracle):
    r = np.random.default_rng(7)
    h = r.standard_normal((2, 3, 40)).astype(np.float32)
    s = r.standard_normal((2, 40)).astype(np.float32)
    t = r.standard_normal((2, 40)).astype(np.float32)
    y = h.copy()
    assert oracle.ew("modulate_inplace", y, s, t, 2, 3, 40) == 0
    exp = h.astype(np.float64) * (1 + s.astype(np.float32)).astype(np.float64)[:, None] + t[:, None]
    assert np.all(np.abs(y - exp) <= 2 ** -23 * np.abs(exp) + 1e-30)   # one rounding
    p = r.standard_normal((2, 50)).astype(np.float32)
    n = r.standard_normal((2, 50)).astype(np.float32)
    g = np.array([3.0, 1.5], np.float32)
    q = p.copy()
    assert oracle.ew("cfg_combine_inplace", q, n, g, 2, 50) == 0
    exp = g[:, None].astype(np.float64) * p - (g[:, None] - 1.0) * n
    assert np.abs(q - exp).max() <= 1e-5
    z = p.copy()
    dt = np.array([0.1, 0.2], np.float32)
    assert oracle.ew("euler_update_inplace", z, n, dt, 2, 50) == 0
    assert np.abs(z - (p - dt[:, None].astype(np.float64) * n)).max() <= 1e-6
    # AB2 with dt == previous dt: sample - dt * (1.5 v - 0.5 v_prev)
    z = p.copy()
    pv = r.standard_normal((2, 50)).astype(np.float32)
    assert oracle.ew("ab2_update_inplace", z, n, pv, dt, dt.copy(), 2, 50) == 0
    exp = p - dt[:, None].astype(np.float64) * (1.5 * n - 0.5 * pv)
    assert np.abs(z - exp).max() <= 1e-5


def test_planted_unfused_gelu_and_modulation_break_parity(oracle, tmp_path):
    """The oracle built with -DORACLE_EW_UNFUSED (the reference's contracted
    fma written as a separate multiply and add) must differ from the
    reference on the golden GELU and modulation cases."""
    src = Path(oracle.__file__).resolve().parent / "tsplat_oracle.c"
    so = tmp_path / "liboracle_ew_planted.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fopenmp",
                    "-DORACLE_EW_UNFUSED", "-o", str(so), str(src), "-lm"], check=True)
    import ctypes

    L = ctypes.CDLL(str(so))
    data = np.load(GOLDEN)
    x = np.ascontiguousarray(data["gelu_4099/in/x"])
    y = np.empty_like(x)
    L.oracle_gelu_tanh.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    assert L.oracle_gelu_tanh(x.ctypes.data, y.ctypes.data, x.size) == 0
    assert not np.array_equal(_bits(y), _bits(data["gelu_4099/out/out"]))
    h = np.ascontiguousarray(data["modulate_2x4x1024/in/h"]).copy()
    s = np.ascontiguousarray(data["modulate_2x4x1024/in/s"])
    t = np.ascontiguousarray(data["modulate_2x4x1024/in/t"])
    L.oracle_modulate_inplace.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3
    assert L.oracle_modulate_inplace(h.ctypes.data, s.ctypes.data, t.ctypes.data, 2, 4, 1024) == 0
    assert not np.array_equal(_bits(h), _bits(data["modulate_2x4x1024/out/h"]))
