"""Pinning of the oracle's bf16 precision modes (no GPU).

oracle.bf16_round is checked bit for bit against torch's float32 ->
bfloat16 conversion (the conversion of the reference's bf16 round-trip
probe, scripts/triposplat_bf16_roundtrip_patch.py:27-31) on random values
and on the cases a rounding mistake shows first: exact ties with even and
odd last kept bits, neighbours of ties, subnormals, the overflow threshold.
The split and the two GEMM term sums are pinned by what the arithmetic
fixes: hi and lo are bf16 values with |a - hi - lo| <= 2^-16 |a|; operands
exact in bf16 make both modes equal the exact product; generic operands stay
within the bf16 / bf16x3 product error bounds (2^-7 and 2^-14 of sum|x w|)
and the bf16 mode is measurably coarser than bf16x3.
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import gemm_f64, gemm_abs_f64


def _torch_bf16(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def test_bf16_round_matches_torch(oracle):
    r = np.random.default_rng(0)
    vals = [r.standard_normal(20000).astype(np.float32) * np.float32(s) for s in (1e-30, 1e-3, 1.0, 1e4, 1e30)]
    hi_bits = r.integers(0, 1 << 16, 4096, dtype=np.uint32) << 16
    ties = (hi_bits | 0x8000).view(np.float32)               # exact ties, both parities of the kept lsb
    below = (hi_bits | 0x7FFF).view(np.float32)
    above = (hi_bits | 0x8001).view(np.float32)
    sub = (r.integers(1, 1 << 23, 4096, dtype=np.uint32)).view(np.float32)  # subnormals
    edge = np.array([0.0, -0.0, 3.3895314e38, 3.3961776e38, -3.3961776e38, 1.0 + 2 ** -8,
                     1.0 + 3 * 2 ** -8, np.finfo(np.float32).max], np.float32)
    a = np.concatenate(vals + [ties, below, above, sub, edge])
    a = a[np.isfinite(a) & ~np.isnan(a)]
    got = oracle.bf16_round(a)
    exp = _torch_bf16(a)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    # ties really went both ways (round to even), so the case is exercised
    t = oracle.bf16_round(ties).view(np.uint32)
    assert np.any(t > (hi_bits & 0xFFFF0000)) and np.any(t == (hi_bits & 0xFFFF0000))


def test_bf16_split_invariants(oracle):
    r = np.random.default_rng(1)
    a = (r.standard_normal(50000) * np.exp(r.uniform(-20, 20, 50000))).astype(np.float32)
    hi, lo = oracle.bf16_split(a)
    assert not np.any(hi.view(np.uint32) & 0xFFFF) and not np.any(lo.view(np.uint32) & 0xFFFF)
    res = np.abs(a.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    assert np.all(res <= 2.0 ** -16 * np.abs(a.astype(np.float64)))
    assert np.mean(res > 0) > 0.9          # 24 bits do not fit in 16: the residual is real
    assert np.all(np.abs(lo) <= 2.0 ** -8 * np.abs(hi) * (1 + 2.0 ** -7))


def test_nf24_bf16_split_w_exact(oracle):
    """wh = bf16(fp32(p*s)), wl = bf16(fp32(p*s - wh)) against exact rational
    arithmetic: the product and the residual are exact in float64 (checked
    here), so their fp32 roundings are the single roundings the definition
    names; and the FMA residual is a different split from bf16_split(w)."""
    from fractions import Fraction
    r = np.random.default_rng(11)
    K, N = 64, 48
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    wh, wl = oracle.nf24_bf16_split_w(c01, q2, s)
    assert not np.any(wh.view(np.uint32) & 0xFFFF) and not np.any(wl.view(np.uint32) & 0xFFFF)
    for k, n in zip(r.integers(0, K, 400), r.integers(0, N, 400)):
        p = int(c01[k, n]) * 256 + int(q2[k, n])
        prod = Fraction(p) * Fraction(float(s[n]))
        assert Fraction(float(prod)) == prod                    # exact in float64
        assert np.float32(float(prod)) == oracle.decode_nf24(c01, q2, s)[k, n]
        assert oracle.bf16_round(np.float32(float(prod))) == wh[k, n]
        res = prod - Fraction(float(wh[k, n]))
        assert Fraction(float(res)) == res                      # exact in float64
        assert oracle.bf16_round(np.float32(float(res))) == wl[k, n]
    wd = oracle.decode_nf24(c01, q2, s).astype(np.float64)
    prod = (c01.astype(np.float64) * 256 + q2) * s.astype(np.float64)[None, :]
    assert np.all(np.abs(prod - wh - wl) <= 2.0 ** -16 * np.abs(prod) + 1e-300)
    h2, l2 = oracle.bf16_split(wd.astype(np.float32))
    assert np.array_equal(h2, wh)
    assert 0 < np.count_nonzero(l2 != wl) < l2.size // 4       # distinct, rarely


def _exact_bf16_linear(oracle, seed, M, K, N):
    """x exact in bf16; NF24 codes with q2 = 0, |q01| < 128 and a power-of-two
    scale, so every decoded weight has at most 8 significant bits."""
    r = np.random.default_rng(seed)
    x = oracle.bf16_round(r.standard_normal((M, K)).astype(np.float32))
    c01 = r.integers(-127, 128, (K, N)).astype(np.int16)
    q2 = np.zeros((K, N), np.int8)
    s = np.full(N, 2.0 ** -14, np.float32)
    b = r.standard_normal(N).astype(np.float32) * np.float32(0.01)
    return x, c01, q2, s, b


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_bf16_terms_exact_operands(oracle, precision):
    x, c01, q2, s, b = _exact_bf16_linear(oracle, 2, 37, 96, 53)
    w = oracle.decode_nf24(c01, q2, s)
    assert np.array_equal(oracle.bf16_round(w), w)
    got = oracle.nf24_gemm_bf16_terms(x, c01, q2, s, b, precision)
    assert got.shape == (37, 53)
    np.testing.assert_allclose(got, gemm_f64(x, w, b), rtol=0, atol=1e-12)


def test_bf16_terms_error_bounds(oracle):
    r = np.random.default_rng(3)
    M, K, N = 64, 512, 96
    x = r.standard_normal((M, K)).astype(np.float32)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    b = (r.standard_normal(N) * 0.01).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    wd = oracle.decode_nf24(c01, q2, s)
    exact = gemm_f64(x, wd, b)
    mag = gemm_abs_f64(x, wd, np.zeros_like(b))
    e1 = oracle.nf24_gemm_bf16_terms(x, c01, q2, s, b, "bf16") - exact
    e3 = oracle.nf24_gemm_bf16_terms(x, c01, q2, s, b, "bf16x3") - exact
    assert np.all(np.abs(e1) <= 2.0 ** -7 * mag)
    assert np.all(np.abs(e3) <= 2.0 ** -14 * mag)
    rel1 = np.sqrt(np.mean(e1 ** 2) / np.mean(exact ** 2))
    rel3 = np.sqrt(np.mean(e3 ** 2) / np.mean(exact ** 2))
    assert 2.0 ** -12 < rel1 < 2.0 ** -6, rel1     # bf16 rounding is applied
    assert rel3 < rel1 / 64, (rel1, rel3)          # the lo terms recover ~8 bits


def test_bf16_round_non_finite(oracle):
    """Inf stays Inf with its sign; every NaN whose upper 7 mantissa bits are
    not all zero stays NaN (its lower 16 bits are dropped, never carried
    into the exponent or the sign); largest finite values round to Inf."""
    r = np.random.default_rng(4)
    inf = np.array([np.inf, -np.inf], np.float32)
    assert np.array_equal(oracle.bf16_round(inf), inf)
    mant = r.integers(1 << 16, 1 << 23, 4096, dtype=np.uint32)
    sign = r.integers(0, 2, 4096, dtype=np.uint32) << 31
    nan = (sign | 0x7F800000 | mant).view(np.float32)
    out = oracle.bf16_round(nan)
    assert np.all(np.isnan(out))
    assert np.array_equal(out.view(np.uint32) >> 31, sign >> 31)
    big = np.array([3.4028235e38, -3.4028235e38], np.float32)
    assert np.array_equal(oracle.bf16_round(big), inf)


def _sdpa_inputs(seed, B, H, Lq, Lk, scale=8.0):
    """RMS-normalised rows of norm `scale` (the flow's q and k after RMSNorm
    with unit gamma), v ~ N(0, 1)."""
    r = np.random.default_rng(seed)

    def rows(n):
        a = r.standard_normal((B, H, n, 64))
        return (a / np.linalg.norm(a, axis=-1, keepdims=True) * scale).astype(np.float32)

    return rows(Lq), rows(Lk), r.standard_normal((B, H, Lk, 64)).astype(np.float32)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("bias_kind", [None, "shared", "per_head"])
def test_sdpa_bf16_terms_error_bounds(oracle, precision, bias_kind):
    """The mode's float64 reference stays within what its rounding allows of
    the textbook softmax(q k^T / 8 + b) v: a score error E (log2 units) moves
    the normalised weights by at most a factor 2^(2E) - 1, and the value
    representation adds eps_v max|v|.  Per product, bf16x3 keeps
    |a b - (ah bh + ah bl + al bh)| <= 3.01 * 2^-18 |a b| and bf16 2^-8 |a b|."""
    from _parity import sdpa_f64

    B, H, Lq, Lk = 1, 3, 40, 70
    q, k, v = _sdpa_inputs(5, B, H, Lq, Lk)
    r = np.random.default_rng(6)
    bias = {None: None, "shared": r.uniform(-2, 0, Lk).astype(np.float32),
            "per_head": r.uniform(-2, 0, (H, Lk)).astype(np.float32)}[bias_kind]
    got, s_abs, _ = oracle.sdpa_bf16_terms(q, k, v, bias, precision)
    exact = sdpa_f64(q, k, v, bias)
    rel, eps_v = (3.01 * 2.0 ** -18, 2.0 ** -17) if precision == "bf16x3" else (2.0 ** -8 * 1.01, 2.0 ** -8)
    E = (rel + 2.0 ** -22) * s_abs + 2.0 ** -22 * (0 if bias is None else 2.0)
    vmax = np.abs(v.astype(np.float64)).max(axis=(-1, -2))[..., None, None]
    bound = ((np.exp2(2 * E) - 1)[..., None] + eps_v) * vmax
    assert np.all(np.abs(got - exact) <= bound * (1 + 1e-9) + 1e-12)
    err = np.sqrt(np.mean((got - exact) ** 2) / np.mean(exact ** 2))
    if precision == "bf16x3":
        assert err < 2.0 ** -14, err
    else:
        assert 2.0 ** -12 < err < 2.0 ** -5, err


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_sdpa_bf16_terms_closed_forms(oracle, precision):
    """One key: the output is the value's representation itself (vh, or
    vh + vl).  Identical keys: equal weights, the mean of the represented
    values.  Both are independent of q and of the score terms."""
    q, k, v = _sdpa_inputs(7, 1, 2, 9, 1)
    got, _, _ = oracle.sdpa_bf16_terms(q, k, v, None, precision)
    vh, vl = oracle.bf16_split(v)
    rep = vh.astype(np.float64) + (vl.astype(np.float64) if precision == "bf16x3" else 0)
    np.testing.assert_array_equal(got, np.broadcast_to(rep, got.shape))
    q, k, v = _sdpa_inputs(8, 1, 2, 9, 33)
    k[:] = k[:, :, :1]
    got, _, _ = oracle.sdpa_bf16_terms(q, k, v, None, precision)
    vh, vl = oracle.bf16_split(v)
    rep = vh.astype(np.float64) + (vl.astype(np.float64) if precision == "bf16x3" else 0)
    np.testing.assert_allclose(got, np.broadcast_to(rep.mean(axis=2, keepdims=True), got.shape),
                               rtol=0, atol=1e-14)
