"""Shared parity helpers: seeded inputs, float64 closed forms, error stats,
and the tolerances the GPU tests use (each stated next to its derivation)."""
from __future__ import annotations

import math

import numpy as np

U = 2.0 ** -24  # fp32 unit roundoff


def seeded_linear(seed, M, K, N, w_scale=0.03, b_scale=0.01):
    """x ~ N(0,1) [M,K], W = w_scale*N(0,1) [N,K], bias = b_scale*N(0,1) [N]
    (the shapes/scales of scripts/smoke_native_rnf8_avx512.py:21-25)."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K), dtype=np.float32) * np.float32(w_scale)).astype(np.float32)
    b = (r.standard_normal(N, dtype=np.float32) * np.float32(b_scale)).astype(np.float32)
    return x, w, b


def gemm_f64(x, w_t, bias):
    """Exact-in-float64 bias + x @ w_t for fp32 inputs (w_t [K, N])."""
    return bias.astype(np.float64)[None, :] + x.astype(np.float64) @ w_t.astype(np.float64)


def gemm_abs_f64(x, w_t, bias):
    return np.abs(bias.astype(np.float64))[None, :] + np.abs(x.astype(np.float64)) @ np.abs(w_t.astype(np.float64))


def gemm_order_bound(x, w_t, bias):
    """Any fp32 evaluation order of bias + sum_k x_k w_k (products of fp32
    values, each rounded or fused) lies within gamma_{K+1} * sum|terms| of
    the exact value (Higham, Accuracy and Stability, Thm 3.1 / 3.4); two
    such evaluations differ by at most twice that.  gamma_n = n u / (1 - n u)."""
    K = x.shape[1]
    n = K + 1
    gamma = n * U / (1.0 - n * U)
    return 2.0 * gamma * gemm_abs_f64(x, w_t, bias)


def sdpa_f64(q, k, v, bias=None):
    """Textbook softmax(q k^T / 8 + bias) v in float64; bias [Lk] or [H, Lk]."""
    q64, k64, v64 = (a.astype(np.float64) for a in (q, k, v))
    s = np.einsum("bhqd,bhkd->bhqk", q64, k64) * 0.125
    if bias is not None:
        b = np.asarray(bias, np.float64)
        s = s + (b[None, None, None, :] if b.ndim == 1 else b[None, :, None, :])
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, v64)


def stats(out, ref):
    d = out.astype(np.float64) - ref.astype(np.float64)
    mse = float(np.mean(d * d))
    den = float(np.mean(ref.astype(np.float64) ** 2))
    return {
        "max_abs": float(np.abs(d).max()) if d.size else 0.0,
        "rmse": math.sqrt(mse),
        "rel_rmse": math.sqrt(mse / max(den, 1e-300)),
    }


# SDPA tolerance against the oracle.  Both sides form o = sum_j p_j v_j /
# sum_j p_j with p_j = exp(s_j - m).  The device evaluates the exponent in
# log2 units, exp2((s_j - m) * log2 e), so its p_j carries a relative error
# of about |s_j - m| * log2(e) * u (argument rounding, |s_j - m| <= 2 * 8 +
# |bias| range) plus ~2 ulp (v_exp_f32); the reference's Cephes exp adds
# ~1 ulp.  A common relative perturbation eps of the weights moves o by at
# most 2 * eps * max|v|.  With |s - m| <= 40 that is 2 * (40 * 1.45 + 4) *
# u * max|v| ~= 7.4e-6 * max|v|; summation-order differences over Lk terms
# stay well below that for the sizes tested.  The errors of different keys
# are independent, so the RMS error over all outputs is far smaller; it is
# measured against rms(v) because |o| itself shrinks like 1/sqrt(Lk).
# Stated tolerances:
SDPA_ATOL_PER_MAXV = 1.0e-5
SDPA_RMSE_PER_RMSV = 1.0e-6
