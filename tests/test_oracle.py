"""Pinning of the CPU oracle (no GPU).

1. Bit-exact against the fixtures in tests/golden/, written by the reference's
   own AVX-512 kernels compiled from its sources (tests/golden/make_golden.py).
2. Bit-exact against oracle/_ref directly on more seeds, when that build is
   present (this container only; the GPU box has no reference sources).
3. Against float64 closed forms and invariants that a plausible mistake
   (dropped bias, transposed operand, wrong scale, off-by-one tail, wrong
   reduction order) would break.
4. A planted mistake: the oracle compiled with the running-sum update
   unfused must NOT match the golden output -- so the fixtures discriminate
   at the level of a single rounding.
5. The NF24 packer: alphabet closed form with its tie margin, brute-force
   nearest-level and round-half-up digits, the reconstruction bound.
"""
from __future__ import annotations

import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

from _parity import gemm_f64, gemm_order_bound, sdpa_f64, stats

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _load(name):
    with np.load(GOLDEN / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------- golden
def test_golden_gemm(oracle):
    g = _load("gemm_25x96x64")
    assert _bits_equal(oracle.nf24_gemm(g["x"], g["code01_t"], g["q2_t"], g["scale"], g["bias"]), g["out"])
    g = _load("gemm_tail_3x96x5")
    assert _bits_equal(oracle.nf24_gemm(g["x"], g["code01_t"], g["q2_t"], g["scale"], g["bias"]), g["out"])
    g = _load("gemm_range_40x96x64_s16_c32")
    got = oracle.nf24_gemm(g["x"], g["code01_t"], g["q2_t"], g["scale"], g["bias"],
                           output_start=int(g["start"]), output_count=int(g["count"]), require_aligned=True)
    assert _bits_equal(got, g["out"])


@pytest.mark.parametrize("name", ["sdpa_self_16", "sdpa_masked_17_log7", "sdpa_cross_15x19", "sdpa_bias_9x530"])
def test_golden_sdpa(oracle, name):
    g = _load(name)
    assert _bits_equal(oracle.sdpa_q8t512(g["q"], g["k"], g["v"], g.get("key_bias")), g["out"])


def test_golden_sdpa_packed(oracle):
    g = _load("sdpa_packed_blhd_15x19")
    got = oracle.sdpa_q8t512_packed_blhd(g["q"], g["packed_k"], g["packed_v"], int(g["lk"]))
    assert _bits_equal(got, g["out"])


def test_golden_qkv(oracle):
    g = _load("qkv_postprocess_2x20x2")
    got = oracle.qkv_rope_rmsnorm_pack(g["qkv"], g["freqs"], g["q_gamma"], g["k_gamma"], 2, 20, 2)
    for a, key in zip(got, ("q", "packed_k", "packed_v")):
        assert _bits_equal(a, g[key])
    g = _load("qkv_direct_1x17x2_k128")
    got = oracle.gemm_nf24_qkv_direct(g["x"], g["code01_t"], g["q2_t"], g["scale"], g["bias"], g["freqs"],
                                      g["q_gamma"], g["k_gamma"], 1, 17, 2)
    for a, key in zip(got, ("q", "packed_k", "packed_v")):
        assert _bits_equal(a, g[key])


def test_golden_qkv_selected(oracle):
    g = _load("qkv_selected_2x21x37")
    st, got = oracle.q_kv_selected_rope_rmsnorm_pack(g["q"], g["kv"], g["freqs"], g["selected"],
                                                     g["q_gamma"], g["k_gamma"], 2, 21, 37, 2)
    assert st == 0
    for a, key in zip(got, ("q_out", "packed_k", "packed_v")):
        assert _bits_equal(a, g[key])
    # an index outside [0, Lk) is rejected (-3) before any work, as the reference does
    bad = g["selected"].copy()
    bad[5] = 37
    assert oracle.q_kv_selected_rope_rmsnorm_pack(g["q"], g["kv"], g["freqs"], bad, g["q_gamma"],
                                                  g["k_gamma"], 2, 21, 37, 2)[0] == -3
    if oracle.ref_available():
        assert oracle.ref_q_kv_selected(g["q"], g["kv"], g["freqs"], bad, g["q_gamma"], g["k_gamma"],
                                        2, 21, 37, 2)[0] == -3


# ---------------------------------------------------------------- _ref
def test_oracle_matches_reference_build(oracle):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    r = np.random.default_rng(2024)
    for (M, K, N) in [(9, 33, 48), (17, 200, 80), (1, 7, 16)]:
        x = r.standard_normal((M, K), dtype=np.float32)
        w = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
        b = (r.standard_normal(N) * 0.01).astype(np.float32)
        c01, q2, s = oracle.quantize_nf24_i16(w)
        assert _bits_equal(oracle.nf24_gemm(x, c01, q2, s, b), oracle.ref_nf24_gemm(x, c01, q2, s, b, 2))
    for (B, H, Lq, Lk, bias) in [(2, 2, 9, 1030, True), (1, 3, 20, 33, False), (1, 1, 3, 1, True)]:
        q = r.standard_normal((B, H, Lq, 64), dtype=np.float32)
        k = r.standard_normal((B, H, Lk, 64), dtype=np.float32) * np.float32(2.0)
        v = r.standard_normal((B, H, Lk, 64), dtype=np.float32)
        kb = r.uniform(-3, 1, Lk).astype(np.float32) if bias else None
        assert _bits_equal(oracle.sdpa_q8t512(q, k, v, kb), oracle.ref_sdpa_q8t512(q, k, v, kb, 2))


# ---------------------------------------------------------------- closed forms
def test_gemm_closed_form(oracle):
    """bias + x @ decode(W) in float64; the sequential chain stays within the
    order bound, and a transposed weight / dropped bias would not."""
    r = np.random.default_rng(5)
    x = r.standard_normal((12, 96), dtype=np.float32)
    w = (r.standard_normal((40, 96)) * 0.03).astype(np.float32)
    b = (r.standard_normal(40) * 0.5).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    w_t = oracle.decode_nf24(c01, q2, s)
    got = oracle.nf24_gemm(x, c01, q2, s, b)
    exact = gemm_f64(x, w_t, b)
    assert np.all(np.abs(got - exact) <= gemm_order_bound(x, w_t, b) / 2)
    assert np.abs(got - (exact - b)).max() > 0.1  # the bias is really added


def test_decode_is_exact(oracle):
    """decode16: fp32((int32)q01*256 + q2) * scale, one rounding; spot values."""
    for q01, q2, s in [(635, 127, 1e-3), (-636, -128, 3.7e-5), (0, 1, 2.0), (1, 0, 0.5)]:
        want = np.float32(np.float64(q01 * 256 + q2) * np.float64(np.float32(s)))
        assert oracle.lib().oracle_nf24_decode(q01, q2, s) == want


@pytest.mark.parametrize("B,H,Lq,Lk,bias", [(1, 2, 16, 16, False), (1, 2, 17, 17, True),
                                            (1, 1, 5, 1500, True), (2, 1, 3, 513, False)])
def test_sdpa_closed_form(oracle, B, H, Lq, Lk, bias):
    r = np.random.default_rng(Lk)
    q = r.standard_normal((B, H, Lq, 64), dtype=np.float32)
    k = r.standard_normal((B, H, Lk, 64), dtype=np.float32)
    v = r.standard_normal((B, H, Lk, 64), dtype=np.float32)
    kb = r.uniform(-2, 0, Lk).astype(np.float32) if bias else None
    got = oracle.sdpa_q8t512(q, k, v, kb)
    # The reference's own agreement with torch is ~5e-9 RMSE (L=8194).
    assert stats(got, sdpa_f64(q, k, v, kb))["max_abs"] < 5e-6


def test_sdpa_invariants(oracle):
    r = np.random.default_rng(8)
    q = r.standard_normal((1, 1, 6, 64), dtype=np.float32)
    k = r.standard_normal((1, 1, 40, 64), dtype=np.float32)
    v = r.standard_normal((1, 1, 40, 64), dtype=np.float32)
    # Lk == 1 returns v exactly
    one = oracle.sdpa_q8t512(q, k[:, :, :1], v[:, :, :1])
    assert np.array_equal(one, np.broadcast_to(v[:, :, :1], one.shape))
    # log(M) bias on key 0 == key 0 repeated M times
    M = 5
    kb = np.zeros(40, np.float32)
    kb[0] = np.float32(math.log(M))
    a = oracle.sdpa_q8t512(q, k, v, kb)
    b = oracle.sdpa_q8t512(q, np.concatenate([k] + [k[:, :, :1]] * (M - 1), 2),
                           np.concatenate([v] + [v[:, :, :1]] * (M - 1), 2))
    assert np.abs(a - b).max() < 1e-6
    # equal scores -> mean of v
    qz = np.zeros_like(q)
    assert np.abs(oracle.sdpa_q8t512(qz, k, v) - v.mean(axis=2, keepdims=True)).max() < 1e-6
    # per-head bias == one call per head
    k2 = r.standard_normal((1, 3, 40, 64), dtype=np.float32)
    v2 = r.standard_normal((1, 3, 40, 64), dtype=np.float32)
    q2 = r.standard_normal((1, 3, 6, 64), dtype=np.float32)
    hb = r.uniform(-2, 0, (3, 40)).astype(np.float32)
    full = oracle.sdpa_q8t512(q2, k2, v2, hb, bias_head_stride=40)
    for h in range(3):
        assert _bits_equal(full[:, h:h + 1], oracle.sdpa_q8t512(q2[:, h:h + 1], k2[:, h:h + 1], v2[:, h:h + 1], hb[h]))


def test_exp512_accuracy(oracle):
    """The restated Cephes exp is within 2 ulp of exp over the softmax range."""
    xs = np.linspace(-87.0, 0.0, 2001, dtype=np.float32)
    got = oracle.exp512(xs).astype(np.float64)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * ulp)


def test_reduce_add16_order(oracle):
    """Lanes are summed 8+8, 4+4, {0,2}+{1,3}: a sum that is order-sensitive."""
    a = np.array([1e8, 1, -1e8, 1] + [0.5] * 12, np.float32)
    f = oracle.lib().oracle_reduce_add16
    got = f(a.ctypes.data)
    t3 = [np.float32(a[i + 8] + a[i]) for i in range(8)]
    t6 = [np.float32(t3[i + 4] + t3[i]) for i in range(4)]
    want = np.float32(np.float32(t6[0] + t6[2]) + np.float32(t6[1] + t6[3]))
    assert got == want


def test_rope_rmsnorm_closed_form(oracle):
    r = np.random.default_rng(3)
    x = r.standard_normal(64, dtype=np.float32)
    ang = r.standard_normal(32)
    f = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(64).astype(np.float32)
    g = np.ones(64, np.float32)
    y = np.empty(64, np.float32)
    oracle.lib().oracle_rope_rmsnorm64(x.ctypes.data, f.ctypes.data, g.ctypes.data, y.ctypes.data)
    z = (x[0::2] + 1j * x[1::2]).astype(np.complex128) * (f[0::2] + 1j * f[1::2])
    want = np.empty(64)
    want[0::2], want[1::2] = z.real, z.imag
    want *= 8.0 / np.linalg.norm(want)
    assert np.abs(y - want).max() < 1e-5
    assert abs(np.linalg.norm(y.astype(np.float64)) - 8.0) < 1e-5  # rotation keeps the norm


# ---------------------------------------------------------------- planted mistake
def test_planted_mistake_is_caught(tmp_path, oracle):
    """Rebuild the oracle with the running-sum update unfused
    (global_sum * old_scale + local_sum * local_scale, two roundings) and
    show the golden fixture of a multi-tile call rejects it."""
    src = Path(oracle.__file__).resolve().parent / "tsplat_oracle.c"
    so = tmp_path / "liboracle_planted.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fopenmp",
                    "-DORACLE_SUM_UNFUSED", "-o", str(so), str(src), "-lm"], check=True)
    import ctypes

    L = ctypes.CDLL(str(so))
    L.oracle_sdpa_q8t512.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 7 + [ctypes.c_int64]
    # Many tiles make the unfused rounding visible; generated like the fixture.
    r = np.random.default_rng(77)
    q = r.standard_normal((1, 1, 64, 64), dtype=np.float32)
    k = r.standard_normal((1, 1, 4000, 64), dtype=np.float32) * np.float32(3.0)
    v = r.standard_normal((1, 1, 4000, 64), dtype=np.float32)
    out = np.empty_like(q)
    assert L.oracle_sdpa_q8t512(q.ctypes.data, k.ctypes.data, v.ctypes.data, None, out.ctypes.data,
                                1, 1, 64, 4000, 64, 0, 0, 0) == 0
    good = oracle.sdpa_q8t512(q, k, v)
    assert not _bits_equal(out, good)
    if oracle.ref_available():
        assert _bits_equal(good, oracle.ref_sdpa_q8t512(q, k, v, None, 2))


# ---------------------------------------------------------------- packer
def test_alphabet_closed_form(oracle):
    from tsplat import nf24

    assert oracle.alphabet_tie_margin() > 1e-4
    assert nf24.alphabet_tie_margin() > 1e-4
    import torch

    a_pkg = nf24.nf24_alphabet(torch).numpy()
    a_orc = oracle.nf24_alphabet()
    assert np.array_equal(a_pkg, a_orc)
    assert a_orc.size == 163 and a_orc[0] == -127 and a_orc[-1] == 127 and 0.0 in a_orc
    assert np.all(np.diff(a_orc) > 0) and np.array_equal(a_orc, -a_orc[::-1])


def test_packer_brute_force(oracle):
    r = np.random.default_rng(6)
    w = (r.standard_normal((37, 53)) * 0.03).astype(np.float32)
    w[3, 7] = 0.0
    w[5] = 0.0
    c01, q2, s = oracle.quantize_nf24_i16(w)
    alphabet = oracle.nf24_alphabet().astype(np.float64)
    base = (np.maximum(np.abs(w).max(axis=1), np.finfo(np.float32).tiny) / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, (base / np.float32(1024)).astype(np.float32))
    for n in range(w.shape[0]):
        for kk in range(w.shape[1]):
            v = np.float32(w[n, kk] / base[n])
            dist = np.abs(alphabet - np.float64(v))
            nearest = alphabet[np.flatnonzero(dist == dist.min())[0]]  # ties -> lower level
            code = int(c01[kk, n])
            q1 = code - 4 * int(nearest)
            assert -128 <= q1 <= 127
            r1 = np.float32(w[n, kk] - np.float32(np.float32(nearest) * base[n]))
            s1 = np.float32(base[n] / np.float32(4))
            assert q1 == int(np.clip(math.floor(np.float32(r1 / s1) + np.float32(0.5)), -128, 127))
    # Reconstruction: half a final step plus the decode's own fp32 rounding
    # (|w_hat| * 2^-24), except where the radix-256 digit saturates (|r2|
    # reaches base/8 = 128 final steps and is clamped to 127), which costs at
    # most one full step.
    w_hat = oracle.decode_nf24(c01, q2, s).T
    err = np.abs(w_hat.astype(np.float64) - w)
    step = s[:, None].astype(np.float64)
    rnd = np.abs(w_hat.astype(np.float64)) * 2.0 ** -23 + 1e-12
    assert np.all(err <= step + rnd)
    over = err > 0.5 * step + rnd
    assert np.all(np.abs(q2.T[over]) >= 127)
