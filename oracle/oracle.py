"""CPU oracle for the NF24 GEMM and exact SDPA paths.

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg are the only callers.  The product package never imports
this module.

Two parts:

* ``tsplat_oracle.c`` (built to ``libtsplat_oracle.so`` by the Makefile here) --
  scalar C restatements of the reference kernels, bit-identical to them;
  wrapped below with NumPy in/out.
* a NumPy restatement of the reference's NF24 packer and its NF8-derived
  alphabet (scripts/native_linear_rnf8_avx512_patch.py:14-87,
  scripts/native_linear_nf8_avx512_patch.py:12-20).

Pinning: see the header of tsplat_oracle.c and tests/test_oracle.py.  The
packer is pinned by the alphabet closed form (erfinv quantiles, each
127*level at least 1e-4 away from a rounding tie) and by brute-force
nearest-level / round-half-up checks on small matrices.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "libtsplat_oracle.so"
REF_DIR = HERE / "_ref"

_c_float_p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i = ctypes.c_int


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


_LIB = None


def lib():
    """Load (building if needed) the oracle shared library."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not ORACLE_LIB.is_file():
        import subprocess

        subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    L = ctypes.CDLL(str(ORACLE_LIB))
    L.oracle_nf24_gemm_range.argtypes = [_vp] * 6 + [_i] * 8
    L.oracle_nf24_gemm_range.restype = _i
    L.oracle_sdpa_q8t512.argtypes = [_vp] * 5 + [_i] * 7 + [ctypes.c_int64]
    L.oracle_sdpa_q8t512.restype = _i
    L.oracle_sdpa_q8t512_packed_blhd.argtypes = [_vp] * 5 + [_i] * 8
    L.oracle_sdpa_q8t512_packed_blhd.restype = _i
    L.oracle_qkv_rope_rmsnorm_pack.argtypes = [_vp] * 7 + [_i] * 6
    L.oracle_qkv_rope_rmsnorm_pack.restype = _i
    L.oracle_gemm_nf24_qkv_direct.argtypes = [_vp] * 11 + [_i] * 8
    L.oracle_gemm_nf24_qkv_direct.restype = _i
    L.oracle_exp512.argtypes = [ctypes.c_float]
    L.oracle_exp512.restype = ctypes.c_float
    L.oracle_nf24_decode.argtypes = [_i, _i, ctypes.c_float]
    L.oracle_nf24_decode.restype = ctypes.c_float
    L.oracle_reduce_add16.argtypes = [_vp]
    L.oracle_reduce_add16.restype = ctypes.c_float
    L.oracle_rope_rmsnorm64.argtypes = [_vp] * 4
    L.oracle_rope_rmsnorm64.restype = None
    L.oracle_threads.argtypes = []
    L.oracle_threads.restype = _i
    _LIB = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------
# NF24 GEMM
def nf24_gemm(x, code01_t, q2_t, scale, bias, output_start=0, output_count=None,
              require_aligned=False):
    """out[M, count] = bias + x @ decode(code01_t, q2_t, scale)[:, start:start+count].

    Restates scripts/gemm_nf24_i16_avx512.c:151-197 (status codes included).
    """
    x = _f32(x)
    code01_t = np.ascontiguousarray(code01_t, dtype=np.int16)
    q2_t = np.ascontiguousarray(q2_t, dtype=np.int8)
    scale, bias = _f32(scale), _f32(bias)
    M, K = x.shape
    N = code01_t.shape[1]
    count = N - output_start if output_count is None else output_count
    out = np.empty((M, max(count, 1)), dtype=np.float32)
    st = lib().oracle_nf24_gemm_range(_ptr(x), _ptr(code01_t), _ptr(q2_t), _ptr(scale),
                                      _ptr(bias), _ptr(out), M, K, N, output_start, count, K,
                                      out.shape[1], int(require_aligned))
    if st != 0:
        raise RuntimeError(f"oracle NF24 GEMM status {st}")
    return out


def decode_nf24(code01_t, q2_t, scale):
    """Exact fp32 decode in the [in, out] layout (prepacked.py:17-31)."""
    q = code01_t.astype(np.int32) * 256 + q2_t.astype(np.int32)
    return q.astype(np.float32) * np.asarray(scale, dtype=np.float32)[None, :]


# --------------------------------------------------------------------------
# Opt-in bf16-MFMA precision of the NF24 GEMM.  The reference has no bf16
# GEMM; its bf16 evidence is the float32 -> bfloat16 -> float32 round trip of
# scripts/triposplat_bf16_roundtrip_patch.py:27-31 (torch's conversion, round
# to nearest even), the rounding bf16_round restates.  Pinned in
# tests/test_oracle.py against torch's conversion, by the split invariants
# and by operands that are exact in bf16 (the products then need no rounding).
def bf16_round(a):
    """fp32 -> nearest bf16, ties to even, returned as fp32; Inf and NaN keep
    their upper 16 bits (scripts/native_qkv_postprocess_bf16_probe_avx512.c:11-22)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    finite = (u & 0x7F800000) != 0x7F800000
    r = np.where(finite, u + 0x7FFF + ((u >> 16) & 1), u) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(a))


def bf16_split(a):
    """(hi, lo) = (bf16(a), bf16(a - hi)); a - hi is exact in fp32."""
    a = np.asarray(a, dtype=np.float32)
    hi = bf16_round(a)
    return hi, bf16_round((a - hi).astype(np.float32))


def nf24_bf16_split_w(code01_t, q2_t, scale):
    """(wh, wl) of the bf16 modes' weights: w = fp32(p * s), the reference's
    decode of payload p = q01 * 256 + q2 and row scale s; wh = bf16(w);
    wl = bf16(fp32(p * s - wh)), the exact product minus wh rounded once to
    fp32 (the device forms it with one FMA).  p * s is exact in float64
    (24-bit by 24-bit significands) and so is p * s - wh (|p*s - wh| <=
    2^-8 |p*s|, on the product's grid)."""
    p = (np.asarray(code01_t).astype(np.int64) * 256 + np.asarray(q2_t).astype(np.int64))
    prod = p.astype(np.float64) * np.asarray(scale, np.float32).astype(np.float64)[None, :]
    wh = bf16_round(prod.astype(np.float32))
    wl = bf16_round((prod - wh.astype(np.float64)).astype(np.float32))
    return wh, wl


def nf24_gemm_bf16_terms(x, code01_t, q2_t, scale, bias, precision):
    """float64 value of bias + sum_k of the products the bf16 modes form:
    "bf16": xh*wh; "bf16x3": xh*wh + xh*wl + xl*wh (x split by bf16_split,
    w by nf24_bf16_split_w).  Products of two bf16 values are exact in fp32
    and float64, so a device result differs from this only by its fp32
    summation order."""
    if precision not in ("bf16", "bf16x3"):
        raise ValueError(precision)
    xh, xl = bf16_split(x)
    wh, wl = nf24_bf16_split_w(code01_t, q2_t, scale)
    f = lambda a: a.astype(np.float64)  # noqa: E731
    y = f(xh) @ f(wh)
    if precision == "bf16x3":
        y += f(xh) @ f(wl) + f(xl) @ f(wh)
    return y + f(np.asarray(bias, np.float32))[None, :]


def nf24_gemm_bf16_abs_terms(x, code01_t, q2_t, scale, bias, precision):
    """|bias| + sum_k |terms| of nf24_gemm_bf16_terms (for order bounds)."""
    xh, xl = bf16_split(x)
    wh, wl = nf24_bf16_split_w(code01_t, q2_t, scale)
    f = lambda a: np.abs(a.astype(np.float64))  # noqa: E731
    y = f(xh) @ f(wh)
    if precision == "bf16x3":
        y += f(xh) @ f(wl) + f(xl) @ f(wh)
    return y + f(np.asarray(bias, np.float32))[None, :]


# --------------------------------------------------------------------------
# SDPA
def sdpa_q8t512(q, k, v, key_bias=None, bias_head_stride=0):
    """Exact SDPA of scripts/native_sdpa_avx512_exact_q8t512.c:137-332.

    q [B,H,Lq,64], k/v [B,H,Lk,64]; key_bias [Lk] shared, or [H,Lk] with
    bias_head_stride=Lk (extension: one bias row per head).
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    out = np.empty((B, H, Lq, D), dtype=np.float32)
    kb = None if key_bias is None else _f32(key_bias)
    st = lib().oracle_sdpa_q8t512(_ptr(q), _ptr(k), _ptr(v), _ptr(kb), _ptr(out), B, H, Lq, Lk,
                                  D, int(kb is not None), 0 if kb is None else Lk,
                                  int(bias_head_stride))
    if st != 0:
        raise RuntimeError(f"oracle SDPA status {st}")
    return out


LOG2E_F32 = np.float32(1.4426950408889634)
SDPA_Q_SCALE_F32 = np.float32(np.float32(0.125) * LOG2E_F32)


def sdpa_bf16_terms(q, k, v, key_bias=None, precision="bf16x3"):
    """float64 reference of the opt-in bf16-MFMA SDPA modes.

    The scores are the float64 value of the terms the mode forms from
    q' = fp32(q * 0.125 * log2 e) and k ("bf16": qh.kh; "bf16x3": qh.kh +
    qh.kl + ql.kh, bf16 = nearest-even rounding, bf16_split), plus
    fp32(bias * log2 e), in log2 units; the softmax is exact (base 2) and the
    values are the mode's representation of v (vh, or vh + vl).  key_bias:
    None, [Lk] shared or [H, Lk] per head.  Returns (out [B,H,Lq,64] float64,
    s_abs [B,H,Lq] = max over keys of the sum of |terms| (+ |bias|),
    x_abs [B,H,Lq] = max over keys of |score|).  What this leaves open -- the
    fp32 summation order, exp2, the split of the unnormalised exponentials
    and the fp32 accumulation of P V -- is bounded by the caller."""
    if precision not in ("bf16", "bf16x3"):
        raise ValueError(precision)
    q, k, v = _f32(q), _f32(k), _f32(v)
    three = precision == "bf16x3"
    qs = (q * SDPA_Q_SCALE_F32).astype(np.float32)
    (qh, ql), (kh, kl), (vh, vl) = bf16_split(qs), bf16_split(k), bf16_split(v)
    f = lambda a: a.astype(np.float64)  # noqa: E731
    t = lambda a, b: a @ np.swapaxes(b, -1, -2)  # noqa: E731
    x = t(f(qh), f(kh))
    s_abs = t(np.abs(f(qh)), np.abs(f(kh)))
    if three:
        x += t(f(qh), f(kl)) + t(f(ql), f(kh))
        s_abs += t(np.abs(f(qh)), np.abs(f(kl))) + t(np.abs(f(ql)), np.abs(f(kh)))
    if key_bias is not None:
        kb = f((_f32(key_bias) * LOG2E_F32).astype(np.float32))
        kb = kb[None, None, None, :] if kb.ndim == 1 else kb[None, :, None, :]
        x = x + kb
        s_abs = s_abs + np.abs(kb)
    w = np.exp2(x - x.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    vv = f(vh) + f(vl) if three else f(vh)
    return w @ vv, s_abs.max(-1), np.abs(x).max(-1)


def sdpa_q8t512_packed_blhd(q, packed_k, packed_v, Lk, key_bias=None):
    """scripts/native_sdpa_avx512_exact_q8t512_packed.c:3-158 -> out [B,Lq,H,64]."""
    q, pk, pv = _f32(q), _f32(packed_k), _f32(packed_v)
    B, H, Lq, D = q.shape
    Lkp = pk.shape[3]
    out = np.empty((B, Lq, H, D), dtype=np.float32)
    kb = None if key_bias is None else _f32(key_bias)
    st = lib().oracle_sdpa_q8t512_packed_blhd(_ptr(q), _ptr(pk), _ptr(pv), _ptr(kb), _ptr(out), B,
                                              H, Lq, Lk, D, Lkp, int(kb is not None),
                                              0 if kb is None else Lk)
    if st != 0:
        raise RuntimeError(f"oracle packed SDPA status {st}")
    return out


def qkv_rope_rmsnorm_pack(qkv, freqs, q_gamma, k_gamma, B, L, H, L_padded=None):
    """scripts/native_qkv_postprocess_v2_avx512.c:45-105."""
    qkv, freqs = _f32(qkv), _f32(freqs)
    q_gamma, k_gamma = _f32(q_gamma), _f32(k_gamma)
    D = 64
    Lp = ((L + 15) // 16) * 16 if L_padded is None else L_padded
    fb = freqs.shape[0]
    q = np.empty((B, H, L, D), np.float32)
    pk = np.empty((B, H, D, Lp), np.float32)
    pv = np.empty((B, H, D, Lp), np.float32)
    st = lib().oracle_qkv_rope_rmsnorm_pack(_ptr(qkv), _ptr(freqs), _ptr(q_gamma), _ptr(k_gamma),
                                            _ptr(q), _ptr(pk), _ptr(pv), B, L, H, D, Lp, fb)
    if st != 0:
        raise RuntimeError(f"oracle postprocess status {st}")
    return q, pk, pv


def _selected_call(fn, q, kv, freqs, selected, q_gamma, k_gamma, B, Lq, Lk, H, Lk_padded, extra):
    q, kv, freqs = _f32(q), _f32(kv), _f32(freqs)
    q_gamma, k_gamma = _f32(q_gamma), _f32(k_gamma)
    sel = np.ascontiguousarray(selected, dtype=np.int64)
    Lp = ((Lk + 15) // 16) * 16 if Lk_padded is None else Lk_padded
    qo = np.empty((B, H, Lq, 64), np.float32)
    pk = np.empty((B, H, 64, Lp), np.float32)
    pv = np.empty((B, H, 64, Lp), np.float32)
    st = fn(_ptr(q), _ptr(kv), _ptr(freqs), _ptr(sel), _ptr(q_gamma), _ptr(k_gamma), _ptr(qo),
            _ptr(pk), _ptr(pv), B, Lq, Lk, H, 64, Lp, freqs.shape[0], *extra)
    return st, (qo, pk, pv)


def q_kv_selected_rope_rmsnorm_pack(q, kv, freqs, selected, q_gamma, k_gamma, B, Lq, Lk, H,
                                    Lk_padded=None):
    """scripts/native_qkv_postprocess_v2_avx512.c:107-191 (returns (status, outputs))."""
    fn = lib().oracle_q_kv_selected_rope_rmsnorm_pack
    fn.argtypes = [_vp] * 9 + [_i] * 7
    fn.restype = _i
    return _selected_call(fn, q, kv, freqs, selected, q_gamma, k_gamma, B, Lq, Lk, H, Lk_padded, ())


def ref_q_kv_selected(q, kv, freqs, selected, q_gamma, k_gamma, B, Lq, Lk, H, Lk_padded=None,
                      threads=0):
    fn = ref_lib("libref_qkv_postprocess_v2.so").triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2
    fn.argtypes = [_vp] * 9 + [_i] * 8
    fn.restype = _i
    return _selected_call(fn, q, kv, freqs, selected, q_gamma, k_gamma, B, Lq, Lk, H, Lk_padded,
                          (threads,))


def gemm_nf24_qkv_direct(x, code01_t, q2_t, scale, bias, freqs, q_gamma, k_gamma, B, L, H,
                         L_padded=None):
    """scripts/gemm_nf24_qkv_direct_avx512.c:87-199."""
    x = _f32(x)
    code01_t = np.ascontiguousarray(code01_t, dtype=np.int16)
    q2_t = np.ascontiguousarray(q2_t, dtype=np.int8)
    scale, bias, freqs = _f32(scale), _f32(bias), _f32(freqs)
    q_gamma, k_gamma = _f32(q_gamma), _f32(k_gamma)
    K = x.shape[1]
    N = code01_t.shape[1]
    D = 64
    Lp = ((L + 15) // 16) * 16 if L_padded is None else L_padded
    q = np.empty((B, H, L, D), np.float32)
    pk = np.empty((B, H, D, Lp), np.float32)
    pv = np.empty((B, H, D, Lp), np.float32)
    st = lib().oracle_gemm_nf24_qkv_direct(_ptr(x), _ptr(code01_t), _ptr(q2_t), _ptr(scale),
                                           _ptr(bias), _ptr(freqs), _ptr(q_gamma), _ptr(k_gamma),
                                           _ptr(q), _ptr(pk), _ptr(pv), B, L, K, N, H, D, Lp,
                                           freqs.shape[0])
    if st != 0:
        raise RuntimeError(f"oracle QKV direct status {st}")
    return q, pk, pv


def exp512(x):
    f = lib().oracle_exp512
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).reshape(-1)], np.float32)


def threads():
    return int(lib().oracle_threads())


# --------------------------------------------------------------------------
# NF24 packer (NumPy restatement).
def nf8_levels_f64():
    """The 256 NF8 levels in float64: 255 normal quantiles (p = (i+0.5)/255)
    scaled to max |level| = 1, plus a duplicate zero, sorted
    (scripts/native_linear_nf8_avx512_patch.py:12-20)."""
    from scipy.special import erfinv

    p = (np.arange(255, dtype=np.float64) + 0.5) / 255.0
    levels = math.sqrt(2.0) * erfinv(2.0 * p - 1.0)
    levels = levels / np.abs(levels).max()
    return np.sort(np.concatenate([levels, np.zeros(1)]))


def nf24_alphabet():
    """Integer alphabet unique(round(127 * codebook_f32)) clamped to +-127,
    as fp32 (native_linear_rnf8_avx512_patch.py:24)."""
    cb = nf8_levels_f64().astype(np.float32)
    scaled = cb * np.float32(127.0)
    return np.unique(np.clip(np.rint(scaled), -127, 127)).astype(np.float32)


def alphabet_tie_margin():
    """Smallest distance of any 127*level from a rounding tie (x.5)."""
    scaled = nf8_levels_f64() * 127.0
    frac = np.abs(scaled - np.floor(scaled) - 0.5)
    return float(frac.min())


def quantize_nf24_i16(weight):
    """Pack fp32 W [out, in] -> (code01_t int16 [in,out], q2_t int8 [in,out],
    scale fp32 [out]) with scale = max|w_row| / 127 / 1024.

    Restates native_linear_rnf8_avx512_patch.py:14-87 in fp32 NumPy.
    """
    w = np.ascontiguousarray(weight, dtype=np.float32)
    tiny = np.finfo(np.float32).tiny
    max_abs = np.maximum(np.abs(w).max(axis=1), np.float32(tiny)).astype(np.float32)
    base = (max_abs / np.float32(127.0)).astype(np.float32)
    alphabet = nf24_alphabet()
    mid = ((alphabet[:-1] + alphabet[1:]) * np.float32(0.5)).astype(np.float32)
    norm = (w / base[:, None]).astype(np.float32)
    q0 = alphabet[np.searchsorted(mid, norm, side="left")]
    r1 = (w - (q0 * base[:, None]).astype(np.float32)).astype(np.float32)
    s1 = (base / np.float32(4.0)).astype(np.float32)
    q1 = np.clip(np.floor((r1 / s1[:, None]).astype(np.float32) + np.float32(0.5)), -128, 127)
    q1 = q1.astype(np.float32)
    r2 = (r1 - (q1 * s1[:, None]).astype(np.float32)).astype(np.float32)
    final = (base / np.float32(1024.0)).astype(np.float32)
    q2 = np.clip(np.floor((r2 / final[:, None]).astype(np.float32) + np.float32(0.5)), -128, 127)
    code01 = (q0.astype(np.int16) * 4 + q1.astype(np.int16)).astype(np.int16)
    return (np.ascontiguousarray(code01.T), np.ascontiguousarray(q2.astype(np.int8).T),
            final.astype(np.float32))


# --------------------------------------------------------------------------
# Reference build (oracle/_ref) loaders, used to pin the oracle.
# Instruction sets the reference build is compiled for (oracle/Makefile
# REF_FLAGS); on a host without them its kernels would die on an illegal
# instruction, so they count as unavailable there.
REF_CPU_FLAGS = ("avx512f", "avx512dq", "avx512bw", "avx512vl", "fma")


def host_supports_ref():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    have = set(line.split(":", 1)[1].split())
                    return all(flag in have for flag in REF_CPU_FLAGS)
    except OSError:
        pass
    return False


def ref_available():
    return (REF_DIR / "libref_gemm_nf24_i16.so").is_file() and host_supports_ref()


def ref_lib(name):
    return ctypes.CDLL(str(REF_DIR / name))


def ref_nf24_gemm(x, code01_t, q2_t, scale, bias, threads=0, output_start=0, output_count=None,
                  tail=False):
    L = ref_lib("libref_gemm_nf24_i16.so")
    x = _f32(x)
    code01_t = np.ascontiguousarray(code01_t, dtype=np.int16)
    q2_t = np.ascontiguousarray(q2_t, dtype=np.int8)
    scale, bias = _f32(scale), _f32(bias)
    M, K = x.shape
    N = code01_t.shape[1]
    codebook = np.zeros(256, np.float32)
    if tail:
        fn = L.triposplat_gemm_rnf8_avx512_tail
        fn.argtypes = [_vp] * 10 + [_i] * 7
        out = np.empty((M, N), np.float32)
        st = fn(_ptr(x), _ptr(code01_t), _ptr(q2_t), _ptr(q2_t), _ptr(scale), _ptr(scale),
                _ptr(scale), _ptr(codebook), _ptr(bias), _ptr(out), M, K, N, K, N, threads, 3)
    else:
        count = N - output_start if output_count is None else output_count
        fn = L.triposplat_gemm_rnf8_avx512_range
        fn.argtypes = [_vp] * 10 + [_i] * 9
        out = np.empty((M, count), np.float32)
        st = fn(_ptr(x), _ptr(code01_t), _ptr(q2_t), _ptr(q2_t), _ptr(scale), _ptr(scale),
                _ptr(scale), _ptr(codebook), _ptr(bias), _ptr(out), M, K, N, output_start, count,
                K, count, threads, 3)
    if st != 0:
        raise RuntimeError(f"reference GEMM status {st}")
    return out


def ref_sdpa_q8t512(q, k, v, key_bias=None, threads=0):
    L = ref_lib("libref_sdpa_q8t512.so")
    fn = L.triposplat_sdpa_f32_avx512_exact_q8t512
    fn.argtypes = [_vp] * 5 + [_i] * 8
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    out = np.empty_like(q)
    kb = None if key_bias is None else _f32(key_bias)
    st = fn(_ptr(q), _ptr(k), _ptr(v), _ptr(kb), _ptr(out), B, H, Lq, Lk, D, int(kb is not None),
            0 if kb is None else kb.size, threads)
    if st != 0:
        raise RuntimeError(f"reference SDPA status {st}")
    return out


def ref_sdpa_packed_blhd(q, packed_k, packed_v, Lk, key_bias=None, threads=0):
    L = ref_lib("libref_sdpa_q8t512_packed.so")
    fn = L.triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd
    fn.argtypes = [_vp] * 5 + [_i] * 9
    q, pk, pv = _f32(q), _f32(packed_k), _f32(packed_v)
    B, H, Lq, D = q.shape
    out = np.empty((B, Lq, H, D), np.float32)
    kb = None if key_bias is None else _f32(key_bias)
    st = fn(_ptr(q), _ptr(pk), _ptr(pv), _ptr(kb), _ptr(out), B, H, Lq, Lk, D, pk.shape[3],
            int(kb is not None), 0 if kb is None else kb.size, threads)
    if st != 0:
        raise RuntimeError(f"reference packed SDPA status {st}")
    return out


def ref_qkv_postprocess_v2(qkv, freqs, q_gamma, k_gamma, B, L, H, threads=0):
    Lib = ref_lib("libref_qkv_postprocess_v2.so")
    fn = Lib.triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2
    fn.argtypes = [_vp] * 7 + [_i] * 7
    qkv, freqs = _f32(qkv), _f32(freqs)
    q_gamma, k_gamma = _f32(q_gamma), _f32(k_gamma)
    Lp = ((L + 15) // 16) * 16
    q = np.empty((B, H, L, 64), np.float32)
    pk = np.empty((B, H, 64, Lp), np.float32)
    pv = np.empty((B, H, 64, Lp), np.float32)
    st = fn(_ptr(qkv), _ptr(freqs), _ptr(q_gamma), _ptr(k_gamma), _ptr(q), _ptr(pk), _ptr(pv), B,
            L, H, 64, Lp, freqs.shape[0], threads)
    if st != 0:
        raise RuntimeError(f"reference postprocess status {st}")
    return q, pk, pv


def ref_gemm_nf24_qkv_direct(x, code01_t, q2_t, scale, bias, freqs, q_gamma, k_gamma, B, L, H,
                             threads=0):
    Lib = ref_lib("libref_gemm_nf24_qkv_direct.so")
    fn = Lib.triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512
    fn.argtypes = [_vp] * 15 + [_i] * 10
    x = _f32(x)
    code01_t = np.ascontiguousarray(code01_t, dtype=np.int16)
    q2_t = np.ascontiguousarray(q2_t, dtype=np.int8)
    scale, bias, freqs = _f32(scale), _f32(bias), _f32(freqs)
    q_gamma, k_gamma = _f32(q_gamma), _f32(k_gamma)
    K = x.shape[1]
    N = code01_t.shape[1]
    Lp = ((L + 15) // 16) * 16
    cb = np.zeros(256, np.float32)
    q = np.empty((B, H, L, 64), np.float32)
    pk = np.empty((B, H, 64, Lp), np.float32)
    pv = np.empty((B, H, 64, Lp), np.float32)
    st = fn(_ptr(x), _ptr(code01_t), _ptr(q2_t), _ptr(q2_t), _ptr(scale), _ptr(scale),
            _ptr(scale), _ptr(cb), _ptr(bias), _ptr(freqs), _ptr(q_gamma), _ptr(k_gamma), _ptr(q),
            _ptr(pk), _ptr(pv), B, L, K, N, H, 64, Lp, freqs.shape[0], threads, 3)
    if st != 0:
        raise RuntimeError(f"reference QKV direct status {st}")
    return q, pk, pv


# --------------------------------------------------------------------------
# The reference's elementwise AVX-512 kernels (oracle/_ref), used by the
# reference backend of flow_ref.CpuFlow so the CPU baseline of the model-level
# configurations is the repository's own AVX-512 pipeline.
_REF_EW = {}


def _ref_ew(lib_name, sym, argtypes):
    key = (lib_name, sym)
    if key not in _REF_EW:
        fn = getattr(ref_lib(lib_name), sym)
        fn.argtypes = argtypes
        fn.restype = _i
        _REF_EW[key] = fn
    return _REF_EW[key]


_i64t = ctypes.c_int64


def ref_layernorm(x, eps, weight=None, bias=None, threads=0):
    """scripts/native_norm_rope_avx512.c:13-49 (rows x cols, optional affine)."""
    x = _f32(x)
    out = np.empty_like(x)
    cols = x.shape[-1]
    fn = _ref_ew("libref_norm_rope.so", "triposplat_layernorm_f32_avx512",
                 [_vp] * 4 + [_i64t, _i, ctypes.c_float, _i, _i])
    w = None if weight is None else _f32(weight)
    b = None if bias is None else _f32(bias)
    st = fn(_ptr(x), _ptr(w), _ptr(b), _ptr(out), x.size // cols, cols, float(eps), int(w is not None), threads)
    if st != 0:
        raise RuntimeError(f"reference layernorm status {st}")
    return out


def ref_multihead_rmsnorm(x, gamma, eps=1e-12, threads=0):
    """native_norm_rope_avx512.c:51-83: x [..., H, D] * sqrt(D)/max(||x||, eps) * gamma[H, D]."""
    x = _f32(x)
    gamma = _f32(gamma)
    H, D = gamma.shape
    out = np.empty_like(x)
    fn = _ref_ew("libref_norm_rope.so", "triposplat_multihead_rmsnorm_f32_avx512",
                 [_vp] * 3 + [_i64t, _i, _i, ctypes.c_float, _i])
    st = fn(_ptr(x), _ptr(gamma), _ptr(out), x.size // (H * D), H, D, float(eps), threads)
    if st != 0:
        raise RuntimeError(f"reference rmsnorm status {st}")
    return out


def ref_modulate_inplace(h, scale, shift, threads=0):
    """native_block_elementwise_avx512.c:9-22: h[b] = h[b] * (1 + scale[b]) + shift[b]."""
    B, L, C = h.shape
    fn = _ref_ew("libref_block_elementwise.so", "triposplat_modulate_inplace_f32_avx512",
                 [_vp] * 3 + [_i] * 4)
    sc, sh = _f32(scale), _f32(shift)
    st = fn(_ptr(h), _ptr(sc), _ptr(sh), B, L, C, threads)
    if st != 0:
        raise RuntimeError(f"reference modulate status {st}")
    return h


def ref_gated_residual_inplace(x, h, gate, threads=0):
    """native_block_elementwise_avx512.c:24-35: h *= gate; x += h."""
    B, L, C = x.shape
    fn = _ref_ew("libref_block_elementwise.so", "triposplat_gated_residual_inplace_f32_avx512",
                 [_vp] * 3 + [_i] * 4)
    g = _f32(gate)
    st = fn(_ptr(x), _ptr(h), _ptr(g), B, L, C, threads)
    if st != 0:
        raise RuntimeError(f"reference gated residual status {st}")
    return x


def ref_add_inplace(x, d, threads=0):
    fn = _ref_ew("libref_block_elementwise.so", "triposplat_add_inplace_f32_avx512", [_vp, _vp, _i64t, _i])
    d = _f32(d)
    st = fn(_ptr(x), _ptr(d), x.size, threads)
    if st != 0:
        raise RuntimeError(f"reference add status {st}")
    return x


def ref_gelu_tanh(x, threads=0):
    x = _f32(x)
    out = np.empty_like(x)
    fn = _ref_ew("libref_activations.so", "triposplat_gelu_tanh_f32_avx512", [_vp, _vp, _i64t, _i])
    st = fn(_ptr(x), _ptr(out), x.size, threads)
    if st != 0:
        raise RuntimeError(f"reference gelu status {st}")
    return out


def ref_silu(x, threads=0):
    x = _f32(x)
    out = np.empty_like(x)
    fn = _ref_ew("libref_activations.so", "triposplat_silu_f32_avx512", [_vp, _vp, _i64t, _i])
    st = fn(_ptr(x), _ptr(out), x.size, threads)
    if st != 0:
        raise RuntimeError(f"reference silu status {st}")
    return out


def ref_cfg_euler(z, v_pos, v_neg, guidance, dt, threads=0):
    """native_sampler_avx512.c:19-89: v = g*v_pos - (g-1)*v_neg; z -= dt*v."""
    pos = _f32(v_pos).copy()
    neg = _f32(v_neg)
    g = np.array([guidance], np.float32)
    fn = _ref_ew("libref_sampler.so", "triposplat_cfg_combine_inplace_f32_avx512", [_vp] * 3 + [_i, _i64t, _i])
    st = fn(_ptr(pos), _ptr(neg), _ptr(g), 1, pos.size, threads)
    if st != 0:
        raise RuntimeError(f"reference cfg status {st}")
    out = _f32(z).copy()
    d = np.array([dt], np.float32)
    fn = _ref_ew("libref_sampler.so", "triposplat_euler_update_inplace_f32_avx512", [_vp] * 3 + [_i, _i64t, _i])
    st = fn(_ptr(out), _ptr(pos), _ptr(d), 1, out.size, threads)
    if st != 0:
        raise RuntimeError(f"reference euler status {st}")
    return out, pos


# --------------------------------------------------------------------------
# Flow-block and sampler elementwise ops: the oracle restatements
# (tsplat_oracle.c, backend="oracle") and the reference build
# (oracle/_ref, backend="reference") behind one calling convention -- the
# reference's C argument list without the trailing `threads`.
_EW_OPS = {
    "layernorm": ("libref_norm_rope.so", "triposplat_layernorm_f32_avx512",
                  [_vp] * 4 + [ctypes.c_int64, _i, ctypes.c_float, _i]),
    "multihead_rmsnorm": ("libref_norm_rope.so", "triposplat_multihead_rmsnorm_f32_avx512",
                          [_vp] * 3 + [ctypes.c_int64, _i, _i, ctypes.c_float]),
    "rope_complex": ("libref_norm_rope.so", "triposplat_rope_complex_f32_avx512",
                     [_vp] * 3 + [ctypes.c_int64, _i]),
    "modulate_inplace": ("libref_block_elementwise.so", "triposplat_modulate_inplace_f32_avx512",
                         [_vp] * 3 + [_i] * 3),
    "gated_residual_inplace": ("libref_block_elementwise.so",
                               "triposplat_gated_residual_inplace_f32_avx512", [_vp] * 3 + [_i] * 3),
    "add_inplace": ("libref_block_elementwise.so", "triposplat_add_inplace_f32_avx512",
                    [_vp] * 2 + [ctypes.c_int64]),
    "gelu_tanh": ("libref_activations.so", "triposplat_gelu_tanh_f32_avx512", [_vp] * 2 + [ctypes.c_int64]),
    "silu": ("libref_activations.so", "triposplat_silu_f32_avx512", [_vp] * 2 + [ctypes.c_int64]),
    "cfg_combine_inplace": ("libref_sampler.so", "triposplat_cfg_combine_inplace_f32_avx512",
                            [_vp] * 3 + [_i, ctypes.c_int64]),
    "euler_update_inplace": ("libref_sampler.so", "triposplat_euler_update_inplace_f32_avx512",
                             [_vp] * 3 + [_i, ctypes.c_int64]),
    "ab2_update_inplace": ("libref_sampler.so", "triposplat_ab2_update_inplace_f32_avx512",
                           [_vp] * 5 + [_i, ctypes.c_int64]),
}
EW_OPS = tuple(_EW_OPS)
_EW_FNS = {}


def _ew_fn(op, backend):
    key = (op, backend)
    if key not in _EW_FNS:
        lib_name, sym, argtypes = _EW_OPS[op]
        if backend == "oracle":
            fn = getattr(lib(), "oracle_" + op)
            fn.argtypes = argtypes
        elif backend == "reference":
            fn = getattr(ref_lib(lib_name), sym)
            fn.argtypes = argtypes + [_i]
        else:
            raise ValueError(backend)
        fn.restype = _i
        _EW_FNS[key] = fn
    return _EW_FNS[key]


def ew(op, *args, backend="oracle", threads=0):
    """Run one block/sampler op in place on NumPy arrays and return its status.

    ``args`` follow the reference's C signature without ``threads``: arrays
    (contiguous fp32, None for a null pointer) then the integer / float
    arguments.  Outputs are written into the arrays passed.
    """
    conv = []
    for a in args:
        if isinstance(a, np.ndarray):
            if a.dtype != np.float32 or not a.flags.c_contiguous:
                raise ValueError("ew arrays must be contiguous float32")
            conv.append(_ptr(a))
        else:
            conv.append(a)
    fn = _ew_fn(op, backend)
    return int(fn(*conv, threads) if backend == "reference" else fn(*conv))
