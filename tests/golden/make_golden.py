#!/usr/bin/env python3
"""Write the golden fixtures in this folder from the reference's own kernels.

Runs only where the reference sources are mounted: `make -C oracle` compiles
them (scripts/gemm_nf24_i16_avx512.c + _tail.c,
native_sdpa_avx512_exact_q8t512.c, native_sdpa_avx512_exact_q8t512_packed.c,
native_qkv_postprocess_v2_avx512.c, gemm_nf24_qkv_direct_avx512.c, and the
block / sampler elementwise kernels) into oracle/_ref/, and this script calls
those builds through ctypes on small seeded inputs.  `make_golden.py NAME...`
rewrites only the named fixtures.  Each .npz holds the inputs and the reference's outputs; the
tests check the oracle against them bit for bit.  The weight codes come from
the oracle's NumPy packer (a fixture input, not a reference output).
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "oracle"))
import oracle as O  # noqa: E402


def linear_inputs(seed, M, K, N):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K), dtype=np.float32) * np.float32(0.03)).astype(np.float32)
    b = (r.standard_normal(N, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    c01, q2, s = O.quantize_nf24_i16(w)
    return x, c01, q2, s, b


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref is not built (needs the reference sources): make -C oracle")
    out = {}
    # NF24 GEMM: the reference smoke shape, the N=5 tail, and a range call.
    x, c01, q2, s, b = linear_inputs(22, 25, 96, 64)
    out["gemm_25x96x64"] = dict(x=x, code01_t=c01, q2_t=q2, scale=s, bias=b,
                                out=O.ref_nf24_gemm(x, c01, q2, s, b, threads=2))
    x, c01, q2, s, b = linear_inputs(27, 3, 96, 5)
    out["gemm_tail_3x96x5"] = dict(x=x, code01_t=c01, q2_t=q2, scale=s, bias=b,
                                   out=O.ref_nf24_gemm(x, c01, q2, s, b, threads=2, tail=True))
    x, c01, q2, s, b = linear_inputs(31, 40, 96, 64)
    out["gemm_range_40x96x64_s16_c32"] = dict(
        x=x, code01_t=c01, q2_t=q2, scale=s, bias=b, start=np.int32(16), count=np.int32(32),
        out=O.ref_nf24_gemm(x, c01, q2, s, b, threads=2, output_start=16, output_count=32))

    # SDPA: scripts/smoke_custom_sdpa_backend.py cases + a 512-key tile crossing.
    def qkv(seed, B, H, Lq, Lk):
        r = np.random.default_rng(seed)
        return (r.standard_normal((B, H, Lq, 64), dtype=np.float32),
                r.standard_normal((B, H, Lk, 64), dtype=np.float32),
                r.standard_normal((B, H, Lk, 64), dtype=np.float32))

    q, k, v = qkv(11, 1, 2, 16, 16)
    out["sdpa_self_16"] = dict(q=q, k=k, v=v, out=O.ref_sdpa_q8t512(q, k, v, None, 2))
    q, k, v = qkv(12, 1, 2, 17, 17)
    bias = np.zeros(17, np.float32)
    bias[0] = np.float32(math.log(7.0))
    out["sdpa_masked_17_log7"] = dict(q=q, k=k, v=v, key_bias=bias, out=O.ref_sdpa_q8t512(q, k, v, bias, 2))
    q, k, v = qkv(13, 1, 2, 15, 19)
    out["sdpa_cross_15x19"] = dict(q=q, k=k, v=v, out=O.ref_sdpa_q8t512(q, k, v, None, 2))
    q, k, v = qkv(14, 1, 1, 9, 530)
    bias = np.random.default_rng(15).uniform(-2.0, 0.0, 530).astype(np.float32)
    out["sdpa_bias_9x530"] = dict(q=q, k=k, v=v, key_bias=bias, out=O.ref_sdpa_q8t512(q, k, v, bias, 2))

    # packed K/V with BLHD output
    q, k, v = qkv(16, 1, 2, 15, 19)
    pk = np.zeros((1, 2, 64, 32), np.float32)
    pv = np.zeros_like(pk)
    pk[..., :19] = k.transpose(0, 1, 3, 2)
    pv[..., :19] = v.transpose(0, 1, 3, 2)
    out["sdpa_packed_blhd_15x19"] = dict(q=q, packed_k=pk, packed_v=pv, lk=np.int32(19),
                                         out=O.ref_sdpa_packed_blhd(q, pk, pv, 19, None, 2))

    # QKV postprocess v2 and fused QKV direct
    r = np.random.default_rng(17)
    B, L, H = 2, 20, 2
    qkv_in = r.standard_normal((B * L, 3 * H * 64), dtype=np.float32)
    ang = r.standard_normal((B, L, H, 32)).astype(np.float32)
    fr = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(B, L, H, 64).astype(np.float32)
    qg = (r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32)
    kg = (r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32)
    qo, pko, pvo = O.ref_qkv_postprocess_v2(qkv_in, fr, qg, kg, B, L, H, 2)
    out["qkv_postprocess_2x20x2"] = dict(qkv=qkv_in, freqs=fr, q_gamma=qg, k_gamma=kg, q=qo,
                                         packed_k=pko, packed_v=pvo)
    B, L, H = 1, 17, 2
    x, c01, q2, s, b = linear_inputs(18, B * L, 128, 3 * H * 64)
    ang = np.random.default_rng(19).standard_normal((1, L, H, 32)).astype(np.float32)
    fr = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(1, L, H, 64).astype(np.float32)
    qo, pko, pvo = O.ref_gemm_nf24_qkv_direct(x, c01, q2, s, b, fr, qg, kg, B, L, H, 2)
    out["qkv_direct_1x17x2_k128"] = dict(x=x, code01_t=c01, q2_t=q2, scale=s, bias=b, freqs=fr,
                                         q_gamma=qg, k_gamma=kg, q=qo, packed_k=pko, packed_v=pvo)

    # selected-rows postprocess (the final block's latent queries), one index out of order
    r = np.random.default_rng(23)
    B, Lq, Lk, H = 2, 21, 37, 2
    C = H * 64
    qsel = r.standard_normal((B, Lq, C), dtype=np.float32)
    kv = r.standard_normal((B, Lk, 2 * C), dtype=np.float32)
    ang = r.standard_normal((B, Lk, H, 32)).astype(np.float32)
    fr = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(B, Lk, H, 64).astype(np.float32)
    sel = np.concatenate([np.arange(Lq - 1), [Lk - 1]]).astype(np.int64)
    qg = (r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32)
    kg = (r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32)
    st, (qo, pko, pvo) = O.ref_q_kv_selected(qsel, kv, fr, sel, qg, kg, B, Lq, Lk, H, threads=2)
    assert st == 0
    out["qkv_selected_2x21x37"] = dict(q=qsel, kv=kv, freqs=fr, selected=sel, q_gamma=qg, k_gamma=kg,
                                       q_out=qo, packed_k=pko, packed_v=pvo)

    ew = ew_fixture()
    out["ew_ops"] = ew
    only = set(sys.argv[1:])
    for name, arrays in out.items():
        if only and name not in only:
            continue
        np.savez(HERE / f"{name}.npz", **arrays)
        print(name, len(arrays), "arrays")


def ew_fixture():
    """Flow-block / sampler ops (tests/_ew_cases.py) through the reference
    build: keys '<case>/in/<array>' and '<case>/out/<array>'."""
    sys.path.insert(0, str(HERE.parent))
    import _ew_cases as EC

    arrays = {}
    for name, case in EC.cases().items():
        for k, v in case[1].items():
            arrays[f"{name}/in/{k}"] = v
        got = EC.run(O, case, backend="reference")
        for k in case[3]:
            arrays[f"{name}/out/{k}"] = got[k]
    return arrays


if __name__ == "__main__":
    main()
