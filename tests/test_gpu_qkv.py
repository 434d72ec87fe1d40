"""GPU parity of the QKV postprocess (RoPE -> RMSNorm -> pack), the fused NF24
QKV projection and the device NF24 packer, against the oracle.

Postprocess (full-sequence and selected-rows forms): the device repeats
scripts/native_qkv_postprocess_v2_avx512.c's arithmetic in its lane order
(fmaf RoPE, the 16-lane fma chains and reduce tree of ||y||^2), so outputs
must be bit-identical to the oracle and the reference fixtures.
Fused projection: the GEMM part is bounded as in test_gpu_gemm; RMSNorm maps
an input perturbation dx to |dy| <= 8 * ||dx|| / ||x|| * max|gamma|; the
fused epilogue equals GEMM + postprocess bit for bit.
Packer: integer codes and scales must be bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import gemm_order_bound

pytestmark = pytest.mark.gpu
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _freqs(B, L, H, seed):
    ang = np.random.default_rng(seed).standard_normal((B, L, H, 32)).astype(np.float32)
    return np.stack([np.cos(ang), np.sin(ang)], -1).reshape(B, L, H, 64).astype(np.float32)


def _gammas(H, seed):
    r = np.random.default_rng(seed)
    return ((r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32),
            (r.standard_normal((H, 64)) * 0.05 + 1.0).astype(np.float32))


@pytest.mark.parametrize("B,L,H,fb", [(1, 37, 2, 1), (2, 20, 3, 2), (1, 130, 16, 1), (2, 64, 4, 1)])
def test_qkv_postprocess(oracle, cuda, B, L, H, fb):
    import torch
    from tsplat.qkv import qkv_rope_rmsnorm_pack

    C = H * 64
    qkv = np.random.default_rng(L).standard_normal((B * L, 3 * C), dtype=np.float32)
    fr = _freqs(fb, L, H, 3)
    qg, kg = _gammas(H, 4)
    t = lambda a: torch.from_numpy(a).to(cuda)
    got = qkv_rope_rmsnorm_pack(t(qkv), t(fr), t(qg), t(kg), B, L, H)
    ref = oracle.qkv_rope_rmsnorm_pack(qkv, fr, qg, kg, B, L, H)
    for g, r_ in zip(got, ref):
        g = g.cpu().numpy()
        assert g.shape == r_.shape
        assert np.array_equal(g.view(np.uint32), r_.view(np.uint32))
    Lp = ref[1].shape[-1]
    if Lp > L:
        assert not got[1].cpu().numpy()[..., L:].any()


@pytest.mark.parametrize("B,L,H,fb,Lp", [(2, 45, 2, 2, None), (1, 17, 4, 1, None), (3, 20, 2, 1, 64),
                                         (2, 61, 3, 1, None)])
def test_qkv_direct(oracle, cuda, B, L, H, fb, Lp):
    """The fused projection (RoPE, RMSNorm and the packed stores in the GEMM
    epilogue) against the oracle's projection + postprocess; covers rows of
    two sequences in one tile, L % 4 != 0 (scalar packed stores), a padded
    length beyond roundup16(L) (tail-zero kernel) and a tiny M."""
    import torch
    from tsplat.qkv import gemm_nf24_qkv_direct

    print(f"qkv_direct B={B} L={L} H={H} fb={fb} Lp={Lp}", flush=True)
    C = H * 64
    r = np.random.default_rng(8 + L)
    x = r.standard_normal((B * L, C), dtype=np.float32)
    w = (r.standard_normal((3 * C, C)) * 0.03).astype(np.float32)
    b = (r.standard_normal(3 * C) * 0.01).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    fr = _freqs(fb, L, H, 5)
    qg, kg = _gammas(H, 6)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    got = gemm_nf24_qkv_direct(t(x), t(c01), t(q2), t(s), t(b), t(fr), t(qg), t(kg), B, L, H,
                               L_padded=Lp)
    ref = oracle.gemm_nf24_qkv_direct(x, c01, q2, s, b, fr, qg, kg, B, L, H)
    if Lp is not None:
        assert not got[1].cpu().numpy()[..., L:].any() and not got[2].cpu().numpy()[..., L:].any()
    proj = oracle.nf24_gemm(x, c01, q2, s, b)
    bound = gemm_order_bound(x, oracle.decode_nf24(c01, q2, s), b)  # [B*L, 3C]
    for which, (g, r_) in enumerate(zip(got, ref)):
        g = g.cpu().numpy()
        part = slice(which * C, (which + 1) * C)
        xb = bound[:, part].reshape(B, L, H, 64)
        xn = np.linalg.norm(proj[:, part].reshape(B, L, H, 64).astype(np.float64), axis=-1)
        if which < 2:
            tol = 8.0 * np.linalg.norm(xb, axis=-1) / xn * 1.2 + 1e-5   # [B, L, H]
            tol = tol.transpose(0, 2, 1)[..., None]                      # [B, H, L, 1]
        else:
            tol = xb.transpose(0, 2, 1, 3)                                # [B, H, L, 64]
        if which == 0:
            d = np.abs(g - r_)
        else:
            d = np.abs(g[..., :L] - r_[..., :L]).transpose(0, 1, 3, 2)   # -> [B, H, L, 64]
        assert np.all(d <= tol), (which, float(d.max()))


@pytest.mark.parametrize("B,L,H,fb", [(1, 16384, 16, 1), (1, 4096, 16, 1), (2, 300, 4, 2), (3, 257, 2, 1),
                                     (1, 5000, 16, 1), (1, 8194, 16, 1), (1, 3000, 16, 1),
                                     (1, 18432, 16, 1),   # split into whole-round row launches
                                     (1, 2048, 16, 1), (1, 16385, 16, 1), (1, 2200, 16, 1),
                                     (1, 2600, 16, 1)])
def test_qkv_fused_matches_unfused(oracle, cuda, B, L, H, fb):
    """Fused epilogue == NF24 GEMM then the postprocess kernel, at shapes that
    route to each tile configuration (256x256: L=16384, 5000, 16385 (plus its
    1-row tail); 256x192: L=4096, 3000, 8194 (plus its 2-row tail); 256x128:
    L=2200; 128x128: L=2600; 128x64: L=2048, the last 2048 rows of L=18432
    and the small shapes), with partial row tiles and odd L.
    Both paths run the same GEMM main loop and the same postprocess
    arithmetic, so all three outputs are bit-identical."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct, qkv_rope_rmsnorm_pack

    print(f"qkv fused vs unfused B={B} L={L} H={H}", flush=True)
    C = H * 64
    g = torch.Generator(device=cuda).manual_seed(L)
    x = torch.randn((B * L, 1024), generator=g, device=cuda)
    w = torch.randn((3 * C, 1024), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    fr = torch.from_numpy(_freqs(fb, L, H, 7)).to(cuda)
    qg, kg = (torch.from_numpy(a).to(cuda) for a in _gammas(H, 9))
    fused = gemm_nf24_qkv_direct(x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H)
    proj = nf24_linear(x, codes[0], codes[1], scales[0], bias)
    unfused = qkv_rope_rmsnorm_pack(proj, fr, qg, kg, B, L, H)
    torch.cuda.synchronize(cuda)
    for a_, b_ in zip(fused, unfused):
        assert bool(torch.isfinite(a_).all())
        assert torch.equal(a_, b_)


@pytest.mark.parametrize("B,L,H", [(1, 16384, 16), (2, 300, 4), (3, 257, 2), (1, 5000, 16), (1, 18432, 16)])
def test_qkv_direct_bhld_layout(cuda, B, L, H):
    """kv_layout="bhld": the same epilogue arithmetic storing k and v
    [B, H, L, 64] like q -- bit-identical to the packed outputs transposed
    (and q unchanged), at shapes routed to each tile configuration."""
    import torch
    from tsplat.nf24 import quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct

    print(f"qkv direct bhld B={B} L={L} H={H}", flush=True)
    C = H * 64
    g = torch.Generator(device=cuda).manual_seed(L + 1)
    x = torch.randn((B * L, 1024), generator=g, device=cuda)
    w = torch.randn((3 * C, 1024), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    fr = torch.from_numpy(_freqs(1, L, H, 11)).to(cuda)
    qg, kg = (torch.from_numpy(a).to(cuda) for a in _gammas(H, 12))
    args = (x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H)
    q0, pk, pv = gemm_nf24_qkv_direct(*args)
    q1, k1, v1 = gemm_nf24_qkv_direct(*args, kv_layout="bhld")
    torch.cuda.synchronize(cuda)
    assert k1.shape == (B, H, L, 64) and v1.shape == (B, H, L, 64)
    assert torch.equal(q0, q1)
    assert torch.equal(k1, pk[..., :L].transpose(2, 3))
    assert torch.equal(v1, pv[..., :L].transpose(2, 3))
    for p_ in ("bf16x3",):
        qb, kb, vb = gemm_nf24_qkv_direct(*args, kv_layout="bhld", precision=p_)
        _, pkb, pvb = gemm_nf24_qkv_direct(*args, precision=p_)
        torch.cuda.synchronize(cuda)
        assert torch.equal(kb, pkb[..., :L].transpose(2, 3)) and torch.equal(vb, pvb[..., :L].transpose(2, 3))


@pytest.mark.parametrize("symbol", ["triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2",
                                    "triposplat_qkv_rope_rmsnorm_pack_f32_avx512"])
def test_qkv_postprocess_golden(oracle, cuda, hiplib, symbol):
    """The reference's own outputs (tests/golden) through the reference-named
    blocking symbols (the second version and the first, which zeroed all of
    packed k/v), bit for bit; outputs start as NaN, so the padding tokens
    must be written as zeros."""
    import torch

    g = np.load(GOLDEN / "qkv_postprocess_2x20x2.npz")
    d = {k: torch.from_numpy(np.ascontiguousarray(g[k])).to(cuda) for k in g.files}
    q, pk, pv = (torch.full_like(d[k], float("nan")) for k in ("q", "packed_k", "packed_v"))
    assert getattr(hiplib, symbol)(
        d["qkv"].data_ptr(), d["freqs"].data_ptr(), d["q_gamma"].data_ptr(), d["k_gamma"].data_ptr(),
        q.data_ptr(), pk.data_ptr(), pv.data_ptr(), 2, 20, 2, 64, int(pk.shape[-1]),
        int(g["freqs"].shape[0]), 0) == 0
    for got, key in ((q, "q"), (pk, "packed_k"), (pv, "packed_v")):
        diff = int((got.cpu().numpy().view(np.uint32) != g[key].view(np.uint32)).sum())
        assert diff == 0, (key, diff)


@pytest.mark.parametrize("B,Lq,Lk,H,fb,Lkp", [(2, 21, 37, 2, 2, None), (1, 130, 200, 4, 1, 256),
                                            (1, 8193, 8194, 16, 1, None)])
def test_qkv_selected_rows(oracle, cuda, hiplib, B, Lq, Lk, H, fb, Lkp):
    """triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2 and its async
    form against the oracle bit for bit (the last case: the reference's final
    block, 8193 latent queries over 8194 keys); an index outside [0, Lk) is
    -3 from the blocking symbol and an all-zero q row from the async one."""
    import torch

    print(f"qkv selected B={B} Lq={Lq} Lk={Lk} H={H}", flush=True)
    r = np.random.default_rng(Lq + Lk)
    C = H * 64
    q = r.standard_normal((B, Lq, C), dtype=np.float32)
    kv = r.standard_normal((B, Lk, 2 * C), dtype=np.float32)
    fr = _freqs(fb, Lk, H, 11)
    sel = np.sort(r.choice(Lk, Lq, replace=False)).astype(np.int64)
    qg, kg = _gammas(H, 12)
    st, ref = oracle.q_kv_selected_rope_rmsnorm_pack(q, kv, fr, sel, qg, kg, B, Lq, Lk, H, Lkp)
    assert st == 0
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    d = [t(a) for a in (q, kv, fr, sel, qg, kg)]
    Lp = ref[1].shape[-1]
    outs = [torch.full((B, H, Lq, 64), float("nan"), device=cuda),
            torch.full((B, H, 64, Lp), float("nan"), device=cuda),
            torch.full((B, H, 64, Lp), float("nan"), device=cuda)]
    args = [a.data_ptr() for a in d] + [o.data_ptr() for o in outs] + [B, Lq, Lk, H, 64, Lp, fb]
    assert hiplib.triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2(*args, 0) == 0
    for got, exp in zip(outs, ref):
        assert np.array_equal(got.cpu().numpy().view(np.uint32), exp.view(np.uint32))
    bad = sel.copy()
    bad[min(3, Lq - 1)] = Lk
    d[3] = t(bad)
    args[3] = d[3].data_ptr()
    assert hiplib.triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2(*args, 0) == -3
    assert hiplib.tsplat_q_kv_selected_postprocess_async(
        *args, 0, torch.cuda.current_stream(cuda).cuda_stream) == 0
    torch.cuda.synchronize(cuda)
    qo = outs[0].cpu().numpy()
    row = min(3, Lq - 1)
    assert not qo[:, :, row].any()
    keep = [i for i in range(Lq) if i != row]
    assert np.array_equal(qo[:, :, keep].view(np.uint32), ref[0][:, :, keep].view(np.uint32))


@pytest.mark.parametrize("out_f,in_f", [(64, 96), (17, 64), (3072, 1024), (5, 1024), (100, 33)])
def test_device_packer_bit_exact(oracle, cuda, out_f, in_f):
    import torch
    from tsplat.nf24 import quantize_nf24_i16_per_output_channel

    w = (np.random.default_rng(out_f + in_f).standard_normal((out_f, in_f)) * 0.03).astype(np.float32)
    w[0, :] = 0.0  # an all-zero row (scale from FLT_MIN)
    codes, scales, err = quantize_nf24_i16_per_output_channel(torch.from_numpy(w).to(cuda))
    c01, q2, s = oracle.quantize_nf24_i16(w)
    assert np.array_equal(codes[0].cpu().numpy(), c01)
    assert np.array_equal(codes[1].cpu().numpy(), q2)
    assert np.array_equal(scales[0].cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert err["weight_rmse"] < 1e-6 and err["nf8_derived_alphabet_size"] == 163


@pytest.mark.parametrize("mode", ["k", "v", "kv"])
def test_kv_bf16_round_probe(oracle, cuda, hiplib, mode):
    """The bf16 K/V sensitivity probe (native_qkv_postprocess_bf16_probe_avx512.c):
    with kv_round=mode, every postprocess form stores k and/or v as the
    nearest bf16 of the exact value -- the oracle's exact outputs passed
    through oracle.bf16_round, bit for bit -- and q and the unselected
    operand stay exact; the fused projection equals GEMM + postprocess.
    The mode is per call: a call without it right after stays exact."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct, q_kv_selected_rope_rmsnorm_pack, qkv_rope_rmsnorm_pack

    print(f"kv bf16 round mode={mode}", flush=True)
    B, L, H = 2, 37, 3
    C = H * 64
    r = np.random.default_rng(77)
    qkv = r.standard_normal((B * L, 3 * C), dtype=np.float32)
    fr = _freqs(1, L, H, 13)
    qg, kg = _gammas(H, 14)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    exact = oracle.qkv_rope_rmsnorm_pack(qkv, fr, qg, kg, B, L, H)
    rk, rv = "k" in mode, "v" in mode
    want = (exact[0], oracle.bf16_round(exact[1]) if rk else exact[1],
            oracle.bf16_round(exact[2]) if rv else exact[2])
    assert not np.array_equal(want[1 if rk else 2], exact[1 if rk else 2])   # the rounding is visible
    got = qkv_rope_rmsnorm_pack(t(qkv), t(fr), t(qg), t(kg), B, L, H, kv_round=mode)
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_.cpu().numpy().view(np.uint32), w_.view(np.uint32))
    plain = qkv_rope_rmsnorm_pack(t(qkv), t(fr), t(qg), t(kg), B, L, H)
    for g_, w_ in zip(plain, exact):
        assert np.array_equal(g_.cpu().numpy().view(np.uint32), w_.view(np.uint32))

    sel = np.sort(r.choice(L, 20, replace=False)).astype(np.int64)
    qs = r.standard_normal((B, 20, C), dtype=np.float32)
    kv = np.ascontiguousarray(qkv.reshape(B, L, 3 * C)[..., C:])
    st, ref = oracle.q_kv_selected_rope_rmsnorm_pack(qs, kv, fr, sel, qg, kg, B, 20, L, H)
    assert st == 0
    got = q_kv_selected_rope_rmsnorm_pack(t(qs), t(kv), t(fr), t(sel), t(qg), t(kg), B, 20, L, H,
                                          kv_round=mode)
    for g_, w_, rnd in zip(got, ref, (False, rk, rv)):
        w_ = oracle.bf16_round(w_) if rnd else w_
        assert np.array_equal(g_.cpu().numpy().view(np.uint32), w_.view(np.uint32))

    x = torch.from_numpy(r.standard_normal((B * L, 256), dtype=np.float32)).to(cuda)
    w = torch.from_numpy((r.standard_normal((3 * C, 256)) * 0.02).astype(np.float32)).to(cuda)
    bias = torch.zeros(3 * C, device=cuda)
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    args = (x, codes[0], codes[1], scales[0], bias, t(fr), t(qg), t(kg), B, L, H)
    fused = gemm_nf24_qkv_direct(*args, kv_round=mode)
    unfused = qkv_rope_rmsnorm_pack(nf24_linear(*args[:5]), *args[5:], kv_round=mode)
    bhld = gemm_nf24_qkv_direct(*args, kv_layout="bhld", kv_round=mode)
    exact_fused = gemm_nf24_qkv_direct(*args)
    torch.cuda.synchronize(cuda)
    for a_, b_ in zip(fused, unfused):
        assert torch.equal(a_, b_)
    assert torch.equal(bhld[1], fused[1][..., :L].transpose(2, 3))
    assert torch.equal(bhld[2], fused[2][..., :L].transpose(2, 3))
    assert not fused[1][..., L:].any() and not fused[2][..., L:].any()
    assert torch.equal(exact_fused[0], fused[0])
    assert not torch.equal(exact_fused[1 if rk else 2], fused[1 if rk else 2])
    assert hiplib.triposplat_qkv_postprocess_bf16_probe_mode() == 0


@pytest.mark.parametrize("B,L,H,K,precision", [(1, 1, 2, 64, "fp32"), (1, 7, 4, 256, "fp32"),
                                                (2, 5, 2, 1024, "fp32"), (1, 16, 16, 1024, "fp32"),
                                                (2, 16, 4, 128, "fp32"), (1, 32, 2, 256, "fp32"),
                                                (2, 9, 16, 4096, "bf16x3")])
def test_qkv_fused_few_rows_match_unfused(cuda, B, L, H, K, precision):
    """At most 32 rows the fused projection runs the plain few-row GEMM and
    then the QKV epilogue (in every precision), so it equals the NF24 GEMM
    followed by the postprocess kernel bit for bit, as at M > 32."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct, qkv_rope_rmsnorm_pack

    print(f"qkv few rows B={B} L={L} H={H} K={K} {precision}", flush=True)
    C = H * 64
    g = torch.Generator(device=cuda).manual_seed(B * 100 + L + K)
    x = torch.randn((B * L, K), generator=g, device=cuda)
    w = torch.randn((3 * C, K), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    fr = torch.from_numpy(_freqs(1, L, H, L + 3)).to(cuda)
    qg, kg = (torch.from_numpy(a).to(cuda) for a in _gammas(H, H + 5))
    fused = gemm_nf24_qkv_direct(x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H,
                                 precision=precision)
    proj = nf24_linear(x, codes[0], codes[1], scales[0], bias, precision=precision)
    unfused = qkv_rope_rmsnorm_pack(proj, fr, qg, kg, B, L, H)
    torch.cuda.synchronize(cuda)
    for a_, b_ in zip(fused, unfused):
        assert bool(torch.isfinite(a_).all())
        assert torch.equal(a_, b_)


def _sweep_cases(seed, n):
    """Seeded random fused projections: batch, odd and tail-row lengths, head
    counts from 1 to 16, K aligned or ragged, one shared or per-batch
    frequency table, strict or bf16x3 products."""
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        B = int(r.integers(1, 4))
        H = int(r.choice([1, 2, 3, 4, 16]))
        L = int([r.integers(1, 40), r.integers(40, 700), r.integers(700, 3000)][r.integers(0, 3)])
        if B * L * H > 40000:
            L = max(1, 40000 // (B * H))
        L = max(L, -(-33 // B))  # M = B * L > 32: the plain GEMM takes the tile kernels too
        K = int(r.choice([64, 100, 256, 1024, 36]))
        out.append((B, L, H, K, int(r.choice([1, B])), str(r.choice(["fp32", "bf16x3"]))))
    return out


@pytest.mark.parametrize("B,L,H,K,fb,precision", _sweep_cases(2030, 16))
def test_qkv_fused_random_sweep(cuda, B, L, H, K, fb, precision):
    """Fused projection == the same precision's NF24 GEMM then the
    postprocess kernel, bit for bit, at seeded random shapes (M > 32: fewer
    rows go to the few-row kernels, checked against the oracle instead)."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct, qkv_rope_rmsnorm_pack

    print(f"qkv sweep B={B} L={L} H={H} K={K} fb={fb} {precision}", flush=True)
    C = H * 64
    g = torch.Generator(device=cuda).manual_seed(B * 1000 + L + K)
    x = torch.randn((B * L, K), generator=g, device=cuda)
    w = torch.randn((3 * C, K), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    fr = torch.from_numpy(_freqs(fb, L, H, L + 1)).to(cuda)
    qg, kg = (torch.from_numpy(a).to(cuda) for a in _gammas(H, H + 2))
    fused = gemm_nf24_qkv_direct(x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H,
                                 precision=precision)
    proj = nf24_linear(x, codes[0], codes[1], scales[0], bias, precision=precision)
    unfused = qkv_rope_rmsnorm_pack(proj, fr, qg, kg, B, L, H)
    torch.cuda.synchronize(cuda)
    for a_, b_ in zip(fused, unfused):
        assert bool(torch.isfinite(a_).all())
        assert torch.equal(a_, b_)
