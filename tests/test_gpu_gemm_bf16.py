"""GPU parity of the opt-in bf16-MFMA precision modes of the NF24 GEMM
(tsplat_nf24_gemm_precision_async, tsplat_gemm_nf24_qkv_direct_ex_async).

Oracle: oracle.nf24_gemm_bf16_terms, the float64 value of the terms the mode
defines (bf16: xh*wh; bf16x3: xh*wh + xh*wl + xl*wh, bf16 = round to nearest
even of the fp32 value).  Those products are exact in fp32, so the device
result may differ from the oracle only by its fp32 summation order over the
T*K products and the bias (T = 1 or 3): within 2 * gamma_{T*K+1} * sum|terms|
(Higham Thm 3.1), checked elementwise.  The relative RMSE of each mode
against the strict fp32 path is reported and held to its expected band
(bf16 about 2^-9, bf16x3 about 2^-17 of the output RMS).  The epilogues and
the fused QKV postprocess are fp32 functions of the accumulator, so each
equals, bit for bit, the oracle's elementwise step / postprocess applied to
the same mode's plain GEMM output.  Tile shapes sum in one order, so
128-row tiles equal the same rows inside 256-row tiles; a row tail split off a
call (at most 32 rows, when keeping them in the grid would add a round) runs
on the strict few-row path, like whole calls of at most 32 rows, and equals a
strict call over exactly those rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import U, gemm_order_bound, seeded_linear, stats

pytestmark = pytest.mark.gpu

MODES = {"bf16": 1, "bf16x3": 2}
TERMS = {"bf16": 1, "bf16x3": 3}


def _dev(torch, a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _run(torch, hiplib, device, x, c01, q2, s, b, precision, epilogue=0, out=None, gate=None,
         rows_per_batch=1, stride_x=None):
    M, K = x.shape
    N = c01.shape[1]
    sx = K if stride_x is None else stride_x
    xs = np.zeros((M, sx), np.float32)
    xs[:, :K] = x
    d = [_dev(torch, a, device) for a in (xs, c01, q2, s, b)]
    o = (torch.full((M, N), float("nan"), dtype=torch.float32, device=device) if out is None
         else _dev(torch, out, device))
    g = _dev(torch, gate, device) if gate is not None else None
    st = hiplib.tsplat_nf24_gemm_precision_async(
        d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(), d[4].data_ptr(),
        o.data_ptr(), M, K, N, 0, N, sx, N, epilogue, g.data_ptr() if g is not None else None,
        N if g is not None else 0, rows_per_batch, MODES.get(precision, 0),
        torch.cuda.current_stream(device).cuda_stream)
    assert st == 0, st
    torch.cuda.synchronize(device)
    return o.cpu().numpy()


def _check_terms(oracle, x, c01, q2, s, b, got, precision):
    ref = oracle.nf24_gemm_bf16_terms(x, c01, q2, s, b, precision)
    mag = oracle.nf24_gemm_bf16_abs_terms(x, c01, q2, s, b, precision)
    n = TERMS[precision] * x.shape[1] + 1
    bound = 2.0 * (n * U / (1.0 - n * U)) * mag
    diff = np.abs(got.astype(np.float64) - ref)
    assert np.all(np.isfinite(got))
    assert np.all(diff <= bound), (float(diff.max()), float((diff - bound).max()))
    return stats(got, ref)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("M,K,N", [
    (300, 1024, 3072),   # 256 x 192 tiles (fewer than one round), partial row tile
    (768, 1024, 512),    # 256 x 192 tiles with a partial column tile (512 = 2 x 192 + 128)
    (64, 256, 512),      # 128 x 128 tiles
    (520, 96, 200),      # N below one 256-column tile
    (520, 100, 200),     # K not a multiple of 32: a partial last K step (vector loads)
    (100, 33, 50),       # K, N not multiples of 4: the scalar-load kernel
    (544, 256, 512),     # 512 + 32 tail rows, kept in the 256-row grid (no extra round)
])
def test_bf16_gemm_matches_oracle(oracle, cuda, hiplib, precision, M, K, N):
    import torch

    print(f"bf16 gemm {precision} M={M} K={K} N={N}", flush=True)
    x, w, b = seeded_linear(M * 7 + K + N, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision)
    e = _check_terms(oracle, x, c01, q2, s, b, got, precision)
    assert e["rel_rmse"] < 1e-6, e


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_bf16_unaligned_x_stride(oracle, cuda, hiplib, precision):
    import torch

    x, w, b = seeded_linear(11, 272, 256, 256, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, stride_x=258)
    _check_terms(oracle, x, c01, q2, s, b, got, precision)


def test_bf16_few_rows_run_strict(oracle, cuda, hiplib):
    """M <= 32 runs the strict kernels in every precision."""
    import torch

    x, w, b = seeded_linear(5, 16, 1024, 1024, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    strict = _run(torch, hiplib, cuda, x, c01, q2, s, b, "fp32")
    for p in MODES:
        got = _run(torch, hiplib, cuda, x, c01, q2, s, b, p)
        assert np.array_equal(got.view(np.uint32), strict.view(np.uint32))


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("M,K,N", [
    (528, 256, 512),     # 16 tail rows in a 256 x 192 grid of one round
    (12294, 64, 3072),   # 6 tail rows: the 12288 head rows fill 3 rounds of 256 x 192 tiles
    (16400, 64, 1024),   # 256 full tiles = one round on 256 CUs; the tail would add one: split off
    (12294, 64, 4096),   # the reference's fc1 shape: 768 tiles = 3 rounds, the tail would add a fourth
    (16416, 1024, 1024),  # the most split-off rows (32), K long enough for the few-row K split
])
def test_bf16_tail_rows_bitwise(oracle, cuda, hiplib, precision, M, K, N):
    """Rows past a multiple of 256 either stay in the 256-row grid (then they
    equal, bit for bit, the same rows computed inside a larger grid) or,
    when they would add a round, are split off onto the strict few-row path
    (then they equal a strict call over exactly those rows, and the strict
    oracle bound); the head rows equal a call over exactly them, and 128-row
    tiles equal 256-row tiles."""
    import torch

    print(f"bf16 tail rows {precision} M={M} K={K} N={N}", flush=True)
    r = M % 256
    x, w, b = seeded_linear(21 + M, M - r + 256, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run(torch, hiplib, cuda, x[:M], c01, q2, s, b, precision)
    head = _run(torch, hiplib, cuda, x[:M - r], c01, q2, s, b, precision)
    full = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision)
    small = _run(torch, hiplib, cuda, x[:128], c01, q2, s, b[:N], precision)   # 128-row tiles
    assert np.array_equal(got[:M - r].view(np.uint32), head.view(np.uint32))
    assert np.array_equal(small.view(np.uint32), full[:128].view(np.uint32))
    # Kept in the grid (the launch model's choice) the tail rows equal the
    # same rows of the larger grid; split off, a strict call over exactly them.
    strict = _run(torch, hiplib, cuda, x[M - r:M], c01, q2, s, b, "fp32")
    split = np.array_equal(got[M - r:].view(np.uint32), strict.view(np.uint32))
    print(f"tail rows split off: {split}", flush=True)
    if split:
        want = oracle.nf24_gemm(x[M - r:M], c01, q2, s, b)     # the reference's fp32 chain
        bound = gemm_order_bound(x[M - r:M], oracle.decode_nf24(c01, q2, s), b)
        assert np.all(np.abs(got[M - r:].astype(np.float64) - want) <= bound)
    else:
        assert np.array_equal(got[M - r:].view(np.uint32), full[M - r:M].view(np.uint32))
    if (M, N) in ((16400, 1024), (12294, 4096)):       # a tail that would add a round
        assert split
    rows = np.arange(0, 256) if split else np.concatenate([np.arange(0, 256), np.arange(M - r - 64, M)])
    _check_terms(oracle, x[rows], c01, q2, s, b, got[rows], precision)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("epilogue", [2, 3, 4])
def test_bf16_epilogue_tail_split_bitwise(oracle, cuda, hiplib, precision, epilogue):
    """The reference's 12294 rows at N = 1024 in a bf16 mode: the 6 rows past
    12288 would add a round of tiles, so they run on the strict few-row path
    with the same epilogue (GELU, gated residual, add) at their own row
    positions -- equal, bit for bit, to a strict call over exactly those rows
    (the gated form reading gate batch 1, where rows 12288-12293 of two
    batches of 6147 lie) -- while rows 0-12287 equal a call of the mode over
    exactly them."""
    import torch

    M, K, N, B = 12294, 256, 1024, 2
    head_rows = M - M % 256
    print(f"bf16 epilogue tail {precision} epilogue={epilogue}", flush=True)
    x, w, b = seeded_linear(700 + epilogue, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    r = np.random.default_rng(epilogue)
    base = r.standard_normal((M, N)).astype(np.float32)
    gate = r.standard_normal((B, N)).astype(np.float32) if epilogue == 3 else None
    kw = dict(epilogue=epilogue, out=base if epilogue in (3, 4) else None, gate=gate,
              rows_per_batch=M // B if epilogue == 3 else 1)
    got = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, **kw)
    kw_head = dict(kw, out=base[:head_rows] if epilogue in (3, 4) else None)
    head = _run(torch, hiplib, cuda, x[:head_rows], c01, q2, s, b, precision, **kw_head)
    assert np.array_equal(got[:head_rows].view(np.uint32), head.view(np.uint32))
    kw_tail = dict(kw, out=base[head_rows:] if epilogue in (3, 4) else None,
                   gate=gate[1:] if epilogue == 3 else None, rows_per_batch=M)
    tail = _run(torch, hiplib, cuda, x[head_rows:], c01, q2, s, b, "fp32", **kw_tail)
    assert np.array_equal(got[head_rows:].view(np.uint32), tail.view(np.uint32))


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_bf16_qkv_tail_split_matches_unfused(cuda, precision):
    """Fused QKV projection at B = 2, L = 6147 (12294 rows, N = 3072): in
    bf16x3 the 6 rows past 12288 run the strict path's QKV epilogue at their
    own token positions (bf16 keeps them in its 256 x 256 grid: three rounds
    either way); in both modes the whole result equals the same mode's GEMM
    (whose tail takes the same path) followed by the postprocess kernel, bit
    for bit."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct, qkv_rope_rmsnorm_pack

    B, L, H, K = 2, 6147, 16, 256
    C = H * 64
    print(f"bf16 qkv tail {precision}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(6147)
    x = torch.randn((B * L, K), generator=g, device=cuda)
    w = torch.randn((3 * C, K), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    r = np.random.default_rng(L)
    ang = r.standard_normal((1, L, H, 32)).astype(np.float32)
    fr = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1).reshape(1, L, H, 64)).to(cuda)
    qg = torch.from_numpy((1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)).to(cuda)
    kg = torch.from_numpy((1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)).to(cuda)
    fused = gemm_nf24_qkv_direct(x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H,
                                 precision=precision)
    proj = nf24_linear(x, codes[0], codes[1], scales[0], bias, precision=precision)
    strict_tail = nf24_linear(x[B * L - 6:], codes[0], codes[1], scales[0], bias)
    unfused = qkv_rope_rmsnorm_pack(proj, fr, qg, kg, B, L, H)
    torch.cuda.synchronize(cuda)
    if precision == "bf16x3":
        assert torch.equal(proj[B * L - 6:], strict_tail)   # the tail took the strict path
    for a_, b_ in zip(fused, unfused):
        assert bool(torch.isfinite(a_).all())
        assert torch.equal(a_, b_)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_bf16_tile_shapes_bitwise(oracle, cuda, hiplib, precision):
    """Calls the launch model sends to the other tile shapes -- 12288 rows at
    N = 1024 (192 x 256), 8192 (256 x 128), 2048 (128 x 64), 4096 at N = 3072
    (256 x 192) -- equal the same rows of a 16384-row call (256 x 256) bit for
    bit (every shape sums each output in one order), and the mode's terms on
    sampled rows."""
    import torch

    K = 64
    for N, rows_list in ((1024, (12288, 8192, 2048)), (3072, (4096,))):
        x, w, b = seeded_linear(40 + N, 16384, K, N, w_scale=0.02)
        c01, q2, s = oracle.quantize_nf24_i16(w)
        full = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision)
        for M in rows_list:
            print(f"bf16 tile shapes {precision} M={M} N={N}", flush=True)
            got = _run(torch, hiplib, cuda, x[:M], c01, q2, s, b, precision)
            assert np.array_equal(got.view(np.uint32), full[:M].view(np.uint32)), (M, N)
            rows = np.sort(np.random.default_rng(M).choice(M, 24, replace=False))
            _check_terms(oracle, x[rows], c01, q2, s, b, got[rows], precision)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("M", [300, 100])
def test_bf16_epilogues(oracle, cuda, hiplib, precision, M):
    import torch

    K, N, B = 256, 512, 2
    x, w, b = seeded_linear(31 + M, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    acc = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision)
    r = np.random.default_rng(M)
    gelu = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, epilogue=2)
    exp = np.empty_like(acc)
    assert oracle.ew("gelu_tanh", acc, exp, acc.size) == 0
    assert np.array_equal(gelu.view(np.uint32), exp.view(np.uint32))
    base = r.standard_normal((M, N)).astype(np.float32)
    gate = r.standard_normal((B, N)).astype(np.float32)
    gated = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, epilogue=3, out=base, gate=gate,
                 rows_per_batch=M // B)
    exp, delta = base.copy(), acc.copy()
    assert oracle.ew("gated_residual_inplace", exp, delta, gate, B, M // B, N) == 0
    assert np.array_equal(gated.view(np.uint32), exp.view(np.uint32))
    added = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, epilogue=4, out=base)
    exp = base.copy()
    assert oracle.ew("add_inplace", exp, acc, exp.size) == 0
    assert np.array_equal(added.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("B,L", [(1, 300), (2, 70)])
def test_bf16_qkv_direct(oracle, cuda, hiplib, precision, B, L):
    import torch
    from tsplat.qkv import gemm_nf24_qkv_direct

    H = 4
    C = 64 * H
    x, w, b = seeded_linear(41 + L, B * L, C, 3 * C, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    r = np.random.default_rng(L)
    ang = r.uniform(-np.pi, np.pi, (1, L, H, 32))
    freqs = np.stack([np.cos(ang), np.sin(ang)], -1).reshape(1, L, H, 64).astype(np.float32)
    qg = (1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)
    kg = (1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)
    qkv = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision)
    exp = oracle.qkv_rope_rmsnorm_pack(qkv, freqs, qg, kg, B, L, H)
    d = {k: _dev(torch, a, cuda) for k, a in (("x", x), ("c", c01), ("q", q2), ("s", s), ("b", b),
                                             ("f", freqs), ("qg", qg), ("kg", kg))}
    got = gemm_nf24_qkv_direct(d["x"], d["c"], d["q"], d["s"], d["b"], d["f"], d["qg"], d["kg"], B, L, H,
                               precision=precision)
    torch.cuda.synchronize(cuda)
    for g_, e_ in zip(got, exp):
        assert np.array_equal(g_.cpu().numpy().view(np.uint32), np.asarray(e_).view(np.uint32))


def test_bf16_config0_rmse_vs_strict(oracle, cuda, hiplib):
    """configs[0] (X [4096 x 1024], W [3072 x 1024] ~ 0.02 N(0,1)): each mode
    against strict fp32, and sampled rows against the oracle terms."""
    import torch
    from tsplat.nf24 import nf24_linear

    M, K, N = 4096, 1024, 3072
    r = np.random.default_rng(0)
    x = r.standard_normal((M, K), dtype=np.float32)
    w = (r.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    b = (r.standard_normal(N, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    d = [_dev(torch, a, cuda) for a in (x, c01, q2, s, b)]
    strict = nf24_linear(*d).cpu().numpy()
    rows = np.sort(r.choice(M, 48, replace=False))
    rel = {}
    for p in MODES:
        got = nf24_linear(*d, precision=p).cpu().numpy()
        _check_terms(oracle, x[rows], c01, q2, s, b, got[rows], p)
        rel[p] = stats(got, strict)["rel_rmse"]
    print("relative RMSE vs strict fp32:", rel, flush=True)
    assert 2.0 ** -11 < rel["bf16"] < 2.0 ** -7, rel
    assert rel["bf16x3"] < 2.0 ** -14, rel


def test_bf16_rejects_unknown_precision(cuda, hiplib):
    import torch

    x = torch.zeros((64, 64), device=cuda)
    c = torch.zeros((64, 64), dtype=torch.int16, device=cuda)
    q = torch.zeros((64, 64), dtype=torch.int8, device=cuda)
    v = torch.zeros(64, device=cuda)
    out = torch.zeros((64, 64), device=cuda)
    st = hiplib.tsplat_nf24_gemm_precision_async(x.data_ptr(), c.data_ptr(), q.data_ptr(), v.data_ptr(),
                                                 v.data_ptr(), out.data_ptr(), 64, 64, 64, 0, 64, 64, 64,
                                                 0, None, 0, 1, 3, None)
    assert st == -2


def _sweep_shapes(seed, n, max_work=1.5e8):
    """Seeded random calls of the opt-in modes: M from the strict few-row
    range to several 256-row tiles, K and N aligned (vector loads, every tile
    shape) or ragged (scalar loads), some with a padded x row stride."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int([r.integers(33, 300), r.integers(256, 1100)][r.integers(0, 2)])
        K = int(4 * r.integers(1, 300) if r.random() < 0.7 else r.integers(1, 1200))
        N = int(4 * r.integers(1, 200) if r.random() < 0.7 else r.integers(1, 800))
        if M * K * N > max_work:
            continue
        sx = K + (4 * int(r.integers(1, 3)) if r.random() < 0.3 else 0)
        out.append((M, K, N, sx))
    return out


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("M,K,N,sx", _sweep_shapes(2027, 16))
def test_bf16_random_shape_sweep(oracle, cuda, hiplib, precision, M, K, N, sx):
    import torch

    print(f"bf16 gemm sweep {precision} M={M} K={K} N={N} sx={sx}", flush=True)
    x, w, b = seeded_linear(M * 17 + K * 5 + N, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run(torch, hiplib, cuda, x, c01, q2, s, b, precision, stride_x=sx)
    e = _check_terms(oracle, x, c01, q2, s, b, got, precision)
    assert e["rel_rmse"] < 1e-6, e
