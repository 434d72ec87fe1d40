"""GPU parity of the opt-in bf16-MFMA SDPA modes (tsplat_sdpa_precision_async,
native_sdpa_f32_ex(precision=...)).

Oracle: oracle.sdpa_bf16_terms -- the float64 softmax of the scores the mode
forms (q' = fp32(q * 0.125 * log2 e) and k split into bf16 terms, products
exact) over the mode's representation of v.  What it leaves open is bounded
here, per output element, relative to max|v'| of the (b, h):
  - the fp32 summation of the n score terms (n = 64 or 192, + the bias):
    gamma_n * sum|terms| (Higham Thm 3.1), the exponent argument x - m
    (2^-24 * 2 max|x|) and v_exp_f32 (2^-23 relative): a score error E moves
    the normalised weights by at most 2^(2E) - 1;
  - the split of the unnormalised exponential p: bf16x3 keeps
    |p v - (ph vh + ph vl + pl vh)| <= 2^-17 |p v|, bf16 2^-9 |p v|;
  - the fp32 accumulation of P V and of the row sum over Lk keys (plus
    one rescale per key tile) and the final 1/l: gamma_{3 Lk + T} +
    gamma_{Lk + T + 1} + 2^-22; a key-split tail adds one more exp2 per part.
The bound is rigorous and is checked on every element for small shapes
(both grids: 4-wave for small grids, the wide shape for grids that fill the
GPU).  At L = 8192-16384 the accumulation term is loose, so sampled rows are
also held to a relative RMSE against the oracle well below what a dropped
bf16 term would leave (about 2^-9).  One key gives p = 1 exactly, so the
output is the value's representation bit for bit (vh, or fp32(vh + vl)).
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import U, stats

pytestmark = pytest.mark.gpu


def _gamma(n):
    return n * U / (1.0 - n * U)


def _inputs(seed, B, H, Lq, Lk, scale=8.0):
    r = np.random.default_rng(seed)

    def rows(n):
        a = r.standard_normal((B, H, n, 64))
        return (a / np.linalg.norm(a, axis=-1, keepdims=True) * scale).astype(np.float32)

    return rows(Lq), rows(Lk), r.standard_normal((B, H, Lk, 64)).astype(np.float32)


def _run(torch, device, q, k, v, precision, bias=None, per_head=False, packed=False, blhd=False):
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    qd = torch.from_numpy(np.ascontiguousarray(q)).to(device)
    Lk = k.shape[2]
    if packed:
        Lkp = (Lk + 15) // 16 * 16
        pk = np.zeros(k.shape[:2] + (64, Lkp), np.float32)
        pv = np.zeros_like(pk)
        pk[..., :Lk] = k.transpose(0, 1, 3, 2)
        pv[..., :Lk] = v.transpose(0, 1, 3, 2)
        kd, vd = torch.from_numpy(pk).to(device), torch.from_numpy(pv).to(device)
    else:
        kd = torch.from_numpy(np.ascontiguousarray(k)).to(device)
        vd = torch.from_numpy(np.ascontiguousarray(v)).to(device)
    kw = {}
    if bias is not None:
        kw["key_bias_per_head" if per_head else "key_bias"] = torch.from_numpy(bias).to(device)
    out = native_sdpa_f32_ex(qd, kd, vd, kv_packed=packed, key_count=Lk,
                             out_layout="blhd" if blhd else "bhld", precision=precision, **kw)
    torch.cuda.synchronize(device)
    out = out.cpu().numpy()
    return out.transpose(0, 2, 1, 3) if blhd else out


def _bound(oracle, q, k, v, bias, precision, rows=None, key_tile=64, splits=1):
    """(reference, per-element bound) for query rows `rows` (all if None)."""
    qs = q if rows is None else q[:, :, rows]
    ref, s_abs, x_abs = oracle.sdpa_bf16_terms(qs, k, v, bias, precision)
    Lk = k.shape[2]
    three = precision == "bf16x3"
    n = (192 if three else 64) + (bias is not None)
    E = _gamma(n) * s_abs + 4 * U * x_abs + 2.0 ** -22
    eps_p = 2.0 ** -17 if three else 2.0 ** -9 * 1.01
    T = (Lk + key_tile - 1) // key_tile
    eps_acc = _gamma((3 if three else 1) * Lk + T) + _gamma(Lk + T + 1) + 2.0 ** -22 + splits * 2.0 ** -22
    vh, vl = oracle.bf16_split(v)
    vrep = vh.astype(np.float64) + (vl.astype(np.float64) if three else 0.0)
    vmax = np.abs(vrep).max(axis=(-1, -2))[:, :, None, None]
    return ref, ((np.exp2(2 * E) - 1)[..., None] + eps_p + eps_acc) * vmax * (1 + 1e-6)


def _check(got, ref, bound):
    assert np.all(np.isfinite(got))
    d = np.abs(got.astype(np.float64) - ref)
    assert np.all(d <= bound), (float(d.max()), float((d - bound).max()))


def _bias(kind, H, Lk, seed):
    r = np.random.default_rng(seed)
    if kind == "shared":
        return r.uniform(-2, 0, Lk).astype(np.float32)
    if kind == "per_head":
        return r.uniform(-2, 0, (H, Lk)).astype(np.float32)
    return None


PRECISIONS = ["bf16", "bf16x3"]


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("B,H,Lq,Lk,bias,packed,blhd", [
    (1, 2, 37, 45, None, False, False),
    (2, 3, 70, 200, "shared", False, False),
    (1, 2, 130, 64, "per_head", False, True),
    (1, 2, 50, 77, None, True, False),
    (1, 3, 33, 300, "shared", True, True),
    (1, 1, 1, 1, None, False, False),
])
def test_bf16_sdpa_small_grid_bound(oracle, cuda, precision, B, H, Lq, Lk, bias, packed, blhd):
    import torch

    print(f"sdpa {precision} B={B} H={H} Lq={Lq} Lk={Lk} bias={bias} packed={packed}", flush=True)
    q, k, v = _inputs(Lq * 31 + Lk, B, H, Lq, Lk)
    b = _bias(bias, H, Lk, Lk)
    got = _run(torch, cuda, q, k, v, precision, b, per_head=bias == "per_head", packed=packed, blhd=blhd)
    ref, bound = _bound(oracle, q, k, v, b, precision)
    _check(got, ref, bound)


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("B,L,Lk,bias,packed", [
    (1, 8192, 8192, None, False),          # 256 query tiles of 512: the wide grid, no key split
    (1, 8192, 2048, "per_head", False),    # cross-attention shape with a per-head bias
    (1, 8192 + 512, 8192 + 512, None, True),   # last round split along the keys, packed K/V
    (1, 8192 + 512, 8193, "shared", False),    # key split with a ragged key tail and a bias
    # too few query tiles per head for the pre-split pass: K/V staged in the kernel
    (16, 2048, 2048, None, True),
    (2, 4096 + 100, 4099, "per_head", False),
])
def test_bf16_sdpa_wide_grid_rows(oracle, cuda, precision, B, L, Lk, bias, packed):
    import torch

    H = 16
    print(f"sdpa wide {precision} B={B} L={L} Lk={Lk} bias={bias} packed={packed}", flush=True)
    q, k, v = _inputs(L + Lk, B, H, L, Lk)
    b = _bias(bias, H, Lk, 3)
    got = _run(torch, cuda, q, k, v, precision, b, per_head=bias == "per_head", packed=packed)
    rows = np.unique(np.concatenate([np.random.default_rng(L).choice(L, 40 if B == 1 else 12, replace=False),
                                     [0, L - 1, L - 512, L - 257]]))
    ref, bound = _bound(oracle, q, k, v, b, precision, rows=rows, splits=16)
    sub = got[:, :, rows]
    _check(sub, ref, bound)
    rel = stats(sub, ref)["rel_rmse"]
    print("relative RMSE vs oracle", rel, flush=True)
    assert rel < (2.0 ** -15 if precision == "bf16x3" else 2.0 ** -9), rel


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("Lq", [40, 8192])
def test_bf16_sdpa_single_key_exact(oracle, cuda, precision, Lq):
    """Lk = 1: p = exp2(0) = 1 splits exactly (ph = 1, pl = 0), the sum is 1,
    so every output row is the value's representation bit for bit."""
    import torch

    H = 16
    q, k, v = _inputs(Lq, 1, H, Lq, 1)
    got = _run(torch, cuda, q, k, v, precision)
    vh, vl = oracle.bf16_split(v)
    rep = (vh + vl).astype(np.float32) if precision == "bf16x3" else vh
    assert np.array_equal(got.view(np.uint32), np.broadcast_to(rep, got.shape).view(np.uint32))


def test_bf16_sdpa_config1_vs_strict(oracle, cuda):
    """configs[1] (B=1, H=16, Lq=Lk=16384, RMS-normalised q, k of norm 8 as
    after the flow's RMSNorm, v ~ N(0, 1)): each mode against the strict
    fp32 kernel, and sampled rows against the oracle within the bound."""
    import torch
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    B, H, L = 1, 16, 16384
    q, k, v = _inputs(99, B, H, L, L)
    d = [torch.from_numpy(a).to(cuda) for a in (q, k, v)]
    strict = native_sdpa_f32_ex(*d).cpu().numpy()
    rows = np.sort(np.random.default_rng(1).choice(L, 24, replace=False))
    rel = {}
    for p in PRECISIONS:
        got = native_sdpa_f32_ex(*d, precision=p).cpu().numpy()
        ref, bound = _bound(oracle, q, k, v, None, p, rows=rows)
        _check(got[:, :, rows], ref, bound)
        rel[p] = stats(got, strict)["rel_rmse"]
    print("relative RMSE vs strict fp32:", rel, flush=True)
    assert rel["bf16x3"] < 2.0 ** -15, rel
    assert rel["bf16"] < 2.0 ** -6, rel


@pytest.mark.parametrize("precision", ["fp32", "bf16", "bf16x3"])
@pytest.mark.parametrize("B,H,Lq,Lk,bias", [(1, 2, 70, 77, "shared"), (1, 16, 8192 + 512, 8193, None),
                                            (2, 3, 40, 300, "per_head")])
def test_packed_kv_layout_matches(cuda, precision, B, H, Lq, Lk, bias):
    """Key-contiguous k/v [B,H,64,Lkp] stage the same values into the same
    LDS positions as [B,H,Lk,64] k/v, on the same tile plan, so each query
    row sees the same operations: bit-identical output in every precision
    (small grid, wide grid with a key-split tail)."""
    import torch
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    print(f"packed layout {precision} B={B} H={H} Lq={Lq} Lk={Lk}", flush=True)
    q, k, v = _inputs(Lq + 7 * Lk, B, H, Lq, Lk)
    b = _bias(bias, H, Lk, 5)
    kw = {}
    if b is not None:
        kw["key_bias_per_head" if bias == "per_head" else "key_bias"] = torch.from_numpy(b).to(cuda)
    qd, kd, vd = (torch.from_numpy(a).to(cuda) for a in (q, k, v))
    Lkp = (Lk + 15) // 16 * 16 + 16
    vp = torch.zeros((B, H, 64, Lkp), device=cuda)
    vp[..., :Lk] = vd.transpose(2, 3)
    kp = torch.zeros_like(vp)
    kp[..., :Lk] = kd.transpose(2, 3)
    rows = native_sdpa_f32_ex(qd, kd, vd, precision=precision, **kw)
    packed = native_sdpa_f32_ex(qd, kp, vp, kv_packed=True, key_count=Lk, precision=precision, **kw)
    torch.cuda.synchronize(cuda)
    assert bool(torch.isfinite(rows).all())
    assert torch.equal(packed, rows)


def _sweep_cases(seed, n, max_work=2e8):
    """Seeded random calls of the opt-in modes: ragged Lq / Lk, no bias or
    a shared or per-head bias, [B,H,L,64] or packed K/V, BHLD or BLHD."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B, H = int(r.integers(1, 3)), int(r.integers(1, 4))
        Lq, Lk = int(r.integers(1, 600)), int(r.integers(1, 1200))
        if B * H * Lq * Lk * 128 > max_work:
            continue
        out.append((B, H, Lq, Lk, [None, "shared", "per_head"][r.integers(0, 3)], bool(r.random() < 0.5),
                    bool(r.random() < 0.5)))
    return out


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("B,H,Lq,Lk,bias,packed,blhd", _sweep_cases(2029, 12))
def test_sdpa_bf16_random_case_sweep(oracle, cuda, precision, B, H, Lq, Lk, bias, packed, blhd):
    import torch

    print(f"sdpa bf16 sweep {precision} B={B} H={H} Lq={Lq} Lk={Lk} bias={bias} packed={packed} "
          f"blhd={blhd}", flush=True)
    q, k, v = _inputs(Lq * 5 + Lk + B + H, B, H, Lq, Lk)
    b = _bias(bias, H, Lk, Lq + Lk)
    got = _run(torch, cuda, q, k, v, precision, bias=b, per_head=bias == "per_head", packed=packed, blhd=blhd)
    ref, bound = _bound(oracle, q, k, v, b, precision)
    _check(got, ref, bound)


def _raw(lib, fn, torch, cuda, q, k, v, b, out, precision, blhd, Lk, Lkp, stream=None):
    """One call of a C-ABI SDPA entry (precision 1 = bf16, 2 = bf16x3)."""
    B, H, Lq, _ = q.shape
    st = torch.cuda.current_stream(cuda).cuda_stream if stream is None else stream
    return getattr(lib, fn)(q.data_ptr(), k.data_ptr(), v.data_ptr(), None if b is None else b.data_ptr(),
                            out.data_ptr(), B, H, Lq, Lk, 64, int(b is not None), 0 if b is None else Lk,
                            0 if b is None or b.dim() == 1 else Lk, int(Lkp > 0), Lkp, int(blhd), precision, st)


def _workspace_bytes(lib):
    import ctypes

    vals = [ctypes.c_uint64(0) for _ in range(2)]
    assert lib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(x) for x in vals]) == 0
    return vals[0].value, vals[1].value


# (B, H, Lq, Lk, bias, packed, blhd): wide grids with enough query tiles of
# 512 per head for the pre-split pass (12 with [Lk, 64] k/v, 6 with packed
# k/v): a ragged key tail with a key-split last round, a per-head bias with
# BLHD output, a shared bias, packed k/v with and without a bias
PRESPLIT = [(2, 16, 6144 + 100, 6147, None, False, False),
            (1, 16, 8192, 8192, "per_head", False, True),
            (1, 16, 8704, 1000, "shared", False, False),
            (3, 16, 3100, 3001, "per_head", True, False),
            (4, 8, 4096, 4096, None, True, True)]


@pytest.mark.parametrize("precision", [1, 2])
@pytest.mark.parametrize("B,H,Lq,Lk,bias,packed,blhd", PRESPLIT)
def test_bf16_sdpa_presplit_matches_direct(cuda, hiplib, precision, B, H, Lq, Lk, bias, packed, blhd):
    """The precision entry stages K/V once in a pre-split pass where the
    no-allocation entry stages them in the kernel: the LDS tiles, the tile
    plan and so the outputs are the same bit for bit.  The workspace grows
    to hold the pre-split image (the pass ran)."""
    import torch

    print(f"presplit {precision} B={B} H={H} Lq={Lq} Lk={Lk} bias={bias} packed={packed} blhd={blhd}",
          flush=True)
    g = torch.Generator(device=cuda).manual_seed(Lq + Lk + B)
    q = torch.nn.functional.normalize(torch.randn((B, H, Lq, 64), generator=g, device=cuda), dim=-1) * 8
    k = torch.nn.functional.normalize(torch.randn((B, H, Lk, 64), generator=g, device=cuda), dim=-1) * 8
    v = torch.randn((B, H, Lk, 64), generator=g, device=cuda)
    b = None
    if bias == "shared":
        b = torch.rand((Lk,), generator=g, device=cuda) * -2.0
    elif bias == "per_head":
        b = torch.rand((H, Lk), generator=g, device=cuda) * -2.0
    Lkp = 0
    if packed:
        Lkp = -(-Lk // 16) * 16
        kp = torch.zeros((B, H, 64, Lkp), device=cuda)
        vp = torch.zeros_like(kp)
        kp[..., :Lk] = k.transpose(2, 3)
        vp[..., :Lk] = v.transpose(2, 3)
        k, v = kp, vp
    shape = (B, Lq, H, 64) if blhd else (B, H, Lq, 64)
    pre, direct = (torch.full(shape, float("nan"), device=cuda) for _ in range(2))
    assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, b, pre, precision, blhd, Lk, Lkp) == 0
    assert _raw(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, q, k, v, b, direct, precision, blhd, Lk,
                Lkp) == 0
    torch.cuda.synchronize(cuda)
    image = B * H * -(-Lk // 64) * (4 if precision == 2 else 2) * 64 * 64 * 2
    assert _workspace_bytes(hiplib)[1] >= image
    assert bool(torch.isfinite(pre).all())
    assert torch.equal(pre, direct)


def test_bf16_sdpa_presplit_capture_without_workspace(cuda, hiplib):
    """Captured on a fresh stream, whose pre-split workspace cannot be
    allocated under capture, the precision entry stages K/V in the kernel;
    replays (with eager calls between them) equal the eager pre-split
    result bit for bit and the capture allocates nothing."""
    import torch

    B, H, L = 1, 16, 8192   # 256 query tiles of 512: no key split, so no partials workspace
    g = torch.Generator(device=cuda).manual_seed(11)
    q, k = (torch.nn.functional.normalize(torch.randn((B, H, L, 64), generator=g, device=cuda), dim=-1) * 8
            for _ in range(2))
    v = torch.randn((B, H, L, 64), generator=g, device=cuda)
    want = torch.empty((B, H, L, 64), device=cuda)
    assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, None, want, 2, 0, L, 0) == 0
    torch.cuda.synchronize(cuda)
    out = torch.empty_like(want)
    other = torch.empty_like(want)
    s = torch.cuda.Stream(device=cuda)
    before = _workspace_bytes(hiplib)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s, capture_error_mode="relaxed"):
        assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, None, out, 2, 0, L, 0,
                    stream=s.cuda_stream) == 0
    torch.cuda.synchronize(cuda)
    assert _workspace_bytes(hiplib) == before
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, want)
        assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, k, q, v, None, other, 2, 0, L, 0) == 0
        torch.cuda.synchronize(cuda)


def test_bf16_sdpa_presplit_image_cap(cuda, hiplib):
    """A call whose pre-split image would exceed 2 GiB (1024 heads x 65 key
    tiles x 32 KiB in bf16x3) stages in the kernel: the workspace does not
    grow by the image, and the result equals the no-allocation entry's."""
    import torch

    B, H, Lq, Lk = 64, 16, 6144, 4160
    g = torch.Generator(device=cuda).manual_seed(21)
    q = torch.randn((B, H, Lq, 64), generator=g, device=cuda)
    k = torch.randn((B, H, Lk, 64), generator=g, device=cuda)
    v = torch.randn((B, H, Lk, 64), generator=g, device=cuda)
    assert B * H * -(-Lk // 64) * 4 * 64 * 64 * 2 > 2 << 30
    before = _workspace_bytes(hiplib)[1]
    got, want = (torch.full((B, H, Lq, 64), float("nan"), device=cuda) for _ in range(2))
    assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, None, got, 2, 0, Lk, 0) == 0
    assert _raw(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, q, k, v, None, want, 2, 0, Lk, 0) == 0
    torch.cuda.synchronize(cuda)
    assert _workspace_bytes(hiplib)[1] - before < 1 << 30
    assert bool(torch.isfinite(got).all())
    assert torch.equal(got, want)


def test_bf16_sdpa_presplit_captured_then_grown(cuda, hiplib):
    """Captured on a stream whose pre-split workspace already holds the image
    (an eager call first), the graph records the pre-split pass; a larger
    eager call then grows the stream's buffer, and later replays (which keep
    the buffer the capture recorded) still equal the eager result bit for
    bit, with eager calls between them."""
    import torch

    H, L = 16, 8192   # 256 query tiles of 512: no key split
    g = torch.Generator(device=cuda).manual_seed(12)

    def inputs(Lk):
        q = torch.nn.functional.normalize(torch.randn((1, H, L, 64), generator=g, device=cuda), dim=-1) * 8
        k = torch.nn.functional.normalize(torch.randn((1, H, Lk, 64), generator=g, device=cuda), dim=-1) * 8
        return q, k, torch.randn((1, H, Lk, 64), generator=g, device=cuda)

    small, large = inputs(L), inputs(2 * L)
    s = torch.cuda.Stream(device=cuda)
    want = torch.empty((1, H, L, 64), device=cuda)
    out = torch.empty_like(want)
    other = torch.empty_like(want)
    torch.cuda.synchronize(cuda)
    with torch.cuda.stream(s):
        assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, *small, None, want, 2, 0, L, 0,
                    stream=s.cuda_stream) == 0
    torch.cuda.synchronize(cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s, capture_error_mode="relaxed"):
        assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, *small, None, out, 2, 0, L, 0,
                    stream=s.cuda_stream) == 0
    torch.cuda.synchronize(cuda)
    allocations = _workspace_bytes(hiplib)[0]
    with torch.cuda.stream(s):
        assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, *large, None, other, 2, 0, 2 * L, 0,
                    stream=s.cuda_stream) == 0
    torch.cuda.synchronize(cuda)
    assert _workspace_bytes(hiplib)[0] == allocations + 1   # the larger image grew s's buffer
    for _ in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, want)
        with torch.cuda.stream(s):
            assert _raw(hiplib, "tsplat_sdpa_precision_async", torch, cuda, *large, None, other, 2, 0, 2 * L,
                        0, stream=s.cuda_stream) == 0
        torch.cuda.synchronize(cuda)


def _presplit_sweep(seed, n):
    """Seeded wide-grid calls that take the pre-split pass: 12+ query tiles
    of 512 per head ([Lk, 64] k/v) or 6+ (packed), B*H*tiles >= 256, ragged
    Lq and Lk, no / shared / per-head bias, BHLD or BLHD output."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        packed = bool(r.random() < 0.4)
        tiles = int(r.integers(6 if packed else 12, 18))
        Lq = (tiles - 1) * 512 + int(r.integers(1, 513))
        H = int(r.integers(1, 17))
        B = max(1, -(-256 // (H * tiles)) + int(r.integers(0, 2)))
        if B * H * tiles > 600:
            continue
        out.append((B, H, Lq, int(r.integers(1, 3000)), [None, "shared", "per_head"][r.integers(0, 3)], packed,
                    bool(r.random() < 0.5)))
    return out


@pytest.mark.parametrize("precision", [1, 2])
@pytest.mark.parametrize("B,H,Lq,Lk,bias,packed,blhd", _presplit_sweep(4242, 8))
def test_bf16_sdpa_presplit_random_sweep(cuda, hiplib, precision, B, H, Lq, Lk, bias, packed, blhd):
    test_bf16_sdpa_presplit_matches_direct(cuda, hiplib, precision, B, H, Lq, Lk, bias, packed, blhd)
