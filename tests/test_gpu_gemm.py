"""GPU parity of the NF24 GEMM (libtsplat_hip.so) against the CPU oracle.

The oracle (oracle/tsplat_oracle.c) is the reference's scalar fmaf chain,
bit-exact with scripts/gemm_nf24_i16_avx512.c; the device sums the same
decoded products with fp32 MFMA, so agreement is bounded by the
order-of-summation bound in _parity.gemm_order_bound (stated there).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from _parity import gemm_f64, gemm_order_bound, seeded_linear, stats

pytestmark = pytest.mark.gpu


def _dev(torch, a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _run_async(torch, hiplib, device, x, c01, q2, s, b, start=0, count=None, stride_x=None,
               stride_out=None):
    M, K = x.shape
    N = c01.shape[1]
    count = N - start if count is None else count
    sx = K if stride_x is None else stride_x
    so = count if stride_out is None else stride_out
    xs = np.zeros((M, sx), np.float32)
    xs[:, :K] = x
    # keep every device buffer referenced until the asynchronous kernel is done
    d = [_dev(torch, a, device) for a in (xs, c01, q2, s, b)]
    out = torch.full((M, so), float("nan"), dtype=torch.float32, device=device)
    st = hiplib.tsplat_nf24_gemm_async(
        d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(), d[4].data_ptr(),
        out.data_ptr(), M, K, N, start, count, sx, so, torch.cuda.current_stream(device).cuda_stream)
    assert st == 0, st
    torch.cuda.synchronize(device)
    return out.cpu().numpy()


def _check(oracle, x, c01, q2, s, b, got, start=0):
    count = got.shape[1]
    ref = oracle.nf24_gemm(x, c01, q2, s, b, output_start=start, output_count=count)
    w_t = oracle.decode_nf24(c01, q2, s)[:, start:start + count]
    bound = gemm_order_bound(x, w_t, b[start:start + count])
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(np.isfinite(got))
    assert np.all(diff <= bound), (float(diff.max()), float((diff - bound).max()))
    exact = gemm_f64(x, w_t, b[start:start + count])
    e_dev, e_ref = stats(got, exact), stats(ref, exact)
    # statistically the device sum is no worse than the sequential chain
    assert e_dev["rmse"] <= 2.0 * e_ref["rmse"] + 1e-9, (e_dev, e_ref)
    return e_dev, e_ref


# The reference smoke shapes (scripts/smoke_native_rnf8_avx512.py:72-79),
# including the N=5 tail, plus skinny and ragged shapes.
SHAPES = [(25, 96, 64), (40, 96, 64), (10, 96, 64), (3, 96, 5), (1, 1024, 3072), (2, 1024, 256),
          (8, 4096, 64), (16, 64, 1024), (33, 130, 48), (129, 257, 200), (200, 64, 129),
          (7, 3, 17), (300, 1024, 96),
          # the single-stream graph's camera Linears: cam_refiner 5 -> 1024, cam_out_layer 1024 -> 5
          (1, 5, 1024), (1, 1024, 5),
          # vector (buffer-load) path with a partial last K step: K % 4 == 0, K % 16 != 0
          (70, 100, 96), (300, 1000, 384), (260, 36, 200),
          # few-row (HBM-bound) kernels: every row-count template, split and unsplit K,
          # ragged last K split, narrow and partial 512-column slabs
          (4, 2048, 640), (16, 1024, 3072), (32, 512, 384), (5, 4096, 1024), (12, 1000, 130),
          (3, 1000, 512), (7, 70, 1032), (1, 8200, 1024), (6, 4096, 8), (2, 1024, 6144),
          # 9-16 rows on the wide kernel (two LDS reduction passes), partial slab
          (9, 1024, 520), (13, 2048, 1032),
          # more K splits than the staged merge holds: the one-thread-per-output merge
          (1, 40000, 96),
          # the MFMA few-row form (4..16 rows, >= 192 slabs of 16 columns; 32-column slabs
          # where those alone give 192): both slab widths, the row-count edges, ragged K (a
          # partial last chunk and a partial last wave), a K only two waves reach; 3 rows and
          # 190 slabs stay on the split kernel
          (6, 1024, 3072), (8, 1000, 3072), (11, 2048, 6144), (16, 40, 3072), (13, 4100, 3104),
          (4, 1024, 6144), (4, 96, 3072), (3, 1024, 3072), (16, 1024, 3040),
          # ... with K split across workgroups when the slabs alone are fewer than 192
          # (N = 1024: four splits of 1024 rows; ragged K: a partial last split and chunk;
          # splits that rounding to whole chunks leaves empty are dropped)
          (16, 4096, 1024), (8, 4096, 1024), (5, 4096, 1024), (13, 2048, 1024), (10, 4100, 1024),
          (4, 1000, 1024), (4, 2048, 640)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_matches_oracle(oracle, cuda, hiplib, M, K, N):
    import torch

    print(f"gemm M={M} K={K} N={N}", flush=True)
    x, w, b = seeded_linear(19 + N, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    _check(oracle, x, c01, q2, s, b, got)


def test_gemm_reference_smoke_tolerance(oracle, cuda, hiplib):
    """scripts/smoke_native_rnf8_avx512.py:58: assert_close(rtol=2e-5, atol=2e-5)
    against F.linear on the exactly reconstructed weight."""
    import torch

    for (M, K, N) in [(25, 96, 64), (40, 96, 64), (10, 96, 64), (3, 96, 5)]:
        x, w, b = seeded_linear(19 + 3 + N, M, K, N)
        c01, q2, s = oracle.quantize_nf24_i16(w)
        got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
        w_hat = oracle.decode_nf24(c01, q2, s)
        ref = torch.nn.functional.linear(torch.from_numpy(x), torch.from_numpy(w_hat.T.copy()),
                                         torch.from_numpy(b))
        torch.testing.assert_close(torch.from_numpy(got), ref, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("K,N,start,count", [(1024, 3200, 64, 3072),   # one workgroup per slab
                                             (2048, 1088, 16, 1024)])   # K split across workgroups
def test_few_row_mfma_range_and_strides(oracle, cuda, hiplib, K, N, start, count):
    """The MFMA few-row form on an output range with row strides (x padded,
    out wider than the range), equal to the same columns of the full call."""
    import torch

    M = 12
    x, w, b = seeded_linear(71, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b, start, count, stride_x=K + 12,
                     stride_out=count + 32)[:, :count]
    _check(oracle, x, c01, q2, s, b, got, start)
    full = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    assert np.array_equal(got, full[:, start:start + count])


@pytest.mark.parametrize("K", [96, 100])
@pytest.mark.parametrize("start,count", [(0, 16), (16, 32), (48, 80), (5, 7), (100, 28)])
def test_gemm_range_and_strides(oracle, cuda, hiplib, start, count, K):
    import torch

    M, N = 37, 128
    x, w, b = seeded_linear(7, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b, start, count, stride_x=K + 8,
                     stride_out=count + 3)[:, :count]
    _check(oracle, x, c01, q2, s, b, got, start)
    # range == the corresponding columns of the full product (same kernel, same order)
    full = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    assert np.array_equal(got, full[:, start:start + count])


def test_gemm_config1_sampled_rows(oracle, cuda, hiplib):
    """Config 1 (4096x1024 @ 1024x3072, QKV): full GPU GEMM, oracle on 48
    sampled rows (rows are independent, so the oracle's rows are exact)."""
    import torch

    M, K, N = 4096, 1024, 3072
    r = np.random.default_rng(0)
    x = r.standard_normal((M, K), dtype=np.float32)
    w = (np.random.default_rng(1).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    b = (np.random.default_rng(2).standard_normal(N, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    rows = np.sort(r.choice(M, 48, replace=False))
    rows[0], rows[-1] = 0, M - 1
    e_dev, e_ref = _check(oracle, x[rows], c01, q2, s, b, got[rows])
    print("config1 sampled rows", e_dev, e_ref)


@pytest.mark.parametrize("M,K,N", [(16384, 1024, 1024), (32768, 1002, 1024), (2048, 1024, 2048),
                                   (9000, 998, 1030), (18432, 1024, 3072), (4096, 1024, 2048),
                                   (8192, 1002, 1024), (2600, 1024, 3072), (2048, 1002, 1024)])
def test_gemm_large_tiles_sampled_rows(oracle, cuda, hiplib, M, K, N):
    """Shapes that route to each tile configuration (256x256: 16384 and
    32768 rows; 256x192: 9000 x 1030; 256x128: 4096 x 2048 and 8192 x 1024;
    128x128: 2600 x 3072; 128x64: 2048 x 2048 and 2048 x 1024; 18432 rows:
    256x256 over 16384 rows plus 128x64 over the rest), with the vectorised
    and the scalar-load paths (K % 4 != 0 or odd N); the oracle checks 32
    sampled rows."""
    import torch

    print(f"gemm large M={M} K={K} N={N}", flush=True)
    x, w, b = seeded_linear(M + N, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    rows = np.sort(np.random.default_rng(M).choice(M, 32, replace=False))
    rows[0], rows[-1] = 0, M - 1
    _check(oracle, x[rows], c01, q2, s, b, got[rows])


def test_reference_named_entry_points(oracle, cuda, hiplib):
    """The blocking reference-named symbols take device pointers and keep the
    reference's status codes (scripts/gemm_nf24_i16_avx512.c:171-175)."""
    import torch

    M, K, N = 40, 96, 64
    x, w, b = seeded_linear(3, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    d = {k: _dev(torch, v, cuda) for k, v in dict(x=x, c01=c01, q2=q2, s=s, b=b).items()}
    cb = torch.zeros(256, dtype=torch.float32, device=cuda)
    out = torch.empty((M, N), dtype=torch.float32, device=cuda)
    ptrs = [d["x"].data_ptr(), d["c01"].data_ptr(), d["q2"].data_ptr(), d["q2"].data_ptr(),
            d["s"].data_ptr(), d["s"].data_ptr(), d["s"].data_ptr(), cb.data_ptr(), d["b"].data_ptr(),
            out.data_ptr()]
    assert hiplib.triposplat_gemm_rnf8_avx512(*ptrs, M, K, N, K, N, 4, 3) == 0
    _check(oracle, x, c01, q2, s, b, out.cpu().numpy())
    out2 = torch.empty((M, N), dtype=torch.float32, device=cuda)
    ptrs2 = ptrs[:-1] + [out2.data_ptr()]
    assert hiplib.triposplat_gemm_rnf8_avx512_tail(*ptrs2, M, K, N, K, N, 4, 3) == 0
    assert torch.equal(out, out2)
    # status codes
    assert hiplib.triposplat_gemm_rnf8_avx512(*ptrs, M, K, N, K, N, 4, 2) == -2        # stages
    assert hiplib.triposplat_gemm_rnf8_avx512_range(*ptrs, M, K, N, 8, 16, K, 16, 4, 3) == -4
    assert hiplib.triposplat_gemm_rnf8_avx512_range(*ptrs, M, K, N, 48, 32, K, 32, 4, 3) == -3
    nullp = list(ptrs)
    nullp[7] = None
    assert hiplib.triposplat_gemm_rnf8_avx512(*nullp, M, K, N, K, N, 4, 3) == -1
    host = np.zeros((M, N), np.float32)
    hostp = ptrs[:-1] + [host.ctypes.data_as(ctypes.c_void_p).value]
    assert hiplib.triposplat_gemm_rnf8_avx512(*hostp, M, K, N, K, N, 4, 3) == -6
    assert hiplib.triposplat_gemm_rnf8_avx512_residual_mode() == 4


def test_pointer_checks_within_one_allocation(oracle, cuda, hiplib):
    """A call's pointer checks accept a range inside an allocation an earlier
    check of the same call validated without asking the runtime again; a
    pointer into that same allocation whose extent runs past its end must
    still be rejected with -6 before any launch, and the in-bounds call must
    equal the same GEMM on separate tensors bit for bit."""
    import torch

    M, K, N = 8, 256, 512
    x, w, b = seeded_linear(M, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    ref = _run_async(torch, hiplib, cuda, x, c01, q2, s, b)
    hip = ctypes.CDLL("libamdhip64.so")
    size = 4 << 20
    base = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(base), ctypes.c_size_t(size)) == 0
    try:
        h2d = 1
        def put(off, a):
            a = np.ascontiguousarray(a)
            assert hip.hipMemcpy(ctypes.c_void_p(base.value + off), a.ctypes.data_as(ctypes.c_void_p),
                                 ctypes.c_size_t(a.nbytes), h2d) == 0
        put(0, x)
        put(65536, s)
        put(131072, b)
        d01, dq2 = _dev(torch, c01, cuda), _dev(torch, q2, cuda)
        stream = torch.cuda.current_stream(cuda).cuda_stream
        def call(out_off):
            return hiplib.tsplat_nf24_gemm_async(
                base.value, d01.data_ptr(), dq2.data_ptr(), base.value + 65536, base.value + 131072,
                base.value + out_off, M, K, N, 0, N, K, N, stream)
        assert call(size - M * N * 4 + 4) == -6          # 4 bytes past the allocation's end
        assert call(size - M * N * 4) == 0               # ends exactly at the end
        torch.cuda.synchronize(cuda)
        got = np.empty((M, N), np.float32)
        assert hip.hipMemcpy(got.ctypes.data_as(ctypes.c_void_p),
                             ctypes.c_void_p(base.value + size - M * N * 4),
                             ctypes.c_size_t(got.nbytes), 2) == 0
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        torch.cuda.synchronize(cuda)
        assert hip.hipFree(base) == 0


@pytest.mark.parametrize("M,K,N", [(16385, 1024, 1024), (8194, 1024, 3072), (12294, 256, 1024),
                                   (2818, 256, 3072), (8194, 1024, 1024), (12294, 4096, 1024),
                                   (16416, 1024, 1024), (16401, 1000, 1024), (16400, 256, 1024)])
def test_gemm_tail_rows(oracle, cuda, hiplib, M, K, N):
    """M = 256 k + r with r <= 32 (e.g. the compressed negative branch, L + 1
    tokens): 16385 x 1024, 8194 x 3072 and 8194 x 1024 (main rows on 256 x
    128 tiles, the 8448-row call on 256 x 192), 16416 x 1024 (the most tail
    rows, 32), 16401 x 1000 x 1024 (17 rows) and 16400 x 256 x 1024 (16 rows
    at a short K: the skinny MFMA tile, as a call over exactly them) run the
    tail rows on the few-row kernels (in the main grid they would add a
    round), 12294 x 256 / 4096 x 1024 (the
    reference's sequence length) runs 12288 rows on 192 x 256 tiles -- one
    round of 256 -- and the 6-row tail on the few-row kernels, 2818 x 3072
    keeps its two tail rows in its 256 x 192 grid (their tiles fit the last
    round).  Either way rows of the main part equal a GEMM over exactly those
    rows, and the same rows of a larger M with no tail (another tile shape),
    bit for bit; the tail rows equal a GEMM over exactly the tail rows bit for
    bit (split-off tails) or the same rows inside a tile (kept tails), repeat
    bit for bit, and lie within the summation-order bound of the same rows
    inside a 256-row tile; sampled rows and the tail against the oracle."""
    import torch

    print(f"gemm tail rows M={M} K={K} N={N}", flush=True)
    x, w, b = seeded_linear(M + 7, M + 256, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    r = M % 256
    big = M - r + 256                                             # a multiple of 256: no tail split
    got = _run_async(torch, hiplib, cuda, x[:M], c01, q2, s, b)
    again = _run_async(torch, hiplib, cuda, x[:M], c01, q2, s, b)
    head = _run_async(torch, hiplib, cuda, x[:M - r], c01, q2, s, b)
    tail = _run_async(torch, hiplib, cuda, x[M - r:M], c01, q2, s, b)
    full = _run_async(torch, hiplib, cuda, x[:big], c01, q2, s, b)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    assert np.array_equal(got[:M - r].view(np.uint32), head.view(np.uint32))
    assert np.array_equal(head.view(np.uint32), full[:M - r].view(np.uint32))
    split_off = (M, N) != (2818, 3072)
    same = tail if split_off else full[M - r:M]
    assert np.array_equal(got[M - r:].view(np.uint32), same.view(np.uint32))
    # two fp32 evaluation orders of the same sums
    bound = gemm_order_bound(x[M - r:M], oracle.decode_nf24(c01, q2, s), b)
    assert np.all(np.abs(got[M - r:].astype(np.float64) - full[M - r:M]) <= bound)
    rows = np.concatenate([np.sort(np.random.default_rng(M).choice(M - r, 16, replace=False)),
                           np.arange(M - r, M)])
    _check(oracle, x[rows], c01, q2, s, b, got[rows])


@pytest.mark.parametrize("precision", [0, 2])
def test_gemm_wide_row_stride_scalar_path(oracle, cuda, hiplib, precision):
    """A row stride so wide that a tile's x rows span 2^31 bytes: the vector
    path addresses them with 32-bit buffer offsets, so such calls take the
    scalar-load path.  Its result equals the vector path's on compact rows,
    bit for bit (strict fp32 and bf16x3), and the strict one the oracle."""
    import torch

    M, K, N = 40, 96, 128
    sx = ((1 << 31) // (4 * 127) + 64) // 4 * 4      # (127 * sx + K) * 4 bytes > 2^31
    x, w, b = seeded_linear(17, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    d_c01, d_q2, d_s, d_b = (_dev(torch, a, cuda) for a in (c01, q2, s, b))

    def run(xd, stride):
        out = torch.full((M, N), float("nan"), dtype=torch.float32, device=cuda)
        st = hiplib.tsplat_nf24_gemm_precision_async(
            xd.data_ptr(), d_c01.data_ptr(), d_q2.data_ptr(), d_s.data_ptr(), d_b.data_ptr(),
            out.data_ptr(), M, K, N, 0, N, stride, N, 0, None, 0, 1, precision, stream)
        assert st == 0, st
        torch.cuda.synchronize(cuda)
        return out.cpu().numpy()

    wide = torch.zeros((M, sx), dtype=torch.float32, device=cuda)
    wide[:, :K] = _dev(torch, x, cuda)
    got = run(wide, sx)
    del wide
    compact = run(_dev(torch, x, cuda), K)
    assert np.array_equal(got.view(np.uint32), compact.view(np.uint32))
    if precision == 0:
        _check(oracle, x, c01, q2, s, b, got)


def _sweep_shapes(seed, n, max_work=1.5e8):
    """Seeded random calls: ragged and aligned M, K, N (vector and scalar
    load paths, few-row kernels, row tails), an output range on 16-column
    boundaries (the reference's range contract) for some, and padded x /
    output row strides for some."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int([r.integers(1, 33), r.integers(33, 300), r.integers(256, 900)][r.integers(0, 3)])
        K = int(4 * r.integers(1, 300) if r.random() < 0.5 else r.integers(1, 1200))
        N = int(16 * r.integers(1, 50) if r.random() < 0.5 else r.integers(1, 800))
        if M * K * N > max_work:
            continue
        start, count = 0, N
        if N % 16 == 0 and N >= 32 and r.random() < 0.5:
            start = 16 * int(r.integers(0, N // 16))
            count = 16 * int(r.integers(1, (N - start) // 16 + 1))
        sx = K + (int(r.integers(1, 9)) if r.random() < 0.3 else 0)
        so = count + (int(r.integers(1, 9)) if r.random() < 0.3 else 0)
        out.append((M, K, N, start, count, sx, so))
    return out


@pytest.mark.parametrize("M,K,N,start,count,sx,so", _sweep_shapes(2026, 40))
def test_gemm_random_shape_sweep(oracle, cuda, hiplib, M, K, N, start, count, sx, so):
    """Random shapes, ranges and strides against the oracle within the
    summation-order bound; the padding columns of the output rows stay
    unwritten."""
    import torch

    print(f"gemm sweep M={M} K={K} N={N} start={start} count={count} sx={sx} so={so}", flush=True)
    x, w, b = seeded_linear(M * 131 + K * 7 + N, M, K, N)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    got = _run_async(torch, hiplib, cuda, x, c01, q2, s, b, start=start, count=count, stride_x=sx,
                     stride_out=so)
    assert np.all(np.isnan(got[:, count:]))
    _check(oracle, x, c01, q2, s, b, np.ascontiguousarray(got[:, :count]), start=start)
