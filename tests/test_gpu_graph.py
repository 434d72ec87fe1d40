"""HIP-graph capture of the calls that use a library-owned workspace (the
few-row GEMM's split-K partials, the SDPA's key-split tail partials).

A stream under capture cannot allocate: the first such call captured on a
stream that has no buffer yet must fail cleanly (status -5, raised by the
wrapper) without recording anything.  After one eager call on that stream
the capture succeeds, and every replay -- with eager work and
synchronisations between replays -- equals the eager result bit for bit.
"""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def _replays_match(torch, cuda, g, out, expected, eager_between):
    for _ in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, expected)
        eager_between()
        torch.cuda.synchronize(cuda)


@pytest.mark.parametrize("M,K,N", [(2, 1024, 3072),    # the wide few-row kernel, K split
                                   (12, 4096, 1024)])  # the MFMA few-row form, K split
def test_graph_few_row_gemm(cuda, M, K, N):
    """A few-row GEMM that splits K captures into a graph once its stream has
    a workspace (a capture cannot allocate: before that it fails with -5),
    and every replay equals the eager result bit for bit."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel

    print(f"graph few-row gemm M={M} K={K} N={N}", flush=True)
    g0 = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn((M, K), generator=g0, device=cuda)
    w = torch.randn((N, K), generator=g0, device=cuda) * 0.02
    b = torch.randn((N,), generator=g0, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    args = (x, codes[0], codes[1], scales[0], b)
    expected = nf24_linear(*args)
    out = torch.empty_like(expected)
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)

    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="-5"):
        with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
            nf24_linear(*args, out=out)
    torch.cuda.synchronize(cuda)

    with torch.cuda.stream(s):
        nf24_linear(*args, out=out)                   # eager call: the stream's buffer exists
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        nf24_linear(*args, out=out)
    torch.cuda.synchronize(cuda)
    _replays_match(torch, cuda, g, out, expected, lambda: nf24_linear(*args))


@pytest.mark.parametrize("kind", ["gelu", "gated", "qkv"])
def test_graph_epilogue_gemm_row_tail(cuda, kind):
    """An epilogue GEMM whose <= 32-row tail runs on the few-row kernels
    through the workspace (16385 rows = 64 x 256 + 1): captured before its
    stream has a workspace it fails with -5 and enqueues nothing (the tail
    goes first), after one eager call it captures, and every replay equals
    the eager result bit for bit."""
    import torch
    from tsplat import block_ops as bo
    from tsplat.nf24 import quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct

    M, K = 16385, 1024
    N = 3 * 1024 if kind == "qkv" else 1024
    print(f"graph epilogue gemm {kind} M={M} K={K} N={N}", flush=True)
    g0 = torch.Generator(device=cuda).manual_seed(5)
    x = torch.randn((M, K), generator=g0, device=cuda)
    w = torch.randn((N, K), generator=g0, device=cuda) * 0.02
    b = torch.randn((N,), generator=g0, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    args = (x, codes[0], codes[1], scales[0], b)
    base = torch.randn((M, N), generator=g0, device=cuda)
    gate = torch.randn((1, N), generator=g0, device=cuda)
    if kind == "qkv":
        H = 16
        i = torch.arange(32, dtype=torch.float64, device=cuda)
        ang = torch.arange(M, dtype=torch.float64, device=cuda)[:, None] * 1e4 ** (-2.0 * i / 64.0)[None, :]
        fr = torch.stack((ang.cos(), ang.sin()), -1).reshape(M, 64).float()[None, :, None, :].expand(1, M, H, 64)
        fr = fr.contiguous()
        qg = torch.ones((H, 64), device=cuda)
        outs = gemm_nf24_qkv_direct(*args, fr, qg, qg, 1, M, H)

        def call():
            q_, k_, v_ = gemm_nf24_qkv_direct(*args, fr, qg, qg, 1, M, H)
            for dst, src in zip(outs, (q_, k_, v_)):
                dst.copy_(src)
        expected = [t.clone() for t in outs]
        out = outs[0]
    else:
        out = base.clone()

        def call():
            if kind == "gelu":
                bo.nf24_linear_epilogue(*args, bo.EPILOGUE_GELU, out=out)
            else:
                out.copy_(base)
                bo.nf24_linear_epilogue(*args, bo.EPILOGUE_GATED, out=out, gate=gate)
        call()
        expected = [out.clone()]
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)

    if kind != "qkv":   # the QKV wrapper allocates its outputs, which a capture cannot hold here
        g = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="-5"):
            with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
                call()
        torch.cuda.synchronize(cuda)

    with torch.cuda.stream(s):
        call()                                   # eager call: the stream's buffers exist
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        call()
    torch.cuda.synchronize(cuda)
    results = outs if kind == "qkv" else [out]
    for _ in range(3):
        for t in results:
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(cuda)
        for got, want in zip(results, expected):
            assert torch.equal(got, want)
        call()                                   # eager work between replays
        torch.cuda.synchronize(cuda)


def test_graph_sdpa_key_split_tail(cuda):
    import torch
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    g0 = torch.Generator(device=cuda).manual_seed(4)
    B, H, L = 1, 16, 8192 + 512                      # 272 query tiles: the last 16 are key-split
    q = torch.nn.functional.normalize(torch.randn((B, H, L, 64), generator=g0, device=cuda), dim=-1) * 8
    k = torch.nn.functional.normalize(torch.randn((B, H, L, 64), generator=g0, device=cuda), dim=-1) * 8
    v = torch.randn((B, H, L, 64), generator=g0, device=cuda)
    expected = native_sdpa_f32_ex(q, k, v)
    out = torch.empty_like(expected)
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)

    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="-5"):
        with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
            native_sdpa_f32_ex(q, k, v, out=out)
    torch.cuda.synchronize(cuda)

    with torch.cuda.stream(s):
        native_sdpa_f32_ex(q, k, v, out=out)
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        native_sdpa_f32_ex(q, k, v, out=out)
    torch.cuda.synchronize(cuda)
    _replays_match(torch, cuda, g, out, expected, lambda: native_sdpa_f32_ex(q, k, v))


def _canaries(torch, cuda, n=4, mib=96):
    """Fresh device allocations filled with a pattern: if the library had
    freed a buffer a graph still writes to, the caching allocator could hand
    that memory out here and a replay would overwrite the pattern."""
    return [torch.full(((mib << 20) // 4,), 1234.5, device=cuda) for _ in range(n)]


def test_graph_survives_workspace_growth_gemm(cuda):
    """Capture a few-row GEMM at a small shape, then grow the capture
    stream's workspace with a larger eager call on the same stream: the
    captured buffer is retired, not freed, so replays still equal the eager
    result bit for bit and no other allocation is written."""
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel

    g0 = torch.Generator(device=cuda).manual_seed(5)

    def linear(M, K, N):
        x = torch.randn((M, K), generator=g0, device=cuda)
        w = torch.randn((N, K), generator=g0, device=cuda) * 0.02
        b = torch.randn((N,), generator=g0, device=cuda) * 0.01
        codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
        return x, codes[0], codes[1], scales[0], b

    small = linear(2, 1024, 3072)     # K split into 32 partials: ~0.8 MB of workspace
    large = linear(2, 4096, 6144)     # 64 partials of 2 rows: ~3.1 MB
    expected = nf24_linear(*small)
    expected_large = nf24_linear(*large)
    out = torch.empty_like(expected)
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)
    with torch.cuda.stream(s):
        nf24_linear(*small, out=out)            # sizes s's buffer for the small call
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        nf24_linear(*small, out=out)
    torch.cuda.synchronize(cuda)
    with torch.cuda.stream(s):
        got_large = nf24_linear(*large)        # grows s's buffer: the captured one is retired
    torch.cuda.synchronize(cuda)
    assert torch.equal(got_large, expected_large)
    canaries = _canaries(torch, cuda)
    torch.cuda.synchronize(cuda)
    for _ in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, expected)
        with torch.cuda.stream(s):
            assert torch.equal(nf24_linear(*large), expected_large)
        torch.cuda.synchronize(cuda)
    for c in canaries:
        assert bool((c == 1234.5).all())


def test_graph_survives_workspace_growth_sdpa(cuda, hiplib):
    """The same for the SDPA's key-split partials: capture a call whose
    split tail needs ~17 MB (a 32 MiB buffer), grow the stream's buffer with
    an eager call that needs ~35 MB, then replay."""
    import ctypes

    import torch
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    props = torch.cuda.get_device_properties(cuda)
    if props.multi_processor_count != 256:
        pytest.skip(f"the split plan assumes 256 CUs, the device has {props.multi_processor_count}")
    g0 = torch.Generator(device=cuda).manual_seed(6)

    def qkv(H, Lq, Lk):
        q = torch.nn.functional.normalize(torch.randn((1, H, Lq, 64), generator=g0, device=cuda), dim=-1) * 8
        k = torch.nn.functional.normalize(torch.randn((1, H, Lk, 64), generator=g0, device=cuda), dim=-1) * 8
        v = torch.randn((1, H, Lk, 64), generator=g0, device=cuda)
        return q, k, v

    small = qkv(16, 8292, 512)       # 272 tiles: 16 split 8 ways (17.3 MB)
    large = qkv(16, 8704, 1024)      # 272 tiles: 16 split 16 ways (34.6 MB)
    expected = native_sdpa_f32_ex(*small)
    expected_large = native_sdpa_f32_ex(*large)
    out = torch.empty_like(expected)
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)
    with torch.cuda.stream(s):
        native_sdpa_f32_ex(*small, out=out)
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        native_sdpa_f32_ex(*small, out=out)
    torch.cuda.synchronize(cuda)
    vals = [ctypes.c_uint64(0) for _ in range(2)]
    assert hiplib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(v) for v in vals]) == 0
    allocations = vals[0].value
    with torch.cuda.stream(s):
        got_large = native_sdpa_f32_ex(*large)
    torch.cuda.synchronize(cuda)
    assert hiplib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(v) for v in vals]) == 0
    assert vals[0].value == allocations + 1        # the large call grew s's buffer
    assert torch.equal(got_large, expected_large)
    canaries = _canaries(torch, cuda)
    torch.cuda.synchronize(cuda)
    for _ in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, expected)
        with torch.cuda.stream(s):
            assert torch.equal(native_sdpa_f32_ex(*large), expected_large)
        torch.cuda.synchronize(cuda)
    for c in canaries:
        assert bool((c == 1234.5).all())
