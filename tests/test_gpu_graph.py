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


def test_graph_few_row_gemm(cuda):
    import torch
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel

    g0 = torch.Generator(device=cuda).manual_seed(3)
    M, K, N = 2, 1024, 3072                          # few-row kernel with a K split
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
