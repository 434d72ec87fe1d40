"""tsplat_sdpa_noalloc_async: the SDPA entry point that allocates nothing.

It must give the same bytes as tsplat_sdpa_precision_async (same launch
plan and LDS tiles; the key-split partials live in the static array, and
the precision entry may stage K/V in a pre-split pass), on two
calls in a row with the second smaller (the static array keeps the first
call's contents), in each precision and layout it shares with the existing
entry, and it must work where the workspace path cannot: captured into a
HIP graph on a stream that never ran an eager call.  The library's
workspace allocation count must not move.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(torch, cuda, seed, H, Lq, Lk, bias):
    g = torch.Generator(device=cuda).manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn((1, H, Lq, 64), generator=g, device=cuda), dim=-1) * 8
    k = torch.nn.functional.normalize(torch.randn((1, H, Lk, 64), generator=g, device=cuda), dim=-1) * 8
    v = torch.randn((1, H, Lk, 64), generator=g, device=cuda)
    b = (torch.rand((H, Lk), generator=g, device=cuda) * -2.0) if bias else None
    return q, k, v, b


def _packed(torch, t):
    """[1, H, Lk, 64] -> key-contiguous [1, H, 64, Lkp], Lkp = roundup16(Lk), tail keys zero."""
    _, H, Lk, _ = t.shape
    Lkp = -(-Lk // 16) * 16
    p = torch.zeros((1, H, 64, Lkp), device=t.device)
    p[..., :Lk] = t.transpose(2, 3)
    return p


def _call(lib, fn, torch, cuda, q, k, v, b, out, precision, blhd, Lk_packed=0):
    """Lk_packed > 0: k and v are key-contiguous [1, H, 64, Lkp] of Lk_packed keys."""
    _, H, Lq, _ = q.shape
    Lk = Lk_packed if Lk_packed else k.shape[2]
    Lkp = k.shape[3] if Lk_packed else 0
    return getattr(lib, fn)(q.data_ptr(), k.data_ptr(), v.data_ptr(), None if b is None else b.data_ptr(),
                            out.data_ptr(), 1, H, Lq, Lk, 64, int(b is not None), Lk if b is not None else 0,
                            Lk if b is not None else 0, int(bool(Lk_packed)), Lkp, int(blhd), precision,
                            torch.cuda.current_stream(cuda).cuda_stream)


def _allocations(lib):
    vals = [ctypes.c_uint64(0) for _ in range(2)]
    assert lib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(x) for x in vals]) == 0
    return vals[0].value


# (H, Lq, Lk, bias, precision, blhd, packed k/v): the first of each pair
# needs the key split (16 heads x 17 tiles of 512 queries on 256 CUs), the
# second is smaller than the first; every precision (0 fp32, 1 bf16,
# 2 bf16x3) and both K/V layouts
CALLS = [
    [(16, 8704, 1024, True, 0, True, False), (16, 8292, 512, False, 0, False, False)],
    [(16, 8704, 1024, False, 2, False, False), (16, 8500, 320, True, 2, True, False)],
    [(16, 8704, 1024, False, 1, True, True), (16, 8292, 520, True, 1, False, True)],
    [(16, 8704, 1000, True, 0, False, True), (16, 8500, 700, False, 2, True, True)],
]


@pytest.mark.parametrize("pair", range(len(CALLS)))
def test_noalloc_matches_precision_entry(cuda, hiplib, pair):
    import torch

    props = torch.cuda.get_device_properties(cuda)
    if props.multi_processor_count != 256:
        pytest.skip(f"the split shapes assume 256 CUs, the device has {props.multi_processor_count}")
    before = _allocations(hiplib)
    got_all, want_all = [], []
    for i, (H, Lq, Lk, bias, precision, blhd, packed) in enumerate(CALLS[pair]):
        print(f"noalloc pair {pair} call {i}: H={H} Lq={Lq} Lk={Lk} bias={bias} precision={precision} "
              f"blhd={blhd} packed={packed}", flush=True)
        q, k, v, b = _inputs(torch, cuda, 100 * pair + i, H, Lq, Lk, bias)
        if packed:
            k, v = _packed(torch, k), _packed(torch, v)
        shape = (1, Lq, H, 64) if blhd else (1, H, Lq, 64)
        got = torch.full(shape, float("nan"), device=cuda)
        assert _call(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, q, k, v, b, got, precision, blhd,
                     Lk if packed else 0) == 0
        torch.cuda.synchronize(cuda)
        got_all.append(got)
        want_all.append((q, k, v, b, shape, precision, blhd, Lk if packed else 0))
    assert _allocations(hiplib) == before          # no workspace allocation
    for got, (q, k, v, b, shape, precision, blhd, lkp) in zip(got_all, want_all):
        want = torch.full(shape, float("nan"), device=cuda)
        assert _call(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, b, want, precision, blhd,
                     lkp) == 0
        torch.cuda.synchronize(cuda)
        assert bool(torch.isfinite(got).all())
        assert torch.equal(got, want)


def test_noalloc_captured_without_warmup(cuda, hiplib):
    """Captured on a fresh stream with no eager call before it (the
    workspace path returns -5 there), replayed with eager work between
    replays: every replay equals the eager result bit for bit."""
    import torch

    props = torch.cuda.get_device_properties(cuda)
    if props.multi_processor_count != 256:
        pytest.skip(f"the split shapes assume 256 CUs, the device has {props.multi_processor_count}")
    q, k, v, b = _inputs(torch, cuda, 7, 16, 8704, 1024, True)
    want = torch.empty((1, 16, 8704, 64), device=cuda)
    assert _call(hiplib, "tsplat_sdpa_precision_async", torch, cuda, q, k, v, b, want, 0, False) == 0
    out = torch.empty_like(want)
    # set-up on this device (the scratch address lookup) by a small eager call
    # on the current stream -- not on the capture stream
    tiny = _inputs(torch, cuda, 10, 1, 16, 16, False)
    tiny_out = torch.empty_like(tiny[0])
    assert _call(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, *tiny, tiny_out, 0, False) == 0
    s = torch.cuda.Stream(device=cuda)
    torch.cuda.synchronize(cuda)
    before = _allocations(hiplib)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        assert _call(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, q, k, v, b, out, 0, False) == 0
    torch.cuda.synchronize(cuda)
    other = _inputs(torch, cuda, 8, 16, 8292, 512, False)
    other_out = torch.empty((1, 16, 8292, 64), device=cuda)
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, want)
        # an eager call between replays overwrites the shared scratch; ordered, so no race
        assert _call(hiplib, "tsplat_sdpa_noalloc_async", torch, cuda, *other, other_out, 0, False) == 0
        torch.cuda.synchronize(cuda)
    assert _allocations(hiplib) == before


_FIRST_CALL_CAPTURED = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
dev = torch.device("cuda", 0)
torch.cuda.set_device(dev)
g = torch.Generator(device=dev).manual_seed(5)
q = torch.nn.functional.normalize(torch.randn((1, 16, 8704, 64), generator=g, device=dev), dim=-1) * 8
k = torch.nn.functional.normalize(torch.randn((1, 16, 1024, 64), generator=g, device=dev), dim=-1) * 8
v = torch.randn((1, 16, 1024, 64), generator=g, device=dev)
out = torch.full_like(q, float("nan"))
want = torch.full_like(q, float("nan"))
s = torch.cuda.Stream(device=dev)
torch.cuda.synchronize(dev)
from tsplat import load_library
lib = load_library()
def call(fn, o, stream):
    return getattr(lib, fn)(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, o.data_ptr(), 1, 16, 8704, 1024,
                            64, 0, 0, 0, 0, 0, 0, 0, stream)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    st = call("tsplat_sdpa_noalloc_async", out, s.cuda_stream)
print("captured status", st, flush=True)
assert st == 0, st
for _ in range(2):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize(dev)
    assert bool(torch.isfinite(out).all())
assert call("tsplat_sdpa_precision_async", want, torch.cuda.current_stream(dev).cuda_stream) == 0
torch.cuda.synchronize(dev)
assert torch.equal(out, want)
print("first call captured: ok", flush=True)
"""


def test_noalloc_first_library_call_captured(cuda):
    """A fresh process whose first call into the library is a captured
    no-allocation SDPA (so the per-device scratch address is looked up
    inside the capture, with global capture mode), replayed twice: the
    capture succeeds and every replay equals the eager result bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    import torch

    props = torch.cuda.get_device_properties(cuda)
    if props.multi_processor_count != 256:
        pytest.skip(f"the split shape assumes 256 CUs, the device has {props.multi_processor_count}")
    pkg = Path(__file__).resolve().parents[1] / "triposplat-cpu-avx512_amd"
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, str(pkg)], capture_output=True, text=True,
                       timeout=100)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert "first call captured: ok" in r.stdout


def test_noalloc_argument_errors(cuda, hiplib):
    """The existing entry's argument checks, before any launch."""
    import torch

    q, k, v, _ = _inputs(torch, cuda, 9, 2, 16, 16, False)
    out = torch.empty_like(q)
    fn = hiplib.tsplat_sdpa_noalloc_async
    s = torch.cuda.current_stream(cuda).cuda_stream
    assert fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, out.data_ptr(), 1, 2, 16, 16, 32, 0, 0, 0, 0, 0, 0, 0,
              s) == -2                                   # D != 64
    assert fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, out.data_ptr(), 1, 2, 16, 16, 64, 0, 0, 0, 0, 0, 0, 5,
              s) == -2                                   # precision
    assert fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, out.data_ptr(), 1, 2, 16, 16, 64, 1, 16, 0, 0, 0, 0, 0,
              s) == -3                                   # bias null
    host = np.zeros((1, 2, 16, 64), np.float32)
    assert fn(host.ctypes.data, k.data_ptr(), v.data_ptr(), None, out.data_ptr(), 1, 2, 16, 16, 64, 0, 0, 0, 0, 0, 0,
              0, s) == -6                                # host pointer
