"""The reference-named SDPA entry points, called on the device through the C ABI.

scripts/native_sdpa_ctypes.py:10-76 binds `triposplat_sdpa_f32_avx512_exact_q8`
by default (any symbol of the same ABI through `symbol=` or
TRIPOSPLAT_NATIVE_SDPA_SYMBOL); the q8t512 library also exports
`triposplat_sdpa_f32` (native_sdpa_avx512_exact_q8t512.c:334-351) and the
packed/BLHD entry (native_sdpa_avx512_exact_q8t512_packed.c:3-158).  Each is
checked here against the oracle (bit-exact with the reference build) on:

- a self-attention shape with the reference's log(7) key bias
  (scripts/smoke_custom_sdpa_backend.py:121-133),
- a cross shape (Lq != Lk),
- a grid large enough that the last round of 512-query tiles is split
  along the keys into the library's workspace (sampled query rows; rows are
  independent, so the oracle computes them exactly).

The probes (query tile, workspace stats, the blocking-call profile) are
checked against what the calls did.  Tolerance: tests/_parity.py.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from _parity import SDPA_ATOL_PER_MAXV, SDPA_RMSE_PER_RMSV, stats

pytestmark = pytest.mark.gpu

BLOCKING = ["triposplat_sdpa_f32_avx512_exact_q8", "triposplat_sdpa_f32",
            "triposplat_sdpa_f32_avx512_exact_q8t512"]


def _qkv(seed, B, H, Lq, Lk):
    r = np.random.default_rng(seed)
    return (r.standard_normal((B, H, Lq, 64), dtype=np.float32),
            r.standard_normal((B, H, Lk, 64), dtype=np.float32),
            r.standard_normal((B, H, Lk, 64), dtype=np.float32))


def _close(got, ref, v):
    s = stats(got, ref)
    assert np.all(np.isfinite(got))
    assert s["max_abs"] <= SDPA_ATOL_PER_MAXV * float(np.abs(v).max()), s
    assert s["rmse"] <= SDPA_RMSE_PER_RMSV * float(np.sqrt(np.mean(v.astype(np.float64) ** 2))), s


def _profile(lib):
    vals = [ctypes.c_uint64(0) for _ in range(5)]
    assert lib.triposplat_sdpa_q8t512_profile_get(*[ctypes.byref(v) for v in vals]) == 0
    return [v.value for v in vals]


def _workspace(lib):
    vals = [ctypes.c_uint64(0) for _ in range(2)]
    assert lib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(v) for v in vals]) == 0
    return [v.value for v in vals]


CASES = [(1, 2, 17, 17, "log7"), (1, 2, 15, 19, None), (2, 3, 40, 530, "uniform")]


def _bias(spec, Lk):
    if spec is None:
        return None
    if spec == "log7":
        b = np.zeros(Lk, np.float32)
        b[0] = np.float32(math.log(7.0))
        return b
    return np.random.default_rng(Lk).uniform(-2.0, 0.0, Lk).astype(np.float32)


@pytest.mark.parametrize("symbol", BLOCKING + [None])
@pytest.mark.parametrize("B,H,Lq,Lk,bspec", CASES)
def test_native_sdpa_f32_symbols(oracle, cuda, hiplib, symbol, B, H, Lq, Lk, bspec):
    """native_sdpa_f32(symbol=...) with each reference-named symbol and the
    default (None: the reference's default name), against the oracle."""
    import torch
    from tsplat.native_sdpa_ctypes import DEFAULT_SYMBOL, native_sdpa_f32

    assert DEFAULT_SYMBOL == "triposplat_sdpa_f32_avx512_exact_q8"
    print(f"sdpa abi symbol={symbol} B={B} H={H} Lq={Lq} Lk={Lk} bias={bspec}", flush=True)
    q, k, v = _qkv(100 + Lq + Lk, B, H, Lq, Lk)
    bias = _bias(bspec, Lk)
    t = lambda a: torch.from_numpy(a).to(cuda)
    hiplib.triposplat_sdpa_q8t512_profile_reset()
    got = native_sdpa_f32(t(q), t(k), t(v), key_bias=None if bias is None else t(bias), symbol=symbol)
    ref = oracle.sdpa_q8t512(q, k, v, bias)
    _close(got.cpu().numpy(), ref, v)
    calls, alloc_ns, pack_ns, compute_ns, free_ns = _profile(hiplib)
    assert calls == 1 and compute_ns > 0 and pack_ns == 0
    assert hiplib.triposplat_sdpa_query_block() == 128   # a grid below one 512-query tile per CU


def test_blocking_symbols_direct_ctypes(oracle, cuda):
    """The binding a reference user writes: an unmodified reference ctypes
    binding (argtypes of scripts/native_sdpa_ctypes.py:18-19) on the library
    file, device pointers, the reference's `threads` argument."""
    import torch
    from tsplat._lib import DEFAULT_LIBRARY

    lib = ctypes.CDLL(str(DEFAULT_LIBRARY))
    q, k, v = _qkv(7, 1, 2, 17, 17)
    bias = _bias("log7", 17)
    ref = oracle.sdpa_q8t512(q, k, v, bias)
    qd, kd, vd, bd = (torch.from_numpy(a).to(cuda) for a in (q, k, v, bias))
    torch.cuda.synchronize()
    for name in BLOCKING:
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8
        fn.restype = ctypes.c_int
        out = torch.full_like(qd, float("nan"))
        torch.cuda.synchronize()
        st = fn(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), bd.data_ptr(), out.data_ptr(),
                1, 2, 17, 17, 64, 1, 17, 4)
        assert st == 0, (name, st)
        _close(out.cpu().numpy(), ref, v)
        # the reference's argument errors, before any launch
        assert fn(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), bd.data_ptr(), out.data_ptr(),
                  1, 2, 17, 17, 64, 1, 16, 4) == -3
        assert fn(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), None, out.data_ptr(),
                  1, 2, 17, 17, 32, 0, 0, 4) == -2


@pytest.mark.parametrize("B,H,Lq,Lk,bspec", [(1, 2, 15, 19, None), (2, 3, 130, 70, "uniform")])
def test_packed_blhd_symbol(oracle, cuda, hiplib, B, H, Lq, Lk, bspec):
    """triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd (5 pointers + 9
    ints, native_qkv_packed_attention_patch_v3.py:33-36): packed K/V with a
    zero tail, BLHD output."""
    import torch

    q, k, v = _qkv(31 + Lk, B, H, Lq, Lk)
    bias = _bias(bspec, Lk)
    Lkp = (Lk + 15) // 16 * 16
    pk = np.zeros((B, H, 64, Lkp), np.float32)
    pv = np.zeros_like(pk)
    pk[..., :Lk] = k.transpose(0, 1, 3, 2)
    pv[..., :Lk] = v.transpose(0, 1, 3, 2)
    ref = oracle.sdpa_q8t512_packed_blhd(q, pk, pv, Lk, bias)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    qd, pkd, pvd = t(q), t(pk), t(pv)
    bd = None if bias is None else t(bias)
    out = torch.full((B, Lq, H, 64), float("nan"), device=cuda)
    hiplib.triposplat_sdpa_q8t512_profile_reset()
    torch.cuda.synchronize()
    st = hiplib.triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd(
        qd.data_ptr(), pkd.data_ptr(), pvd.data_ptr(), None if bd is None else bd.data_ptr(), out.data_ptr(),
        B, H, Lq, Lk, 64, Lkp, int(bias is not None), Lk if bias is not None else 0, 4)
    assert st == 0
    assert hiplib.triposplat_sdpa_packed_output_is_blhd() == 1
    _close(out.cpu().numpy(), ref, v)
    assert _profile(hiplib)[0] == 1


def test_blocking_symbol_key_split_workspace(oracle, cuda, hiplib):
    """A grid of 16 heads x 17 tiles of 512 queries = 272 workgroups on 256
    CUs: the 16 tiles of the last round are split along the keys into the
    library's workspace and merged.  Sampled rows of the first and last
    (split) tiles of four heads are compared with the oracle; the probes
    report the 512-query tile, the workspace and its allocation."""
    import torch

    B, H, Lq, Lk = 1, 16, 8704, 1024
    props = torch.cuda.get_device_properties(cuda)
    if props.multi_processor_count != 256:
        pytest.skip(f"the split plan assumes 256 CUs, the device has {props.multi_processor_count}")
    q, k, v = _qkv(5, B, H, Lq, Lk)
    bias = _bias("uniform", Lk)
    t = lambda a: torch.from_numpy(a).to(cuda)
    qd, kd, vd, bd = t(q), t(k), t(v), t(bias)
    out = torch.full_like(qd, float("nan"))
    hiplib.triposplat_sdpa_q8t512_profile_reset()
    torch.cuda.synchronize()
    for _ in range(2):   # the second call reuses the workspace: no allocation
        st = hiplib.triposplat_sdpa_f32_avx512_exact_q8(
            qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), bd.data_ptr(), out.data_ptr(),
            B, H, Lq, Lk, 64, 1, Lk, 4)
        assert st == 0
    assert hiplib.triposplat_sdpa_query_block() == 512
    allocations, capacity = _workspace(hiplib)
    assert allocations >= 1 and capacity >= 16 * 16 * 512 * 66 * 4
    calls, alloc_ns, pack_ns, compute_ns, _ = _profile(hiplib)
    assert calls == 2 and compute_ns > 0 and pack_ns == 0
    got = out.cpu().numpy()
    rows = np.r_[0:64, 8192:8256, 8640:8704]
    for h in (0, 5, 10, 15):
        ref = oracle.sdpa_q8t512(np.ascontiguousarray(q[:, h:h + 1, rows]), k[:, h:h + 1], v[:, h:h + 1], bias)
        _close(got[:, h:h + 1, rows], ref, v)
    # release frees the (uncaptured) buffer; the next call allocates again
    hiplib.triposplat_sdpa_q8t512_workspace_release()
    assert _workspace(hiplib)[1] == 0
    assert _profile(hiplib)[4] > 0   # free time recorded
    st = hiplib.triposplat_sdpa_f32_avx512_exact_q8t512(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), bd.data_ptr(), out.data_ptr(), B, H, Lq, Lk, 64, 1, Lk, 4)
    assert st == 0
    assert _workspace(hiplib)[0] == allocations + 1
    assert np.array_equal(out.cpu().numpy(), got)
