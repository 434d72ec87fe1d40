"""C-ABI and host-side checks that need no GPU.

* libtsplat_hip.so loads and exports every function include/tsplat_hip.h
  declares (and the Python signature table covers exactly that set);
* pure query symbols return the reference's values;
* argument validation returns the reference's status codes before any
  device call (scripts/gemm_nf24_i16_avx512.c:171-175,
  scripts/native_sdpa_avx512_exact_q8t512.c:151-153);
* the Python wrappers keep the reference's error behaviour, with the device
  check flipped (CPU tensors are rejected).
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tsplat_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text)
    skip = {"if", "defined"}
    return sorted({n for n in names if n not in skip and (n.startswith("triposplat_") or n.startswith("tsplat_"))})


@pytest.fixture(scope="module")
def lib():
    from tsplat import load_library

    return load_library()


def test_every_declared_symbol_is_exported(lib):
    from tsplat._lib import SIGNATURES

    declared = _declared()
    assert len(declared) >= 25
    for name in declared:
        assert hasattr(lib, name), name
    assert set(SIGNATURES) == set(declared)


def test_loader_checks_abi_version(lib, monkeypatch):
    """The bindings' argument lists are those of ABI_VERSION; a library that
    reports another version is refused at load time, not called with shifted
    arguments."""
    from tsplat import _lib

    assert lib.tsplat_abi_version() == _lib.ABI_VERSION
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION - 1)
    monkeypatch.setattr(_lib, "_CACHE", {})
    with pytest.raises(RuntimeError, match="ABI version"):
        _lib.load_library()


def test_query_symbols(lib):
    assert lib.triposplat_gemm_rnf8_avx512_residual_mode() == 4
    assert lib.triposplat_gemm_nf24_qkv_direct_residual_mode() == 4
    assert lib.triposplat_gemm_nf24_qkv_direct_row_tile() > 0
    assert lib.triposplat_gemm_nf24_qkv_direct_tile_bytes() == 0
    assert lib.triposplat_gemm_rnf8_avx512_row_tile() > 0
    assert lib.triposplat_sdpa_packed_output_is_blhd() == 1
    assert lib.triposplat_sdpa_key_tile() == 64
    assert lib.triposplat_sdpa_query_block() in (128, 512)   # the last launch's query tile
    assert lib.tsplat_abi_version() >= 1
    assert lib.tsplat_build_arch() == b"gfx950"
    import ctypes

    vals = [ctypes.c_uint64(7) for _ in range(5)]
    lib.triposplat_sdpa_q8t512_profile_reset()
    assert lib.triposplat_sdpa_q8t512_profile_get(*[ctypes.byref(v) for v in vals]) == 0
    assert [v.value for v in vals] == [0, 0, 0, 0, 0]
    assert lib.triposplat_sdpa_q8t512_profile_get(None, None, None, None, None) == -1
    stats = [ctypes.c_uint64(7) for _ in range(2)]
    assert lib.triposplat_sdpa_q8t512_workspace_stats(*[ctypes.byref(v) for v in stats]) == 0
    assert [v.value for v in stats] == [0, 0]          # no SDPA has needed a workspace here
    assert lib.triposplat_sdpa_q8t512_workspace_stats(None, None) == -1


def test_status_codes_before_any_device_call(lib):
    """Validation order and codes of the reference; dummy non-null pointers
    are never dereferenced because every case fails validation first."""
    P = [0x1000 + 16 * i for i in range(10)]
    g = lib.triposplat_gemm_rnf8_avx512_range
    nul = list(P)
    nul[7] = None  # codebook
    assert g(*nul, 4, 8, 32, 0, 32, 8, 32, 1, 3) == -1
    assert g(*P, 0, 8, 32, 0, 32, 8, 32, 1, 3) == -2        # M <= 0
    assert g(*P, 4, 8, 32, 0, 32, 8, 32, 1, 2) == -2        # stages != 3
    assert g(*P, 4, 8, 32, 16, 32, 8, 32, 1, 3) == -3       # start + count > N
    assert g(*P, 4, 8, 32, 0, 32, 7, 32, 1, 3) == -3        # stride_x < K
    assert g(*P, 4, 8, 32, 8, 16, 8, 16, 1, 3) == -4        # start % 16
    assert lib.triposplat_gemm_rnf8_avx512(*P, 4, 8, 40, 8, 40, 1, 3) == -4   # N % 16 -> use _tail
    assert lib.triposplat_gemm_rnf8_avx512_tail(*P, 4, 8, 40, 8, 39, 1, 3) == -2
    s = lib.triposplat_sdpa_f32_avx512_exact_q8t512
    assert s(None, P[1], P[2], None, P[4], 1, 2, 16, 16, 64, 0, 0, 1) == -1
    assert s(P[0], P[1], P[2], None, P[4], 1, 2, 16, 16, 32, 0, 0, 1) == -2   # D != 64
    assert s(P[0], P[1], P[2], None, P[4], 1, 2, 16, 16, 64, 1, 16, 1) == -3  # bias null
    assert s(P[0], P[1], P[2], P[3], P[4], 1, 2, 16, 16, 64, 1, 15, 1) == -3  # bias len
    pk = lib.triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd
    assert pk(P[0], P[1], P[2], None, P[4], 1, 2, 16, 20, 64, 24, 0, 0, 1) == -2  # Lkp % 16
    assert pk(P[0], P[1], P[2], None, P[4], 1, 2, 16, 20, 64, 16, 0, 0, 1) == -2  # Lkp < Lk
    for post in (lib.triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2,
                 lib.triposplat_qkv_rope_rmsnorm_pack_f32_avx512):
        assert post(*P[:7], 1, 20, 2, 64, 24, 1, 1) == -2      # L_padded % 16
        assert post(*P[:7], 2, 20, 2, 64, 32, 3, 1) == -2      # frequency_batches
        assert post(None, *P[1:7], 1, 20, 2, 64, 32, 1, 1) == -1
    assert lib.triposplat_qkv_postprocess_token_tile() == 64
    assert lib.triposplat_qkv_postprocess_v2_tail_only_clear() == 1
    d = lib.triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512
    assert d(*(P + P[:5]), 1, 20, 128, 384, 2, 64, 32, 1, 1, 2) == -2   # stages
    assert d(*(P + P[:5]), 1, 20, 128, 380, 2, 64, 32, 1, 1, 3) == -2   # N != 3*H*64


def test_wrappers_reject_cpu_tensors():
    import torch
    from tsplat.native_sdpa_ctypes import native_sdpa_f32, native_sdpa_f32_ex

    q = torch.zeros(1, 2, 16, 64)
    with pytest.raises(ValueError, match="GPU-only"):
        native_sdpa_f32(q, q, q)
    with pytest.raises(ValueError, match="GPU"):
        native_sdpa_f32_ex(q, q, q)


def test_patch_rejects_other_residual_modes():
    """Asking for a mode the library does not implement raises the
    reference's mismatch error (native_linear_rnf8_avx512_patch.py:196-200)."""
    import torch.nn as nn
    from tsplat.native_linear_rnf8_patch import apply_triposplat_native_rnf8_avx512_patch as patch

    m = nn.Sequential(nn.Linear(8, 16))
    assert patch(m, enabled=False) == {"enabled": False}
    with pytest.raises(ValueError):
        patch(m, enabled=True, strict=False)
    with pytest.raises(ValueError):
        patch(m, enabled=True, residual_mode="nf24_i16", stages=2)
    with pytest.raises(RuntimeError, match="mismatch"):
        patch(m, enabled=True, residual_mode="nf8", stages=2)


def test_nf8_codebook_matches_closed_form():
    import torch
    from tsplat.nf24 import make_nf8_codebook, nf8_levels

    cb = make_nf8_codebook(torch).numpy()
    assert cb.shape == (256,) and cb.dtype == np.float32
    assert cb[0] == -1.0 and cb[-1] == 1.0 and np.count_nonzero(cb == 0.0) == 2
    assert np.all(np.diff(cb) >= 0)
    lv = np.array(nf8_levels())
    assert np.allclose(lv, -lv[::-1], atol=1e-15)


def test_precision_and_layout_validation_before_any_device_call(lib):
    """The opt-in precision / K-V layout entry points reject unknown values
    with -2 before any pointer is examined (dummy pointers)."""
    P = [0x1000 + 16 * i for i in range(11)]
    g = lib.tsplat_nf24_gemm_precision_async
    assert g(*P[:6], 64, 64, 64, 0, 64, 64, 64, 0, None, 0, 1, 3, None) == -2   # precision 3
    assert g(*P[:6], 64, 64, 64, 0, 64, 64, 64, 1, None, 0, 1, 1, None) == -2   # epilogue 1 (QKV only)
    assert g(*P[:6], 64, 64, 64, 32, 64, 64, 64, 0, None, 0, 1, 1, None) == -3  # range past N
    d = lib.tsplat_gemm_nf24_qkv_direct_ex_async
    assert d(*P, 1, 20, 128, 384, 2, 64, 32, 1, 2, 0, 0, None) == -2   # kv_layout 2
    assert d(*P, 1, 20, 128, 384, 2, 64, 32, 1, 0, 7, 0, None) == -2   # precision 7
    assert d(*P, 1, 20, 128, 380, 2, 64, 32, 1, 1, 0, 0, None) == -2   # N != 3*H*64
    assert d(*P, 1, 20, 128, 384, 2, 64, 32, 1, 0, 0, 4, None) == -2   # kv_round 4
    s = lib.tsplat_sdpa_precision_async
    assert s(*P[:5], 1, 2, 16, 16, 64, 0, 0, 0, 0, 0, 0, 3, None) == -2     # precision 3
    assert s(*P[:5], 1, 2, 16, 16, 64, 0, 0, 0, 0, 0, 0, -1, None) == -2    # precision -1
    assert s(*P[:5], 1, 2, 16, 16, 32, 0, 0, 0, 0, 0, 0, 2, None) == -2     # D != 64


def test_python_wrappers_reject_bad_options():
    import torch
    from tsplat.nf24 import nf24_linear, precision_id
    from tsplat.qkv import gemm_nf24_qkv_direct

    assert [precision_id(p) for p in ("fp32", "bf16", "bf16x3")] == [0, 1, 2]
    z = torch.zeros(4, 4)
    with pytest.raises(ValueError, match="precision"):
        nf24_linear(z, z, z, z, z, precision="fp16")
    with pytest.raises(ValueError, match="kv_layout"):
        gemm_nf24_qkv_direct(z, z, z, z, z, z, z, z, 1, 4, 1, kv_layout="bshd")
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    q = torch.zeros(1, 2, 16, 64)
    with pytest.raises(ValueError, match="precision"):
        native_sdpa_f32_ex(q, q, q, precision="fp16")


def test_bench_refuses_more_than_one_gpu():
    import json
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_kv_bf16_round_is_per_call(lib):
    """The K/V bf16 probe mode is a per-call argument, not library state: the
    reference-named postprocess entries report the exact build (0), a mode
    outside 0..3 is -2 before any pointer is examined, and the Python
    wrappers reject unknown mode names."""
    from tsplat.qkv import kv_round_id

    assert lib.triposplat_qkv_postprocess_bf16_probe_mode() == 0
    P = [0x1000 + 16 * i for i in range(7)]
    for bad in (-1, 4):
        assert lib.tsplat_qkv_postprocess_async(*P, 1, 16, 2, 64, 16, 1, bad, None) == -2
    assert [kv_round_id(m) for m in (None, "k", "v", "kv")] == [0, 1, 2, 3]
    with pytest.raises(ValueError, match="kv_round"):
        kv_round_id("q")
    assert lib.triposplat_qkv_postprocess_bf16_probe_mode() == 0


def test_sdpa_layout_validation(lib):
    """kv_packed other than 0 / 1, or a packed stride short of Lk / not a
    multiple of 16, is -2 before any pointer is examined."""
    P = [0x1000 + 16 * i for i in range(5)]
    s = lib.tsplat_sdpa_precision_async
    assert s(*P, 1, 2, 16, 20, 64, 0, 0, 0, 2, 32, 0, 0, None) == -2
    assert s(*P, 1, 2, 16, 20, 64, 0, 0, 0, 1, 16, 0, 0, None) == -2
    assert s(*P, 1, 2, 16, 20, 64, 0, 0, 0, 1, 24, 0, 0, None) == -2


def test_block_patches_disabled_and_missing_library():
    """Disabled patches touch nothing; a missing library is reported at
    patch time, as the reference's patches report theirs."""
    import torch
    from tsplat import native_block_patches as P

    for fn in (P.apply_triposplat_native_gelu_avx512_patch, P.apply_triposplat_native_silu_avx512_patch,
               P.apply_triposplat_native_norm_rope_avx512_patch,
               P.apply_triposplat_native_block_elementwise_avx512_patch):
        assert fn(None) == {"enabled": False}
    with pytest.raises(FileNotFoundError):
        P.apply_triposplat_native_silu_avx512_patch(torch.nn.Sequential(torch.nn.SiLU()), enabled=True,
                                                    library_path="/nonexistent/libtsplat_hip.so")


def test_sampler_backend_reference_name():
    from tsplat import native_sampler_backend as nsb

    assert nsb.NativeSamplerAVX512Backend is nsb.NativeSamplerBackend
    assert nsb.create_triposplat_native_sampler_avx512_backend() == (None, {"enabled": False})
