"""Loader for libtsplat_hip.so (gfx950 kernels behind a C ABI).

torch is imported before the library is opened so that the HIP runtime torch
already loaded (SONAME libamdhip64.so.7) is the one the library binds to.
There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
DEFAULT_LIBRARY = PACKAGE_DIR / "lib" / "libtsplat_hip.so"

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64

# name -> (argtypes, restype); the C declarations are in include/tsplat_hip.h.
SIGNATURES = {
    "triposplat_gemm_rnf8_avx512": ([_vp] * 10 + [_i] * 7, _i),
    "triposplat_gemm_rnf8_avx512_range": ([_vp] * 10 + [_i] * 9, _i),
    "triposplat_gemm_rnf8_avx512_tail": ([_vp] * 10 + [_i] * 7, _i),
    "triposplat_gemm_rnf8_avx512_row_tile": ([], _i),
    "triposplat_gemm_rnf8_avx512_residual_mode": ([], _i),
    "tsplat_nf24_gemm_async": ([_vp] * 6 + [_i] * 7 + [_vp], _i),
    "triposplat_sdpa_f32_avx512_exact_q8t512": ([_vp] * 5 + [_i] * 8, _i),
    "triposplat_sdpa_f32": ([_vp] * 5 + [_i] * 8, _i),
    "triposplat_sdpa_f32_avx512_exact_q8": ([_vp] * 5 + [_i] * 8, _i),
    "triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd": ([_vp] * 5 + [_i] * 9, _i),
    "triposplat_sdpa_key_tile": ([], _i),
    "triposplat_sdpa_query_block": ([], _i),
    "triposplat_sdpa_packed_output_is_blhd": ([], _i),
    "triposplat_sdpa_q8t512_profile_reset": ([], None),
    "triposplat_sdpa_q8t512_profile_get": ([ctypes.POINTER(ctypes.c_uint64)] * 5, _i),
    "triposplat_sdpa_q8t512_workspace_stats": ([ctypes.POINTER(ctypes.c_uint64)] * 2, _i),
    "triposplat_sdpa_q8t512_workspace_release": ([], None),
    "tsplat_sdpa_async": ([_vp] * 5 + [_i] * 7 + [_i64] + [_i] * 3 + [_vp], _i),
    "tsplat_sdpa_precision_async": ([_vp] * 5 + [_i] * 7 + [_i64] + [_i] * 4 + [_vp], _i),
    "tsplat_sdpa_noalloc_async": ([_vp] * 5 + [_i] * 7 + [_i64] + [_i] * 4 + [_vp], _i),
    "triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2": ([_vp] * 7 + [_i] * 7, _i),
    "triposplat_qkv_rope_rmsnorm_pack_f32_avx512": ([_vp] * 7 + [_i] * 7, _i),
    "triposplat_qkv_postprocess_token_tile": ([], _i),
    "triposplat_qkv_postprocess_v2_tail_only_clear": ([], _i),
    "triposplat_qkv_postprocess_bf16_probe_mode": ([], _i),
    "triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512": ([_vp] * 15 + [_i] * 10, _i),
    "triposplat_gemm_nf24_qkv_direct_row_tile": ([], _i),
    "triposplat_gemm_nf24_qkv_direct_tile_bytes": ([], _i),
    "triposplat_gemm_nf24_qkv_direct_residual_mode": ([], _i),
    "triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2": ([_vp] * 9 + [_i] * 8, _i),
    "tsplat_q_kv_selected_postprocess_async": ([_vp] * 9 + [_i] * 8 + [_vp], _i),
    "tsplat_qkv_postprocess_async": ([_vp] * 7 + [_i] * 7 + [_vp], _i),
    "tsplat_gemm_nf24_qkv_direct_async": ([_vp] * 11 + [_i] * 8 + [_vp], _i),
    "tsplat_gemm_nf24_qkv_direct_ex_async": ([_vp] * 11 + [_i] * 11 + [_vp], _i),
    "tsplat_nf24_pack_async": ([_vp, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp], _i),
    "tsplat_nf24_decode_async": ([_vp] * 4 + [_i] * 3 + [_vp], _i),
    "tsplat_nf24_gemm_epilogue_async": ([_vp] * 6 + [_i] * 8 + [_vp, _i64, _i, _vp], _i),
    "tsplat_nf24_gemm_precision_async": ([_vp] * 6 + [_i] * 8 + [_vp, _i64, _i, _i, _vp], _i),
    "tsplat_nf24_gemm_planes_async": ([_vp] * 6 + [_i] * 8 + [_vp, _i64, _i, _i, _vp, _vp, _vp], _i),
    "tsplat_nf24_bf16_planes_async": ([_vp] * 3 + [_i] * 3 + [_vp] * 3, _i),
    "tsplat_gemm_nf24_qkv_direct_planes_async": ([_vp] * 11 + [_i] * 11 + [_vp] * 3, _i),
    "triposplat_layernorm_f32_avx512": ([_vp] * 4 + [_i64, _i, ctypes.c_float, _i, _i], _i),
    "triposplat_multihead_rmsnorm_f32_avx512": ([_vp] * 3 + [_i64, _i, _i, ctypes.c_float, _i], _i),
    "triposplat_rope_complex_f32_avx512": ([_vp] * 3 + [_i64, _i, _i], _i),
    "triposplat_modulate_inplace_f32_avx512": ([_vp] * 3 + [_i] * 4, _i),
    "triposplat_gated_residual_inplace_f32_avx512": ([_vp] * 3 + [_i] * 4, _i),
    "triposplat_add_inplace_f32_avx512": ([_vp] * 2 + [_i64, _i], _i),
    "triposplat_gelu_tanh_f32_avx512": ([_vp] * 2 + [_i64, _i], _i),
    "triposplat_silu_f32_avx512": ([_vp] * 2 + [_i64, _i], _i),
    "triposplat_cfg_combine_inplace_f32_avx512": ([_vp] * 3 + [_i, _i64, _i], _i),
    "triposplat_euler_update_inplace_f32_avx512": ([_vp] * 3 + [_i, _i64, _i], _i),
    "triposplat_ab2_update_inplace_f32_avx512": ([_vp] * 5 + [_i, _i64, _i], _i),
    "tsplat_layernorm_modulate_async": ([_vp] * 4 + [_i64, _i, ctypes.c_float, _i, _vp, _vp, _i64,
                                         _i64, _vp], _i),
    "tsplat_head_rmsnorm_async": ([_vp, _i64, _vp, _vp] + [_i] * 4 + [ctypes.c_float, _i, _i, _vp], _i),
    "tsplat_rope_complex_async": ([_vp] * 3 + [_i64, _i, _vp], _i),
    "tsplat_modulate_async": ([_vp] * 3 + [_i] * 3 + [_vp], _i),
    "tsplat_gated_residual_async": ([_vp] * 3 + [_i] * 3 + [_vp], _i),
    "tsplat_add_async": ([_vp] * 2 + [_i64, _vp], _i),
    "tsplat_gelu_tanh_async": ([_vp] * 2 + [_i64, _vp], _i),
    "tsplat_silu_async": ([_vp] * 2 + [_i64, _vp], _i),
    "tsplat_cfg_combine_async": ([_vp] * 3 + [_i, _i64, _vp], _i),
    "tsplat_euler_update_async": ([_vp] * 3 + [_i, _i64, _vp], _i),
    "tsplat_ab2_update_async": ([_vp] * 5 + [_i, _i64, _vp], _i),
    "tsplat_abi_version": ([], _i),
    "tsplat_last_hip_error": ([], _i),
    "tsplat_build_arch": ([], ctypes.c_char_p),
}

STATUS_TEXT = {
    -1: "null pointer",
    -2: "bad sizes / stages / head dim",
    -3: "range, stride or key-bias length mismatch",
    -4: "range not 16-aligned or pointer not 16-byte aligned",
    -5: "device workspace allocation failed",
    -6: "not device memory of the current device, or allocation too small",
    -7: "HIP launch / runtime error",
    -8: "needs more scratch than the no-allocation entry point's static buffer",
}

# tsplat_abi_version() of the library these bindings describe: it moves
# whenever an entry's argument list changes (ABI 3 put kv_round before the
# stream argument of the asynchronous QKV entries: a library reporting another
# version would read its arguments shifted) or entries are added (ABI 4: the
# bf16 weight planes).
ABI_VERSION = 4

_CACHE: dict[str, ctypes.CDLL] = {}


def library_path(path: str | os.PathLike | None = None) -> Path:
    if path is not None:
        return Path(path).resolve()
    env = os.environ.get("TSPLAT_HIP_LIBRARY")
    return Path(env).resolve() if env else DEFAULT_LIBRARY


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Open libtsplat_hip.so once per path and set every argtypes/restype."""
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)

    resolved = library_path(path)
    key = resolved.as_posix()
    lib = _CACHE.get(key)
    if lib is not None:
        return lib
    if not resolved.is_file():
        raise FileNotFoundError(
            f"libtsplat_hip.so not found at {resolved}; build it with "
            "`make -C triposplat-cpu-avx512_amd` (there is no CPU fallback)"
        )
    lib = ctypes.CDLL(key)
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    found = lib.tsplat_abi_version()
    if found != ABI_VERSION:
        raise RuntimeError(
            f"{resolved} reports ABI version {found}, these bindings expect {ABI_VERSION}; "
            "rebuild it with `make -C triposplat-cpu-avx512_amd`"
        )
    _CACHE[key] = lib
    return lib


def check_status(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} returned status {status} ({STATUS_TEXT.get(status, 'unknown')})")


def current_stream_handle(device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    import torch

    return int(torch.cuda.current_stream(device).cuda_stream)
