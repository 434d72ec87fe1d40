"""tsplat -- gfx950 (MI355X) NF24 packed-weight Linear and exact SDPA for
TripoSplat's flow model, behind the reference's Python/ctypes interface.

Modules mirror the reference files they replace:
  native_sdpa_ctypes        <- scripts/native_sdpa_ctypes.py
  native_linear_rnf8_patch  <- scripts/native_linear_rnf8_avx512_patch.py
  nf24                      <- the NF24 packer / decode of
                               scripts/native_linear_rnf8_avx512_patch.py and
                               scripts/native_linear_nf24_prepacked.py
  qkv                       <- scripts/native_qkv_postprocess_v2_avx512.c and
                               scripts/gemm_nf24_qkv_direct_avx512.c entry points
Every compute call goes to libtsplat_hip.so; there is no CPU fallback.
"""
from ._lib import DEFAULT_LIBRARY, library_path, load_library

__all__ = ["DEFAULT_LIBRARY", "library_path", "load_library"]
