"""Flow-block elementwise kernels on the device.

Counterparts of the reference's AVX-512 block kernels and their Python
patches -- scripts/native_norm_rope_avx512.c (+ native_norm_rope_avx512_patch.py),
native_block_elementwise_avx512.c (+ native_block_elementwise_avx512_patch.py:18-40:
``modulate``, ``residual``, ``add_inplace``), native_gelu_avx512.c and
native_silu_avx512_extra.c -- with the same arithmetic per element, bit for
bit.  Every function takes contiguous fp32 tensors on the GPU, runs on
torch's current stream and raises on anything else (the reference's strict
mode: no torch fallback).
"""
from __future__ import annotations

from ._lib import check_status, current_stream_handle, load_library

# epilogue ids of tsplat_nf24_gemm_epilogue_async (include/tsplat_hip.h)
EPILOGUE_STORE, EPILOGUE_GELU, EPILOGUE_GATED, EPILOGUE_ADD = 0, 2, 3, 4


def _check(torch, name, t):
    if not (torch.is_tensor(t) and t.device.type == "cuda" and t.dtype == torch.float32
            and t.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous fp32 GPU tensor")


def _call(lib, fn_name, device, *args):
    import torch

    with torch.cuda.device(device):
        status = getattr(lib, fn_name)(*args, current_stream_handle(device))
    check_status(status, fn_name)


def layer_norm(x, eps, weight=None, bias=None, *, scale=None, shift=None, out=None, library=None):
    """LayerNorm over the last dim (native_norm_rope_avx512.c:13-49), optionally
    followed by the adaLN modulation y * (1 + scale[b]) + shift[b]
    (native_block_elementwise_avx512.c:9-22) in the same pass.  x is
    [..., C] with batch dim 0 when modulating; scale / shift are [B, C] views
    whose rows may be strided (e.g. chunks of a [B, 6C] tensor)."""
    import torch

    _check(torch, "x", x)
    C = int(x.shape[-1])
    rows = x.numel() // C
    out = torch.empty_like(x) if out is None else out
    _check(torch, "out", out)
    affine = weight is not None
    if affine:
        _check(torch, "weight", weight)
        _check(torch, "bias", bias)
    modulate = scale is not None
    stride, per_batch = 0, 1
    if modulate:
        B = int(x.shape[0])
        for name, t in (("scale", scale), ("shift", shift)):
            if (t.device.type != "cuda" or t.dtype != torch.float32 or t.dim() != 2
                    or int(t.shape[0]) != B or int(t.shape[1]) != C or t.stride(1) != 1):
                raise ValueError(f"{name} must be a [B, C] fp32 GPU tensor with unit column stride")
        if scale.stride(0) != shift.stride(0):
            raise ValueError("scale and shift must share the row stride")
        stride, per_batch = int(scale.stride(0)), rows // B
    lib = load_library(library)
    _call(lib, "tsplat_layernorm_modulate_async", x.device, x.data_ptr(),
          weight.data_ptr() if affine else None, bias.data_ptr() if affine else None, out.data_ptr(),
          rows, C, float(eps), int(affine), scale.data_ptr() if modulate else None,
          shift.data_ptr() if modulate else None, stride, per_batch)
    return out


def head_rmsnorm(x, gamma, B, L, H, *, dim=64, token_stride=None, eps=1.0e-12, out_bhld=True,
                 normalize=True, out=None, library=None):
    """Per-head RMSNorm x * sqrt(dim) / max(||x||, eps) * gamma[h]
    (native_norm_rope_avx512.c:51-83) of the vectors (b, l, h) stored at
    x + (b*L + l) * token_stride + h*dim, written [B, H, L, dim] (out_bhld) or
    [B, L, H, dim]; normalize=False only moves the vectors."""
    import torch

    if x.device.type != "cuda" or x.dtype != torch.float32:
        raise ValueError("x must be an fp32 GPU tensor")
    token_stride = H * dim if token_stride is None else int(token_stride)
    shape = (B, H, L, dim) if out_bhld else (B, L, H, dim)
    out = torch.empty(shape, dtype=torch.float32, device=x.device) if out is None else out
    _check(torch, "out", out)
    if normalize:
        _check(torch, "gamma", gamma)
    lib = load_library(library)
    _call(lib, "tsplat_head_rmsnorm_async", x.device, x.data_ptr(), token_stride,
          gamma.data_ptr() if normalize else None, out.data_ptr(), int(B), int(L), int(H), int(dim),
          float(eps), int(out_bhld), int(normalize))
    return out


def rope_complex(x, freqs, out=None, library=None):
    """Interleaved complex RoPE (native_norm_rope_avx512.c:85-119)."""
    import torch

    _check(torch, "x", x)
    _check(torch, "freqs", freqs)
    out = torch.empty_like(x) if out is None else out
    dim = int(x.shape[-1])
    lib = load_library(library)
    _call(lib, "tsplat_rope_complex_async", x.device, x.data_ptr(), freqs.data_ptr(), out.data_ptr(),
          x.numel() // dim, dim)
    return out


def modulate(h, scale, shift, library=None):
    """h [B, L, C] *= (1 + scale[B, C]), += shift[B, C], in place."""
    import torch

    for name, t in (("h", h), ("scale", scale), ("shift", shift)):
        _check(torch, name, t)
    B, L, C = (int(s) for s in h.shape)
    _call(load_library(library), "tsplat_modulate_async", h.device, h.data_ptr(), scale.data_ptr(),
          shift.data_ptr(), B, L, C)
    return h


def residual(x, h, gate, library=None):
    """h *= gate[B, C]; x += h (both in place), as the reference's gated residual."""
    import torch

    for name, t in (("x", x), ("h", h), ("gate", gate)):
        _check(torch, name, t)
    B, L, C = (int(s) for s in x.shape)
    _call(load_library(library), "tsplat_gated_residual_async", x.device, x.data_ptr(), h.data_ptr(),
          gate.data_ptr(), B, L, C)
    return x


def add_inplace(x, h, library=None):
    import torch

    _check(torch, "x", x)
    _check(torch, "h", h)
    if x.numel() != h.numel():
        raise ValueError("add_inplace operands differ in size")
    _call(load_library(library), "tsplat_add_async", x.device, x.data_ptr(), h.data_ptr(), x.numel())
    return x


def _unary(fn_name, x, out, library):
    import torch

    _check(torch, "x", x)
    out = torch.empty_like(x) if out is None else out
    _check(torch, "out", out)
    _call(load_library(library), fn_name, x.device, x.data_ptr(), out.data_ptr(), x.numel())
    return out


def gelu_tanh(x, out=None, library=None):
    """GELU, tanh form (native_gelu_avx512.c:44-68)."""
    return _unary("tsplat_gelu_tanh_async", x, out, library)


def silu(x, out=None, library=None):
    """SiLU (native_silu_avx512_extra.c:28-45)."""
    return _unary("tsplat_silu_async", x, out, library)


def nf24_linear_epilogue(x2, code01_t, q2_t, scale, bias, epilogue, *, out=None, gate=None,
                         rows_per_batch=None, precision="fp32", planes=None, library=None):
    """NF24 Linear with the next elementwise step applied before the store:
    EPILOGUE_GELU -> gelu_tanh(x @ W + b); EPILOGUE_GATED -> out += (x @ W + b) * gate[b];
    EPILOGUE_ADD -> out += x @ W + b.  gate is [B, N] (row stride may exceed N).
    precision and planes as tsplat.nf24.nf24_linear."""
    import torch

    from .nf24 import planes_pointers, precision_id

    mode = precision_id(precision)

    _check(torch, "x", x2)
    M, K = (int(s) for s in x2.shape)
    N = int(code01_t.shape[1])
    if out is None:
        if epilogue in (EPILOGUE_GATED, EPILOGUE_ADD):
            raise ValueError("the residual epilogues update `out` in place")
        out = torch.empty((M, N), dtype=torch.float32, device=x2.device)
    gate_stride, per_batch = 0, 1
    if epilogue == EPILOGUE_GATED:
        if gate is None or gate.dim() != 2 or gate.stride(1) != 1 or int(gate.shape[1]) != N:
            raise ValueError("gate must be [B, N] with unit column stride")
        gate_stride = int(gate.stride(0))
        per_batch = int(rows_per_batch) if rows_per_batch is not None else M // int(gate.shape[0])
    args = (x2.data_ptr(), code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(), bias.data_ptr(),
            out.data_ptr(), M, K, N, 0, N, int(x2.stride(0)), int(out.stride(0)), int(epilogue),
            gate.data_ptr() if gate is not None else None, gate_stride, per_batch)
    if mode == 0:
        _call(load_library(library), "tsplat_nf24_gemm_epilogue_async", x2.device, *args)
    elif planes is not None:
        _call(load_library(library), "tsplat_nf24_gemm_planes_async", x2.device, *args, mode,
              *planes_pointers(planes, K, N, mode))
    else:
        _call(load_library(library), "tsplat_nf24_gemm_precision_async", x2.device, *args, mode)
    return out
