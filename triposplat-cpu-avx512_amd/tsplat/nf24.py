"""NF24 weight format on the device: alphabet, packer, decode, GEMM call.

Format (residual mode id 4, "nf24_i16"), as the reference defines it in
scripts/native_linear_rnf8_avx512_patch.py:14-87 and
scripts/native_linear_nf24_prepacked.py:17-31:

    w[k, n] = fp32((int32)code01_t[k, n] * 256 + q2_t[k, n]) * scale[n]

code01_t int16 [in, out] holds 4*q0 + q1, q2_t int8 [in, out], scale fp32
[out] = max|W[n, :]| / 127 / 1024.  q0 is the nearest level of an integer
alphabet derived from a 256-entry normal-float codebook; q1 and q2 are
round-half-up residual digits in radix 4 and 256.
"""
from __future__ import annotations

import math
from statistics import NormalDist

from ._lib import check_status, current_stream_handle, load_library

RESIDUAL_MODE_ID = 4
FORMAT_NAME = "nf24_i16"


def nf8_levels():
    """The 256 normal-float levels as Python floats (float64): the 255
    quantiles sqrt(2)*erfinv(2p-1) at p = (i + 0.5)/255, scaled so that
    max |level| = 1, plus a second zero, sorted
    (scripts/native_linear_nf8_avx512_patch.py:12-20)."""
    nd = NormalDist()
    levels = [nd.inv_cdf((i + 0.5) / 255.0) for i in range(255)]
    peak = max(abs(x) for x in levels)
    levels = [x / peak for x in levels] + [0.0]
    return sorted(levels)


def make_nf8_codebook(torch_module):
    """fp32 codebook tensor [256] (the reference's make_nf8_codebook)."""
    return torch_module.tensor(nf8_levels(), dtype=torch_module.float64).float().contiguous()


def nf24_alphabet(torch_module, device=None):
    """unique(round(127 * codebook_f32)).clamp(-127, 127) as fp32
    (native_linear_rnf8_avx512_patch.py:24).  Every 127*level lies at least
    8e-3 away from a rounding tie, so float64 quantile error cannot move it."""
    torch = torch_module
    cb = make_nf8_codebook(torch)
    alphabet = torch.unique(torch.round(cb * 127.0).clamp_(-127, 127)).to(torch.float32)
    return alphabet.to(device) if device is not None else alphabet


def quantize_nf24_i16_per_output_channel(weight, codebook=None):
    """Pack an fp32 weight [out, in] on the GPU.

    Returns ([code01_t, q2_t, q2_t], [scale, scale, scale], error) with the
    reference's layout (native_linear_rnf8_avx512_patch.py:75-87).  The
    packing itself runs in the tsplat_nf24_pack_async kernel; ``error``
    reports the decoded-weight error against the source weight.
    """
    import torch

    if weight.dtype != torch.float32 or weight.ndim != 2:
        raise ValueError("NF24 packing requires a float32 2D weight")
    device = weight.device if weight.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    w = weight.detach().to(device).contiguous()
    out_f, in_f = (int(s) for s in w.shape)
    alphabet = nf24_alphabet(torch, device)
    base = torch.empty(out_f, dtype=torch.float32, device=device)
    code01_t = torch.empty((in_f, out_f), dtype=torch.int16, device=device)
    q2_t = torch.empty((in_f, out_f), dtype=torch.int8, device=device)
    scale = torch.empty(out_f, dtype=torch.float32, device=device)
    lib = load_library()
    with torch.cuda.device(device):
        status = lib.tsplat_nf24_pack_async(
            w.data_ptr(), out_f, in_f, alphabet.data_ptr(), int(alphabet.numel()), base.data_ptr(),
            code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(), current_stream_handle(device),
        )
    check_status(status, "tsplat_nf24_pack_async")
    error = _stage_errors(torch, w, base, alphabet)
    return [code01_t, q2_t, q2_t], [scale, scale, scale], error


def _stage_errors(torch, w, base, alphabet):
    """The packer's error report, keys and statistics as the reference's
    (native_linear_rnf8_avx512_patch.py:38-87): the residual left after each
    digit -- the NF8-derived level q0 at the base scale, then the radix-4 and
    radix-1024 corrections -- with its RMSE, max-abs and the count of
    corrections clamped to int8; weight_rmse / weight_max_abs are those of the
    last residual.  The digits are recomputed here with the same fp32
    elementwise steps as the packing kernel (the int16 code 4 q0 + q1 does not
    give the digits back); base is the kernel's max|row| / 127."""
    b = base[:, None]
    midpoints = ((alphabet[:-1] + alphabet[1:]) * 0.5).contiguous()
    q0 = alphabet[torch.bucketize(w / b, midpoints)]
    r1 = w - q0 * b
    s1 = b / 4.0
    q1u = torch.floor(r1 / s1 + 0.5)
    r2 = r1 - q1u.clamp(-128, 127) * s1
    s2 = b / 1024.0
    q2u = torch.floor(r2 / s2 + 0.5)
    r3 = r2 - q2u.clamp(-128, 127) * s2
    stages = []
    for stage, (rem, quantizer, unclamped) in enumerate(
            ((r1, "nf8_derived_int8_alphabet", None), (r2, "shared_scale_int8_radix4", q1u),
             (r3, "shared_scale_int8_radix256", q2u)), start=1):
        stages.append({
            "stage": stage,
            "quantizer": quantizer,
            "residual_rmse": float(torch.sqrt(torch.mean(rem * rem)).item()),
            "residual_max_abs": float(rem.abs().max().item()),
            "saturated_values": 0 if unclamped is None else int(((unclamped < -128) | (unclamped > 127)).sum().item()),
        })
    weight_rms = float(torch.sqrt(torch.mean(w * w)).item())
    return {
        "weight_rmse": stages[-1]["residual_rmse"],
        "weight_max_abs": stages[-1]["residual_max_abs"],
        "weight_rms": weight_rms,
        "weight_relative_rmse": stages[-1]["residual_rmse"] / max(weight_rms, 1.0e-30),
        "residual_mode": FORMAT_NAME,
        "nf8_derived_alphabet_size": int(alphabet.numel()),
        "stages": stages,
        "storage_layout": "int16(q0*4+q1) + int8(q2)",
    }


def _decode(code01_t, q2_t, scale, transposed):
    import torch

    if code01_t.dtype != torch.int16 or q2_t.dtype != torch.int8:
        raise ValueError("NF24 decode requires int16 code01_t and int8 q2_t")
    if tuple(code01_t.shape) != tuple(q2_t.shape):
        raise ValueError("NF24 code tensor shape mismatch")
    if scale.dtype != torch.float32 or scale.ndim != 1 or scale.numel() != code01_t.shape[1]:
        raise ValueError("NF24 scale shape mismatch")
    for name, t in (("code01_t", code01_t), ("q2_t", q2_t), ("scale", scale)):
        if t.device.type != "cuda" or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous GPU tensor")
    in_f, out_f = (int(s) for s in code01_t.shape)
    shape = (out_f, in_f) if transposed else (in_f, out_f)
    out = torch.empty(shape, dtype=torch.float32, device=code01_t.device)
    lib = load_library()
    with torch.cuda.device(code01_t.device):
        status = lib.tsplat_nf24_decode_async(code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(),
                                              out.data_ptr(), in_f, out_f, int(transposed),
                                              current_stream_handle(code01_t.device))
    check_status(status, "tsplat_nf24_decode_async")
    return out


def decode_nf24_i16_weight_t(code01_t, q2_t, scale):
    """Exact fp32 weights in the GEMM's [in, out] layout
    (scripts/native_linear_nf24_prepacked.py:17-31), decoded on the device."""
    return _decode(code01_t, q2_t, scale, False)


def decode_nf24_i16_weight(code01_t, q2_t, scale):
    """Exact fp32 weights as a contiguous [out, in] Linear weight
    (native_linear_nf24_prepacked.py:34-36)."""
    return _decode(code01_t, q2_t, scale, True)


# Product precision of the GEMM (tsplat_nf24_gemm_precision_async): "fp32" is
# the strict default; "bf16" and "bf16x3" are the opt-in bf16-MFMA modes.
PRECISIONS = {"fp32": 0, "bf16": 1, "bf16x3": 2}


def precision_id(precision) -> int:
    if precision not in PRECISIONS:
        raise ValueError(f"unknown product precision {precision!r}; expected one of {sorted(PRECISIONS)}")
    return PRECISIONS[precision]


def bf16_planes(code01_t, q2_t, scale, precision="bf16x3", library=None):
    """The bf16 planes of a packed weight for the opt-in modes
    (tsplat_nf24_bf16_planes_async): (w_hi, w_lo), bfloat16, w_hi = bf16(w)
    and for "bf16x3" w_lo = bf16 of the exact decode minus w_hi (None for
    "bf16") -- what the bf16 kernels otherwise decode and split from the
    codes in every call.  k-blocked: [ceil(K / 32), N, 32], weight (k, n) at
    [k // 32, n, k % 32], zeros past K (planes_to_kn gives [K, N]).  Pass them
    as planes= to nf24_linear, block_ops.nf24_linear_epilogue and
    qkv.gemm_nf24_qkv_direct: same results bit for bit, 2 (bf16) or 4
    (bf16x3) bytes per weight."""
    import torch

    mode = precision_id(precision)
    if mode == 0:
        raise ValueError("the bf16 planes serve precision 'bf16' or 'bf16x3'")
    K, N = (int(s) for s in code01_t.shape)
    w_hi = torch.empty(((K + 31) // 32, N, 32), dtype=torch.bfloat16, device=code01_t.device)
    w_lo = torch.empty_like(w_hi) if mode == 2 else None
    lib = load_library(library)
    with torch.cuda.device(code01_t.device):
        status = lib.tsplat_nf24_bf16_planes_async(
            code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(), K, N, mode, w_hi.data_ptr(),
            w_lo.data_ptr() if w_lo is not None else None, current_stream_handle(code01_t.device))
    check_status(status, "tsplat_nf24_bf16_planes_async")
    return w_hi, w_lo


def planes_to_kn(plane, K):
    """A k-blocked plane of bf16_planes as a [K, N] tensor (a view's copy)."""
    kb, N, _ = (int(s) for s in plane.shape)
    return plane.permute(0, 2, 1).reshape(kb * 32, N)[:K]


def planes_pointers(planes, K, N, mode):
    """(w_hi, w_lo) device pointers of bf16_planes' result for a call of
    precision id `mode` over a [K, N] weight."""
    import torch

    w_hi, w_lo = planes
    shape = ((K + 31) // 32, N, 32)
    for name, t in (("w_hi", w_hi), ("w_lo", w_lo if mode == 2 else w_hi)):
        if t is None or t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"planes: {name} must be a contiguous bfloat16 {list(shape)} tensor (bf16_planes)")
    return w_hi.data_ptr(), (w_lo.data_ptr() if mode == 2 else None)


def nf24_linear(x2, code01_t, q2_t, scale, bias, *, output_start=0, output_count=None, out=None,
                precision="fp32", planes=None, library=None):
    """out[M, count] = bias[start:start+count] + x2[M, K] @ W[:, start:start+count]
    on torch's current stream.  x2 must be a contiguous fp32 GPU matrix.
    precision "bf16" / "bf16x3" selects the opt-in bf16-MFMA products
    (include/tsplat_hip.h); M <= 32 always runs the strict kernels.  planes:
    bf16_planes(...) of this weight for those modes (same result)."""
    import torch

    mode = precision_id(precision)
    M, K = (int(s) for s in x2.shape)
    N = int(code01_t.shape[1])
    count = N - int(output_start) if output_count is None else int(output_count)
    if out is None:
        out = torch.empty((M, count), dtype=torch.float32, device=x2.device)
    lib = load_library(library)
    with torch.cuda.device(x2.device):
        stream = current_stream_handle(x2.device)
        args = (x2.data_ptr(), code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(), bias.data_ptr(),
                out.data_ptr(), M, K, N, int(output_start), count, int(x2.stride(0)), int(out.stride(0)))
        if mode == 0:
            name, status = "tsplat_nf24_gemm_async", lib.tsplat_nf24_gemm_async(*args, stream)
        elif planes is not None:
            name = "tsplat_nf24_gemm_planes_async"
            status = lib.tsplat_nf24_gemm_planes_async(*args, 0, None, 0, 1, mode,
                                                       *planes_pointers(planes, K, N, mode), stream)
        else:
            name = "tsplat_nf24_gemm_precision_async"
            status = lib.tsplat_nf24_gemm_precision_async(*args, 0, None, 0, 1, mode, stream)
    check_status(status, name)
    return out


def alphabet_tie_margin() -> float:
    """Smallest distance of any 127*level from a rounding tie."""
    margins = []
    for level in nf8_levels():
        scaled = 127.0 * level
        margins.append(abs(scaled - math.floor(scaled) - 0.5))
    return min(margins)
