"""Exact SDPA entry point: the device counterpart of the reference's
scripts/native_sdpa_ctypes.py:23-76 (``native_sdpa_f32``).

Same name, keyword arguments, default symbol
(``triposplat_sdpa_f32_avx512_exact_q8``, overridable by ``symbol=`` or
TRIPOSPLAT_NATIVE_SDPA_SYMBOL) and error behaviour, with the device check
flipped: q/k/v must be GPU tensors (the reference raises on non-CPU tensors,
this raises on non-GPU ones).  Inputs are cast to fp32 and made contiguous
and ``out`` is allocated here.  A reference-named symbol is blocking, as the
CPU call was: torch's current stream is waited for, the kernel runs on the
null stream and the call returns once it has finished.  The symbol
``tsplat_sdpa_async`` instead enqueues on torch's current stream and returns
at once.  A nonzero kernel status raises RuntimeError; nothing falls back to
torch.

``native_sdpa_f32_ex`` adds what the device path offers beyond the reference
ABI: a per-head key bias [H, Lk], key-contiguous packed K/V [B, H, 64, Lkp]
input, BLHD [B, Lq, H, 64] output and a caller-provided output buffer.
"""
from __future__ import annotations

import os

from ._lib import check_status, current_stream_handle, load_library

DEFAULT_SYMBOL = "triposplat_sdpa_f32_avx512_exact_q8"


def _as_f32_contig(t):
    import torch

    return t.to(dtype=torch.float32).contiguous()


def native_sdpa_f32(q, k, v, *, key_bias=None, library=None, symbol=None, threads=None):
    """softmax(q k^T / 8 + key_bias) v for q [B,H,Lq,64], k/v [B,H,Lk,64]; key_bias [Lk]."""
    import torch

    if q.device.type != "cuda" or k.device.type != "cuda" or v.device.type != "cuda":
        raise ValueError("native MI355X SDPA is GPU-only")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q/k/v must be [B,H,L,D]")
    if q.shape[:2] != k.shape[:2] or k.shape != v.shape:
        raise ValueError(f"unsupported q/k/v shapes: q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if int(q.shape[-1]) != 64 or int(k.shape[-1]) != 64:
        raise ValueError("native MI355X SDPA requires head_dim=64")
    if not (q.device == k.device == v.device):
        raise ValueError("q/k/v must be on one device")

    orig_dtype = q.dtype
    q_f, k_f, v_f = _as_f32_contig(q), _as_f32_contig(k), _as_f32_contig(v)
    bias_f = None
    if key_bias is not None:
        if int(key_bias.numel()) != int(k_f.shape[-2]):
            raise ValueError(f"key bias length mismatch: bias={key_bias.numel()} keys={k_f.shape[-2]}")
        bias_f = key_bias.to(device=q.device, dtype=torch.float32).reshape(-1).contiguous()

    out = torch.empty((int(q_f.shape[0]), int(q_f.shape[1]), int(q_f.shape[2]), 64),
                      dtype=torch.float32, device=q.device)
    _ = threads if threads is not None else os.environ.get("TRIPOSPLAT_NATIVE_SDPA_THREADS")
    lib = load_library(library or os.environ.get("TRIPOSPLAT_NATIVE_SDPA_LIBRARY"))
    name = symbol or os.environ.get("TRIPOSPLAT_NATIVE_SDPA_SYMBOL", DEFAULT_SYMBOL)
    with torch.cuda.device(q.device):
        if name == "tsplat_sdpa_async":
            status = lib.tsplat_sdpa_async(
                q_f.data_ptr(), k_f.data_ptr(), v_f.data_ptr(),
                0 if bias_f is None else bias_f.data_ptr(), out.data_ptr(),
                int(q_f.shape[0]), int(q_f.shape[1]), int(q_f.shape[2]), int(k_f.shape[2]), 64,
                int(bias_f is not None), 0 if bias_f is None else int(bias_f.numel()),
                0, 0, 0, 0, current_stream_handle(q.device),
            )
        else:  # a reference-named blocking symbol (runs on the null stream)
            torch.cuda.current_stream(q.device).synchronize()
            status = getattr(lib, name)(
                q_f.data_ptr(), k_f.data_ptr(), v_f.data_ptr(),
                0 if bias_f is None else bias_f.data_ptr(), out.data_ptr(),
                int(q_f.shape[0]), int(q_f.shape[1]), int(q_f.shape[2]), int(k_f.shape[2]), 64,
                int(bias_f is not None), 0 if bias_f is None else int(bias_f.numel()), 0,
            )
    if status != 0:
        raise RuntimeError(
            f"native MI355X SDPA returned status {status}; "
            f"q={tuple(q_f.shape)} k={tuple(k_f.shape)} bias={bias_f is not None}"
        )
    return out.to(dtype=orig_dtype)


def native_sdpa_f32_ex(q, k, v, *, key_bias=None, key_bias_per_head=None, kv_packed=False,
                       key_count=None, out=None, out_layout="bhld", precision="fp32", library=None):
    """Extended device SDPA.

    q [B,H,Lq,64] fp32.  k/v [B,H,Lk,64], or with kv_packed=True
    [B,H,64,Lkp] key-contiguous (Lkp % 16 == 0) with key_count = Lk valid keys.
    key_bias [Lk] (shared) or key_bias_per_head [H,Lk].  out_layout "bhld"
    -> [B,H,Lq,64], "blhd" -> [B,Lq,H,64].  precision: "fp32" (strict, the
    default), or the opt-in bf16-MFMA products "bf16" / "bf16x3" of
    tsplat_sdpa_precision_async.  Returns the output tensor.
    """
    import torch

    from .nf24 import precision_id

    prec = precision_id(precision)

    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.device.type != "cuda" or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 GPU tensor")
    if q.dim() != 4 or q.shape[-1] != 64:
        raise ValueError("q must be [B,H,Lq,64]")
    B, H, Lq, _ = (int(s) for s in q.shape)
    if kv_packed:
        if tuple(k.shape[:3]) != (B, H, 64) or k.shape != v.shape:
            raise ValueError("packed k/v must be [B,H,64,Lkp]")
        Lkp = int(k.shape[3])
        Lk = int(key_count if key_count is not None else Lkp)
    else:
        if tuple(k.shape[:2]) != (B, H) or k.shape[-1] != 64 or k.shape != v.shape:
            raise ValueError("k/v must be [B,H,Lk,64]")
        Lk, Lkp = int(k.shape[2]), 0
    if key_bias is not None and key_bias_per_head is not None:
        raise ValueError("pass key_bias or key_bias_per_head, not both")
    bias, stride = None, 0
    if key_bias is not None:
        bias = key_bias.to(device=q.device, dtype=torch.float32).reshape(-1).contiguous()
        if bias.numel() != Lk:
            raise ValueError(f"key bias length mismatch: bias={bias.numel()} keys={Lk}")
    elif key_bias_per_head is not None:
        bias = key_bias_per_head.to(device=q.device, dtype=torch.float32).contiguous()
        if tuple(bias.shape) != (H, Lk):
            raise ValueError(f"per-head key bias must be [H, Lk] = [{H}, {Lk}]")
        stride = Lk
    blhd = {"bhld": 0, "blhd": 1}[out_layout]
    shape = (B, Lq, H, 64) if blhd else (B, H, Lq, 64)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=q.device)
    elif tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 tensor of shape {shape}")
    lib = load_library(library)
    with torch.cuda.device(q.device):
        status = lib.tsplat_sdpa_precision_async(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), 0 if bias is None else bias.data_ptr(),
            out.data_ptr(), B, H, Lq, Lk, 64, int(bias is not None), Lk if bias is not None else 0,
            stride, int(bool(kv_packed)), Lkp, blhd, prec, current_stream_handle(q.device),
        )
    check_status(status, "tsplat_sdpa_precision_async")
    return out
