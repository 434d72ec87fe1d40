"""QKV postprocess and the fused NF24 QKV projection on the device.

Counterparts of scripts/native_qkv_postprocess_v2_avx512.c:45-105
(``triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2``) and
scripts/gemm_nf24_qkv_direct_avx512.c:87-199
(``triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512``), as called by
scripts/native_qkv_packed_attention_patch_v3.py:93-158: RoPE first, then
RMSNorm (``y * 8 / max(||y||, 1e-12) * gamma``) on q and k; q comes back as
[B, H, L, 64], k and v packed key-contiguous [B, H, 64, L_padded] with the
tail tokens zero -- the layout the packed SDPA consumes.
"""
from __future__ import annotations

from ._lib import check_status, current_stream_handle, load_library


# bf16 rounding of the stored k and/or v (the K/V sensitivity probe,
# scripts/native_qkv_postprocess_bf16_probe_avx512.c:34-94, whose three builds
# scripts/build_native_qkv_postprocess_bf16_probe_avx512.sh selects with
# BF16_TARGET): None stores them exact (the default), "k", "v" or "kv" round
# them to the nearest bf16 after the exact computation.  Per call: no other
# call's numerics change.
KV_BF16_ROUND_MODES = {None: 0, "k": 1, "v": 2, "kv": 3}


def kv_round_id(mode) -> int:
    if mode not in KV_BF16_ROUND_MODES:
        raise ValueError(f"kv_round must be one of {sorted(KV_BF16_ROUND_MODES, key=str)}")
    return KV_BF16_ROUND_MODES[mode]


def padded_length(L: int) -> int:
    return (int(L) + 15) & ~15


def _outputs(torch, B, L, H, Lp, device):
    q = torch.empty((B, H, L, 64), dtype=torch.float32, device=device)
    pk = torch.empty((B, H, 64, Lp), dtype=torch.float32, device=device)
    pv = torch.empty((B, H, 64, Lp), dtype=torch.float32, device=device)
    return q, pk, pv


def _check(torch, name, t):
    if t.device.type != "cuda" or t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous fp32 GPU tensor")


def qkv_rope_rmsnorm_pack(qkv, frequencies, q_gamma, k_gamma, B, L, H, *, L_padded=None, kv_round=None,
                          library=None):
    """qkv [B*L, 3*H*64]; frequencies [fb, L, H, 64] (cos, sin pairs), fb in {1, B};
    kv_round: the bf16 probe mode of the stored k/v (None = exact)."""
    import torch

    rnd = kv_round_id(kv_round)
    for name, t in (("qkv", qkv), ("frequencies", frequencies), ("q_gamma", q_gamma), ("k_gamma", k_gamma)):
        _check(torch, name, t)
    Lp = padded_length(L) if L_padded is None else int(L_padded)
    q, pk, pv = _outputs(torch, B, L, H, Lp, qkv.device)
    lib = load_library(library)
    with torch.cuda.device(qkv.device):
        status = lib.tsplat_qkv_postprocess_async(
            qkv.data_ptr(), frequencies.data_ptr(), q_gamma.data_ptr(), k_gamma.data_ptr(),
            q.data_ptr(), pk.data_ptr(), pv.data_ptr(), int(B), int(L), int(H), 64, Lp,
            int(frequencies.shape[0]), rnd, current_stream_handle(qkv.device),
        )
    check_status(status, "tsplat_qkv_postprocess_async")
    return q, pk, pv


def gemm_nf24_qkv_direct(x2, code01_t, q2_t, scale, bias, frequencies, q_gamma, k_gamma, B, L, H, *,
                         L_padded=None, precision="fp32", kv_layout="packed", kv_round=None, planes=None,
                         library=None):
    """NF24 QKV projection of x2 [B*L, K] (N = 3*H*64) then the postprocess;
    precision (and planes) of the projection as tsplat.nf24.nf24_linear.
    kv_layout "packed" returns k/v [B, H, 64, L_padded] (the reference's
    layout), "bhld" returns k/v [B, H, L, 64] like q (what the unpacked SDPA
    reads).  kv_round: the bf16 probe mode of the stored k/v (None = exact)."""
    import torch

    from .nf24 import planes_pointers, precision_id

    mode = precision_id(precision)
    rnd = kv_round_id(kv_round)
    if kv_layout not in ("packed", "bhld"):
        raise ValueError(f"kv_layout must be 'packed' or 'bhld', not {kv_layout!r}")
    for name, t in (("x", x2), ("frequencies", frequencies), ("q_gamma", q_gamma), ("k_gamma", k_gamma)):
        _check(torch, name, t)
    Lp = padded_length(L) if L_padded is None else int(L_padded)
    if kv_layout == "packed":
        q, pk, pv = _outputs(torch, B, L, H, Lp, x2.device)
    else:
        q, pk, pv = (torch.empty((B, H, L, 64), dtype=torch.float32, device=x2.device) for _ in range(3))
    lib = load_library(library)
    with torch.cuda.device(x2.device):
        args = (x2.data_ptr(), code01_t.data_ptr(), q2_t.data_ptr(), scale.data_ptr(), bias.data_ptr(),
                frequencies.data_ptr(), q_gamma.data_ptr(), k_gamma.data_ptr(), q.data_ptr(), pk.data_ptr(),
                pv.data_ptr(), int(B), int(L), int(x2.shape[1]), int(code01_t.shape[1]), int(H), 64, Lp,
                int(frequencies.shape[0]))
        stream = current_stream_handle(x2.device)
        if mode == 0 and kv_layout == "packed" and rnd == 0:
            name, status = "tsplat_gemm_nf24_qkv_direct_async", lib.tsplat_gemm_nf24_qkv_direct_async(*args, stream)
        elif mode != 0 and planes is not None:
            name = "tsplat_gemm_nf24_qkv_direct_planes_async"
            ptrs = planes_pointers(planes, int(x2.shape[1]), int(code01_t.shape[1]), mode)
            status = lib.tsplat_gemm_nf24_qkv_direct_planes_async(*args, int(kv_layout == "bhld"), mode, rnd,
                                                                    *ptrs, stream)
        else:
            name = "tsplat_gemm_nf24_qkv_direct_ex_async"
            status = lib.tsplat_gemm_nf24_qkv_direct_ex_async(*args, int(kv_layout == "bhld"), mode, rnd,
                                                                stream)
    check_status(status, name)
    return q, pk, pv


def q_kv_selected_rope_rmsnorm_pack(q, kv, frequencies, selected_indices, q_gamma, k_gamma, B, Lq, Lk, H,
                                    *, L_padded=None, kv_round=None, library=None):
    """Selected query rows (scripts/native_qkv_postprocess_v2_avx512.c:107-191):
    q [B, Lq, H*64] from a Q-only projection, kv [B, Lk, 2*H*64] = [k | v];
    query t is rotated with frequency row selected_indices[t] (int64 GPU
    tensor).  Returns q [B, H, Lq, 64] and packed k/v [B, H, 64, L_padded].
    kv_round: the bf16 probe mode of the stored k/v (None = exact)."""
    import torch

    rnd = kv_round_id(kv_round)
    for name, t in (("q", q), ("kv", kv), ("frequencies", frequencies), ("q_gamma", q_gamma),
                    ("k_gamma", k_gamma)):
        _check(torch, name, t)
    if (selected_indices.device.type != "cuda" or selected_indices.dtype != torch.int64
            or not selected_indices.is_contiguous() or selected_indices.numel() != int(Lq)):
        raise ValueError("selected_indices must be a contiguous int64 GPU tensor of length Lq")
    Lp = padded_length(Lk) if L_padded is None else int(L_padded)
    qo = torch.empty((B, H, Lq, 64), dtype=torch.float32, device=q.device)
    pk = torch.empty((B, H, 64, Lp), dtype=torch.float32, device=q.device)
    pv = torch.empty((B, H, 64, Lp), dtype=torch.float32, device=q.device)
    lib = load_library(library)
    with torch.cuda.device(q.device):
        status = lib.tsplat_q_kv_selected_postprocess_async(
            q.data_ptr(), kv.data_ptr(), frequencies.data_ptr(), selected_indices.data_ptr(),
            q_gamma.data_ptr(), k_gamma.data_ptr(), qo.data_ptr(), pk.data_ptr(), pv.data_ptr(),
            int(B), int(Lq), int(Lk), int(H), 64, Lp, int(frequencies.shape[0]), rnd,
            current_stream_handle(q.device),
        )
    check_status(status, "tsplat_q_kv_selected_postprocess_async")
    return qo, pk, pv
