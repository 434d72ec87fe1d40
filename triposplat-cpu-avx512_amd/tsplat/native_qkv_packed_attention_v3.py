"""Packed exact attention helpers on the device.

Mirror of scripts/native_qkv_packed_attention_patch_v3.py:9-346
(``apply_triposplat_native_qkv_packed_attention_helpers_patch``): the same
module selection (self-attention ``RopeMultiHeadAttention`` with RoPE, q/k
RMSNorm and head dim 64), the same three replaced helpers of the model's
attention module (``_rope_self_attention_standard``,
``_rope_self_attention_with_key_bias``, ``_rope_self_attention_selected_rows``),
the same runtime counters and metadata keys, and strict mode raising instead
of falling back.  Each helper runs the QKV projection (the patched NF24
Linear), RoPE -> RMSNorm -> pack (tsplat.qkv), the packed exact SDPA with
BLHD output (tsplat.native_sdpa_ctypes) and the out projection, all on the
GPU; the selected-rows helper projects Q only for the selected rows (the
Linear's range forward) and K/V for all rows.

The attention module is ``triposplat_attention_patch`` when importable (it
belongs to the upstream model integration); callers may pass it explicitly.
"""
from __future__ import annotations

import re
import time

from ._lib import library_path
from .native_sdpa_ctypes import native_sdpa_f32_ex
from .qkv import q_kv_selected_rope_rmsnorm_pack, qkv_rope_rmsnorm_pack

BACKEND = "native_avx512_exact"  # the backend name the model's callers pass


def apply_triposplat_native_qkv_packed_attention_helpers_patch(
    flow_model,
    *,
    postprocess_library: str | None = None,
    sdpa_library: str | None = None,
    threads: int = 0,
    include_regex: str = r"^blocks[.][0-9]+[.]attn$",
    strict: bool = True,
    attention_module=None,
):
    import torch

    if attention_module is None:
        import triposplat_attention_patch as attention_module  # noqa: N813 (upstream integration)

    include = re.compile(include_regex)
    selected_names, selected_ids = [], set()
    for name, module in flow_model.named_modules():
        if module.__class__.__name__ != "RopeMultiHeadAttention" or include.search(name) is None:
            continue
        if module._type == "self" and module.use_rope and module.qk_rms_norm and module.head_dim == 64:
            selected_names.append(name)
            selected_ids.add(id(module))
    if strict and not selected_names:
        raise RuntimeError(f"packed Attention helper patch selected no modules with {include_regex!r}")

    runtime = {
        "calls": 0, "selected_row_calls": 0, "key_bias_calls": 0, "postprocess_seconds": 0.0,
        "sdpa_seconds": 0.0, "workspace_allocations": 0, "workspace_capacity_bytes": 0,
        "qkv_input_copies": 0, "frequency_copies": 0, "selected_index_copies": 0, "fallbacks": 0,
    }

    def stage(timing_callback, name, function, shape):
        if timing_callback is None:
            return function()
        started = time.perf_counter()
        try:
            return function()
        finally:
            timing_callback(name, time.perf_counter() - started, shape=shape)

    def frequency_view(rope_emb, b, length, heads, dim):
        """complex (cos, sin) [fb, L, H, 32] -> interleaved fp32 [fb, L, H, 64]."""
        frequency = torch.view_as_real(rope_emb).reshape(*rope_emb.shape[:-1], dim)
        if not frequency.is_contiguous():
            frequency = frequency.contiguous()
            runtime["frequency_copies"] += 1
        fb = int(frequency.shape[0])
        if fb not in (1, b) or frequency.numel() != fb * length * heads * dim:
            raise RuntimeError(f"packed Attention frequency mismatch: {tuple(rope_emb.shape)}")
        return frequency

    def usable(attn, x, rope_emb):
        return (id(attn) in selected_ids and x.device.type == "cuda" and x.dtype == torch.float32
                and rope_emb is not None and rope_emb.device == x.device
                and rope_emb.dtype == torch.complex64)

    def timed(key, callback, label, shape, function):
        started = time.perf_counter()
        result = function()
        elapsed = time.perf_counter() - started
        runtime[key] += elapsed
        if callback is not None:
            callback(label, elapsed, shape=shape)
        return result

    def run(attn, x, rope_emb, key_bias, timing_callback):
        b, length, channels = (int(v) for v in x.shape)
        heads, dim = int(attn.num_heads), int(attn.head_dim)
        if not usable(attn, x, rope_emb):
            return None
        qkv = stage(timing_callback, "attention.qkv_projection", lambda: attn.qkv(x), [b, length, 3 * channels])
        if not qkv.is_contiguous():
            qkv = qkv.contiguous()
            runtime["qkv_input_copies"] += 1
        frequency = frequency_view(rope_emb, b, length, heads, dim)
        q, pk, pv = timed("postprocess_seconds", timing_callback, "attention.rope_qknorm_layout_pack",
                          [b, heads, length, dim],
                          lambda: qkv_rope_rmsnorm_pack(qkv.view(b * length, 3 * channels), frequency,
                                                        attn.q_norm.gamma, attn.k_norm.gamma, b, length,
                                                        heads, library=postprocess_library))
        bias = None
        if key_bias is not None:
            bias = key_bias.to(device=x.device, dtype=torch.float32).reshape(-1).contiguous()
            if bias.numel() != length:
                raise RuntimeError(f"packed Attention key bias mismatch: {bias.numel()} != {length}")
            runtime["key_bias_calls"] += 1
        out = timed("sdpa_seconds", timing_callback, "attention.sdpa", [b, heads, length, dim],
                    lambda: native_sdpa_f32_ex(q, pk, pv, key_bias=bias, kv_packed=True, key_count=length,
                                               out_layout="blhd", library=sdpa_library))
        runtime["calls"] += 1
        return stage(timing_callback, "attention.out_projection",
                     lambda: attn.out(out.view(b, length, channels)), [b, length, channels])

    def run_selected(attn, x, selected_idx, rope_emb, timing_callback):
        b, length, channels = (int(v) for v in x.shape)
        heads, dim = int(attn.num_heads), int(attn.head_dim)
        native_range = getattr(attn.qkv, "_native_avx512_forward_range", None)
        if (not usable(attn, x, rope_emb) or native_range is None or selected_idx.device != x.device
                or selected_idx.dtype != torch.int64):
            return None
        if not selected_idx.is_contiguous():
            selected_idx = selected_idx.contiguous()
            runtime["selected_index_copies"] += 1
        lq = int(selected_idx.numel())
        x_sel = stage(timing_callback, "attention.selected_index", lambda: x.index_select(1, selected_idx),
                      [b, lq, channels])
        q = stage(timing_callback, "attention.q_projection", lambda: native_range(x_sel, 0, channels),
                  [b, lq, channels])
        kv = stage(timing_callback, "attention.kv_projection", lambda: native_range(x, channels, 2 * channels),
                   [b, length, 2 * channels])
        if not q.is_contiguous():
            q = q.contiguous()
            runtime["qkv_input_copies"] += 1
        if not kv.is_contiguous():
            kv = kv.contiguous()
            runtime["qkv_input_copies"] += 1
        frequency = frequency_view(rope_emb, b, length, heads, dim)
        qp, pk, pv = timed("postprocess_seconds", timing_callback, "attention.rope_qknorm_layout_pack",
                           {"q": [b, heads, lq, dim], "k": [b, heads, length, dim]},
                           lambda: q_kv_selected_rope_rmsnorm_pack(q, kv, frequency, selected_idx,
                                                                   attn.q_norm.gamma, attn.k_norm.gamma,
                                                                   b, lq, length, heads,
                                                                   library=postprocess_library))
        out = timed("sdpa_seconds", timing_callback, "attention.sdpa",
                    {"q": [b, heads, lq, dim], "k": [b, heads, length, dim]},
                    lambda: native_sdpa_f32_ex(qp, pk, pv, kv_packed=True, key_count=length,
                                               out_layout="blhd", library=sdpa_library))
        runtime["calls"] += 1
        runtime["selected_row_calls"] += 1
        return stage(timing_callback, "attention.out_projection", lambda: attn.out(out.view(b, lq, channels)),
                     [b, lq, channels])

    original_standard = attention_module._rope_self_attention_standard
    original_key_bias = attention_module._rope_self_attention_with_key_bias
    original_selected = attention_module._rope_self_attention_selected_rows

    def fell_back(attn, what):
        runtime["fallbacks"] += 1
        if strict and id(attn) in selected_ids:
            raise RuntimeError(f"selected {what} Attention fell back from packed path")

    def packed_standard(attn, x, rope_emb, *, backend="default", compute_dtype="model", query_chunk_size=128,
                        contiguous_qkv=True, timing_callback=None):
        if backend == BACKEND and compute_dtype == "model":
            result = run(attn, x, rope_emb, None, timing_callback)
            if result is not None:
                return result
        fell_back(attn, "standard")
        return original_standard(attn, x, rope_emb, backend=backend, compute_dtype=compute_dtype,
                                 query_chunk_size=query_chunk_size, contiguous_qkv=contiguous_qkv,
                                 timing_callback=timing_callback)

    def packed_key_bias(attn, x, rope_emb, key_bias, *, backend="default", timing_callback=None):
        if backend == BACKEND:
            result = run(attn, x, rope_emb, key_bias, timing_callback)
            if result is not None:
                return result
        fell_back(attn, "key-bias")
        return original_key_bias(attn, x, rope_emb, key_bias, backend=backend, timing_callback=timing_callback)

    def packed_selected(attn, x, selected_idx, rope_emb, *, backend, compute_dtype, query_chunk_size,
                        round_qkv_to_fp16=False, round_v_to_fp16=False, round_attn_core_to_fp16=False,
                        half_sequence=False, key_bias=None, timing_callback=None):
        exact = (backend == BACKEND and compute_dtype == "model" and not round_qkv_to_fp16
                 and not round_v_to_fp16 and not round_attn_core_to_fp16 and not half_sequence
                 and key_bias is None)
        if exact:
            result = run_selected(attn, x, selected_idx, rope_emb, timing_callback)
            if result is not None:
                return result
            fell_back(attn, "selected-row")
        return original_selected(attn, x, selected_idx, rope_emb, backend=backend, compute_dtype=compute_dtype,
                                 query_chunk_size=query_chunk_size, round_qkv_to_fp16=round_qkv_to_fp16,
                                 round_v_to_fp16=round_v_to_fp16, round_attn_core_to_fp16=round_attn_core_to_fp16,
                                 half_sequence=half_sequence, key_bias=key_bias, timing_callback=timing_callback)

    attention_module._rope_self_attention_standard = packed_standard
    attention_module._rope_self_attention_with_key_bias = packed_key_bias
    attention_module._rope_self_attention_selected_rows = packed_selected
    lib = library_path(postprocess_library).as_posix()
    return {
        "enabled": bool(selected_names),
        "kind": "native_attention_helpers_qkv_packed_exact_v3_mi355x",
        "postprocess_library": lib,
        "sdpa_library": library_path(sdpa_library).as_posix(),
        "threads": int(threads),
        "include_regex": include_regex,
        "selected_count": len(selected_names),
        "selected": selected_names,
        "runtime": runtime,
        "coverage": "positive standard, negative key-bias, and final positive selected-query helpers",
        "semantics": "Exact RoPE/RMSNorm (bit-identical to the reference) and online-softmax SDPA on the "
                     "GPU; Q is computed only for consumed rows in the final selected-query helper.",
    }
