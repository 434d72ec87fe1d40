"""Strict NF24 Linear patch on the device: the counterpart of the reference's
scripts/native_linear_rnf8_avx512_patch.py:145-463
(``apply_triposplat_native_rnf8_avx512_patch``).

Same name, keyword arguments, buffer names (``_native_rnf8_*``), range hook
(``_native_avx512_forward_range``), metadata keys and error behaviour.  The
differences are those of the device:

* the library is libtsplat_hip.so (gfx950); it implements residual mode 4
  (``nf24_i16``, stages=3) only, so any other mode raises the reference's
  "residual quantizer/library mismatch" RuntimeError;
* weights are packed on the GPU by the tsplat_nf24_pack_async kernel and
  the packed buffers live on the module's GPU;
* the patched forward takes contiguous fp32 GPU activations (CPU or
  non-fp32 input is a strict violation and raises) and enqueues the GEMM on
  torch's current stream.  ``runtime["seconds"]`` is host time spent in the
  call (the kernel runs asynchronously).
"""
from __future__ import annotations

import math
import re
import time
import types
from pathlib import Path
from typing import Any

from ._lib import library_path as _default_library_path
from ._lib import load_library
from .nf24 import (RESIDUAL_MODE_ID, make_nf8_codebook, nf24_linear, precision_id,
                   quantize_nf24_i16_per_output_channel)
from .nf24 import bf16_planes as make_bf16_planes

_MODE_NAMES = {0: "nf8", 1: "symmetric_int8", 4: "nf24_i16"}


def apply_triposplat_native_rnf8_avx512_patch(
    flow_model,
    *,
    enabled: bool = False,
    include_regex: str | None = None,
    exclude_regex: str | None = None,
    library_path: str | None = None,
    optimized_library_path: str | None = None,
    optimized_shapes: tuple[tuple[int, int], ...] = (),
    threads: int = 2,
    strict: bool = True,
    stages: int = 2,
    residual_mode: str = "nf8",
    precision: str = "fp32",
    bf16_planes: bool = True,
) -> dict[str, Any]:
    """``precision`` (no counterpart in the reference): "fp32" (strict, the
    default) or the opt-in bf16-MFMA products "bf16" / "bf16x3" of
    tsplat.nf24.nf24_linear; it is recorded in the returned metadata.  With
    a bf16 mode and ``bf16_planes``, each Linear's weight planes
    (tsplat.nf24.bf16_planes) are built here and read by its calls instead of
    decoding the codes (same results; 2 or 4 more bytes per weight)."""
    if not enabled:
        return {"enabled": False}
    precision_id(precision)
    if not strict:
        raise ValueError("residual NF8 releases float32 weights and requires strict=True")
    if stages not in (2, 3):
        raise ValueError("residual NF8 stages must be 2 or 3")
    if residual_mode not in ("nf8", "symmetric_int8", "nf24_i16"):
        raise ValueError(f"unsupported residual quantizer: {residual_mode}")
    if residual_mode == "nf24_i16" and stages != 3:
        raise ValueError("NF24 int16 layout requires exactly 3 stages")

    import torch
    import torch.nn as nn

    include = re.compile(include_regex) if include_regex else None
    exclude = re.compile(exclude_regex) if exclude_regex else None
    lib_path = Path(library_path).resolve() if library_path else _default_library_path()
    if not lib_path.is_file():
        raise FileNotFoundError(lib_path)
    lib = load_library(lib_path)
    row_tile = int(lib.triposplat_gemm_rnf8_avx512_row_tile())
    mode_id = int(lib.triposplat_gemm_rnf8_avx512_residual_mode())
    library_residual_mode = _MODE_NAMES.get(mode_id)
    if library_residual_mode is None:
        raise RuntimeError(f"unsupported residual mode id from library: {mode_id}")
    if library_residual_mode != residual_mode:
        raise RuntimeError(
            f"residual quantizer/library mismatch: requested={residual_mode}, "
            f"library={library_residual_mode}"
        )
    if optimized_library_path is not None:
        # The reference can route chosen shapes to a second build; one gfx950
        # build serves every shape here, so the option is accepted only if it
        # names the same library.
        if Path(optimized_library_path).resolve() != lib_path:
            raise ValueError("optimized_library_path must be the same libtsplat_hip.so on the device")
    optimized_shapes_set = {tuple(int(v) for v in shape) for shape in optimized_shapes}

    runtime = {
        "calls": 0,
        "range_calls": 0,
        "optimized_calls": 0,
        "rows": 0,
        "seconds": 0.0,
        "contiguous_copies": 0,
        "fallbacks": 0,
        "per_module": {},
    }
    selected, skipped = [], []
    selected_dims, packing = {}, {}
    codebook = make_nf8_codebook(torch)
    prepacked_manifest = getattr(flow_model, "_native_rnf8_prepacked_manifest", None)
    if prepacked_manifest is not None and (stages != 3 or residual_mode != "nf24_i16"):
        raise ValueError("prepacked NF24 int16 requires stages=3 and residual_mode=nf24_i16")
    original_bytes = packed_bytes = weight_elements = plane_bytes = 0
    use_planes = bool(bf16_planes) and precision != "fp32"
    weighted_squared_error = 0.0
    max_abs_error = 0.0

    def matches(name: str) -> bool:
        return not (
            (include is not None and include.search(name) is None)
            or (exclude is not None and exclude.search(name) is not None)
        )

    def prepare_input(module, x, module_name: str):
        if torch.is_grad_enabled():
            raise RuntimeError(f"residual NF8 strict violation for {module_name}: grad_enabled")
        if x.device.type != "cuda" or x.dtype != torch.float32:
            raise RuntimeError(f"residual NF8 strict violation for {module_name}: input_{x.device.type}_{x.dtype}")
        if x.device != module._native_rnf8_codes0_t.device:
            raise RuntimeError(f"residual NF8 strict violation for {module_name}: input_device_mismatch")
        if int(x.shape[-1]) != int(module.in_features):
            raise RuntimeError(f"residual NF8 strict violation for {module_name}: input_feature_mismatch")
        x2 = x.reshape(-1, int(module.in_features))
        if not x2.is_contiguous():
            x2 = x2.contiguous()
            runtime["contiguous_copies"] += 1
        return x2

    def record(name: str, rows: int, elapsed: float, is_range: bool, optimized: bool = False):
        runtime["calls"] += 1
        runtime["range_calls"] += int(is_range)
        runtime["optimized_calls"] += int(optimized)
        runtime["rows"] += rows
        runtime["seconds"] += elapsed
        item = runtime["per_module"].setdefault(
            name, {"calls": 0, "range_calls": 0, "optimized_calls": 0, "rows": 0, "seconds": 0.0}
        )
        item["calls"] += 1
        item["range_calls"] += int(is_range)
        item["optimized_calls"] += int(optimized)
        item["rows"] += rows
        item["seconds"] += elapsed

    def call(module, module_name, x2, start, count, is_range):
        started = time.perf_counter()
        try:
            planes = None
            if use_planes:
                planes = (module._native_rnf8_bf16_hi, getattr(module, "_native_rnf8_bf16_lo", None))
            out = nf24_linear(x2, module._native_rnf8_codes0_t, module._native_rnf8_codes1_t,
                              module._native_rnf8_scales0, module._native_rnf8_bias,
                              output_start=start, output_count=count, precision=precision,
                              planes=planes, library=lib_path)
        except RuntimeError as exc:
            runtime["fallbacks"] += 1
            kind = "range kernel" if is_range else "kernel"
            raise RuntimeError(f"residual NF8 {kind} failed for {module_name}: {exc}") from exc
        shape = (int(module.in_features), int(module.out_features))
        record(module_name, int(x2.shape[0]), time.perf_counter() - started, is_range,
               (not is_range) and shape in optimized_shapes_set)
        return out

    def make_forward(module_name: str):
        def forward(self, x):
            x2 = prepare_input(self, x, module_name)
            out = call(self, module_name, x2, 0, int(self.out_features), False)
            return out.view(*x.shape[:-1], int(self.out_features))

        return forward

    def make_range_forward(module_name: str):
        def range_forward(self, x, output_start: int, output_count: int):
            start, count = int(output_start), int(output_count)
            if start < 0 or count <= 0 or start + count > int(self.out_features):
                raise ValueError(f"invalid residual NF8 output range for {module_name}")
            x2 = prepare_input(self, x, module_name)
            out = call(self, module_name, x2, start, count, True)
            return out.view(*x.shape[:-1], count)

        return range_forward

    for name, module in flow_model.named_modules():
        if not isinstance(module, nn.Linear):
            continue
        if not matches(name):
            skipped.append(name)
            continue
        if prepacked_manifest is None:
            if module.weight.dtype != torch.float32:
                raise ValueError(f"residual NF8 requires float32 weight: {name}")
            codes, scales, error = quantize_nf24_i16_per_output_channel(module.weight.detach(), codebook)
            device = codes[0].device
            bias = (
                torch.zeros(int(module.out_features), dtype=torch.float32, device=device)
                if module.bias is None
                else module.bias.detach().to(device=device, dtype=torch.float32).contiguous()
            )
            module.register_buffer("_native_rnf8_codes0_t", codes[0], persistent=False)
            module.register_buffer("_native_rnf8_codes1_t", codes[1], persistent=False)
            module.register_buffer("_native_rnf8_codes2_t", codes[2], persistent=False)
            module.register_buffer("_native_rnf8_scales0", scales[0], persistent=False)
            module.register_buffer("_native_rnf8_scales1", scales[1], persistent=False)
            module.register_buffer("_native_rnf8_scales2", scales[2], persistent=False)
            module.register_buffer("_native_rnf8_bias", bias, persistent=False)
        else:
            item = prepacked_manifest["linears"].get(name)
            if item is None:
                raise ValueError(f"prepacked checkpoint has no Linear entry: {name}")
            codes = [module._native_rnf8_codes0_t, module._native_rnf8_codes1_t, module._native_rnf8_codes2_t]
            scales = [module._native_rnf8_scales0, module._native_rnf8_scales1, module._native_rnf8_scales2]
            bias = module._native_rnf8_bias
            if codes[0].device.type != "cuda":
                raise RuntimeError(f"prepacked NF24 buffers for {name} must be on the GPU")
            error = item["quantization"]
        module.register_buffer("_native_rnf8_codebook", codebook.to(codes[0].device), persistent=False)
        if use_planes:
            w_hi, w_lo = make_bf16_planes(codes[0], codes[1], scales[0], precision, library=lib_path)
            module.register_buffer("_native_rnf8_bf16_hi", w_hi, persistent=False)
            plane_bytes += w_hi.numel() * 2
            if w_lo is not None:
                module.register_buffer("_native_rnf8_bf16_lo", w_lo, persistent=False)
                plane_bytes += w_lo.numel() * 2
        module.weight = nn.Parameter(torch.empty(0, dtype=torch.float32, device=codes[0].device), requires_grad=False)
        if module.bias is not None:
            module.bias = nn.Parameter(torch.empty(0, dtype=torch.float32, device=codes[0].device), requires_grad=False)
        module.forward = types.MethodType(make_forward(name), module)
        module._native_avx512_forward_range = types.MethodType(make_range_forward(name), module)

        count = int(codes[0].numel())
        original = count * 4 + int(bias.numel()) * 4
        packed = count * 3 + int(scales[0].numel()) * 4 + int(bias.numel()) * 4 + 1024
        original_bytes += original
        packed_bytes += packed
        weight_elements += count
        weighted_squared_error += error["weight_rmse"] ** 2 * count
        max_abs_error = max(max_abs_error, error["weight_max_abs"])
        packing[name] = {**error, "weight_elements": count, "original_bytes": original, "packed_bytes": packed}
        selected.append(name)
        selected_dims[name] = f"{int(module.in_features)}x{int(module.out_features)}"

    if skipped:
        raise ValueError(f"residual NF8 strict mode left {len(skipped)} Linear modules unquantized")
    return {
        "enabled": bool(selected),
        "kind": "native_residual_nonlinear_nf8_weight_only_mi355x_linear_patch",
        "residual_stages": int(stages),
        "first_stage_quantizer": "nf8_derived_int8_alphabet",
        "residual_quantizer": residual_mode,
        "bits_per_weight": 24,
        "activation_dtype": "float32",
        "gemm_precision": precision,
        "gemm_bf16_planes": use_planes,
        "bf16_plane_bytes": plane_bytes,
        "float32_weight_retained": False,
        "library_path": lib_path.as_posix(),
        "optimized_library_path": None if optimized_library_path is None else lib_path.as_posix(),
        "optimized_shapes": [list(shape) for shape in sorted(optimized_shapes_set)],
        "row_tile": row_tile,
        "residual_mode_id": RESIDUAL_MODE_ID,
        "symbols": ["tsplat_nf24_gemm_async", "triposplat_gemm_rnf8_avx512",
                    "triposplat_gemm_rnf8_avx512_range", "triposplat_gemm_rnf8_avx512_tail",
                    "triposplat_gemm_rnf8_avx512_row_tile", "triposplat_gemm_rnf8_avx512_residual_mode"],
        "threads": int(threads),
        "strict": True,
        "prepacked_load": getattr(flow_model, "_native_rnf8_prepacked_load", {"enabled": False}),
        "selected_count": len(selected),
        "selected": selected,
        "selected_dims": selected_dims,
        "skipped_count": 0,
        "original_bytes": original_bytes,
        "packed_bytes": packed_bytes,
        "storage_ratio": packed_bytes / max(original_bytes, 1),
        "aggregate_weight_rmse": math.sqrt(weighted_squared_error / max(weight_elements, 1)),
        "aggregate_weight_max_abs": max_abs_error,
        "packing": packing,
        "runtime": runtime,
        "semantics": "All selected Linear weights are decoded in registers inside the gfx950 NF24 GEMM "
                     + ("(fp32 MFMA accumulate)" if precision == "fp32" else
                        f"({precision} products on bf16 MFMA, fp32 accumulate; opt-in)")
                     + "; no fp32 weight copy is kept.",
    }


def redirect_native_linear(flow_model, **kwargs):
    """The hook the reference's NF24 runners install in place of
    ``apply_triposplat_native_linear_avx512_patch``
    (scripts/run_triposplat_rnf8_param_batch.py:40-50): the Linear patch with
    the stage count / residual mode from TRIPOSPLAT_RNF8_STAGES and
    TRIPOSPLAT_RNF8_RESIDUAL_MODE (defaults 3 / nf24_i16, the only form this
    library implements)."""
    import os

    return apply_triposplat_native_rnf8_avx512_patch(
        flow_model,
        stages=int(os.environ.get("TRIPOSPLAT_RNF8_STAGES", "3")),
        residual_mode=os.environ.get("TRIPOSPLAT_RNF8_RESIDUAL_MODE", "nf24_i16"),
        **kwargs,
    )
