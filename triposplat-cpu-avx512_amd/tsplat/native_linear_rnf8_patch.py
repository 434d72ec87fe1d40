"""Strict NF24 Linear patch on the device: the counterpart of the reference's
scripts/native_linear_rnf8_avx512_patch.py:145-463
(``apply_triposplat_native_rnf8_avx512_patch``).

Same name, keyword arguments, buffer names (``_native_rnf8_*``), range hook
(``_native_avx512_forward_range``), metadata keys, runtime counters and error
messages.  The differences are those of the device:

* the library is libtsplat_hip.so (gfx950); it implements residual mode 4
  (``nf24_i16``, stages=3) only, so any other mode raises the reference's
  "residual quantizer/library mismatch" RuntimeError;
* weights are packed on the GPU by the tsplat_nf24_pack_async kernel and
  the packed buffers live on the module's GPU;
* the patched forward takes contiguous fp32 GPU activations (CPU or
  non-fp32 input is a strict violation and raises) and enqueues the GEMM on
  torch's current stream.  ``runtime["seconds"]`` is host time spent in the
  call (the kernel runs asynchronously).

Structure: the option and library checks run first; each selected Linear
then gets its packed buffers and a ``_DeviceLinear`` bound as its forward
and range hook, which checks the input, runs the GEMM and counts the call
in the shared ``_Runtime``.
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
_COUNTERS = ("calls", "range_calls", "optimized_calls", "rows", "seconds")
_SYMBOLS = ["tsplat_nf24_gemm_async", "triposplat_gemm_rnf8_avx512", "triposplat_gemm_rnf8_avx512_range",
            "triposplat_gemm_rnf8_avx512_tail", "triposplat_gemm_rnf8_avx512_row_tile",
            "triposplat_gemm_rnf8_avx512_residual_mode"]


def _check_options(strict: bool, stages: int, residual_mode: str) -> None:
    """The reference's argument checks, in its order and with its messages
    (native_linear_rnf8_avx512_patch.py:161-168)."""
    problems = (
        (not strict, "residual NF8 releases float32 weights and requires strict=True"),
        (stages not in (2, 3), "residual NF8 stages must be 2 or 3"),
        (residual_mode not in _MODE_NAMES.values(), f"unsupported residual quantizer: {residual_mode}"),
        (residual_mode == "nf24_i16" and stages != 3, "NF24 int16 layout requires exactly 3 stages"),
    )
    for failed, message in problems:
        if failed:
            raise ValueError(message)


def _check_library_mode(lib, residual_mode: str) -> None:
    """The library's residual quantizer must be the requested one."""
    mode_id = int(lib.triposplat_gemm_rnf8_avx512_residual_mode())
    library_mode = _MODE_NAMES.get(mode_id)
    if library_mode is None:
        raise RuntimeError(f"unsupported residual mode id from library: {mode_id}")
    if library_mode != residual_mode:
        raise RuntimeError(
            f"residual quantizer/library mismatch: requested={residual_mode}, library={library_mode}")


def _name_filter(include_regex: str | None, exclude_regex: str | None):
    """Module-name predicate: matched by the include pattern (if any) and
    not by the exclude pattern (if any)."""
    include = re.compile(include_regex) if include_regex else None
    exclude = re.compile(exclude_regex) if exclude_regex else None
    return lambda name: ((include is None or include.search(name) is not None)
                         and (exclude is None or exclude.search(name) is None))


def _storage_bytes(weights: int, scales: int, biases: int) -> tuple[int, int]:
    """(fp32 bytes, packed bytes) of one Linear: 4-byte weights and bias
    against 3-byte codes, the stage-0 scales, the bias and the 256-entry
    fp32 codebook."""
    return 4 * (weights + biases), 3 * weights + 4 * (scales + biases) + 1024


class _Runtime:
    """Call statistics, as the metadata's live ``runtime`` dict: totals and
    per-module counters, plus input copies and failed calls."""

    def __init__(self):
        self.data: dict[str, Any] = {key: 0 for key in _COUNTERS}
        self.data.update(seconds=0.0, contiguous_copies=0, fallbacks=0, per_module={})

    def count(self, name: str, rows: int, seconds: float, is_range: bool, optimized: bool) -> None:
        values = (1, int(is_range), int(optimized), rows, seconds)
        module = self.data["per_module"].setdefault(
            name, {key: 0.0 if key == "seconds" else 0 for key in _COUNTERS})
        for target in (self.data, module):
            for key, value in zip(_COUNTERS, values):
                target[key] += value


class _DeviceLinear:
    """The patched forward and range hook of one nn.Linear."""

    def __init__(self, name: str, runtime: _Runtime, lib_path: Path, precision: str, use_planes: bool,
                 optimized: bool):
        self.name, self.runtime, self.lib_path = name, runtime, lib_path
        self.precision, self.use_planes, self.optimized = precision, use_planes, optimized

    def _rows(self, module, x):
        """x as contiguous [rows, in_features] after the strict checks."""
        import torch

        checks = (
            ("grad_enabled", lambda: torch.is_grad_enabled()),
            (f"input_{x.device.type}_{x.dtype}", lambda: x.device.type != "cuda" or x.dtype != torch.float32),
            ("input_device_mismatch", lambda: x.device != module._native_rnf8_codes0_t.device),
            ("input_feature_mismatch", lambda: int(x.shape[-1]) != int(module.in_features)),
        )
        for reason, failed in checks:
            if failed():
                raise RuntimeError(f"residual NF8 strict violation for {self.name}: {reason}")
        rows = x.reshape(-1, int(module.in_features))
        if rows.is_contiguous():
            return rows
        self.runtime.data["contiguous_copies"] += 1
        return rows.contiguous()

    def _run(self, module, x, start: int, count: int, is_range: bool):
        rows = self._rows(module, x)
        planes = None
        if self.use_planes:
            planes = (module._native_rnf8_bf16_hi, getattr(module, "_native_rnf8_bf16_lo", None))
        t0 = time.perf_counter()
        try:
            out = nf24_linear(rows, module._native_rnf8_codes0_t, module._native_rnf8_codes1_t,
                              module._native_rnf8_scales0, module._native_rnf8_bias, output_start=start,
                              output_count=count, precision=self.precision, planes=planes,
                              library=self.lib_path)
        except RuntimeError as exc:
            self.runtime.data["fallbacks"] += 1
            kind = "range kernel" if is_range else "kernel"
            raise RuntimeError(f"residual NF8 {kind} failed for {self.name}: {exc}") from exc
        self.runtime.count(self.name, int(rows.shape[0]), time.perf_counter() - t0, is_range,
                           self.optimized and not is_range)
        return out.view(*x.shape[:-1], count)

    def forward(self, module, x):
        return self._run(module, x, 0, int(module.out_features), False)

    def forward_range(self, module, x, output_start: int, output_count: int):
        start, count = int(output_start), int(output_count)
        if start < 0 or count <= 0 or start + count > int(module.out_features):
            raise ValueError(f"invalid residual NF8 output range for {self.name}")
        return self._run(module, x, start, count, True)


def _packed_linear(torch, module, name: str, manifest, codebook):
    """(codes, scales, bias, quantization statistics) of one Linear: packed
    here from its fp32 weight (and attached as buffers), or the buffers a
    prepacked load attached, with the statistics from its manifest."""
    if manifest is not None:
        item = manifest["linears"].get(name)
        if item is None:
            raise ValueError(f"prepacked checkpoint has no Linear entry: {name}")
        codes = [getattr(module, f"_native_rnf8_codes{i}_t") for i in range(3)]
        if codes[0].device.type != "cuda":
            raise RuntimeError(f"prepacked NF24 buffers for {name} must be on the GPU")
        scales = [getattr(module, f"_native_rnf8_scales{i}") for i in range(3)]
        return codes, scales, module._native_rnf8_bias, item["quantization"]
    if module.weight.dtype != torch.float32:
        raise ValueError(f"residual NF8 requires float32 weight: {name}")
    codes, scales, stats = quantize_nf24_i16_per_output_channel(module.weight.detach(), codebook)
    device = codes[0].device
    if module.bias is None:
        bias = torch.zeros(int(module.out_features), dtype=torch.float32, device=device)
    else:
        bias = module.bias.detach().to(device=device, dtype=torch.float32).contiguous()
    buffers = {f"codes{i}_t": c for i, c in enumerate(codes)}
    buffers.update({f"scales{i}": s for i, s in enumerate(scales)}, bias=bias)
    for suffix, tensor in buffers.items():
        module.register_buffer(f"_native_rnf8_{suffix}", tensor, persistent=False)
    return codes, scales, bias, stats


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
    _check_options(strict, stages, residual_mode)

    import torch
    import torch.nn as nn

    selected_by_name = _name_filter(include_regex, exclude_regex)
    lib_path = Path(library_path).resolve() if library_path else _default_library_path()
    if not lib_path.is_file():
        raise FileNotFoundError(lib_path)
    lib = load_library(lib_path)
    row_tile = int(lib.triposplat_gemm_rnf8_avx512_row_tile())
    _check_library_mode(lib, residual_mode)
    if optimized_library_path is not None and Path(optimized_library_path).resolve() != lib_path:
        # The reference can route chosen shapes to a second build; one gfx950
        # build serves every shape here, so the option is accepted only if it
        # names the same library.
        raise ValueError("optimized_library_path must be the same libtsplat_hip.so on the device")
    optimized = {tuple(int(v) for v in shape) for shape in optimized_shapes}
    manifest = getattr(flow_model, "_native_rnf8_prepacked_manifest", None)
    if manifest is not None and (stages != 3 or residual_mode != "nf24_i16"):
        raise ValueError("prepacked NF24 int16 requires stages=3 and residual_mode=nf24_i16")

    runtime = _Runtime()
    codebook = make_nf8_codebook(torch)
    use_planes = bool(bf16_planes) and precision != "fp32"
    linears = [(name, m) for name, m in flow_model.named_modules() if isinstance(m, nn.Linear)]
    packing, selected_dims, plane_bytes = {}, {}, 0
    for name, module in linears:
        if not selected_by_name(name):
            continue
        codes, scales, bias, stats = _packed_linear(torch, module, name, manifest, codebook)
        device = codes[0].device
        module.register_buffer("_native_rnf8_codebook", codebook.to(device), persistent=False)
        if use_planes:
            w_hi, w_lo = make_bf16_planes(codes[0], codes[1], scales[0], precision, library=lib_path)
            for suffix, plane in (("hi", w_hi), ("lo", w_lo)):
                if plane is not None:
                    module.register_buffer(f"_native_rnf8_bf16_{suffix}", plane, persistent=False)
                    plane_bytes += plane.numel() * 2
        module.weight = nn.Parameter(torch.empty(0, dtype=torch.float32, device=device), requires_grad=False)
        if module.bias is not None:
            module.bias = nn.Parameter(torch.empty(0, dtype=torch.float32, device=device), requires_grad=False)
        shape = (int(module.in_features), int(module.out_features))
        hook = _DeviceLinear(name, runtime, lib_path, precision, use_planes, shape in optimized)
        module.forward = types.MethodType(hook.forward, module)
        module._native_avx512_forward_range = types.MethodType(hook.forward_range, module)

        weights = int(codes[0].numel())
        original, packed = _storage_bytes(weights, int(scales[0].numel()), int(bias.numel()))
        packing[name] = {**stats, "weight_elements": weights, "original_bytes": original, "packed_bytes": packed}
        selected_dims[name] = f"{shape[0]}x{shape[1]}"

    unselected = len(linears) - len(packing)
    if unselected:
        raise ValueError(f"residual NF8 strict mode left {unselected} Linear modules unquantized")
    original_bytes = sum(p["original_bytes"] for p in packing.values())
    packed_bytes = sum(p["packed_bytes"] for p in packing.values())
    weight_elements = sum(p["weight_elements"] for p in packing.values())
    squared = sum(p["weight_rmse"] ** 2 * p["weight_elements"] for p in packing.values())
    products = ("(fp32 MFMA accumulate)" if precision == "fp32" else
                f"({precision} products on bf16 MFMA, fp32 accumulate; opt-in)")
    return {
        "enabled": bool(packing),
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
        "optimized_shapes": [list(shape) for shape in sorted(optimized)],
        "row_tile": row_tile,
        "residual_mode_id": RESIDUAL_MODE_ID,
        "symbols": list(_SYMBOLS),
        "threads": int(threads),
        "strict": True,
        "prepacked_load": getattr(flow_model, "_native_rnf8_prepacked_load", {"enabled": False}),
        "selected_count": len(packing),
        "selected": list(packing),
        "selected_dims": selected_dims,
        "skipped_count": 0,
        "original_bytes": original_bytes,
        "packed_bytes": packed_bytes,
        "storage_ratio": packed_bytes / max(original_bytes, 1),
        "aggregate_weight_rmse": math.sqrt(squared / max(weight_elements, 1)),
        "aggregate_weight_max_abs": max((p["weight_max_abs"] for p in packing.values()), default=0.0),
        "packing": packing,
        "runtime": runtime.data,
        "semantics": "All selected Linear weights are decoded in registers inside the gfx950 NF24 GEMM "
                     + products + "; no fp32 weight copy is kept.",
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
