"""Model patches that route the flow block's elementwise steps to the device.

Counterparts of the reference's four block-kernel patches, with their names,
keyword arguments, module selection, strict checks and metadata keys:

  apply_triposplat_native_gelu_avx512_patch          scripts/native_gelu_avx512_patch.py:11-96
  apply_triposplat_native_silu_avx512_patch          scripts/native_silu_avx512_patch.py:6-38
  apply_triposplat_native_norm_rope_avx512_patch     scripts/native_norm_rope_avx512_patch.py:10-165
  apply_triposplat_native_block_elementwise_avx512_patch
                                                     scripts/native_block_elementwise_avx512_patch.py:6-61

The patched forwards run tsplat.block_ops (bit-identical to the reference's
AVX-512 kernels) on torch's current stream.  Where the reference requires
fp32 CPU tensors these require fp32 GPU tensors; strict mode raises on a
violation (grad mode, device / dtype, shape), non-strict mode counts it and
calls the module's original forward.  ``library_path`` names
libtsplat_hip.so (default: the in-tree build, or $TSPLAT_HIP_LIBRARY);
``threads`` is accepted and ignored.  ``seconds`` in the runtime counters is
host time spent in the call: the kernels run asynchronously on the stream.

The norm/RoPE and block-elementwise patches rewire module-level functions of
the upstream model (``model.apply_rotary_emb``) and of the reference's
attention patch (``triposplat_attention_patch``); they import those modules
by the same names unless ``model_module`` / ``attention_module`` is given.
"""
from __future__ import annotations

import re
import time
import types
from typing import Any

from . import block_ops
from ._lib import library_path as _library_path
from ._lib import load_library


def _open(library_path):
    path = _library_path(library_path)
    if not path.is_file():
        raise FileNotFoundError(f"libtsplat_hip.so not found: {path}")
    load_library(path)
    return path


def _gpu_f32(torch, t) -> bool:
    return torch.is_tensor(t) and t.device.type == "cuda" and t.dtype == torch.float32


def _input_reason(torch, x):
    if torch.is_grad_enabled():
        return "grad_enabled"
    if not _gpu_f32(torch, x):
        return f"input_{x.device.type}_{x.dtype}"
    return None


def _count(stats: dict, key: str, amount: int, started: float) -> None:
    stats["calls"] += 1
    stats[key] += int(amount)
    stats["seconds"] += time.perf_counter() - started


def _unary_patch(flow_model, module_type_name, kernel, kind, symbol, attr, *, include_regex=None,
                 exclude_regex=None, library_path=None, threads=2, strict=True, gelu=False):
    """Shared body of the GELU and SiLU patches: every module of the given
    nn type (filtered by the regexes) gets a forward that runs `kernel`."""
    import torch
    import torch.nn as nn

    path = _open(library_path)
    include = re.compile(include_regex) if include_regex else None
    exclude = re.compile(exclude_regex) if exclude_regex else None
    runtime = {"calls": 0, "elements": 0, "seconds": 0.0, "fallbacks": 0, "fallback_reasons": {},
               "per_module": {}}
    selected, skipped = [], []
    cls = getattr(nn, module_type_name)

    def wanted(name):
        return not ((include is not None and include.search(name) is None)
                    or (exclude is not None and exclude.search(name) is not None))

    def make_forward(module_name):
        def forward(self, x):
            reason = _input_reason(torch, x)
            if reason is None and gelu and getattr(self, "approximate", "none") != "tanh":
                reason = f"approximate_{getattr(self, 'approximate', 'none')}"
            if reason is not None:
                runtime["fallbacks"] += 1
                runtime["fallback_reasons"][reason] = runtime["fallback_reasons"].get(reason, 0) + 1
                if strict:
                    raise RuntimeError(f"native {module_type_name} strict violation for {module_name}: {reason}")
                return getattr(self, attr)(x)
            started = time.perf_counter()
            out = kernel(x.contiguous(), library=path)
            _count(runtime, "elements", x.numel(), started)
            item = runtime["per_module"].setdefault(module_name, {"calls": 0, "elements": 0, "seconds": 0.0})
            _count(item, "elements", x.numel(), started)
            return out.view_as(x)
        return forward

    for name, module in flow_model.named_modules():
        if not isinstance(module, cls):
            continue
        if not wanted(name):
            skipped.append(name)
            continue
        if gelu and getattr(module, "approximate", "none") != "tanh":
            if strict:
                raise ValueError(f"native GELU requires approximate=tanh: {name}")
            skipped.append(name)
            continue
        setattr(module, attr, module.forward)
        module.forward = types.MethodType(make_forward(name), module)
        selected.append(name)
    if strict and gelu and skipped:
        raise ValueError(f"native GELU strict mode left {len(skipped)} GELU modules unpatched")
    meta = {"enabled": bool(selected), "kind": kind, "library_path": path.as_posix(), "symbol": symbol,
            "threads": int(threads), "strict": bool(strict), "selected_count": len(selected),
            "selected": selected, "runtime": runtime}
    if gelu:
        meta.update({"skipped_count": len(skipped), "skipped": skipped})
    return meta


def apply_triposplat_native_gelu_avx512_patch(flow_model, *, enabled: bool = False,
                                              include_regex: str | None = None,
                                              exclude_regex: str | None = None, library_path=None,
                                              threads: int = 2, strict: bool = True) -> dict[str, Any]:
    """Every nn.GELU(approximate="tanh") of flow_model (matching the
    regexes) runs tsplat.block_ops.gelu_tanh; strict mode rejects other
    approximations at patch time."""
    if not enabled:
        return {"enabled": False}
    return _unary_patch(flow_model, "GELU", block_ops.gelu_tanh, "native_f32_gfx950_gelu_tanh_patch",
                        "tsplat_gelu_tanh_async", "_original_forward_native_gelu_avx512",
                        include_regex=include_regex, exclude_regex=exclude_regex,
                        library_path=library_path, threads=threads, strict=strict, gelu=True)


def apply_triposplat_native_silu_avx512_patch(flow_model, *, enabled: bool = False, library_path=None,
                                              threads: int = 2, strict: bool = True) -> dict[str, Any]:
    """Every nn.SiLU of flow_model runs tsplat.block_ops.silu."""
    if not enabled:
        return {"enabled": False}
    return _unary_patch(flow_model, "SiLU", block_ops.silu, "native_f32_gfx950_silu_patch",
                        "tsplat_silu_async", "_original_forward_native_silu_avx512",
                        library_path=library_path, threads=threads, strict=strict)


def apply_triposplat_native_norm_rope_avx512_patch(flow_model, *, enabled: bool = False, library_path=None,
                                                   threads: int = 2, strict: bool = True,
                                                   model_module=None) -> dict[str, Any]:
    """nn.LayerNorm over one trailing dim -> the device LayerNorm (eps inside
    the sqrt, optional affine); modules of class MultiHeadRMSNorm with a
    [heads, dim] gamma -> the device per-head RMSNorm (eps 1e-12);
    model_module.apply_rotary_emb(hidden, freqs complex64) -> the device
    interleaved RoPE; flow_model._native_avx512_functional_layernorm -> the
    device LayerNorm without affine."""
    if not enabled:
        return {"enabled": False}
    import torch
    import torch.nn as nn

    if model_module is None:
        import model as model_module  # the upstream TripoSplat model module, as the reference imports it
    path = _open(library_path)
    runtime = {"layernorm": {"calls": 0, "rows": 0, "seconds": 0.0, "fallbacks": 0},
               "rmsnorm": {"calls": 0, "vectors": 0, "seconds": 0.0, "fallbacks": 0},
               "rope": {"calls": 0, "vectors": 0, "seconds": 0.0, "fallbacks": 0, "input_copies": 0,
                        "freq_copies": 0}}
    ln_selected, rms_selected, skipped = [], [], []

    def violation(kind, name, reason):
        runtime[kind]["fallbacks"] += 1
        if strict:
            raise RuntimeError(f"native {kind} strict violation for {name}: {reason}")

    def make_layernorm(module_name):
        def forward(self, x):
            reason = _input_reason(torch, x)
            C = int(self.normalized_shape[0])
            if reason is None and (len(self.normalized_shape) != 1 or int(x.shape[-1]) != C):
                reason = "shape"
            affine = self.weight is not None
            if reason is None and affine and (self.bias is None or not _gpu_f32(torch, self.weight)
                                              or not _gpu_f32(torch, self.bias)):
                reason = "affine_parameters"
            if reason is not None:
                violation("layernorm", module_name, reason)
                return self._original_forward_native_norm_rope(x)
            started = time.perf_counter()
            src = x.contiguous()
            out = block_ops.layer_norm(src, float(self.eps), self.weight if affine else None,
                                       self.bias if affine else None, library=path)
            _count(runtime["layernorm"], "rows", src.numel() // C, started)
            return out.view_as(x)
        return forward

    def make_rmsnorm(module_name):
        def forward(self, x):
            heads, dim = (int(v) for v in self.gamma.shape)
            reason = _input_reason(torch, x)
            if reason is None and tuple(int(v) for v in x.shape[-2:]) != (heads, dim):
                reason = "shape"
            if reason is None and not _gpu_f32(torch, self.gamma):
                reason = "gamma"
            if reason is not None:
                violation("rmsnorm", module_name, reason)
                return self._original_forward_native_norm_rope(x)
            started = time.perf_counter()
            src = x.contiguous()
            outer = src.numel() // (heads * dim)
            out = block_ops.head_rmsnorm(src, self.gamma.contiguous(), 1, outer, heads, dim=dim,
                                         token_stride=heads * dim, eps=1.0e-12, out_bhld=False,
                                         library=path)
            _count(runtime["rmsnorm"], "vectors", outer * heads, started)
            return out.view_as(x)
        return forward

    for name, module in flow_model.named_modules():
        if isinstance(module, nn.LayerNorm):
            if len(module.normalized_shape) != 1:
                skipped.append(name)
                continue
            module._original_forward_native_norm_rope = module.forward
            module.forward = types.MethodType(make_layernorm(name), module)
            ln_selected.append(name)
        elif type(module).__name__ == "MultiHeadRMSNorm":
            if getattr(module, "gamma", None) is None or module.gamma.ndim != 2:
                skipped.append(name)
                continue
            module._original_forward_native_norm_rope = module.forward
            module.forward = types.MethodType(make_rmsnorm(name), module)
            rms_selected.append(name)
    if strict and skipped:
        raise ValueError(f"native norm strict mode left {len(skipped)} norm modules unpatched: {skipped[:8]}")

    original_rope = model_module.apply_rotary_emb

    def native_rope(hidden_states, freqs):
        reason = _input_reason(torch, hidden_states)
        if reason is None and (freqs.device.type != "cuda" or freqs.dtype != torch.complex64):
            reason = f"freq_{freqs.device.type}_{freqs.dtype}"
        if reason is None and int(hidden_states.shape[-1]) != 2 * int(freqs.shape[-1]):
            reason = "shape"
        if reason is None and freqs.numel() * 2 != hidden_states.numel():
            reason = "shape"
        if reason is not None:
            violation("rope", "model.apply_rotary_emb", reason)
            return original_rope(hidden_states, freqs)
        started = time.perf_counter()
        src = hidden_states
        if not src.is_contiguous():
            src = src.contiguous()
            runtime["rope"]["input_copies"] += 1
        dim = int(src.shape[-1])
        freq = torch.view_as_real(freqs).reshape(*freqs.shape[:-1], dim)
        if not freq.is_contiguous():
            freq = freq.contiguous()
            runtime["rope"]["freq_copies"] += 1
        out = block_ops.rope_complex(src, freq, library=path)
        _count(runtime["rope"], "vectors", src.numel() // dim, started)
        return out.view_as(hidden_states)

    def native_functional_layernorm(x, eps=1.0e-5):
        reason = _input_reason(torch, x)
        if reason is None and (x.ndim < 1 or int(x.shape[-1]) <= 0):
            reason = "shape"
        if reason is not None:
            violation("layernorm", "functional_final_layernorm", reason)
            return torch.nn.functional.layer_norm(x.float(), x.shape[-1:], eps=float(eps)).type_as(x)
        started = time.perf_counter()
        src = x.contiguous()
        out = block_ops.layer_norm(src, float(eps), library=path)
        _count(runtime["layernorm"], "rows", src.numel() // int(src.shape[-1]), started)
        return out.view_as(x)

    flow_model._native_avx512_functional_layernorm = native_functional_layernorm
    model_module.apply_rotary_emb = native_rope
    return {"enabled": True, "kind": "native_f32_gfx950_layernorm_rmsnorm_rope_patch",
            "library_path": path.as_posix(),
            "symbols": ["tsplat_layernorm_modulate_async", "tsplat_head_rmsnorm_async",
                        "tsplat_rope_complex_async"],
            "threads": int(threads), "strict": bool(strict),
            "layernorm_selected_count": len(ln_selected), "layernorm_selected": ln_selected,
            "rmsnorm_selected_count": len(rms_selected), "rmsnorm_selected": rms_selected,
            "skipped_count": len(skipped), "skipped": skipped, "rope_patched": True, "runtime": runtime}


def apply_triposplat_native_block_elementwise_avx512_patch(flow_model, *, enabled: bool = False,
                                                           library_path=None, threads: int = 2,
                                                           strict: bool = True,
                                                           attention_module=None) -> dict[str, Any]:
    """The adaLN modulation h = h * (1 + scale) + shift, the gated residual
    x += h * gate and x += h run on the device: they replace the attention
    patch's _modulate_inplace_preserve_order / _residual_gate_inplace_preserve_order
    and drive every UnifiedTransformerBlock's forward in the reference's
    order (modulation blocks: mod (+ shift_table) -> 6 chunks, attention and
    MLP branches each modulate -> sub-layer -> gated residual; other blocks:
    plain residual adds)."""
    if not enabled:
        return {"enabled": False}
    import torch

    if attention_module is None:
        import triposplat_attention_patch as attention_module  # as the reference imports it
    tap = attention_module
    path = _open(library_path)
    runtime = {k: {"calls": 0, "elements": 0, "seconds": 0.0, "fallbacks": 0}
               for k in ("modulate", "residual", "add")}

    def valid(t):
        return _gpu_f32(torch, t) and t.is_contiguous()

    def refuse(kind):
        runtime[kind]["fallbacks"] += 1
        if strict:
            raise RuntimeError(f"native {kind} strict violation")

    def modulate(h, scale, shift):
        if not (valid(h) and valid(scale) and valid(shift)):
            refuse("modulate")
            return tap._native_original_modulate(h, scale, shift)
        started = time.perf_counter()
        b, r, c = int(h.shape[0]), int(h.shape[-2]), int(h.shape[-1])
        block_ops.modulate(h.view(b, r, c), scale, shift, library=path)
        _count(runtime["modulate"], "elements", h.numel(), started)
        return h

    def residual(x, h, gate):
        if not (valid(x) and valid(h) and valid(gate)):
            refuse("residual")
            return tap._native_original_residual(x, h, gate)
        started = time.perf_counter()
        b, r, c = int(x.shape[0]), int(x.shape[-2]), int(x.shape[-1])
        block_ops.residual(x.view(b, r, c), h.view(b, r, c), gate, library=path)
        _count(runtime["residual"], "elements", x.numel(), started)
        return x

    def add_inplace(x, h):
        if not (valid(x) and valid(h) and x.shape == h.shape):
            refuse("add")
            x.add_(h)
            return x
        started = time.perf_counter()
        block_ops.add_inplace(x, h, library=path)
        _count(runtime["add"], "elements", x.numel(), started)
        return x

    tap._native_original_modulate = tap._modulate_inplace_preserve_order
    tap._native_original_residual = tap._residual_gate_inplace_preserve_order
    tap._modulate_inplace_preserve_order = modulate
    tap._residual_gate_inplace_preserve_order = residual

    def block_forward(self, x, mod=None, rotary_emb=None):
        if not self.modulation:
            x = add_inplace(x, self.attn(self.norm1(x), rope_emb=rotary_emb))
            return add_inplace(x, self.mlp(self.norm2(x)))
        if not self.share_mod:
            mod = self.adaLN_modulation(mod)
        table = getattr(self, "shift_table", None)
        if table is not None:
            mod = add_inplace(mod.contiguous().clone(), table.type(mod.dtype).contiguous())
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = mod.chunk(6, dim=1)
        h = self.attn(modulate(self.norm1(x), scale_msa, shift_msa), rope_emb=rotary_emb)
        x = residual(x, h, gate_msa)
        h = self.mlp(modulate(self.norm2(x), scale_mlp, shift_mlp))
        return residual(x, h, gate_mlp)

    selected = []
    for name, module in flow_model.named_modules():
        if type(module).__name__ != "UnifiedTransformerBlock":
            continue
        module._native_avx512_add_inplace = add_inplace
        module._native_avx512_modulate_inplace = modulate
        module._original_forward_native_block_elementwise = module.forward
        module.forward = types.MethodType(block_forward, module)
        selected.append(name)
    flow_model._native_avx512_add_inplace = add_inplace
    flow_model._native_avx512_modulate_inplace = modulate
    return {"enabled": True, "kind": "native_f32_gfx950_block_elementwise_patch",
            "library_path": path.as_posix(), "threads": int(threads), "strict": bool(strict),
            "selected_count": len(selected), "selected": selected, "runtime": runtime}
