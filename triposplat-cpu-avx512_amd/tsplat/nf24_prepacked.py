"""NF24 int16 prepacked checkpoints (format ``triposplat_nf24_i16_v1``), GPU side.

Counterpart of scripts/native_linear_nf24_prepacked.py (and its CLI,
scripts/pack_triposplat_nf24_i16_checkpoint.py).  The on-disk format is the
reference's, unchanged, so directories written by either side load on the
other:

  <dir>/manifest.json            format, completeness flag, source file
                                 (name, bytes, sha256), per-Linear entries
                                 {file, sha256, bytes, in/out_features,
                                 has_bias, weight_elements, quantization},
                                 the non-Linear entry and packed_bytes
  <dir>/linears/NNN_<sha12>.safetensors
                                 code01_t int16 [in, out], q2_t int8 [in, out],
                                 scale fp32 [out], bias fp32 [out]
  <dir>/non_linear.safetensors   every other tensor of the source checkpoint (fp32)

What differs is where the work happens: the packer runs on the GPU (the
tsplat_nf24_pack_async kernel, bit-identical codes), the loader places the
packed planes straight into device memory as the ``_native_rnf8_*`` buffers
the Linear patch (tsplat.native_linear_rnf8_patch) consumes -- no fp32
weight is ever formed -- and ``materialize_nf24_i16_linears`` decodes on
the device for the fp32 BLAS alternative.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import re
import time
import types
from contextlib import contextmanager
from pathlib import Path
from typing import Any, Callable

from .nf24 import decode_nf24_i16_weight, decode_nf24_i16_weight_t, quantize_nf24_i16_per_output_channel

FORMAT = "triposplat_nf24_i16_v1"
_PACKED_ATTRS = ("_native_rnf8_codes0_t", "_native_rnf8_codes1_t", "_native_rnf8_codes2_t",
                 "_native_rnf8_scales0", "_native_rnf8_scales1", "_native_rnf8_scales2",
                 "_native_rnf8_codebook", "_native_rnf8_bias")

__all__ = ["FORMAT", "decode_nf24_i16_weight", "decode_nf24_i16_weight_t",
           "materialize_nf24_i16_linears", "pack_nf24_i16_checkpoint",
           "load_nf24_i16_prepacked_model"]


def _device(device):
    import torch

    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("the NF24 prepacked path keeps its tensors on the GPU")
    return device


# ------------------------------------------------------------------ files
def file_sha256(path: Path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as f:
        while True:
            block = f.read(8 << 20)
            if not block:
                return h.hexdigest()
            h.update(block)


def _atomic_json(path: Path, value: Any) -> None:
    tmp = path.with_suffix(path.suffix + ".tmp")
    tmp.write_text(json.dumps(value, indent=2, sort_keys=True) + "\n")
    os.replace(tmp, path)


def linear_shard_name(index: int, name: str) -> str:
    """linears/<index, 3 digits>_<first 12 hex of sha256(name)>.safetensors."""
    return "linears/%03d_%s.safetensors" % (index, hashlib.sha256(name.encode("utf-8")).hexdigest()[:12])


def _entry_ok(root: Path, entry: dict | None) -> bool:
    """A manifest entry counts as done when its file exists with the recorded
    size and checksum (what makes an interrupted pack resumable)."""
    if not entry or "file" not in entry or "sha256" not in entry:
        return False
    path = root / entry["file"]
    return (path.is_file() and path.stat().st_size == entry.get("bytes")
            and file_sha256(path) == entry["sha256"])


def _save_atomic(tensors: dict, target: Path) -> None:
    from safetensors.torch import save_file

    tmp = target.with_suffix(target.suffix + ".tmp")
    save_file(tensors, tmp.as_posix())
    os.replace(tmp, target)


# ------------------------------------------------------------------ packing
def pack_nf24_i16_checkpoint(source_checkpoint, output_dir, *, expected_linear_count: int = 206,
                             device=None) -> dict[str, Any]:
    """Convert a safetensors checkpoint into the NF24 int16 prepacked format.

    Every 2-D ``*.weight`` is a Linear (their count must equal
    ``expected_linear_count``); each is packed on the GPU and written with its
    bias (zeros when the source has none) to its own shard, the manifest is
    rewritten after every shard, and shards already present with a matching
    checksum are kept -- a rerun resumes an interrupted conversion and
    returns the finished manifest unchanged.
    """
    import torch
    from safetensors import safe_open

    dev = _device(device)
    src = Path(source_checkpoint).resolve()
    root = Path(output_dir).resolve()
    (root / "linears").mkdir(parents=True, exist_ok=True)
    manifest_path = root / "manifest.json"
    source = {"name": src.name, "bytes": src.stat().st_size, "sha256": file_sha256(src)}

    with safe_open(src.as_posix(), framework="pt", device="cpu") as reader:
        keys = sorted(reader.keys())
        weight_keys = [k for k in keys if k.endswith(".weight") and len(reader.get_slice(k).get_shape()) == 2]
        if len(weight_keys) != expected_linear_count:
            raise RuntimeError(f"expected {expected_linear_count} Linear weights, found {len(weight_keys)}")
        names = [k[: -len(".weight")] for k in weight_keys]
        linear_keys = set(weight_keys) | {n + ".bias" for n in names if n + ".bias" in keys}

        manifest = json.loads(manifest_path.read_text()) if manifest_path.is_file() else None
        if manifest is not None:
            if (manifest.get("format") != FORMAT or manifest.get("source") != source
                    or manifest.get("linear_count") != len(names)):
                raise RuntimeError("existing prepacked manifest does not match source checkpoint")
        else:
            manifest = {"format": FORMAT, "complete": False, "source": source,
                        "residual_mode": "nf24_i16", "bits_per_weight": 24,
                        "linear_count": len(names), "linears": {}}
        done = (len(manifest["linears"]) == len(names)
                and all(_entry_ok(root, e) for e in manifest["linears"].values()))
        if manifest.get("complete") and done and _entry_ok(root, manifest.get("non_linear")):
            return manifest
        manifest["complete"] = False

        for index, (name, wkey) in enumerate(zip(names, weight_keys)):
            if _entry_ok(root, manifest["linears"].get(name)):
                continue
            rel = linear_shard_name(index, name)
            w = reader.get_tensor(wkey).to(torch.float32).contiguous()
            codes, scales, error = quantize_nf24_i16_per_output_channel(w.to(dev))
            has_bias = name + ".bias" in keys
            bias = (reader.get_tensor(name + ".bias").to(torch.float32).contiguous() if has_bias
                    else torch.zeros(w.shape[0], dtype=torch.float32))
            _save_atomic({"code01_t": codes[0].cpu(), "q2_t": codes[1].cpu(), "scale": scales[0].cpu(),
                          "bias": bias}, root / rel)
            target = root / rel
            manifest["linears"][name] = {
                "file": rel, "sha256": file_sha256(target), "bytes": target.stat().st_size,
                "in_features": int(w.shape[1]), "out_features": int(w.shape[0]),
                "has_bias": has_bias, "weight_elements": int(w.numel()), "quantization": error,
            }
            _atomic_json(manifest_path, manifest)
            del w, codes, scales, bias

        rest = None
        if not _entry_ok(root, manifest.get("non_linear")):
            rest = {k: reader.get_tensor(k).to(torch.float32).contiguous() for k in keys if k not in linear_keys}

    if rest is not None:
        path = root / "non_linear.safetensors"
        _save_atomic(rest, path)
        manifest["non_linear"] = {"file": path.name, "sha256": file_sha256(path),
                                  "bytes": path.stat().st_size, "tensor_count": len(rest)}
    manifest["packed_bytes"] = (sum(e["bytes"] for e in manifest["linears"].values())
                                + manifest["non_linear"]["bytes"])
    manifest["complete"] = True
    _atomic_json(manifest_path, manifest)
    return manifest


# ------------------------------------------------------------------ loading
@contextmanager
def _meta_linears(torch):
    """nn.Linear parameters are created on the meta device while the model
    factory runs: the fp32 Linear weights are never allocated."""
    nn = torch.nn
    original = nn.Linear.__init__

    def init(module, in_features, out_features, bias=True, device=None, dtype=None):
        original(module, in_features, out_features, bias=bias, device="meta", dtype=dtype)

    nn.Linear.__init__ = init
    try:
        yield
    finally:
        nn.Linear.__init__ = original


def load_nf24_i16_prepacked_model(packed_dir, model_factory: Callable[[], Any], *,
                                  verify_checksums: bool = False, device=None):
    """Build ``model_factory()`` with every Linear's packed planes in GPU memory.

    Non-Linear tensors come from non_linear.safetensors (loaded onto the
    device); each Linear gets the ``_native_rnf8_*`` buffers the NF24 Linear
    patch reads, and empty placeholder parameters.  The model returned is on
    the device; ``model._native_rnf8_prepacked_load`` records what was loaded.
    """
    import torch
    from safetensors.torch import load_file

    root = Path(packed_dir).resolve()
    manifest = json.loads((root / "manifest.json").read_text())
    if manifest.get("format") != FORMAT or not manifest.get("complete"):
        raise RuntimeError(f"invalid or incomplete NF24 checkpoint: {root}")
    if manifest.get("residual_mode") != "nf24_i16":
        raise RuntimeError("prepacked checkpoint is not NF24 int16")
    dev = _device(device)

    with _meta_linears(torch):
        model = model_factory()
    linears = {n: m for n, m in model.named_modules() if isinstance(m, torch.nn.Linear)}
    if set(linears) != set(manifest["linears"]):
        missing = sorted(set(linears) - set(manifest["linears"]))
        extra = sorted(set(manifest["linears"]) - set(linears))
        raise RuntimeError(f"prepacked/model Linear mismatch: missing={missing} extra={extra}")

    info = manifest["non_linear"]
    path = root / info["file"]
    if verify_checksums and file_sha256(path) != info["sha256"]:
        raise RuntimeError(f"checksum mismatch: {path}")
    state = load_file(path.as_posix(), device=str(dev))
    result = model.load_state_dict(state, strict=False, assign=True)
    expected = {f"{n}.{f}" for n, m in linears.items()
                for f in (("weight", "bias") if m.bias is not None else ("weight",))}
    if set(result.missing_keys) != expected or result.unexpected_keys:
        raise RuntimeError(f"non-Linear state mismatch: missing={result.missing_keys} "
                           f"unexpected={result.unexpected_keys}")

    loaded = info["bytes"]
    for name, module in linears.items():
        entry = manifest["linears"][name]
        path = root / entry["file"]
        if verify_checksums and file_sha256(path) != entry["sha256"]:
            raise RuntimeError(f"checksum mismatch: {path}")
        t = load_file(path.as_posix(), device=str(dev))
        if tuple(t["code01_t"].shape) != (int(entry["in_features"]), int(entry["out_features"])):
            raise RuntimeError(f"packed shape mismatch for {name}")
        for attr, key in (("_native_rnf8_codes0_t", "code01_t"), ("_native_rnf8_codes1_t", "q2_t"),
                          ("_native_rnf8_codes2_t", "q2_t"), ("_native_rnf8_scales0", "scale"),
                          ("_native_rnf8_scales1", "scale"), ("_native_rnf8_scales2", "scale"),
                          ("_native_rnf8_bias", "bias")):
            module.register_buffer(attr, t[key], persistent=False)
        module.weight = torch.nn.Parameter(torch.empty(0, dtype=torch.float32, device=dev),
                                           requires_grad=False)
        if module.bias is not None:
            module.bias = torch.nn.Parameter(torch.empty(0, dtype=torch.float32, device=dev),
                                             requires_grad=False)
        loaded += entry["bytes"]

    model.to(dev)
    model._native_rnf8_prepacked_manifest = manifest
    model._native_rnf8_prepacked_load = {
        "enabled": True, "format": FORMAT, "directory": root.as_posix(),
        "linear_count": len(linears), "loaded_bytes": loaded,
        "checksums_verified": bool(verify_checksums), "source_checkpoint_loaded": False,
        "device": str(dev),
    }
    return model


# ------------------------------------------------------------------ fp32 alternative
def materialize_nf24_i16_linears(model, *, include_regex: str | None = None,
                                 native_weight_t_view: bool = False, release_packed: bool = True,
                                 profile: bool = True):
    """Give packed Linears exact fp32 weights (decoded on the device) and an
    ``F.linear`` forward (hipBLASLt), plus the range helper.  The weight
    values are the NF24 values exactly; only the GEMM summation order differs
    from the NF24 kernel.  Costs 4 bytes per weight of HBM instead of 3.
    """
    import torch
    import torch.nn.functional as F

    pattern = re.compile(include_regex) if include_regex else None
    available = {n for n, m in model.named_modules()
                 if isinstance(m, torch.nn.Linear) and hasattr(m, "_native_rnf8_codes0_t")}
    if not available:
        raise RuntimeError("no packed NF24 Linear modules found to materialize")
    chosen = {n for n in available if pattern is None or pattern.search(n) is not None}
    if not chosen:
        raise RuntimeError(f"NF24 materialization selected no modules with {include_regex!r}")

    runtime = {"calls": 0, "range_calls": 0, "rows": 0, "seconds": 0.0, "per_module": {}}

    def record(name, rows, seconds, is_range):
        for slot in (runtime, runtime["per_module"].setdefault(
                name, {"calls": 0, "range_calls": 0, "rows": 0, "seconds": 0.0})):
            slot["calls"] += 1
            slot["range_calls"] += int(is_range)
            slot["rows"] += rows
            slot["seconds"] += seconds

    def forward_for(name):
        def forward(self, x):
            t0 = time.perf_counter() if profile else 0.0
            y = F.linear(x, self.weight, self.bias)
            if profile:
                record(name, int(x.numel() // x.shape[-1]), time.perf_counter() - t0, False)
            return y

        return forward

    def range_for(name):
        def forward_range(self, x, output_start: int, output_count: int):
            s, c = int(output_start), int(output_count)
            if s < 0 or c <= 0 or s + c > int(self.out_features):
                raise ValueError(f"invalid materialized NF24 output range for {name}")
            t0 = time.perf_counter() if profile else 0.0
            y = F.linear(x, self.weight[s:s + c], None if self.bias is None else self.bias[s:s + c])
            if profile:
                record(name, int(x.numel() // x.shape[-1]), time.perf_counter() - t0, True)
            return y

        return forward_range

    selected, weight_bytes, bias_bytes = [], 0, 0
    for name, module in model.named_modules():
        if name not in chosen:
            continue
        args = (module._native_rnf8_codes0_t, module._native_rnf8_codes1_t, module._native_rnf8_scales0)
        weight = decode_nf24_i16_weight_t(*args).t() if native_weight_t_view else decode_nf24_i16_weight(*args)
        bias = module._native_rnf8_bias
        module.weight = torch.nn.Parameter(weight, requires_grad=False)
        module.bias = torch.nn.Parameter(bias, requires_grad=False)
        module.forward = types.MethodType(forward_for(name), module)
        module._native_avx512_forward_range = types.MethodType(range_for(name), module)
        weight_bytes += weight.numel() * weight.element_size()
        bias_bytes += bias.numel() * bias.element_size()
        selected.append(name)
        if release_packed:
            for attr in _PACKED_ATTRS:
                if hasattr(module, attr):
                    delattr(module, attr)

    metadata = {
        "enabled": True, "kind": "nf24_i16_materialized_fp32_blas_linear",
        "selected_count": len(selected), "selected": selected, "available_count": len(available),
        "include_regex": include_regex,
        "weight_layout": ("noncontiguous_out_in_view_of_contiguous_in_out" if native_weight_t_view
                          else "contiguous_out_in"),
        "weight_bytes": weight_bytes, "bias_bytes": bias_bytes,
        "packed_buffers_released": bool(release_packed), "activation_dtype": "float32",
        "weight_dtype": "float32", "source_values": "NF24 int16 nonlinear quantized weights",
        "range_api": "torch.nn.functional.linear output-row slice", "profile_enabled": bool(profile),
        "runtime": runtime, "device": "gpu (hipBLASLt fp32)",
        "semantics": "Materializes the same NF24 code values once; BLAS changes only GEMM accumulation order.",
    }
    model._nf24_materialized_linear = metadata
    return metadata


# ------------------------------------------------------------------ CLI
def main(argv=None) -> int:
    """python -m tsplat.nf24_prepacked --checkpoint X --output-dir D
    (the reference's scripts/pack_triposplat_nf24_i16_checkpoint.py)."""
    ap = argparse.ArgumentParser(description="Convert a flow checkpoint to resumable NF24 int16 shards (GPU packer).")
    ap.add_argument("--checkpoint", type=Path, required=True)
    ap.add_argument("--output-dir", type=Path, required=True)
    ap.add_argument("--expected-linear-count", type=int, default=206)
    args = ap.parse_args(argv)
    manifest = pack_nf24_i16_checkpoint(args.checkpoint, args.output_dir,
                                        expected_linear_count=args.expected_linear_count)
    print(json.dumps({"format": manifest["format"], "linear_count": manifest["linear_count"],
                      "packed_bytes": manifest["packed_bytes"],
                      "manifest": (args.output_dir / "manifest.json").resolve().as_posix()}, indent=2))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
