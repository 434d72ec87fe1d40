"""Device sampler backend: CFG combine, Euler and AB2 state updates.

Mirror of scripts/native_sampler_avx512_backend.py (class
NativeSamplerAVX512Backend and create_triposplat_native_sampler_avx512_backend):
same methods, state dictionaries, runtime counters and metadata keys, with
the device check flipped -- every tensor, including the per-batch guidance
/ dt vectors, must be a contiguous fp32 GPU tensor.  The kernels
(block_ops.hip) repeat the reference's arithmetic
(scripts/native_sampler_avx512.c:19-134) bit for bit and run on torch's
current stream.
"""
from __future__ import annotations

import time
from typing import Any

from ._lib import check_status, current_stream_handle, library_path, load_library


class NativeSamplerBackend:
    def __init__(self, *, library_path: str | None = None, threads: int = 0, strict: bool = True):
        import torch

        self.torch = torch
        self.threads = int(threads)  # accepted for signature parity; unused on the device
        self.strict = bool(strict)
        self.lib = load_library(library_path)
        self.path = _path(library_path)
        self.runtime = {
            "cfg": {"calls": 0, "tensors": 0, "elements": 0, "seconds": 0.0, "fallbacks": 0},
            "euler": {"calls": 0, "tensors": 0, "elements": 0, "seconds": 0.0, "fallbacks": 0},
            "ab2": {"calls": 0, "tensors": 0, "elements": 0, "seconds": 0.0, "fallbacks": 0},
        }

    def _is_dev(self, t) -> bool:
        torch = self.torch
        return (torch.is_tensor(t) and t.device.type == "cuda" and t.dtype == torch.float32
                and t.is_contiguous())

    def _valid_vector(self, value, batch: int) -> bool:
        return self._is_dev(value) and value.ndim == 1 and int(value.numel()) == int(batch)

    def _valid_state_pair(self, left: dict, right: dict, batch: int) -> bool:
        if left.keys() != right.keys():
            return False
        for key, value in left.items():
            other = right[key]
            if not (self._is_dev(value) and self._is_dev(other) and value.shape == other.shape
                    and value.device == other.device and value.ndim >= 1
                    and int(value.shape[0]) == int(batch)):
                return False
        return True

    def _reject(self, section: str, reason: str) -> bool:
        self.runtime[section]["fallbacks"] += 1
        if self.strict:
            raise RuntimeError(f"native sampler strict violation ({section}): {reason}")
        return False

    def _run(self, section, fn_name, state, extra, vectors, batch):
        torch = self.torch
        started = time.perf_counter()
        elements = 0
        for key, value in state.items():
            per_batch = int(value.numel() // batch)
            with torch.cuda.device(value.device):
                status = getattr(self.lib, fn_name)(
                    value.data_ptr(), *[d[key].data_ptr() for d in extra],
                    *[v.data_ptr() for v in vectors], batch, per_batch,
                    current_stream_handle(value.device))
            check_status(status, fn_name)
            elements += int(value.numel())
        rt = self.runtime[section]
        rt["seconds"] += time.perf_counter() - started
        rt["calls"] += 1
        rt["tensors"] += len(state)
        rt["elements"] += elements
        return True

    def cfg_combine_inplace(self, positive: dict, negative: dict, guidance) -> bool:
        """positive = g * positive - (g - 1) * negative, per batch."""
        batch = int(guidance.numel()) if self.torch.is_tensor(guidance) else -1
        if not self._valid_vector(guidance, batch):
            return self._reject("cfg", "guidance must be a contiguous GPU float32 [batch]")
        if not self._valid_state_pair(positive, negative, batch):
            return self._reject("cfg", "prediction states must be matching contiguous GPU float32 tensors")
        return self._run("cfg", "tsplat_cfg_combine_async", positive, [negative], [guidance], batch)

    def euler_update_inplace(self, sample: dict, prediction: dict, dt) -> bool:
        """sample -= dt[b] * prediction."""
        batch = int(dt.numel()) if self.torch.is_tensor(dt) else -1
        if not self._valid_vector(dt, batch):
            return self._reject("euler", "dt must be a contiguous GPU float32 [batch]")
        if not self._valid_state_pair(sample, prediction, batch):
            return self._reject("euler", "state and prediction must be matching contiguous GPU float32 tensors")
        return self._run("euler", "tsplat_euler_update_async", sample, [prediction], [dt], batch)

    def ab2_update_inplace(self, sample: dict, prediction: dict, previous_prediction: dict, dt,
                           previous_dt) -> bool:
        batch = int(dt.numel()) if self.torch.is_tensor(dt) else -1
        valid = self._valid_vector(dt, batch) and self._valid_vector(previous_dt, batch)
        valid = valid and self._valid_state_pair(sample, prediction, batch)
        valid = valid and self._valid_state_pair(sample, previous_prediction, batch)
        if not valid:
            return self._reject("ab2", "AB2 inputs must be matching contiguous GPU float32 tensors")
        return self._run("ab2", "tsplat_ab2_update_async", sample, [prediction, previous_prediction],
                         [dt, previous_dt], batch)

    def metadata(self) -> dict[str, Any]:
        return {
            "enabled": True,
            "kind": "native_f32_gfx950_fused_cfg_euler_ab2_sampler",
            "library_path": self.path,
            "symbols": [
                "triposplat_cfg_combine_inplace_f32_avx512",
                "triposplat_euler_update_inplace_f32_avx512",
                "triposplat_ab2_update_inplace_f32_avx512",
            ],
            "threads": self.threads,
            "strict": self.strict,
            "inplace_cfg": True,
            "inplace_state_update": True,
            "runtime": self.runtime,
        }


# The reference's class name (native_sampler_avx512_backend.py:9), so code
# that constructs or type-checks against it switches by import alone.
NativeSamplerAVX512Backend = NativeSamplerBackend


def _path(p):
    return library_path(p).as_posix()


def create_triposplat_native_sampler_avx512_backend(*, enabled: bool = False,
                                                    library_path: str | None = None,
                                                    threads: int = 0, strict: bool = True):
    """Same contract as the reference factory: (None, {"enabled": False}) when
    disabled, else (backend, backend.metadata())."""
    if not enabled:
        return None, {"enabled": False}
    backend = NativeSamplerBackend(library_path=library_path, threads=threads, strict=strict)
    return backend, backend.metadata()
