#!/usr/bin/env python3
"""Write tests/golden/prepacked_toy/ with the reference's own NF24 prepacked writer.

The on-disk format triposplat_nf24_i16_v1 (manifest keys, shard naming,
tensor names, non-Linear file) is pinned by nothing but the reference's
writer, scripts/native_linear_nf24_prepacked.py:200-350
(pack_nf24_i16_checkpoint, with the packer of
native_linear_rnf8_avx512_patch.py:14-87 and the codebook of
native_linear_nf8_avx512_patch.py:12-20).  This script runs that writer --
only here, where the reference repository is mounted (REFERENCE_ROOT,
default /root/reference) -- on a small seeded checkpoint with the toy
model's layout (fc1 96->64 with bias, a LayerNorm, fc2 64->17 without
bias), and keeps the source checkpoint and the directory the writer
produced as fixtures.  Nothing of the reference travels with them: the
fixtures are the safetensors / JSON files the writer emitted.
"""
from __future__ import annotations

import os
import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "prepacked_toy_source.safetensors"
OUT = HERE / "prepacked_toy"


def source_tensors():
    r = np.random.default_rng(2024)
    return {
        "fc1.weight": (r.standard_normal((64, 96)) * 0.03).astype(np.float32),
        "fc1.bias": (r.standard_normal(64) * 0.01).astype(np.float32),
        "norm.weight": (1.0 + r.standard_normal(64) * 0.05).astype(np.float32),
        "norm.bias": (r.standard_normal(64) * 0.02).astype(np.float32),
        "fc2.weight": (r.standard_normal((17, 64)) * 0.03).astype(np.float32),
    }


def main():
    import torch
    from safetensors.torch import save_file

    ref = Path(os.environ.get("REFERENCE_ROOT", "/root/reference")) / "scripts"
    if not (ref / "native_linear_nf24_prepacked.py").is_file():
        raise SystemExit(f"reference scripts not found at {ref}")
    sys.path.insert(0, str(ref))
    from native_linear_nf24_prepacked import pack_nf24_i16_checkpoint  # the reference writer

    save_file({k: torch.from_numpy(v) for k, v in source_tensors().items()}, SOURCE.as_posix())
    if OUT.exists():
        shutil.rmtree(OUT)
    manifest = pack_nf24_i16_checkpoint(SOURCE, OUT, expected_linear_count=2)
    print({"complete": manifest["complete"], "linears": sorted(manifest["linears"]),
           "packed_bytes": manifest["packed_bytes"]})


if __name__ == "__main__":
    main()
