"""Host-side checks of the NF24 prepacked format (no GPU): shard naming,
manifest validation order and the resumability rule, against
scripts/native_linear_nf24_prepacked.py:177-197 and :331-343."""
from __future__ import annotations

import hashlib
import json

import pytest


def test_shard_names_and_checksums(tmp_path):
    from tsplat import nf24_prepacked as P

    name = "blocks.3.attn.qkv"
    assert P.linear_shard_name(7, name) == "linears/007_%s.safetensors" % hashlib.sha256(name.encode()).hexdigest()[:12]
    f = tmp_path / "x.bin"
    f.write_bytes(b"abc" * 1000)
    assert P.file_sha256(f) == hashlib.sha256(b"abc" * 1000).hexdigest()
    entry = {"file": "x.bin", "sha256": P.file_sha256(f), "bytes": f.stat().st_size}
    assert P._entry_ok(tmp_path, entry)
    assert not P._entry_ok(tmp_path, dict(entry, bytes=1))        # size mismatch
    assert not P._entry_ok(tmp_path, dict(entry, sha256="0" * 64))  # checksum mismatch
    assert not P._entry_ok(tmp_path, None)


@pytest.mark.parametrize("manifest,match", [
    ({"format": "other", "complete": True, "residual_mode": "nf24_i16"}, "invalid or incomplete"),
    ({"format": "triposplat_nf24_i16_v1", "complete": False, "residual_mode": "nf24_i16"}, "invalid or incomplete"),
    ({"format": "triposplat_nf24_i16_v1", "complete": True, "residual_mode": "nf8"}, "not NF24 int16"),
])
def test_loader_rejects_bad_manifests_before_touching_the_device(tmp_path, manifest, match):
    from tsplat import nf24_prepacked as P

    (tmp_path / "manifest.json").write_text(json.dumps(manifest))
    with pytest.raises(RuntimeError, match=match):
        P.load_nf24_i16_prepacked_model(tmp_path, lambda: None)


GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def test_reference_written_directory(oracle):
    """tests/golden/prepacked_toy was written by the reference's own writer
    (scripts/native_linear_nf24_prepacked.py:200-350, run by
    tests/golden/make_prepacked_golden.py).  Its manifest validates with this
    package's checks, every shard's size and checksum match the manifest, the
    shard names follow this package's naming, and the packed codes, scales
    and biases equal the oracle's packer on the source checkpoint, bit for bit
    (the reference saturated 6 stage-3 residuals of fc1: the oracle must too)."""
    import numpy as np
    from safetensors.numpy import load_file
    from tsplat import nf24_prepacked as P

    root = GOLDEN / "prepacked_toy"
    manifest = json.loads((root / "manifest.json").read_text())
    assert manifest["format"] == P.FORMAT and manifest["complete"] is True
    assert manifest["residual_mode"] == "nf24_i16" and manifest["bits_per_weight"] == 24
    src = GOLDEN / "prepacked_toy_source.safetensors"
    assert manifest["source"] == {"name": src.name, "bytes": src.stat().st_size, "sha256": P.file_sha256(src)}
    assert P._entry_ok(root, manifest["non_linear"]) and manifest["non_linear"]["tensor_count"] == 2
    source = load_file(src.as_posix())
    for index, name in enumerate(sorted(manifest["linears"])):
        entry = manifest["linears"][name]
        assert entry["file"] == P.linear_shard_name(index, name)
        assert P._entry_ok(root, entry)
        shard = load_file((root / entry["file"]).as_posix())
        assert sorted(shard) == ["bias", "code01_t", "q2_t", "scale"]
        w = source[f"{name}.weight"]
        assert (entry["out_features"], entry["in_features"]) == w.shape
        c01, q2, s = oracle.quantize_nf24_i16(w)
        assert shard["code01_t"].dtype == np.int16 and shard["q2_t"].dtype == np.int8
        assert np.array_equal(shard["code01_t"], c01) and np.array_equal(shard["q2_t"], q2)
        assert np.array_equal(shard["scale"].view(np.uint32), s.view(np.uint32))
        assert np.array_equal(shard["bias"], source.get(f"{name}.bias", np.zeros(w.shape[0], np.float32)))
        assert entry["has_bias"] == (f"{name}.bias" in source)
    nl = load_file((root / "non_linear.safetensors").as_posix())
    assert sorted(nl) == ["norm.bias", "norm.weight"]    # Linear biases live in the shards
    assert manifest["packed_bytes"] == sum(e["bytes"] for e in manifest["linears"].values()) + \
        manifest["non_linear"]["bytes"]
