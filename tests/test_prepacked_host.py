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
