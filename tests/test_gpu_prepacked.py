"""GPU tests of the NF24 prepacked checkpoint path and the device decode.

Mirrors the reference's scripts/smoke_nf24_prepacked.py (toy model: pack,
resume, load with checksums, patch, forward; rmse < 1e-4, max-abs < 5e-4
against the fp32 model) and adds: shard codes bit-identical to the oracle's
packer, a directory written on the CPU from the oracle's codes loads and
runs to the same outputs (format interchange), resume after a lost shard,
and the device decode bit-identical to the closed form.
"""
from __future__ import annotations

import json
import shutil

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _toy():
    import torch.nn as nn
    import torch

    class ToyModel(nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = nn.Linear(96, 64, bias=True)
            self.norm = nn.LayerNorm(64)
            self.fc2 = nn.Linear(64, 17, bias=False)

        def forward(self, x):
            return self.fc2(torch.tanh(self.norm(self.fc1(x))))

    return ToyModel


@pytest.mark.parametrize("in_f,out_f", [(96, 64), (64, 17), (1024, 3072), (33, 100)])
def test_device_decode_bit_exact(oracle, cuda, in_f, out_f):
    import torch
    from tsplat.nf24 import decode_nf24_i16_weight, decode_nf24_i16_weight_t

    w = (np.random.default_rng(in_f * out_f).standard_normal((out_f, in_f)) * 0.03).astype(np.float32)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    exp_t = oracle.decode_nf24(c01, q2, s)  # [in, out], fp32(256 q01 + q2) * scale
    d = [torch.from_numpy(a).to(cuda) for a in (c01, q2, s)]
    got_t = decode_nf24_i16_weight_t(*d).cpu().numpy()
    got = decode_nf24_i16_weight(*d).cpu().numpy()
    assert np.array_equal(got_t.view(np.uint32), exp_t.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(exp_t.T).view(np.uint32))


def test_prepacked_smoke_resume_and_interchange(oracle, cuda, tmp_path):
    import torch
    from safetensors.numpy import save_file as save_np
    from safetensors.torch import save_file
    from tsplat import nf24_prepacked as P
    from tsplat.native_linear_rnf8_patch import apply_triposplat_native_rnf8_avx512_patch

    ToyModel = _toy()
    torch.manual_seed(0)
    source = ToyModel().eval()
    x = torch.randn(25, 96, dtype=torch.float32)
    with torch.inference_mode():
        reference = source(x)
    ckpt = tmp_path / "toy.safetensors"
    packed = tmp_path / "packed"
    save_file(source.state_dict(), ckpt.as_posix())

    manifest = P.pack_nf24_i16_checkpoint(ckpt, packed, expected_linear_count=2)
    assert P.pack_nf24_i16_checkpoint(ckpt, packed, expected_linear_count=2) == manifest
    assert manifest["complete"] and manifest["linear_count"] == 2
    with pytest.raises(RuntimeError, match="expected 3 Linear weights"):
        P.pack_nf24_i16_checkpoint(ckpt, tmp_path / "other", expected_linear_count=3)

    # shard codes == the oracle's packer, bit for bit; bias zeros for fc2
    from safetensors.numpy import load_file as load_np

    sd = {k: v.numpy() for k, v in source.state_dict().items()}
    for name in ("fc1", "fc2"):
        shard = load_np((packed / manifest["linears"][name]["file"]).as_posix())
        c01, q2, s = oracle.quantize_nf24_i16(sd[f"{name}.weight"])
        assert np.array_equal(shard["code01_t"], c01) and np.array_equal(shard["q2_t"], q2)
        assert np.array_equal(shard["scale"].view(np.uint32), s.view(np.uint32))
        exp_bias = sd.get(f"{name}.bias", np.zeros(s.shape, np.float32))
        assert np.array_equal(shard["bias"], exp_bias)

    # resume: a lost shard is rewritten identically, the manifest unchanged
    lost = packed / manifest["linears"]["fc2"]["file"]
    lost.unlink()
    assert P.pack_nf24_i16_checkpoint(ckpt, packed, expected_linear_count=2) == manifest

    def run(directory):
        model = P.load_nf24_i16_prepacked_model(directory, ToyModel, verify_checksums=True).eval()
        meta = apply_triposplat_native_rnf8_avx512_patch(
            model, enabled=True, include_regex=r".*", threads=2, strict=True, stages=3,
            residual_mode="nf24_i16")
        with torch.inference_mode():
            out = model(x.to(cuda))
        return out.cpu(), meta, model

    observed, meta, model = run(packed)
    diff = observed - reference
    rmse = float(torch.sqrt(torch.mean(diff.square())))
    max_abs = float(diff.abs().max())
    assert meta["selected_count"] == 2 and meta["runtime"]["fallbacks"] == 0
    assert meta["prepacked_load"]["source_checkpoint_loaded"] is False
    assert model.fc1._native_rnf8_codes0_t.device.type == "cuda"
    assert rmse < 1.0e-4 and max_abs < 5.0e-4, (rmse, max_abs)

    # interchange: a directory written on the CPU from the oracle's codes
    other = tmp_path / "cpu_written"
    (other / "linears").mkdir(parents=True)
    shutil.copy(packed / "non_linear.safetensors", other / "non_linear.safetensors")
    m2 = json.loads((packed / "manifest.json").read_text())
    for index, name in enumerate(("fc1", "fc2")):
        c01, q2, s = oracle.quantize_nf24_i16(sd[f"{name}.weight"])
        rel = P.linear_shard_name(index, name)
        save_np({"code01_t": c01, "q2_t": q2, "scale": s,
                 "bias": sd.get(f"{name}.bias", np.zeros(s.shape, np.float32))}, (other / rel).as_posix())
        m2["linears"][name].update(file=rel, sha256=P.file_sha256(other / rel),
                                   bytes=(other / rel).stat().st_size)
    (other / "manifest.json").write_text(json.dumps(m2))
    observed2, _, _ = run(other)
    assert torch.equal(observed, observed2)


def test_materialize_decodes_exactly(oracle, cuda, tmp_path):
    import torch
    from safetensors.torch import save_file
    from tsplat import nf24_prepacked as P

    ToyModel = _toy()
    torch.manual_seed(1)
    source = ToyModel().eval()
    ckpt = tmp_path / "toy.safetensors"
    save_file(source.state_dict(), ckpt.as_posix())
    P.pack_nf24_i16_checkpoint(ckpt, tmp_path / "p", expected_linear_count=2)
    model = P.load_nf24_i16_prepacked_model(tmp_path / "p", ToyModel).eval()
    c01, q2, s = (getattr(model.fc1, a).cpu().numpy() for a in
                  ("_native_rnf8_codes0_t", "_native_rnf8_codes1_t", "_native_rnf8_scales0"))
    meta = P.materialize_nf24_i16_linears(model)
    assert meta["selected_count"] == 2 and not hasattr(model.fc1, "_native_rnf8_codes0_t")
    exp = np.ascontiguousarray(oracle.decode_nf24(c01, q2, s).T)
    assert np.array_equal(model.fc1.weight.detach().cpu().numpy().view(np.uint32), exp.view(np.uint32))
    x = torch.randn(9, 96, device=cuda)
    with torch.inference_mode():
        y = model(x)
        yr = model.fc1._native_avx512_forward_range(x, 16, 32)
        yf = model.fc1(x)
    assert y.shape == (9, 17) and bool(torch.isfinite(y).all())
    assert torch.allclose(yr, yf[:, 16:48], rtol=1e-5, atol=1e-6)
    assert meta["runtime"]["range_calls"] == 1


def test_reference_written_directory_interchange(oracle, cuda, tmp_path):
    """The directory the reference's own writer produced
    (tests/golden/prepacked_toy, see make_prepacked_golden.py) against this
    package: (1) packing the same source checkpoint here gives the same
    manifest (the float quantization statistics to 1e-5 relative, everything
    else equal) and byte-identical shard files (same sha256); (2) the
    reference-written directory loads through load_nf24_i16_prepacked_model
    with checksum verification and runs the toy model on the device, matching
    the oracle GEMM chain on the decoded weights."""
    from pathlib import Path

    import torch
    from safetensors.numpy import load_file as load_np
    from tsplat import nf24_prepacked as P
    from tsplat.native_linear_rnf8_patch import apply_triposplat_native_rnf8_avx512_patch

    golden = Path(__file__).resolve().parent / "golden"
    ref_dir = golden / "prepacked_toy"
    ref_manifest = json.loads((ref_dir / "manifest.json").read_text())
    src = tmp_path / "prepacked_toy_source.safetensors"   # same name: the manifest records it
    shutil.copy(golden / "prepacked_toy_source.safetensors", src)
    ours = P.pack_nf24_i16_checkpoint(src, tmp_path / "ours", expected_linear_count=2)

    def strip(m):
        m = json.loads(json.dumps(m))
        stats = {}
        for name, e in m["linears"].items():
            stats[name] = e.pop("quantization")
        return m, stats

    a, sa = strip(ours)
    b, sb = strip(ref_manifest)
    assert a == b                                         # names, files, sha256, sizes, shapes, source
    for name in sa:
        qa, qb = sa[name], sb[name]
        assert sorted(qa) == sorted(qb)
        assert qa["nf8_derived_alphabet_size"] == qb["nf8_derived_alphabet_size"] == 163
        for st_a, st_b in zip(qa["stages"], qb["stages"]):
            assert st_a["saturated_values"] == st_b["saturated_values"]
            assert st_a["quantizer"] == st_b["quantizer"]
            for key in ("residual_max_abs", "residual_rmse"):
                assert abs(st_a[key] - st_b[key]) <= 1e-5 * abs(st_b[key]) + 1e-12, (name, key)

    ToyModel = _toy()
    model = P.load_nf24_i16_prepacked_model(ref_dir, ToyModel, verify_checksums=True).eval()
    meta = apply_triposplat_native_rnf8_avx512_patch(
        model, enabled=True, include_regex=r".*", threads=2, strict=True, stages=3, residual_mode="nf24_i16")
    assert meta["selected_count"] == 2 and meta["prepacked_load"]["checksums_verified"] is True
    x = np.random.default_rng(8).standard_normal((25, 96)).astype(np.float32)
    with torch.inference_mode():
        h1 = model.fc1(torch.from_numpy(x).to(cuda)).cpu().numpy()
    shard = load_np((ref_dir / ref_manifest["linears"]["fc1"]["file"]).as_posix())
    want = oracle.nf24_gemm(x, shard["code01_t"], shard["q2_t"], shard["scale"], shard["bias"])
    assert np.abs(h1 - want).max() <= 2e-5
