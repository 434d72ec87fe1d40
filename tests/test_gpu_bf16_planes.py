"""GPU tests of the bf16 weight planes (tsplat_nf24_bf16_planes_async and the
*_planes_async GEMM / fused-QKV entries; no counterpart in the reference).

The planes hold what the bf16 kernels otherwise decode and split from the
NF24 codes in every call, so a call that reads them must equal, bit for bit,
the same call that decodes the codes: on every tile shape the launch model
picks, with every epilogue, on column ranges, with a row tail split off to
the strict path, and through a flow model.  The builder itself is held to
oracle.nf24_bf16_split_w (pinned against exact rationals in
tests/test_oracle_bf16.py).
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import seeded_linear

pytestmark = pytest.mark.gpu


def _packed(torch, oracle, cuda, M, K, N, seed):
    x, w, b = seeded_linear(seed, M, K, N, w_scale=0.02)
    c01, q2, s = oracle.quantize_nf24_i16(w)
    d = [torch.from_numpy(np.ascontiguousarray(a)).to(cuda) for a in (x, c01, q2, s, b)]
    return d


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("K,N", [(64, 128), (100, 72), (1024, 3072), (4096, 1024)])
def test_planes_equal_oracle_split(oracle, cuda, precision, K, N):
    """w_hi / w_lo equal the oracle's split of the exact decode, k-blocked
    [ceil(K / 32), N, 32] with zeros past K."""
    import torch
    from tsplat.nf24 import bf16_planes, planes_to_kn

    _, c01, q2, s, _ = _packed(torch, oracle, cuda, 1, K, N, 900 + K + N)
    w_hi, w_lo = bf16_planes(c01, q2, s, precision)
    torch.cuda.synchronize(cuda)
    wh, wl = oracle.nf24_bf16_split_w(c01.cpu().numpy(), q2.cpu().numpy(), s.cpu().numpy())
    planes = [(w_hi, wh)] + ([(w_lo, wl)] if precision == "bf16x3" else [])
    for plane, want in planes:
        assert tuple(plane.shape) == ((K + 31) // 32, N, 32)
        got = planes_to_kn(plane, K).float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
        pad = plane.permute(0, 2, 1).reshape(-1, N)[K:]
        assert not bool(pad.float().abs().sum())
    if precision != "bf16x3":
        assert w_lo is None


# (M, K, N, output range): rows / columns that reach each tile shape of the
# launch model (256 x 256, 192 x 256, 256 x 128, 128 x 64, 256 x 192, and the
# 128 x 128 tile for narrow calls), a split-off row tail, K not a multiple of
# 32 (the last block's zero padding), a column range.
SHAPES = [(16384, 256, 1024, None), (12288, 256, 1024, None), (8192, 256, 1024, None),
          (2048, 256, 1024, None), (4096, 256, 3072, None), (600, 256, 128, None),
          (12294, 256, 1024, None), (700, 100, 512, None), (3000, 512, 2048, (256, 1280))]


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("M,K,N,rng", SHAPES)
def test_planes_gemm_bitwise(oracle, cuda, precision, M, K, N, rng):
    import torch
    from tsplat.nf24 import bf16_planes, nf24_linear

    print(f"planes gemm {precision} M={M} K={K} N={N} range={rng}", flush=True)
    x, c01, q2, s, b = _packed(torch, oracle, cuda, M, K, N, 910 + M + K)
    planes = bf16_planes(c01, q2, s, precision)
    start, count = rng if rng else (0, None)
    want = nf24_linear(x, c01, q2, s, b, output_start=start, output_count=count, precision=precision)
    got = nf24_linear(x, c01, q2, s, b, output_start=start, output_count=count, precision=precision,
                      planes=planes)
    torch.cuda.synchronize(cuda)
    assert torch.equal(got, want)


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("epilogue", [2, 3, 4])
@pytest.mark.parametrize("M,N", [(8192, 1024), (4096, 3072), (12294, 1024)])
def test_planes_epilogues_bitwise(oracle, cuda, precision, epilogue, M, N):
    import torch
    from tsplat import block_ops as bo
    from tsplat.nf24 import bf16_planes

    print(f"planes epilogue {precision} epi={epilogue} M={M} N={N}", flush=True)
    K = 256
    x, c01, q2, s, b = _packed(torch, oracle, cuda, M, K, N, 930 + M + epilogue)
    planes = bf16_planes(c01, q2, s, precision)
    g = torch.Generator(device=cuda).manual_seed(M + epilogue)
    base = torch.randn((M, N), generator=g, device=cuda)
    gate = torch.randn((2, N), generator=g, device=cuda) if epilogue == 3 else None
    outs = []
    for pl in (None, planes):
        out = base.clone() if epilogue in (3, 4) else None
        outs.append(bo.nf24_linear_epilogue(x, c01, q2, s, b, epilogue, out=out, gate=gate,
                                            precision=precision, planes=pl))
    torch.cuda.synchronize(cuda)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
@pytest.mark.parametrize("B,L,H,kv_layout", [(2, 700, 4, "bhld"), (1, 2048, 16, "packed"),
                                             (2, 6147, 16, "bhld")])
def test_planes_qkv_bitwise(cuda, precision, B, L, H, kv_layout):
    import torch
    from tsplat.nf24 import bf16_planes, quantize_nf24_i16_per_output_channel
    from tsplat.qkv import gemm_nf24_qkv_direct

    print(f"planes qkv {precision} B={B} L={L} H={H} {kv_layout}", flush=True)
    C, K = H * 64, 256
    g = torch.Generator(device=cuda).manual_seed(B * L + H)
    x = torch.randn((B * L, K), generator=g, device=cuda)
    w = torch.randn((3 * C, K), generator=g, device=cuda) * 0.02
    bias = torch.randn((3 * C,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    r = np.random.default_rng(L)
    ang = r.standard_normal((1, L, H, 32)).astype(np.float32)
    fr = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1).reshape(1, L, H, 64)).to(cuda)
    qg = torch.from_numpy((1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)).to(cuda)
    kg = torch.from_numpy((1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)).to(cuda)
    planes = bf16_planes(codes[0], codes[1], scales[0], precision)
    args = (x, codes[0], codes[1], scales[0], bias, fr, qg, kg, B, L, H)
    want = gemm_nf24_qkv_direct(*args, precision=precision, kv_layout=kv_layout)
    got = gemm_nf24_qkv_direct(*args, precision=precision, kv_layout=kv_layout, planes=planes)
    torch.cuda.synchronize(cuda)
    for a_, b_ in zip(got, want):
        assert torch.equal(a_, b_)


def test_planes_rejected_shapes(oracle, cuda):
    """Planes of the wrong shape or dtype raise before any launch; precision
    'fp32' has no planes."""
    import torch
    from tsplat.nf24 import bf16_planes, nf24_linear

    x, c01, q2, s, b = _packed(torch, oracle, cuda, 300, 64, 128, 950)
    w_hi, w_lo = bf16_planes(c01, q2, s, "bf16x3")
    with pytest.raises(ValueError):
        nf24_linear(x, c01, q2, s, b, precision="bf16x3", planes=(w_hi, None))
    with pytest.raises(ValueError):
        nf24_linear(x, c01, q2, s, b, precision="bf16x3", planes=(w_hi.transpose(0, 1).contiguous(), w_lo))
    with pytest.raises(ValueError):
        bf16_planes(c01, q2, s, "fp32")


def test_flow_model_planes_bitwise(cuda):
    """A CFG Euler step with the bf16x3 block Linears and attention reading
    their weight planes equals the same step decoding the codes, bit for bit."""
    import torch
    from tsplat.flow import FlowConfig, FlowModel

    cfg = FlowConfig(hidden=256, heads=4, blocks=2, latent_tokens=300, cond_tokens=40)
    model = FlowModel(cfg, cuda)
    r = np.random.default_rng(7)
    z = torch.from_numpy(r.standard_normal((cfg.latent_tokens, cfg.hidden), dtype=np.float32)).to(cuda)
    c = torch.from_numpy(r.standard_normal((cfg.cond_tokens, cfg.hidden), dtype=np.float32)).to(cuda)
    outs = []
    for planes in (False, True):
        model.set_precision("bf16x3", include=("blocks", "attention"), planes=planes)
        outs.append(model.euler_cfg_step(z, c))
    torch.cuda.synchronize(cuda)
    assert all(lin.planes is not None for lin in model.blocks[0].lin.values())
    for a_, b_ in zip(outs[0], outs[1]):
        assert torch.equal(a_, b_)


def test_linear_patch_planes_bitwise(cuda):
    """The reference-named Linear patch in bf16x3 with and without the weight
    planes: same outputs bit for bit (forward and the range hook), the planes
    recorded in the metadata."""
    import copy

    import torch
    from torch import nn
    from tsplat.native_linear_rnf8_patch import apply_triposplat_native_rnf8_avx512_patch

    torch.manual_seed(5)
    base = nn.Sequential(nn.Linear(256, 512), nn.GELU(approximate="tanh"), nn.Linear(512, 256)).to(cuda).eval()
    x = torch.randn(300, 256, device=cuda)
    outs, metas, models = [], [], []
    for planes in (False, True):
        model = copy.deepcopy(base)
        metas.append(apply_triposplat_native_rnf8_avx512_patch(
            model, enabled=True, include_regex=r".*", strict=True, stages=3, residual_mode="nf24_i16",
            precision="bf16x3", bf16_planes=planes))
        with torch.inference_mode():
            outs.append((model(x), model[0]._native_avx512_forward_range(x, 128, 256)))
        models.append(model)
    torch.cuda.synchronize(cuda)
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert metas[1]["gemm_bf16_planes"] and not metas[0]["gemm_bf16_planes"]
    assert metas[1]["bf16_plane_bytes"] == (256 * 512 + 512 * 256) * 4
    assert hasattr(models[1][0], "_native_rnf8_bf16_lo") and not hasattr(models[0][0], "_native_rnf8_bf16_hi")
