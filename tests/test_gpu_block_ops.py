"""GPU parity of the flow-block / sampler kernels and the NF24 GEMM
epilogues, bit for bit.

The device kernels repeat the reference's per-element arithmetic (operation
order, fused multiply-adds, AVX-512 lane order of the reductions), so every
output must be bit-identical to the oracle restatement -- which is itself
bit-identical to the reference build (tests/test_oracle_block_ops.py) -- and
to the committed fixtures tests/golden/ew_ops.npz.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import _ew_cases as EC

pytestmark = pytest.mark.gpu
CASES = EC.cases()
GOLDEN = Path(__file__).resolve().parent / "golden" / "ew_ops.npz"


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _run_device(torch, hiplib, oracle, case, device):
    """Call the reference-named blocking symbol with device copies of the
    case's arrays; returns the arrays back on the host."""
    op, arrays, args, _ = case
    dev = {k: torch.from_numpy(v.copy()).to(device) for k, v in arrays.items()}
    conv = [dev[a].data_ptr() if isinstance(a, str) else a for a in args]
    fn = getattr(hiplib, oracle._EW_OPS[op][1])
    st = fn(*conv, 0)
    assert st == 0, (op, st)
    return {k: v.cpu().numpy() for k, v in dev.items()}


@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_named_symbols_bit_exact(oracle, cuda, hiplib, name):
    import torch

    print(f"block op {name}", flush=True)
    case = CASES[name]
    got = _run_device(torch, hiplib, oracle, case, cuda)
    exp = EC.run(oracle, case)
    gold = np.load(GOLDEN)
    for k in case[3]:
        assert np.array_equal(_bits(got[k]), _bits(exp[k])), (name, k)
        assert np.array_equal(_bits(got[k]), _bits(gold[f"{name}/out/{k}"])), (name, k)


@pytest.mark.parametrize("rows,cols,offset", [(16384, 1024, 0), (513, 1000, 0), (64, 2100, 0), (7, 100, 0),
                                             (33, 36, 0), (300, 1024, 1), (129, 1000, 1)])
def test_layernorm_full_size_bit_exact(oracle, cuda, hiplib, rows, cols, offset):
    """L = 16384 rows of C = 1024 (the block's LayerNorm) and ragged widths.
    Widths that are a multiple of 4 up to 1024 with 16-byte aligned rows take
    the LDS-staged 128-bit kernel (cols 1000, 100, 36: a partial last 16-column
    chunk, whose padded lanes the reference's variance counts); offset = 1
    misaligns the rows by one float and 2100 columns exceed the staged width,
    both taking the per-column kernel.  Every path equals the oracle bit for
    bit."""
    import torch

    print(f"layernorm {rows}x{cols} offset {offset}", flush=True)
    r = np.random.default_rng(rows + cols)
    x = (r.standard_normal((rows, cols)) * 1.5 + 0.3).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    b = (0.1 * r.standard_normal(cols)).astype(np.float32)
    exp = np.empty_like(x)
    assert oracle.ew("layernorm", x, w, b, exp, rows, cols, np.float32(1e-6), 1) == 0
    dx = torch.zeros(rows * cols + offset, device=cuda)
    dx[offset:] = torch.from_numpy(x.reshape(-1)).to(cuda)
    dw, db = (torch.from_numpy(a).to(cuda) for a in (w, b))
    out = torch.full((rows * cols + offset,), float("nan"), device=cuda)
    assert hiplib.triposplat_layernorm_f32_avx512(dx.data_ptr() + 4 * offset, dw.data_ptr(), db.data_ptr(),
                                                  out.data_ptr() + 4 * offset, rows, cols, 1e-6, 1, 0) == 0
    assert np.array_equal(_bits(out[offset:].cpu().numpy().reshape(rows, cols)), _bits(exp))


def test_fused_layernorm_modulate_and_head_norm(oracle, cuda):
    """The fused forms the flow block uses equal the reference's two-call
    sequences bit for bit: LayerNorm then modulate (scale/shift as strided
    chunks of a [B, 6C] tensor), and multi-head RMSNorm then the
    [B,L,H,64] -> [B,H,L,64] permute from inside a fused k/v projection."""
    import torch
    from tsplat import block_ops as bo

    B, L, C, H = 2, 300, 1024, 16
    r = np.random.default_rng(3)
    x = r.standard_normal((B, L, C)).astype(np.float32)
    mod = (0.2 * r.standard_normal((B, 6 * C))).astype(np.float32)
    sc, sh = mod[:, C:2 * C].copy(), mod[:, 0:C].copy()
    ln = np.empty_like(x)
    assert oracle.ew("layernorm", x, None, None, ln, B * L, C, np.float32(1e-6), 0) == 0
    assert oracle.ew("modulate_inplace", ln, sc, sh, B, L, C) == 0
    dmod = torch.from_numpy(mod).to(cuda)
    got = bo.layer_norm(torch.from_numpy(x).to(cuda), 1e-6, scale=dmod[:, C:2 * C],
                        shift=dmod[:, 0:C])
    assert np.array_equal(_bits(got.cpu().numpy()), _bits(ln))

    kv = r.standard_normal((B, L, 2, H, 64)).astype(np.float32)
    g = (1 + 0.05 * r.standard_normal((H, 64))).astype(np.float32)
    kn = np.empty((B, L, H, 64), np.float32)
    assert oracle.ew("multihead_rmsnorm", np.ascontiguousarray(kv[:, :, 0]), g, kn, B * L, H, 64,
                     np.float32(1e-12)) == 0
    dkv = torch.from_numpy(kv).to(cuda)
    dg = torch.from_numpy(g).to(cuda)
    k_bhld = bo.head_rmsnorm(dkv, dg, B, L, H, token_stride=2 * C)
    v_bhld = bo.head_rmsnorm(dkv[:, :, 1], None, B, L, H, token_stride=2 * C, normalize=False)
    assert np.array_equal(_bits(k_bhld.cpu().numpy()), _bits(kn.transpose(0, 2, 1, 3)))
    assert np.array_equal(v_bhld.cpu().numpy(), kv[:, :, 1].transpose(0, 2, 1, 3))


@pytest.mark.parametrize("M,K,N", [(600, 256, 1024), (16384, 1024, 4096), (3000, 4096, 1024), (20, 128, 96),
                                   (18432, 1024, 1024),   # whole-round split inside the second gate batch
                                   (16386, 1024, 1024),   # 2-row tail tile inside the second gate batch
                                   (8194, 1024, 1024),    # 256 x 128 tiles + the 2-row tail
                                   (17, 256, 1024),       # few rows on the 32-row skinny tile
                                   (6, 4096, 1024),       # few rows on the K-split few-row kernel
                                   (32, 1024, 3072)])
def test_gemm_epilogues(oracle, cuda, M, K, N):
    """GELU / gated-residual / add epilogues == NF24 Linear then the separate
    elementwise kernel, bit for bit, at every M (at M <= 32 the epilogue call
    runs the plain few-row call and then the epilogue, as a row tail does);
    at M <= 32 also against the oracle within the GEMM bound."""
    import torch
    from tsplat import block_ops as bo
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel

    print(f"gemm epilogues M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(M + K)
    x = torch.randn((M, K), generator=g, device=cuda)
    w = torch.randn((N, K), generator=g, device=cuda) * 0.02
    b = torch.randn((N,), generator=g, device=cuda) * 0.01
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    B = 2 if M % 2 == 0 else 1
    gate_full = torch.randn((B, 3 * N), generator=g, device=cuda)
    gate = gate_full[:, N:2 * N]
    base = torch.randn((M, N), generator=g, device=cuda)
    args = (x, codes[0], codes[1], scales[0], b)

    y_gelu = bo.nf24_linear_epilogue(*args, bo.EPILOGUE_GELU)
    y_gated = bo.nf24_linear_epilogue(*args, bo.EPILOGUE_GATED, out=base.clone(), gate=gate)
    y_add = bo.nf24_linear_epilogue(*args, bo.EPILOGUE_ADD, out=base.clone())
    lin = nf24_linear(*args)
    exp_gelu = bo.gelu_tanh(lin)
    exp_gated = base.clone().view(B, M // B, N)
    bo.residual(exp_gated, lin.clone().view(B, M // B, N), gate.contiguous())
    exp_add = bo.add_inplace(base.clone(), lin)
    torch.cuda.synchronize(cuda)
    assert torch.equal(y_gelu, exp_gelu)
    assert torch.equal(y_gated, exp_gated.view(M, N))
    assert torch.equal(y_add, exp_add)
    if M <= 32:
        xh = x.cpu().numpy()
        c01, q2, s, bh = (t.cpu().numpy() for t in (codes[0], codes[1], scales[0], b))
        lin = oracle.nf24_gemm(xh, c01, q2, s, bh)
        gl = np.empty_like(lin)
        assert oracle.ew("gelu_tanh", lin, gl, lin.size) == 0
        assert np.abs(y_gelu.cpu().numpy() - gl).max() <= 1e-5
        exp = base.cpu().numpy() + lin
        assert np.abs(y_add.cpu().numpy() - exp).max() <= 1e-5
        # gated: base[b] += lin[b] * gate[b] with rows M / B per gate batch
        gh = np.ascontiguousarray(gate.cpu().numpy())
        exp_gated = np.ascontiguousarray(base.cpu().numpy())
        delta = lin.copy()
        assert oracle.ew("gated_residual_inplace", exp_gated, delta, gh, B, M // B, N) == 0
        tol = 1e-5 * max(1.0, float(np.abs(gh).max()))
        assert np.abs(y_gated.cpu().numpy() - exp_gated).max() <= tol


def test_sampler_backend_and_flow_of_calls(oracle, cuda):
    """NativeSamplerBackend (the reference backend's interface) on device
    state dicts: CFG, Euler and AB2 equal the oracle bit for bit; strict mode
    raises on CPU tensors and counts the rejection."""
    import torch
    from tsplat.native_sampler_backend import create_triposplat_native_sampler_avx512_backend

    be, meta = create_triposplat_native_sampler_avx512_backend(enabled=True)
    assert meta["enabled"] and len(meta["symbols"]) == 3
    assert create_triposplat_native_sampler_avx512_backend(enabled=False) == (None, {"enabled": False})
    r = np.random.default_rng(9)
    pos = r.standard_normal((2, 64, 33)).astype(np.float32)
    neg = r.standard_normal((2, 64, 33)).astype(np.float32)
    g = np.array([3.0, 2.0], np.float32)
    d = lambda a: torch.from_numpy(a.copy()).to(cuda)
    P = {"latent": d(pos)}
    assert be.cfg_combine_inplace(P, {"latent": d(neg)}, d(g))
    exp = pos.copy()
    assert oracle.ew("cfg_combine_inplace", exp, neg, g, 2, 64 * 33) == 0
    assert np.array_equal(_bits(P["latent"].cpu().numpy()), _bits(exp))
    z = r.standard_normal((2, 64, 33)).astype(np.float32)
    dt = np.array([0.05, 0.05], np.float32)
    S = {"latent": d(z)}
    assert be.euler_update_inplace(S, {"latent": d(exp)}, d(dt))
    ez = z.copy()
    assert oracle.ew("euler_update_inplace", ez, exp, dt, 2, 64 * 33) == 0
    assert np.array_equal(_bits(S["latent"].cpu().numpy()), _bits(ez))
    pdt = np.array([0.04, 0.0], np.float32)
    assert be.ab2_update_inplace(S, {"latent": d(exp)}, {"latent": d(neg)}, d(dt), d(pdt))
    assert oracle.ew("ab2_update_inplace", ez, exp, neg, dt, pdt, 2, 64 * 33) == 0
    assert np.array_equal(_bits(S["latent"].cpu().numpy()), _bits(ez))
    assert be.runtime["cfg"]["calls"] == 1 and be.runtime["ab2"]["elements"] == ez.size
    with pytest.raises(RuntimeError, match="strict violation"):
        be.cfg_combine_inplace({"latent": torch.zeros(2, 3)}, {"latent": torch.zeros(2, 3)},
                               torch.ones(2))
    assert be.runtime["cfg"]["fallbacks"] == 1
