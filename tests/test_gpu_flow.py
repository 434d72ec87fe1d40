"""Model-level parity (configs 4 and 5 graph, reduced sizes): the device flow
model (tsplat/flow.py) against its CPU fp32 restatement (oracle/flow_ref.py)
on bit-identical packed weights and seeded inputs.

Gate: latent RMSE <= 1e-4 after one CFG Euler step (the north-star gate,
metric of scripts/compare_latent_npz.py:22-48), plus the velocity RMSE
relative to its RMS.  Kernel-level differences (MFMA summation order, exp2
form) are bounded in test_gpu_gemm / test_gpu_sdpa; here they propagate
through LayerNorm, attention and 2 or 4 residual blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(cfg, seed=20):
    z = np.random.default_rng(seed).standard_normal((cfg.latent_tokens, cfg.hidden), dtype=np.float32)
    c = np.random.default_rng(seed + 1).standard_normal((cfg.cond_tokens, cfg.hidden), dtype=np.float32)
    return z, c


@pytest.mark.parametrize("hidden,heads,blocks,L,Lc", [(128, 2, 2, 200, 40), (256, 4, 4, 130, 70)])
def test_flow_step_matches_cpu(oracle, cuda, hidden, heads, blocks, L, Lc):
    import torch
    from flow_ref import CpuFlow, combined_rmse
    from tsplat.flow import FlowConfig, FlowModel

    cfg = FlowConfig(hidden=hidden, heads=heads, blocks=blocks, latent_tokens=L, cond_tokens=Lc)
    model = FlowModel(cfg, cuda)
    z, c = _inputs(cfg)
    zn_d, v_d = model.euler_cfg_step(torch.from_numpy(z).to(cuda), torch.from_numpy(c).to(cuda))
    torch.cuda.synchronize()
    cpu = CpuFlow(model.host(), cfg, backend="oracle")
    zn_c, v_c = cpu.euler_cfg_step(z, c)
    zn_d, v_d = zn_d.cpu().numpy(), v_d.cpu().numpy()
    assert np.all(np.isfinite(zn_d))
    latent_rmse = combined_rmse(zn_d, zn_c)
    v_rel = combined_rmse(v_d, v_c) / float(np.sqrt(np.mean(v_c.astype(np.float64) ** 2)))
    print({"latent_rmse": latent_rmse, "velocity_rel_rmse": v_rel})
    assert latent_rmse <= 1e-4
    assert v_rel <= 1e-4


def test_flow_block_matches_cpu(oracle, cuda):
    """One block (config 4 structure), batch 2 with different conditions."""
    import torch
    from flow_ref import CpuFlow, combined_rmse
    from tsplat.flow import FlowConfig, FlowModel

    cfg = FlowConfig(hidden=128, heads=2, blocks=1, latent_tokens=300, cond_tokens=64)
    model = FlowModel(cfg, cuda)
    r = np.random.default_rng(3)
    x = r.standard_normal((2, 300, 128), dtype=np.float32)
    c = r.standard_normal((2, 64, 128), dtype=np.float32)
    t_mod = (r.standard_normal((2, 6 * 128)) * 0.1).astype(np.float32)
    got = model.block_forward(model.blocks[0], torch.from_numpy(x).to(cuda), torch.from_numpy(c).to(cuda),
                              torch.from_numpy(t_mod).to(cuda)).cpu().numpy()
    cpu = CpuFlow(model.host(), cfg, backend="oracle")
    want = cpu.block(cpu.p["blocks"][0], x, c, t_mod)
    rel = combined_rmse(got, want) / float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert rel <= 2e-6, rel


def test_flow_step_opt_in_bf16(oracle, cuda):
    """The opt-in bf16-MFMA products: bf16x3 in the block Linears, and in
    the block Linears and the SDPA, keeps the step within the latent gate
    against the CPU fp32 path; plain bf16 is reported (it is expected to
    miss the gate) and must be coarser than bf16x3."""
    import torch
    from flow_ref import CpuFlow, combined_rmse
    from tsplat.flow import FlowConfig, FlowModel

    cfg = FlowConfig(hidden=256, heads=4, blocks=4, latent_tokens=300, cond_tokens=70)
    model = FlowModel(cfg, cuda)
    z, c = _inputs(cfg, seed=30)
    zd, cd = torch.from_numpy(z).to(cuda), torch.from_numpy(c).to(cuda)
    strict, _ = model.euler_cfg_step(zd, cd)
    res = {}
    for name, p, include in (("bf16x3", "bf16x3", ("blocks",)), ("bf16", "bf16", ("blocks",)),
                             ("bf16x3_attn", "bf16x3", ("blocks", "attention"))):
        model.set_precision(p, include=include)
        assert model.attention_precision == (p if "attention" in include else "fp32")
        zn, _ = model.euler_cfg_step(zd, cd)
        res[name] = zn.cpu().numpy()
    model.set_precision("fp32")
    again, _ = model.euler_cfg_step(zd, cd)
    torch.cuda.synchronize()
    assert torch.equal(again, strict)
    zn_c, _ = CpuFlow(model.host(), cfg, backend="oracle").euler_cfg_step(z, c)
    rm = {p: combined_rmse(a, zn_c) for p, a in res.items()}
    rm["fp32"] = combined_rmse(strict.cpu().numpy(), zn_c)
    print({"latent_rmse_vs_cpu": rm})
    assert np.all(np.isfinite(res["bf16"])) and np.all(np.isfinite(res["bf16x3"]))
    assert rm["bf16x3"] <= 1e-4 and rm["bf16x3_attn"] <= 1e-4
    assert not np.array_equal(res["bf16x3"], strict.cpu().numpy())
    assert not np.array_equal(res["bf16x3_attn"], res["bf16x3"])
    assert rm["bf16"] > 4 * rm["bf16x3"]
