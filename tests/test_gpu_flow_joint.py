"""The single-stream graph and the reference's exactness-preserving work
reduction (tsplat/flow_joint.py), at reduced sizes.

* the selected-rows final block gives the latent rows of the full final
  block bit for bit (same per-row arithmetic; only unused rows are skipped);
* the compressed negative branch (one condition row + log(M) key bias)
  matches the full negative branch (M identical rows) to rounding:
  exp(s + log M) versus M exp(s) summed key by key;
* a CFG Euler step with both reductions matches the CPU restatement of the
  full computation (oracle/flow_ref.py CpuJointFlow) within the north-star
  gate, latent RMSE <= 1e-4.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _model(cuda, hidden=128, heads=2, blocks=3, L=200, Lc=40):
    from tsplat.flow import FlowConfig
    from tsplat.flow_joint import JointFlowModel

    cfg = FlowConfig(hidden=hidden, heads=heads, blocks=blocks, latent_tokens=L, cond_tokens=Lc)
    return cfg, JointFlowModel(cfg, cuda)


def _inputs(cfg, seed=30):
    z = np.random.default_rng(seed).standard_normal((cfg.latent_tokens, cfg.hidden), dtype=np.float32)
    c = np.random.default_rng(seed + 1).standard_normal((cfg.cond_tokens, cfg.hidden), dtype=np.float32)
    return z, c


def test_selected_final_block_is_exact(cuda):
    import torch

    cfg, model = _model(cuda)
    z, c = (torch.from_numpy(a).to(cuda) for a in _inputs(cfg))
    t = torch.full((1,), 700.0, device=cuda)
    full = model.velocity(z, c, t, selected_final=False)
    sel = model.velocity(z, c, t, selected_final=True)
    torch.cuda.synchronize(cuda)
    assert torch.equal(full, sel)


@pytest.mark.parametrize("Lc", [40, 2048])
def test_negative_compression_matches_full_branch(cuda, Lc):
    import torch

    cfg, model = _model(cuda, Lc=Lc)
    z = torch.from_numpy(_inputs(cfg)[0]).to(cuda)
    zero = torch.zeros((Lc, cfg.hidden), device=cuda)
    t = torch.full((1,), 1000.0, device=cuda)
    full = model.velocity(z, zero, t, compress=False, selected_final=False)
    comp = model.velocity(z, zero, t, compress=True, selected_final=True)
    d = (comp - full).double()
    rms = float(full.double().square().mean().sqrt())
    rel = float(d.square().mean().sqrt()) / rms
    print({"Lc": Lc, "rel_rmse": rel, "max_abs": float(d.abs().max())})
    assert rel <= 2e-6


def test_reduced_step_matches_cpu_full_computation(oracle, cuda):
    import torch
    from flow_ref import CpuJointFlow, combined_rmse

    cfg, model = _model(cuda, hidden=128, heads=2, blocks=2, L=150, Lc=48)
    z, c = _inputs(cfg)
    zn_d, v_d = model.euler_cfg_step(torch.from_numpy(z).to(cuda), torch.from_numpy(c).to(cuda),
                                     reduce_work=True)
    torch.cuda.synchronize(cuda)
    cpu = CpuJointFlow(model.host(), cfg, backend="oracle")
    zn_c, v_c = cpu.joint_euler_cfg_step(z, c)
    zn_d, v_d = zn_d.cpu().numpy(), v_d.cpu().numpy()
    latent_rmse = combined_rmse(zn_d, zn_c)
    v_rel = combined_rmse(v_d, v_c) / float(np.sqrt(np.mean(v_c.astype(np.float64) ** 2)))
    print({"latent_rmse": latent_rmse, "velocity_rel_rmse": v_rel})
    assert np.all(np.isfinite(zn_d))
    assert latent_rmse <= 1e-4 and v_rel <= 1e-4


def test_reduced_step_opt_in_bf16x3_attention(oracle, cuda):
    """The single-stream graph with bf16x3 products in its block Linears and
    in every SDPA (key-bias self attention, the packed selected-rows final
    block) stays within the latent gate against the CPU fp32 full
    computation, differs from the strict step, and the strict step is
    restored bit for bit afterwards."""
    import torch
    from flow_ref import CpuJointFlow, combined_rmse

    cfg, model = _model(cuda, hidden=128, heads=2, blocks=2, L=150, Lc=48)
    z, c = _inputs(cfg)
    zd, cd = torch.from_numpy(z).to(cuda), torch.from_numpy(c).to(cuda)
    strict, _ = model.euler_cfg_step(zd, cd, reduce_work=True)
    model.set_precision("bf16x3", include=("blocks", "attention"))
    assert model.attention_precision == "bf16x3"
    zn3, v3 = model.euler_cfg_step(zd, cd, reduce_work=True)
    model.set_precision("fp32")
    again, _ = model.euler_cfg_step(zd, cd, reduce_work=True)
    torch.cuda.synchronize(cuda)
    assert torch.equal(again, strict)
    assert not torch.equal(zn3, strict)
    zn_c, v_c = CpuJointFlow(model.host(), cfg, backend="oracle").joint_euler_cfg_step(z, c)
    latent_rmse = combined_rmse(zn3.cpu().numpy(), zn_c)
    print({"bf16x3_latent_rmse": latent_rmse})
    assert np.all(np.isfinite(zn3.cpu().numpy()))
    assert latent_rmse <= 1e-4
