"""The single-stream graph and the reference's exactness-preserving work
reduction (tsplat/flow_joint.py), at reduced sizes.

* the selected-rows final block gives the latent and camera rows of the
  full final block bit for bit (same per-row arithmetic; only unused rows
  are skipped);
* the compressed negative branch (one condition row + log(M) key bias)
  matches the full negative branch (M identical rows) to rounding:
  exp(s + log M) versus M exp(s) summed key by key;
* a CFG Euler step with both reductions matches the CPU restatement of the
  full computation (oracle/flow_ref.py CpuJointFlow) within the north-star
  gate, RMSE <= 1e-4 for the latent and for the camera state.
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
    from tsplat.flow_joint import camera_state

    z = np.random.default_rng(seed).standard_normal((cfg.latent_tokens, cfg.hidden), dtype=np.float32)
    c = np.random.default_rng(seed + 1).standard_normal((cfg.cond_tokens, cfg.hidden), dtype=np.float32)
    return z, c, camera_state(cfg, seed + 2)


def test_selected_final_block_is_exact(cuda):
    import torch

    cfg, model = _model(cuda)
    z, c, cam = (torch.from_numpy(a).to(cuda) for a in _inputs(cfg))
    t = torch.full((1,), 700.0, device=cuda)
    full, full_cam = model.velocity(z, c, cam, t, selected_final=False)
    sel, sel_cam = model.velocity(z, c, cam, t, selected_final=True)
    torch.cuda.synchronize(cuda)
    assert full_cam.shape == (1, cfg.cam_channels)
    assert torch.equal(full, sel) and torch.equal(full_cam, sel_cam)


@pytest.mark.parametrize("Lc", [40, 2048])
def test_negative_compression_matches_full_branch(cuda, Lc):
    import torch

    cfg, model = _model(cuda, Lc=Lc)
    z, _, cam = (torch.from_numpy(a).to(cuda) for a in _inputs(cfg))
    zero = torch.zeros((Lc, cfg.hidden), device=cuda)
    t = torch.full((1,), 1000.0, device=cuda)
    full = model.velocity(z, zero, cam, t, compress=False, selected_final=False)
    comp = model.velocity(z, zero, cam, t, compress=True, selected_final=True)
    for name, f, c in zip(("latent", "camera"), full, comp):
        d = (c - f).double()
        rel = float(d.square().mean().sqrt()) / float(f.double().square().mean().sqrt())
        print({"Lc": Lc, "rows": name, "rel_rmse": rel, "max_abs": float(d.abs().max())})
        assert rel <= 2e-6


def test_reduced_step_matches_cpu_full_computation(oracle, cuda):
    import torch
    from flow_ref import CpuJointFlow, combined_rmse

    cfg, model = _model(cuda, hidden=128, heads=2, blocks=2, L=150, Lc=48)
    z, c, cam = _inputs(cfg)
    dev = model.euler_cfg_step(*(torch.from_numpy(a).to(cuda) for a in (z, c, cam)), reduce_work=True)
    torch.cuda.synchronize(cuda)
    zn_d, v_d, cn_d, vc_d = (a.cpu().numpy() for a in dev)
    cpu = CpuJointFlow(model.host(), cfg, backend="oracle")
    zn_c, v_c, cn_c, vc_c = cpu.joint_euler_cfg_step(z, c, cam)
    latent_rmse, camera_rmse = combined_rmse(zn_d, zn_c), combined_rmse(cn_d, cn_c)
    v_rel = combined_rmse(v_d, v_c) / float(np.sqrt(np.mean(v_c.astype(np.float64) ** 2)))
    vc_rel = combined_rmse(vc_d, vc_c) / float(np.sqrt(np.mean(vc_c.astype(np.float64) ** 2)))
    print({"latent_rmse": latent_rmse, "camera_rmse": camera_rmse, "velocity_rel_rmse": v_rel,
           "camera_velocity_rel_rmse": vc_rel})
    assert np.all(np.isfinite(zn_d)) and np.all(np.isfinite(cn_d))
    assert cn_d.shape == (1, cfg.cam_channels)
    assert latent_rmse <= 1e-4 and camera_rmse <= 1e-4
    assert v_rel <= 1e-4 and vc_rel <= 1e-4


def test_reduced_step_opt_in_bf16x3_attention(oracle, cuda):
    """The single-stream graph with bf16x3 products in its block Linears and
    in every SDPA (key-bias self attention, the packed selected-rows final
    block) stays within the latent gate against the CPU fp32 full
    computation, differs from the strict step, and the strict step is
    restored bit for bit afterwards."""
    import torch
    from flow_ref import CpuJointFlow, combined_rmse

    cfg, model = _model(cuda, hidden=128, heads=2, blocks=2, L=150, Lc=48)
    z, c, cam = _inputs(cfg)
    args = [torch.from_numpy(a).to(cuda) for a in (z, c, cam)]
    strict = model.euler_cfg_step(*args, reduce_work=True)
    model.set_precision("bf16x3", include=("blocks", "attention"))
    assert model.attention_precision == "bf16x3"
    zn3, _, cn3, _ = model.euler_cfg_step(*args, reduce_work=True)
    model.set_precision("fp32")
    again = model.euler_cfg_step(*args, reduce_work=True)
    torch.cuda.synchronize(cuda)
    assert all(torch.equal(a, b) for a, b in zip(again, strict))
    assert not torch.equal(zn3, strict[0])
    zn_c, _, cn_c, _ = CpuJointFlow(model.host(), cfg, backend="oracle").joint_euler_cfg_step(z, c, cam)
    latent_rmse = combined_rmse(zn3.cpu().numpy(), zn_c)
    camera_rmse = combined_rmse(cn3.cpu().numpy(), cn_c)
    print({"bf16x3_latent_rmse": latent_rmse, "bf16x3_camera_rmse": camera_rmse})
    assert np.all(np.isfinite(zn3.cpu().numpy()))
    assert latent_rmse <= 1e-4 and camera_rmse <= 1e-4
