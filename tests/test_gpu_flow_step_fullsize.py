"""BASELINE configs[4] at its stated size in the driver's GPU run: the whole
28-block CFG Euler step (hidden 1024, 16 x 64 heads, MLP 4096, 16384 latent
+ 2048 condition tokens, CFG batch 2, guidance 3, shift 3) on the device,
checked stage by stage against the reference's own AVX-512 kernels
(oracle/_ref through oracle/flow_ref.py's CpuFlow, backend "reference") on
the same packed weights:

* blocks 0, 13 and 27 are recomputed on the host from the device's own input
  to each of them (both CFG branches) and compared with the device's output
  of that block;
* the final layer, the CFG combine and the Euler update are recomputed from
  the device's hidden state after block 27; the velocity is compared (its
  error does not depend on dt) and the next latent of two schedules: step 0
  of K = 20 (dt = 1 - t_1 = 1/58) and the one-step s1 schedule (dt = 1),
  where the latent gate bounds the velocity error itself;
* the statistics are those of scripts/compare_latent_npz.py:22-48 (RMSE,
  max-abs, MAE, percentiles, NaN / Inf counts); the gates are the north
  star's latent RMSE <= 1e-4 and no NaN / Inf (the reference's promotion
  gates, docs/triposplat_p3_bounded_approx_audit_20260722_ja.md:7).

The step is run once more without the observer and must give the same bytes
(the observer only copies).  The whole 28-block chain against the host's
full step is reported by bench.py (flow.config4_step.cpu_reference_full_step).
"""
from __future__ import annotations

import os
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CHECKED_BLOCKS = (0, 13, 27)


@pytest.mark.timeout(600)
def test_config4_step_stagewise_against_reference_build(oracle, cuda):
    import torch
    from flow_ref import CpuFlow, latent_stats, non_finite
    from tsplat.flow import FlowConfig, FlowModel

    if not oracle.ref_available():
        pytest.skip("oracle/_ref (the reference's AVX-512 build) is absent or the host lacks AVX-512")
    cfg = FlowConfig()
    L, Lc, C, nb = cfg.latent_tokens, cfg.cond_tokens, cfg.hidden, cfg.blocks
    print(f"configs[4] step: {nb} blocks, L={L} Lc={Lc} C={C}, CFG batch 2", flush=True)
    model = FlowModel(cfg, cuda)
    z_h = np.random.default_rng(20).standard_normal((L, C), dtype=np.float32)
    c_h = np.random.default_rng(21).standard_normal((Lc, C), dtype=np.float32)
    z, c = torch.from_numpy(z_h).to(cuda), torch.from_numpy(c_h).to(cuda)

    keep_at = set(CHECKED_BLOCKS) | {i + 1 for i in CHECKED_BLOCKS}
    kept = {}

    def observe(i, x):
        if i in keep_at:
            kept[i] = x.cpu().numpy()          # synchronous copy: the next block updates x in place

    zn, v = model.euler_cfg_step(z, c, step=0, observe=observe)
    zn_again, v_again = model.euler_cfg_step(z, c, step=0)
    z1 = z[None].clone()                        # the s1 schedule's step: dt = 1 on the same velocity
    model.sampler.euler_update_inplace({"x": z1}, {"x": v[None].contiguous()},
                                       torch.ones(1, dtype=torch.float32, device=cuda))
    torch.cuda.synchronize(cuda)
    assert torch.equal(zn, zn_again) and torch.equal(v, v_again)
    assert sorted(kept) == sorted(keep_at)
    zn, v, z1 = zn.cpu().numpy(), v.cpu().numpy(), z1[0].cpu().numpy()

    threads = len(os.sched_getaffinity(0))
    cpu = CpuFlow(model.host(), cfg, backend="reference", threads=threads)
    del model
    t1000, dt = cpu.step_times(0)
    assert t1000 == np.float32(1000.0) and abs(float(dt) - 1.0 / 58.0) < 1e-8
    t_emb, t_mod = cpu.timestep(np.full(2, t1000, np.float32))
    cc = np.ascontiguousarray(np.stack((c_h, np.zeros_like(c_h))))
    report = {}
    t0 = time.perf_counter()
    for i in CHECKED_BLOCKS:
        want = cpu.block(cpu.p["blocks"][i], kept[i], cc, np.ascontiguousarray(t_mod, np.float32))
        st = latent_stats(want, kept[i + 1])
        rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        report[f"block{i}"] = {"rel_rmse": st["rmse"] / rms, "max_abs": st["max_abs"],
                               "non_finite": non_finite(st)}
        print(f"block {i}: {report[f'block{i}']} ({time.perf_counter() - t0:.0f} s)", flush=True)
    v_both = cpu.final_layer(kept[nb], t_emb)
    zn_c, v_c = cpu.cfg_euler(v_both[0], v_both[1], z_h, dt)
    z1_c, _ = cpu.cfg_euler(v_both[0], v_both[1], z_h, np.float32(1.0))
    sv, sz, s1 = latent_stats(v_c, v), latent_stats(zn_c, zn), latent_stats(z1_c, z1)
    v_rms = float(np.sqrt(np.mean(v_c.astype(np.float64) ** 2)))
    report["velocity"] = {"rel_rmse": sv["rmse"] / v_rms, "max_abs": sv["max_abs"], "p99_abs": sv["p99_abs"]}
    report["latent_k20_step0"] = {"rmse": sz["rmse"], "max_abs": sz["max_abs"]}
    report["latent_s1"] = {"rmse": s1["rmse"], "max_abs": s1["max_abs"], "mae": s1["mae"]}
    print(report, flush=True)

    for i in CHECKED_BLOCKS:
        r = report[f"block{i}"]
        assert r["non_finite"] == 0
        assert r["rel_rmse"] <= 2e-6, (i, r)    # the full-size single-block test's bound
    for st in (sv, sz, s1):
        assert non_finite(st) == 0 and st["finite_count"] == L * C
    assert report["velocity"]["rel_rmse"] <= 1e-5
    assert sz["rmse"] <= 1e-4 and s1["rmse"] <= 1e-4
