"""The north-star accuracy gate at full size, in the driver's GPU run.

One configs[3] flow block at its stated size -- hidden 1024, 16 x 64 heads,
MLP 4096, L = 16384 latent + 2048 condition tokens -- on both CFG branches
(the condition and the zero condition, batch 2), computed on the device and
by the reference's own AVX-512 kernels (oracle/_ref, compiled from the
reference sources: NF24 GEMM, QKV-direct, exact SDPA, LayerNorm, modulate,
gated residual, GELU, RMSNorm) on the same packed weights, inputs and
timestep modulation.  Metric: scripts/compare_latent_npz.py:22-71 (RMSE of
the difference) plus max-abs, relative to the output's RMS.

The whole 28-block CFG Euler step is the same graph repeated: it is checked
stage by stage at full size by tests/test_gpu_flow_step_fullsize.py, gated
end to end at reduced sizes by tests/test_gpu_flow.py, and compared end to
end at full size against this CPU path by bench.py
(flow.config4_step.cpu_reference_full_step).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_full_size_block_matches_reference_build(oracle, cuda):
    import os
    import time

    import torch
    from flow_ref import CpuFlow, combined_rmse
    from tsplat.flow import FlowConfig, FlowModel

    if not oracle.ref_available():
        pytest.skip("oracle/_ref (the reference's AVX-512 build) is absent or the host lacks AVX-512")
    cfg = FlowConfig(blocks=1)
    L, Lc, C = cfg.latent_tokens, cfg.cond_tokens, cfg.hidden
    print(f"full-size block L={L} Lc={Lc} C={C}, CFG batch 2", flush=True)
    model = FlowModel(cfg, cuda)
    z = np.random.default_rng(20).standard_normal((L, C), dtype=np.float32)
    c = np.random.default_rng(21).standard_normal((Lc, C), dtype=np.float32)
    xx = np.ascontiguousarray(np.stack((z, z)))
    cc = np.ascontiguousarray(np.stack((c, np.zeros_like(c))))
    params = model.host()
    cpu = CpuFlow(params, cfg, backend="reference", threads=len(os.sched_getaffinity(0)))
    t_h = np.full(2, cpu.schedule()[0] * 1000.0, np.float32)
    _, tm = cpu.timestep(t_h)
    tm = np.ascontiguousarray(tm, np.float32)

    got = model.block_forward(model.blocks[0], torch.from_numpy(xx).to(cuda), torch.from_numpy(cc).to(cuda),
                              torch.from_numpy(tm).to(cuda))
    torch.cuda.synchronize(cuda)
    got = got.cpu().numpy()
    t0 = time.perf_counter()
    want = cpu.block(params["blocks"][0], xx.copy(), cc, tm)
    cpu_s = time.perf_counter() - t0
    assert np.all(np.isfinite(got))
    rmse = combined_rmse(got, want)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    max_abs = float(np.abs(got.astype(np.float64) - want).max())
    print({"block_rmse": rmse, "rel_rmse": rmse / rms, "max_abs": max_abs, "rms": rms,
           "cpu_reference_s": round(cpu_s, 2)}, flush=True)
    assert rmse <= 1e-4                 # the north star's latent gate, applied to one block's output
    assert rmse / rms <= 2e-6           # the reduced-size block test's relative bound
    assert max_abs <= 1e-4 * max(1.0, float(np.abs(want).max()))
