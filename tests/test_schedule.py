"""The sampler schedule both flow graphs use, pinned to closed-form values.

scripts/triposplat_quantized_sampler.py:398-400 builds
t = s u / (1 + (s - 1) u), u = linspace(1, 0, K + 1) in float64, and passes
float32(t_i * 1000) and float32(t_i - t_{i+1}) to the model and the Euler
update (:413-414).  With shift s = 3 this is t_i = 3 (K - i) / (3K - 2i):
for K = 20, t_1 = 57/58 and t_10 = 3/4, so step 0 has dt = 1/58; the
one-step s1 schedule has t = (1, 0), dt = 1.
"""
from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "triposplat-cpu-avx512_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def _closed(K, i):
    return 3.0 * (K - i) / (3.0 * K - 2.0 * i)


def test_schedule_closed_form_and_literals():
    from flow_ref import CpuFlow
    from tsplat.flow import FlowConfig, FlowModel

    for K in (20, 1, 4):
        cfg = FlowConfig(steps=K)
        cpu = CpuFlow(None, cfg, backend="oracle")
        host = cpu.schedule()
        dev = FlowModel.schedule(SimpleNamespace(cfg=cfg))    # the device graph's own schedule code
        want = np.array([_closed(K, i) for i in range(K + 1)])
        assert np.max(np.abs(host - want)) <= 4e-16
        assert np.max(np.abs(np.array(dev) - want)) <= 4e-16
        for i in range(K):
            t1000, dt = cpu.step_times(i)
            # what both graphs hand to the model and the Euler update, bit for bit
            assert t1000 == np.float32(dev[i] * 1000.0) and dt == np.float32(dev[i] - dev[i + 1])
    t = CpuFlow(None, FlowConfig(steps=20), backend="oracle").schedule()
    assert t[0] == 1.0 and t[20] == 0.0 and t[10] == 0.75
    assert abs(t[1] - 57.0 / 58.0) <= 4e-16 and abs(t[1] - 0.98275862068965517) <= 4e-16
    t1000, dt = CpuFlow(None, FlowConfig(steps=20), backend="oracle").step_times(0)
    assert t1000 == np.float32(1000.0) and dt == np.float32(1.0 / 58.0)
    t1000, dt = CpuFlow(None, FlowConfig(steps=1), backend="oracle").step_times(0)
    assert t1000 == np.float32(1000.0) and dt == np.float32(1.0)


def test_latent_stats_restate_compare_latent_npz():
    """latent_stats / combined_rmse_from_key_mse against hand-computed values
    (compare_latent_npz.py:22-48, 67-71), including the NaN / Inf counts."""
    from flow_ref import combined_rmse_from_key_mse, latent_stats, non_finite

    ref = np.array([1.0, -2.0, 0.0, 4.0], np.float32)
    cand = np.array([1.5, -2.0, 1e-9, 3.0], np.float32)
    st = latent_stats(ref, cand)
    d = np.array([0.5, 0.0, float(np.float32(1e-9)), -1.0])
    assert np.isclose(st["mse"], np.mean(d * d)) and np.isclose(st["rmse"], np.sqrt(np.mean(d * d)))
    assert np.isclose(st["mae"], np.mean(np.abs(d))) and st["max_abs"] == 1.0
    rel = np.abs(d) / np.maximum(np.abs(ref.astype(np.float64)), 1e-8)
    assert np.isclose(st["mean_relative_abs"], rel.mean())
    assert np.isclose(st["p50_abs"], np.percentile(np.abs(d), 50))
    assert st["finite_count"] == 4 and non_finite(st) == 0
    bad = latent_stats(ref, np.array([np.nan, np.inf, -np.inf, 4.0], np.float32))
    assert (bad["nan_count"], bad["posinf_count"], bad["neginf_count"], bad["finite_count"]) == (1, 1, 1, 1)
    assert non_finite(bad) == 3
    a, b = latent_stats(ref, cand), latent_stats(ref[:2], ref[:2] + 1)
    assert np.isclose(combined_rmse_from_key_mse({"latent": a, "camera": b}), np.sqrt((a["mse"] + b["mse"]) / 2))
