#!/usr/bin/env python3
"""Benchmark of the MI355X NF24 GEMM + exact SDPA path (one GPU).

Headline workload (benchmark configs[1]): exact dense self-attention SDPA,
B=1, H=16, head dim 64, Lq = Lk = 16384, q/k RoPE (theta 10000) + RMSNorm
applied, v ~ N(0,1), scale 1/8, no mask.  One step = one SDPA call on inputs
already resident in HBM.  value = 4*B*H*Lq*Lk*64 FLOP / step time (TFLOP/s).

Also measured in the same run (extra keys): configs[0], the NF24 GEMM
4096x1024 @ 1024x3072 (QKV shape) with W ~ N(0, 0.02) packed by the device
packer.

roofline: the SDPA kernel's average duration from HIP events on the stream it
is launched on (torch's current stream), FLOPs per launch as above, against
MI355X dense fp32 MFMA peak 157.3 TFLOP/s.  traffic: HBM bytes per launch
from the committed rocprofv3 PMC summary (profiles/), or null.

cpu_baseline: the reference's own AVX-512 kernel (oracle/_ref, compiled from
the reference sources) on the host cores, on a bounded sample of the same
workload (all 16 heads, a subset of query rows against all 16384 keys),
scaled to TFLOP/s.  Falls back to the oracle port if _ref is absent.
Each timed CPU run follows a device call (alternating order), with all host
threads and with the reference's published thread counts (SDPA 4, GEMM 8).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "triposplat-cpu-avx512_amd"))
# Host threads for the CPU baselines, taken before anything starts an OpenMP
# runtime.  (Binding OpenMP threads with OMP_PROC_BIND=true pins the main
# thread to one core, after which its affinity mask -- and any thread count
# read from it -- is a single CPU; the baselines therefore leave binding to
# the environment and report it.)
HOST_THREADS = len(os.sched_getaffinity(0))
# Input seeds of every workload (configs/workloads.json describes the inputs).
SEEDS = json.loads((ROOT / "configs" / "workloads.json").read_text())["seeds"]


def omp_binding():
    return {k: os.environ.get(k) for k in ("OMP_PROC_BIND", "OMP_PLACES", "OMP_NUM_THREADS")}

METRIC = "NF24 GEMM + exact SDPA TFLOP/s (% MFMA peak) at L=16384; s/denoise step"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
PEAK_BF16_MFMA = 2500.0  # TFLOP/s, MI355X dense bf16 matrix
PEAK_HBM = 8000.0       # GB/s
# host seconds the configs[4] CPU reference step may take (projected from its
# first block); beyond it the bench reports the projection instead
FLOW_CPU_BUDGET_S = 480.0


def rope_rmsnorm_host(x, theta=10000.0):
    import numpy as np

    L = x.shape[2]
    i = np.arange(32, dtype=np.float64)
    ang = np.arange(L, dtype=np.float64)[:, None] * theta ** (-2.0 * i / 64.0)[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x64 = x.astype(np.float64)
    re, im = x64[..., 0::2], x64[..., 1::2]
    y = np.empty_like(x64)
    y[..., 0::2] = re * c - im * s
    y[..., 1::2] = re * s + im * c
    y *= 8.0 / np.linalg.norm(y, axis=-1, keepdims=True)
    return y.astype(np.float32)


def host_cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the CPU baselines."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def host_cpu_topology():
    """lscpu's description of the host the CPU baselines ran on: model, family
    / model / stepping, sockets, cores, threads per core, NUMA nodes, L3, the
    CPUs this process may use and whether AVX-512 F/BW/DQ/VL (what the
    reference build is compiled for) are present."""
    import subprocess

    keys = {"Model name": "model", "CPU family": "family", "Model": "model_id", "Stepping": "stepping",
            "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "NUMA node(s)": "numa_nodes",
            "L3 cache": "l3", "CPU(s)": "cpus", "Hypervisor vendor": "hypervisor"}
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    flags = ""
    for line in out.splitlines():
        k, _, v = line.partition(":")
        k, v = k.strip(), v.strip()
        if k in keys:
            info[keys[k]] = v
        elif k == "Flags":
            flags = v
    info["usable_cpus"] = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    info["avx512_f_bw_dq_vl"] = all(f in flags.split() for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl"))
    return info


def warm_up(torch, fn, seconds=0.05):
    """Call fn until `seconds` of device work have run: after the host-side
    reference runs the GPU sits idle and its clock ramps up again over the
    first milliseconds, which a short call would otherwise be timed in."""
    t0 = time.perf_counter()
    n = 0
    while n < 2 or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_events(torch, fn, iters):
    """Average device duration of fn() (ms) from events on the current stream."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def load_traffic(name):
    p = ROOT / "profiles" / f"{name}.json"
    if p.is_file():
        try:
            return json.loads(p.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def parity_stats(got, ref, tol_abs=None):
    """max-abs / relative error of a device result against the reference's
    output on the same inputs (float64 arithmetic)."""
    import numpy as np

    d = got.astype(np.float64) - ref.astype(np.float64)
    max_abs = float(np.abs(d).max())
    rms_ref = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    out = {"max_abs": max_abs, "max_rel": max_abs / float(np.abs(ref).max()),
           "rmse": float(np.sqrt(np.mean(d * d))), "rel_rmse": float(np.sqrt(np.mean(d * d))) / rms_ref}
    if tol_abs is not None:
        out.update({"tolerance_max_abs": tol_abs, "within_tolerance": bool(max_abs <= tol_abs)})
    return out


def cpu_baseline_sdpa(q, k, v, budget_s=12.0, gpu_out=None, gpu_fn=None):
    """Time the reference AVX-512 SDPA (or the oracle port) on the host.

    The sample is the whole configs[1] call when it fits the budget (it does
    on a 16-core host: ~1.5 s), else the first `rows` query rows of every
    head against all keys.  Median of 3 after one warmup, with all host
    threads; a second figure uses the reference's published SDPA thread
    count (4).  With `gpu_out` (the device result, [B, L, H, D]) and the
    reference build present, the sampled rows of the reference's own output
    are also compared with it (`parity_vs_reference`; the GPU tests' bound
    is 1e-5 * max|v| max-abs).  With `gpu_fn` (one timed device call, ms)
    each timed CPU run follows a device call, so both sides see the same
    host and clock state (`alternating_gpu_ms`)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    threads = HOST_THREADS
    kind = "reference" if O.ref_available() else "port"
    B, H, L, D = q.shape

    last = {}

    def run(rows, nthreads):
        qs = np.ascontiguousarray(q[:, :, :rows])
        t0 = time.perf_counter()
        if kind == "reference":
            last[rows] = O.ref_sdpa_q8t512(qs, k, v, None, nthreads)
        else:
            O.sdpa_q8t512(qs, k, v)
        return time.perf_counter() - t0

    gpu_ms = []

    def measure(nthreads):
        run(256, nthreads)  # warmup: K/V pack workspace, page-in, thread pool
        t1 = run(1024, nthreads)
        rows = L if t1 * L / 1024 * 3 <= budget_s else max(1024, int(budget_s / 3 / t1 * 1024) // 128 * 128)
        times = []
        for _ in range(3):  # device call, CPU run, alternating
            if gpu_fn is not None:
                gpu_ms.append(gpu_fn())
            times.append(run(rows, nthreads))
        return rows, sorted(times)[1]

    rows, t_med = measure(threads)
    parity = None
    if gpu_out is not None and rows in last:
        got = np.ascontiguousarray(gpu_out[:, :rows].transpose(0, 2, 1, 3))
        parity = parity_stats(got, last[rows], tol_abs=1e-5 * float(np.abs(v).max()))
        parity["rows"] = f"{rows} of {L} query rows, all heads"
    flop = 4.0 * B * H * rows * L * D
    rows4, t4 = measure(4)
    flop4 = 4.0 * B * H * rows4 * L * D
    return {
        "value": flop / t_med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "host_cpu": host_cpu_model(),
        "host_lscpu": host_cpu_topology(),
        "kind": kind,
        "sample": f"exact SDPA q8t512 (reference AVX-512 build), B=1 H=16 D=64, {rows} of {L} query rows "
                  f"vs all {L} keys; median of 3 = {t_med:.3f} s; {threads} OpenMP threads",
        "seconds_per_call": t_med * L / rows,
        "threads4_tflops": flop4 / t4 / 1e12,
        "threads4_seconds_per_call": t4 * L / rows4,
        "order": "device call then CPU run, three times per thread count (median of the CPU runs)",
        "alternating_gpu_ms": gpu_ms,
        "omp": omp_binding(),
        "parity_vs_reference": parity,
    }


def sdpa_inputs(torch, dev):
    import numpy as np

    B, H, L, D = 1, 16, 16384, 64
    q_h = rope_rmsnorm_host(np.random.default_rng(SEEDS["c2_q"]).standard_normal((B, H, L, D), dtype=np.float32))
    k_h = rope_rmsnorm_host(np.random.default_rng(SEEDS["c2_k"]).standard_normal((B, H, L, D), dtype=np.float32))
    v_h = np.random.default_rng(SEEDS["c2_v"]).standard_normal((B, H, L, D), dtype=np.float32)
    return q_h, k_h, v_h


def run_sdpa(torch, dev, steps, warmup, host, precision="fp32", keep_out=False):
    """one exact SDPA call per step; returns (wall s/step, kernel
    ms, the output on the host if keep_out else None).
    precision: the product precision (the headline is "fp32"; the opt-in
    modes are timed this way only for `--only sdpa --precision ...` profiles)."""
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    q_h, k_h, v_h = host
    B, H, L, D = q_h.shape
    q = torch.from_numpy(q_h).to(dev)
    k = torch.from_numpy(k_h).to(dev)
    v = torch.from_numpy(v_h).to(dev)
    out = torch.empty((B, L, H, D), dtype=torch.float32, device=dev)

    def step():
        native_sdpa_f32_ex(q, k, v, out=out, out_layout="blhd", precision=precision)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    kernel_ms = time_events(torch, step, max(3, steps))
    assert torch.isfinite(out).all().item()
    return wall, kernel_ms, (out.cpu().numpy() if keep_out else None)


def run_sdpa_opt_in(torch, dev, host, fp32_ms, iters=5):
    """configs[1] with the opt-in bf16-MFMA SDPA products: time, the
    equivalent rate (the same 4*B*H*L^2*64 algorithmic FLOP), the MFMA work
    against the bf16 peak (three products per term for bf16x3), and the
    error against the strict fp32 output."""
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    q_h, k_h, v_h = host
    B, H, L, D = q_h.shape
    q, k, v = (torch.from_numpy(a).to(dev) for a in (q_h, k_h, v_h))
    flop = 4.0 * B * H * L * L * D
    strict = native_sdpa_f32_ex(q, k, v)
    out = torch.empty_like(strict)
    res = {}
    for precision, terms in (("bf16", 1), ("bf16x3", 3)):
        def step(p=precision):
            native_sdpa_f32_ex(q, k, v, out=out, precision=p)

        warm_up(torch, step)
        ms = sorted(time_events(torch, step, iters) for _ in range(3))[1]
        d = out.double() - strict.double()
        res[precision] = {
            "ms": ms, "tflops_equiv": flop / (ms * 1e-3) / 1e12,
            "frac_bf16_mfma_peak": terms * flop / (ms * 1e-3) / 1e12 / PEAK_BF16_MFMA,
            "speedup_vs_fp32": fp32_ms / ms,
            "rel_rmse_vs_fp32": float(d.pow(2).mean().sqrt() / strict.double().pow(2).mean().sqrt()),
            "max_abs_vs_fp32": float(d.abs().max()),
        }
    del strict, out
    return res


def run_sdpa_variants(torch, dev, host, iters=5, ref_parity=False):
    """key-bias self attention (per-head bias [16, 16384] ~ U(-2, 0),
    and the reference-faithful shared [Lk] bias with log(2048) on one key),
    and cross attention (16384 queries vs 2048 condition keys, k/v ~ N(0,1)).
    With ref_parity and the reference build present, each output is compared
    with the reference's AVX-512 SDPA on the same inputs (its kernel takes a
    shared [Lk] bias, so the per-head case runs it once per head)."""
    import numpy as np
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

    q_h, k_h, v_h = host
    B, H, L, D = q_h.shape
    q = torch.from_numpy(q_h).to(dev)
    k = torch.from_numpy(k_h).to(dev)
    v = torch.from_numpy(v_h).to(dev)
    out = torch.empty((B, L, H, D), dtype=torch.float32, device=dev)
    bias_h = np.random.default_rng(SEEDS["c3_key_bias"]).uniform(-2.0, 0.0, (H, L)).astype(np.float32)
    bias = torch.from_numpy(bias_h).to(dev)
    shared = torch.zeros(L, dtype=torch.float32, device=dev)
    shared[4096] = math.log(2048.0)
    Lc = 2048
    kc = torch.from_numpy(np.random.default_rng(SEEDS["c3_cross_k"]).standard_normal((B, H, Lc, D), dtype=np.float32)).to(dev)
    vc = torch.from_numpy(np.random.default_rng(SEEDS["c3_cross_v"]).standard_normal((B, H, Lc, D), dtype=np.float32)).to(dev)
    O = None
    if ref_parity:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        if not O.ref_available():
            O = None
    threads = HOST_THREADS

    def ref_per_head():
        return np.concatenate([O.ref_sdpa_q8t512(q_h[:, h:h + 1], k_h[:, h:h + 1], v_h[:, h:h + 1], bias_h[h],
                                                 threads) for h in range(H)], axis=1)

    res = {}
    for name, fn, flop, ref_fn, v_max in (
        ("keybias_per_head", lambda: native_sdpa_f32_ex(q, k, v, key_bias_per_head=bias, out=out, out_layout="blhd"),
         4.0 * B * H * L * L * D, ref_per_head, float(np.abs(v_h).max())),
        ("keybias_shared_log2048", lambda: native_sdpa_f32_ex(q, k, v, key_bias=shared, out=out, out_layout="blhd"),
         4.0 * B * H * L * L * D,
         lambda: O.ref_sdpa_q8t512(q_h, k_h, v_h, shared.cpu().numpy(), threads), float(np.abs(v_h).max())),
        ("cross_16384x2048", lambda: native_sdpa_f32_ex(q, kc, vc, out=out, out_layout="blhd"),
         4.0 * B * H * L * Lc * D,
         lambda: O.ref_sdpa_q8t512(q_h, kc.cpu().numpy(), vc.cpu().numpy(), None, threads),
         float(vc.abs().max())),
    ):
        warm_up(torch, fn)
        ms = sorted(time_events(torch, fn, iters) for _ in range(3))[1]
        tf = flop / (ms * 1e-3) / 1e12
        res[name] = {"ms": ms, "tflops": tf, "frac_fp32_mfma_peak": tf / PEAK_FP32_MFMA}
        if O is not None:
            fn()
            got = np.ascontiguousarray(out.cpu().numpy().transpose(0, 2, 1, 3))
            res[name]["parity_vs_reference"] = parity_stats(got, ref_fn(), tol_abs=1e-5 * v_max)
    return res


def run_gemm(torch, dev, iters, ref_parity=False):
    """NF24 Linear 4096x1024 @ 1024x3072 (+ bias).  With
    ref_parity and the reference build present, the device result is also
    compared with the reference's own AVX-512 NF24 GEMM on the same inputs
    (`parity_vs_reference`; the GPU tests bound each output by the fp32
    summation-order bound 2*gamma_(K+1)*sum|terms|)."""
    import numpy as np
    from tsplat.nf24 import bf16_planes, nf24_linear, quantize_nf24_i16_per_output_channel

    M, K, N = 4096, 1024, 3072
    x = torch.from_numpy(np.random.default_rng(SEEDS["c1_x"]).standard_normal((M, K), dtype=np.float32)).to(dev)
    w = torch.from_numpy((np.random.default_rng(SEEDS["c1_w"]).standard_normal((N, K), dtype=np.float32)
                          * np.float32(0.02)).astype(np.float32)).to(dev)
    bias = torch.from_numpy((np.random.default_rng(SEEDS["c1_bias"]).standard_normal(N, dtype=np.float32)
                             * np.float32(0.01)).astype(np.float32)).to(dev)
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    gout = torch.empty((M, N), dtype=torch.float32, device=dev)

    def step():
        nf24_linear(x, codes[0], codes[1], scales[0], bias, out=gout)

    # 0.5 s of warm-up calls: the clock settles over the first ~100 calls of a
    # 0.2 ms kernel (a 40-call warm-up left the timed batches 5-10 % slower)
    warm_up(torch, step, 0.5)
    # median of 5 batches: clocks on these boxes vary by ~10 % between batches
    g_ms = sorted(time_events(torch, step, iters) for _ in range(5))[2]
    g_flop = 2.0 * M * N * K
    g_tf = g_flop / (g_ms * 1e-3) / 1e12
    strict = gout.clone()
    opt_in = {}
    for precision in ("bf16", "bf16x3"):
        # the opt-in bf16-MFMA products, with their error against strict fp32
        def step_p(p=precision):
            nf24_linear(x, codes[0], codes[1], scales[0], bias, out=gout, precision=p)

        warm_up(torch, step_p, 0.5)
        p_ms = sorted(time_events(torch, step_p, iters) for _ in range(5))[2]
        d = (gout.double() - strict.double())
        p_tf = g_flop / (p_ms * 1e-3) / 1e12
        terms = 3 if precision == "bf16x3" else 1  # MFMA work per algorithmic FLOP
        decoded = gout.clone()
        # the same products with the weights' bf16 planes built once
        # (tsplat.nf24.bf16_planes): no decode in the K loop, same result
        planes = bf16_planes(codes[0], codes[1], scales[0], precision)

        def step_planes(p=precision):
            nf24_linear(x, codes[0], codes[1], scales[0], bias, out=gout, precision=p, planes=planes)

        warm_up(torch, step_planes, 0.5)
        pl_ms = sorted(time_events(torch, step_planes, iters) for _ in range(5))[2]
        pl_tf = g_flop / (pl_ms * 1e-3) / 1e12
        opt_in[precision] = {
            "ms": p_ms, "tflops": p_tf, "frac_bf16_mfma_peak": terms * p_tf / PEAK_BF16_MFMA,
            "speedup_vs_fp32": g_ms / p_ms,
            "rmse_vs_fp32": float(d.pow(2).mean().sqrt()),
            "rel_rmse_vs_fp32": float(d.pow(2).mean().sqrt() / strict.double().pow(2).mean().sqrt()),
            "max_abs_vs_fp32": float(d.abs().max()),
            "planes_ms": pl_ms, "planes_frac_bf16_mfma_peak": terms * pl_tf / PEAK_BF16_MFMA,
            "planes_equal_decoded": bool(torch.equal(gout, decoded)),
        }
        del planes
    parity = cpu_ref = None
    if ref_parity:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        if O.ref_available():
            host = [t.cpu().numpy() for t in (x, codes[0], codes[1], scales[0], bias)]
            threads = HOST_THREADS
            ref = O.ref_nf24_gemm(*host, threads=threads)
            parity = parity_stats(strict.cpu().numpy(), ref)
            parity["rows"] = f"all {M} rows"
            # the reference kernel on the host: all cores and the reference's
            # published GEMM thread count (8); device batch and CPU call
            # alternate, median of 3 CPU calls after one warmup
            cpu_ref = {"host_cpu": host_cpu_model(), "omp": omp_binding(),
                       "order": "device batch then CPU call, three times per thread count"}
            for tag, nthr in (("", threads), ("threads8_", 8)):
                O.ref_nf24_gemm(*host, threads=nthr)
                times, gms = [], []
                for _ in range(3):
                    gms.append(time_events(torch, step, iters))
                    t0 = time.perf_counter()
                    O.ref_nf24_gemm(*host, threads=nthr)
                    times.append(time.perf_counter() - t0)
                t_med = sorted(times)[1]
                cpu_ref[tag + "threads"] = nthr
                cpu_ref[tag + "s_per_call"] = t_med
                cpu_ref[tag + "tflops"] = g_flop / t_med / 1e12
                cpu_ref[tag + "alternating_gpu_ms"] = gms
            cpu_ref["speedup_gpu_vs_cpu_threads8"] = cpu_ref["threads8_s_per_call"] / (g_ms * 1e-3)
    return {
        "workload": "configs[0] NF24 Linear X[4096x1024] @ W[1024x3072] + bias, fp32 MFMA accumulate",
        "ms": g_ms,
        "tflops": g_tf,
        "frac_fp32_mfma_peak": g_tf / PEAK_FP32_MFMA,
        "algorithmic_bytes": float(M * K * 4 + K * N * 3 + N * 8 + M * N * 4),
        "traffic": load_traffic("nf24_gemm_config0"),
        "opt_in_bf16": opt_in,
        "parity_vs_reference": parity,
        "cpu_reference": cpu_ref,
    }


def time_interleaved(torch, fns, iters, rounds=5):
    """Median per-call device time (ms) of each callable, timed in
    interleaved rounds (clocks drift between rounds on these boxes)."""
    warm_up(torch, lambda: [f() for f in fns.values()], 0.5)
    ts = {k: [] for k in fns}
    for _ in range(rounds):
        for k, f in fns.items():
            ts[k].append(time_events(torch, f, iters))
    return {k: sorted(v)[len(v) // 2] for k, v in ts.items()}


def packed_linear(torch, dev, K, N, seed):
    """A seeded NF24 Linear (W ~ N(0, 0.02), bias ~ N(0, 0.01)), packed on the device."""
    import numpy as np
    from tsplat.nf24 import quantize_nf24_i16_per_output_channel

    w = torch.from_numpy((np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32)
                          * np.float32(0.02)).astype(np.float32)).to(dev)
    b = torch.from_numpy((np.random.default_rng(seed + 1).standard_normal(N, dtype=np.float32)
                          * np.float32(0.01)).astype(np.float32)).to(dev)
    codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
    return codes[0], codes[1], scales[0], b


GEMM_L16384 = (("qkv", 1024, 3072), ("mlp_fc1", 1024, 4096), ("mlp_fc2", 4096, 1024), ("attn_out", 1024, 1024))


def run_gemm_l16384(torch, dev, iters=8):
    """The flow block's four NF24 Linear shapes at the metric's L = 16384 rows
    (strict fp32 MFMA, plain store), TFLOP/s and fraction of the fp32 peak."""
    import numpy as np
    from tsplat.nf24 import nf24_linear

    M = 16384
    res = {}
    fns, meta = {}, {}
    for i, (name, K, N) in enumerate(GEMM_L16384):
        x = torch.from_numpy(np.random.default_rng(SEEDS["l16384_gemm_x_base"] + i).standard_normal((M, K), dtype=np.float32)).to(dev)
        c01, q2, sc, b = packed_linear(torch, dev, K, N, SEEDS["l16384_gemm_w_base"] + 2 * i)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        fns[name] = (lambda x=x, c01=c01, q2=q2, sc=sc, b=b, out=out: nf24_linear(x, c01, q2, sc, b, out=out))
        meta[name] = (K, N)
    ms = time_interleaved(torch, fns, iters)
    for name, (K, N) in meta.items():
        tf = 2.0 * M * N * K / (ms[name] * 1e-3) / 1e12
        res[name] = {"M": M, "K": K, "N": N, "ms": ms[name], "tflops": tf, "frac_fp32_mfma_peak": tf / PEAK_FP32_MFMA}
    return res


# The reference's own published timings of this path (AMD EPYC 9654, 4 CPUs;
# seconds per call, GCC 9 build / GCC 13 -march=znver4 build):
# docs/triposplat_cpu_p0_p1_validation_20260722_ja.md:43-46 (SDPA),
# :99-104 (GEMM, GCC 9) and docs/triposplat_high_memory_native_f32_audit_20260723_ja.md:66-71
# (GEMM, GCC 13).
PUBLISHED_S = {
    "sdpa_L12294_dense": (2.597, 2.006),
    "sdpa_L8194_keybias_log4101": (0.993, 0.841),
    "gemm_12294x1024x3072_qkv": (0.302, 0.332),
    "gemm_12294x1024x4096_fc1": (0.498, 0.371),
    "gemm_12294x4096x1024_fc2": (0.539, 0.418),
    "gemm_12294x1024x1024_out": (0.121, 0.075),
}


def run_reference_shapes(torch, dev, with_cpu, iters=5):
    """The reference's real TripoSplat sequence shapes on the device, with the
    reference's AVX-512 build timed beside them on the host at its published
    thread count (4), and each device output compared with the reference's
    on the rows the CPU computed:
      * SDPA L = 12294 dense (the positive CFG branch, attention_patch:5357-5363);
      * SDPA L = 8194 with the compressed negative branch's key bias (log 4101
        on the single condition key, attention_patch:5468-5475, 5618-5628);
      * SDPA 8193 selected latent queries x 12294 keys (the final block);
      * the block's four NF24 GEMMs at M = 12294.
    The CPU SDPA runs on the first 2048 query rows of every head (rows are
    independent) and is scaled to the whole call; the CPU GEMMs run in full."""
    import numpy as np
    from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex
    from tsplat.nf24 import nf24_linear

    O = None
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        if not O.ref_available():
            O = None
    threads = 4
    H, D = 16, 64
    res = {}
    for name, Lq, Lk, logm in (("sdpa_L12294_dense", 12294, 12294, False),
                               ("sdpa_L8194_keybias_log4101", 8194, 8194, True),
                               ("sdpa_selected_8193x12294", 8193, 12294, False)):
        q_h = rope_rmsnorm_host(np.random.default_rng(SEEDS["refshapes_q"]).standard_normal((1, H, Lq, D), dtype=np.float32))
        k_h = rope_rmsnorm_host(np.random.default_rng(SEEDS["refshapes_k"]).standard_normal((1, H, Lk, D), dtype=np.float32))
        v_h = np.random.default_rng(SEEDS["refshapes_v"]).standard_normal((1, H, Lk, D), dtype=np.float32)
        bias_h = None
        if logm:
            bias_h = np.zeros(Lk, np.float32)
            bias_h[Lk - 1] = np.float32(math.log(4101.0))
        q, k, v = (torch.from_numpy(a).to(dev) for a in (q_h, k_h, v_h))
        bias = None if bias_h is None else torch.from_numpy(bias_h).to(dev)
        out = torch.empty((1, H, Lq, D), dtype=torch.float32, device=dev)
        fn = lambda: native_sdpa_f32_ex(q, k, v, key_bias=bias, out=out)
        ms = time_interleaved(torch, {"x": fn}, iters)["x"]
        flop = 4.0 * H * Lq * Lk * D
        row = {"Lq": Lq, "Lk": Lk, "key_bias": "log(4101) on key Lk-1" if logm else None, "ms": ms,
               "tflops": flop / (ms * 1e-3) / 1e12, "frac_fp32_mfma_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA}
        if name in PUBLISHED_S:
            row["published_cpu_s_4cpu_gcc9_gcc13"] = PUBLISHED_S[name]
            row["speedup_vs_published_gcc13"] = PUBLISHED_S[name][1] / (ms * 1e-3)
        if O is not None:
            rows = 2048
            qs = np.ascontiguousarray(q_h[:, :, :rows])
            O.ref_sdpa_q8t512(qs[:, :, :256], k_h, v_h, bias_h, threads)
            times, ref = [], None
            for _ in range(3):
                t0 = time.perf_counter()
                ref = O.ref_sdpa_q8t512(qs, k_h, v_h, bias_h, threads)
                times.append(time.perf_counter() - t0)
            cpu_s = sorted(times)[1] * Lq / rows
            row["cpu_reference"] = {"threads": threads, "s_per_call": cpu_s, "sample": f"{rows} of {Lq} query rows, all heads",
                                    "speedup_gpu_vs_cpu": cpu_s / (ms * 1e-3)}
            fn()
            torch.cuda.synchronize()
            row["parity_vs_reference"] = parity_stats(out[:, :, :rows].cpu().numpy(), ref,
                                                      tol_abs=1e-5 * float(np.abs(v_h).max()))
        res[name] = row
        del q, k, v, out
    M = 12294
    for i, (tag, K, N) in enumerate((("qkv", 1024, 3072), ("fc1", 1024, 4096), ("fc2", 4096, 1024), ("out", 1024, 1024))):
        name = f"gemm_{M}x{K}x{N}_{tag}"
        x_h = np.random.default_rng(SEEDS["refshapes_gemm_x_base"] + i).standard_normal((M, K), dtype=np.float32)
        x = torch.from_numpy(x_h).to(dev)
        c01, q2, sc, b = packed_linear(torch, dev, K, N, SEEDS["refshapes_gemm_w_base"] + 2 * i)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        fn = lambda: nf24_linear(x, c01, q2, sc, b, out=out)
        ms = time_interleaved(torch, {"x": fn}, iters)["x"]
        flop = 2.0 * M * N * K
        row = {"M": M, "K": K, "N": N, "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12,
               "frac_fp32_mfma_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA,
               "published_cpu_s_4cpu_gcc9_gcc13": PUBLISHED_S[name],
               "speedup_vs_published_gcc13": PUBLISHED_S[name][1] / (ms * 1e-3)}
        if O is not None:
            ch, qh, sh, bh = (t.cpu().numpy() for t in (c01, q2, sc, b))
            O.ref_nf24_gemm(x_h[:256], ch, qh, sh, bh, threads)
            times, ref = [], None
            for _ in range(3):
                t0 = time.perf_counter()
                ref = O.ref_nf24_gemm(x_h, ch, qh, sh, bh, threads)
                times.append(time.perf_counter() - t0)
            cpu_s = sorted(times)[1]
            row["cpu_reference"] = {"threads": threads, "s_per_call": cpu_s, "sample": "the whole call",
                                    "speedup_gpu_vs_cpu": cpu_s / (ms * 1e-3)}
            fn()
            torch.cuda.synchronize()
            row["parity_vs_reference"] = parity_stats(out.cpu().numpy(), ref)
        res[name] = row
        del x, out
    return res


def flow_inputs(cfg):
    import numpy as np

    z = np.random.default_rng(SEEDS["flow_latent"]).standard_normal((cfg.latent_tokens, cfg.hidden), dtype=np.float32)
    c = np.random.default_rng(SEEDS["flow_condition"]).standard_normal((cfg.cond_tokens, cfg.hidden), dtype=np.float32)
    return z, c


def run_flow(torch, dev, steps, with_cpu, validate):
    """configs[3] (one block, one branch) and configs[4] (28 blocks, CFG pair,
    one Euler step) of the frozen synthetic flow graph (tsplat/flow.py)."""
    import numpy as np
    from tsplat.flow import FlowConfig, FlowModel

    cfg = FlowConfig()
    C, L, Lc = cfg.hidden, cfg.latent_tokens, cfg.cond_tokens
    t0 = time.perf_counter()
    model = FlowModel(cfg, dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    z_h, c_h = flow_inputs(cfg)
    z = torch.from_numpy(z_h).to(dev)
    c = torch.from_numpy(c_h).to(dev)

    # one block on one branch, t_mod from the step-0 timestep
    t_emb, t_mod = model.timestep(torch.full((1,), 1000.0, device=dev))
    # block_forward updates x in place: time it on a copy, not on z itself
    x1, c1 = z[None].clone(), c[None].contiguous()
    for _ in range(2):
        model.block_forward(model.blocks[0], x1, c1, t_mod)
    torch.cuda.synchronize()
    blk_ms = time_events(torch, lambda: model.block_forward(model.blocks[0], x1, c1, t_mod), 5)
    per_branch_flop = 2.0 * L * C * (3 * C + C + C + C + 4 * C + 4 * C) + 2.0 * Lc * C * 2 * C \
        + 4.0 * cfg.heads * L * L * 64 + 4.0 * cfg.heads * L * Lc * 64

    # one CFG Euler step over all 28 blocks
    for _ in range(1):
        model.euler_cfg_step(z, c)
    torch.cuda.synchronize()
    times = []
    for _ in range(max(1, steps)):
        t0 = time.perf_counter()
        zn, v = model.euler_cfg_step(z, c)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    step_s = sorted(times)[len(times) // 2]
    step_flop = 2 * cfg.blocks * per_branch_flop
    # opt-in: bf16x3 products in the block Linears, then also in the SDPA
    # (timestep / io Linears and everything else unchanged); latent RMSE
    # against the strict step
    def opt_in_step(include):
        model.set_precision("bf16x3", include=include)
        model.euler_cfg_step(z, c)
        torch.cuda.synchronize()
        times3 = []
        for _ in range(max(1, steps)):
            t0 = time.perf_counter()
            zn3, v3 = model.euler_cfg_step(z, c)
            torch.cuda.synchronize()
            times3.append(time.perf_counter() - t0)
        model.set_precision("fp32")
        step3_s = sorted(times3)[len(times3) // 2]
        return {
            "s_per_denoise_step": step3_s, "speedup_vs_fp32": step_s / step3_s,
            "latent_rmse_vs_fp32_step": float((zn3.double() - zn.double()).pow(2).mean().sqrt()),
            "velocity_rmse_vs_fp32_step": float((v3.double() - v.double()).pow(2).mean().sqrt()),
        }

    bf16x3_step = opt_in_step(("blocks",))
    bf16x3_attn_step = opt_in_step(("blocks", "attention"))
    out = {
        "config3_block": {"workload": "configs[3] one flow block, L=16384 latent + 2048 condition tokens, one branch",
                          "ms": blk_ms, "tflops": per_branch_flop / (blk_ms * 1e-3) / 1e12},
        "config4_step": {"workload": "configs[4] 28 blocks, CFG batch 2, one Euler step (guidance 3, shift 3)",
                         "s_per_denoise_step": step_s, "tflops": step_flop / step_s / 1e12,
                         "model_setup_s": setup_s, "finite": bool(torch.isfinite(zn).all().item()),
                         "opt_in_bf16x3_block_linears": bf16x3_step,
                         "opt_in_bf16x3_block_linears_and_attention": bf16x3_attn_step},
    }
    if with_cpu or validate:
        out["config4_step"]["cpu_reference_full_step"] = flow_step_vs_cpu(
            torch, dev, model, cfg, z_h, c_h, zn, v, step_s, out["config3_block"])
    del model
    out["joint"] = run_flow_joint(torch, dev, steps, with_cpu)
    return out


class _CpuBudget(Exception):
    pass


def flow_step_vs_cpu(torch, dev, model, cfg, z_h, c_h, zn, v, step_s, block_row):
    """configs[4]'s whole step on the host through the reference's own AVX-512
    kernels (oracle/_ref; the oracle port when that is absent): all 28 blocks
    on both CFG branches, the final layer, CFG and the Euler update, from the
    same packed weights and inputs.  Against it, the device step's velocity
    (relative RMSE: independent of dt), the next latent of step 0 of the K = 20
    schedule (dt = 1/58) and of the one-step s1 schedule (dt = 1), each with
    the statistics of scripts/compare_latent_npz.py:22-48 reduced to RMSE,
    max-abs, p99 and the NaN / Inf count; gates: latent RMSE <= 1e-4 and no
    NaN / Inf.  configs[3]'s block parity comes from the same run: the hidden
    state after block 0 on both sides.  The host step is abandoned (and only
    estimated from its first block) if that block projects it past
    FLOW_CPU_BUDGET_S."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from flow_ref import CpuFlow, latent_stats, non_finite

    backend = "reference" if O.ref_available() else "oracle"
    dev_after0 = {}
    model.euler_cfg_step(torch.from_numpy(z_h).to(dev), torch.from_numpy(c_h).to(dev), step=0,
                         observe=lambda i, x: dev_after0.setdefault(i, x.cpu().numpy()) if i == 1 else None)
    z1 = torch.from_numpy(z_h).to(dev)[None].clone()
    model.sampler.euler_update_inplace({"x": z1}, {"x": v[None].contiguous()},
                                       torch.ones(1, dtype=torch.float32, device=dev))
    z1 = z1[0].cpu().numpy()
    cpu = CpuFlow(model.host(), cfg, backend=backend, threads=HOST_THREADS)
    cpu_after0 = {}
    cpu.observe = lambda i, x: cpu_after0.setdefault(i, np.array(x, copy=True)) if i == 1 else None
    t0 = time.perf_counter()

    def progress(i):
        el = time.perf_counter() - t0
        if i == 0 and el * cfg.blocks > FLOW_CPU_BUDGET_S:
            raise _CpuBudget(el)
        if (i + 1) % 7 == 0:
            print(f"cpu configs[4] step: block {i + 1}/{cfg.blocks} ({el:.0f} s)", file=sys.stderr, flush=True)

    cpu.progress = progress
    res = {"kind": "reference" if backend == "reference" else "port", "cores": HOST_THREADS}
    t1000, dt = cpu.step_times(0)
    try:
        vb = cpu.velocity(np.stack((z_h, z_h)), np.stack((c_h, np.zeros_like(c_h))), np.full(2, t1000, np.float32))
    except _CpuBudget as e:
        res["s_per_denoise_step_estimated"] = float(e.args[0]) * cfg.blocks
        res["speedup_gpu_vs_cpu"] = res["s_per_denoise_step_estimated"] / step_s
        return res
    cpu_s = time.perf_counter() - t0
    zc, vc = cpu.cfg_euler(vb[0], vb[1], z_h, dt)
    z1c, _ = cpu.cfg_euler(vb[0], vb[1], z_h, np.float32(1.0))
    zn_h, v_h = zn.cpu().numpy(), v.cpu().numpy()
    sv, sz, s1 = latent_stats(vc, v_h), latent_stats(zc, zn_h), latent_stats(z1c, z1)
    vrms = float(np.sqrt(np.mean(vc.astype(np.float64) ** 2)))
    b0 = latent_stats(cpu_after0[1], dev_after0[1])
    b0rms = float(np.sqrt(np.mean(cpu_after0[1].astype(np.float64) ** 2)))
    block_row["parity_vs_reference"] = {"rmse": b0["rmse"], "rel_rmse": b0["rmse"] / b0rms,
                                        "max_abs": b0["max_abs"], "within_gate": bool(b0["rmse"] <= 1e-4)}
    res.update({
        "s_per_denoise_step": cpu_s, "speedup_gpu_vs_cpu": cpu_s / step_s,
        "velocity_rel_rmse": sv["rmse"] / vrms, "velocity_max_abs": sv["max_abs"],
        "latent_rmse_k20": sz["rmse"], "latent_max_abs_k20": sz["max_abs"], "latent_p99_abs_k20": sz["p99_abs"],
        "latent_rmse_s1": s1["rmse"], "latent_max_abs_s1": s1["max_abs"], "latent_p99_abs_s1": s1["p99_abs"],
        "nan_inf": non_finite(sv) + non_finite(sz) + non_finite(s1), "gate_rmse": 1e-4,
    })
    res["within_gate"] = bool(max(sz["rmse"], s1["rmse"]) <= 1e-4 and res["nan_inf"] == 0)
    return res


def run_flow_joint(torch, dev, steps, with_cpu=False):
    """The reference-faithful single-stream graph (tsplat/flow_joint.py): one
    block over 18433 = 16384 latent + 2048 condition + 1 camera tokens
    (1.855 TFLOP), and one 28-block CFG Euler step of the latent and the
    camera state computed in full and with the reference's
    exactness-preserving reductions (negative branch with one condition row +
    log(M) key bias, selected-rows final block)."""
    from tsplat.flow import FlowConfig
    from tsplat.flow_joint import JointFlowModel, camera_state

    cfg = FlowConfig()
    C, L, Lc, H = cfg.hidden, cfg.latent_tokens, cfg.cond_tokens, cfg.heads
    model = JointFlowModel(cfg, dev)
    z_h, c_h = flow_inputs(cfg)
    z, c = torch.from_numpy(z_h).to(dev), torch.from_numpy(c_h).to(dev)
    cam = torch.from_numpy(camera_state(cfg, SEEDS["flow_camera"])).to(dev)
    Lt = L + Lc + 1
    _, t_mod = model.timestep(torch.full((1,), 1000.0, device=dev))
    x = torch.cat((z, c, model.cam_refiner(cam)), 0)[None].contiguous()
    for _ in range(2):
        model.block_forward(model.blocks[0], x, t_mod, L)
    torch.cuda.synchronize()
    blk_ms = time_events(torch, lambda: model.block_forward(model.blocks[0], x, t_mod, L), 5)
    blk_flop = 2.0 * Lt * C * 12 * C + 4.0 * H * Lt * Lt * 64

    def step_time(reduce):
        model.euler_cfg_step(z, c, cam, reduce_work=reduce)
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(1, steps)):
            t0 = time.perf_counter()
            zn, _, cn, _ = model.euler_cfg_step(z, c, cam, reduce_work=reduce)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2], zn, cn

    full_s, zf, cf = step_time(False)
    red_s, zr, cr = step_time(True)
    rmse_lat = float((zr - zf).double().square().mean().sqrt())
    rmse_cam = float((cr - cf).double().square().mean().sqrt())
    del model, x, zf, cf, zr, cr
    return {
        "workload": "single-stream graph: 28 blocks over 16384 latent + 2048 condition + 1 camera tokens, "
                    "CFG pair, one Euler step of latent and camera state",
        "block_ms": blk_ms, "block_tflops": blk_flop / (blk_ms * 1e-3) / 1e12,
        "s_per_denoise_step_full": full_s, "s_per_denoise_step_reduced": red_s,
        "speedup_from_reduction": full_s / red_s,
        "reduced_vs_full_latent_rmse": rmse_lat,
        "reduced_vs_full_camera_rmse": rmse_cam,
        "reference_shapes": run_flow_joint_reference_shapes(torch, dev, steps, with_cpu),
    }


# The reference's published s20 run (docs/triposplat_cpu_p0_p1_validation_20260722_ja.md:139-143):
# 2747.270 s for 20 denoise steps on 4 EPYC 9654 cores, of which NF24 Linear 1008.472 s and exact SDPA 1432.319 s.
PUBLISHED_S20 = {"s_per_denoise_step": 2747.270 / 20, "hot_path_s_per_denoise_step": (1008.472 + 1432.319) / 20,
                 "cpus": 4, "host": "AMD EPYC 9654"}


def run_flow_joint_reference_shapes(torch, dev, steps, with_cpu=False):
    """The single-stream graph at the reference model's real sequence lengths:
    8192 latent + 4101 condition + 1 camera tokens, 28 blocks, CFG pair with
    both reductions -- positive branch L = 12294, compressed negative branch
    L = 8194, final block 8193 selected queries against 12294 keys, the
    shapes of the reference's published s20 step.  (The real model runs 4 of
    its 28 blocks as refiners over the latent or the condition rows only, so
    28 joint blocks are an upper bound of its block work.)  With with_cpu and
    the reference's AVX-512 build on the host, the same step is computed in
    full (both branches over all 12294 rows, all 28 blocks) by the
    reference's kernels on the host cores: its wall time, and the latent and
    camera RMSE of the device's reduced step against it (the north star's
    full-sampler-step gate, compare_latent_npz.py:22-71)."""
    from tsplat.flow import FlowConfig
    from tsplat.flow_joint import JointFlowModel, camera_state

    cfg = FlowConfig(latent_tokens=8192, cond_tokens=4101)
    model = JointFlowModel(cfg, dev)
    z_h, c_h = flow_inputs(cfg)
    z, c = torch.from_numpy(z_h).to(dev), torch.from_numpy(c_h).to(dev)
    cam = torch.from_numpy(camera_state(cfg, SEEDS["flow_camera"])).to(dev)

    def step_time():
        model.euler_cfg_step(z, c, cam, reduce_work=True)
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(1, steps)):
            t0 = time.perf_counter()
            model.euler_cfg_step(z, c, cam, reduce_work=True)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    strict = step_time()
    zn, vn, cn, vcn = (a.cpu().numpy() for a in model.euler_cfg_step(z, c, cam, reduce_work=True))
    model.set_precision("bf16x3", include=("blocks", "attention"))
    fast = step_time()
    zn3, _, cn3, _ = model.euler_cfg_step(z, c, cam, reduce_work=True)
    zn3, cn3 = zn3.cpu().numpy(), cn3.cpu().numpy()
    model.set_precision("fp32")
    cpu_res = None
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import numpy as np
        import oracle as O
        from flow_ref import CpuJointFlow, combined_rmse, combined_rmse_from_key_mse, latent_stats, non_finite

        if O.ref_available():
            cpu = CpuJointFlow(model.host(), cfg, backend="reference", threads=HOST_THREADS)
            t0 = time.perf_counter()
            cpu.progress = lambda i: (print(f"cpu joint step: block {i + 1}/{cfg.blocks} "
                                            f"({time.perf_counter() - t0:.0f} s)", file=sys.stderr, flush=True)
                                      if (i + 1) % 7 == 0 else None)
            zc, vc, cc, vcc = cpu.joint_euler_cfg_step(z_h, c_h, camera_state(cfg, SEEDS["flow_camera"]))
            cpu_s = time.perf_counter() - t0
            keys = {"latent": latent_stats(zc, zn), "camera": latent_stats(cc, cn)}
            rel = lambda ref, got: combined_rmse(got, ref) / float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
            cpu_res = {
                "kind": "reference", "cores": HOST_THREADS,
                "s_per_denoise_step": cpu_s, "speedup_gpu_vs_cpu": cpu_s / strict,
                "speedup_gpu_bf16x3_vs_cpu": cpu_s / fast,
                "latent_rmse_vs_cpu": keys["latent"]["rmse"], "camera_rmse_vs_cpu": keys["camera"]["rmse"],
                "combined_rmse_vs_cpu": combined_rmse_from_key_mse(keys),
                "velocity_rel_rmse": rel(vc, vn), "camera_velocity_rel_rmse": rel(vcc, vcn),
                "nan_inf": sum(non_finite(k) for k in keys.values()),
                "bf16x3_latent_rmse_vs_cpu": combined_rmse(zn3, zc),
                "bf16x3_camera_rmse_vs_cpu": combined_rmse(cn3, cc), "gate_rmse": 1e-4,
            }
            cpu_res["within_gate"] = bool(max(cpu_res["latent_rmse_vs_cpu"], cpu_res["camera_rmse_vs_cpu"],
                                              cpu_res["bf16x3_latent_rmse_vs_cpu"],
                                              cpu_res["bf16x3_camera_rmse_vs_cpu"]) <= 1e-4
                                          and cpu_res["nan_inf"] == 0)
    return {
        "workload": "single-stream graph at the reference's real lengths: 28 blocks over 8192 latent + 4101 condition "
                    "+ 1 camera tokens, CFG pair with negative-branch compression (L = 12294 / 8194) and the "
                    "selected final block (8193 x 12294), one Euler step",
        "s_per_denoise_step": strict,
        "opt_in_bf16x3_block_linears_and_attention_s_per_denoise_step": fast,
        "published_reference_cpu": PUBLISHED_S20,
        "speedup_vs_published_cpu_step": PUBLISHED_S20["s_per_denoise_step"] / strict,
        "speedup_vs_published_cpu_hot_path": PUBLISHED_S20["hot_path_s_per_denoise_step"] / strict,
        "cpu_reference_full_step": cpu_res,
    }


def run_gemm_skinny(torch, dev, replays=5):
    """configs[0] skinny-M variants (HBM-bound): M in {1, 2, 8, 16} rows against
    the K x N weights {1024 x 3072, 1024 x 6144, 4096 x 1024}.  GB/s counts the
    algorithmic bytes 3*K*N + 8*N + 4*M*(K+N) per call against the 8 TB/s HBM
    peak.  Each Linear of a denoise step runs once with its own weights, so
    the calls cycle through enough distinct weight copies (> 640 MB) that no
    copy is still in the 256 MB last-level cache when it is read again; the
    calls are captured once in a HIP graph (so host launch cost is not
    counted) and the replays are timed with HIP events."""
    from tsplat.nf24 import nf24_linear, quantize_nf24_i16_per_output_channel

    g = torch.Generator(device=dev).manual_seed(SEEDS["skinny_torch"])
    rows = []
    stream = torch.cuda.Stream(device=dev)
    for K, N in ((1024, 3072), (1024, 6144), (4096, 1024)):
        w = torch.randn((N, K), generator=g, device=dev) * 0.02
        b = torch.randn((N,), generator=g, device=dev) * 0.01
        codes, scales, _ = quantize_nf24_i16_per_output_channel(w)
        copies = -(-(640 << 20) // (3 * K * N))
        c01 = [codes[0].clone() for _ in range(copies)]
        q2 = [codes[1].clone() for _ in range(copies)]
        for M in (1, 2, 8, 16):
            x = torch.randn((M, K), generator=g, device=dev)
            out = torch.empty((M, N), device=dev)
            ref = nf24_linear(x, codes[0], codes[1], scales[0], b).clone()

            def chain():
                for i in range(copies):
                    nf24_linear(x, c01[i], q2[i], scales[0], b, out=out)

            stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(stream):
                chain()  # sizes this stream's workspace before the capture
                stream.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream, capture_error_mode="relaxed"):
                    chain()
                graph.replay()
                stream.synchronize()
                same = bool(torch.equal(out, ref))
                ms = sorted(time_events(torch, graph.replay, 1) for _ in range(replays))
            us = ms[len(ms) // 2] * 1e3 / copies
            byts = 3 * K * N + 8 * N + 4 * M * (K + N)
            rows.append({"M": M, "K": K, "N": N, "us": us, "GBps": byts / us / 1e3,
                         "frac_hbm_peak": byts / us / 1e3 / PEAK_HBM, "calls_per_graph": copies,
                         "graph_equals_eager": same})
            del graph
        del c01, q2
    return rows


def run_copy(torch, dev, iters):
    """Calibration kernel for the HBM counters: a plain 256 MiB device copy."""
    n = 64 << 20
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = time_events(torch, lambda: dst.copy_(src), iters)
    return {"bytes_read": n * 4, "bytes_written": n * 4, "ms": ms, "GBps": 2 * n * 4 / (ms * 1e-3) / 1e9}


# Keys whose content is prose or provenance the DESIGN and profiles already
# state; the printed line keeps the numbers (the driver keeps ~10 KB of output).
_PROSE = {"workload", "compared", "host_lscpu", "order", "omp", "alternating_gpu_ms", "sample", "host_cpu",
          "threads8_alternating_gpu_ms",
          "published_reference_cpu", "published_cpu_s_4cpu_gcc9_gcc13", "rows", "calls_per_graph"}


_PARITY_KEEP = ("max_abs", "rel_rmse", "within_tolerance", "rmse", "within_gate")


def compact(o, key=None):
    """The bench line's figures: floats to 4 significant digits (more than
    any of them is reproducible to), prose keys dropped below the top level;
    parity records keep max-abs, relative RMSE and the verdict (plus the RMSE
    where a gate is on it); the skinny-M rows become a table; the reference
    shapes' rows drop the sizes their names carry."""
    if isinstance(o, float):
        return float(f"{o:.4g}")
    if isinstance(o, dict):
        if key == "parity_vs_reference":
            o = {k: v for k, v in o.items() if k in _PARITY_KEEP and (k != "rmse" or "within_gate" in o)}
        if key == "reference_shapes":
            o = {n: ({k: v for k, v in r.items() if k not in ("M", "K", "N", "Lq", "Lk", "key_bias")}
                     if isinstance(r, dict) and (n.startswith("gemm_") or n.startswith("sdpa_")) else r)
                 for n, r in o.items()}
        return {k: compact(v, k) for k, v in o.items() if k not in _PROSE}
    if isinstance(o, (list, tuple)):
        if key == "skinny_m" and o and isinstance(o[0], dict):
            cols = ("M", "K", "N", "us", "GBps", "frac_hbm_peak")
            return {"cols": list(cols), "rows": [[compact(r[c]) for c in cols] for r in o],
                    "graph_equals_eager": all(r.get("graph_equals_eager", False) for r in o)}
        return [compact(v) for v in o]
    return o


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=("sdpa", "gemm", "copy", "flow", "skinny", "gemm16k", "refshapes",
                                       "joint_ref"),
                    default=None,
                    help="run one workload alone (for profiler runs) and print its figures")
    ap.add_argument("--no-flow", action="store_true", help="skip configs[3]/[4] (flow block / step)")
    ap.add_argument("--precision", choices=("fp32", "bf16", "bf16x3"), default="fp32",
                    help="SDPA product precision for --only sdpa (profiling the opt-in modes)")
    ap.add_argument("--validate-flow", action="store_true",
                    help="run the configs[4] CPU reference step even with --no-cpu-baseline (minutes of CPU time)")
    ap.add_argument("--detail", default=None,
                    help="also write the line with every field and full-precision figures to this JSON file")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(multi-GPU sharding is a design note, not implemented)"}))
        return 2

    import torch
    from tsplat import load_library

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    load_library()

    if args.only == "gemm":
        print(json.dumps(run_gemm(torch, dev, max(3, args.steps))))
        return 0
    if args.only == "copy":
        print(json.dumps(run_copy(torch, dev, max(3, args.steps))))
        return 0
    if args.only == "skinny":
        print(json.dumps(run_gemm_skinny(torch, dev)))
        return 0
    if args.only == "gemm16k":
        print(json.dumps(run_gemm_l16384(torch, dev)))
        return 0
    if args.only == "refshapes":
        print(json.dumps(run_reference_shapes(torch, dev, not args.no_cpu_baseline)))
        return 0
    if args.only == "flow":
        print(json.dumps(run_flow(torch, dev, 3, not args.no_cpu_baseline, args.validate_flow)))
        return 0
    if args.only == "joint_ref":
        print(json.dumps(run_flow_joint_reference_shapes(torch, dev, 3, not args.no_cpu_baseline)))
        return 0

    host = sdpa_inputs(torch, dev)
    B, H, L, D = host[0].shape
    if args.only == "sdpa":
        wall, kernel_ms, _ = run_sdpa(torch, dev, args.steps, args.warmup, host, args.precision)
        print(json.dumps({"sdpa_ms": kernel_ms, "precision": args.precision,
                          "tflops_equiv": 4.0 * B * H * L * L * D / (kernel_ms * 1e-3) / 1e12}))
        return 0
    if args.precision != "fp32":
        print("--precision applies to --only sdpa; the full line measures fp32 and reports the "
              "opt-in modes beside it", file=sys.stderr)
        return 2
    wall, kernel_ms, sdpa_out = run_sdpa(torch, dev, args.steps, args.warmup, host,
                                         keep_out=not args.no_cpu_baseline)
    sdpa_flop = 4.0 * B * H * L * L * D
    achieved = sdpa_flop / (kernel_ms * 1e-3) / 1e12

    variants = run_sdpa_variants(torch, dev, host, ref_parity=not args.no_cpu_baseline)
    sdpa_opt_in = run_sdpa_opt_in(torch, dev, host, kernel_ms)
    gemm = run_gemm(torch, dev, 20, ref_parity=not args.no_cpu_baseline)
    gemm["skinny_m"] = run_gemm_skinny(torch, dev)
    gemm["l16384"] = run_gemm_l16384(torch, dev)
    refshapes = run_reference_shapes(torch, dev, not args.no_cpu_baseline)
    flow = None if args.no_flow else run_flow(torch, dev, 3, not args.no_cpu_baseline, args.validate_flow)
    cpu = None
    if not args.no_cpu_baseline:
        from tsplat.native_sdpa_ctypes import native_sdpa_f32_ex

        qd, kd, vd = (torch.from_numpy(a).to(dev) for a in host)
        od = torch.empty((B, L, H, D), dtype=torch.float32, device=dev)
        gpu_fn = lambda: time_events(  # noqa: E731
            torch, lambda: native_sdpa_f32_ex(qd, kd, vd, out=od, out_layout="blhd"), 1)
        cpu = cpu_baseline_sdpa(*host, gpu_out=sdpa_out, gpu_fn=gpu_fn)
        del qd, kd, vd, od

    line = {
        "metric": METRIC,
        "value": sdpa_flop / wall / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy PCG64 inputs; q/k RoPE theta 1e4 + RMSNorm)",
        "config": {
            "workload": "configs[1] exact dense self-attention SDPA, B=1 H=16 D=64 Lq=Lk=16384, scale 1/8, no mask, BLHD out",
            "B": B, "H": H, "Lq": L, "Lk": L, "head_dim": D,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_FP32_MFMA,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_FP32_MFMA,
            "traffic": load_traffic("sdpa_config1"),
            "kernel_ms": kernel_ms,
            "flop_per_launch": sdpa_flop,
        },
        "cpu_baseline": cpu,
        "sdpa_opt_in_bf16": sdpa_opt_in,
        "sdpa_config2": variants,
        "gemm_config0": gemm,
        "reference_shapes": refshapes,
        "flow": flow,
    }
    if args.detail:
        Path(args.detail).write_text(json.dumps(line, indent=1))
    out = {k: (v if k in ("config", "metric", "unit", "dtype", "data", "scaling") else compact(v, k))
           for k, v in line.items()}
    if cpu is not None:
        out["cpu_baseline"]["sample"] = cpu["sample"]
        out["cpu_baseline"]["host_cpu"] = cpu["host_cpu"]
    print(json.dumps(out, separators=(",", ":")))
    return 0


if __name__ == "__main__":
    sys.exit(main())
