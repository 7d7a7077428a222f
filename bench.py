"""Benchmark of the strict owned-tensor hot path on one MI355X.

Headline (BASELINE.json `metric`): strict F32 MatMul 4096^3, A and B uniform[-1,1]
(seeded), inputs resident in HBM. One step = one complete strict MatMul call through the C
ABI: exponent prefilter, main tile kernel, exact-replay check and the terminal fault-word
readback. `value` is GFLOP/s = 2*M*N*K / step time. The dominant kernel's live duration
(HIP events on its own stream) gives the roofline; `cpu_baseline` times the faithful
single-thread CPU port of the reference's integer-law MatMul on a bounded row sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "fusion-pcu_amd")

METRIC = "strict F32 MatMul GFLOP/s @4096³ (% FP32 vector peak); MLP train steps/s"
FP32_PEAK_TFLOPS = 157.3       # MI355X FP32 vector peak (counts an FMA as 2 flop)
# A strict (cell, k) step is a rounded multiply plus a rounded add worth 2 flop. gfx950
# issues at most two VALU instructions per SIMD per 4 cycles (32 lanes/clk) and issues no
# VALU while an F32 MFMA runs, so either engine (v_mul + v_add, or an MFMA product +
# v_add) reaches at most half of the FMA-counted peak.
FP32_STRICT_CEILING = 78.6
FP64_PEAK_TFLOPS = 78.6
HBM_PEAK_GBS = 8000.0


def _package():
    if "fusion_pcu_amd" in sys.modules:
        return sys.modules["fusion_pcu_amd"]
    spec = importlib.util.spec_from_file_location(
        "fusion_pcu_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["fusion_pcu_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_matmul(pkg, ctx, m, k, n, dtype, steps, warmup, seed_a=11, seed_b=12):
    from fusion_pcu_amd import synthetic as syn
    a = syn.uniform(seed_a, (m, k), dtype)
    b = syn.uniform(seed_b, (k, n), dtype)
    da, db = ctx.upload(a), ctx.upload(b)
    dc = ctx.empty((m, n), dtype)
    for _ in range(warmup):
        ctx.strict_matmul(da, db, out=dc)
    ctx.synchronize()
    ctx.profile(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.strict_matmul(da, db, out=dc)
    ctx.synchronize()
    t1 = time.perf_counter()
    gemm_ms, gemm_n = ctx.kernel_time("strict_gemm")
    pre_ms, _ = ctx.kernel_time("gemm_prefilter")
    rep_ms, _ = ctx.kernel_time("gemm_replay")
    ctx.profile(False)
    for x in (da, db, dc):
        x.free()
    ms_step = (t1 - t0) * 1e3 / steps
    return {
        "ms_per_step": ms_step,
        "gflops": 2.0 * m * n * k / (ms_step * 1e-3) / 1e9,
        "gemm_avg_ms": gemm_ms / max(gemm_n, 1),
        "gemm_launches": gemm_n,
        "prefilter_avg_ms": pre_ms / max(gemm_n, 1),
        "replay_avg_ms": rep_ms / max(gemm_n, 1),
    }


def bench_sgd(pkg, ctx, n, steps, warmup):
    """C4: strict F32 SGD over 2^28 elements (12 B/elem compulsory traffic)."""
    from fusion_pcu_amd import synthetic as syn
    w = syn.normal(41, (n,), 1.0, np.float32)
    g = syn.normal(42, (n,), 1e-3, np.float32)
    w[: n // 100] = np.float32(1e-38)
    dw, dg = ctx.upload(w), ctx.upload(g)
    del w, g
    out = ctx.empty((n,), np.float32)
    for _ in range(warmup):
        ctx.strict_sgd(dw, dg, 0.01, out=out)
    ctx.synchronize()
    ctx.profile(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.strict_sgd(dw, dg, 0.01, out=out)
    ctx.synchronize()
    t1 = time.perf_counter()
    k_ms, k_n = ctx.kernel_time("sgd")
    ctx.profile(False)
    for x in (dw, dg):
        x.free()
    avg = k_ms / max(k_n, 1)
    res = {"elements": n, "ms_per_step": (t1 - t0) * 1e3 / steps, "kernel_avg_ms": avg,
           "kernel_GBps": 12.0 * n / (avg * 1e-3) / 1e9,
           "kernel_hbm_frac": 12.0 * n / (avg * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # C4's checked add then ReLU over the same size, fused (one kernel, 12 B/element).
    dw, dg = ctx.upload(syn.normal(41, (n,), 1.0, np.float32)), ctx.upload(syn.normal(42, (n,), 1e-3, np.float32))
    for _ in range(2):
        ctx.checked_add_relu(dw, dg, out=out)
    ctx.synchronize()
    ctx.profile(True)
    for _ in range(steps):
        ctx.checked_add_relu(dw, dg, out=out)
    ctx.synchronize()
    a_ms, a_n = ctx.kernel_time("add_relu")
    ctx.profile(False)
    for x in (dw, dg, out):
        x.free()
    a_avg = a_ms / max(a_n, 1)
    res["add_relu_kernel_avg_ms"] = a_avg
    res["add_relu_kernel_GBps"] = 12.0 * n / (a_avg * 1e-3) / 1e9
    res["add_relu_hbm_frac"] = res["add_relu_kernel_GBps"] / HBM_PEAK_GBS
    return res


def bench_native_matmul(pkg, ctx, m, k, n, dtype, steps, warmup):
    """Native (BackendDefined) MatMul: matrix-core accumulation for F32."""
    from fusion_pcu_amd import synthetic as syn
    da = ctx.upload(syn.uniform(11, (m, k), dtype))
    db = ctx.upload(syn.uniform(12, (k, n), dtype))
    dc = ctx.empty((m, n), dtype)
    for _ in range(warmup):
        ctx.native_matmul(da, db, out=dc)
    ctx.synchronize()
    ctx.profile(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.native_matmul(da, db, out=dc)
    ctx.synchronize()
    t1 = time.perf_counter()
    k_ms, k_n = ctx.kernel_time("native_gemm")
    ctx.profile(False)
    for x in (da, db, dc):
        x.free()
    avg = k_ms / max(k_n, 1)
    return {"gflops": 2.0 * m * n * k / ((t1 - t0) / steps) / 1e9, "kernel_avg_ms": avg,
            "kernel_tflops": 2.0 * m * n * k / (avg * 1e-3) / 1e12}


def bench_mlp(pkg, ctx, steps, warmup, native=False):
    """C5: strict F32 MLP 1024->4096->4096->1024, batch 4096, lr 1e-3, Xavier weights,
    inputs and weights resident; one step = forward, MSE, backward, three SGD updates.
    ``native`` captures the same step with flag(native_compound) (Boundary mode)."""
    from fusion_pcu_amd import graph as G
    from fusion_pcu_amd import synthetic as syn
    dims, batch = (1024, 4096, 4096, 1024), 4096
    x = G.PcuTensor(ctx.upload(syn.uniform(51, (batch, dims[0]), np.float32)))
    y = G.PcuTensor(ctx.upload(syn.uniform(52, (batch, dims[3]), np.float32)))
    ws = [G.PcuTensor(ctx.upload(syn.xavier_uniform(53 + i, dims[i], dims[i + 1], np.float32)))
          for i in range(3)]
    step = G.mlp_training_step(1e-3, native=native)
    for _ in range(warmup):
        *ws, loss = step(x, *ws, y)
    ctx.synchronize()
    # steps/s without per-kernel timing: its HIP events cost every kernel a gap.
    t0 = time.perf_counter()
    for _ in range(steps):
        *ws, loss = step(x, *ws, y)
    ctx.synchronize()
    t1 = time.perf_counter()
    # The per-kernel breakdown from a second, timed pass of the same number of steps.
    ctx.profile(True)
    for _ in range(steps):
        *ws, loss = step(x, *ws, y)
    ctx.synchronize()
    kern = {k: ctx.kernel_time(k) for k in ("strict_gemm", "gemm_prefilter", "gemm_replay",
                                            "sgd", "binary", "relu", "relu_backward", "mse",
                                            "native_gemm", "native_sgd", "native_mse")}
    ctx.profile(False)
    flops = 2.0 * batch * (dims[0] * dims[1] + dims[1] * dims[2] + dims[2] * dims[3]) * 3 \
        - 2.0 * batch * dims[0] * dims[1]  # no input-gradient MatMul for X
    ms = (t1 - t0) * 1e3 / steps
    return {
        "steps_per_s": 1e3 / ms,
        "ms_per_step": ms,
        "matmul_gflop_per_step": flops / 1e9,
        "gemm_ms_per_step": (kern["native_gemm"] if native else kern["strict_gemm"])[0] / steps,
        "mse_ms_per_step": (kern["native_mse"] if native else kern["mse"])[0] / steps,
        "elementwise_ms_per_step": sum(kern[k][0] for k in ("sgd", "binary", "relu", "relu_backward",
                                                            "native_sgd")) / steps,
        "loss": float(loss.numpy()),
    }


def cpu_baseline(m, k, n, rows):
    """Faithful port (integer-significand law, one thread) on `rows` output rows."""
    sys.path.insert(0, ROOT)
    import oracle
    from fusion_pcu_amd import synthetic as syn
    a = syn.uniform(11, (m, k), np.float32)
    b = syn.uniform(12, (k, n), np.float32)
    t0 = time.perf_counter()
    _, fault = oracle.matmul(a, b, rows_subset=(0, rows), fast=False)
    dt = time.perf_counter() - t0
    assert fault is None
    return {
        "value": 2.0 * rows * n * k / dt / 1e9,
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"output rows 0..{rows - 1} of the strict F32 MatMul {m}x{k}x{n} "
                  f"({rows * n} cells, {rows * n * k} ordered multiply/add pairs) with the "
                  f"faithful single-thread integer-law port of the reference CPU backend; "
                  f"{dt:.1f} s",
    }


def cpu_fast_oracle(m, k, n, seconds=5.0):
    """The same MatMul on the oracle's fast path (host IEEE arithmetic with a conservative
    screen re-run through the integer law, OpenMP on all the host cores we may use), on a
    leading block of output rows sized to about `seconds`."""
    sys.path.insert(0, ROOT)
    import oracle
    from fusion_pcu_amd import synthetic as syn
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    a = syn.uniform(11, (m, k), np.float32)
    b = syn.uniform(12, (k, n), np.float32)
    rows, dt = 64, 0.0
    while True:
        t0 = time.perf_counter()
        _, fault = oracle.matmul(a[:rows], b, threads=threads)
        dt = time.perf_counter() - t0
        assert fault is None
        if dt >= seconds / 4 or rows >= m:
            break
        rows = min(m, rows * 4)
    return {
        "value": 2.0 * rows * n * k / dt / 1e9,
        "unit": "GFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"output rows 0..{rows - 1} of the strict F32 MatMul {m}x{k}x{n} with the "
                  f"oracle's fast path ({threads} OpenMP threads); {dt:.1f} s",
    }


def probe(pkg, M, K, N) -> int:
    """One launch of each kernel whose counters are read with rocprofv3 --pmc: the strict
    F32 MatMul 4096^3 (both engines), a copy-like calibration kernel (checked Add of +0 over
    2^26 f32: 256 MiB read + 256 MiB written), strict SGD over 2^26 f32 and the strict F64
    MatMul 4096^3 (after one warm-up launch)."""
    from fusion_pcu_amd import synthetic as syn
    n = 1 << 26
    with pkg.Context(0) as ctx:
        da = ctx.upload(syn.uniform(11, (M, K), np.float32))
        db = ctx.upload(syn.uniform(12, (K, N), np.float32))
        dc = ctx.empty((M, N), np.float32)
        x = ctx.upload(syn.uniform(21, (n,), np.float32))
        g = ctx.upload(syn.uniform(22, (n,), np.float32))
        y = ctx.empty((n,), np.float32)
        log("probe: warmup")
        ctx.strict_matmul(da, db, out=dc)
        ctx.checked_binary(0, x, 0.0, out=y)
        ctx.strict_sgd(x, g, 0.01, out=y)
        log("probe: one launch each (MatMul: matrix-core products, then vector-unit engine)")
        ctx.strict_matmul(da, db, out=dc)
        ctx.checked_binary(0, x, 0.0, out=y)
        ctx.strict_sgd(x, g, 0.01, out=y)
        ctx.set_matmul_engine("valu")
        ctx.strict_matmul(da, db, out=dc)
        ctx.set_matmul_engine("auto")
        log("probe: F64 MatMul (C3 shape), warm-up then one launch")
        for x_ in (da, db, dc):
            x_.free()
        da = ctx.upload(syn.uniform(31, (M, K), np.float64))
        db = ctx.upload(syn.uniform(32, (K, N), np.float64))
        dc = ctx.empty((M, N), np.float64)
        ctx.strict_matmul(da, db, out=dc)
        ctx.strict_matmul(da, db, out=dc)
        ctx.synchronize()
    log("probe: done")
    return 0


def _traffic(workload: str):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as fh:
            return json.load(fh).get(workload)
    except (OSError, ValueError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=32)
    ap.add_argument("--probe", action="store_true",
                    help="run each profiled kernel once (for rocprofv3 --pmc passes) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the strict path has no multi-GPU leg in this "
              f"build (requested --gpus {args.gpus})", file=sys.stderr)
        return 2

    pkg = _package()
    M = N = K = 4096
    if args.probe:
        return probe(pkg, M, K, N)
    from fusion_pcu_amd import graph as G
    G.configure(0)
    ctx = G.default_context()
    if True:
        log("strict F32 MatMul 4096^3")
        mm = bench_matmul(pkg, ctx, M, K, N, np.float32, args.steps, args.warmup)
        extra = {}
        if not args.no_extra:
            log("strict F32 MLP training step (C5)")
            extra["mlp_c5"] = bench_mlp(pkg, ctx, max(5, args.steps), 2)
            log("native (BackendDefined) F32 MatMul 4096^3")
            extra["native_f32_matmul_4096"] = bench_native_matmul(pkg, ctx, M, K, N, np.float32,
                                                                  args.steps, args.warmup)
            log("native (BackendDefined) C5 MLP training step")
            extra["mlp_c5_native"] = bench_mlp(pkg, ctx, max(5, args.steps), 2, native=True)
            log("strict F32 MatMul 4096^3, vector-unit engine")
            ctx.set_matmul_engine("valu")
            v = bench_matmul(pkg, ctx, M, K, N, np.float32, args.steps, args.warmup)
            ctx.set_matmul_engine("auto")
            extra["f32_matmul_4096_valu_engine"] = {
                "gflops": v["gflops"], "gemm_avg_ms": v["gemm_avg_ms"],
                "gemm_tflops": 2.0 * M * N * K / (v["gemm_avg_ms"] * 1e-3) / 1e12}
            log("strict F64 MatMul 4096^3 (C3 shape)")
            f64 = bench_matmul(pkg, ctx, M, K, N, np.float64, max(2, args.steps // 3), 1, 31, 32)
            extra["f64_matmul_4096"] = {
                "gflops": f64["gflops"], "gemm_avg_ms": f64["gemm_avg_ms"],
                "gemm_tflops": 2.0 * M * N * K / (f64["gemm_avg_ms"] * 1e-3) / 1e12,
                "frac_fp64_vector_peak": 2.0 * M * N * K / (f64["gemm_avg_ms"] * 1e-3) / 1e12 / FP64_PEAK_TFLOPS,
            }
            log("strict F32 SGD 2^28 (C4 shape)")
            extra["sgd_f32_2p28"] = bench_sgd(pkg, ctx, 1 << 28, max(5, args.steps), 2)

    gemm_s = mm["gemm_avg_ms"] * 1e-3
    achieved = 2.0 * M * N * K / gemm_s / 1e12
    roofline = {
        "bound": "mfma",
        "achieved": round(achieved, 3),
        "peak": FP32_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
        "traffic": _traffic("strict_gemm_f32_4096"),
        "kernel": "k_strict_gemm_mfma<GemmCfg> (main tile kernel: matrix-core products, ordered vector-unit adds)",
        "kernel_avg_ms": round(mm["gemm_avg_ms"], 4),
        "algorithmic_flops_per_launch": 2 * M * N * K,
        "peak_kind": "FP32 peak (vector FMA = dense matrix, 157.3 TFLOP/s)",
        "strict_valu_ceiling_tflops": FP32_STRICT_CEILING,
        "frac_of_strict_ceiling": round(achieved / FP32_STRICT_CEILING, 4),
    }
    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline: faithful port on {args.cpu_rows} rows")
        cpu = cpu_baseline(M, K, N, args.cpu_rows)
        if not args.no_extra:
            log("CPU reference point: the oracle's fast path on all allowed host cores")
            extra["cpu_fast_oracle"] = cpu_fast_oracle(M, K, N)
    line = {
        "metric": METRIC,
        "value": round(mm["gflops"], 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mm["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64 uniform[-1,1], seeds 11/12)",
        "config": {"workload": "strict F32 MatMul 4096x4096x4096 (A,B uniform[-1,1]); one step = "
                               "prefilter + tile kernel + replay check + fault readback",
                   "m": M, "k": K, "n": N},
        "pct_fp32_vector_peak": round(100.0 * mm["gflops"] / 1e3 / FP32_PEAK_TFLOPS, 3),
        "mlp_train_steps_per_s": (round(extra["mlp_c5"]["steps_per_s"], 3)
                                  if "mlp_c5" in extra else None),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
