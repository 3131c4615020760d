"""Benchmark of the MI355X FP8 linear path (one JSON line on stdout).

Workload ("c2"): the fused gated-GELU MLP at Gemma-3-4B width,
X bf16 [4096, 2560], W_gate/W_up [10240, 2560], W_down [2560, 10240]. One step is the
whole FP8 forward with inputs resident in HBM:
  quantize X, [W_gate; W_up], W_down (amax -> scale -> e4m3 cast, per tensor)
  gate/up GEMM with the gated-GELU epilogue (+ per-tile amax of H)
  H scale, H e4m3 cast, down GEMM -> Y bf16 [4096, 2560]
``value`` = 2*M*(2I*K + K*I) FLOP per step / step time (TFLOP/s). Weight quantization is
inside the step (the first-microbatch case); the cached-weight rate is reported beside it.

``roofline`` covers the dominant kernel (gate/up GEMM + gated-GELU epilogue): algorithmic
FLOP per launch / its average launch time from HIP events on the launch stream, against
the dense FP8 MFMA peak. ``traffic`` comes from rocprofv3 FETCH_SIZE/WRITE_SIZE runs
summarised in profiles/ (null when no such summary exists).

``cpu_baseline`` times the CPU oracle (torch CPU: amax, clamp, .to(float8), fp32 matmul,
bf16 gelu chain -- torchao's emulate path) on the same step, on this host's cores.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA (AMD public spec), no sparsity
HBM_PEAK_GBPS = 8000.0
METRIC = "FP8 linear TFLOP/s & % MFMA peak at 4B shapes; quantize cast GB/s"


def _args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--rows", type=int, default=4096)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-reps", type=int, default=1)
    return p.parse_args()


def _load_traffic():
    f = ROOT / "profiles" / "traffic_gemm_geglu_c2.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text())
    except (OSError, ValueError):
        return None


def main():
    args = _args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (every box has one MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import torch

    from bongard_amd import ops, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M = args.rows
    K, I = workloads.HIDDEN, workloads.INTERMEDIATE
    c = workloads.config2(rows=M)
    x = c["x"].to(dev)
    w_gu = torch.cat([c["w_gate"], c["w_up"]], 0).to(dev)
    w_d = c["w_down"].to(dev)
    flop = 2.0 * M * (2 * I * K + K * I)

    def step(cached=None):
        xq = ops.quantize(x, ops.E4M3)
        if cached is None:
            gq = ops.quantize(w_gu, ops.E4M3)
            dq = ops.quantize(w_d, ops.E4M3)
        else:
            gq, dq = cached
        H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
        hq = ops.cast_partials(H, hparts, ops.E4M3)
        hm = hq.meta
        return ops.gemm(hq.data, ops.E4M3, hm, dq.data, ops.E4M3, dq.meta)

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    sec = timed(step, args.steps, args.warmup)
    cached = (ops.quantize(w_gu, ops.E4M3), ops.quantize(w_d, ops.E4M3))
    sec_cached = timed(lambda: step(cached), args.steps, args.warmup)

    # ---- dominant kernel: gate/up GEMM + gated-GELU epilogue, HIP events on its stream
    xq = ops.quantize(x, ops.E4M3)
    gq = cached[0]
    stream = torch.cuda.current_stream()
    n_launch = max(10, args.steps)
    for _ in range(3):
        ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(n_launch):
        ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
    ev1.record(stream)
    torch.cuda.synchronize()
    geglu_s = ev0.elapsed_time(ev1) / 1e3 / n_launch
    geglu_flop = 2.0 * M * (2 * I) * K
    achieved = geglu_flop / geglu_s / 1e12

    # ---- down GEMM and the activation quantize (HBM-bound), same method
    H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
    hq = ops.cast_partials(H, hparts, ops.E4M3)
    hm = hq.meta
    dq = cached[1]

    def ev_time(fn, n=n_launch):
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / 1e3 / n

    down_s = ev_time(lambda: ops.gemm(hq.data, 0, hm, dq.data, 0, dq.meta))
    qx_s = ev_time(lambda: ops.quantize(x, ops.E4M3))
    qh_s = ev_time(lambda: ops.cast(H, hm, ops.E4M3))
    qw_s = ev_time(lambda: ops.quantize(w_gu, ops.E4M3))

    traffic = _load_traffic()
    roofline = {
        "kernel": "gemm_kernel<e4m3,e4m3,GEGLU,bf16> (gate/up GEMM + gated-GELU epilogue)",
        "bound": "mfma",
        "achieved": round(achieved, 1),
        "peak": FP8_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
        "traffic": traffic.get("bytes_per_launch") if traffic else None,
        "flop_per_launch": geglu_flop,
        "avg_launch_us": round(geglu_s * 1e6, 2),
    }

    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(c, reps=args.cpu_reps)

    line = {
        "metric": METRIC,
        "value": round(flop / sec / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded randn, BASELINE config 2)",
        "config": {"workload": "c2 gated-GELU MLP fwd, FP8 current scaling",
                   "M": M, "hidden": K, "intermediate": I, "parallelism": "none (1 GPU)"},
        "frac_of_fp8_peak": round(flop / sec / 1e12 / FP8_PEAK_TFLOPS, 4),
        "value_cached_weights": round(flop / sec_cached / 1e12, 2),
        "kernels": {
            "gemm_geglu_us": round(geglu_s * 1e6, 2),
            "gemm_geglu_tflops": round(achieved, 1),
            "gemm_down_us": round(down_s * 1e6, 2),
            "gemm_down_tflops": round(2.0 * M * K * I / down_s / 1e12, 1),
            "quantize_x_us": round(qx_s * 1e6, 2),
            "quantize_x_gbps": round(3.0 * M * K / qx_s / 1e9, 1),
            "cast_h_us": round(qh_s * 1e6, 2),
            "cast_h_gbps": round(3.0 * M * I / qh_s / 1e9, 1),
            "quantize_wgu_us": round(qw_s * 1e6, 2),
            "quantize_wgu_gbps": round(3.0 * 2 * I * K / qw_s / 1e9, 1),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _cpu_baseline(c, reps=1):
    """Time the CPU oracle's c2 step (fp32 emulated matmuls) on this host's cores."""
    import torch

    from oracle import fp8_oracle as orc

    cores = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(cores)
    x, wg, wu, wd = c["x"], c["w_gate"], c["w_up"], c["w_down"]
    M = x.shape[0]
    K, I = wg.shape[1], wg.shape[0]
    orc.mlp_forward(x[:64], wg[:256], wu[:256], wd[:, :256], precise=False)  # warm-up
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.mlp_forward(x, wg, wu, wd, precise=False)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    flop = 2.0 * M * (2 * I * K + K * I)
    return {"value": round(flop / best / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
            "kind": "port",
            "sample": f"one full c2 step (M={M}) of the CPU oracle: torch CPU amax/clamp/"
                      f".to(float8) for X, W_gate||W_up, W_down and H, fp32 emulated "
                      f"matmuls, bf16 gelu chain; {best:.2f} s, best of {reps}"}


if __name__ == "__main__":
    main()
