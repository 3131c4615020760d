"""Benchmark of the MI355X FP8 linear path (one JSON line on stdout).

Headline workload ("c2"): the fused gated-GELU MLP at
Gemma-3-4B width, X bf16 [4096, 2560], W_gate/W_up [10240, 2560], W_down [2560, 10240].
One step is the whole FP8 forward with inputs resident in HBM:
  quantize X, [W_gate; W_up], W_down (amax -> scale -> e4m3 cast, per tensor)
  gate/up GEMM with the gated-GELU epilogue (+ per-tile amax of H)
  H e4m3 cast, down GEMM -> Y bf16 [4096, 2560]
``value`` = 2*M*(2I*K + K*I) FLOP per step / step time (TFLOP/s). Weight quantization is
inside the step (the first-microbatch case); the cached-weight rate is reported beside it.
The step is timed twice: launched eagerly from Python, and captured once as a HIP graph
and replayed (the form a training loop gets from stream capture); the graph replay's
output must equal an eager step's bit for bit to count. ``value`` is the faster of the two
(``timing`` names it; ``value_eager`` and ``value_graph`` are both reported). Before any
timing the step runs ``PREWARM_STEPS`` times untimed (besides the W warmup steps): the
first steps of a fresh process pay lazy code-object loads and allocator growth.

``roofline`` covers the dominant kernel (gate/up GEMM + gated-GELU epilogue): algorithmic
FLOP per launch / its average launch time from HIP events on the launch stream, against
the dense FP8 MFMA peak. ``traffic`` comes from rocprofv3 FETCH_SIZE/WRITE_SIZE runs
summarised in profiles/ (null when no such summary exists). The rocprofv3 kernel-trace
summary in profiles/ is taken with ``--only-c2``, so that the kernel's name covers the c2
shape alone and its average duration is comparable with ``avg_launch_us``.
``quantize_roofline`` does the same for the H cast against HBM bandwidth, with cold
caches: the cast rotates over enough H-sized buffers (> 2x the 256 MB MALL) that no input
is cache resident; ``copy_gbps`` is the same box's rate for a plain device copy, and
``quantize_current_scaling`` the amax + cast of W_gate||W_up (cold) counted at 3 B/elem.

``configs`` reports the other BASELINE configurations, each timed the same way:
  c1  one FP8 linear, X [512, 2560] (8 outlier columns) . W [2048, 2560]^T, both quantized
  c3  an encoder layer's linears on a packed varlen batch (M = sum of 8 lengths ~ 16k):
      fused QKV (3 per-segment scales), O, and the c2 MLP; cached weights
  c4  decoder-branch skinny GEMMs (M = 512) on pre-quantized weights; reports HBM GB/s
      (weights + activations + outputs) against peak as well as TFLOP/s
  c5  FP8 training step of the c2 MLP at M = 8192 (forward + backward, grad_out e5m2),
      delayed scaling with an amax history of 16 on every tensor role
and two entries beyond the BASELINE configurations:
  fused_norm  FusedMLP's RMSNorm -> e4m3 fc1 input at [8192, 2560], fused kernel vs torch
  c1_rowwise  c1 under torchao's 'rowwise' recipe (per-row power-of-2 scales), and the
              per-row + per-column quantization of [8192, 2560]
  c2_mxfp8    the c2 MLP forward under TE's 'mxfp8' recipe (block-scaled MFMA)
  c2_nvfp4    the c2 MLP forward under TE's 'nvfp4' recipe (bf16 MFMA on exactly
              dequantized NVFP4 operands, the gated GELU in the gate/up epilogue)
  state_kv    the decoder's state-bank K/V projection of the c3 packed state

``cpu_baseline`` times the CPU oracle (torch CPU: amax, clamp, .to(float8), fp32 matmul,
bf16 gelu chain -- torchao's emulate path) on the same c2 step, on this host's cores.
"""

import argparse
import json
import os
import sys
import time
import types
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA (AMD public spec), no sparsity
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (the NVFP4 recipe's GEMMs)
METRIC = "FP8 linear TFLOP/s & % MFMA peak at 4B shapes; quantize cast GB/s"
PREWARM_STEPS = 20


def _args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--rows", type=int, default=4096)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only-c2", action="store_true", help="skip the other configurations")
    return p.parse_args()


def _load_traffic():
    f = ROOT / "profiles" / "traffic_gemm_geglu_c2.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text())
    except (OSError, ValueError):
        return None


def _timed(torch, fn, steps, warmup):
    """Wall time per call of ``fn`` between two device synchronisations."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _graph_timed(torch, fn, steps, warmup, per_graph=1):
    """(seconds per call, verified) for ``fn`` captured as a HIP graph of ``per_graph``
    back-to-back calls and replayed ``steps`` times.

    Several calls per graph keep the host's graph-launch cost out of the figure for steps
    of a few microseconds (the device time is what is measured). The replay's (last) output
    must equal an eager call's bit for bit, else the time is not used.
    """
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            out = fn()
    eager = fn().clone()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    ok = torch.equal(out.view(torch.int16), eager.view(torch.int16))
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps / per_graph, ok


# Calls per captured graph for the few-microsecond steps (c1, c4): device time without the
# host's per-replay launch cost.
GRAPH_CALLS = 20


def _first(out):
    """The first tensor of an op's result (gemm_geglu returns a tuple)."""
    return out[0] if isinstance(out, tuple) else out


def _ev_time(torch, fn, n):
    """Average time per call from HIP events recorded on the launch stream."""
    stream = torch.cuda.current_stream()
    for _ in range(3):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(n):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / n


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
        if cached is None:
            # x and both weights: one amax launch and one cast launch (as the MLP forward
            # does under current scaling when no transposed copies are needed)
            xq, gq, dq = ops.quantize_many([x, w_gu, w_d])
        else:
            xq = ops.quantize(x, ops.E4M3)
            gq, dq = cached
        H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
        hq = ops.cast_partials(H, hparts, ops.E4M3)
        return ops.gemm(hq.data, ops.E4M3, hq.meta, dq.data, ops.E4M3, dq.meta)

    # pre-warm before any timing (not part of the W warmup steps): the first ~20 steps of a
    # fresh process run slower (lazy code-object loads, allocator growth, clock ramp)
    cached = (ops.quantize(w_gu, ops.E4M3), ops.quantize(w_d, ops.E4M3))
    for _ in range(PREWARM_STEPS):
        step()
        step(cached)
    torch.cuda.synchronize()
    sec_eager = _timed(torch, step, args.steps, args.warmup)
    sec_cached_eager = _timed(torch, lambda: step(cached), args.steps, args.warmup)
    sec_graph, graph_ok = _graph_timed(torch, step, args.steps, args.warmup)
    sec_cached_graph, cached_ok = _graph_timed(torch, lambda: step(cached), args.steps,
                                               args.warmup)
    use_graph = graph_ok and sec_graph < sec_eager
    sec = sec_graph if use_graph else sec_eager
    sec_cached = min(sec_cached_eager, sec_cached_graph if cached_ok else sec_cached_eager)

    # ---- dominant kernel: gate/up GEMM + gated-GELU epilogue, HIP events on its stream
    xq = ops.quantize(x, ops.E4M3)
    gq = cached[0]
    n_launch = max(10, args.steps)
    geglu_s = _ev_time(torch, lambda: ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I),
                       n_launch)
    geglu_flop = 2.0 * M * (2 * I) * K
    achieved = geglu_flop / geglu_s / 1e12

    # ---- down GEMM and the quantize kernels (HBM-bound), same method
    H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
    hq = ops.cast_partials(H, hparts, ops.E4M3)
    hm = hq.meta
    dq = cached[1]
    down_s = _ev_time(torch, lambda: ops.gemm(hq.data, 0, hm, dq.data, 0, dq.meta), n_launch)
    qx_s = _ev_time(torch, lambda: ops.quantize(x, ops.E4M3), n_launch)
    qh_s = _ev_time(torch, lambda: ops.cast(H, hm, ops.E4M3), n_launch)
    qw_s = _ev_time(torch, lambda: ops.quantize(w_gu, ops.E4M3), n_launch)
    amax_w_s = _ev_time(torch, lambda: ops.amax(w_gu), n_launch)
    qmany_s = _ev_time(torch, lambda: ops.quantize_many([x, w_gu, w_d]), n_launch)
    qsep_s = _ev_time(torch, lambda: [ops.quantize(t, ops.E4M3) for t in (x, w_gu, w_d)],
                      n_launch)
    qht_s = _ev_time(torch, lambda: ops.cast(H, hm, ops.E4M3, rowwise=True, transpose=True),
                     n_launch)
    cold = _cold_quantize(torch, ops, H, hm, w_gu, n_launch)

    traffic = _load_traffic()
    roofline = {
        "kernel": "gemm_kernel<256x256 tile of eight waves, e4m3 x e4m3, gated-GELU epilogue> "
                  "(gate/up GEMM)",
        "bound": "mfma",
        "achieved": round(achieved, 1),
        "peak": FP8_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
        "traffic": traffic.get("bytes_per_launch") if traffic else None,
        "flop_per_launch": geglu_flop,
        "avg_launch_us": round(geglu_s * 1e6, 2),
    }
    cast_h_gbps = 3.0 * M * I / qh_s / 1e9
    cold_gbps = 3.0 * M * I / cold["cast_s"] / 1e9
    quant_roofline = {
        "kernel": f"cast_kernel<e4m3> (H [{M}, {I}] bf16 -> e4m3, given scale), cold caches",
        "bound": "hbm", "achieved": round(cold_gbps, 1), "peak": HBM_PEAK_GBPS,
        "unit": "GB/s", "frac": round(cold_gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_launch": 3 * M * I, "avg_launch_us": round(cold["cast_s"] * 1e6, 2),
        "rotation": f"{cold['buffers']} H-sized inputs ({cold['rotation_mb']:.0f} MB) in turn",
        "warm_avg_launch_us": round(qh_s * 1e6, 2),
        "warm_gbps": round(cast_h_gbps, 1),
        "copy_gbps": round(cold["copy_gbps"], 1),
        "frac_of_copy": round(cold_gbps / cold["copy_gbps"], 4),
    }
    quant_cs = {
        "kernel": f"amax_partials_kernel + cast_kernel (W_gate||W_up [{2 * I}, {K}], "
                  "current scaling), cold caches",
        "bytes_per_elem": 3, "avg_us": round(cold["quant_s"] * 1e6, 2),
        "achieved_gbps": round(3.0 * 2 * I * K / cold["quant_s"] / 1e9, 1),
        "frac": round(3.0 * 2 * I * K / cold["quant_s"] / 1e9 / HBM_PEAK_GBPS, 4),
    }

    configs = None
    if not args.only_c2:
        configs = {
            "c1": _bench_c1(torch, ops, workloads, dev),
            "c3": _bench_c3(torch, ops, workloads, dev),
            "c4": _bench_c4(torch, ops, workloads, dev),
            "c5": _bench_c5(torch, workloads, dev),
            "fused_norm": _bench_norm(torch, ops, workloads, dev),
            "c1_rowwise": _bench_c1_rowwise(torch, ops, workloads, dev),
            "c2_mxfp8": _bench_c2_mx(torch, ops, workloads, dev),
            "c2_nvfp4": _bench_c2_nvfp4(torch, ops, workloads, dev),
            "state_kv": _bench_state_kv(torch, workloads, dev),
        }

    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(c, seconds=args.cpu_seconds)

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
        "timing": "HIP graph replay (verified bit-exact against eager)" if use_graph
                  else "eager launches",
        "prewarm_steps": PREWARM_STEPS,
        "value_eager": round(flop / sec_eager / 1e12, 2),
        "value_graph": round(flop / sec_graph / 1e12, 2) if graph_ok else None,
        "graph_replay_bit_exact": bool(graph_ok and cached_ok),
        "value_cached_weights": round(flop / sec_cached / 1e12, 2),
        "value_cached_weights_eager": round(flop / sec_cached_eager / 1e12, 2),
        "kernels": {
            "gemm_geglu_us": round(geglu_s * 1e6, 2),
            "gemm_geglu_tflops": round(achieved, 1),
            "gemm_down_us": round(down_s * 1e6, 2),
            "gemm_down_tflops": round(2.0 * M * K * I / down_s / 1e12, 1),
            "quantize_x_us": round(qx_s * 1e6, 2),
            "quantize_x_gbps": round(3.0 * M * K / qx_s / 1e9, 1),
            "amax_wgu_us": round(amax_w_s * 1e6, 2),
            "amax_wgu_gbps": round(2.0 * 2 * I * K / amax_w_s / 1e9, 1),
            "cast_h_us": round(qh_s * 1e6, 2),
            "cast_h_gbps": round(cast_h_gbps, 1),
            "cast_transpose_h_us": round(qht_s * 1e6, 2),
            "cast_transpose_h_gbps": round(4.0 * M * I / qht_s / 1e9, 1),
            "quantize_wgu_us": round(qw_s * 1e6, 2),
            "quantize_wgu_gbps": round(3.0 * 2 * I * K / qw_s / 1e9, 1),
            "quantize_x_wgu_wd_shared_launches_us": round(qmany_s * 1e6, 2),
            "quantize_x_wgu_wd_separate_us": round(qsep_s * 1e6, 2),
        },
        "roofline": roofline,
        "quantize_roofline": quant_roofline,
        "quantize_current_scaling": quant_cs,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _cold_quantize(torch, ops, H, hm, w, n_launch):
    """Cast of H (given scale) and current-scaling quantize of W with inputs rotated over
    buffers totalling more than twice the 256 MB MALL, so every launch reads from HBM;
    plus a plain device copy of 1 GiB on the same box for reference."""
    mall = 256 << 20
    nh = max(3, -(-2 * mall // (H.numel() * 3)) + 1)
    hs = [H.clone() for _ in range(nh)]
    outs = [torch.empty(H.shape, dtype=torch.float8_e4m3fn, device=H.device) for _ in range(nh)]
    i = [0]

    def cast():
        k = i[0] % nh
        i[0] += 1
        ops.cast(hs[k], hm, ops.E4M3, out=outs[k])

    n = max(n_launch, 2 * nh)
    cast_s = _ev_time(torch, cast, n - n % nh)
    del outs
    nw = max(3, -(-2 * mall // (w.numel() * 3)) + 1)
    ws = [w.clone() for _ in range(nw)]
    j = [0]

    def quant():
        k = j[0] % nw
        j[0] += 1
        ops.quantize(ws[k], ops.E4M3)

    n = max(n_launch, 2 * nw)
    quant_s = _ev_time(torch, quant, n - n % nw)
    del ws, hs
    src = torch.empty(1 << 30, dtype=torch.uint8, device=H.device)
    dst = torch.empty_like(src)
    copy_s = _ev_time(torch, lambda: dst.copy_(src), 20)
    return {"cast_s": cast_s, "quant_s": quant_s, "buffers": nh,
            "rotation_mb": nh * H.numel() * 3 / 1e6, "copy_gbps": 2.0 * src.numel() / copy_s / 1e9}


def _bench_c1(torch, ops, workloads, dev, steps=50):
    """c1: Y = X W^T with both operands quantized each call (TELinear, first microbatch)."""
    c = workloads.config1()
    x, w = c["x"].to(dev), c["w"].to(dev)
    M, K = x.shape
    N = w.shape[0]

    def step():
        xq, wq = ops.quantize_many([x, w])
        return ops.gemm(xq.data, 0, xq.meta, wq.data, 0, wq.meta)

    s = _timed(torch, step, steps, 5)
    s_graph1, graph1_ok = _graph_timed(torch, step, steps, 5)
    s_graph, graph_ok = _graph_timed(torch, step, steps, 5, per_graph=GRAPH_CALLS)
    xq, wq = ops.quantize(x, ops.E4M3), ops.quantize(w, ops.E4M3)
    g, g_ok = _graph_timed(torch, lambda: ops.gemm(xq.data, 0, xq.meta, wq.data, 0, wq.meta),
                           steps, 5, per_graph=GRAPH_CALLS)
    flop = 2.0 * M * N * K
    return {"workload": f"linear [{M},{K}] x [{N},{K}]^T, both quantized per call",
            "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "us_per_step_graph": round(s_graph * 1e6, 2) if graph_ok else None,
            "tflops_graph": round(flop / s_graph / 1e12, 1) if graph_ok else None,
            "us_per_step_graph_one_step_per_replay": (round(s_graph1 * 1e6, 2)
                                                      if graph1_ok else None),
            "gemm_us": round(g * 1e6, 2) if g_ok else None,
            "gemm_tflops": round(flop / g / 1e12, 1) if g_ok else None,
            "note": "eager launches are host-bound at this size (three small kernels from "
                    f"Python); graph figures are device time: {GRAPH_CALLS} steps (or GEMMs) "
                    "per captured graph, so the host's graph-launch cost stays out; one step "
                    "per replay is host-bound on the graph launch"}


def _qkv_weight(torch, ops, c, dev):
    """[W_q; W_k; W_v] in one fp8 buffer with one meta per segment (fused QKV)."""
    parts = [c["w_q"], c["w_k"], c["w_v"]]
    K = parts[0].shape[1]
    n = sum(p.shape[0] for p in parts)
    w8 = torch.empty(n, K, dtype=torch.float8_e4m3fn, device=dev)
    metas = ops.new_meta(dev, 3)
    start, ends = 0, []
    for i, p in enumerate(parts):
        ops.quantize(p.to(dev), ops.E4M3, meta=metas[i], out=w8[start:start + p.shape[0]])
        start += p.shape[0]
        ends.append(start)
    return w8, metas, ends


def _bench_c3(torch, ops, workloads, dev, steps=20):
    """c3: packed varlen encoder layer: fused QKV, O, MLP (cached weights)."""
    c = workloads.config3()
    x = c["x"].to(dev)
    M, K = x.shape
    I = c["w_gate"].shape[0]
    g = torch.Generator().manual_seed(33)
    attn = torch.randn(M, c["w_o"].shape[1], generator=g).to(torch.bfloat16).to(dev)
    # the MLP's input (the post-attention residual stream after its norm): its own tensor
    hmid = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w8, metas, ends = _qkv_weight(torch, ops, c, dev)
    oq = ops.quantize(c["w_o"].to(dev), ops.E4M3)
    gq = ops.quantize(torch.cat([c["w_gate"], c["w_up"]]).to(dev), ops.E4M3)
    dq = ops.quantize(c["w_down"].to(dev), ops.E4M3)

    def step():
        xq = ops.quantize(x, ops.E4M3)
        qkv = ops.gemm(xq.data, 0, xq.meta, w8, 0, metas[0], seg_ends=ends, b_meta_stride=4)
        aq = ops.quantize(attn, ops.E4M3)
        o = ops.gemm(aq.data, 0, aq.meta, oq.data, 0, oq.meta)
        mq = ops.quantize(hmid, ops.E4M3)
        H, _, hp = ops.gemm_geglu(mq.data, mq.meta, gq.data, gq.meta, I)
        hq = ops.cast_partials(H, hp, ops.E4M3)
        y = ops.gemm(hq.data, 0, hq.meta, dq.data, 0, dq.meta)
        return qkv, o, y

    s = _timed(torch, step, steps, 3)
    flop = 2.0 * M * (K * ends[-1] + oq.cols * K + 2 * I * K + I * K)
    return {"workload": f"packed varlen encoder layer, M={M} (8 lengths {c['lengths'].tolist()}): "
                        "fused QKV (3 scales) + O + gated MLP, cached weights; X, the "
                        "attention output, the MLP input and H quantized in the step",
            "M": M, "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "frac_of_fp8_peak": round(flop / s / 1e12 / FP8_PEAK_TFLOPS, 4)}


def _bench_c4(torch, ops, workloads, dev, steps=50):
    """c4: decoder-branch skinny GEMMs at M=512 on pre-quantized weights."""
    c = workloads.config4()
    x = c["x"].to(dev)
    M, K = x.shape
    I = c["w_gate"].shape[0]
    g = torch.Generator().manual_seed(44)
    attn = torch.randn(M, c["w_o"].shape[1], generator=g).to(torch.bfloat16).to(dev)
    w8, metas, ends = _qkv_weight(torch, ops, c, dev)
    oq = ops.quantize(c["w_o"].to(dev), ops.E4M3)
    gq = ops.quantize(torch.cat([c["w_gate"], c["w_up"]]).to(dev), ops.E4M3)
    dq = ops.quantize(c["w_down"].to(dev), ops.E4M3)
    xq = ops.quantize(x, ops.E4M3)
    aq = ops.quantize(attn, ops.E4M3)
    H, _, hp = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
    hq = ops.cast_partials(H, hp, ops.E4M3)
    gemms = {
        "qkv": (lambda: ops.gemm(xq.data, 0, xq.meta, w8, 0, metas[0], seg_ends=ends,
                                 b_meta_stride=4), ends[-1], K, True),
        "o": (lambda: ops.gemm(aq.data, 0, aq.meta, oq.data, 0, oq.meta), K, oq.cols, True),
        "gate_up_geglu": (lambda: ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I),
                          2 * I, K, False),
        "down": (lambda: ops.gemm(hq.data, 0, hq.meta, dq.data, 0, dq.meta), K, I, True),
    }
    out, tot_s, tot_b, tot_f = {}, 0.0, 0.0, 0.0
    all_ok = True
    for name, (fn, N, KK, full_out) in gemms.items():
        t, ok = _graph_timed(torch, lambda fn=fn: _first(fn()), steps, 5, per_graph=GRAPH_CALLS)
        if not ok:   # a replay that differs from eager gives no figure
            out[name] = None
            all_ok = False
            continue
        out_cols = N if full_out else N // 2
        nbytes = N * KK + M * KK + 2 * M * out_cols  # fp8 W + fp8 X + bf16 out
        f = 2.0 * M * N * KK
        out[name] = {"us": round(t * 1e6, 2), "gbps": round(nbytes / t / 1e9, 1),
                     "tflops": round(f / t / 1e12, 1)}
        tot_s += t
        tot_b += nbytes
        tot_f += f
    gbps = tot_b / tot_s / 1e9 if all_ok else None

    # the four GEMMs captured once and replayed: device time without Python's per-call
    # launch cost (eager back-to-back calls of these ~5-30 us kernels are host-bound)
    def all_four():
        outs = [fn() for fn, _, _, _ in gemms.values()]
        return outs[-1]

    s_graph, graph_ok = _graph_timed(torch, all_four, steps, 5, per_graph=GRAPH_CALLS)
    graph_ok = graph_ok and all_ok
    g_gbps = tot_b / s_graph / 1e9 if graph_ok else None

    # the same step with the activations' current-scaling quantization inside it (X, the
    # attention output and H; the weights stay pre-quantized)
    def with_quant():
        xq2, aq2 = ops.quantize_many([x, attn])
        ops.gemm(xq2.data, 0, xq2.meta, w8, 0, metas[0], seg_ends=ends, b_meta_stride=4)
        ops.gemm(aq2.data, 0, aq2.meta, oq.data, 0, oq.meta)
        H2, _, hp2 = ops.gemm_geglu(xq2.data, xq2.meta, gq.data, gq.meta, I)
        hq2 = ops.cast_partials(H2, hp2, ops.E4M3)
        return ops.gemm(hq2.data, 0, hq2.meta, dq.data, 0, dq.meta)

    s_q, q_ok = _graph_timed(torch, with_quant, steps, 5, per_graph=GRAPH_CALLS)
    q_ok = q_ok and all_ok
    q_bytes = tot_b + 3.0 * M * (K + oq.cols + I)   # + X, attention output, H casts
    return {"workload": "decoder-branch GEMMs at M=512 (QKV, O, gate/up+GELU, down), "
                        "pre-quantized e4m3 weights",
            "us_total_graph": round(s_graph * 1e6, 2) if graph_ok else None,
            "us_total_graph_with_activation_quantize": round(s_q * 1e6, 2) if q_ok else None,
            "hbm_gbps_graph_with_activation_quantize":
                round(q_bytes / s_q / 1e9, 1) if q_ok else None,
            "hbm_gbps_graph": round(g_gbps, 1) if graph_ok else None,
            "hbm_frac_graph": round(g_gbps / HBM_PEAK_GBPS, 4) if graph_ok else None,
            "gemms": out, "us_total": round(tot_s * 1e6, 2) if all_ok else None,
            "hbm_gbps": round(gbps, 1) if all_ok else None,
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4) if all_ok else None,
            "tflops": round(tot_f / tot_s / 1e12, 1) if all_ok else None,
            "mfma_frac": round(tot_f / tot_s / 1e12 / FP8_PEAK_TFLOPS, 4) if all_ok else None,
            "note": "arithmetic intensity 600-1000 FLOP/B is above the 625 FLOP/B ridge for "
                    "most of these GEMMs, so the MFMA roof binds before HBM; every figure is "
                    f"device time from graphs of {GRAPH_CALLS} calls (or steps) per replay"}


def _bench_c5(torch, workloads, dev, steps=10):
    """c5: FP8 training step of the c2 MLP at M=8192 with delayed scaling (history 16)."""
    from bongard_amd import linear, scaling

    c = workloads.config5()
    x = c["x"].to(dev)
    dy = c["dy"].to(dev)
    M, K = x.shape
    I = c["w_gate"].shape[0]
    w_gu = torch.cat([c["w_gate"], c["w_up"]]).to(dev).requires_grad_(True)
    w_d = c["w_down"].to(dev).requires_grad_(True)
    sc = (scaling.LinearScaling(c["history"]), scaling.LinearScaling(c["history"]))
    xg = x.requires_grad_(True)

    def step():
        w_gu.grad = None
        w_d.grad = None
        xg.grad = None
        y = linear.Fp8GegluMlpFunction.apply(xg, w_gu, w_d, None, None, I, False, sc)
        y.backward(dy)

    s = _timed(torch, step, steps, 3)
    flop = 3 * 2.0 * M * (2 * I * K + K * I)
    return {"workload": f"c2 MLP training step (fwd + dgrad + wgrad) at M={M}, e4m3 fwd / "
                        f"e5m2 grads, delayed scaling with amax history {c['history']}, "
                        "weights re-quantized every step",
            "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "frac_of_fp8_peak": round(flop / s / 1e12 / FP8_PEAK_TFLOPS, 4)}


def _bench_state_kv(torch, workloads, dev, steps=20):
    """The decoder's state-bank K/V projection (once per decoder layer) on the c3 packed
    state [M, 2560] with cached FP8 k/v weights: the shared-input form (state quantized
    once) against the two separate projection calls of the reference form."""
    from torch import nn

    from bongard_amd import state_kv, te_linear

    c = workloads.config3()
    x = c["x"].to(dev)
    M, K = x.shape
    head_dim = 256

    def proj(w):
        lin = nn.Linear(K, w.shape[0], bias=False)
        lin.weight.data = w.float()
        return te_linear.TELinear([lin], "fp8").to(dev).train()

    att = types.SimpleNamespace(k_proj=proj(c["w_k"]), v_proj=proj(c["w_v"]),
                                k_norm=nn.Identity(), head_dim=head_dim)
    state = x.reshape(1, M, K)

    def shared():
        with torch.no_grad():
            return state_kv.project_state_kv(att, state)

    def separate():
        with torch.no_grad():
            return att.k_proj(state), att.v_proj(state)

    s_sh = _timed(torch, shared, steps, 3)
    s_sep = _timed(torch, separate, steps, 3)
    flop = 2.0 * M * K * (c["w_k"].shape[0] + c["w_v"].shape[0])
    return {"workload": f"k/v projections of a packed state [{M},{K}] on cached FP8 weights",
            "shared_input_us": round(s_sh * 1e6, 2), "separate_calls_us": round(s_sep * 1e6, 2),
            "shared_input_tflops": round(flop / s_sh / 1e12, 1)}


def _bench_c2_mx(torch, ops, workloads, dev, steps=30):
    """The c2 MLP forward under TE's 'mxfp8' recipe: X, [W_gate; W_up], W_down quantized in
    32-element blocks (E8M0 scales), gated-GELU GEMM on the block-scaled MFMA with H
    quantized in blocks in its epilogue, down GEMM (and, for comparison, the same step with
    a separate bf16 H and quantize pass)."""
    c = workloads.config2()
    x = c["x"].to(dev)
    w_gu = torch.cat([c["w_gate"], c["w_up"]]).to(dev)
    w_d = c["w_down"].to(dev)
    M, K = x.shape
    I = c["w_gate"].shape[0]

    def step(fused=True):
        xq, gq, dq = ops.quantize_mx_many([x, w_gu, w_d])   # one launch, as the MX forward
        if fused:  # H quantized in the gate/up GEMM's epilogue (the product path)
            hq, _, _ = ops.gemm_geglu_mx_quant(xq.data, xq.scales, gq.data, gq.scales, I)
        else:
            H, _ = ops.gemm_geglu_mx(xq.data, xq.scales, gq.data, gq.scales, I)
            hq = ops.quantize_mx(H)
        return ops.gemm_mx(hq.data, hq.scales, dq.data, dq.scales)

    for _ in range(PREWARM_STEPS):
        step()
        step(False)
    s = _timed(torch, step, steps, 3)
    s_unfused = _timed(torch, lambda: step(False), steps, 3)
    s_graph, graph_ok = _graph_timed(torch, step, steps, 3)
    xq, gq, dq = ops.quantize_mx(x), ops.quantize_mx(w_gu), ops.quantize_mx(w_d)
    H, _ = ops.gemm_geglu_mx(xq.data, xq.scales, gq.data, gq.scales, I)
    hq = ops.quantize_mx(H)
    g_s = _ev_time(torch, lambda: ops.gemm_geglu_mx(xq.data, xq.scales, gq.data, gq.scales, I),
                   steps)
    gq_s = _ev_time(torch, lambda: ops.gemm_geglu_mx_quant(xq.data, xq.scales, gq.data,
                                                           gq.scales, I), steps)
    d_s = _ev_time(torch, lambda: ops.gemm_mx(hq.data, hq.scales, dq.data, dq.scales), steps)
    h_s = _ev_time(torch, lambda: ops.quantize_mx(H), steps)
    qm_s = _ev_time(torch, lambda: ops.quantize_mx_many([x, w_gu, w_d]), steps)
    qs_s = _ev_time(torch, lambda: [ops.quantize_mx(t) for t in (x, w_gu, w_d)], steps)
    flop = 2.0 * M * (2 * I * K + K * I)
    return {"workload": f"c2 MLP forward [{M},{K}] x [2*{I},{K}] -> [{M},{I}] x [{K},{I}], MXFP8",
            "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "us_per_step_graph": round(s_graph * 1e6, 2) if graph_ok else None,
            "us_per_step_unfused_h": round(s_unfused * 1e6, 2),
            "gemm_geglu_quant_h_us": round(gq_s * 1e6, 2),
            "gemm_geglu_us": round(g_s * 1e6, 2),
            "gemm_geglu_tflops": round(2.0 * M * 2 * I * K / g_s / 1e12, 1),
            "gemm_down_us": round(d_s * 1e6, 2),
            "gemm_down_tflops": round(2.0 * M * K * I / d_s / 1e12, 1),
            "quantize_h_us": round(h_s * 1e6, 2),
            "quantize_h_gbps": round((3.0 * M * I + M * I / 32) / h_s / 1e9, 1),
            "quantize_x_wgu_wd_one_launch_us": round(qm_s * 1e6, 2),
            "quantize_x_wgu_wd_separate_us": round(qs_s * 1e6, 2)}


def _bench_c2_nvfp4(torch, ops, workloads, dev, steps=20):
    """The c2 MLP forward under TE's 'nvfp4' recipe as TEMLP runs it: X, [W_gate; W_up] and
    W_down quantized to NVFP4 (e2m1, 16-blocks, e4m3 block scales, per-tensor scale), each
    GEMM on the bf16 MFMA over the exactly dequantized operands, the gated GELU in the
    gate/up GEMM's epilogue (no [gate | up] stored without grad), H quantized to NVFP4 for
    the down GEMM from the amax partials that epilogue wrote (X and H written as their exact
    bf16 dequantization by the quantizer itself). The unfused step (the linear GEMM, then the elementwise gated GELU over
    the stored [gate | up], bit-identical H) is timed beside it."""
    c = workloads.config2()
    x = c["x"].to(dev)
    w_gu = torch.cat([c["w_gate"], c["w_up"]]).to(dev)
    w_d = c["w_down"].to(dev)
    M, K = x.shape
    I = c["w_gate"].shape[0]

    def q(t):
        return ops.quantize_nvfp4(t, rowwise=True, colwise=False)

    def qd(t, partials=None):
        # an activation whose rowwise copy only feeds the next GEMM: written dequantized
        return ops.quantize_nvfp4(t, rowwise=True, colwise=False, partials=partials,
                                  dequant_rows=True)

    def step():
        xq, gq, dq = qd(x), q(w_gu), q(w_d)
        H, _, hp = ops.gemm_geglu_nvfp4(None, None, xq.meta, gq.data, gq.scales, gq.meta, I,
                                        a_deq=ops.nvfp4_dequant(xq))
        hq = qd(H, hp)
        return ops.gemm_nvfp4(None, None, hq.meta, dq.data, dq.scales, dq.meta,
                              a_deq=ops.nvfp4_dequant(hq))

    def step_unfused():
        xq, gq, dq = q(x), q(w_gu), q(w_d)
        GU = ops.gemm_nvfp4(xq.data, xq.scales, xq.meta, gq.data, gq.scales, gq.meta)
        H, _ = ops.geglu(GU)
        hq = q(H)
        return ops.gemm_nvfp4(hq.data, hq.scales, hq.meta, dq.data, dq.scales, dq.meta)

    gc, dc = q(w_gu), q(w_d)
    gc.cache_dequant = dc.cache_dequant = True

    def step_cached():
        # weights cached across microbatches (TEMLP / FusedMLP): quantized and dequantized
        # once, their bf16 operands kept
        xq = qd(x)
        H, _, hp = ops.gemm_geglu_nvfp4(None, None, xq.meta, gc.data, gc.scales, gc.meta, I,
                                        a_deq=ops.nvfp4_dequant(xq),
                                        b_deq=ops.nvfp4_dequant(gc))
        hq = qd(H, hp)
        return ops.gemm_nvfp4(None, None, hq.meta, dc.data, dc.scales, dc.meta,
                              a_deq=ops.nvfp4_dequant(hq), b_deq=ops.nvfp4_dequant(dc))

    for _ in range(5):
        step()
        step_unfused()
        step_cached()
    s = _timed(torch, step, steps, 3)
    su = _timed(torch, step_unfused, steps, 3)
    sc = _timed(torch, step_cached, steps, 3)
    xq, gq, dq = q(x), q(w_gu), q(w_d)
    xb, gb = ops.dequant_nvfp4(xq.data, xq.scales), ops.dequant_nvfp4(gq.data, gq.scales)
    GU = ops.gemm_bf16(xb, gb, xq.meta[2:3], gq.meta[2:3])
    H, _ = ops.geglu(GU)
    hq = q(H)
    hb, db = ops.dequant_nvfp4(hq.data, hq.scales), ops.dequant_nvfp4(dq.data, dq.scales)
    gu_s = _ev_time(torch, lambda: ops.gemm_bf16(xb, gb, xq.meta[2:3], gq.meta[2:3]), steps)
    gg_s = _ev_time(torch, lambda: ops.gemm_geglu_bf16(xb, gb, xq.meta[2:3], gq.meta[2:3], I),
                    steps)
    d_s = _ev_time(torch, lambda: ops.gemm_bf16(hb, db, hq.meta[2:3], dq.meta[2:3]), steps)
    qh_s = _ev_time(torch, lambda: q(H), steps)
    dqh_s = _ev_time(torch, lambda: ops.dequant_nvfp4(hq.data, hq.scales), steps)
    gl_s = _ev_time(torch, lambda: ops.geglu(GU), steps)
    flop = 2.0 * M * (2 * I * K + K * I)
    nh = M * I
    return {"workload": f"c2 MLP forward [{M},{K}] x [2*{I},{K}] -> [{M},{I}] x [{K},{I}], NVFP4 "
                        "(bf16 MFMA on exactly dequantized operands, gated GELU in the gate/up "
                        "epilogue)",
            "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "us_per_step_unfused_geglu": round(su * 1e6, 2),
            "us_per_step_cached_weights": round(sc * 1e6, 2),
            "tflops_cached_weights": round(flop / sc / 1e12, 1),
            "gemm_gate_up_geglu_bf16_us": round(gg_s * 1e6, 2),
            "gemm_gate_up_geglu_frac_of_bf16_peak": round(2.0 * M * 2 * I * K / gg_s / 1e12
                                                          / BF16_PEAK_TFLOPS, 4),
            "gemm_gate_up_bf16_us": round(gu_s * 1e6, 2),
            "gemm_gate_up_bf16_tflops": round(2.0 * M * 2 * I * K / gu_s / 1e12, 1),
            "gemm_gate_up_frac_of_bf16_peak": round(2.0 * M * 2 * I * K / gu_s / 1e12
                                                    / BF16_PEAK_TFLOPS, 4),
            "gemm_down_bf16_us": round(d_s * 1e6, 2),
            "gemm_down_bf16_tflops": round(2.0 * M * K * I / d_s / 1e12, 1),
            "geglu_elementwise_us": round(gl_s * 1e6, 2),
            "geglu_elementwise_gbps": round(6.0 * nh / gl_s / 1e9, 1),
            "quantize_h_us": round(qh_s * 1e6, 2),
            "quantize_h_gbps": round((4.0 + 0.5 + 1 / 16) * nh / qh_s / 1e9, 1),
            "dequant_h_us": round(dqh_s * 1e6, 2),
            "dequant_h_gbps": round((2.0 + 0.5 + 1 / 16) * nh / dqh_s / 1e9, 1)}


def _bench_c1_rowwise(torch, ops, workloads, dev, steps=50):
    """c1 under torchao's 'rowwise' recipe: per-row power-of-2 scales for X and W, the GEMM
    with a scale vector on each side; plus the per-column (transposed) quantization of the
    c5 activation [8192, 2560] that the recipe's wgrad needs."""
    c = workloads.config1()
    x, w = c["x"].to(dev), c["w"].to(dev)
    M, K = x.shape
    N = w.shape[0]

    def step():
        xq = ops.quantize_axiswise(x, ops.E4M3)
        wq = ops.quantize_axiswise(w, ops.E4M3)
        return ops.gemm_axiswise(xq.data, 0, xq.row_sinv, wq.data, 0, wq.row_sinv)

    s = _timed(torch, step, steps, 5)
    s_graph, graph_ok = _graph_timed(torch, step, steps, 5, per_graph=GRAPH_CALLS)
    xq, wq = ops.quantize_axiswise(x, ops.E4M3), ops.quantize_axiswise(w, ops.E4M3)
    gs, _ok = _graph_timed(torch, lambda: ops.gemm_axiswise(xq.data, 0, xq.row_sinv, wq.data, 0,
                                                            wq.row_sinv), steps, 5,
                           per_graph=GRAPH_CALLS)
    flop = 2.0 * M * N * K
    a = workloads.config5()["x"].to(dev)
    R, C = a.shape
    both = _ev_time(torch, lambda: ops.quantize_axiswise(a, ops.E4M3, colwise=True), steps)
    rows_only = _ev_time(torch, lambda: ops.quantize_axiswise(a, ops.E4M3), steps)
    return {"workload": f"linear [{M},{K}] x [{N},{K}]^T, axiswise (rowwise recipe) per call",
            "us_per_step": round(s * 1e6, 2), "tflops": round(flop / s / 1e12, 1),
            "us_per_step_graph": round(s_graph * 1e6, 2) if graph_ok else None,
            "gemm_us": round(gs * 1e6, 2), "gemm_tflops": round(flop / gs / 1e12, 1),
            "quantize_rows_8192x2560_us": round(rows_only * 1e6, 2),
            "quantize_rows_gbps": round(3.0 * R * C / rows_only / 1e9, 1),
            "quantize_rows_and_cols_8192x2560_us": round(both * 1e6, 2),
            "quantize_rows_and_cols_gbps": round(4.0 * R * C / both / 1e9, 1)}


def _bench_norm(torch, ops, workloads, dev, steps=50):
    """FusedMLP's norm -> e4m3 input of fc1 at the c5 shape: the fused RMSNorm (which writes
    the amax partials of its output) + cast from those partials, against the same norm in
    torch ops + the two-pass quantize. Both cast rowwise only: the training backward reads
    the fc1 input's fp8 bytes as a K-major operand, so no transposed copy is made."""
    from bongard_amd import fused_mlp

    c = workloads.config5()
    x = c["x"].to(dev)
    M, K = x.shape
    g = torch.Generator(device=dev).manual_seed(3)
    w = (torch.randn(K, device=dev, generator=g) * 0.1).to(torch.bfloat16)

    def fused():
        y, _, parts = ops.rmsnorm(x, w, 1e-6)
        return ops.cast_partials(y, parts, ops.E4M3, rowwise=True, transpose=False)

    def unfused():
        y = fused_mlp._rms_norm(x, w, 1e-6)
        return ops.quantize(y, ops.E4M3, rowwise=True, transpose=False)

    a, b = fused(), unfused()
    torch.cuda.synchronize()
    # the norms' means are summed in different orders (fp64 vs torch's fp32), so a rare
    # element may round to the neighbouring bf16 and then e4m3 value
    flips = (a.data.view(torch.uint8) != b.data.view(torch.uint8)).float().mean().item()
    s_f = _timed(torch, fused, steps, 5)
    s_u = _timed(torch, unfused, steps, 5)
    s_n = _ev_time(torch, lambda: ops.rmsnorm(x, w, 1e-6), steps)
    gbps = 4.0 * M * K / s_n / 1e9
    return {"workload": f"RMSNorm [{M},{K}] bf16 -> e4m3 (rowwise, as training casts it)",
            "fused_us": round(s_f * 1e6, 2), "torch_norm_then_quantize_us": round(s_u * 1e6, 2),
            "rmsnorm_kernel_us": round(s_n * 1e6, 2), "rmsnorm_kernel_gbps": round(gbps, 1),
            "rmsnorm_kernel_frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
            "fp8_bytes_differing_from_torch_norm_path": flips}


def _cpu_baseline(c, seconds=10.0):
    """Time the CPU oracle's c2 step (fp32 emulated matmuls) on this host's cores: whole
    steps repeated for about ``seconds`` of CPU work (at least one), median reported."""
    import torch

    from oracle import fp8_oracle as orc

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    x, wg, wu, wd = c["x"], c["w_gate"], c["w_up"], c["w_down"]
    M = x.shape[0]
    K, I = wg.shape[1], wg.shape[0]
    orc.mlp_forward(x[:64], wg[:256], wu[:256], wd[:, :256], precise=False)  # warm-up
    times = []
    start = time.perf_counter()
    while not times or (time.perf_counter() - start < seconds and len(times) < 100):
        t0 = time.perf_counter()
        orc.mlp_forward(x, wg, wu, wd, precise=False)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    flop = 2.0 * M * (2 * I * K + K * I)
    return {"value": round(flop / med / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
            "kind": "port",
            "sample": f"full c2 steps (M={M}) of the CPU oracle: torch CPU amax/clamp/"
                      f".to(float8) for X, W_gate||W_up, W_down and H, fp32 emulated "
                      f"matmuls, bf16 gelu chain; median {med:.2f} s of {len(times)} steps "
                      f"({sum(times):.1f} s of CPU work)"}


if __name__ == "__main__":
    main()
