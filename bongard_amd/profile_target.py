"""Profiling target: launches the FP8 path's kernels a few times at BASELINE config-2 size.

Run under rocprofv3 (kernel trace or PMC counters). Besides the FP8 kernels it launches a
plain device-to-device copy of a known byte count, the calibration that turns the
FETCH_SIZE / WRITE_SIZE counters into bytes.

    python -m bongard_amd.profile_target [--iters N] [--rows M] [--case c2|square]

``c2``: the whole config-2 MLP forward (quantize X and weights, gate/up GEMM + gated-GELU
epilogue, H scale + cast, down GEMM). ``square``: one 8192^3 e4m3 GEMM, the steady-state
main loop with no epilogue-heavy work. ``recipes``: the kernels of the other recipes and
the fused norm: the config-2 MLP forward under MXFP8 (block quantize, MX gated-GELU GEMM with H
quantized in its epilogue, MX down GEMM), the axiswise (torchao rowwise) quantization of a [8192, 2560] activation
per row and per column, the fused RMSNorm of the same activation, and the config-2 MLP
forward under NVFP4 (block quantize, exact dequantization, bf16 MFMA GEMMs, elementwise
gated GELU). ``c5``: the
config-5 training step (the c2 MLP at M = 8192, forward and backward, delayed scaling with
an amax history of 16). ``vs_hipblaslt``: this library's FP8 GEMM and hipBLASLt's (through
``torch._scaled_mm``) on the c2 / c4 / square shapes, each captured as a HIP graph of 20
calls and timed from HIP events around its replay; prints one line per shape.
``vs_hipblaslt_eager``: the same two libraries on 8192^3 and the c2 down shape, a few eager
calls each (for per-dispatch PMC counters). ``c4``: the
config-4 decoder-branch step at M = 512 on pre-quantized weights (current-scaling quantize
of the branch input and the attention output, fused QKV with three segment scales, O,
gate/up + gated GELU, H cast, down), captured as one HIP graph and replayed.
"""

import argparse

import torch

from . import ops, workloads

COPY_BYTES = 256 << 20


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--iters", type=int, default=5)
    p.add_argument("--rows", type=int, default=4096)
    p.add_argument("--case", choices=("c2", "square", "recipes", "c5", "vs_hipblaslt", "c4",
                                      "vs_hipblaslt_eager"),
                   default="c2")
    args = p.parse_args()
    dev = torch.device("cuda:0")
    if args.case == "square":
        g = torch.Generator(device=dev).manual_seed(0)
        a = torch.randn(8192, 8192, device=dev, generator=g).to(torch.bfloat16)
        b = (torch.randn(8192, 8192, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        aq, bq = ops.quantize(a), ops.quantize(b)
        for _ in range(args.iters):
            ops.gemm(aq.data, ops.E4M3, aq.meta, bq.data, ops.E4M3, bq.meta)
        torch.cuda.synchronize()
        print(f"profile_target done: {args.iters} x 8192^3 GEMM", flush=True)
        return
    if args.case == "recipes":
        _recipes(dev, args.iters)
        return
    if args.case == "c5":
        _c5(dev, args.iters)
        return
    if args.case == "vs_hipblaslt_eager":
        _vs_hipblaslt_eager(dev, args.iters)
        return
    if args.case == "vs_hipblaslt":
        _vs_hipblaslt(dev, args.iters)
        return
    if args.case == "c4":
        _c4(dev, args.iters)
        return
    c = workloads.config2(rows=args.rows)
    I = workloads.INTERMEDIATE
    x = c["x"].to(dev)
    w_gu = torch.cat([c["w_gate"], c["w_up"]], 0).to(dev)
    w_d = c["w_down"].to(dev)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.iters):
        dst.copy_(src)
        xq, gq, dq = ops.quantize_many([x, w_gu, w_d])
        H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
        hq = ops.cast_partials(H, hparts, ops.E4M3)
        hm = hq.meta
        ops.gemm(hq.data, ops.E4M3, hm, dq.data, ops.E4M3, dq.meta)
    torch.cuda.synchronize()
    print(f"profile_target done: {args.iters} iterations, copy {COPY_BYTES} bytes", flush=True)


def _graph_time(fn, n=20, reps=5):
    """Seconds per call of ``fn``: n calls captured in one HIP graph, median of reps replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            fn()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / 1e3 / n)
    return sorted(ts)[len(ts) // 2]


def _c4(dev, iters):
    c = workloads.config4()
    x = c["x"].to(dev)
    I = c["w_gate"].shape[0]
    g = torch.Generator().manual_seed(44)
    attn = torch.randn(x.shape[0], c["w_o"].shape[1], generator=g).to(torch.bfloat16).to(dev)
    metas = ops.new_meta(dev, 3)
    rows = [c["w_q"].shape[0], c["w_k"].shape[0], c["w_v"].shape[0]]
    w8 = torch.empty(sum(rows), x.shape[1], dtype=torch.float8_e4m3fn, device=dev)
    start = 0
    for i, name in enumerate(("w_q", "w_k", "w_v")):
        ops.quantize(c[name].to(dev), ops.E4M3, meta=metas[i], out=w8[start:start + rows[i]])
        start += rows[i]
    ends = [rows[0], rows[0] + rows[1], sum(rows)]
    oq = ops.quantize(c["w_o"].to(dev), ops.E4M3)
    gq = ops.quantize(torch.cat([c["w_gate"], c["w_up"]]).to(dev), ops.E4M3)
    dq = ops.quantize(c["w_down"].to(dev), ops.E4M3)

    def step():
        xq, aq = ops.quantize_many([x, attn])
        ops.gemm(xq.data, 0, xq.meta, w8, 0, metas[0], seg_ends=ends, b_meta_stride=4)
        ops.gemm(aq.data, 0, aq.meta, oq.data, 0, oq.meta)
        H, _, hp = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, I)
        hq = ops.cast_partials(H, hp, ops.E4M3)
        return ops.gemm(hq.data, 0, hq.meta, dq.data, 0, dq.meta)

    t = _graph_time(step, n=max(iters, 1))
    print(f"profile_target done: c4 step {t * 1e6:.2f} us (graph-replayed)", flush=True)


def _vs_hipblaslt(dev, iters):
    meta = torch.tensor([1.0, 1.0, 1.0, 0.0], device=dev)
    one = torch.tensor(1.0, device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)

    def rnd(r, c):  # finite e4m3 bytes
        v = torch.randint(0, 0x70, (r, c), dtype=torch.int16, device=dev, generator=gen)
        return v.to(torch.uint8).view(torch.float8_e4m3fn)

    for M, N, K in [(512, 4096, 2560), (512, 2560, 2048), (512, 2560, 10240),
                    (512, 20480, 2560), (4096, 20480, 2560), (4096, 2560, 10240),
                    (8192, 8192, 8192)]:
        a, b = rnd(M, K), rnd(N, K)
        bt = b.t()

        def lt():
            return torch._scaled_mm(a, bt, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)

        def ours():
            return ops.gemm(a, ops.E4M3, meta, b, ops.E4M3, meta)

        for _ in range(iters):
            lt()
            ours()
        t_lt, t_ours = _graph_time(lt), _graph_time(ours)
        f = 2.0 * M * N * K
        print(f"{M}x{N}x{K}: hipBLASLt {t_lt * 1e6:8.2f} us {f / t_lt / 1e12:6.0f} TFLOP/s   "
              f"bf8_gemm {t_ours * 1e6:8.2f} us {f / t_ours / 1e12:6.0f} TFLOP/s", flush=True)


def _vs_hipblaslt_eager(dev, iters):
    """hipBLASLt (torch._scaled_mm) and bf8_gemm on 8192^3 and the c2 down shape, ``iters``
    eager calls each (no graphs): a target for PMC counters per dispatch."""
    meta = torch.tensor([1.0, 1.0, 1.0, 0.0], device=dev)
    one = torch.tensor(1.0, device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    for M, N, K in [(8192, 8192, 8192), (4096, 2560, 10240)]:
        v = torch.randint(0, 0x70, (M, K), dtype=torch.int16, device=dev, generator=gen)
        a = v.to(torch.uint8).view(torch.float8_e4m3fn)
        v = torch.randint(0, 0x70, (N, K), dtype=torch.int16, device=dev, generator=gen)
        b = v.to(torch.uint8).view(torch.float8_e4m3fn)
        for _ in range(iters):
            torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
            ops.gemm(a, ops.E4M3, meta, b, ops.E4M3, meta)
    torch.cuda.synchronize()
    print(f"profile_target done: {iters} x hipBLASLt and bf8_gemm on two shapes", flush=True)


def _c5(dev, iters):
    from . import linear, scaling

    c = workloads.config5()
    x = c["x"].to(dev).requires_grad_(True)
    dy = c["dy"].to(dev)
    I = c["w_gate"].shape[0]
    w_gu = torch.cat([c["w_gate"], c["w_up"]]).to(dev).requires_grad_(True)
    w_d = c["w_down"].to(dev).requires_grad_(True)
    sc = (scaling.LinearScaling(c["history"]), scaling.LinearScaling(c["history"]))
    for _ in range(iters):
        x.grad = w_gu.grad = w_d.grad = None
        y = linear.Fp8GegluMlpFunction.apply(x, w_gu, w_d, None, None, I, False, sc)
        y.backward(dy)
    torch.cuda.synchronize()
    print(f"profile_target done: {iters} c5 training steps", flush=True)


def _recipes(dev, iters):
    c = workloads.config2()
    I = workloads.INTERMEDIATE
    x = c["x"].to(dev)
    w_gu = torch.cat([c["w_gate"], c["w_up"]], 0).to(dev)
    w_d = c["w_down"].to(dev)
    a = workloads.config5()["x"].to(dev)
    gamma = torch.zeros(a.shape[1], dtype=torch.bfloat16, device=dev)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
        xq, gq, dq = ops.quantize_mx(x), ops.quantize_mx(w_gu), ops.quantize_mx(w_d)
        hq, _, _ = ops.gemm_geglu_mx_quant(xq.data, xq.scales, gq.data, gq.scales, I)
        ops.gemm_mx(hq.data, hq.scales, dq.data, dq.scales)
        ops.quantize_axiswise(a, ops.E4M3, rowwise=True, colwise=True)
        ops.rmsnorm(a, gamma, 1e-6)
        # NVFP4 as the modules run it: X and H written as their bf16 dequantization, H's
        # amax from the gate/up epilogue's partials, the weights quantized per iteration
        xn = ops.quantize_nvfp4(x, dequant_rows=True)
        gn, dn = ops.quantize_nvfp4(w_gu), ops.quantize_nvfp4(w_d)
        H, _, hp = ops.gemm_geglu_nvfp4(None, None, xn.meta, gn.data, gn.scales, gn.meta, I,
                                        a_deq=ops.nvfp4_dequant(xn))
        hn = ops.quantize_nvfp4(H, partials=hp, dequant_rows=True)
        ops.gemm_nvfp4(None, None, hn.meta, dn.data, dn.scales, dn.meta,
                       a_deq=ops.nvfp4_dequant(hn))
    torch.cuda.synchronize()
    print(f"profile_target done: {iters} iterations (recipes), copy {COPY_BYTES} bytes", flush=True)


if __name__ == "__main__":
    main()
