"""Shared checks of the GPU parity tests (imported by tests/test_gpu_*.py).

The bars (north star of BASELINE.json):
  * FP8 bytes, amax, scale and scale_inv: bit-exact against the oracle on the same input;
  * a GEMM's fp32 output against the oracle's dequantized matmul of the SAME fp8 operands
    (bytes and scales): max |err| <= 1% of the output RMS; its bf16 output is the RNE
    rounding of that fp32 output;
  * the gated GELU on the kernel's own bf16 pre-activations: bit-exact.
Large outputs are compared on a sample of rows (every element of a row depends only on
that row of A), so the fp64 reference stays cheap at the BASELINE sizes.
"""

import torch

from oracle import fp8_oracle as orc

RMS_TOL = 0.01


def rms(t):
    return t.double().pow(2).mean().sqrt().item()


def sample_rows(M, n=384, seed=0):
    """Sorted row indices: the first and last 32 rows (tile and tensor edges) and n random
    rows in between (all rows when M is small)."""
    if M <= n + 64:
        return torch.arange(M)
    g = torch.Generator().manual_seed(seed)
    mid = torch.randperm(M - 64, generator=g)[:n] + 32
    return torch.unique(torch.cat([torch.arange(32), mid, torch.arange(M - 32, M)]))


def assert_fp32_close(got, ref, tol=RMS_TOL, what="gemm"):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs().max().item()
    r = rms(ref)
    print(f"[{what}] max|err|/RMS = {err / max(r, 1e-30):.3e}", flush=True)
    assert err <= tol * r, f"{what}: max|err| {err:.3e} > {tol} * RMS {r:.3e}"
    return err / max(r, 1e-30)


def assert_bf16_near(got16, ref_f32, what, tol=1e-3):
    """bf16 GEMM output against the fp64 GEMM: half an ulp of rounding plus an fp32
    accumulation error of at most tol * RMS."""
    got, ref = got16.float().cpu(), ref_f32.float().cpu()
    r = rms(ref)
    excess = (got - ref).abs() - 0.5 * orc.bf16_ulp(ref)
    worst = excess.max().item() / max(r, 1e-30)
    print(f"[{what}] max(|err| - ulp/2)/RMS = {worst:.3e}", flush=True)
    assert worst <= tol, what


def assert_bits_equal(got, want, what):
    g = got.cpu().contiguous().view(torch.int16 if got.element_size() == 2 else torch.uint8)
    w = want.cpu().contiguous().view(torch.int16 if want.element_size() == 2 else torch.uint8)
    assert g.shape == w.shape, f"{what}: shape {tuple(g.shape)} != {tuple(w.shape)}"
    n = int((g != w).sum())
    assert n == 0, f"{what}: {n} of {g.numel()} elements differ"


def assert_quantized_like_oracle(q_data, q_meta, x_cpu, fmt, what, data_t=None):
    """Bytes (and the transposed copy) and meta of a current-scaling quantization of x."""
    rq, ra, rs, rsi = orc.quantize(x_cpu, fmt)
    m = q_meta.float().cpu()
    assert m[0].item() == ra.item() or (m[0].isnan() and ra.isnan()), f"{what}: amax"
    assert m[1].item() == rs.item() and m[2].item() == rsi.item(), f"{what}: scale"
    if q_data is not None:
        assert_bits_equal(q_data.view(torch.uint8), rq, f"{what} bytes")
    if data_t is not None:
        assert_bits_equal(data_t.view(torch.uint8), rq.t().contiguous(), f"{what} transposed")
    return rq, rs


def dequant_mm_rows(aq, a_scale, a_fmt, bq, b_scale, b_fmt, rows, **kw):
    """The oracle's fp64 dequantized matmul restricted to rows of A (fp32 result)."""
    return orc.scaled_mm(aq[rows], a_scale, a_fmt, bq, b_scale, b_fmt, **kw)


def gemm_matches_oracle_on_own_operands(out32, a8, a_meta, a_fmt, b8, b_meta, b_fmt, what,
                                        rows=None, out16=None, **kw):
    """The GEMM output (fp32) against the oracle's matmul of the kernel's own operands."""
    a = a8.view(torch.uint8).cpu()
    b = b8.view(torch.uint8).cpu()
    sa = a_meta.float().cpu()[1]
    sb = b_meta.float().cpu()[1]
    rows = torch.arange(a.shape[0]) if rows is None else rows
    ref = dequant_mm_rows(a, sa, a_fmt, b, sb, b_fmt, rows, **kw)
    rel = assert_fp32_close(out32.cpu()[rows], ref, what=what)
    if out16 is not None:
        want = out32.cpu()[rows].to(torch.bfloat16)
        assert_bits_equal(out16.cpu()[rows], want, f"{what}: bf16 = RNE(fp32)")
    return rel
