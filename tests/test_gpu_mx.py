"""GPU parity of the MXFP8 path (TE MXFP8BlockScaling arithmetic) against the CPU oracle.

  * quantize: fp8 bytes and E8M0 scale rows (padding bytes included) bit-exact against
    oracle.quantize_mx, blocks along rows and (transposed) along columns;
  * block-scaled GEMM: fp32 output within 1% of RMS of the oracle's fp64 dequantized
    matmul, bf16 output the RNE rounding of the same kernel's fp32 output;
  * gated-GELU GEMM on MX operands: bf16 pre-activations within 0.1% RMS (after half an
    ulp) of the fp64 GEMMs, and H within 2 bf16 ulps of the gelu chain on its own g, u.
"""

import pytest
import torch

from bongard_amd import ops
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _rms(t):
    return t.double().pow(2).mean().sqrt().item()


def _x(rows, cols, seed, spread=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g)
    if spread and rows >= 8 and cols >= 64:
        x *= torch.logspace(-6, 6, rows)[:, None]       # many binades across rows
        x[:, 5] *= 300.0                                 # an outlier column
        x[3, 32:64] = 0.0                                # an all-zero block
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(32, 32), (64, 2560), (96, 4096), (4096, 2560),
                                       (160, 10240), (32, 48)])
@pytest.mark.parametrize("fmt", [ops.E4M3, ops.E5M2])
def test_quantize_mx_bit_exact(gpu, rows, cols, fmt):
    x = _x(rows, cols, rows + cols + fmt)
    rowwise = cols % 32 == 0
    q = ops.quantize_mx(x.to(gpu), fmt, rowwise=rowwise, colwise=True)
    torch.cuda.synchronize()
    if rowwise:
        rq, re = orc.quantize_mx(x, fmt, -1)
        same_q = torch.equal(q.data.view(torch.uint8).cpu(), rq)
        same_s = torch.equal(q.scales.cpu(), orc.mx_scale_rows(re))
        print(f"[mx rows {rows}x{cols} fmt {fmt}] bytes {same_q} scales {same_s}", flush=True)
        assert same_q and same_s
    cq, ce = orc.quantize_mx(x, fmt, 0)
    same_q = torch.equal(q.data_t.view(torch.uint8).cpu(), cq)
    same_s = torch.equal(q.scales_t.cpu(), orc.mx_scale_rows(ce))
    print(f"[mx cols {rows}x{cols} fmt {fmt}] bytes {same_q} scales {same_s}", flush=True)
    assert same_q and same_s


def test_quantize_mx_errors(gpu):
    with pytest.raises(Exception, match="cols"):
        ops.quantize_mx(torch.zeros(32, 48, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(Exception, match="rows"):
        ops.quantize_mx(torch.zeros(48, 64, dtype=torch.bfloat16, device=gpu), colwise=True)


def _mx_gemm_case(gpu, M, N, K, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(M, K, generator=g) * torch.logspace(-2, 2, K)[None, :]).to(torch.bfloat16)
    b = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias_t = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    qa = ops.quantize_mx(a.to(gpu))
    qb = ops.quantize_mx(b.to(gpu))
    bias_g = bias_t.to(gpu) if bias else None
    y32 = ops.gemm_mx(qa.data, qa.scales, qb.data, qb.scales, out_dtype=torch.float32, bias=bias_g)
    y16 = ops.gemm_mx(qa.data, qa.scales, qb.data, qb.scales, bias=bias_g)
    torch.cuda.synchronize()
    ra, ea = orc.quantize_mx(a, ops.E4M3)
    rb, eb = orc.quantize_mx(b, ops.E4M3)
    assert torch.equal(qa.data.view(torch.uint8).cpu(), ra)
    assert torch.equal(qb.data.view(torch.uint8).cpu(), rb)
    ref = orc.scaled_mm_mx(ra, ea, rb, eb, bias=bias_t)
    err = (y32.cpu() - ref).abs().max().item() / max(_rms(ref), 1e-30)
    print(f"[mx gemm {M}x{N}x{K}] max|err|/RMS = {err:.3e}", flush=True)
    assert err <= 0.01
    assert torch.equal(y16.cpu().view(torch.int16), y32.cpu().to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("M,N,K", [
    (512, 2048, 2560),     # c1 shape
    (100, 264, 352),       # ragged M, N; K % 128 = 96 (a partial last K step)
    (4096, 2560, 2560),    # large tiles
    (512, 2560, 10240),    # split-K (partials reduced with unit scale)
    (64, 128, 32),         # a single block of K
])
def test_gemm_mx(gpu, M, N, K):
    _mx_gemm_case(gpu, M, N, K, seed=M + N + K)


def test_gemm_mx_bias(gpu):
    _mx_gemm_case(gpu, 200, 256, 512, seed=5, bias=True)


@pytest.mark.parametrize("M,I,K", [(300, 384, 512), (512, 1024, 2560), (64, 128, 96)])
def test_gemm_geglu_mx(gpu, M, I, K):
    g = torch.Generator().manual_seed(M + I)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, generator=g) * 0.02).to(torch.bfloat16)
    qx = ops.quantize_mx(x.to(gpu))
    qw = ops.quantize_mx(w.to(gpu))
    H, GU = ops.gemm_geglu_mx(qx.data, qx.scales, qw.data, qw.scales, I, keep_gu=True)
    torch.cuda.synchronize()
    rx, ex = orc.quantize_mx(x, ops.E4M3)
    rw, ew = orc.quantize_mx(w, ops.E4M3)
    gate = orc.scaled_mm_mx(rx, ex, rw[:I], ew[:I])
    up = orc.scaled_mm_mx(rx, ex, rw[I:], ew[I:])
    GU_c, H_c = GU.cpu(), H.cpu()
    for got, ref, what in ((GU_c[:, :I], gate, "gate"), (GU_c[:, I:], up, "up")):
        excess = ((got.float() - ref).abs() - 0.5 * orc.bf16_ulp(ref)).max().item()
        rel = excess / max(_rms(ref), 1e-30)
        print(f"[mx geglu {what} {M}x{I}x{K}] max(|err| - ulp/2)/RMS = {rel:.3e}", flush=True)
        assert rel <= 1e-3
    H_ref = orc.geglu(GU_c[:, :I], GU_c[:, I:])
    diff = (H_c.float() - H_ref.float()).abs()
    ulp = orc.bf16_ulp(H_ref.float())
    slack = 2.0 ** -20 * H_ref.float().abs().max()
    assert bool((diff <= 2 * ulp + slack).all()), "H beyond 2 bf16 ulps of the gelu chain"
    assert (diff > 0).float().mean().item() <= 0.05
