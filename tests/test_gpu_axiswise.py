"""GPU parity of the axiswise (torchao rowwise-recipe) path against the CPU oracle.

  * quantize: fp8 bytes and inverse scales bit-exact against oracle.quantize_axiswise
    (per row, and per column stored transposed), with and without power-of-2 scales;
  * GEMM with scale vectors: fp32 output within 1% of RMS of the oracle's fp64 dequantized
    matmul, bf16 output the RNE rounding of the same kernel's fp32 output;
  * TrainingLinear under 'rowwise' / 'rowwise_with_gw_hp': y, dX, dW against the oracle's
    recipe chain, max(|err| - ulp/2) <= 1% of RMS (one quantization per operand).
"""

import pytest
import torch
from torch import nn

from bongard_amd import float8_training, ops
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _rms(t):
    return t.double().pow(2).mean().sqrt().item()


def _x(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g)
    if rows > 3 and cols > 16:
        x[2] *= 500.0          # an outlier row
        x[:, 7] *= 1e-3        # a small column
        x[3] = 0.0             # a zero row (clamped amax)
        x[:, 9] = 0.0          # a zero column
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(1, 16), (37, 48), (512, 2560), (300, 4096),
                                       (64, 10240), (130, 16384), (2049, 1024), (16, 6144)])
@pytest.mark.parametrize("fmt", [ops.E4M3, ops.E5M2])
def test_quantize_axiswise_bit_exact(gpu, rows, cols, fmt):
    x = _x(rows, cols, rows + cols + fmt)
    for pow2 in (True, False):
        q = ops.quantize_axiswise(x.to(gpu), fmt, rowwise=True, colwise=True, pow2=pow2)
        torch.cuda.synchronize()
        rq, rs = orc.quantize_axiswise(x, fmt, -1, pow2)
        cq, cs = orc.quantize_axiswise(x, fmt, 0, pow2)
        same_r = torch.equal(q.data.view(torch.uint8).cpu(), rq)
        same_c = torch.equal(q.data_t.view(torch.uint8).cpu(), cq.t().contiguous())
        print(f"[axis {rows}x{cols} fmt {fmt} pow2 {pow2}] rows {same_r} cols {same_c}", flush=True)
        assert same_r and same_c
        assert torch.equal(q.row_sinv.cpu(), rs[:, 0].reciprocal())
        assert torch.equal(q.col_sinv.cpu(), cs[0].reciprocal())


def test_quantize_axiswise_one_side_and_specials(gpu):
    x = _x(96, 256, 5)
    x[10, 4] = float("nan")
    x[20, 6] = float("inf")
    x[30, 8] = float("-inf")
    only_r = ops.quantize_axiswise(x.to(gpu), ops.E4M3, rowwise=True, colwise=False)
    only_c = ops.quantize_axiswise(x.to(gpu), ops.E4M3, rowwise=False, colwise=True)
    torch.cuda.synchronize()
    assert only_r.data_t is None and only_c.data is None
    rq, rs = orc.quantize_axiswise(x, ops.E4M3, -1)
    cq, cs = orc.quantize_axiswise(x, ops.E4M3, 0)
    assert torch.equal(only_r.data.view(torch.uint8).cpu(), rq)
    got_c = only_c.data_t.view(torch.uint8).cpu()
    want_c = cq.t().contiguous()
    # A NaN column amax makes the whole column NaN bytes. Their sign is the sign of the NaN
    # torch's CPU reduction happens to produce (its amax over dim 0 returns a negative NaN,
    # over dim -1 a positive one); the kernel always uses a positive NaN. Compare those
    # columns modulo the sign bit.
    nan_col = cs[0].isnan()
    got_c = torch.where(nan_col[:, None], got_c & 0x7F, got_c)
    want_c = torch.where(nan_col[:, None], want_c & 0x7F, want_c)
    assert bool(nan_col[4]) and bool((got_c[4] == 0x7F).all())
    bad = (got_c != want_c).nonzero()
    for c, r in bad[:8].tolist():
        print(f"[colwise mismatch] col {c} row {r}: got {int(got_c[c, r]):#04x} "
              f"want {int(want_c[c, r]):#04x} x {float(x[r, c])} scale {float(cs[0, c])}",
              flush=True)
    assert bad.numel() == 0
    assert torch.equal(only_r.row_sinv.cpu().isnan(), rs[:, 0].isnan())
    with pytest.raises(Exception, match="cols"):
        ops.quantize_axiswise(torch.zeros(4, 24, dtype=torch.bfloat16, device=gpu))


def _axis_gemm_case(gpu, M, N, K, a_vec, b_vec, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 4).to(torch.bfloat16)
    b = (torch.randn(N, K, generator=g) * 0.02 * torch.rand(N, 1, generator=g)).to(torch.bfloat16)
    bias_t = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    if a_vec:
        ra, sa = orc.quantize_axiswise(a, ops.E4M3, -1)
        qa = ops.quantize_axiswise(a.to(gpu), ops.E4M3)
        a8, asv = qa.data, qa.row_sinv
    else:
        ra, _, sa, _ = orc.quantize(a, ops.E4M3)
        qa = ops.quantize(a.to(gpu), ops.E4M3)
        a8, asv = qa.data, qa.meta[2:3]
    if b_vec:
        rb, sb = orc.quantize_axiswise(b, ops.E4M3, -1)
        qb = ops.quantize_axiswise(b.to(gpu), ops.E4M3)
        b8, bsv = qb.data, qb.row_sinv
    else:
        rb, _, sb, _ = orc.quantize(b, ops.E4M3)
        qb = ops.quantize(b.to(gpu), ops.E4M3)
        b8, bsv = qb.data, qb.meta[2:3]
    bias_g = bias_t.to(gpu) if bias else None
    y32 = ops.gemm_axiswise(a8, ops.E4M3, asv, b8, ops.E4M3, bsv, out_dtype=torch.float32,
                            bias=bias_g)
    y16 = ops.gemm_axiswise(a8, ops.E4M3, asv, b8, ops.E4M3, bsv, bias=bias_g)
    torch.cuda.synchronize()
    assert torch.equal(a8.view(torch.uint8).cpu(), ra) and torch.equal(b8.view(torch.uint8).cpu(), rb)
    ref = orc.scaled_mm(ra, sa, ops.E4M3, rb, sb, ops.E4M3, bias=bias_t)
    err = (y32.cpu() - ref).abs().max().item() / max(_rms(ref), 1e-30)
    print(f"[axis gemm {M}x{N}x{K} a_vec {a_vec} b_vec {b_vec}] max|err|/RMS = {err:.3e}",
          flush=True)
    assert err <= 0.01
    assert torch.equal(y16.cpu().view(torch.int16), y32.cpu().to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("M,N,K,a_vec,b_vec", [
    (512, 2048, 2560, 1, 1),      # c1 shape, both sides per row
    (300, 384, 256, 1, 0),        # ragged M, tensorwise B (rowwise_with_gw_hp dgrad)
    (256, 512, 384, 0, 1),
    (512, 2560, 10240, 1, 1),     # a split-K plan: scales applied by the reduction
    (4096, 2560, 2560, 1, 1),     # a large-tile plan
])
def test_gemm_axiswise(gpu, M, N, K, a_vec, b_vec):
    _axis_gemm_case(gpu, M, N, K, a_vec, b_vec, seed=M + N + K)


def test_gemm_axiswise_tail_split(gpu, monkeypatch):
    """Per-row and per-column scale vectors reach the tail tiles' reduction (tail split
    forced: 272 tiles of 256x256, 16 of them split along K)."""
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x256:t")
    _axis_gemm_case(gpu, 4160, 3848, 4096, 1, 1, seed=64, bias=True)


def test_gemm_axiswise_bias(gpu):
    _axis_gemm_case(gpu, 200, 256, 512, 1, 1, seed=9, bias=True)


def _close(got, ref, what, tol=0.01):
    got, ref = got.float().cpu(), ref.float().cpu()
    excess = ((got - ref).abs() - 0.5 * orc.bf16_ulp(ref)).clamp(min=0).max().item()
    rel = excess / max(_rms(ref), 1e-30)
    print(f"[{what}] max(|err| - ulp/2)/RMS = {rel:.3e}", flush=True)
    assert rel <= tol, what


@pytest.mark.parametrize("recipe", ["rowwise", "rowwise_with_gw_hp"])
@pytest.mark.parametrize("rows", [256, 200])
def test_training_linear_axiswise_fwd_bwd(gpu, recipe, rows):
    g = torch.Generator().manual_seed(rows + len(recipe))
    x = torch.randn(rows, 512, generator=g).to(torch.bfloat16)
    w = (torch.randn(384, 512, generator=g) * 0.02).to(torch.bfloat16)
    w[:, 5] *= 30.0
    dy = (torch.randn(rows, 384, generator=g) * 1e-3).to(torch.bfloat16)
    lin = nn.Linear(512, 384, bias=False).to(torch.bfloat16)
    lin.weight.data = w.clone()
    cfg = float8_training.Float8LinearConfig(recipe=recipe, pad_inner_dim=True)
    f8 = float8_training.Float8Linear.from_float(lin, cfg)
    f8.__class__ = float8_training.TrainingLinear
    f8 = f8.to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = f8(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    pad = (rows + 15) // 16 * 16 - rows
    ry, rdx, rdw = orc.linear_fwd_bwd_axiswise(torch.nn.functional.pad(x, (0, 0, 0, pad)), w,
                                               torch.nn.functional.pad(dy, (0, 0, 0, pad)),
                                               recipe)
    _close(y, ry[:rows], f"{recipe} y")
    _close(xg.grad, rdx[:rows], f"{recipe} dx")
    _close(f8.weight.grad, rdw, f"{recipe} dw")
