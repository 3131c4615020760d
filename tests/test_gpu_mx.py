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


def test_gemm_mx_tail_split(gpu, monkeypatch):
    """MX operands under the tail split (272 tiles of 256x256, 16 of them split along K):
    the tail tiles' pieces are reduced with unit scales."""
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x256:t")
    M, N, K = 4160, 3848, 4096
    assert ops._lib.lib().bf8_gemm_mx_workspace(M, N, K) % (16 * 256 * 256 * 4) == 0
    _mx_gemm_case(gpu, M, N, K, seed=63, bias=True)


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


GEGLU_TILES = ["256x256", "160x256", "192x256", "128x128", "64x128", "256x128"]


@pytest.mark.parametrize("tile", ["auto"] + GEGLU_TILES)
@pytest.mark.parametrize("M,I,K", [(320, 384, 256), (100, 256, 128)])
def test_gemm_geglu_mx_quant(gpu, monkeypatch, tile, M, I, K):
    """H quantized in the GEGLU epilogue == bf8_quantize_mx_bf16 of the bf16 H of the
    unfused kernel, byte for byte (fp8 payloads, E8M0 scales, the transposed copy and its
    padding), on every tile with a gated-GELU variant, with inf / NaN blocks in H."""
    if tile != "auto":
        monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M + I + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[7] *= 1e-4                      # a row of small activations
    w = (torch.randn(2 * I, K, generator=g) * 0.02).to(torch.bfloat16)
    qx = ops.quantize_mx(x.to(gpu))
    qw = ops.quantize_mx(w.to(gpu))
    qx.scales[5, 0] = 254             # row 5: 2^127 on its first block -> +-inf gate/up, NaN H
    qx.data.view(torch.uint8)[9, 3] = 0x7F  # row 9: an e4m3 NaN operand -> NaN row of H
    colwise = M % 32 == 0
    args = (qx.data, qx.scales, qw.data, qw.scales, I)
    hq, GU, H = ops.gemm_geglu_mx_quant(*args, colwise=colwise, keep_gu=True, keep_h=True)
    hq2, GU2, H2 = ops.gemm_geglu_mx_quant(*args, colwise=colwise)
    H_ref, GU_ref = ops.gemm_geglu_mx(*args, keep_gu=True)
    ref = ops.quantize_mx(H_ref, rowwise=True, colwise=colwise)
    torch.cuda.synchronize()
    assert GU2 is None and H2 is None and (hq2.data_t is None) == (not colwise)
    assert torch.equal(H.view(torch.int16), H_ref.view(torch.int16))
    assert torch.equal(GU.view(torch.int16), GU_ref.view(torch.int16))
    hc = H_ref.cpu()
    assert bool(hc[9].isnan().any()) and bool(hc[5].isinf().any() or hc[5].isnan().any())
    for q, what in ((hq, "with H"), (hq2, "without H")):
        same = [torch.equal(q.data.view(torch.uint8), ref.data.view(torch.uint8)),
                torch.equal(q.scales, ref.scales)]
        if colwise:
            same += [torch.equal(q.data_t.view(torch.uint8), ref.data_t.view(torch.uint8)),
                     torch.equal(q.scales_t, ref.scales_t)]
        print(f"[mx geglu quant {tile} {M}x{I}x{K} {what}] rows, scales, cols, scales_t: "
              f"{same}", flush=True)
        assert all(same)
    # and the oracle on the finite rows (the kernel's own H as input)
    finite = hc.isfinite().all(dim=1)
    rq, re_ = orc.quantize_mx(hc[finite], ops.E4M3)
    assert torch.equal(hq.data.view(torch.uint8).cpu()[finite], rq)
    assert torch.equal(hq.scales.cpu()[finite][:, :I // 32], re_.to(torch.uint8))


def test_gemm_geglu_mx_quant_errors(gpu):
    qx = ops.quantize_mx(torch.randn(100, 128, device=gpu).to(torch.bfloat16))
    qw = ops.quantize_mx(torch.randn(512, 128, device=gpu).to(torch.bfloat16))
    with pytest.raises(RuntimeError, match="M % 32"):
        ops.gemm_geglu_mx_quant(qx.data, qx.scales, qw.data, qw.scales, 256, colwise=True)


# ---- the TE modules under 'mxfp8' ------------------------------------------------------
import types  # noqa: E402

from torch import nn  # noqa: E402
from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2MLP, T5Gemma2RMSNorm  # noqa: E402

from bongard_amd import fused_mlp, te_linear  # noqa: E402


def _close(got, ref, what, tol=0.01):
    got, ref = got.float().cpu(), ref.float().cpu()
    excess = ((got - ref).abs() - 0.5 * orc.bf16_ulp(ref)).clamp(min=0).max().item()
    rel = excess / max(_rms(ref), 1e-30)
    print(f"[{what}] max(|err| - ulp/2)/RMS = {rel:.3e}", flush=True)
    assert rel <= tol, what


def _close_requant(got, ref, what, max_tol=0.05, rms_tol=0.005):
    """H (and dGU) are requantized inside the chain: sparse legitimate fp8 flips where
    GPU and oracle round a value to neighbouring bf16s; statistical bar as for 'fp8'."""
    got, ref = got.float().cpu(), ref.float().cpu()
    rms = max(_rms(ref), 1e-30)
    max_rel = (got - ref).abs().max().item() / rms
    rms_rel = _rms(got - ref) / rms
    print(f"[{what}] max|err|/RMS = {max_rel:.3e}, RMS(err)/RMS = {rms_rel:.3e}", flush=True)
    assert max_rel <= max_tol and rms_rel <= rms_tol, what


def _mlp(hidden, inter, seed):
    cfg = types.SimpleNamespace(hidden_size=hidden, intermediate_size=inter,
                                hidden_activation="gelu_pytorch_tanh", dropout_rate=0.0)
    torch.manual_seed(seed)
    m = T5Gemma2MLP(cfg)
    with torch.no_grad():
        m.gate_proj.weight.normal_(std=0.02)
        m.up_proj.weight.normal_(std=0.02)
        m.down_proj.weight.normal_(std=0.014)
    return m.to(torch.bfloat16)


@pytest.mark.parametrize("rows", [256, 200])
def test_telinear_mxfp8_fwd_bwd(gpu, rows):
    g = torch.Generator().manual_seed(rows + 1)
    x = torch.randn(rows, 512, generator=g).to(torch.bfloat16)
    w = (torch.randn(384, 512, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(rows, 384, generator=g) * 1e-3).to(torch.bfloat16)
    lin = nn.Linear(512, 384, bias=False)
    lin.weight.data = w.clone().float()
    t = te_linear.TELinear([lin], "mxfp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = t(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    pad = (rows + 31) // 32 * 32 - rows
    ry, rdx, rdw = orc.linear_fwd_bwd_mx(torch.nn.functional.pad(x, (0, 0, 0, pad)), w,
                                         torch.nn.functional.pad(dy, (0, 0, 0, pad)))
    _close(y, ry[:rows], "mx telinear y")
    _close(xg.grad, rdx[:rows], "mx telinear dx")
    _close(t.weight.grad, rdw, "mx telinear dw")
    t(xg)
    assert t.counts == {"weight_quantizations": 1, "cached_weights": 1}


def _temlp_mx_step(gpu, mlp, x, dy, split, monkeypatch):
    monkeypatch.setenv("BONGARD_TE_SPLIT_GATE_UP", "1" if split else "0")
    t = te_linear.TEMLP(mlp, "mxfp8").to(gpu).train()
    assert t.fused_gate_up != split
    xg = x.to(gpu).requires_grad_(True)
    y = t(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    dwgu = (t.gate_up.weight.grad if not split
            else torch.cat([t.gate_proj.weight.grad, t.up_proj.weight.grad]))
    return y, xg.grad, dwgu, t.down.weight.grad


def test_temlp_mxfp8_fwd_bwd(gpu, monkeypatch):
    """TEMLP under 'mxfp8' against the oracle chain (statistical bar: H and dGU are
    requantized in blocks; where GPU and oracle round a block's largest element to
    neighbouring bf16s across a power of two, the whole block's E8M0 scale moves and its 32
    values requantize on a grid twice as coarse or fine, so single outputs can move by up to
    ~0.1 RMS). The split gate/up layout (BONGARD_TE_SPLIT_GATE_UP=1) quantizes the same
    blocks, so it must reproduce the fused layout bit for bit."""
    hidden, inter, rows = 256, 512, 512
    g = torch.Generator().manual_seed(61)
    mlp = _mlp(hidden, inter, 61)
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
    fused = _temlp_mx_step(gpu, mlp, x, dy, False, monkeypatch)
    split = _temlp_mx_step(gpu, mlp, x, dy, True, monkeypatch)
    for a, b in zip(fused, split):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ref = orc.mlp_fwd_bwd_mx(x, wg, wu, wd, dy)
    y, dx, dwgu, dwd = fused
    _close_requant(y, ref["y"], "mx temlp y", max_tol=0.10)
    _close_requant(dx, ref["dx"], "mx temlp dx", max_tol=0.2)
    _close_requant(dwgu, ref["dwgu"], "mx temlp dWgu", max_tol=0.2)
    _close_requant(dwd, ref["dwd"], "mx temlp dWd", max_tol=0.2)


def test_fused_mlp_mxfp8_fwd_bwd(gpu):
    hidden, inter, rows = 256, 512, 480
    g = torch.Generator().manual_seed(62)
    mlp = _mlp(hidden, inter, 62)
    norm = T5Gemma2RMSNorm(hidden, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.normal_(std=0.1)
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    nw = norm.weight.detach().clone()
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
    f = fused_mlp.FusedMLP(mlp, norm, "mxfp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = f(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    xr = x.clone().requires_grad_(True)
    normed = orc.rmsnorm(xr, nw, 1e-6)
    ref = orc.mlp_fwd_bwd_mx(normed.detach(), wg, wu, wd, dy)
    normed.backward(ref["dx"].to(torch.bfloat16))
    _close_requant(y, ref["y"], "mx fused y", max_tol=0.10)
    _close_requant(xg.grad, xr.grad, "mx fused dx", max_tol=0.2)
    _close_requant(f.fc1_weight.grad, ref["dwgu"], "mx fused dWgu", max_tol=0.2)
    _close_requant(f.fc2_weight.grad, ref["dwd"], "mx fused dWd", max_tol=0.2)
    assert f.state_dict()["_extra_state"].numel() == 0


@pytest.mark.parametrize("tile", ["256x256", "256x160", "160x256", "128x128", "192x256",
                                  "128x64", "64x128", "256x128"])
def test_gemm_mx_every_tile(gpu, monkeypatch, tile):
    """Every block tile's MX variant (those whose stages would overflow the LDS with the
    scale dwords run with one stage fewer), forced through the tuning override."""
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", tile)
    _mx_gemm_case(gpu, 300, 392, 544, seed=17)


def test_quantize_mx_many_equals_quantize_mx(gpu, monkeypatch):
    """Rowwise MX quantization of several tensors in one launch gives each tensor's own
    bytes and scales (formats mixed, a ragged row count, an empty tensor skipped); the MX
    gated MLP's inference forward, which uses it, equals its training forward bit for bit."""
    from bongard_amd import linear
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(300, 2560, generator=g).to(torch.bfloat16).to(gpu),
          (torch.randn(8192, 4096, generator=g) * 40).to(torch.bfloat16).to(gpu),
          torch.randn(64, 96, generator=g).to(torch.bfloat16).to(gpu),
          torch.empty(0, 64, dtype=torch.bfloat16, device=gpu)]
    xs[2][3, 5] = float("nan")
    fmts = [ops.E4M3, ops.E5M2, ops.E4M3, ops.E4M3]
    qs = ops.quantize_mx_many(xs, fmts)
    for x, q, f in zip(xs[:3], qs, fmts):
        r = ops.quantize_mx(x, f)
        assert torch.equal(q.data.view(torch.uint8), r.data.view(torch.uint8))
        assert torch.equal(q.scales, r.scales)
    assert qs[3].data.numel() == 0
    with pytest.raises(RuntimeError):
        ops.quantize_mx_many([xs[0], torch.zeros(32, 48, dtype=torch.bfloat16, device=gpu)])
    # the inference forwards (no_grad) of the MX MLP and linear on trainable weights take
    # the shared launch; their outputs equal the training forwards' bit for bit
    calls = []
    real = ops.quantize_mx_many

    def counted(*a, **k):
        calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(ops, "quantize_mx_many", counted)
    x = torch.randn(256, 256, generator=g).to(torch.bfloat16).to(gpu)
    w_gu = torch.nn.Parameter((torch.randn(1024, 256, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
    w_d = torch.nn.Parameter((torch.randn(256, 512, generator=g) * 0.014).to(torch.bfloat16).to(gpu))
    y_train = linear.Fp8GegluMlpMxFunction.apply(x, w_gu, w_d, None, None, 512)
    assert len(calls) == 0
    with torch.no_grad():
        y_inf = linear.Fp8GegluMlpMxFunction.apply(x, w_gu, w_d, None, None, 512)
    assert len(calls) == 1
    assert torch.equal(y_train.detach(), y_inf)
    w_o = torch.nn.Parameter(w_d.detach().t().contiguous())
    y_train = linear.Fp8LinearMxFunction.apply(x, w_o, None)
    with torch.no_grad():
        y_inf = linear.Fp8LinearMxFunction.apply(x, w_o, None)
    assert len(calls) == 2
    assert torch.equal(y_train.detach(), y_inf)
