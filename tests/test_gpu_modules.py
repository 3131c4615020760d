"""GPU tests of the drop-in modules in training mode against the oracle's FP8 chains.

Linear layers (one quantization per operand): forward and gradients within max |err| <=
1% of RMS of the oracle's fp64 dequantized GEMMs (after half a bf16 ulp of output
rounding).

Gated MLP: H (and in the backward dGU) is re-quantized inside the chain. The gelu chain
itself is bit-exact (given g and u, H and dGU equal torch's CPU chain bit for bit:
tests/test_gpu_gemm.py), but the gate/up GEMM accumulates in another order than the
oracle's CPU matmul, so g and u, and then H, can differ by one bf16 ulp; where that
straddles an e4m3 (e5m2) rounding boundary the requantized byte moves by a whole fp8 step
(6-25% of that element). Those flips are legitimate and sparse, so the end-to-end MLP bar
is statistical: RMS(err) <= 0.5% of RMS(ref) (measured 0.17-0.28%), and max |err| <= 5%
of RMS(ref) for the TEMLP forward (measured 1.4-3.3%), 10% for its backward and the fused
forward, 20% for the fused and delayed backwards (dGU is requantized to e5m2, whose step
is twice e4m3's; measured up to 15%). The strict 1% bar holds for every GEMM given its own
FP8 inputs (tests/test_gpu_gemm.py::test_mlp_down_gemm_on_own_h8, tests/test_gpu_configs.py
at the c2-c5 sizes: ~1e-4 of RMS).
"""

import types

import pytest
import torch
from torch import nn
from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2MLP, T5Gemma2RMSNorm

from bongard_amd import float8_training, fused_mlp, ops, te_linear
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _rms(t):
    return t.double().pow(2).mean().sqrt().item()


def _close(got, ref, what, tol=0.01):
    got, ref = got.float().cpu(), ref.float().cpu()
    excess = ((got - ref).abs() - 0.5 * orc.bf16_ulp(ref)).clamp(min=0).max().item()
    rel = excess / max(_rms(ref), 1e-30)
    print(f"[{what}] max(|err| - ulp/2)/RMS = {rel:.3e}", flush=True)
    assert rel <= tol, what


def _close_requant(got, ref, what, max_tol=0.05, rms_tol=0.005):
    got, ref = got.float().cpu(), ref.float().cpu()
    rms = max(_rms(ref), 1e-30)
    max_rel = (got - ref).abs().max().item() / rms
    rms_rel = _rms(got - ref) / rms
    print(f"[{what}] max|err|/RMS = {max_rel:.3e}, RMS(err)/RMS = {rms_rel:.3e}", flush=True)
    assert max_rel <= max_tol and rms_rel <= rms_tol, what


def _mlp(hidden, inter, seed, dev):
    cfg = types.SimpleNamespace(hidden_size=hidden, intermediate_size=inter,
                                hidden_activation="gelu_pytorch_tanh", dropout_rate=0.0)
    torch.manual_seed(seed)
    m = T5Gemma2MLP(cfg)
    with torch.no_grad():
        m.gate_proj.weight.normal_(std=0.02)
        m.up_proj.weight.normal_(std=0.02)
        m.down_proj.weight.normal_(std=0.014)
    return m.to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("rows", [512, 300, 17])
def test_telinear_train_fwd_bwd(gpu, rows):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 512, generator=g).to(torch.bfloat16)
    w = (torch.randn(384, 512, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(rows, 384, generator=g) * 1e-3).to(torch.bfloat16)
    lin = nn.Linear(512, 384, bias=False)
    lin.weight.data = w.clone().float()
    t = te_linear.TELinear([lin], "fp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = t(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    pad = (rows + 31) // 32 * 32 - rows
    xp = torch.nn.functional.pad(x, (0, 0, 0, pad))
    dyp = torch.nn.functional.pad(dy, (0, 0, 0, pad))
    ry, rdx, rdw = orc.linear_fwd_bwd(xp, w, dyp)
    _close(y, ry[:rows], "telinear y")
    _close(xg.grad, rdx[:rows], "telinear dx")
    _close(t.weight.grad, rdw, "telinear dw")
    assert t.counts == {"weight_quantizations": 1}
    t(xg)
    assert t.counts == {"weight_quantizations": 1, "cached_weights": 1}
    with torch.no_grad():
        t.weight.add_(1e-3)  # an optimizer step bumps weight._version
    t(xg)
    assert t.counts["weight_quantizations"] == 2


def test_training_linear_fwd_bwd(gpu):
    g = torch.Generator().manual_seed(3)
    rows = 200
    x = torch.randn(rows, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(128, 256, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(rows, 128, generator=g) * 1e-3).to(torch.bfloat16)
    lin = nn.Linear(256, 128, bias=False).to(torch.bfloat16)
    lin.weight.data = w.clone()
    f8 = float8_training.Float8Linear.from_float(lin, float8_training.Float8LinearConfig())
    f8.__class__ = float8_training.TrainingLinear
    f8 = f8.to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = f8(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    pad = (rows + 15) // 16 * 16 - rows
    ry, rdx, rdw = orc.linear_fwd_bwd(torch.nn.functional.pad(x, (0, 0, 0, pad)), w,
                                      torch.nn.functional.pad(dy, (0, 0, 0, pad)))
    _close(y, ry[:rows], "trainlinear y")
    _close(xg.grad, rdx[:rows], "trainlinear dx")
    _close(f8.weight.grad, rdw, "trainlinear dw")
    f8.eval()
    assert torch.equal(f8(xg.detach()), nn.functional.linear(xg.detach(), f8.weight))


@pytest.mark.parametrize("rows,hidden,inter", [(256, 256, 512), (1024, 512, 1024)])
def test_temlp_train_fwd_bwd(gpu, rows, hidden, inter):
    g = torch.Generator().manual_seed(rows + inter)
    mlp = _mlp(hidden, inter, rows, "cpu")
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
    t = te_linear.TEMLP(mlp, "fp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = t(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    fwd = orc.mlp_forward(x, wg, wu, wd)
    _close_requant(y, fwd["y"], "temlp y")
    rdx, rdwgu, rdwd, _ = orc.mlp_backward(fwd, x, wg, wu, wd, dy)
    _close_requant(xg.grad, rdx, "temlp dx", max_tol=0.10)
    _close_requant(t.gate_up.weight.grad, rdwgu, "temlp dWgu", max_tol=0.10)
    _close_requant(t.down.weight.grad, rdwd, "temlp dWd", max_tol=0.10)
    assert t.gate_up.counts["weight_quantizations"] == 1
    assert t.down.counts["weight_quantizations"] == 1


def test_temlp_split_gate_up(gpu, monkeypatch):
    """BONGARD_TE_SPLIT_GATE_UP=1: two projections, one scale each (bongard/te_linear.py
    :90-95,98-103). Stage check given the kernels' own dGU (bf16, rebuilt with the same
    kernel calls the module makes): each half's e5m2 bytes and scale bit-exact against the
    oracle's own quantization of that half, each half's dgrad within 1% of RMS of the
    oracle's on the same bytes, the module's dx the bf16 sum of the two bf16 halves bit for
    bit, and each half's wgrad within 1%. End to end the statistical bar of the fused MLP
    (1.8% of dGU values one bf16 ulp off the oracle's at this size flip e5m2 bytes), and
    the compiled custom op (split_scales=True) bit-identical to the module."""
    monkeypatch.setenv("BONGARD_TE_SPLIT_GATE_UP", "1")
    g = torch.Generator().manual_seed(44)
    rows, hidden, I = 512, 256, 512
    mlp = _mlp(hidden, I, 44, "cpu")
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
    t = te_linear.TEMLP(mlp, "fp8").to(gpu).train()
    assert not t.fused_gate_up
    xg = x.to(gpu).requires_grad_(True)
    y = t(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    fwd = orc.mlp_forward(x, wg, wu, wd, shared_gate_up_scale=False)
    # one H8 flip moves an output by ~1/8 |h| |w_down| ~ 5% of RMS(y) at I = 512
    _close_requant(y, fwd["y"], "split y", max_tol=0.10)
    # the kernels' own dGU: the module's forward and dH calls, repeated (deterministic)
    from bongard_amd import linear as lin
    xq = ops.quantize(x.to(gpu), ops.E4M3, rowwise=True, transpose=True)
    gu_q = lin.quantize_gate_up(torch.cat([wg, wu]).to(gpu), I, True, transpose=True)
    _, GU, _ = ops.gemm_geglu(xq.data, xq.meta, gu_q.data, gu_q.meta, I, w_meta_stride=4,
                              keep_gu=True)
    dq = ops.quantize(wd.to(gpu), ops.E4M3, rowwise=True, transpose=True)
    dyq = ops.quantize(dy.to(gpu), ops.E5M2, rowwise=True, transpose=True)
    dH = ops.gemm(dyq.data, ops.E5M2, dyq.meta, dq.data_t, ops.E4M3, dq.meta)
    dGU, _ = ops.geglu_bwd(dH, GU)
    parts, dw_parts = [], []
    for half in range(2):
        d = dGU[:, half * I:(half + 1) * I].contiguous()
        q = ops.quantize(d, ops.E5M2, rowwise=True, transpose=True)
        parts.append((ops.gemm(q.data, ops.E5M2, q.meta, gu_q.data_t[:, half * I:(half + 1) * I],
                               ops.E4M3, gu_q.meta[half], out_dtype=torch.float32),
                      ops.gemm(q.data, ops.E5M2, q.meta, gu_q.data_t[:, half * I:(half + 1) * I],
                               ops.E4M3, gu_q.meta[half])))
        dw_parts.append(ops.gemm(q.data_t, ops.E5M2, q.meta, xq.data_t, ops.E4M3, xq.meta,
                                 out_dtype=torch.float32))
        torch.cuda.synchronize()
        rq, _, rs, _ = orc.quantize(d.cpu(), orc.E5M2)
        assert torch.equal(q.data.view(torch.uint8).cpu(), rq), f"dGU half {half} bytes"
        assert q.meta[1].item() == rs.item(), f"dGU half {half} scale"
    torch.cuda.synchronize()
    assert torch.equal(xg.grad.view(torch.int16), (parts[0][1] + parts[1][1]).view(torch.int16))
    sdx, sdwgu, _, _ = orc.mlp_backward(fwd, x, wg, wu, wd, dy, shared_gate_up_scale=False,
                                        dgu=dGU.cpu())
    for half in range(2):
        d = dGU.cpu()[:, half * I:(half + 1) * I]
        rq, _, rs, _ = orc.quantize(d, orc.E5M2)
        w_half = fwd["wgu_q"][half * I:(half + 1) * I].t().contiguous()
        ref = orc.scaled_mm(rq, rs, orc.E5M2, w_half, fwd["w_scales"][half], orc.E4M3)
        _close(parts[half][0], ref, f"split dgrad half {half} (fp32)")
        assert torch.equal(parts[half][1].view(torch.int16).cpu(),
                           parts[half][0].cpu().to(torch.bfloat16).view(torch.int16))
        _close(dw_parts[half], sdwgu[half * I:(half + 1) * I], f"split wgrad half {half}")
    _close(xg.grad, sdx, "split dx given dGU", tol=0.02)   # two bf16 roundings + the sum's
    # end to end against the oracle chain (requantized dGU: statistical bar)
    rdx, rdwgu, rdwd, _ = orc.mlp_backward(fwd, x, wg, wu, wd, dy, shared_gate_up_scale=False)
    _close_requant(xg.grad, rdx, "split dx", max_tol=0.2, rms_tol=0.01)
    _close_requant(t.gate_proj.weight.grad, rdwgu[:I], "split dW_gate", max_tol=0.2,
                   rms_tol=0.01)
    _close_requant(t.up_proj.weight.grad, rdwgu[I:], "split dW_up", max_tol=0.2, rms_tol=0.01)
    _close_requant(t.down.weight.grad, rdwd, "split dW_down", max_tol=0.10)
    # the same arithmetic as one compile-visible op (split_scales=True), under Inductor
    torch._dynamo.reset()
    from bongard_amd import custom_ops
    w_gu = torch.cat([wg, wu], 0).to(gpu).requires_grad_(True)
    w_d = wd.to(gpu).requires_grad_(True)
    xc = x.to(gpu).requires_grad_(True)
    fn = torch.compile(lambda a, b, c: custom_ops.fp8_geglu_mlp(a, b, c, I, True),
                       fullgraph=True)
    yc = fn(xc, w_gu, w_d)
    yc.backward(dy.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(yc.view(torch.int16), y.view(torch.int16))
    assert torch.equal(xc.grad.view(torch.int16), xg.grad.view(torch.int16))
    dw_split = torch.cat([t.gate_proj.weight.grad, t.up_proj.weight.grad], 0)
    assert torch.equal(w_gu.grad.view(torch.int16), dw_split.view(torch.int16))
    assert torch.equal(w_d.grad.view(torch.int16), t.down.weight.grad.view(torch.int16))


def test_fused_mlp_train_forward(gpu):
    g = torch.Generator().manual_seed(9)
    hidden, inter, rows = 256, 512, 160
    mlp = _mlp(hidden, inter, 9, "cpu")
    norm = T5Gemma2RMSNorm(hidden, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.normal_(std=0.1)
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    nw = norm.weight.detach().clone()
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
    f = fused_mlp.FusedMLP(mlp, norm, "fp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    y = f(xg)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    xr = x.clone().requires_grad_(True)
    nr = nw.clone().requires_grad_(True)
    normed = orc.rmsnorm(xr, nr, 1e-6)
    fwd = orc.mlp_forward(normed.detach(), wg, wu, wd)
    rdn, rdwgu, rdwd, _ = orc.mlp_backward(fwd, normed.detach(), wg, wu, wd, dy)
    normed.backward(rdn.to(torch.bfloat16))
    # the norm output (a GPU reduction) is itself requantized to e4m3: a second source of
    # legitimate byte flips, hence the backward-sized max bound
    _close_requant(y, fwd["y"], "fused y", max_tol=0.10)
    _close_requant(xg.grad, xr.grad, "fused dx", max_tol=0.2)
    _close_requant(f.fc1_weight.grad, rdwgu, "fused dW_fc1", max_tol=0.2)
    _close_requant(f.fc2_weight.grad, rdwd, "fused dW_fc2", max_tol=0.2)
    _close_requant(f.layer_norm_weight.grad, nr.grad, "fused dW_norm", max_tol=0.2)
    assert f.counts["real_tokens"] == rows and f.counts["kernel_tokens"] == 160
    f.eval()
    ref_eval = f._hf_mlp(f._hf_norm(xg.detach()))
    assert torch.equal(f(xg.detach()), ref_eval)


def test_temlp_delayed_train_steps(gpu):
    """'fp8_delayed': three training steps (an in-place update between them re-quantizes
    the weights, as an optimizer step does) against the oracle chain whose every tensor
    role is quantized by a DelayedQuantizer with the same history length."""
    hidden, inter, rows = 256, 512, 256
    g = torch.Generator().manual_seed(77)
    mlp = _mlp(hidden, inter, 77, "cpu")
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    t = te_linear.TEMLP(mlp, "fp8_delayed").to(gpu).train()
    quant = orc.DelayedQuantizer(16)
    for step in range(3):
        with torch.no_grad():                       # new weight versions: re-quantize
            t.gate_up.weight.mul_(1.0)
            t.down.weight.mul_(1.0)
        x = (torch.randn(rows, hidden, generator=g) * (1 + step)).to(torch.bfloat16)
        dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
        xg = x.to(gpu).requires_grad_(True)
        y = t(xg)
        y.backward(dy.to(gpu))
        torch.cuda.synchronize()
        fwd = orc.mlp_forward(x, wg, wu, wd, quant=quant)
        rdx, rdwgu, rdwd, _ = orc.mlp_backward(fwd, x, wg, wu, wd, dy, quant=quant)
        _close_requant(y, fwd["y"], f"delayed y step {step}")
        _close_requant(xg.grad, rdx, f"delayed dx step {step}", max_tol=0.2)
        _close_requant(t.gate_up.weight.grad, rdwgu, f"delayed dWgu step {step}", max_tol=0.2)
        _close_requant(t.down.weight.grad, rdwd, f"delayed dWd step {step}", max_tol=0.2)
        t.gate_up.weight.grad = None
        t.down.weight.grad = None
    assert t.gate_up.scaling.input.recorded == 2    # amaxes of steps 0, 1 folded in
    assert t.state_dict()["down._extra_state"].numel() == 3 * (3 + 16 + 4)


def test_fused_mlp_delayed_train_steps(gpu):
    """'fp8_delayed' FusedMLP: the fused norm writes the amax partials of its output into
    the fc1 input role's producer buffer, and three training steps follow the oracle chain
    (norm -> delayed-scaled MLP; backward through the norm under CPU autograd).

    Step 0 quantizes with the initial scale 1, so its dGU (~1e-5) mostly flushes to zero in
    e5m2; step 1 is the first with a live backward. A single legitimate e5m2 flip of an
    outlier dGU element moves a whole row of dW_gu by up to ~4 RMS(dGU) RMS(X), i.e. about
    4/sqrt(rows) of RMS(dW_gu): 512 rows keep that under the 0.2 bar."""
    hidden, inter, rows = 256, 512, 512
    g = torch.Generator().manual_seed(78)
    mlp = _mlp(hidden, inter, 78, "cpu")
    norm = T5Gemma2RMSNorm(hidden, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.normal_(std=0.1)
    wg, wu, wd = (m.weight.detach().clone() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    nw = norm.weight.detach().clone()
    f = fused_mlp.FusedMLP(mlp, norm, "fp8_delayed").to(gpu).train()
    quant = orc.DelayedQuantizer(16)
    for step in range(3):
        with torch.no_grad():
            f.fc1_weight.mul_(1.0)
            f.fc2_weight.mul_(1.0)
        x = (torch.randn(rows, hidden, generator=g) * (1 + step)).to(torch.bfloat16)
        dy = (torch.randn(rows, hidden, generator=g) * 1e-3).to(torch.bfloat16)
        xg = x.to(gpu).requires_grad_(True)
        y = f(xg)
        y.backward(dy.to(gpu))
        torch.cuda.synchronize()
        xr = x.clone().requires_grad_(True)
        normed = orc.rmsnorm(xr, nw, 1e-6)
        fwd = orc.mlp_forward(normed.detach(), wg, wu, wd, quant=quant)
        rdn, rdwgu, rdwd, _ = orc.mlp_backward(fwd, normed.detach(), wg, wu, wd, dy, quant=quant)
        normed.backward(rdn.to(torch.bfloat16))
        _close_requant(y, fwd["y"], f"fused delayed y step {step}", max_tol=0.10)
        _close_requant(xg.grad, xr.grad, f"fused delayed dx step {step}", max_tol=0.2)
        _close_requant(f.fc1_weight.grad, rdwgu, f"fused delayed dWgu step {step}", max_tol=0.2)
        _close_requant(f.fc2_weight.grad, rdwd, f"fused delayed dWd step {step}", max_tol=0.2)
        f.fc1_weight.grad = None
        f.fc2_weight.grad = None
    fc1, _ = f.scaling
    assert fc1.input.recorded == 2


def test_telinear_second_call_per_step_reuses_cached_weight(gpu):
    """The decoder's state-bank K/V projection (bongard/model.py:342-347, 349-359) calls a
    layer's k_proj / v_proj a second time in the same step, on the encoded state: the
    second call reuses the step's FP8 weight (no re-quantization), and the weight gradient
    is the sum of both calls' wgrad GEMMs."""
    g = torch.Generator().manual_seed(91)
    hidden, out = 512, 256
    x = torch.randn(160, hidden, generator=g).to(torch.bfloat16)       # decoder tokens
    state = torch.randn(2, 96, hidden, generator=g).to(torch.bfloat16)  # encoded state bank
    w = (torch.randn(out, hidden, generator=g) * 0.02).to(torch.bfloat16)
    dy1 = (torch.randn(160, out, generator=g) * 1e-3).to(torch.bfloat16)
    dy2 = (torch.randn(2, 96, out, generator=g) * 1e-3).to(torch.bfloat16)
    lin = nn.Linear(hidden, out, bias=False)
    lin.weight.data = w.clone().float()
    t = te_linear.TELinear([lin], "fp8").to(gpu).train()
    xg = x.to(gpu).requires_grad_(True)
    sg = state.to(gpu).requires_grad_(True)
    y1 = t(xg)
    y2 = t(sg)
    assert t.counts == {"weight_quantizations": 1, "cached_weights": 1}
    (y1.float() * dy1.to(gpu).float()).sum().add_((y2.float() * dy2.to(gpu).float()).sum()).backward()
    torch.cuda.synchronize()
    s_flat = state.reshape(-1, hidden)
    r1 = orc.linear_fwd_bwd(x, w, dy1)
    r2 = orc.linear_fwd_bwd(s_flat, w, dy2.reshape(-1, out))
    _close(y1, r1[0], "state pass 1 y")
    _close(y2.reshape(-1, out), r2[0], "state pass 2 y")
    _close(xg.grad, r1[1], "state pass 1 dx")
    _close(sg.grad.reshape(-1, hidden), r2[1], "state pass 2 dx")
    # two bf16-rounded wgrads summed in bf16: half an ulp of each term and of the sum
    got, ref = t.weight.grad.float().cpu(), r1[2] + r2[2]
    slack = 0.5 * (orc.bf16_ulp(r1[2]) + orc.bf16_ulp(r2[2]) + orc.bf16_ulp(ref))
    rel = ((got - ref).abs() - slack).clamp(min=0).max().item() / _rms(ref)
    print(f"[summed dW] max(|err| - rounding)/RMS = {rel:.3e}", flush=True)
    assert rel <= 0.01


def test_state_kv_shared_input_matches_separate_calls(gpu):
    """bongard_amd.state_kv.project_state_kv (one quantization of the state for k and v)
    against the reference form (k_proj(state), v_proj(state)) on copies of the same
    projections: outputs and all gradients bit-identical; counters as two calls."""
    from bongard_amd import state_kv

    g = torch.Generator().manual_seed(92)
    hidden, nk, head_dim = 512, 256, 64
    state = torch.randn(3, 64, hidden, generator=g).to(torch.bfloat16)
    wk = (torch.randn(nk, hidden, generator=g) * 0.02).to(torch.bfloat16)
    wv = (torch.randn(nk, hidden, generator=g) * 0.02).to(torch.bfloat16)
    dk = (torch.randn(3, nk // head_dim, 64, head_dim, generator=g) * 1e-3).to(torch.bfloat16)
    dv = (torch.randn(3, nk // head_dim, 64, head_dim, generator=g) * 1e-3).to(torch.bfloat16)

    def attention():
        lk, lv = nn.Linear(hidden, nk, bias=False), nn.Linear(hidden, nk, bias=False)
        lk.weight.data, lv.weight.data = wk.clone().float(), wv.clone().float()
        norm = T5Gemma2RMSNorm(head_dim, eps=1e-6).to(torch.bfloat16).to(gpu)
        return types.SimpleNamespace(
            k_proj=te_linear.TELinear([lk], "fp8").to(gpu).train(),
            v_proj=te_linear.TELinear([lv], "fp8").to(gpu).train(),
            k_norm=norm, head_dim=head_dim)

    results = []
    compiled_kv = torch.compile(state_kv.project_state_kv, dynamic=True, backend="aot_eager")
    for mode in ("shared", "separate", "shared_compiled"):
        fused = mode != "separate"
        att = attention()
        sg = state.to(gpu).requires_grad_(True)
        if mode == "shared_compiled":
            keys, values = compiled_kv(att, sg)
        elif fused:
            keys, values = state_kv.project_state_kv(att, sg)
        else:
            shape = (*sg.shape[:-1], -1, head_dim)
            keys = att.k_norm(att.k_proj(sg).view(shape).transpose(1, 2))
            values = att.v_proj(sg).view(shape).transpose(1, 2)
        ((keys.float() * dk.to(gpu).float()).sum()
         + (values.float() * dv.to(gpu).float()).sum()).backward()
        torch.cuda.synchronize()
        assert att.k_proj.counts == {"weight_quantizations": 1}
        results.append((keys, values, sg.grad, att.k_proj.weight.grad, att.v_proj.weight.grad))
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))


class _Block(nn.Module):
    """A text block in miniature: norm -> FP8 linear -> gelu -> FP8 linear, residual."""

    def __init__(self, make_linear, hidden, inter):
        super().__init__()
        self.norm = T5Gemma2RMSNorm(hidden, eps=1e-6).to(torch.bfloat16)
        self.up = make_linear(hidden, inter)
        self.down = make_linear(inter, hidden)

    def forward(self, x):
        h = self.up(self.norm(x))
        return x + self.down(torch.nn.functional.gelu(h, approximate="tanh"))


@pytest.mark.parametrize("kind", ["tensorwise", "rowwise", "te_fp8", "te_mxfp8"])
def test_fp8_linears_inside_a_compiled_region(gpu, kind):
    """The reference compiles each text layer (bongard/model.py:249-281, module.compile(
    dynamic=True)); the FP8 linears inside must run there and give the eager results."""
    hidden, inter, rows = 256, 512, 96

    def make_linear(i, o):
        torch.manual_seed(i * 7 + o)
        lin = nn.Linear(i, o, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            lin.weight.normal_(std=0.02)
        if kind in ("tensorwise", "rowwise"):
            cfg = float8_training.Float8LinearConfig(recipe=kind, pad_inner_dim=True)
            f8 = float8_training.Float8Linear.from_float(lin, cfg)
            f8.__class__ = float8_training.TrainingLinear
            return f8
        return te_linear.TELinear([lin], "fp8" if kind == "te_fp8" else "mxfp8")

    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, rows // 2, hidden, generator=g).to(torch.bfloat16).to(gpu)
    dy = (torch.randn(2, rows // 2, hidden, generator=g) * 1e-2).to(torch.bfloat16).to(gpu)
    results = []
    for compiled in (False, True):
        block = _Block(make_linear, hidden, inter).to(gpu).train()
        if compiled:
            block.compile(dynamic=True, backend="aot_eager")
        xg = x.clone().requires_grad_(True)
        y = block(xg)
        y.backward(dy)
        torch.cuda.synchronize()
        results.append((y.detach(), xg.grad, block.up.weight.grad, block.down.weight.grad))
    for a, b in zip(*results):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _count_calls(monkeypatch, module, name):
    calls = []
    real = getattr(module, name)

    def counted(*a, **k):
        calls.append(name)
        return real(*a, **k)

    monkeypatch.setattr(module, name, counted)
    return calls


def test_inference_forward_shares_quantize_launches(gpu, monkeypatch):
    """The FP8 linear and gated MLP quantize x and their weights in shared launches
    (ops.quantize_many) under no_grad, and in training too, where their backward reads the
    forward's own fp8 tensors as K-major operands (no transposed copy to make); outputs are
    bit-identical either way."""
    from bongard_amd import linear
    calls = _count_calls(monkeypatch, ops, "quantize_many")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(300, 256, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.nn.Parameter((torch.randn(384, 256, generator=g) * 0.05).to(torch.bfloat16).to(gpu))
    w_gu = torch.nn.Parameter((torch.randn(2 * 512, 256, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
    w_d = torch.nn.Parameter((torch.randn(256, 512, generator=g) * 0.014).to(torch.bfloat16).to(gpu))
    x16 = x[:288]
    y_train = linear.Fp8LinearFunction.apply(x16, w, None, None)
    assert calls == ["quantize_many"]    # training, K-major backward: shared launches
    with torch.no_grad():
        y_inf = linear.Fp8LinearFunction.apply(x16, w, None, None)
    assert calls == ["quantize_many"] * 2
    assert torch.equal(y_train.detach(), y_inf)
    with torch.inference_mode():         # any row count: no transposed copy is made
        y_odd = linear.Fp8LinearFunction.apply(x, w, None, None)
        xq, wq = ops.quantize(x), ops.quantize(w)
        y_sep = ops.gemm(xq.data, ops.E4M3, xq.meta, wq.data, ops.E4M3, wq.meta)
    assert calls == ["quantize_many"] * 3
    assert torch.equal(y_odd, y_sep)
    # the gated MLP's backward reads the forward's own fp8 tensors (K-major GEMM operands),
    # so its training forward makes no transposed copy and shares the launches too
    y_train = linear.Fp8GegluMlpFunction.apply(x16, w_gu, w_d, None, None, 512, False)
    assert len(calls) == 4
    with torch.no_grad():
        y_inf = linear.Fp8GegluMlpFunction.apply(x16, w_gu, w_d, None, None, 512, False)
    assert len(calls) == 5
    assert torch.equal(y_train.detach(), y_inf)

