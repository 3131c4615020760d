"""Pins the CPU oracle (oracle/fp8_oracle.py) before it is trusted as the GPU checker.

The reference ships no tests, fixtures or golden vectors for this path, and torchao /
TransformerEngine are not installed, so each oracle function is pinned by checks a
plausible mistake would fail: hand-computed known answers, a second independent encoder
(table-driven, from the OCP bit layout) on all 65,536 bf16 patterns, fp64 closed forms,
integer-exact matmuls, and torch's own ops where the oracle restates them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8_oracle as orc

E4M3, E5M2 = orc.E4M3, orc.E5M2


# ---- known answers (hand-computed from the OCP formats) ---------------------------------
E4M3_KNOWN = [
    (0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (-1.0, 0xB8), (448.0, 0x7E), (-448.0, 0xFE),
    (17.0, 0x58),            # 17 = 16 + 1, tie between 16 and 18 -> even mantissa (16)
    (19.0, 0x5A),            # tie between 18 and 20 -> 20
    (2.0 ** -6, 0x08),       # min normal
    (2.0 ** -9, 0x01),       # min subnormal
    (2.0 ** -10, 0x00),      # half the min subnormal: tie -> 0
    (1.5 * 2.0 ** -10, 0x01),
    (7 * 2.0 ** -9, 0x07),   # max subnormal
    (240.0, 0x77), (256.0, 0x78), (0.1, 0x1D),
    (500.0, 0x7E), (1e30, 0x7E), (-1e30, 0xFE),  # saturate
]
E5M2_KNOWN = [
    (0.0, 0x00), (-0.0, 0x80), (1.0, 0x3C), (57344.0, 0x7B), (-57344.0, 0xFB),
    (2.0 ** -14, 0x04), (2.0 ** -16, 0x01), (2.0 ** -17, 0x00), (3 * 2.0 ** -17, 0x02),
    (1.125, 0x3C),           # tie between 1 and 1.25 -> even (1)
    (1.375, 0x3E),           # tie between 1.25 and 1.5 -> 1.5
    (61440.0, 0x7B), (1e30, 0x7B),  # saturate (no inf through the saturating cast)
]


@pytest.mark.parametrize("fmt,table", [(E4M3, E4M3_KNOWN), (E5M2, E5M2_KNOWN)])
def test_known_answers(fmt, table):
    vals = torch.tensor([v for v, _ in table], dtype=torch.float32)
    want = torch.tensor([b for _, b in table], dtype=torch.uint8)
    got = orc.cast(vals, torch.tensor(1.0), fmt)
    assert got.tolist() == want.tolist()
    got_np = orc.cast_np(vals.numpy(), np.float32(1.0), fmt)
    assert got_np.tolist() == want.tolist()


def test_value_table_round_trip():
    for fmt, dt in ((E4M3, torch.float8_e4m3fn), (E5M2, torch.float8_e5m2)):
        table = orc.fp8_value_table(fmt)
        torch_vals = torch.arange(256, dtype=torch.uint8).view(dt).to(torch.float64).numpy()
        same = (table == torch_vals) | (np.isnan(table) & np.isnan(torch_vals))
        assert same.all()


# ---- two witnesses on every bf16 bit pattern ---------------------------------------------
ALL_BF16 = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
@pytest.mark.parametrize("scale", [1.0, 6.9457, 2.0 ** -13, 3.0e4, 4.48e14, 0.0, float("nan")])
def test_torch_cast_equals_table_encoder(fmt, scale):
    s = torch.tensor(scale, dtype=torch.float32)
    a = orc.cast(ALL_BF16, s, fmt).numpy()
    b = orc.cast_np(ALL_BF16.float().numpy(), np.float32(scale), fmt)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_nan_convention_is_torch_cpu(fmt):
    """The explicit NaN rule equals what torch's own clamp(x*s).to(fp8) yields on this CPU."""
    m = orc.FP8_MAX[fmt]
    xs = torch.tensor([float("nan"), -float("nan"), float("inf"), -float("inf"), 1.0, -2.0])
    for scale in (torch.tensor(2.0), torch.tensor(0.0), torch.tensor(float("nan"))):
        raw = torch.clamp(xs * scale, -m, m).to(orc.TORCH_FP8[fmt]).view(torch.uint8)
        assert orc.cast(xs, scale, fmt).tolist() == raw.tolist()


# ---- amax / scale ---------------------------------------------------------------------
def test_amax_exact_and_nan_propagating():
    x = torch.tensor([[1.0, -3.5], [2.0, 0.25]], dtype=torch.bfloat16)
    assert orc.amax(x).item() == 3.5
    x[0, 0] = float("nan")
    assert math.isnan(orc.amax(x).item())
    g = torch.Generator().manual_seed(0)
    y = torch.randn(300, 17, generator=g).to(torch.bfloat16)
    brute = max(abs(float(v)) for v in y.flatten().tolist())
    assert orc.amax(y).item() == brute


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_scale_closed_form(fmt):
    g = torch.Generator().manual_seed(1)
    amaxes = torch.cat([torch.rand(2000, generator=g) * 100,
                        torch.tensor([0.0, 1e-13, 1e-12, 64.5, 0.1035, 3.0e38])])
    for a in amaxes.tolist():
        s, si = orc.amax_to_scale(torch.tensor(a, dtype=torch.float32), fmt)
        want = np.float32(orc.FP8_MAX[fmt] / max(float(np.float32(a)), 1e-12))
        assert s.item() == float(want)
        assert si.item() == float(np.float32(1.0) / want)
        assert s.item() == float(orc.scale_np(float(np.float32(a)), fmt))


def test_scale_config1_probe_value():
    # BASELINE config 1 note: amax 64.5 -> scale 448 / 64.5 = 6.9457
    s, _ = orc.amax_to_scale(torch.tensor(64.5), E4M3)
    assert abs(s.item() - 448 / 64.5) < 1e-6 and s.dtype == torch.float32


# ---- dequantized matmul -----------------------------------------------------------------
def test_scaled_mm_integer_exact():
    """Power-of-two scales and small integers: the dequant matmul is exact."""
    a = torch.tensor([[1.0, 2.0, -3.0], [0.5, 0.0, 4.0]])
    b = torch.tensor([[2.0, 1.0, 1.0], [-1.0, 0.25, 2.0]])
    sa, sb = torch.tensor(4.0), torch.tensor(0.5)
    aq = orc.cast(a, sa, E4M3)
    bq = orc.cast(b, sb, E4M3)
    y = orc.scaled_mm(aq, sa, E4M3, bq, sb, E4M3)
    assert torch.equal(y, a @ b.T)
    y32 = orc.scaled_mm(aq, sa, E4M3, bq, sb, E4M3, precise=False)
    assert torch.equal(y32, a @ b.T)


def test_scaled_mm_transposition_and_bias():
    g = torch.Generator().manual_seed(2)
    a = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(7, 32, generator=g).to(torch.bfloat16)
    bias = torch.randn(7, generator=g).to(torch.bfloat16)
    aq, _, sa, _ = orc.quantize(a, E4M3)
    bq, _, sb, _ = orc.quantize(b, E4M3)
    y = orc.scaled_mm(aq, sa, E4M3, bq, sb, E4M3, bias=bias)
    deq_a = orc.dequant(aq, sa, E4M3).double()
    deq_b = orc.dequant(bq, sb, E4M3).double()
    for i in range(5):
        for j in range(7):
            want = sum(deq_a[i, k] * deq_b[j, k] for k in range(32)) + float(bias[j])
            assert abs(y[i, j].item() - want) <= 1e-6 * max(1.0, abs(want))


def test_segment_scales_equal_separate_mms():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4, 16, generator=g).to(torch.bfloat16)
    ws = [torch.randn(n, 16, generator=g).to(torch.bfloat16) * s for n, s in ((3, 1), (5, 9))]
    aq, _, sa, _ = orc.quantize(a, E4M3)
    qs = [orc.quantize(w, E4M3) for w in ws]
    fused = orc.scaled_mm(aq, sa, E4M3, torch.cat([q[0] for q in qs]), None, E4M3,
                          seg_ends=[3, 8], b_scales=[q[2] for q in qs])
    sep = torch.cat([orc.scaled_mm(aq, sa, E4M3, q[0], q[2], E4M3) for q in qs], 1)
    assert torch.equal(fused, sep)


# ---- gated GELU chain --------------------------------------------------------------------
def test_geglu_matches_formula_and_hf_mlp():
    g = torch.Generator().manual_seed(4)
    gate = (torch.randn(64, 32, generator=g) * 3).to(torch.bfloat16)
    up = torch.randn(64, 32, generator=g).to(torch.bfloat16)
    h = orc.geglu(gate, up)
    x = gate.double()
    want = 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    want = (want.to(torch.bfloat16).double() * up.double()).to(torch.bfloat16)
    diff = (h.double() - want.double()).abs()
    # a one-ulp change of the bf16 gelu moves the rounded product by at most two ulps
    # (plus an absolute 2^-20 * max|h| where fp32 cancels 1 + tanh to exactly zero)
    slack = 2.0 ** -20 * want.double().abs().max()
    assert (diff <= 2 * orc.bf16_ulp(want.float()).double() + slack).all()
    # fp32 evaluation of 1 + tanh(inner) cancels in the negative tail, so torch's fp32
    # chain and the fp64 formula differ by one bf16 ulp on a few percent of elements
    assert (diff > 0).float().mean() < 0.15
    # HF activation used by T5Gemma2MLP (gelu_pytorch_tanh) is the same op
    from transformers.activations import ACT2FN
    assert torch.equal(ACT2FN["gelu_pytorch_tanh"](gate) * up, h)


def test_geglu_bwd_against_finite_differences():
    g = torch.Generator().manual_seed(5)
    gate = torch.randn(8, 8, generator=g, dtype=torch.float64)
    up = torch.randn(8, 8, generator=g, dtype=torch.float64)
    dh = torch.randn(8, 8, generator=g, dtype=torch.float64)
    dg, du = orc.geglu_bwd(gate.to(torch.bfloat16), up.to(torch.bfloat16), dh.to(torch.bfloat16))

    def f(x):
        return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))

    gb, ub = gate.to(torch.bfloat16).double(), up.to(torch.bfloat16).double()
    eps = 1e-6
    dfdx = (f(gb + eps) - f(gb - eps)) / (2 * eps)
    want_dg = dh.to(torch.bfloat16).double() * ub * dfdx
    want_du = dh.to(torch.bfloat16).double() * f(gb)
    assert torch.allclose(dg.double(), want_dg, rtol=3e-2, atol=1e-3)
    assert torch.allclose(du.double(), want_du, rtol=2e-2, atol=1e-3)


# ---- RMSNorm ------------------------------------------------------------------------------
def test_rmsnorm_matches_hf_module():
    from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2RMSNorm
    norm = T5Gemma2RMSNorm(64, eps=1e-6)
    with torch.no_grad():
        norm.weight.normal_()
    x = torch.randn(10, 64).to(torch.bfloat16)
    assert torch.equal(orc.rmsnorm(x, norm.weight, 1e-6), norm(x))


# ---- delayed scaling ----------------------------------------------------------------------
def test_delayed_scaling_closed_form():
    d = orc.DelayedScaling(4, E4M3)
    s, si = d.begin()
    assert s == 1.0 and si == 1.0          # empty history keeps the initial scale
    d.end(2.0)
    s, _ = d.begin()
    assert s == np.float32(224.0)          # 448 / 2
    for a in (8.0, 1.0, 1.0, 1.0):
        d.end(a)
    s, _ = d.begin()                        # ring of 4 now holds 8, 1, 1, 1 (2 evicted)
    assert s == np.float32(56.0)
    d.end(float("inf"))
    s2, _ = d.begin()
    assert s2 == s                          # non-finite history keeps the previous scale


def test_delayed_quantizer_uses_previous_amaxes():
    """Each role's scale at step t comes from the amaxes of its steps < t only."""
    g = torch.Generator().manual_seed(12)
    xs = [(torch.randn(8, 16, generator=g) * s).to(torch.bfloat16) for s in (3.0, 0.5, 0.1)]
    q = orc.DelayedQuantizer(16)
    _, s1 = q("x", xs[0], E4M3)
    assert float(s1) == 1.0
    _, s2 = q("x", xs[1], E4M3)
    assert float(s2) == float(np.float32(448.0 / float(orc.amax(xs[0]))))
    _, s3 = q("x", xs[2], E4M3)
    m = max(float(orc.amax(xs[0])), float(orc.amax(xs[1])))
    assert float(s3) == float(np.float32(448.0 / m))
    _, sw = q("w", xs[2], E5M2)                # roles keep separate histories
    assert float(sw) == 1.0


# ---- axiswise scaling (torchao rowwise recipes) -------------------------------------------
def _pow2_floor(v):
    """Largest power of two <= v (> 0, finite) from frexp: independent of log2 rounding."""
    m, e = math.frexp(v)
    return math.ldexp(0.5, e)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_pow2_rounding_equals_mantissa_clear_on_all_bf16_amaxes(fmt):
    """torchao's exp2(floor(log2(scale))) is, on every scale a bf16 amax can produce
    (incl. the 1e-12 clamp), the scale with its mantissa cleared (the kernels' method).
    fp32 log2 rounds up to the next integer only within ~11 ulp below a power of two,
    which fp8_max / bf16 never reaches (fp8_max is 1.75 * 2^k, bf16 has 8 mantissa bits)."""
    bits = torch.arange(0, 0x7F80, dtype=torch.int32).to(torch.int16)
    amax = bits.view(torch.bfloat16).float()
    raw = orc.amax_to_scale_axiswise(amax, fmt, pow2=False)
    got = orc.amax_to_scale_axiswise(amax, fmt, pow2=True)
    cleared = (raw.view(torch.int32) & 0xFF800000).view(torch.float32)
    assert torch.equal(got, cleared)
    assert bool((got <= raw).all()) and bool((got * 2 > raw).all())
    for a in (3.0, 0.1, 448.0, 1e-3):
        s = orc.amax_to_scale_axiswise(torch.tensor([a]).to(torch.bfloat16).float(), fmt)
        want = _pow2_floor(float(np.float32(orc.FP8_MAX[fmt] / float(torch.tensor(a).to(torch.bfloat16)))))
        assert s.item() == want
    assert orc.amax_to_scale_axiswise(torch.tensor([0.0]), fmt).item() == _pow2_floor(
        float(np.float32(orc.FP8_MAX[fmt] / 1e-12)))


def test_pow2_known_answers():
    assert orc.amax_to_scale_axiswise(torch.tensor([3.0]), E4M3).item() == 128.0   # 149.3
    assert orc.amax_to_scale_axiswise(torch.tensor([448.0]), E4M3).item() == 1.0
    assert orc.amax_to_scale_axiswise(torch.tensor([449.0]), E4M3).item() == 0.5   # 0.998
    assert orc.amax_to_scale_axiswise(torch.tensor([1.0]), E5M2).item() == 32768.0  # 57344


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
@pytest.mark.parametrize("dim", [-1, 0])
def test_axiswise_equals_per_slice_tensorwise(fmt, dim):
    """Brute force: each row (dim -1) / column (dim 0) quantized on its own with the
    pinned tensorwise amax, scale and cast, the scale floored to a power of two via frexp."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(37, 48, generator=g)
    x[3] *= 300.0
    x[:, 5] *= 1e-3
    x[7] = 0.0
    x[:, 11] = 0.0
    x = x.to(torch.bfloat16)
    q, s = orc.quantize_axiswise(x, fmt, dim)
    n = x.shape[0] if dim == -1 else x.shape[1]
    for i in range(n):
        sl = x[i] if dim == -1 else x[:, i]
        sc = _pow2_floor(float(orc.amax_to_scale(orc.amax(sl), fmt)[0]))
        want = orc.cast(sl, torch.tensor(sc, dtype=torch.float32), fmt)
        got_q = q[i] if dim == -1 else q[:, i]
        got_s = s[i, 0] if dim == -1 else s[0, i]
        assert got_s.item() == sc
        assert torch.equal(got_q, want)


def test_axiswise_nan_and_inf_rows():
    x = torch.randn(4, 16).to(torch.bfloat16)
    x[1, 3] = float("nan")
    x[2, 5] = float("inf")
    q, s = orc.quantize_axiswise(x, E4M3, -1)
    assert math.isnan(s[1, 0].item()) and bool((q[1] == 0x7F).all())   # NaN scale: +NaN bytes
    assert s[2, 0].item() == 0.0                                         # 448 / inf
    assert q[2, 5].item() == 0xFF and bool((q[2, :5] & 0x7F == 0).all())  # inf * 0 = -NaN


def test_scaled_mm_with_axis_scales_brute_force():
    g = torch.Generator().manual_seed(22)
    a = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    b = (torch.randn(7, 32, generator=g) * 0.02).to(torch.bfloat16)
    aq, sa = orc.quantize_axiswise(a, E4M3, -1)
    bq, sb = orc.quantize_axiswise(b, E4M3, -1)
    y = orc.scaled_mm(aq, sa, E4M3, bq, sb, E4M3)
    da = aq.view(torch.float8_e4m3fn).double()
    db = bq.view(torch.float8_e4m3fn).double()
    for i in range(5):
        for j in range(7):
            want = sum(da[i, k] * db[j, k] for k in range(32)) / (float(sa[i, 0]) * float(sb[j, 0]))
            assert abs(y[i, j].item() - want) <= 1e-6 * max(1e-30, abs(want))


@pytest.mark.parametrize("recipe", ["rowwise", "rowwise_with_gw_hp"])
def test_linear_axiswise_recipes_track_the_bf16_linear(recipe):
    """Shapes, and every output within e4m3 error of the unquantized products (a
    transposed operand or a scale on the wrong axis would be far off)."""
    g = torch.Generator().manual_seed(23)
    x = torch.randn(64, 48, generator=g).to(torch.bfloat16)
    w = (torch.randn(32, 48, generator=g) * 0.05).to(torch.bfloat16)
    w[:, 3] *= 40.0   # an outlier input feature: per-column W scales matter for dX
    dy = (torch.randn(64, 32, generator=g) * 1e-3).to(torch.bfloat16)
    y, dx, dw = orc.linear_fwd_bwd_axiswise(x, w, dy, recipe)
    ref_y = x.double() @ w.double().t()
    ref_dx = dy.double() @ w.double()
    ref_dw = dy.double().t() @ x.double()
    for got, ref in ((y, ref_y), (dx, ref_dx), (dw, ref_dw)):
        assert got.shape == ref.shape
        rel = (got.double() - ref).norm() / ref.norm()
        assert rel < 0.08, rel
    if recipe == "rowwise_with_gw_hp":
        assert torch.equal(dw, ref_dw.float())


# ---- MXFP8 (TE MXFP8BlockScaling) ----------------------------------------------------------
def _ceil_log2(v):
    m, e = math.frexp(v)          # v = m * 2^e, 0.5 <= m < 1
    return e - 1 if m == 0.5 else e


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_mx_exponent_is_ceil_log2_on_all_bf16_amaxes(fmt):
    bits = torch.arange(0, 0x7F81, dtype=torch.int32).to(torch.int16)   # 0 .. +inf
    amax = bits.view(torch.bfloat16).float()
    got = orc.mx_exponent(amax, fmt)
    rcp = float(np.float32(1.0 / orc.FP8_MAX[fmt]))
    for a, e in zip(amax.tolist(), got.tolist()):
        val = float(np.float32(np.float32(a) * np.float32(rcp)))
        if math.isinf(val):
            want = 0xFE
        elif val == 0.0:
            want = 0
        else:
            want = min(max(127 + _ceil_log2(val), 0), 0xFE)
        assert e == want, (a, e, want)
    assert orc.mx_exponent(torch.tensor([float("nan")]), fmt).item() == 0xFF


def test_mx_known_answers():
    x = torch.zeros(2, 32)
    x[0, 3] = 448.0        # amax 448: val exactly 1.0 -> e = 127, q(448) = 0x7E
    x[1, 0] = 1.0          # amax 1: val = 1/448 -> 2^-8 -> e = 119, x * 256 = 256 -> 0x78
    x[1, 1] = -0.5
    q, e = orc.quantize_mx(x.to(torch.bfloat16), E4M3)
    assert e.tolist() == [[127], [119]]
    assert q[0, 3].item() == 0x7E and q[1, 0].item() == 0x78 and q[1, 1].item() == 0xF0


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_mx_block_max_lands_in_top_binade(fmt):
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(64, 256, generator=g) * torch.logspace(-20, 20, 64)[:, None]).to(torch.bfloat16)
    q, e = orc.quantize_mx(x, fmt)
    blocks = x.float().abs().reshape(64, 8, 32).amax(-1)
    scaled = blocks.double() * torch.pow(2.0, (127 - e).double())
    m = orc.FP8_MAX[fmt]
    assert bool((scaled > m / 2).all()) and bool((scaled <= m * (1 + 2 ** -20)).all())
    deq = orc.dequant_mx(q, e, fmt)
    step = 2.0 ** -3 if fmt == E4M3 else 2.0 ** -2          # half the top-binade spacing
    err = (deq - x.double()).abs().reshape(64, 8, 32).amax(-1)
    assert bool((err <= step * blocks.double() + 1e-300).all())


def test_mx_columnwise_is_rowwise_of_transpose_and_padding():
    g = torch.Generator().manual_seed(32)
    x = torch.randn(96, 64, generator=g).to(torch.bfloat16)
    qc, ec = orc.quantize_mx(x, E4M3, 0)
    qr, er = orc.quantize_mx(x.t().contiguous(), E4M3, -1)
    assert torch.equal(qc, qr) and torch.equal(ec, er) and qc.shape == (64, 96)
    rows = orc.mx_scale_rows(ec)          # 3 blocks -> 4 bytes, the last one 127
    assert rows.shape == (64, 4) and bool((rows[:, 3] == 127).all())


def test_scaled_mm_mx_brute_force():
    g = torch.Generator().manual_seed(33)
    a = (torch.randn(5, 64, generator=g) * torch.tensor([1e-3, 1.0, 30.0, 0.2, 5.0])[:, None]).to(torch.bfloat16)
    b = (torch.randn(7, 64, generator=g) * 0.02).to(torch.bfloat16)
    aq, ae = orc.quantize_mx(a, E4M3)
    bq, be = orc.quantize_mx(b, E4M3)
    y = orc.scaled_mm_mx(aq, ae, bq, be)
    da = aq.view(torch.float8_e4m3fn).double()
    db = bq.view(torch.float8_e4m3fn).double()
    for i in range(5):
        for j in range(7):
            want = sum(da[i, k] * db[j, k] * 2.0 ** (int(ae[i, k // 32]) - 127)
                       * 2.0 ** (int(be[j, k // 32]) - 127) for k in range(64))
            assert abs(y[i, j].item() - want) <= 1e-6 * max(abs(want), 1e-30)


def test_mx_chains_track_the_bf16_products():
    """The MXFP8 linear and MLP chains: shapes, and every output within MX e4m3 error of
    the unquantized products (a transposed operand or misplaced block would be far off)."""
    g = torch.Generator().manual_seed(34)
    x = torch.randn(64, 96, generator=g).to(torch.bfloat16)
    w = (torch.randn(32, 96, generator=g) * 0.05).to(torch.bfloat16)
    dy = (torch.randn(64, 32, generator=g) * 1e-3).to(torch.bfloat16)
    y, dx, dw = orc.linear_fwd_bwd_mx(x, w, dy)
    for got, ref in ((y, x.double() @ w.double().t()), (dx, dy.double() @ w.double()),
                     (dw, dy.double().t() @ x.double())):
        assert got.shape == ref.shape
        assert (got.double() - ref).norm() / ref.norm() < 0.08
    wg = (torch.randn(64, 96, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(64, 96, generator=g) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(96, 64, generator=g) * 0.05).to(torch.bfloat16)
    dyo = (torch.randn(64, 96, generator=g) * 1e-3).to(torch.bfloat16)
    out = orc.mlp_fwd_bwd_mx(x, wg, wu, wd, dyo)
    xr = x.double().requires_grad_(True)
    gu = [t.double().requires_grad_(True) for t in (wg, wu, wd)]
    yr = (F.gelu(xr @ gu[0].t(), approximate="tanh") * (xr @ gu[1].t())) @ gu[2].t()
    yr.backward(dyo.double())
    for got, ref in ((out["y"], yr.detach()), (out["dx"], xr.grad),
                     (out["dwgu"], torch.cat([gu[0].grad, gu[1].grad])), (out["dwd"], gu[2].grad)):
        assert got.shape == ref.shape
        assert (got.double() - ref).norm() / ref.norm() < 0.12


# ---- tensorwise chains (torchao tensorwise / TE Float8CurrentScaling HYBRID) -------------
# linear_fwd_bwd, mlp_forward and mlp_backward restate torchao's tensorwise forward and
# backward (bongard/float8_training.py:16-22) and TEMLP.forward (bongard/te_linear.py:98-103).
# Two kinds of check pin them: (1) every output within e4m3 / e5m2 error of fp64 autograd of
# the unquantized bf16 linear / MLP, on non-square shapes whose tensor roles have scales
# orders of magnitude apart (x ~ 1 with outliers, W ~ 0.02, dy ~ 1e-3), so a scale taken
# from the wrong role, a transposed operand or a gate/up mix-up is far outside the bound;
# (2) inputs whose quantization is exact (power-of-two scales, values on the fp8 grid), where
# the chains must reproduce the exact products bit for bit and H must equal the Hugging Face
# T5Gemma2MLP activation on them.
def _rel(got, ref):
    return ((got.double() - ref.double()).norm() / ref.double().norm()).item()


def _tensorwise_inputs(seed, M=48, K=96, N=80):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:3]] *= 20.0
    w = torch.randn(N, K, generator=g) * 0.02
    dy = torch.randn(M, N, generator=g) * 1e-3
    return x.to(torch.bfloat16), w.to(torch.bfloat16), dy.to(torch.bfloat16)


def test_linear_fwd_bwd_tracks_fp64_autograd():
    x, w, dy = _tensorwise_inputs(41)
    y, dx, dw = orc.linear_fwd_bwd(x, w, dy)
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    yr = xr @ wr.t()
    yr.backward(dy.double())
    assert y.shape == yr.shape and dx.shape == xr.shape and dw.shape == wr.shape
    assert _rel(y, yr.detach()) < 0.05         # e4m3 x e4m3
    assert _rel(dx, xr.grad) < 0.08            # e5m2 x e4m3
    assert _rel(dw, wr.grad) < 0.08
    # the roles' scales differ by orders of magnitude: dividing by the wrong one is far off
    _, _, xs, _ = orc.quantize(x, E4M3)
    _, _, ws, _ = orc.quantize(w, E4M3)
    _, _, ds, _ = orc.quantize(dy, E5M2)
    logs = sorted(math.log10(float(s)) for s in (xs, ws, ds))
    assert logs[1] - logs[0] > 1 and logs[2] - logs[1] > 1


def _grid_tensor(gen, shape, top, unit):
    """Integers in [-top, top] times ``unit`` with one element forced to +top * unit, so the
    amax is top * unit; every value is exactly representable after scaling when top * unit
    maps to fp8_max by a power of two."""
    v = torch.randint(-top, top + 1, shape, generator=gen).double()
    v.view(-1)[0] = top
    return (v * unit).to(torch.bfloat16)


def test_linear_fwd_bwd_exact_on_the_fp8_grid():
    """amax_x = 7 * 2^-2 = 448 * 2^-8 (scale 2^8), amax_w = 7 * 2^-6 (scale 2^12), amax_dy
    = 7 * 2^-12 = 57344 * 2^-25 (scale 2^25): every quantization is exact, so y, dx and dw
    must equal the exact products (all partial sums are exact in fp32 and fp64)."""
    g = torch.Generator().manual_seed(42)
    M, K, N = 48, 96, 80
    x = _grid_tensor(g, (M, K), 7, 2.0 ** -2)
    w = _grid_tensor(g, (N, K), 7, 2.0 ** -6)
    dy = _grid_tensor(g, (M, N), 7, 2.0 ** -12)
    for t, fmt, want in ((x, E4M3, 2.0 ** 8), (w, E4M3, 2.0 ** 12), (dy, E5M2, 2.0 ** 25)):
        _, _, s, _ = orc.quantize(t, fmt)
        assert float(s) == want
    y, dx, dw = orc.linear_fwd_bwd(x, w, dy)
    assert torch.equal(y, (x.double() @ w.double().t()).float())
    assert torch.equal(dx, (dy.double() @ w.double()).float())
    assert torch.equal(dw, (dy.double().t() @ x.double()).float())


def _hf_mlp(wg, wu, wd):
    import types

    from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2MLP
    cfg = types.SimpleNamespace(hidden_size=wg.shape[1], intermediate_size=wg.shape[0],
                                hidden_activation="gelu_pytorch_tanh", dropout_rate=0.0)
    m = T5Gemma2MLP(cfg).to(torch.bfloat16)
    with torch.no_grad():
        m.gate_proj.weight.copy_(wg)
        m.up_proj.weight.copy_(wu)
        m.down_proj.weight.copy_(wd)
    return m


def test_mlp_forward_exact_on_the_fp8_grid_and_hf_activation():
    """x, [W_gate; W_up] on the e4m3 grid with power-of-two scales: g and u equal the
    bf16-rounded exact products of the right halves, and H equals the Hugging Face
    T5Gemma2MLP activation act_fn(gate_proj(x)) * up_proj(x) bit for bit."""
    gen = torch.Generator().manual_seed(43)
    M, K, I = 32, 64, 48
    x = _grid_tensor(gen, (M, K), 7, 2.0 ** -2)
    wg = _grid_tensor(gen, (I, K), 7, 2.0 ** -6)
    wu = _grid_tensor(gen, (I, K), 5, 2.0 ** -6)     # amax of [Wg; Wu] stays 7 * 2^-6
    wd = (torch.randn(K, I, generator=gen) * 0.02).to(torch.bfloat16)
    out = orc.mlp_forward(x, wg, wu, wd)
    assert float(out["x_scale"]) == 2.0 ** 8 and float(out["w_scales"][0]) == 2.0 ** 12
    assert torch.equal(out["g"], (x.double() @ wg.double().t()).to(torch.bfloat16))
    assert torch.equal(out["u"], (x.double() @ wu.double().t()).to(torch.bfloat16))
    m = _hf_mlp(wg, wu, wd)
    with torch.no_grad():
        hf_g, hf_u = m.gate_proj(x), m.up_proj(x)
        hf_h = m.act_fn(hf_g) * hf_u
    assert torch.equal(hf_g, out["g"]) and torch.equal(hf_u, out["u"])
    assert torch.equal(out["h"], hf_h)
    # H's own quantization and the down GEMM: within e4m3 error of the HF bf16 output
    with torch.no_grad():
        assert _rel(out["y"], m(x)) < 0.05


def test_mlp_chains_track_fp64_autograd():
    """mlp_forward + mlp_backward against fp64 autograd of the unquantized MLP with the
    reference's rounding points (g, u, gelu(g), H rounded to bf16): shapes, and every output
    within the compounded e4m3 / e5m2 error. A gate/up swap, a dgrad on W instead of W^T or
    a dGU scale on the wrong tensor is far outside these bounds."""
    gen = torch.Generator().manual_seed(44)
    M, K, I = 64, 96, 80
    x = torch.randn(M, K, generator=gen)
    x[:, :2] *= 20.0
    x = x.to(torch.bfloat16)
    wg = (torch.randn(I, K, generator=gen) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, K, generator=gen) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(K, I, generator=gen) * 0.014).to(torch.bfloat16)
    dy = (torch.randn(M, K, generator=gen) * 1e-3).to(torch.bfloat16)
    fwd = orc.mlp_forward(x, wg, wu, wd)
    dx, dwgu, dwd, dgu = orc.mlp_backward(fwd, x, wg, wu, wd, dy)
    xr = x.double().requires_grad_(True)
    ws = [t.double().requires_grad_(True) for t in (wg, wu, wd)]
    gate, up = xr @ ws[0].t(), xr @ ws[1].t()
    h = F.gelu(gate, approximate="tanh") * up
    yr = h @ ws[2].t()
    gate.retain_grad()
    up.retain_grad()
    yr.backward(dy.double())
    assert fwd["y"].shape == yr.shape and dx.shape == xr.shape
    assert dwgu.shape == (2 * I, K) and dwd.shape == wd.shape and dgu.shape == (M, 2 * I)
    assert _rel(fwd["g"], gate.detach()) < 0.05 and _rel(fwd["u"], up.detach()) < 0.05
    assert _rel(fwd["h"], h.detach()) < 0.08
    assert _rel(fwd["y"], yr.detach()) < 0.10
    assert _rel(dgu, torch.cat([gate.grad, up.grad], 1)) < 0.12
    assert _rel(dx, xr.grad) < 0.15
    assert _rel(dwgu, torch.cat([ws[0].grad, ws[1].grad])) < 0.15
    assert _rel(dwd, ws[2].grad) < 0.12
    # split gate/up scales (torchao, split TE): the same chain with one scale per half
    fwd2 = orc.mlp_forward(x, wg, wu, wd, shared_gate_up_scale=False)
    assert float(fwd2["w_scales"][0]) != float(fwd2["w_scales"][1])
    assert _rel(fwd2["y"], yr.detach()) < 0.10


def test_mlp_backward_exact_dh_on_the_fp8_grid():
    """dy and W_down on their fp8 grids with power-of-two scales make dH = dY8 . Wd8 exact:
    the chain's dGU must equal torch autograd of the HF activation at bf16(dy @ W_down),
    and dW_down must equal dy^T . H8 / scale_H computed from H's own pinned quantization."""
    gen = torch.Generator().manual_seed(45)
    M, K, I = 32, 64, 48
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(I, K, generator=gen) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(I, K, generator=gen) * 0.05).to(torch.bfloat16)
    wd = _grid_tensor(gen, (K, I), 7, 2.0 ** -6)
    dy = _grid_tensor(gen, (M, K), 7, 2.0 ** -12)
    fwd = orc.mlp_forward(x, wg, wu, wd)
    assert float(fwd["wd_scale"]) == 2.0 ** 12
    dx, dwgu, dwd, dgu = orc.mlp_backward(fwd, x, wg, wu, wd, dy)
    dh = (dy.double() @ wd.double()).to(torch.bfloat16)
    from transformers.activations import ACT2FN
    gr = fwd["g"].clone().requires_grad_(True)
    ur = fwd["u"].clone().requires_grad_(True)
    (ACT2FN["gelu_pytorch_tanh"](gr) * ur).backward(dh)
    assert torch.equal(dgu, torch.cat([gr.grad, ur.grad], 1))
    hq, _, hs, _ = orc.quantize(fwd["h"], E4M3)
    h_deq = hq.view(torch.float8_e4m3fn).double() / float(hs)
    ref = dy.double().t() @ h_deq
    assert (dwd.double() - ref).abs().max() <= 1e-6 * ref.abs().max()   # fp32 output rounding


def test_mlp_backward_split_scales_exact_on_the_fp8_grid():
    """Split gate/up scales (BONGARD_TE_SPLIT_GATE_UP=1: two TELinears, bongard/te_linear.py
    :93-95,98-103). x, W_gate, W_up, W_down and dy lie on their fp8 grids with power-of-two
    scales, W_gate's (2^12) and W_up's (2^10) a factor 4 apart, so every forward GEMM and dH
    are exact. Each of dG, dU then has its own e5m2 scale (not the one a shared dGU scale
    would give), dW_gate / dW_up are exactly dĜ^T X / dÛ^T X with each half dequantized by
    its own scale, and dX is the bf16 sum of the two bf16 dgrads dĜ Wg and dÛ Wu. A swapped
    half, a W half dequantized with the other half's scale (off by exactly 4) or one shared
    dGU scale fails the bit-for-bit checks."""
    gen = torch.Generator().manual_seed(46)
    M, K, I = 32, 64, 48
    x = _grid_tensor(gen, (M, K), 7, 2.0 ** -2)
    wg = _grid_tensor(gen, (I, K), 7, 2.0 ** -6)
    wu = _grid_tensor(gen, (I, K), 7, 2.0 ** -4)
    wd = _grid_tensor(gen, (K, I), 7, 2.0 ** -6)
    dy = _grid_tensor(gen, (M, K), 7, 2.0 ** -12)
    fwd = orc.mlp_forward(x, wg, wu, wd, shared_gate_up_scale=False)
    assert [float(s) for s in fwd["w_scales"]] == [2.0 ** 12, 2.0 ** 10]
    assert torch.equal(fwd["g"], (x.double() @ wg.double().t()).to(torch.bfloat16))
    assert torch.equal(fwd["u"], (x.double() @ wu.double().t()).to(torch.bfloat16))
    dx, dwgu, dwd, dgu = orc.mlp_backward(fwd, x, wg, wu, wd, dy, shared_gate_up_scale=False)
    assert dx.shape == (M, K) and dwgu.shape == (2 * I, K) and dwd.shape == (K, I)
    # dGU itself: the same exact-dH chain as the shared form
    _, _, _, dgu_shared = orc.mlp_backward(fwd, x, wg, wu, wd, dy)
    assert torch.equal(dgu, dgu_shared)
    dg, du = dgu[:, :I], dgu[:, I:]
    deq = []
    for d in (dg, du):
        q, _, s, _ = orc.quantize(d, E5M2)
        deq.append(orc.dequant(q, s, E5M2).double())
    # each half's own scale differs from the shared dGU scale, and changes the values
    _, _, s_shared, _ = orc.quantize(dgu, E5M2)
    q_sh = orc.cast(dg, s_shared, E5M2)
    assert not torch.equal(orc.dequant(q_sh, s_shared, E5M2).double(), deq[0]) or \
        not torch.equal(orc.dequant(orc.cast(du, s_shared, E5M2), s_shared, E5M2).double(),
                        deq[1])
    assert torch.equal(dwgu[:I], (deq[0].t() @ x.double()).float())
    assert torch.equal(dwgu[I:], (deq[1].t() @ x.double()).float())
    part_g = (deq[0] @ wg.double()).float().to(torch.bfloat16)
    part_u = (deq[1] @ wu.double()).float().to(torch.bfloat16)
    assert torch.equal(dx, (part_g + part_u).float())
    # the shared-scale backward of the same forward would not give these bits
    dx_sh, dwgu_sh, _, _ = orc.mlp_backward(fwd, x, wg, wu, wd, dy)
    assert not torch.equal(dx_sh, dx) and not torch.equal(dwgu_sh, dwgu)


def test_mlp_backward_split_scales_tracks_fp64_autograd():
    """The split-scale chain against fp64 autograd of the unquantized MLP, with W_up's
    scale ~25x W_gate's and dy ~1e-3: every gradient within the compounded e4m3 / e5m2
    error; a half dequantized with the other half's scale is off by ~25x."""
    gen = torch.Generator().manual_seed(47)
    M, K, I = 64, 96, 80
    x = torch.randn(M, K, generator=gen)
    x[:, :2] *= 20.0
    x = x.to(torch.bfloat16)
    wg = (torch.randn(I, K, generator=gen) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, K, generator=gen) * 0.5).to(torch.bfloat16)
    wd = (torch.randn(K, I, generator=gen) * 0.014).to(torch.bfloat16)
    dy = (torch.randn(M, K, generator=gen) * 1e-3).to(torch.bfloat16)
    fwd = orc.mlp_forward(x, wg, wu, wd, shared_gate_up_scale=False)
    ws = [float(s) for s in fwd["w_scales"]]
    assert ws[0] / ws[1] > 10
    dx, dwgu, dwd, dgu = orc.mlp_backward(fwd, x, wg, wu, wd, dy, shared_gate_up_scale=False)
    xr = x.double().requires_grad_(True)
    wr = [t.double().requires_grad_(True) for t in (wg, wu, wd)]
    gate, up = xr @ wr[0].t(), xr @ wr[1].t()
    h = F.gelu(gate, approximate="tanh") * up
    yr = h @ wr[2].t()
    gate.retain_grad()
    up.retain_grad()
    yr.backward(dy.double())
    assert _rel(fwd["y"], yr.detach()) < 0.10
    assert _rel(dgu, torch.cat([gate.grad, up.grad], 1)) < 0.12
    assert _rel(dx, xr.grad) < 0.15
    assert _rel(dwgu[:I], wr[0].grad) < 0.15
    assert _rel(dwgu[I:], wr[1].grad) < 0.15
    assert _rel(dwd, wr[2].grad) < 0.12


# ---- NVFP4 (TE 'nvfp4', bongard/te_linear.py:17,38) --------------------------------------
# Pinned by: e2m1 known answers and an independent nearest-value search with exact
# (fraction) comparisons over a dense sweep and every midpoint; a scalar restatement built
# on the table-driven e4m3 encoder (encode_fp8_np) and that search, bit for bit on small
# tensors; known answers of whole blocks; the reconstruction bound each block's rounding
# implies; columnwise = rowwise of the transpose; a scalar brute-force GEMM.
from fractions import Fraction  # noqa: E402


def _e2m1_nearest(v: float) -> int:
    """Independent e2m1 rounding: nearest grid value (exact comparisons), ties to the
    even code, saturating at 6; the sign bit copied from v."""
    a = Fraction(abs(v)) if math.isfinite(v) else Fraction(100)
    best = None
    for code, g in enumerate(orc.E2M1_VALUES):
        d = abs(a - Fraction(g))
        if best is None or d < best[0] or (d == best[0] and code % 2 == 0):
            best = (d, code)
    return best[1] | (8 if math.copysign(1.0, v) < 0 else 0)


def test_e2m1_known_answers():
    cases = [(0.0, 0), (0.25, 0), (0.2500001, 1), (0.5, 1), (0.75, 2), (1.0, 2), (1.25, 2),
             (1.26, 3), (1.5, 3), (1.75, 4), (2.0, 4), (2.5, 4), (2.51, 5), (3.0, 5),
             (3.5, 6), (4.0, 6), (5.0, 6), (5.01, 7), (6.0, 7), (7.5, 7), (1e30, 7),
             (float("inf"), 7), (-0.0, 8), (-0.3, 9), (-6.0, 15)]
    got = orc.e2m1_code(torch.tensor([v for v, _ in cases], dtype=torch.float32))
    assert got.tolist() == [c for _, c in cases]
    assert orc.e2m1_decode(torch.arange(16, dtype=torch.uint8)).tolist() == \
        [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def test_e2m1_rounding_equals_nearest_even_search():
    grid = torch.linspace(-8.0, 8.0, 4097, dtype=torch.float32)
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=torch.float32)
    eps = torch.tensor([1.0 - 2 ** -23, 1.0, 1.0 + 2 ** -22], dtype=torch.float32)
    near = (mids[:, None] * eps[None, :]).flatten()
    vals = torch.cat([grid, near, -near])
    got = orc.e2m1_code(vals)
    want = [_e2m1_nearest(float(v)) for v in vals]
    assert got.tolist() == want


def _nvfp4_scalar(x_rows):
    """Scalar restatement on numpy float32 with the table-driven e4m3 encoder and the
    independent e2m1 search: (codes per element, scale byte per block, S_enc)."""
    xf = np.asarray(x_rows, dtype=np.float32)
    amax_v = float(np.max(np.abs(xf)))
    s_enc = np.float32(orc.NVFP4_GLOBAL / max(amax_v, 1e-12))
    table = orc.fp8_value_table(E4M3)
    codes, sbytes = [], []
    for row in xf:
        rc, rs = [], []
        for k in range(0, len(row), 16):
            blk = row[k:k + 16]
            v = np.float32(np.float32(np.max(np.abs(blk)) / np.float32(6.0)) * s_enc)
            sb = int(orc.encode_fp8_np(np.clip(np.array([v]), -448, 448), E4M3)[0])
            s = np.float32(table[sb])
            mult = np.float32(0.0) if s == 0 else np.float32(s_enc / s)
            rc += [_e2m1_nearest(float(np.float32(e * mult))) for e in blk]
            rs.append(sb)
        codes.append(rc)
        sbytes.append(rs)
    return codes, sbytes, s_enc


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_nvfp4_quantize_equals_scalar_restatement(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(6, 64, generator=g) * torch.rand(6, 1, generator=g) * 10
    x[0, :16] = 0.0                      # an all-zero block: scale 0, codes 0
    x[1, 3] = 1e-6                       # tiny beside its block's values
    x = x.to(torch.bfloat16)
    packed, sb, s_enc, s_dec, _ = orc.quantize_nvfp4(x)
    codes, sbytes, s_enc_ref = _nvfp4_scalar(x.float().numpy())
    assert float(s_enc) == float(s_enc_ref)
    assert float(s_dec) == float(np.float32(1.0 / float(s_enc)))
    assert sb.tolist() == sbytes
    unpacked = torch.stack([packed & 0xF, packed >> 4], -1).reshape(6, 64)
    assert unpacked.tolist() == codes


def test_nvfp4_known_answers():
    x = torch.zeros(1, 32)
    x[0, 0] = 6.0        # amax 6: S_enc = 448, block 0 scale 448 (0x7E), multiplier 1
    x[0, 1] = -1.0
    x[0, 16] = 0.75      # block 1: b / 6 * 448 = 56 = 1.75 * 2^5 (0x66), multiplier 8: -> 6
    x[0, 17] = 0.0625    # 0.0625 * 8 = 0.5
    x[0, 18] = 0.03125   # 0.25: the tie rounds to 0
    packed, sb, s_enc, s_dec, _ = orc.quantize_nvfp4(x.to(torch.bfloat16))
    assert float(s_enc) == 448.0 and sb.tolist() == [[0x7E, 0x66]]
    codes = torch.stack([packed & 0xF, packed >> 4], -1).reshape(-1)
    assert codes[:2].tolist() == [7, 10] and codes[16:19].tolist() == [7, 1, 0]
    deq = orc.dequant_nvfp4(packed, sb)     # e2m1 * s, exact: 6 * 448, -1 * 448, 6 * 56, 0.5 * 56
    assert deq[0, :2].tolist() == [2688.0, -448.0] and deq[0, 16:18].tolist() == [336.0, 28.0]
    back = deq * s_dec                       # S_dec = f32(1 / 448) is not exact
    assert torch.allclose(back[0, [0, 1, 16, 17]], torch.tensor([6.0, -1.0, 0.75, 0.0625]),
                          rtol=2 ** -23, atol=0)


def test_nvfp4_reconstruction_bound_and_columnwise():
    """|x - x^| <= one unit of the block's e2m1 grid (s / S_enc; the largest half-step
    is 1 and saturation costs less); the columnwise copy is the rowwise quantization of
    the transpose."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(48, 80, generator=g) * torch.rand(48, 1, generator=g) * 3).to(torch.bfloat16)
    packed, sb, s_enc, s_dec, _ = orc.quantize_nvfp4(x)
    deq = orc.dequant_nvfp4(packed, sb) * s_dec
    unit = (sb.view(torch.float8_e4m3fn).float() / s_enc).repeat_interleave(16, dim=1)
    assert bool(((deq - x.float()).abs() <= unit * (1 + 1e-6)).all())
    pc, sc, se2, _, _ = orc.quantize_nvfp4(x, axis=0)
    pt, st, se3, _, _ = orc.quantize_nvfp4(x.t().contiguous())
    assert torch.equal(pc, pt) and torch.equal(sc, st) and float(se2) == float(se3) == float(s_enc)


def test_scaled_mm_nvfp4_brute_force():
    g = torch.Generator().manual_seed(6)
    a = torch.randn(3, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(4, 32, generator=g).to(torch.bfloat16)
    pa, sa, _, da, _ = orc.quantize_nvfp4(a)
    pb, sb, _, db, _ = orc.quantize_nvfp4(b)
    got = orc.scaled_mm_nvfp4(pa, sa, da, pb, sb, db)
    A = orc.dequant_nvfp4(pa, sa).tolist()
    B = orc.dequant_nvfp4(pb, sb).tolist()
    for i in range(3):
        for j in range(4):
            ref = sum(A[i][k] * B[j][k] for k in range(32)) * float(da) * float(db)
            assert abs(float(got[i, j]) - ref) <= 1e-6 * max(1.0, abs(ref))


def test_nvfp4_chains_track_fp64_autograd():
    """Linear and gated-MLP NVFP4 chains against fp64 autograd of the unquantized layers:
    within the e2m1 error (a transposed operand or a scale on the wrong tensor is far off)."""
    g = torch.Generator().manual_seed(48)
    M, K, N = 64, 96, 80
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    y, dx, dw = orc.linear_fwd_bwd_nvfp4(x, w, dy)
    xr, wr = x.double().requires_grad_(True), w.double().requires_grad_(True)
    (xr @ wr.t()).backward(dy.double())
    assert _rel(y, x.double() @ w.double().t()) < 0.25
    assert _rel(dx, xr.grad) < 0.3 and _rel(dw, wr.grad) < 0.3
    I = 64
    wg = (torch.randn(I, K, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(I, K, generator=g) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(K, I, generator=g) * 0.05).to(torch.bfloat16)
    dy2 = (torch.randn(M, K, generator=g) * 1e-3).to(torch.bfloat16)
    y2, dx2, dwgu, dwd = orc.mlp_fwd_bwd_nvfp4(x, wg, wu, wd, dy2)
    xr = x.double().requires_grad_(True)
    ws = [t.double().requires_grad_(True) for t in (wg, wu, wd)]
    yr = (F.gelu(xr @ ws[0].t(), approximate="tanh") * (xr @ ws[1].t())) @ ws[2].t()
    yr.backward(dy2.double())
    assert _rel(y2, yr.detach()) < 0.35
    assert _rel(dx2, xr.grad) < 0.45
    assert _rel(dwgu, torch.cat([ws[0].grad, ws[1].grad])) < 0.45
    assert _rel(dwd, ws[2].grad) < 0.45


def _round_f32(fr: Fraction) -> float:
    """Correctly rounded (ties to even) fp32 of an exact rational."""
    v = float(np.float32(float(fr)))             # within one ulp; settle by exact midpoints
    lo, hi = np.nextafter(np.float32(v), np.float32(-np.inf)), np.nextafter(np.float32(v), np.float32(np.inf))
    best = min((abs(Fraction(float(c)) - fr), 0 if (np.float32(c).view(np.uint32) & 1) == 0 else 1,
                float(c)) for c in (lo, np.float32(v), hi))
    return best[2]


def test_nvfp4_multiplier_is_the_correctly_rounded_quotient():
    """mult = f32(S_enc / s) rounded once: checked with exact rationals over every finite
    positive e4m3 block scale and several global scales (a product with a rounded 1 / s
    differs on some of these pairs)."""
    s_bytes = torch.arange(1, 0x7F, dtype=torch.uint8)
    differs = 0
    for amax_v in (0.37, 1.0, 3.14159, 64.5, 1234.5):
        s_enc, _ = orc.nvfp4_global_scale(torch.tensor(amax_v, dtype=torch.float32))
        got = orc.nvfp4_block_multiplier(s_enc, s_bytes)
        sv = s_bytes.view(torch.float8_e4m3fn).float()
        for b in range(len(s_bytes)):
            want = _round_f32(Fraction(float(s_enc)) / Fraction(float(sv[b])))
            assert float(got[b]) == want
            differs += float(np.float32(float(s_enc) * np.float32(1.0 / float(sv[b])))) != want
    assert differs > 0
