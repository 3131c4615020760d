"""CPU oracle of the FP8 linear path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or the timed CPU baseline). The product path
(bongard_amd) never calls it and has no CPU fallback.

What it restates. The reference (AgentBull/bongard) ships no FP8 arithmetic of its own:
its FP8 linears call torchao 0.17.0 (pyproject.toml:29; bongard/float8_training.py:14,
35-36,57) and TransformerEngine 2.19.0 (pyproject.toml:30; bongard/te_linear.py:31-36,
41,73; bongard/fused_mlp.py:14-19,21,76), neither of which is present here. This module
restates their published per-tensor current-scaling algorithm, the arithmetic torchao
runs on CPU under ``emulate=True`` (bongard/float8_training.py:28):

  amax      = max(|x|)                              torchao tensor_to_amax
  scale     = f32(fp8_max / clamp(f64(amax), 1e-12)) torchao amax_to_scale
  q         = clamp(f32(x) * scale, +-fp8_max).to(fp8)   torchao to_fp8_saturated
  Y         = ((Aq.f32 / sa) @ (Bq.f32 / sb).T).to(out)  emulated scaled mm
  H         = bf16(bf16(gelu_tanh(g)) * u)           bongard/te_linear.py:103
  RMSNorm   = x * rsqrt(mean(x^2) + eps) * (1 + w)   HF T5Gemma2RMSNorm, fused_mlp.py:25-30

and adds the delayed-scaling closed form that config 5 asks for (no reference symbol).

Two independent witnesses pin the cast: ``quantize`` (torch's own float8 conversion,
the emulate path) and ``encode_fp8_np`` (a table-driven encoder built from the OCP FP8
bit layout). tests/test_oracle.py checks them against each other on all 65,536 bf16
bit patterns, against hand-computed known answers, and pins scale/matmul against fp64
closed forms; tests/golden/ holds fixtures this module wrote.

NaN conventions (this torch build's CPU kernels, x86): a NaN product carries the scale's
sign if the scale is NaN, else x's sign if x is NaN, else (inf * 0) the x86 default NaN,
which is negative; both fp8 formats encode NaN as 0x7F | sign.
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

E4M3 = 0
E5M2 = 1
FP8_MAX = {E4M3: 448.0, E5M2: 57344.0}
TORCH_FP8 = {E4M3: torch.float8_e4m3fn, E5M2: torch.float8_e5m2}
EPS = 1e-12  # torchao float8 EPS


# ---------------------------------------------------------------------------------------
# amax / scale  (torchao tensor_to_amax, amax_to_scale)
# ---------------------------------------------------------------------------------------
def amax(x: torch.Tensor) -> torch.Tensor:
    """max(|x|) in x's dtype (exact for bf16), NaN-propagating; returned as fp32 scalar."""
    return x.abs().max().to(torch.float32)


def amax_to_scale(amax_f32: torch.Tensor, fmt: int):
    """(scale, scale_inv) as fp32 scalars: scale = f32(fp8_max / clamp(f64(amax), EPS))."""
    a = amax_f32.to(torch.float64)
    scale = (FP8_MAX[fmt] / torch.clamp(a, min=EPS)).to(torch.float32)
    return scale, scale.reciprocal()


def scale_np(amax_value: float, fmt: int) -> np.float32:
    """Closed form of the scale in plain Python floats (fp64), rounded once to fp32."""
    a = float(amax_value)
    if math.isnan(a):
        return np.float32("nan")
    return np.float32(FP8_MAX[fmt] / max(a, EPS))


# ---------------------------------------------------------------------------------------
# saturating cast  (torchao to_fp8_saturated)
# ---------------------------------------------------------------------------------------
def _nan_sign_bytes(xf: torch.Tensor, prod: torch.Tensor, scale: torch.Tensor, fmt: int):
    """Bytes for NaN products per the conventions in the module docstring."""
    xnan = torch.isnan(xf)
    xsign = (xf.view(torch.int32) < 0)
    if bool(torch.isnan(scale)):
        sign = torch.full_like(xsign, bool(scale.view(torch.int32) < 0))
    else:
        sign = torch.where(xnan, xsign, torch.ones_like(xsign))
    return torch.where(sign, 0xFF, 0x7F).to(torch.uint8)


def cast(x: torch.Tensor, scale: torch.Tensor, fmt: int) -> torch.Tensor:
    """q bytes (uint8) of clamp(f32(x) * scale, +-max).to(fp8) with explicit NaN bytes."""
    xf = x.to(torch.float32)
    prod = xf * scale.to(torch.float32)
    m = FP8_MAX[fmt]
    q = torch.clamp(prod, -m, m).to(TORCH_FP8[fmt]).view(torch.uint8)
    nan = torch.isnan(prod)
    if bool(nan.any()):
        q = torch.where(nan, _nan_sign_bytes(xf, prod, scale, fmt), q)
    return q


def quantize(x: torch.Tensor, fmt: int = E4M3):
    """Current scaling: returns (q uint8 same shape, amax, scale, scale_inv) fp32 scalars."""
    a = amax(x)
    s, si = amax_to_scale(a, fmt)
    return cast(x, s, fmt), a, s, si


def dequant(q: torch.Tensor, scale: torch.Tensor, fmt: int) -> torch.Tensor:
    """q.float() / scale (the emulated dequantization) in fp32."""
    return q.view(TORCH_FP8[fmt]).to(torch.float32) / scale


# ---------------------------------------------------------------------------------------
# Independent witness: table-driven OCP FP8 encoder (numpy)
# ---------------------------------------------------------------------------------------
def fp8_value_table(fmt: int) -> np.ndarray:
    """float64 value of every byte 0..255 (NaN for NaN codes, +-inf for e5m2 inf)."""
    vals = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        if fmt == E4M3:
            e, m = (b >> 3) & 0xF, b & 0x7
            if e == 0xF and m == 0x7:
                v = math.nan
            elif e == 0:
                v = (m / 8.0) * 2.0 ** -6
            else:
                v = (1 + m / 8.0) * 2.0 ** (e - 7)
        else:
            e, m = (b >> 2) & 0x1F, b & 0x3
            if e == 0x1F:
                v = math.inf if m == 0 else math.nan
            elif e == 0:
                v = (m / 4.0) * 2.0 ** -14
            else:
                v = (1 + m / 4.0) * 2.0 ** (e - 15)
        vals[b] = s * v
    return vals


def encode_fp8_np(v: np.ndarray, fmt: int) -> np.ndarray:
    """Round-to-nearest-even encoding of finite fp32 values with |v| <= fp8_max.

    Non-negative finite codes 0..max_code are monotone in value, so the nearest code is
    found by bisection on the magnitude table; ties go to the even code (mantissa LSB 0).
    The sign bit is copied from v (so -0.0 and negative underflow give 0x80).
    """
    v = np.asarray(v, dtype=np.float32)
    table = fp8_value_table(fmt)
    max_code = 0x7E if fmt == E4M3 else 0x7B
    mags = table[: max_code + 1]
    a = np.abs(v.astype(np.float64))
    if np.any(a > FP8_MAX[fmt]) or np.any(~np.isfinite(a)):
        raise ValueError("encode_fp8_np expects finite values within +-fp8_max")
    hi = np.searchsorted(mags, a, side="left")  # first code with mag >= a
    hi = np.clip(hi, 0, max_code)
    lo = np.clip(hi - 1, 0, max_code)
    d_hi = mags[hi] - a
    d_lo = a - mags[lo]
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0))
    code = np.where(pick_lo, lo, hi).astype(np.uint8)
    sign = (np.signbit(v)).astype(np.uint8) << 7
    return code | sign


def cast_np(x_f32: np.ndarray, scale: np.float32, fmt: int) -> np.ndarray:
    """Numpy witness of ``cast``: fp32 product, clamp, table encoder, NaN convention."""
    x_f32 = np.asarray(x_f32, dtype=np.float32)
    scale = np.float32(scale)
    with np.errstate(invalid="ignore", over="ignore"):
        prod = (x_f32 * scale).astype(np.float32)
    nan = np.isnan(prod)
    m = np.float32(FP8_MAX[fmt])
    clamped = np.clip(np.where(nan, np.float32(0), prod), -m, m)
    q = encode_fp8_np(clamped, fmt)
    if nan.any():
        if np.isnan(scale):
            sign = np.full(x_f32.shape, bool(np.signbit(scale)))
        else:
            sign = np.where(np.isnan(x_f32), np.signbit(x_f32), True)
        q = np.where(nan, np.where(sign, 0xFF, 0x7F), q).astype(np.uint8)
    return q


# ---------------------------------------------------------------------------------------
# dequantized matmul  (torchao emulated _scaled_mm / TE GEMM)
# ---------------------------------------------------------------------------------------
def scaled_mm(aq, a_scale, a_fmt, bq, b_scale, b_fmt, *, bias=None, precise=True,
              seg_ends=None, b_scales=None):
    """fp32 result of (Aq/sa) @ (Bq/sb).T (+ bias).

    ``precise``: accumulate in fp64 (the reference truth for tolerance checks); else
    fp32 torch.mm, exactly the emulated path (used for the CPU baseline timing).
    ``seg_ends``/``b_scales``: per-column-segment weight scales (fused projections).
    """
    a = dequant(aq, a_scale, a_fmt)
    if seg_ends is None:
        b = dequant(bq, b_scale, b_fmt)
    else:
        parts, start = [], 0
        for end, s in zip(seg_ends, b_scales):
            parts.append(dequant(bq[start:end], s, b_fmt))
            start = end
        b = torch.cat(parts, 0)
    if precise:
        y = (a.double() @ b.double().T)
        if bias is not None:
            y = y + bias.double()
        return y.to(torch.float32)
    y = a @ b.T
    if bias is not None:
        y = y + bias.float()
    return y


# ---------------------------------------------------------------------------------------
# axiswise scaling  (torchao AXISWISE granularity: the rowwise recipes,
# bongard/float8_training.py:9; torchao 0.17.0 float8 config / float8_utils)
# ---------------------------------------------------------------------------------------
def round_scale_down_to_power_of_2(scale: torch.Tensor) -> torch.Tensor:
    """torchao _round_scale_down_to_power_of_2: exp2(floor(log2(scale))) on fp32."""
    return torch.exp2(torch.floor(torch.log2(scale)))


def amax_to_scale_axiswise(amax_f32: torch.Tensor, fmt: int, pow2: bool = True):
    """torchao amax_to_scale(..., round_scales_to_power_of_2): fp32 scale tensor."""
    a = amax_f32.to(torch.float64)
    scale = (FP8_MAX[fmt] / torch.clamp(a, min=EPS)).to(torch.float32)
    return round_scale_down_to_power_of_2(scale) if pow2 else scale


def cast_bcast(x: torch.Tensor, scale: torch.Tensor, fmt: int) -> torch.Tensor:
    """``cast`` with a scale tensor broadcast against x (same NaN byte conventions)."""
    xf = x.to(torch.float32)
    sc = scale.to(torch.float32).expand_as(xf)
    prod = xf * sc
    m = FP8_MAX[fmt]
    q = torch.clamp(prod, -m, m).to(TORCH_FP8[fmt]).view(torch.uint8)
    nan = torch.isnan(prod)
    if bool(nan.any()):
        xsign = xf.view(torch.int32) < 0
        ssign = sc.view(torch.int32) < 0
        sign = torch.where(torch.isnan(sc), ssign,
                           torch.where(torch.isnan(xf), xsign, torch.ones_like(xsign)))
        q = torch.where(nan, torch.where(sign, 0xFF, 0x7F).to(torch.uint8), q)
    return q


def quantize_axiswise(x: torch.Tensor, fmt: int, dim: int, pow2: bool = True):
    """torchao hp_tensor_to_float8_dynamic with AXISWISE granularity along ``dim``:
    amax = max |x| over ``dim`` (keepdim, NaN-propagating), scale per the remaining axis.
    Returns (q uint8 like x, scale fp32 with a size-1 ``dim``)."""
    a = x.abs().amax(dim=dim, keepdim=True).to(torch.float32)
    scale = amax_to_scale_axiswise(a, fmt, pow2)
    return cast_bcast(x, scale, fmt), scale


def linear_fwd_bwd_axiswise(x, w, dy, recipe, *, precise=True):
    """FP8 linear forward and backward under torchao's ``rowwise`` or ``rowwise_with_gw_hp``
    recipe (every cast e4m3, power-of-2 axiswise scales):

      y  = X8[dim -1] @ W8[dim -1]^T                      (both recipes)
      rowwise:            dX = dY8[dim -1] @ W8[dim 0];  dW = dY8[dim 0]^T @ X8[dim 0]
      rowwise_with_gw_hp: dX = dY8[dim -1] @ W8[tensorwise, pow2];  dW = dY^T @ X in
                          high precision (bf16 operands, exact sum here)
    Returns fp32 (y, dx, dw)."""
    xq, xs = quantize_axiswise(x, E4M3, -1)
    wq, ws = quantize_axiswise(w, E4M3, -1)
    y = scaled_mm(xq, xs, E4M3, wq, ws, E4M3, precise=precise)
    dq, dsc = quantize_axiswise(dy, E4M3, -1)
    if recipe == "rowwise":
        wcq, wcs = quantize_axiswise(w, E4M3, 0)            # scale per column k: [1, K]
        dx = scaled_mm(dq, dsc, E4M3, wcq.t().contiguous(), wcs.t(), E4M3, precise=precise)
        dcq, dcs = quantize_axiswise(dy, E4M3, 0)            # [1, N]
        xcq, xcs = quantize_axiswise(x, E4M3, 0)             # [1, K]
        dw = scaled_mm(dcq.t().contiguous(), dcs.t(), E4M3, xcq.t().contiguous(), xcs.t(),
                       E4M3, precise=precise)
    elif recipe == "rowwise_with_gw_hp":
        a = amax(w)
        wts = round_scale_down_to_power_of_2(amax_to_scale(a, E4M3)[0])
        wtq = cast(w, wts, E4M3)
        dx = scaled_mm(dq, dsc, E4M3, wtq.t().contiguous(), wts, E4M3, precise=precise)
        dw = (dy.double().t() @ x.double()).to(torch.float32)
    else:
        raise ValueError(recipe)
    return y, dx, dw


# ---------------------------------------------------------------------------------------
# MXFP8  (TE 2.19.0 MXFP8BlockScaling: bongard/te_linear.py:17,38-39,
# bongard/fused_mlp.py:9,31-33; OCP MX: 32-element blocks, E8M0 scales)
# ---------------------------------------------------------------------------------------
MX_BLOCK = 32


def mx_exponent(amax_f32: torch.Tensor, fmt: int) -> torch.Tensor:
    """E8M0 byte (int32) of fp32(amax * fp32(1 / fp8_max)) rounded up to a power of two
    (TE float_to_e8m0): NaN -> 0xFF, inf -> 0xFE, the carry never passes 0xFE, values at
    or below 2^-127 -> 0."""
    rcp = torch.tensor(1.0 / FP8_MAX[fmt], dtype=torch.float64).to(torch.float32)
    val = (amax_f32.to(torch.float32) * rcp).to(torch.float32)
    bits = val.view(torch.int32)
    exp = (bits >> 23) & 0xFF
    man = bits & 0x7FFFFF
    inc = (man > 0) & (exp != 0xFE) & ~((exp == 0) & (man <= 0x400000))
    e = exp + inc.to(torch.int32)
    e = torch.where(torch.isinf(val), torch.full_like(e, 0xFE), e)
    return torch.where(torch.isnan(val), torch.full_like(e, 0xFF), e)


def mx_multiplier(e: torch.Tensor) -> torch.Tensor:
    """2^(127 - e) as fp32 (NaN for 0xFF): the factor a block's values are scaled by."""
    m = torch.pow(2.0, (127 - e).to(torch.float64)).to(torch.float32)
    return torch.where(e == 0xFF, torch.full_like(m, float("nan")), m)


def quantize_mx(x: torch.Tensor, fmt: int, axis: int = -1):
    """MXFP8 of bf16 x [R, C] with blocks along ``axis`` (-1: along rows, returns q [R, C]
    and e [R, C/32]; 0: along columns, returned transposed, q [C, R] and e [C, R/32])."""
    xt = x if axis == -1 else x.t().contiguous()
    R, C = xt.shape
    blocks = xt.reshape(R, C // MX_BLOCK, MX_BLOCK)
    amax = blocks.abs().amax(dim=-1).to(torch.float32)
    e = mx_exponent(amax, fmt)
    q = cast_bcast(blocks, mx_multiplier(e)[..., None], fmt).reshape(R, C)
    return q, e


def dequant_mx(q: torch.Tensor, e: torch.Tensor, fmt: int) -> torch.Tensor:
    """q * 2^(e - 127) per block, in fp64 (exact)."""
    R, C = q.shape
    v = q.view(TORCH_FP8[fmt]).to(torch.float64).reshape(R, C // MX_BLOCK, MX_BLOCK)
    return (v * torch.pow(2.0, (e - 127).to(torch.float64))[..., None]).reshape(R, C)


def scaled_mm_mx(aq, ae, bq, be, fmt=E4M3, *, bias=None):
    """fp32 result of dequant_mx(A) @ dequant_mx(B).T (+ bias), accumulated in fp64."""
    y = dequant_mx(aq, ae, fmt) @ dequant_mx(bq, be, fmt).T
    if bias is not None:
        y = y + bias.double()
    return y.to(torch.float32)


def mx_scale_rows(e: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes as the kernels store them: rows padded to a multiple of 4 bytes with 127."""
    R, nb = e.shape
    ld = (nb + 3) // 4 * 4
    out = torch.full((R, ld), 127, dtype=torch.uint8)
    out[:, :nb] = e.to(torch.uint8)
    return out


def linear_fwd_bwd_mx(x, w, dy):
    """te.Linear under MXFP8 (every tensor e4m3 blocks): y = X8 W8^T; dX = dY8 (W^T)8 with
    W's columnwise blocks; dW = (dY^T)8 (X^T)8 with columnwise blocks along M. fp32 out."""
    xq, xe = quantize_mx(x, E4M3, -1)
    wq, we = quantize_mx(w, E4M3, -1)
    y = scaled_mm_mx(xq, xe, wq, we)
    dq, de = quantize_mx(dy, E4M3, -1)
    wtq, wte = quantize_mx(w, E4M3, 0)
    dx = scaled_mm_mx(dq, de, wtq, wte)
    dtq, dte = quantize_mx(dy, E4M3, 0)
    xtq, xte = quantize_mx(x, E4M3, 0)
    dw = scaled_mm_mx(dtq, dte, xtq, xte)
    return y, dx, dw


def mlp_fwd_bwd_mx(x, w_gate, w_up, w_down, dy):
    """The gated MLP (te_linear TEMLP / te.LayerNormMLP) under MXFP8, forward and backward
    through the same chain as the tensorwise ``mlp_forward`` / ``mlp_backward``.
    Returns fp32 y, dx, dW_gate_up [2I, K], dW_down and the bf16 H."""
    I = w_gate.shape[0]
    wgu = torch.cat([w_gate, w_up], 0)
    xq, xe = quantize_mx(x, E4M3, -1)
    wq, we = quantize_mx(wgu, E4M3, -1)
    g = scaled_mm_mx(xq, xe, wq[:I], we[:I]).to(torch.bfloat16)
    u = scaled_mm_mx(xq, xe, wq[I:], we[I:]).to(torch.bfloat16)
    h = geglu(g, u)
    hq, he = quantize_mx(h, E4M3, -1)
    dq_, de_ = quantize_mx(w_down, E4M3, -1)
    y = scaled_mm_mx(hq, he, dq_, de_)
    yq, ye = quantize_mx(dy, E4M3, -1)
    wdt, wdte = quantize_mx(w_down, E4M3, 0)
    dh = scaled_mm_mx(yq, ye, wdt, wdte)
    yt, yte = quantize_mx(dy, E4M3, 0)
    ht, hte = quantize_mx(h, E4M3, 0)
    dwd = scaled_mm_mx(yt, yte, ht, hte)
    dg, du = geglu_bwd(g, u, dh.to(torch.bfloat16))
    dgu = torch.cat([dg, du], 1)
    gq, ge = quantize_mx(dgu, E4M3, -1)
    wgt, wgte = quantize_mx(wgu, E4M3, 0)
    dx = scaled_mm_mx(gq, ge, wgt, wgte)
    gt, gte = quantize_mx(dgu, E4M3, 0)
    xt, xte = quantize_mx(x, E4M3, 0)
    dwgu = scaled_mm_mx(gt, gte, xt, xte)
    return dict(y=y, dx=dx, dwgu=dwgu, dwd=dwd, h=h)


# ---------------------------------------------------------------------------------------
# gated GELU chain and its backward  (bongard/te_linear.py:98-103, HF T5Gemma2MLP)
# ---------------------------------------------------------------------------------------
def geglu(g_bf16: torch.Tensor, u_bf16: torch.Tensor) -> torch.Tensor:
    """H = F.gelu(g, approximate='tanh') * u, on bf16 tensors (torch CPU kernels)."""
    return F.gelu(g_bf16, approximate="tanh") * u_bf16


def geglu_bwd(g_bf16, u_bf16, dh_bf16):
    """(d_g, d_u) from autograd of the bf16 chain geglu(g, u)."""
    g = g_bf16.detach().clone().requires_grad_(True)
    u = u_bf16.detach().clone().requires_grad_(True)
    h = geglu(g, u)
    h.backward(dh_bf16)
    return g.grad, u.grad


def _current(role, x, fmt):
    """Current scaling for every tensor role: (q bytes, scale)."""
    q, _, s, _ = quantize(x, fmt)
    return q, s


def mlp_forward(x_bf16, w_gate, w_up, w_down, *, shared_gate_up_scale=True, precise=True,
                quant=None):
    """FP8 gated MLP as the reference's TEMLP computes it (bf16 tensors in, fp32 Y out).

    ``quant(role, x, fmt) -> (q, scale)`` quantizes each tensor role ('x', 'w_gu', 'h',
    'w_down'); the default is current scaling (bongard/te_linear.py:38-39, 98-103), a
    DelayedQuantizer gives delayed scaling. Returns a dict with every intermediate
    (quantized bytes, scales, G, U, H, H8, Y).
    """
    quant = quant or _current
    xq, xs = quant("x", x_bf16, E4M3)
    I = w_gate.shape[0]
    if shared_gate_up_scale:
        wgu = torch.cat([w_gate, w_up], 0)
        wq, ws = quant("w_gu", wgu, E4M3)
        gate = scaled_mm(xq, xs, E4M3, wq[:I], ws, E4M3, precise=precise)
        up = scaled_mm(xq, xs, E4M3, wq[I:], ws, E4M3, precise=precise)
        w_scales = (ws, ws)
    else:
        gq, gs = quant("w_gate", w_gate, E4M3)
        uq, us = quant("w_up", w_up, E4M3)
        gate = scaled_mm(xq, xs, E4M3, gq, gs, E4M3, precise=precise)
        up = scaled_mm(xq, xs, E4M3, uq, us, E4M3, precise=precise)
        w_scales = (gs, us)
        wq = torch.cat([gq, uq], 0)
    g = gate.to(torch.bfloat16)
    u = up.to(torch.bfloat16)
    h = geglu(g, u)
    hq, hs = quant("h", h, E4M3)
    dq, ds = quant("w_down", w_down, E4M3)
    y = scaled_mm(hq, hs, E4M3, dq, ds, E4M3, precise=precise)
    return dict(xq=xq, x_scale=xs, w_scales=w_scales, wgu_q=wq, g=g, u=u, h=h, hq=hq,
                h_scale=hs, wd_q=dq, wd_scale=ds, y=y)


def linear_fwd_bwd(x, w, dy, *, precise=True):
    """FP8 linear forward and backward (torchao tensorwise / TE HYBRID).

    y = X8 W8^T; dX = dY8 W8; dW = dY8^T X8 with X, W in e4m3 and dY in e5m2, each with
    its own current scale. Returns fp32 (y, dx, dw).
    """
    xq, _, xs, _ = quantize(x, E4M3)
    wq, _, ws, _ = quantize(w, E4M3)
    dq, _, ds, _ = quantize(dy, E5M2)
    y = scaled_mm(xq, xs, E4M3, wq, ws, E4M3, precise=precise)
    dx = scaled_mm(dq, ds, E5M2, wq.t().contiguous(), ws, E4M3, precise=precise)
    dw = scaled_mm(dq.t().contiguous(), ds, E5M2, xq.t().contiguous(), xs, E4M3,
                   precise=precise)
    return y, dx, dw


def mlp_backward(fwd, x_bf16, w_gate, w_up, w_down, dy_bf16, *, precise=True, quant=None,
                 shared_gate_up_scale=True, dgu=None):
    """Backward of ``mlp_forward`` through the FP8 GEMMs.

    dH = dY8 Wd8 (bf16), dWd = dY8^T H8, (dG, dU) = autograd of the bf16 gelu chain.
    Shared gate/up scale (TE's fused ``gate_up``, bongard/te_linear.py:90-92): dGU is
    quantized to e5m2 with one scale, dX = dGU8 Wgu8, dWgu = dGU8^T X8.
    Split (``shared_gate_up_scale=False``: ``BONGARD_TE_SPLIT_GATE_UP=1``, two TELinears,
    bongard/te_linear.py:93-95,98-103; torchao's separate gate/up linears): each of dG and
    dU is quantized to e5m2 with its own current scale, each dgrad uses its own W half and
    that half's scale and is rounded to bf16 (a TE linear's output dtype), and dX is the
    bf16 sum of the two (autograd adding the gradients of x's two uses); dW_gate =
    dG8^T X8 and dW_up = dU8^T X8. The weights' FP8 copies are the forward's; ``quant``
    quantizes the roles 'dy' and 'dgu' (split: 'dg', 'du'). ``dgu``: a bf16 [M, 2I] to use
    in place of the chain's own dGU (checks the GEMM stage given a kernel's dGU).
    Returns fp32 (dx, dw_gate_up [2I, K], dw_down) and the bf16 dGU.
    """
    quant = quant or _current
    dq, ds = quant("dy", dy_bf16, E5M2)
    wdq, wds = fwd["wd_q"], fwd["wd_scale"]
    dh = scaled_mm(dq, ds, E5M2, wdq.t().contiguous(), wds, E4M3, precise=precise)
    dwd = scaled_mm(dq.t().contiguous(), ds, E5M2, fwd["hq"].t().contiguous(), fwd["h_scale"],
                    E4M3, precise=precise)
    if dgu is None:
        dg, du = geglu_bwd(fwd["g"], fwd["u"], dh.to(torch.bfloat16))
        dgu = torch.cat([dg, du], 1)
    else:
        I = w_gate.shape[0]
        dg, du = dgu[:, :I], dgu[:, I:]
    wq = fwd["wgu_q"]
    xqt = fwd["xq"].t().contiguous()
    if shared_gate_up_scale:
        gq, gs = quant("dgu", dgu, E5M2)
        wsc = fwd["w_scales"][0]
        dx = scaled_mm(gq, gs, E5M2, wq.t().contiguous(), wsc, E4M3, precise=precise)
        dwgu = scaled_mm(gq.t().contiguous(), gs, E5M2, xqt, fwd["x_scale"], E4M3,
                         precise=precise)
        return dx, dwgu, dwd, dgu
    I = w_gate.shape[0]
    dx = None
    dws = []
    for half, (role, d) in enumerate((("dg", dg), ("du", du))):
        q, s = quant(role, d, E5M2)
        w_half = wq[half * I:(half + 1) * I].t().contiguous()
        part = scaled_mm(q, s, E5M2, w_half, fwd["w_scales"][half], E4M3,
                         precise=precise).to(torch.bfloat16)
        dx = part if dx is None else dx + part      # bf16 + bf16: one rounding of the sum
        dws.append(scaled_mm(q.t().contiguous(), s, E5M2, xqt, fwd["x_scale"], E4M3,
                             precise=precise))
    return dx.float(), torch.cat(dws, 0), dwd, dgu


# ---------------------------------------------------------------------------------------
# RMSNorm with zero-centred gamma  (HF T5Gemma2RMSNorm; TE LayerNormMLP, fused_mlp.py:25-30)
# ---------------------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    out = out * (1.0 + weight.float())
    return out.type_as(x)


# ---------------------------------------------------------------------------------------
# delayed scaling (config 5; TE DelayedScaling semantics, margin 0, algo "max")
# ---------------------------------------------------------------------------------------
class DelayedScaling:
    """Reference closed form of the amax-history scaling used by config 5.

    Step t quantizes with ``scale_t``; afterwards its amax enters a ring of ``length``.
    scale_{t+1} = fp8_max / max(history) if that maximum is finite and > 0, else scale_t.
    The initial scale is 1.
    """

    def __init__(self, length: int, fmt: int):
        self.length = length
        self.fmt = fmt
        self.history = np.zeros(length, dtype=np.float32)
        self.pos = 0
        self.scale = np.float32(1.0)

    def begin(self):
        h = self.history
        if np.all(np.isfinite(h)) and h.max() > 0:
            self.scale = np.float32(FP8_MAX[self.fmt] / float(h.max()))
        return self.scale, np.float32(1.0 / float(self.scale))

    def end(self, amax_value):
        self.history[self.pos] = np.float32(amax_value)
        self.pos = (self.pos + 1) % self.length


class DelayedQuantizer:
    """``quant(role, x, fmt)`` for mlp_forward / mlp_backward with delayed scaling: one
    DelayedScaling per tensor role; each call quantizes with the role's scale, then
    pushes the tensor's amax into the role's history."""

    def __init__(self, length: int):
        self.length = length
        self.roles = {}

    def __call__(self, role, x, fmt):
        ds = self.roles.setdefault(role, DelayedScaling(self.length, fmt))
        scale, _ = ds.begin()
        s = torch.tensor(scale, dtype=torch.float32)
        q = cast(x, s, fmt)
        ds.end(float(amax(x)))
        return q, s


# ---------------------------------------------------------------------------------------
# NVFP4: e2m1 values in blocks of 16 with e4m3 block scales under a per-tensor fp32 scale
# (TE NVFP4BlockScaling, bongard/te_linear.py:17,38; bongard/fused_mlp.py:9,32; TE 2.19.0 is
# absent, so this restates NVIDIA's published NVFP4 quantization with round-to-nearest-even
# everywhere and 1-D blocks along the reduction dimension; TE's random Hadamard transform,
# stochastic rounding of gradients and 2-D weight blocks are not restated -- parity
# unpinned for those)
# ---------------------------------------------------------------------------------------
NVFP4_GLOBAL = 448.0 * 6.0     # e4m3 max x e2m1 max
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def e2m1_code(p: torch.Tensor) -> torch.Tensor:
    """uint8 e2m1 codes of fp32 values: round to nearest even on {0, .5, 1, 1.5, 2, 3, 4, 6}
    (ties to the even code), saturating at 6, sign bit 3 copied from p (-0 -> 0x8; NaN ->
    code 0 with its sign)."""
    a = p.abs()
    m = ((a > 0.25).int() + (a >= 0.75).int() + (a > 1.25).int() + (a >= 1.75).int()
         + (a > 2.5).int() + (a >= 3.5).int() + (a > 5.0).int())
    return (m | (torch.signbit(p).int() << 3)).to(torch.uint8)


def e2m1_decode(codes: torch.Tensor) -> torch.Tensor:
    """fp32 value of e2m1 codes (low 4 bits)."""
    table = torch.tensor(E2M1_VALUES + tuple(-v for v in E2M1_VALUES), dtype=torch.float32)
    return table[(codes & 0xF).long()]


def nvfp4_global_scale(amax_f32: torch.Tensor):
    """(S_enc, S_dec) = (f32(2688 / max(f64(amax), 1e-12)), f32(1 / S_enc))."""
    a = amax_f32.to(torch.float64)
    s_enc = (NVFP4_GLOBAL / torch.clamp(a, min=EPS)).to(torch.float32)
    return s_enc, s_enc.reciprocal()


def nvfp4_block_multiplier(s_enc: torch.Tensor, sbytes: torch.Tensor) -> torch.Tensor:
    """fp32 multiplier of each block: f32(S_enc / s) (correctly rounded), 0 where s == 0."""
    s = sbytes.view(torch.float8_e4m3fn).float()
    return torch.where(s == 0, torch.zeros_like(s), s_enc / s)


def quantize_nvfp4(x: torch.Tensor, axis: int = -1):
    """NVFP4 quantization of bf16 x [R, C] in blocks of 16 along ``axis`` (-1: rowwise,
    blocks along C; 0: columnwise, the rowwise quantization of x^T). Returns (packed
    uint8 [., ./2] with the even element in the low nibble, block scale bytes e4m3
    [., ./16], S_enc, S_dec, amax). Per block with b = max |x|:
    s = e4m3(f32(f32(b / 6) * S_enc)), mult = s == 0 ? 0 : f32(S_enc / s),
    q = e2m1(f32(x * mult))."""
    if axis == 0:
        x = x.t().contiguous()
    a = amax(x)
    s_enc, s_dec = nvfp4_global_scale(a)
    R, C = x.shape
    blocks = x.float().reshape(R, C // 16, 16)
    bmax = blocks.abs().amax(-1)
    v = (bmax / torch.tensor(6.0)) * s_enc
    sbytes = cast(v, torch.tensor(1.0), E4M3)
    mult = nvfp4_block_multiplier(s_enc, sbytes)
    codes = e2m1_code(blocks * mult[..., None]).reshape(R, C)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    return packed, sbytes, s_enc, s_dec, a


def dequant_nvfp4(packed: torch.Tensor, sbytes: torch.Tensor) -> torch.Tensor:
    """fp32 e2m1(q) * s per element ([R, 2 * packed cols]), without the global S_dec."""
    R = packed.shape[0]
    codes = torch.stack([packed & 0xF, packed >> 4], -1).reshape(R, -1)
    s = sbytes.view(torch.float8_e4m3fn).float()
    return e2m1_decode(codes) * s.repeat_interleave(16, dim=1)


def scaled_mm_nvfp4(aq, a_sb, a_sdec, bq, b_sb, b_sdec):
    """fp32 result of (A^ @ B^T) * a_sdec * b_sdec in fp64 (A^, B^ the block-dequantized
    operands, exact)."""
    a = dequant_nvfp4(aq, a_sb).double()
    b = dequant_nvfp4(bq, b_sb).double()
    return (a @ b.t() * float(a_sdec) * float(b_sdec)).to(torch.float32)


def linear_fwd_bwd_nvfp4(x, w, dy):
    """NVFP4 linear forward and backward, every tensor e2m1 in 16-blocks along the GEMM's
    reduction dimension: y = X^ W^T; dX = dY^ (W^T)^; dW = (dY^T)^ (X^T)^. fp32 (y, dx, dw)."""
    def q(t, axis):
        p, sb, _, sdec, _ = quantize_nvfp4(t, axis)
        return p, sb, sdec
    y = scaled_mm_nvfp4(*q(x, -1), *q(w, -1))
    dx = scaled_mm_nvfp4(*q(dy, -1), *q(w, 0))
    dw = scaled_mm_nvfp4(*q(dy, 0), *q(x, 0))
    return y, dx, dw


def mlp_fwd_bwd_nvfp4(x, w_gate, w_up, w_down, dy):
    """The gated MLP with its two projections in NVFP4 (gate/up stacked as one weight and
    one global scale, as TE's fused gate_up; down on H) and the bf16 gelu chain between
    them (g, u, H rounded to bf16). Returns fp32 (y, dx, dw_gate_up, dw_down)."""
    I = w_gate.shape[0]
    wgu = torch.cat([w_gate, w_up], 0)
    gu = linear_fwd_bwd_nvfp4(x, wgu, torch.zeros(x.shape[0], 2 * I, dtype=torch.bfloat16))[0]
    gu = gu.to(torch.bfloat16)
    g, u = gu[:, :I], gu[:, I:]
    h = geglu(g, u)
    y, dh, dwd = linear_fwd_bwd_nvfp4(h, w_down, dy)
    dg, du = geglu_bwd(g, u, dh.to(torch.bfloat16))
    dgu = torch.cat([dg, du], 1)
    _, dx, dwgu = linear_fwd_bwd_nvfp4(x, wgu, dgu)
    return y, dx, dwgu, dwd


# ---------------------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------------------
def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (fp32), 2^(e-7) for normal x; min-normal spacing below."""
    a = x.abs().float().clamp(min=2.0 ** -126)
    e = torch.floor(torch.log2(a))
    return torch.pow(2.0, e - 7)
