"""FP8 linear and gated-MLP autograd functions on the gfx950 kernels.

Forward: X and W are quantized to e4m3 with per-tensor current scaling, the GEMM runs on
the FP8 MFMA with fp32 accumulation and a dequant epilogue, output bf16.
Backward (torchao tensorwise / TE Float8CurrentScaling "HYBRID" formats): grad_out is
quantized to e5m2 with its own per-tensor scale;
  dgrad  dX = dY8 . W8          (W8 [N, K] read as a K-major operand)
  wgrad  dW = dY8^T . X8        (dY8 and X8 read as K-major operands)
The backward GEMMs read the forward's fp8 tensors as they are and turn them around in LDS
(the LDS transpose read), so no transposed fp8 copy is written. The axiswise, MXFP8 and
NVFP4 recipes scale along the other axis for the backward and quantize separately
transposed copies.

Scaling is per-tensor current scaling by default; passing ``scaling``
(:class:`bongard_amd.scaling.LinearScaling`) switches a linear to delayed scaling with an
amax history (one-pass casts, the scale of each role taken from its history).

Reference behaviour these replace: torchao Float8Linear.forward/backward reached from
bongard/float8_training.py:16-22, te.Linear under TELinear.forward
(bongard/te_linear.py:59-77), and TEMLP/FusedMLP (bongard/te_linear.py:98-103,
bongard/fused_mlp.py:62-79).
"""

import threading
from dataclasses import dataclass
from typing import Optional

import torch

from . import ops
from . import scaling as _scaling
from .ops import E4M3, E5M2


@dataclass
class QuantizedWeight:
    """Cached FP8 copy of a weight (``q``: rowwise [N, K], a transposed [K, N] only where a
    recipe asks for one, and meta) and the weight version it was made from."""

    q: ops.Fp8Tensor
    version: int


class _Fp8Function(torch.autograd.Function):
    """Base of the FP8 autograd functions: remembers whether grad mode was on when the
    function was applied (torch runs ``forward`` itself with grad mode off)."""

    _grad_at_apply = threading.local()

    @classmethod
    def apply(cls, *args, **kwargs):
        tls = _Fp8Function._grad_at_apply
        prev = getattr(tls, "on", None)
        tls.on = torch.is_grad_enabled()
        try:
            return super().apply(*args, **kwargs)
        finally:
            tls.on = prev


def _forward_needs(ctx, n):
    """Which of the first n inputs a backward will need gradients for. Under no_grad /
    inference_mode no backward runs, whatever the inputs' requires_grad says (autograd
    still reports it in ``needs_input_grad``), so no transposed copies are made and the
    inference forwards' shared quantize launches apply to trainable parameters too."""
    on = getattr(_Fp8Function._grad_at_apply, "on", None)
    grad = True if on is None else on
    return tuple(bool(grad and b) for b in ctx.needs_input_grad[:n])


def quantize_weight(weight, *, transpose=False, scaler=None):
    """e4m3 copy of a weight [N, K] (current or the scaler's delayed scale). The backward
    reads it as is (a K-major operand), so no transposed copy is made unless asked for."""
    return _quantize(weight.detach(), E4M3, scaler, rowwise=True, transpose=transpose)


def _quantize(x, fmt, scaler, *, rowwise=True, transpose=False):
    """Current scaling (scaler None) or the scaler's delayed scaling."""
    if scaler is None:
        return ops.quantize(x, fmt, rowwise=rowwise, transpose=transpose)
    return scaler.quantize(x, rowwise=rowwise, transpose=transpose)


def _quantize_input(x, scaler, x_amax, transpose):
    """e4m3 quantization of a GEMM input whose amax partials its producer may have written.

    ``x_amax``: None (amax pass here), the producer's partials tensor (current scaling), or
    the number of partials it wrote into ``scaler.partials_for_producer`` (delayed)."""
    if x_amax is None:
        return _quantize(x, E4M3, scaler, transpose=transpose)
    if scaler is None:
        return ops.cast_partials(x, x_amax, E4M3, rowwise=True, transpose=transpose)
    return scaler.quantize(x, rowwise=True, transpose=transpose, producer_count=int(x_amax))


def linear_kmajor(in_features, out_features):
    """Whether a tensorwise FP8 linear can train: its backward reads the forward's fp8 X and
    W as they are (K-major dgrad / wgrad operands, bf8_gemm_kmajor), which needs both row
    lengths to be multiples of 16 bytes (as transposed fp8 copies would)."""
    return in_features % 16 == 0 and out_features % 16 == 0


def _check_trainable(who, *dims):
    bad = [d for d in dims if d % 16]
    if bad:
        raise ValueError(f"{who}: FP8 training needs feature sizes that are multiples of 16 "
                         f"(got {list(dims)})")


def linear_forward(x, weight, bias, wq, scaling, need_dx, need_dw):
    """Tensorwise FP8 linear forward: ``(y, (x8, x_meta, w8, w_meta))``, X8 and W8 as the
    backward reads them (None where no gradient needs them). ``wq``: a cached quantized
    weight or None; ``scaling``: None (current scaling) or a LinearScaling (delayed).
    No transposed copy is made: under current scaling x and W share one amax and one cast
    launch, in training as in inference."""
    if need_dx or need_dw:
        _check_trainable("fp8 linear", x.shape[-1], weight.shape[0])
    if scaling is None and wq is None:
        xq, wq = ops.quantize_many([x, weight.detach()])
    else:
        xq = _quantize(x, E4M3, scaling and scaling.input)
    if wq is None:
        wq = quantize_weight(weight, scaler=scaling and scaling.weight)
    y = ops.gemm(xq.data, E4M3, xq.meta, wq.data, E4M3, wq.meta, bias=bias)
    return y, (xq.data if need_dw else None, xq.meta, wq.data if need_dx else None, wq.meta)


def linear_backward(dy, saved, scaling, need_dx, need_dw):
    """Tensorwise FP8 linear backward: dY in e5m2 (its own scale), dX = dY8 . W8 and
    dW = dY8^T . X8 with W8 and X8 (and dY8 for dW) read as K-major operands."""
    x8, x_meta, w8, w_meta = saved
    dyq = _quantize(dy.contiguous(), E5M2, scaling and scaling.grad_output)
    dx = ops.gemm_kmajor(dyq.data, E5M2, dyq.meta, w8, E4M3, w_meta) if need_dx else None
    dw = (ops.gemm_kmajor(dyq.data, E5M2, dyq.meta, x8, E4M3, x_meta, a_kmajor=True)
          if need_dw else None)
    return dx, dw


class Fp8LinearFunction(_Fp8Function):
    """y = x @ W^T (+ b) in FP8; x: bf16 [M, K], W [N, K] with K and N multiples of 16
    when grads are needed.

    ``scaling``: None (current scaling) or a LinearScaling (delayed scaling)."""

    @staticmethod
    def forward(ctx, x, weight, bias, wq, scaling=None):
        need_dx, need_dw = _forward_needs(ctx, 2)
        y, saved = linear_forward(x, weight, bias, wq, scaling, need_dx, need_dw)
        ctx.scaling = scaling
        ctx.has_bias = bias is not None
        ctx.save_for_backward(*saved)
        return y

    @staticmethod
    def backward(ctx, dy):
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx, dw = linear_backward(dy, ctx.saved_tensors, ctx.scaling, need_dx, need_dw)
        db = dy.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dx, dw, db, None, None


AXISWISE_RECIPES = ("rowwise", "rowwise_with_gw_hp")


def linear_axiswise_forward(x, weight, bias, recipe, need_dx, need_dw):
    """Forward of torchao's axiswise recipes (see Fp8LinearAxiswiseFunction): ``(y, saved)``
    with saved = (x8t, x_col_sinv, w8t, w_col_sinv) for 'rowwise' (None where unneeded)
    and (x, weight) for 'rowwise_with_gw_hp' (its backward re-quantizes W and keeps dW in
    high precision)."""
    if recipe not in AXISWISE_RECIPES:
        raise ValueError(f"axiswise recipe must be one of {AXISWISE_RECIPES}")
    hp_wgrad = recipe == "rowwise_with_gw_hp"
    xq = ops.quantize_axiswise(x, E4M3, rowwise=True, colwise=need_dw and not hp_wgrad)
    wq = ops.quantize_axiswise(weight.detach(), E4M3, rowwise=True,
                               colwise=need_dx and not hp_wgrad)
    y = ops.gemm_axiswise(xq.data, E4M3, xq.row_sinv, wq.data, E4M3, wq.row_sinv, bias=bias)
    if hp_wgrad:
        return y, (x if need_dw else None, weight.detach() if need_dx else None)
    return y, (xq.data_t, xq.col_sinv, wq.data_t, wq.col_sinv)


def linear_axiswise_backward(dy, saved, recipe, need_dx, need_dw):
    dy = dy.contiguous()
    dx = dw = None
    if recipe == "rowwise":
        x8t, x_cs, w8t, w_cs = saved
        dyq = ops.quantize_axiswise(dy, E4M3, rowwise=need_dx, colwise=need_dw)
        if need_dx:
            dx = ops.gemm_axiswise(dyq.data, E4M3, dyq.row_sinv, w8t, E4M3, w_cs)
        if need_dw:
            dw = ops.gemm_axiswise(dyq.data_t, E4M3, dyq.col_sinv, x8t, E4M3, x_cs)
    else:
        x, weight = saved
        if need_dx:
            dyq = ops.quantize_axiswise(dy, E4M3, rowwise=True)
            wt = ops.quantize(weight, E4M3, rowwise=False, transpose=True, pow2=True)
            dx = ops.gemm_axiswise(dyq.data, E4M3, dyq.row_sinv, wt.data_t, E4M3, wt.meta[2:3])
        if need_dw:
            dw = torch.mm(dy.t().contiguous(), x)
    return dx, dw


class Fp8LinearAxiswiseFunction(_Fp8Function):
    """y = x @ W^T (+ b) under torchao's axiswise recipes; x: bf16 [M, K], M % 16 == 0 when
    grads are needed. Every cast is e4m3 with power-of-2 scales (torchao 0.17.0
    Float8LinearConfig.from_recipe_name, round_scales_to_power_of_2=True):

      forward              y  = X8[per row] . W8[per row]^T
      rowwise              dX = dY8[per row] . W8[per column of W]
                           dW = dY8[per column]^T . X8[per column]
      rowwise_with_gw_hp   dX = dY8[per row] . W8[tensorwise]
                           dW = dY^T . X in bf16 (torch.mm, the high-precision wgrad)

    "per column" quantizations are stored transposed (the reduction dim contiguous), so
    every FP8 GEMM is the same TN kernel with a scale vector on either side.
    Reference: torchao matmul_with_hp_or_float8_args.forward/backward under
    TrainingLinear.forward (bongard/float8_training.py:16-22) for the recipes at :9.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, recipe):
        need_dx, need_dw = _forward_needs(ctx, 2)
        y, saved = linear_axiswise_forward(x, weight, bias, recipe, need_dx, need_dw)
        ctx.recipe = recipe
        ctx.has_bias = bias is not None
        ctx.save_for_backward(*saved)
        return y

    @staticmethod
    def backward(ctx, dy):
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx, dw = linear_axiswise_backward(dy, ctx.saved_tensors, ctx.recipe, need_dx, need_dw)
        db = dy.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dx, dw, db, None


def quantize_weight_nvfp4(weight, *, transpose=True, cache_dequant=False):
    """NVFP4 copy of a weight [N, K]: blocks along K (forward), and with ``transpose`` the
    columnwise copy [K, N] with blocks along N (the input-gradient GEMM's operand).
    ``cache_dequant``: for a copy cached across microbatches, keep each copy's bf16
    dequantization after its first GEMM (the GEMMs' operand; bit-identical)."""
    q = ops.quantize_nvfp4(weight.detach(), rowwise=True, colwise=transpose)
    q.cache_dequant = cache_dequant
    return q


class Fp8LinearNvfp4Function(_Fp8Function):
    """y = x @ W^T under TE's NVFP4BlockScaling as built here (every tensor e2m1 in blocks
    of 16 along the GEMM's reduction dimension, e4m3 block scales, a per-tensor fp32 scale;
    round to nearest even, no Hadamard transform, no stochastic rounding); x: bf16 [M, K]
    with M % 16 == 0 when the weight needs a gradient; x_partials: amax partials of |x|
    from its producer (no amax pass for x) or None. Each GEMM dequantizes its NVFP4
    operands exactly to bf16 and runs the bf16 MFMA, the two tensor scales in its epilogue.

      forward  y  = X^ . W^T           blocks along K on both
      dgrad    dX = dY^ . (W^T)^       dY blocks along N, W's columnwise copy
      wgrad    dW = (dY^T)^ . (X^T)^   columnwise copies of dY and X (blocks along M)

    Reference: te.Linear under the 'nvfp4' recipe (bongard/te_linear.py:17,38,73-74).
    """

    @staticmethod
    def forward(ctx, x, weight, wq, x_partials=None):
        need_dx, need_dw = _forward_needs(ctx, 2)
        xq = ops.quantize_nvfp4(x, rowwise=True, colwise=need_dw, partials=x_partials,
                                dequant_rows=True)
        if wq is None:
            wq = quantize_weight_nvfp4(weight, transpose=need_dx)
        y = ops.gemm_nvfp4(None, None, xq.meta, wq.data, wq.scales, wq.meta,
                           a_deq=ops.nvfp4_dequant(xq), b_deq=ops.nvfp4_dequant(wq))
        ctx.save_for_backward(xq.data_t, xq.scales_t, xq.meta,
                              wq.data_t if need_dx else None,
                              wq.scales_t if need_dx else None, wq.meta)
        # a cached weight lends the dgrad GEMM its kept bf16 columnwise operand
        ctx.wq = wq if need_dx and wq.cache_dequant else None
        return y

    @staticmethod
    def backward(ctx, dy):
        x4t, xst, x_meta, w4t, wst, w_meta = ctx.saved_tensors
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dyq = ops.quantize_nvfp4(dy.contiguous(), rowwise=need_dx, colwise=need_dw,
                                 dequant_rows=True)
        dx = dw = None
        if need_dx:
            wdt = ops.nvfp4_dequant(ctx.wq, transpose=True) if ctx.wq is not None else None
            dx = ops.gemm_nvfp4(None, None, dyq.meta, w4t, wst, w_meta,
                                a_deq=ops.nvfp4_dequant(dyq), b_deq=wdt)
        if need_dw:
            dw = ops.gemm_nvfp4(dyq.data_t, dyq.scales_t, dyq.meta, x4t, xst, x_meta)
        return dx, dw, None, None


class GegluFunction(torch.autograd.Function):
    """H = bf16(bf16(gelu_tanh(gate)) * up) of the bf16 pre-activations GU [M, 2I] (gate |
    up) and its backward, on the elementwise kernels (bit-identical to the bf16 chain
    F.gelu(gate, approximate='tanh') * up, bongard/te_linear.py:103): the activation after
    two separate gate and up projections (the NVFP4 recipe's split layout, one tensor scale
    per projection), whose GEMMs cannot take it into an epilogue. Returns ``(H, amax
    partials of |H|)`` (the partials for the down projection's quantizer; not
    differentiable)."""

    @staticmethod
    def forward(ctx, GU):
        H, parts = ops.geglu(GU)
        ctx.save_for_backward(GU)
        ctx.mark_non_differentiable(parts)
        return H, parts

    @staticmethod
    def backward(ctx, dH, _d_partials):
        (GU,) = ctx.saved_tensors
        dGU, _ = ops.geglu_bwd(dH.contiguous(), GU)
        return dGU


class GegluGateUpNvfp4Function(_Fp8Function):
    """H = geglu(X @ [W_gate; W_up]^T) under the NVFP4 recipe, the gated GELU in the
    gate/up GEMM's epilogue: the NVFP4 operands dequantized exactly to bf16, the bf16
    MFMA, g and u rounded to bf16 from the fp32 sums times the two S_dec, H = bf16(bf16(
    gelu_tanh(g)) * u) (bf8_gemm_geglu_bf16). Equals Fp8LinearNvfp4Function followed by
    GegluFunction bit for bit where that GEMM runs unsplit (the forward and, from the same
    GU, the backward), without the [M, 2I] pre-activations' round trip when no gradient
    is needed. x: bf16 [M, K]; w_gu [2I, K]; x_partials: amax partials of |x| written by
    its producer (the fused RMSNorm) or None. x and dGU are quantized from their producers'
    amax partials, without an amax pass of their own. Returns ``(H, amax partials of |H|)``
    (the partials for the down projection's quantizer; not differentiable).

    Reference: TEMLP's gate_up projection and F.gelu(gate, approximate='tanh') * up
    (bongard/te_linear.py:98-103) and te.LayerNormMLP's fc1 + geglu (bongard/fused_mlp.py:
    25-30) under the 'nvfp4' recipe (bongard/te_linear.py:17,38).
    """

    @staticmethod
    def forward(ctx, x, w_gu, wq, intermediate, x_partials=None):
        need_dx, need_dw = _forward_needs(ctx, 2)
        xq = ops.quantize_nvfp4(x, rowwise=True, colwise=need_dw, partials=x_partials,
                                dequant_rows=True)
        if wq is None:
            wq = quantize_weight_nvfp4(w_gu, transpose=need_dx)
        train = need_dx or need_dw
        H, GU, h_partials = ops.gemm_geglu_nvfp4(None, None, xq.meta, wq.data, wq.scales,
                                                 wq.meta, intermediate, keep_gu=train,
                                                 a_deq=ops.nvfp4_dequant(xq),
                                                 b_deq=ops.nvfp4_dequant(wq))
        ctx.save_for_backward(GU, xq.data_t, xq.scales_t, xq.meta,
                              wq.data_t if need_dx else None,
                              wq.scales_t if need_dx else None, wq.meta)
        ctx.wq = wq if need_dx and wq.cache_dequant else None
        ctx.mark_non_differentiable(h_partials)
        return H, h_partials

    @staticmethod
    def backward(ctx, dH, _d_partials):
        GU, x4t, xst, x_meta, w4t, wst, w_meta = ctx.saved_tensors
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dGU, dparts = ops.geglu_bwd(dH.contiguous(), GU)
        dq = ops.quantize_nvfp4(dGU, rowwise=need_dx, colwise=need_dw, partials=dparts,
                                dequant_rows=True)
        dx = dw = None
        if need_dx:
            wdt = ops.nvfp4_dequant(ctx.wq, transpose=True) if ctx.wq is not None else None
            dx = ops.gemm_nvfp4(None, None, dq.meta, w4t, wst, w_meta,
                                a_deq=ops.nvfp4_dequant(dq), b_deq=wdt)
        if need_dw:
            dw = ops.gemm_nvfp4(dq.data_t, dq.scales_t, dq.meta, x4t, xst, x_meta)
        return dx, dw, None, None, None


def quantize_weight_mx(weight, *, transpose=True):
    """MXFP8 copy of a weight [N, K]: blocks along K (forward), and with ``transpose`` the
    [K, N] copy with blocks along N (the input-gradient GEMM's operand)."""
    return ops.quantize_mx(weight.detach(), E4M3, rowwise=True, colwise=transpose)


class Fp8LinearMxFunction(_Fp8Function):
    """y = x @ W^T under TE's MXFP8BlockScaling (every tensor e4m3 in 32-element blocks
    with E8M0 scales); x: bf16 [M, K] with M % 32 == 0 when grads are needed.

      forward  y  = X8 . W8^T         blocks along K on both
      dgrad    dX = dY8 . (W^T)8      dY blocks along N, W's columnwise copy
      wgrad    dW = (dY^T)8 . (X^T)8  columnwise copies of dY and X (blocks along M)

    Reference: te.Linear under the 'mxfp8' recipe (bongard/te_linear.py:17,38-39,73-74).
    """

    @staticmethod
    def forward(ctx, x, weight, wq):
        need_dx, need_dw = _forward_needs(ctx, 2)
        if wq is None and not (need_dx or need_dw):
            xq, wq = ops.quantize_mx_many([x, weight.detach()])   # inference: one launch
        else:
            xq = ops.quantize_mx(x, E4M3, rowwise=True, colwise=need_dw)
        if wq is None:
            wq = quantize_weight_mx(weight, transpose=need_dx)
        y = ops.gemm_mx(xq.data, xq.scales, wq.data, wq.scales)
        ctx.save_for_backward(xq.data_t, xq.scales_t, wq.data_t if need_dx else None,
                              wq.scales_t if need_dx else None)
        return y

    @staticmethod
    def backward(ctx, dy):
        x8t, xst, w8t, wst = ctx.saved_tensors
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dyq = ops.quantize_mx(dy.contiguous(), E4M3, rowwise=need_dx, colwise=need_dw)
        dx = dw = None
        if need_dx:
            dx = ops.gemm_mx(dyq.data, dyq.scales, w8t, wst)
        if need_dw:
            dw = ops.gemm_mx(dyq.data_t, dyq.scales_t, x8t, xst)
        return dx, dw, None


class Fp8GegluMlpMxFunction(_Fp8Function):
    """The gated MLP of :class:`Fp8GegluMlpFunction` under MXFP8 (e4m3 blocks of 32, E8M0
    scales, gradients e4m3 too): gate/up GEMM whose epilogue applies the gated GELU and
    quantizes H in blocks (no tensor-wide amax, no bf16 H in memory), down GEMM; backward through dH, the gelu chain's dGU and
    the dgrad/wgrad GEMMs on the columnwise copies. ``gu_q`` / ``down_q``: optional cached
    MX weights (with their columnwise copies). Reference: TEMLP / FusedMLP (te.LayerNormMLP)
    under 'mxfp8' (bongard/te_linear.py:98-103, bongard/fused_mlp.py:25-33)."""

    @staticmethod
    def forward(ctx, x, w_gu, w_down, gu_q, down_q, intermediate):
        I = int(intermediate)
        need_dx, need_dgu, need_dd = _forward_needs(ctx, 3)
        train = need_dx or need_dgu or need_dd
        if not train and (gu_q is None or down_q is None):
            # inference: x and the uncached weights in one rowwise launch
            ws = [w for w, q in ((w_gu, gu_q), (w_down, down_q)) if q is None]
            qs = ops.quantize_mx_many([x] + [w.detach() for w in ws])
            xq = qs[0]
            if gu_q is None:
                gu_q = qs[1]
            if down_q is None:
                down_q = qs[-1]
        else:
            xq = ops.quantize_mx(x, E4M3, rowwise=True, colwise=need_dgu)
        if gu_q is None:
            gu_q = quantize_weight_mx(w_gu, transpose=need_dx)
        # H is quantized (rowwise, plus the columnwise copy for the down wgrad) in the
        # GEMM's epilogue; the bf16 H itself is never written
        hq, GU, _ = ops.gemm_geglu_mx_quant(xq.data, xq.scales, gu_q.data, gu_q.scales, I,
                                            colwise=need_dd, keep_gu=train)
        if down_q is None:
            down_q = quantize_weight_mx(w_down, transpose=need_dx or need_dgu)
        y = ops.gemm_mx(hq.data, hq.scales, down_q.data, down_q.scales)
        ctx.intermediate = I
        ctx.save_for_backward(GU, xq.data_t, xq.scales_t, hq.data_t, hq.scales_t, gu_q.data_t,
                              gu_q.scales_t, down_q.data_t, down_q.scales_t)
        return y

    @staticmethod
    def backward(ctx, dy):
        GU, x8t, xst, h8t, hst, gu8t, gust, d8t, dst = ctx.saved_tensors
        need_dx, need_dgu, need_dd = ctx.needs_input_grad[:3]
        dyq = ops.quantize_mx(dy.contiguous(), E4M3, rowwise=need_dx or need_dgu,
                              colwise=need_dd)
        dx = dgu = dd = None
        if need_dd:
            dd = ops.gemm_mx(dyq.data_t, dyq.scales_t, h8t, hst)
        if need_dx or need_dgu:
            dH = ops.gemm_mx(dyq.data, dyq.scales, d8t, dst)
            dGU, _ = ops.geglu_bwd(dH, GU)
            dq = ops.quantize_mx(dGU, E4M3, rowwise=need_dx, colwise=need_dgu)
            if need_dx:
                dx = ops.gemm_mx(dq.data, dq.scales, gu8t, gust)
            if need_dgu:
                dgu = ops.gemm_mx(dq.data_t, dq.scales_t, x8t, xst)
        return dx, dgu, dd, None, None, None


def mlp_forward(x, w_gu, w_down, gu_q, down_q, intermediate, split_scales, scaling, x_amax,
                needs):
    """Forward of the FP8 gated MLP (see Fp8GegluMlpFunction): ``(y, saved)`` with saved =
    (GU, x8, x_meta, h8, h_meta, gu8, gu_meta, d8, d_meta): the bf16 pre-activations and the
    fp8 tensors the forward computed with (X8, H8, W_gu8, W_down8), which the backward reads
    as they are (K-major dgrad / wgrad operands), None where no gradient needs them; no
    transposed fp8 copy is made. ``needs``: (dx, dW_gu, dW_down) wanted."""
    I = int(intermediate)
    need_dx, need_dgu, need_dd = needs
    train = need_dx or need_dgu or need_dd
    if train:
        _check_trainable("fp8 gated MLP", x.shape[-1], I, w_down.shape[0])
    if scaling is not None and split_scales:
        raise NotImplementedError("delayed scaling needs the fused [gate; up] weight")
    gs, ds = scaling if scaling is not None else (None, None)
    if (scaling is None and x_amax is None and not split_scales
            and (gu_q is None or down_q is None)):
        # current scaling: x and the uncached weights in one amax + one cast launch
        ws = [w for w, q in ((w_gu, gu_q), (w_down, down_q)) if q is None]
        qs = ops.quantize_many([x] + [w.detach() for w in ws])
        xq = qs[0]
        if gu_q is None:
            gu_q = _GateUp(qs[1].data, None, qs[1].meta.view(1, 4))
        if down_q is None:
            down_q = qs[-1]
    elif gs is not None and x_amax is None and gu_q is None and down_q is None:
        # delayed scaling with every operand quantized here: x, [W_gate; W_up] and W_down
        # in one launch
        xq, wq, down_q = _scaling.quantize_many([
            (gs.input, x, True, False),
            (gs.weight, w_gu.detach(), True, False),
            (ds.weight, w_down.detach(), True, False)])
        gu_q = _GateUp(wq.data, None, wq.meta.view(1, 4))
    else:
        xq = _quantize_input(x, gs and gs.input, x_amax, False)
    if gu_q is None:
        gu_q = quantize_gate_up(w_gu, I, split_scales, scaler=gs and gs.weight)
    stride = 4 if split_scales else 0
    M = xq.rows
    if ds is None:
        H, GU, hparts = ops.gemm_geglu(xq.data, xq.meta, gu_q.data, gu_q.meta, I,
                                       w_meta_stride=stride, keep_gu=train)
        hq = ops.cast_partials(H, hparts, E4M3, rowwise=True)
    else:
        # H's scale is known before the GEMM: the epilogue casts H itself; no bf16 H round
        # trip
        count = ops.geglu_partials_count(M, I)

        def replay(meta, parts):
            q, gu, _, _ = ops.gemm_geglu_quant(xq.data, xq.meta, gu_q.data, gu_q.meta, I, meta,
                                               keep_gu=train, partials=parts)
            return q, gu

        def launch(st, length, pos, prev, parts):
            return replay(ops.delayed_scale_fold(st, length, pos, prev, E4M3), parts)

        hq, GU = ds.input.produce(count, x.device, launch, replay)
    h_meta = hq.meta
    if down_q is None:
        down_q = quantize_weight(w_down, scaler=ds and ds.weight)
    y = ops.gemm(hq.data, E4M3, h_meta, down_q.data, E4M3, down_q.meta)
    return y, (GU, xq.data if need_dgu else None, xq.meta, hq.data if need_dd else None, h_meta,
               gu_q.data if need_dx else None, gu_q.meta,
               down_q.data if need_dx or need_dgu else None, down_q.meta)


def mlp_backward(dy, saved, intermediate, split_scales, scaling, needs):
    """Backward of the FP8 gated MLP: ``(dx, dW_gu, dW_down)`` (None where not wanted). Every
    GEMM reads its fp8 operands as their producers wrote them (bf8_gemm_kmajor): dY8, the
    saved H8, W_down8, W_gu8, X8 and dGU8; no transposed copy is made."""
    (GU, x8, x_meta, h8, h_meta, gu8, gu_meta, d8, d_meta) = saved
    I = int(intermediate)
    need_dx, need_dgu, need_dd = needs
    gs, ds = scaling if scaling is not None else (None, None)
    dyq = _quantize(dy.contiguous(), E5M2, ds and ds.grad_output)

    def gemm_b(a, a_meta, b, b_meta, *, a_kmajor=False):
        # e5m2 gradient A (or A^T) against the saved e4m3 B, given as B^T [K, N]
        return ops.gemm_kmajor(a, E5M2, a_meta, b, E4M3, b_meta, a_kmajor=a_kmajor)

    dx = dgu = dd = None
    if need_dd:
        dd = gemm_b(dyq.data, dyq.meta, h8, h_meta, a_kmajor=True)   # dW_down = dY^T . H
    if not (need_dx or need_dgu):
        return dx, dgu, dd
    dH = gemm_b(dyq.data, dyq.meta, d8, d_meta)                     # dH = dY . W_down
    if gs is not None:
        # delayed scaling: dGU's scale is known already, so the gelu backward writes
        # fp8 dGU in the same pass
        M = dH.shape[0]
        count = ops.geglu_bwd_delayed_partials_count(M, I)
        scaler = gs.grad_output
        dq = scaler.produce(count, dH.device, lambda st, L, pos, prev, parts:
                            ops.geglu_bwd_delayed(dH, GU, st, L, pos, prev, scaler.fmt,
                                                  partials_out=parts))
        if need_dx:
            dx = gemm_b(dq.data, dq.meta, gu8, gu_meta[0])            # dX = dGU . W_gu
        if need_dgu:
            dgu = gemm_b(dq.data, dq.meta, x8, x_meta, a_kmajor=True)  # dW_gu = dGU^T . X
        return dx, dgu, dd
    dGU, gparts = ops.geglu_bwd(dH, GU)
    if not split_scales:
        dq = ops.cast_partials(dGU, gparts, E5M2, rowwise=True)
        if need_dx:
            dx = gemm_b(dq.data, dq.meta, gu8, gu_meta[0])
        if need_dgu:
            dgu = gemm_b(dq.data, dq.meta, x8, x_meta, a_kmajor=True)
    else:
        # Separate gate/up projections: each gradient has its own e5m2 scale and its
        # own dgrad GEMM; the input gradient is their bf16 sum (autograd of x used twice).
        dx_parts, dw_parts = [], []
        for half in range(2):
            d_half = dGU[:, half * I:(half + 1) * I].contiguous()
            dq = ops.quantize(d_half, E5M2)
            if need_dx:
                dx_parts.append(gemm_b(dq.data, dq.meta, gu8[half * I:(half + 1) * I],
                                       gu_meta[half]))
            if need_dgu:
                dw_parts.append(gemm_b(dq.data, dq.meta, x8, x_meta, a_kmajor=True))
        if need_dx:
            dx = dx_parts[0] + dx_parts[1]
        if need_dgu:
            dgu = torch.cat(dw_parts, 0)
    return dx, dgu, dd


class Fp8GegluMlpFunction(_Fp8Function):
    """y = down(gelu_tanh(x Wg^T) * (x Wu^T)) with every GEMM in FP8.

    w_gu: bf16 [2I, K] (gate rows then up rows), w_down: bf16 [K_out, I]. ``gu_q`` and
    ``down_q`` are optional cached quantized weights. ``split_scales`` selects one scale
    per gate/up half (torchao / split TE) instead of one shared scale (fused TE gate_up).
    ``scaling``: None (current scaling) or ``(gate_up, down)`` LinearScaling objects for
    delayed scaling (roles: x, W_gu, dGU of gate_up; H, W_down, dY of down).
    ``x_amax``: amax partials of x written by its producer (the fused RMSNorm): a partials
    tensor under current scaling, the producer count under delayed scaling; None = none.
    """

    @staticmethod
    def forward(ctx, x, w_gu, w_down, gu_q, down_q, intermediate, split_scales, scaling=None,
                x_amax=None):
        y, saved = mlp_forward(x, w_gu, w_down, gu_q, down_q, intermediate, split_scales,
                               scaling, x_amax, _forward_needs(ctx, 3))
        ctx.intermediate = int(intermediate)
        ctx.split_scales = split_scales
        ctx.scaling = scaling
        ctx.save_for_backward(*saved)
        return y

    @staticmethod
    def backward(ctx, dy):
        dx, dgu, dd = mlp_backward(dy, ctx.saved_tensors, ctx.intermediate, ctx.split_scales,
                                   ctx.scaling, tuple(ctx.needs_input_grad[:3]))
        return dx, dgu, dd, None, None, None, None, None, None


def quantize_gate_up(w_gu, intermediate, split_scales, *, transpose=False, scaler=None):
    """Quantize [W_gate; W_up] into one [2I, K] fp8 buffer (+ with ``transpose`` a [K, 2I]
    transposed copy, which the K-major backward does not need).

    split_scales: gate and up halves get separate metas (meta is then [2, 4]).
    scaler: a DelayedScaler for the shared scale (delayed scaling), or None.
    """
    I = int(intermediate)
    if not split_scales:
        q = _quantize(w_gu.detach(), E4M3, scaler, rowwise=True, transpose=transpose)
        return _GateUp(q.data, q.data_t, q.meta.view(1, 4))
    if scaler is not None:
        raise NotImplementedError("delayed scaling needs the fused [gate; up] weight")
    K = w_gu.shape[1]
    dev = w_gu.device
    data = torch.empty((2 * I, K), dtype=torch.float8_e4m3fn, device=dev)
    meta = ops.new_meta(dev, 2)
    halves_t = []
    for half in range(2):
        part = w_gu.detach()[half * I:(half + 1) * I]
        q = ops.quantize(part, E4M3, rowwise=True, transpose=transpose, meta=meta[half],
                         out=data[half * I:(half + 1) * I])
        halves_t.append(q.data_t)
    data_t = torch.cat(halves_t, 1) if transpose else None
    return _GateUp(data, data_t, meta)


@dataclass
class _GateUp:
    """Quantized gate/up weight: data [2I, K], data_t [K, 2I], meta [1 or 2, 4]."""

    data: torch.Tensor
    data_t: Optional[torch.Tensor]
    meta: torch.Tensor
