"""Compile-visible FP8 ops: torch.library custom ops with fake and autograd registrations.

The reference compiles every text layer (bongard/model.py:249-283) and its torchao
Float8Linear is traced by Inductor inside them (bongard/model.py:265-270). The FP8 kernels
here are ctypes calls that Dynamo cannot trace, so they are registered as custom ops, in
the pattern of bongard/flash_varlen.py:13-58: each op has a fake implementation (shapes and
dtypes only) and an autograd formula whose backward is another custom op. A compiled
region then holds one opaque node per FP8 op instead of breaking its graph around it.

  bongard_fp8::linear             torchao's three recipes (tensorwise, rowwise,
                                  rowwise_with_gw_hp): y and the tensors its backward reads
  bongard_fp8::linear_backward    (dx, dW)
  bongard_fp8::geglu_mlp          the gated MLP under per-tensor current scaling (TEMLP /
                                  FusedMLP arithmetic, 'fp8' recipe): y and its saved tensors
  bongard_fp8::geglu_mlp_backward (dx, dW_gate_up, dW_down)

The ops run the same code as the eager autograd functions of bongard_amd.linear, so a
compiled region gives the eager results bit for bit. Saved tensors a call does not need are
returned as empty tensors (custom ops return no None).
"""

from typing import Optional

import torch
from torch import Tensor

from . import linear as _linear

_F8 = torch.float8_e4m3fn


def _or_empty(t, like, dtype):
    return t if t is not None else like.new_empty(0, dtype=dtype)


def _none_if_empty(t):
    return None if t is None or t.numel() == 0 else t


# ---- linear ----------------------------------------------------------------------------
@torch.library.custom_op("bongard_fp8::linear", mutates_args=())
def _linear_op(x: Tensor, weight: Tensor, bias: Optional[Tensor], recipe: str, need_dx: bool,
               need_dw: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    if recipe == "tensorwise":
        y, (x8, xs, w8, ws) = _linear.linear_forward(x, weight, bias, None, None, need_dx,
                                                     need_dw)
        # x and W share one quantize launch, whose two metas are rows of one [2, 4] tensor;
        # a custom op's outputs may not alias each other, so each meta leaves as its own
        # 4-float copy
        return (y, _or_empty(x8, x, _F8), xs.clone(), _or_empty(w8, x, _F8), ws.clone())
    y, saved = _linear.linear_axiswise_forward(x, weight, bias, recipe, need_dx, need_dw)
    if recipe == "rowwise_with_gw_hp":   # the backward reads the op's inputs themselves
        e8, e32 = x.new_empty(0, dtype=_F8), x.new_empty(0, dtype=torch.float32)
        return y, e8, e32, e8.clone(), e32.clone()
    x8t, xcs, w8t, wcs = saved
    return (y, _or_empty(x8t, x, _F8), _or_empty(xcs, x, torch.float32), _or_empty(w8t, x, _F8),
            _or_empty(wcs, x, torch.float32))


@_linear_op.register_fake
def _linear_fake(x, weight, bias, recipe, need_dx, need_dw):
    M, K = x.shape
    N = weight.shape[0]
    y = x.new_empty((M, N), dtype=torch.bfloat16)

    def f8(shape, keep):
        return x.new_empty(shape if keep else (0,), dtype=_F8)

    def f32(shape, keep):
        return x.new_empty(shape if keep else (0,), dtype=torch.float32)

    if recipe == "tensorwise":
        # the saved fp8 X and W are the forward's own (K-major backward)
        return y, f8((M, K), need_dw), f32((4,), True), f8((N, K), need_dx), f32((4,), True)
    if recipe == "rowwise":
        return (y, f8((K, M), need_dw), f32((K,), need_dw), f8((K, N), need_dx),
                f32((K,), need_dx))
    return y, f8((0,), False), f32((0,), False), f8((0,), False), f32((0,), False)


@torch.library.custom_op("bongard_fp8::linear_backward", mutates_args=())
def _linear_bwd_op(dy: Tensor, s0: Tensor, s1: Tensor, s2: Tensor, s3: Tensor,
                   x: Optional[Tensor], weight: Optional[Tensor], recipe: str,
                   in_features: int, need_dx: bool, need_dw: bool) -> tuple[Tensor, Tensor]:
    if recipe == "tensorwise":
        dx, dw = _linear.linear_backward(dy, (_none_if_empty(s0), s1, _none_if_empty(s2), s3),
                                         None, need_dx, need_dw)
    elif recipe == "rowwise":
        dx, dw = _linear.linear_axiswise_backward(dy, (s0, s1, s2, s3), recipe, need_dx, need_dw)
    else:
        dx, dw = _linear.linear_axiswise_backward(dy, (x, weight), recipe, need_dx, need_dw)
    return _or_empty(dx, dy, torch.bfloat16), _or_empty(dw, dy, torch.bfloat16)


@_linear_bwd_op.register_fake
def _linear_bwd_fake(dy, s0, s1, s2, s3, x, weight, recipe, in_features, need_dx, need_dw):
    M, N = dy.shape
    dx = dy.new_empty((M, in_features) if need_dx else (0,), dtype=torch.bfloat16)
    dw = dy.new_empty((N, in_features) if need_dw else (0,), dtype=torch.bfloat16)
    return dx, dw


def _linear_setup(ctx, inputs, output):
    x, weight, bias, recipe, need_dx, need_dw = inputs
    ctx.recipe = recipe
    ctx.has_bias = bias is not None
    ctx.in_features = x.shape[1]
    hp = recipe == "rowwise_with_gw_hp"
    ctx.save_for_backward(*output[1:], x if hp and need_dw else None,
                          weight if hp and need_dx else None)
    ctx.mark_non_differentiable(*output[1:])


def _linear_grad(ctx, dy, *unused):
    s0, s1, s2, s3, x, weight = ctx.saved_tensors
    need_dx, need_dw, need_db = ctx.needs_input_grad[:3]
    dx, dw = torch.ops.bongard_fp8.linear_backward(dy.contiguous(), s0, s1, s2, s3, x, weight,
                                                   ctx.recipe, ctx.in_features, need_dx,
                                                   need_dw)
    db = dy.sum(0) if ctx.has_bias and need_db else None
    return (dx if need_dx else None, dw if need_dw else None, db, None, None, None)


_linear_op.register_autograd(_linear_grad, setup_context=_linear_setup)


def fp8_linear(x, weight, bias, recipe):
    """y = x @ weight^T (+ bias) in FP8 under a torchao recipe, as one custom op (x: bf16
    [M, K], M % 16 == 0 when x or weight needs a gradient)."""
    grad = torch.is_grad_enabled()
    need_dx = grad and x.requires_grad
    need_dw = grad and weight.requires_grad
    return torch.ops.bongard_fp8.linear(x, weight, bias, recipe, need_dx, need_dw)[0]


# ---- gated MLP (per-tensor current scaling) -----------------------------------------------
@torch.library.custom_op("bongard_fp8::geglu_mlp", mutates_args=())
def _mlp_op(x: Tensor, w_gu: Tensor, w_down: Tensor, intermediate: int, split_scales: bool,
            need_dx: bool, need_dgu: bool, need_dd: bool) -> tuple[Tensor, Tensor, Tensor,
                                                                   Tensor, Tensor, Tensor,
                                                                   Tensor, Tensor, Tensor,
                                                                   Tensor]:
    y, saved = _linear.mlp_forward(x, w_gu, w_down, None, None, intermediate, split_scales,
                                   None, None, (need_dx, need_dgu, need_dd))
    GU, x8, xm, h8, hm, gu8, gum, d8, dm = saved
    return (y, _or_empty(GU, x, torch.bfloat16), _or_empty(x8, x, _F8), xm.clone(),
            _or_empty(h8, x, _F8), hm.clone(), _or_empty(gu8, x, _F8), gum.clone(),
            _or_empty(d8, x, _F8), dm.clone())


@_mlp_op.register_fake
def _mlp_fake(x, w_gu, w_down, intermediate, split_scales, need_dx, need_dgu, need_dd):
    M, K = x.shape
    I = int(intermediate)
    N = w_down.shape[0]
    train = need_dx or need_dgu or need_dd

    def t(shape, dtype, keep=True):
        return x.new_empty(shape if keep else (0,), dtype=dtype)

    # the saved fp8 tensors are the forward's own X8, H8, W_gu8, W_down8 (K-major backward)
    return (t((M, N), torch.bfloat16), t((M, 2 * I), torch.bfloat16, train),
            t((M, K), _F8, need_dgu), t((4,), torch.float32), t((M, I), _F8, need_dd),
            t((4,), torch.float32), t((2 * I, K), _F8, need_dx),
            t((2 if split_scales else 1, 4), torch.float32),
            t((N, I), _F8, need_dx or need_dgu), t((4,), torch.float32))


@torch.library.custom_op("bongard_fp8::geglu_mlp_backward", mutates_args=())
def _mlp_bwd_op(dy: Tensor, GU: Tensor, x8: Tensor, xm: Tensor, h8: Tensor, hm: Tensor,
                gu8: Tensor, gum: Tensor, d8: Tensor, dm: Tensor, intermediate: int,
                split_scales: bool, in_features: int, need_dx: bool, need_dgu: bool,
                need_dd: bool) -> tuple[Tensor, Tensor, Tensor]:
    saved = (GU, _none_if_empty(x8), xm, _none_if_empty(h8), hm, _none_if_empty(gu8), gum,
             _none_if_empty(d8), dm)
    dx, dgu, dd = _linear.mlp_backward(dy, saved, intermediate, split_scales, None,
                                       (need_dx, need_dgu, need_dd))
    return (_or_empty(dx, dy, torch.bfloat16), _or_empty(dgu, dy, torch.bfloat16),
            _or_empty(dd, dy, torch.bfloat16))


@_mlp_bwd_op.register_fake
def _mlp_bwd_fake(dy, GU, x8, xm, h8, hm, gu8, gum, d8, dm, intermediate, split_scales,
                  in_features, need_dx, need_dgu, need_dd):
    M, N = dy.shape
    I = int(intermediate)

    def t(shape, keep):
        return dy.new_empty(shape if keep else (0,), dtype=torch.bfloat16)

    return t((M, in_features), need_dx), t((2 * I, in_features), need_dgu), t((N, I), need_dd)


def _mlp_setup(ctx, inputs, output):
    x, w_gu, w_down, intermediate, split_scales, need_dx, need_dgu, need_dd = inputs
    ctx.intermediate = int(intermediate)
    ctx.split_scales = split_scales
    ctx.in_features = x.shape[1]
    ctx.save_for_backward(*output[1:])
    ctx.mark_non_differentiable(*output[1:])


def _mlp_grad(ctx, dy, *unused):
    need_dx, need_dgu, need_dd = ctx.needs_input_grad[:3]
    dx, dgu, dd = torch.ops.bongard_fp8.geglu_mlp_backward(
        dy.contiguous(), *ctx.saved_tensors, ctx.intermediate, ctx.split_scales, ctx.in_features,
        need_dx, need_dgu, need_dd)
    return (dx if need_dx else None, dgu if need_dgu else None, dd if need_dd else None,
            None, None, None, None, None)


_mlp_op.register_autograd(_mlp_grad, setup_context=_mlp_setup)


def fp8_geglu_mlp(x, w_gu, w_down, intermediate, split_scales=False):
    """y = down(gelu_tanh(x W_gate^T) * (x W_up^T)) with every GEMM in FP8 under per-tensor
    current scaling, as one custom op. w_gu: [W_gate; W_up] bf16 [2I, K]; w_down [K_out, I]."""
    grad = torch.is_grad_enabled()
    return torch.ops.bongard_fp8.geglu_mlp(x, w_gu, w_down, int(intermediate), bool(split_scales),
                                           grad and x.requires_grad, grad and w_gu.requires_grad,
                                           grad and w_down.requires_grad)[0]
