"""The decoder's state-bank K/V projection on the FP8 projections (MI355X).

Drop-in for ``project_state_kv(attention, state)`` (bongard/model.py:342-347), which
``JudgmentModel.state_kv`` (bongard/model.py:349-359) runs once per decoder layer on the
encoded state: ``keys = k_norm(k_proj(state))``, ``values = v_proj(state)`` as
[batch, heads, tokens, head_dim], no RoPE. When k_proj and v_proj are TELinear
projections under per-tensor current scaling ('fp8') in training, both read the same
input: it is quantized once (the two separate calls would quantize the identical tensor
twice, to the identical bytes and scale) and each projection runs its GEMM on its own
cached FP8 weight. Outputs and gradients equal the two separate calls bit for bit: the
input gradient is the bf16 sum of the two dgrad GEMMs, as autograd forms it for an input
used twice. Any other configuration calls the projections as the reference does.
"""

import torch

from . import ops
from .ops import E4M3, E5M2
from .linear import _Fp8Function, _check_trainable, _forward_needs
from .te_linear import Float8CurrentScaling, TELinear, _pad_rows

__all__ = ["project_state_kv"]


class _SharedInputFp8Function(_Fp8Function):
    """y_i = x @ W_i^T for several per-tensor-scaled FP8 projections of one input x
    [M, K] (M % 32 == 0): one e4m3 quantization of x, one GEMM per cached weight; backward
    per projection as Fp8LinearFunction (X8, W8_i and dY8 read as K-major operands), the
    input gradients summed in bf16 in projection order."""

    @staticmethod
    def forward(ctx, x, wqs, *weights):
        needs = _forward_needs(ctx, len(ctx.needs_input_grad))
        need_dx = needs[0]
        need_dw = any(needs[2:])
        if need_dx or need_dw:
            _check_trainable("shared-input projections", x.shape[-1],
                             *[wq.data.shape[0] for wq in wqs])
        xq = ops.quantize(x, E4M3)
        outs = [ops.gemm(xq.data, E4M3, xq.meta, wq.data, E4M3, wq.meta) for wq in wqs]
        ctx.n = len(wqs)
        ctx.need_dx = need_dx
        saved = [xq.data if need_dw else None, xq.meta]
        for wq in wqs:
            saved += [wq.data if need_dx else None, wq.meta]
        ctx.save_for_backward(*saved)
        return tuple(outs)

    @staticmethod
    def backward(ctx, *dys):
        saved = ctx.saved_tensors
        x8, x_meta = saved[0], saved[1]
        dx = None
        dws = []
        for i, dy in enumerate(dys):
            w8, w_meta = saved[2 + 2 * i], saved[3 + 2 * i]
            need_dw = ctx.needs_input_grad[2 + i]
            if dy is None:
                dws.append(None)
                continue
            dyq = ops.quantize(dy.contiguous(), E5M2)
            if ctx.need_dx:
                part = ops.gemm_kmajor(dyq.data, E5M2, dyq.meta, w8, E4M3, w_meta)
                dx = part if dx is None else dx + part
            dws.append(ops.gemm_kmajor(dyq.data, E5M2, dyq.meta, x8, E4M3, x_meta, a_kmajor=True)
                       if need_dw else None)
        return (dx, None, *dws)


def _shared_input_ok(projections):
    return all(isinstance(p, TELinear) and p.training
               and isinstance(p.recipe, Float8CurrentScaling) for p in projections)


@torch.compiler.disable
def shared_input_projections(x, projections):
    """Outputs of several TELinear projections of one input (see module doc). Opaque to
    torch.compile, like the projections themselves: the reference compiles
    project_state_kv (bongard/model.py:279), which then runs this part eagerly."""
    flat = x.reshape(-1, x.shape[-1])
    flat, length, aligned = _pad_rows(flat)
    if flat.dtype != torch.bfloat16:
        flat = flat.to(torch.bfloat16)
    wqs = [p.fp8_weight(p._note_microbatch()) for p in projections]
    outs = _SharedInputFp8Function.apply(flat, wqs, *[p.weight for p in projections])
    res = []
    for out in outs:
        if aligned != length:
            out = out[:length]
        res.append(out.reshape(*x.shape[:-1], out.shape[-1]))
    return res


def project_state_kv(attention, state):
    """keys (k_norm applied) and values of the encoded state, [B, heads, S, head_dim]."""
    shape = (*state.shape[:-1], -1, attention.head_dim)
    k_proj, v_proj = attention.k_proj, attention.v_proj
    if _shared_input_ok((k_proj, v_proj)):
        k, v = shared_input_projections(state, (k_proj, v_proj))
    else:
        k, v = k_proj(state), v_proj(state)
    keys = attention.k_norm(k.view(shape).transpose(1, 2))
    values = v.view(shape).transpose(1, 2)
    return keys, values
