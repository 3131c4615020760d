"""Norm + gated MLP as one FP8 training module with Hugging Face checkpoint weights (MI355X).

Drop-in for bongard/fused_mlp.py (TransformerEngine te.LayerNormMLP path): same
``RECIPES``, ``FusedMLP(mlp, norm, recipe)`` with parameters ``layer_norm_weight``
[hidden], ``fc1_weight`` [2I, hidden] (= [gate; up]), ``fc2_weight`` [hidden, I] and an
``_extra_state`` (empty for 'fp8'; the amax histories for 'fp8_delayed'); HF eval views (``_hf_mlp``, ``_hf_norm``) sharing storage and
refreshed by ``_apply``; counters ``weight_quantizations`` / ``cached_weights`` /
``real_tokens`` / ``kernel_tokens``; ``enable_fused_mlp(model, recipe) -> int``; and
``hf_state_dict(backbone)`` for export.

Training forward: RMSNorm with zero-centred gamma (``x * rsqrt(mean(x^2) + eps) *
(1 + w)`` in fp32, rounded to bf16, as HF T5Gemma2RMSNorm) in one HIP kernel that also
writes the amax partials of its output, so the e4m3 cast of the norm output needs no amax
pass (TE LayerNormMLP fuses norm and cast the same way, bongard/fused_mlp.py:25-30); then
the FP8 gated MLP of bongard_amd.linear.Fp8GegluMlpFunction (fc1 + gated-GELU epilogue,
H quantized, fc2). fc1 keeps one shared scale for [gate; up], as TE's stacked fc1 weight
does. Whether TE rounds the norm output to bf16 before its cast is not pinned by anything
available; this path rounds it (the te_linear chain). The norm's backward (dx and the
weight gradient of the HF formula's autograd, fp32 math) is a kernel as well
(bf8_rmsnorm_bwd_bf16).
"""

from collections import Counter

import torch

from . import linear as _linear
from . import ops as _ops
from . import scaling as _scaling
from .te_linear import (RECIPES, _is_mx, _is_nvfp4, _make_recipe, _new_scaling, _pad_rows, _ScalingExtraState,
                        present)

__all__ = ["RECIPES", "FusedMLP", "enable_fused_mlp", "hf_state_dict"]


def _rms_norm(x, weight, eps):
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + weight.float())).type_as(x)


class _FusedRMSNorm(torch.autograd.Function):
    """bf16 RMSNorm (zero-centred gamma) whose kernel also writes the amax partials of its
    output into ``partials``; the backward is one kernel pass over x and dy for dx plus a
    fixed-order reduction for the weight gradient (the autograd of :func:`_rms_norm`)."""

    @staticmethod
    def forward(ctx, x, weight, eps, partials):
        y, _, _ = _ops.rmsnorm(x, weight, eps, zero_centered=True, partials=partials)
        ctx.eps = eps
        ctx.save_for_backward(x, weight)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        dx, dw = _ops.rmsnorm_backward(x, dy.contiguous(), weight, ctx.eps, zero_centered=True,
                                       need_dx=ctx.needs_input_grad[0],
                                       need_dw=ctx.needs_input_grad[1])
        return dx, dw, None, None


class FusedMLP(_ScalingExtraState, torch.nn.Module):
    """RMSNorm -> fc1 = [gate; up] -> gelu_tanh(gate) * up -> fc2, in FP8 while training."""

    def __init__(self, mlp, norm, recipe):
        super().__init__()
        if mlp.config.hidden_activation != 'gelu_pytorch_tanh' or mlp.dropout.p:
            raise ValueError('Fused MLP requires tanh GELU and zero dropout')
        hidden, inter = mlp.hidden_size, mlp.intermediate_size
        device = mlp.gate_proj.weight.device
        self.hidden_size = hidden
        self.eps = norm.eps
        self.bongard_recipe = recipe
        self.recipe = _make_recipe(recipe)
        self.intermediate_size = inter

        def param(*shape):
            return torch.nn.Parameter(torch.zeros(*shape, dtype=torch.bfloat16, device=device))

        self.layer_norm_weight = param(hidden)
        self.fc1_weight = param(2 * inter, hidden)
        self.fc2_weight = param(hidden, inter)
        with torch.no_grad():
            self.layer_norm_weight.copy_(norm.weight)
            self.fc1_weight[:inter].copy_(mlp.gate_proj.weight)
            self.fc1_weight[inter:].copy_(mlp.up_proj.weight)
            self.fc2_weight.copy_(mlp.down_proj.weight)
        # Evaluation runs the original HF modules on views of these parameters; they are
        # attached with object.__setattr__ so they are not registered submodules.
        object.__setattr__(self, '_hf_mlp', mlp.eval())
        object.__setattr__(self, '_hf_norm', norm.eval())
        self._refresh_hf_views()
        self.counts = Counter()
        self._cached_weight_versions = None
        self._fp8_weights = None
        # delayed scaling: (fc1 roles: norm output, fc1 weight, dGU), (fc2: H, fc2, dY)
        fc1, fc2 = _new_scaling(self.recipe), _new_scaling(self.recipe)
        self.scaling = (fc1, fc2) if fc1 is not None else None

    def _delayed_scalings(self):
        return list(self.scaling) if self.scaling is not None else []

    def _refresh_hf_views(self):
        inter = self.intermediate_size
        self._hf_norm.weight = self.layer_norm_weight
        mlp = self._hf_mlp
        mlp.gate_proj.weight = torch.nn.Parameter(self.fc1_weight[:inter], requires_grad=False)
        mlp.up_proj.weight = torch.nn.Parameter(self.fc1_weight[inter:], requires_grad=False)
        mlp.down_proj.weight = self.fc2_weight

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse=recurse)
        self._refresh_hf_views()
        self._cached_weight_versions = None
        self._fp8_weights = None
        return self

    def forward(self, x):
        if self.training:
            return self._fp8_forward(x)
        return self._hf_mlp(self._hf_norm(x))

    @torch.compiler.disable
    def _fp8_forward(self, x):
        flat = x.reshape(-1, x.shape[-1])
        versions = (self.fc1_weight._version, self.fc2_weight._version)
        first = versions != self._cached_weight_versions or self._fp8_weights is None
        self._cached_weight_versions = versions
        self.counts['weight_quantizations' if first else 'cached_weights'] += 1
        flat, length, aligned = _pad_rows(flat)
        self.counts['real_tokens'] += length
        self.counts['kernel_tokens'] += aligned
        fc1, fc2 = self.scaling if self.scaling is not None else (None, None)
        mx = _is_mx(self.recipe)
        if _is_nvfp4(self.recipe):
            return self._nvfp4_forward(x, flat, length, first)
        if first:
            if mx:
                self._fp8_weights = (_linear.quantize_weight_mx(self.fc1_weight),
                                     _linear.quantize_weight_mx(self.fc2_weight))
            elif fc1 is not None:
                # delayed scaling: both weights in one launch
                wq, dq = _scaling.quantize_many([
                    (fc1.weight, self.fc1_weight.detach(), True, False),
                    (fc2.weight, self.fc2_weight.detach(), True, False)])
                self._fp8_weights = (_linear._GateUp(wq.data, None, wq.meta.view(1, 4)), dq)
            else:
                self._fp8_weights = (
                    _linear.quantize_gate_up(self.fc1_weight, self.intermediate_size,
                                             split_scales=False),
                    _linear.quantize_weight(self.fc2_weight))
        gu_q, down_q = self._fp8_weights
        flat = flat.to(torch.bfloat16).contiguous()
        if mx:
            # block scales need no tensor-wide amax: the norm's partials go unused
            if _ops.rmsnorm_supported(flat.shape[1]):
                parts = torch.empty(_ops.rmsnorm_partials_count(flat.shape[0]),
                                    dtype=torch.int32, device=flat.device)
                normed = _FusedRMSNorm.apply(flat, self.layer_norm_weight, self.eps, parts)
            else:
                normed = _rms_norm(flat, self.layer_norm_weight, self.eps)
            out = _linear.Fp8GegluMlpMxFunction.apply(normed, self.fc1_weight, self.fc2_weight,
                                                      gu_q, down_q, self.intermediate_size)
            return out[:length].reshape_as(x)
        count = _ops.rmsnorm_partials_count(flat.shape[0])
        if not _ops.rmsnorm_supported(flat.shape[1]):
            # rows wider than the fused kernel holds in registers: norm in torch ops on the
            # device, then the cast's own amax pass
            parts, x_amax = None, None
            normed = _rms_norm(flat, self.layer_norm_weight, self.eps)
        elif fc1 is None:
            parts = torch.empty(count, dtype=torch.int32, device=flat.device)
            x_amax = parts
        else:
            parts = fc1.input.partials_for_producer(count, flat.device)
            x_amax = count
        if parts is not None:
            normed = _FusedRMSNorm.apply(flat, self.layer_norm_weight, self.eps, parts)
        out = _linear.Fp8GegluMlpFunction.apply(normed, self.fc1_weight, self.fc2_weight, gu_q,
                                                down_q, self.intermediate_size, False,
                                                self.scaling, x_amax)
        return out[:length].reshape_as(x)


    def _nvfp4_forward(self, x, flat, length, first):
        """'nvfp4': the fused norm, fc1 as an NVFP4 GEMM (operands dequantized exactly to
        bf16 for the MFMA) with the gated GELU in its epilogue, fc2 as an NVFP4 GEMM."""
        if first:
            self._fp8_weights = (
                _linear.quantize_weight_nvfp4(self.fc1_weight, cache_dequant=True),
                _linear.quantize_weight_nvfp4(self.fc2_weight, cache_dequant=True))
        gu_q, down_q = self._fp8_weights
        flat = flat.to(torch.bfloat16).contiguous()
        parts = None
        if _ops.rmsnorm_supported(flat.shape[1]):
            # the norm writes its output's amax partials: fc1's NVFP4 quantizer of the
            # normed rows takes its tensor amax from them (no amax pass of its own)
            parts = torch.empty(_ops.rmsnorm_partials_count(flat.shape[0]), dtype=torch.int32,
                                device=flat.device)
            normed = _FusedRMSNorm.apply(flat, self.layer_norm_weight, self.eps, parts)
        else:
            normed = _rms_norm(flat, self.layer_norm_weight, self.eps)
        h, h_partials = _linear.GegluGateUpNvfp4Function.apply(normed, self.fc1_weight, gu_q,
                                                                self.intermediate_size, parts)
        out = _linear.Fp8LinearNvfp4Function.apply(h, self.fc2_weight, down_q, h_partials)
        return out[:length].reshape_as(x)


def enable_fused_mlp(model, recipe):
    """Replace every text layer's MLP (and its pre-MLP norm) with FusedMLP; returns count.

    The norm moves inside the module, so ``pre_feedforward_layernorm`` becomes Identity.
    """
    if model.device.type != 'cuda' or recipe not in RECIPES:
        raise ValueError('Fused MLP requires CUDA and a supported low-precision recipe')
    from .te_linear import _text_layers

    count = 0
    for layer in _text_layers(model):
        if isinstance(layer.mlp, FusedMLP):
            if layer.mlp.bongard_recipe != recipe:
                raise ValueError('An existing fused MLP must retain its recipe')
        else:
            layer.mlp = FusedMLP(layer.mlp, layer.pre_feedforward_layernorm, recipe)
            layer.pre_feedforward_layernorm = torch.nn.Identity()
        count += 1
    return count


def _fused_export(name, module, state):
    prefix = name + '.'
    if state.pop(prefix + '_extra_state').numel() != 0:
        raise ValueError('Fused MLP export requires stateless quantization scaling')
    gate, up = state.pop(prefix + 'fc1_weight').split(module.intermediate_size)
    state[prefix + 'gate_proj.weight'] = gate
    state[prefix + 'up_proj.weight'] = up
    state[prefix + 'down_proj.weight'] = state.pop(prefix + 'fc2_weight')
    layer_prefix = name.rpartition('.')[0]
    state[layer_prefix + '.pre_feedforward_layernorm.weight'] = state.pop(
        prefix + 'layer_norm_weight')


def hf_state_dict(backbone):
    """The backbone state dict in Hugging Face keys, or None if nothing was converted.

    Undoes both this file's FusedMLP layout and te_linear's projection layout, so the
    result loads into the original T5Gemma2 modules (save_pretrained).
    """
    from . import te_linear

    fused = [(n, m) for n, m in backbone.named_modules()
             if hasattr(m, 'bongard_recipe') and hasattr(m, 'fc1_weight')]
    has_te = present(backbone)
    if not (fused or has_te):
        return None
    state = backbone.state_dict()
    if has_te:
        state = te_linear.restore_hf_layout(backbone, state)
    for name, module in fused:
        _fused_export(name, module, state)
    return state
