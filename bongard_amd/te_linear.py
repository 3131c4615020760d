"""FP8 projections with ordinary Hugging Face checkpoint weights (MI355X).

Drop-in for bongard/te_linear.py (TransformerEngine te.Linear path): same ``RECIPES``,
``TELinear(linears, recipe)``, ``TEMLP(mlp, recipe)``, ``enable_te_linear(model, *,
mlp=None, attention=None) -> dict``, ``present(backbone)`` and
``restore_hf_layout(backbone, state)``, with the reference's attributes
(``bongard_recipe``, ``recipe``, ``splits``, ``counts``, ``_cached_weight_version``,
``intermediate_size``, ``fused_gate_up``), state-dict keys (``weight`` and an empty
``_extra_state`` per projection), pad-to-32 rows, the ``weight._version`` quantization
cache (first microbatch quantizes, later ones reuse) and the
``BONGARD_TE_SPLIT_GATE_UP`` switch.

The 'fp8' recipe is per-tensor current scaling with HYBRID formats (e4m3 forward, e5m2
gradients), on the gfx950 kernels. In training, TEMLP runs the gate/up GEMM with the
gated-GELU fused into its epilogue and feeds H's FP8 copy to the down projection
(bongard_amd.linear.Fp8GegluMlpFunction) instead of three separate passes.
'fp8_delayed' (an addition to the reference's names) is TE's DelayedScaling with an amax
history of 16 and HYBRID formats: each projection keeps the histories of its input,
weight and output gradient in ``_extra_state``, which is then non-empty, so export raises
as the reference does for stateful scaling.
'mxfp8' is TE's MXFP8BlockScaling: every tensor (gradients included) in e4m3 blocks of 32
values sharing an E8M0 scale, on the gfx950 block-scaled MFMA
(bongard_amd.linear.Fp8LinearMxFunction / Fp8GegluMlpMxFunction); stateless, so export
works as for 'fp8'. 'nvfp4' is TE's NVFP4BlockScaling as far as its arithmetic is fixed
without TE: every tensor in e2m1 blocks of 16 with e4m3 block scales under a per-tensor fp32
scale, round to nearest even, 1-D blocks along each GEMM's reduction dimension (TE's random
Hadamard transform, stochastic rounding and 2-D weight blocks are not built). gfx950 has no
MFMA for e4m3-scaled FP4 blocks, so the blocks are dequantized exactly to bf16 and multiplied
on the bf16 MFMA (bongard_amd.linear.Fp8LinearNvfp4Function), the gated GELU in the fused
gate_up GEMM's epilogue (GegluGateUpNvfp4Function; the split projections use the elementwise
GegluFunction); stateless, like 'mxfp8'.
"""

import os
from collections import Counter
from dataclasses import dataclass

import torch
from torch.nn import functional as F

from . import linear as _linear
from . import scaling as _scaling
from .scaling import LinearScaling

RECIPES = ('nvfp4', 'mxfp8', 'fp8', 'fp8_delayed')
ATTENTION_PROJECTIONS = ('q_proj', 'k_proj', 'v_proj', 'o_proj')


@dataclass(frozen=True)
class Float8CurrentScaling:
    """Per-tensor current scaling; HYBRID = e4m3 forward tensors, e5m2 gradients."""

    fp8_format: str = "HYBRID"


@dataclass(frozen=True)
class DelayedScaling:
    """Per-tensor delayed scaling from an amax history (TE DelayedScaling defaults)."""

    fp8_format: str = "HYBRID"
    amax_history_len: int = 16
    margin: int = 0
    amax_compute_algo: str = "max"


@dataclass(frozen=True)
class MXFP8BlockScaling:
    """OCP MXFP8: 32-element blocks with E8M0 scales, e4m3 for every tensor (TE default)."""

    fp8_format: str = "E4M3"


@dataclass(frozen=True)
class NVFP4BlockScaling:
    """NVFP4: e2m1 values in 16-element blocks with e4m3 block scales and a per-tensor fp32
    scale, for every tensor (round to nearest even; no Hadamard transform, no stochastic
    rounding, 1-D blocks)."""

    fp4_format: str = "E2M1"
    block_size: int = 16


def _make_recipe(name):
    if name == 'fp8':
        return Float8CurrentScaling()
    if name == 'fp8_delayed':
        return DelayedScaling()
    if name == 'mxfp8':
        return MXFP8BlockScaling()
    if name == 'nvfp4':
        return NVFP4BlockScaling()
    raise ValueError(f'TE recipe must be one of {RECIPES}')


def _is_mx(recipe):
    return isinstance(recipe, MXFP8BlockScaling)


def _is_nvfp4(recipe):
    return isinstance(recipe, NVFP4BlockScaling)


def _new_scaling(recipe):
    """The delayed-scaling state a module needs for ``recipe`` (None: stateless)."""
    if isinstance(recipe, DelayedScaling):
        return LinearScaling(recipe.amax_history_len)
    return None


def _te_linear(module):
    return hasattr(module, 'bongard_recipe') and hasattr(module, 'splits')


def _te_mlp(module):
    return hasattr(module, 'bongard_recipe') and hasattr(module, 'fused_gate_up')


def _pad_rows(flat, multiple=32):
    length = flat.shape[0]
    aligned = (length + multiple - 1) // multiple * multiple
    if aligned != length:
        flat = F.pad(flat, (0, 0, 0, aligned - length))
    return flat, length, aligned


class _ScalingExtraState:
    """``_extra_state``: an empty uint8 tensor for stateless (current) scaling; the amax
    histories (float32) of the module's delayed-scaling roles otherwise."""

    def _delayed_scalings(self):
        return []

    def get_extra_state(self):
        scalings = self._delayed_scalings()
        if not scalings:
            return torch.empty(0, dtype=torch.uint8)
        return torch.cat([sc.to_tensor() for sc in scalings])

    def set_extra_state(self, state):
        n = state.numel() if state is not None and hasattr(state, 'numel') else 0
        scalings = self._delayed_scalings()
        if not scalings:
            if n:
                raise ValueError('stateless FP8 scaling has no extra state to load')
            return
        if n == 0:
            return
        sizes = [sc.to_tensor().numel() for sc in scalings]
        if n != sum(sizes):
            raise ValueError('delayed-scaling extra state does not match this module')
        start = 0
        for sc, size in zip(scalings, sizes):
            sc.load_tensor(state[start:start + size])
            start += size


class TELinear(_ScalingExtraState, torch.nn.Module):
    """One FP8 linear serving one or more stacked HF Linear weights of the same input."""

    def __init__(self, linears, recipe):
        super().__init__()
        if any(linear.bias is not None for linear in linears):
            raise ValueError('TE projections require bias-free HF linears')
        splits = [linear.out_features for linear in linears]
        self.in_features = linears[0].in_features
        self.out_features = sum(splits)
        self.bongard_recipe = recipe
        self.recipe = _make_recipe(recipe)
        self.weight = torch.nn.Parameter(torch.zeros(
            self.out_features, self.in_features, dtype=torch.bfloat16,
            device=linears[0].weight.device))
        self.splits = splits
        with torch.no_grad():
            self.weight.copy_(torch.cat([linear.weight for linear in linears], 0))
        self.counts = Counter()
        self._cached_weight_version = None
        self._fp8_weight = None
        self.scaling = _new_scaling(self.recipe)

    def _delayed_scalings(self):
        return [self.scaling] if self.scaling is not None else []

    def extra_repr(self):
        return f"in={self.in_features}, out={self.out_features}, recipe={self.bongard_recipe}"

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse=recurse)
        self._fp8_weight = None
        self._cached_weight_version = None
        return self

    def fp8_weight(self, is_first_microbatch):
        """Quantized weight (the block-scaled recipes with their column-wise copy, which their
        backward reads); cached across microbatches like TE."""
        if is_first_microbatch or self._fp8_weight is None:
            if _is_mx(self.recipe):
                q = _linear.quantize_weight_mx(self.weight, transpose=True)
            elif _is_nvfp4(self.recipe):
                q = _linear.quantize_weight_nvfp4(self.weight, transpose=True,
                                                  cache_dequant=is_first_microbatch is not None)
            else:
                q = _linear.quantize_weight(self.weight,
                                            scaler=self.scaling and self.scaling.weight)
            if is_first_microbatch is not None:
                self._fp8_weight = q
            return q
        return self._fp8_weight

    def _note_microbatch(self):
        version = self.weight._version
        first_microbatch = version != self._cached_weight_version
        self._cached_weight_version = version
        self.counts['weight_quantizations' if first_microbatch else 'cached_weights'] += 1
        return first_microbatch

    @torch.compiler.disable
    def geglu_forward(self, x, intermediate):
        """Training forward of a gate_up projection ([W_gate; W_up]) under 'nvfp4' with the
        gated GELU in the GEMM's epilogue: ``(H [..., I], amax partials of |H|)`` (rows
        padded and the weight cached as in :meth:`forward`; the partials, over the padded
        rows, whose H is zero, go to the down projection's ``x_partials``)."""
        flat = x.reshape(-1, x.shape[-1])
        first_microbatch = self._note_microbatch()
        flat, length, aligned = _pad_rows(flat)
        if flat.dtype != torch.bfloat16:
            flat = flat.to(torch.bfloat16)
        out, parts = _linear.GegluGateUpNvfp4Function.apply(flat, self.weight,
                                                            self.fp8_weight(first_microbatch),
                                                            int(intermediate))
        if aligned != length:
            out = out[:length]
        return out.reshape(*x.shape[:-1], out.shape[-1]), parts

    @torch.compiler.disable
    def forward(self, x, x_partials=None):
        """``x_partials`` (the 'nvfp4' recipe only, else ignored): amax partials of |x| that
        x's producer wrote (the gate/up GEMM's epilogue for H), so that x's quantizer needs
        no amax pass of its own."""
        if not self.training:
            return F.linear(x, self.weight)
        flat = x.reshape(-1, x.shape[-1])
        first_microbatch = self._note_microbatch()
        # Pad to a multiple of 32 rows (zeros leave the amax unchanged), slice after.
        flat, length, aligned = _pad_rows(flat)
        if flat.dtype != torch.bfloat16:
            flat = flat.to(torch.bfloat16)
        if _is_mx(self.recipe):
            out = _linear.Fp8LinearMxFunction.apply(flat, self.weight,
                                                    self.fp8_weight(first_microbatch))
        elif _is_nvfp4(self.recipe):
            out = _linear.Fp8LinearNvfp4Function.apply(flat, self.weight,
                                                       self.fp8_weight(first_microbatch),
                                                       x_partials)
        else:
            out = _linear.Fp8LinearFunction.apply(flat, self.weight, None,
                                                  self.fp8_weight(first_microbatch), self.scaling)
        if aligned != length:
            out = out[:length]
        return out.reshape(*x.shape[:-1], out.shape[-1])


class TEMLP(torch.nn.Module):
    """The HF gated MLP with its three projections as two FP8 GEMMs."""

    def __init__(self, mlp, recipe):
        super().__init__()
        if mlp.config.hidden_activation != 'gelu_pytorch_tanh' or mlp.dropout.p:
            raise ValueError('TE MLP requires tanh GELU and zero dropout')
        self.bongard_recipe = recipe
        self.intermediate_size = mlp.intermediate_size
        # Default: one stacked [gate; up] weight sharing one scale; the environment switch
        # keeps two projections (two scales), as in the reference.
        self.fused_gate_up = os.environ.get('BONGARD_TE_SPLIT_GATE_UP', '0') != '1'
        if not self.fused_gate_up and recipe == 'fp8_delayed':
            raise ValueError('delayed scaling needs the fused gate_up projection')
        if self.fused_gate_up:
            self.gate_up = TELinear([mlp.gate_proj, mlp.up_proj], recipe)
        else:
            self.gate_proj = TELinear([mlp.gate_proj], recipe)
            self.up_proj = TELinear([mlp.up_proj], recipe)
        self.down = TELinear([mlp.down_proj], recipe)
        self._split_cache = None

    def _gate_up_weight(self):
        if self.fused_gate_up:
            return self.gate_up.weight
        return torch.cat([self.gate_proj.weight, self.up_proj.weight], 0)

    def forward(self, x):
        if not self.training:
            if self.fused_gate_up:
                gate, up = self.gate_up(x).split(self.intermediate_size, dim=-1)
            else:
                gate, up = self.gate_proj(x), self.up_proj(x)
            return self.down(F.gelu(gate, approximate='tanh') * up)
        return self._fp8_forward(x)

    @torch.compiler.disable
    def _fp8_forward(self, x):
        if _is_nvfp4(self.down.recipe):
            # NVFP4: the projections' own forwards (pad to 32, weight cache, NVFP4 GEMMs);
            # the fused gate_up GEMM takes the gated GELU into its epilogue, the split
            # projections feed the elementwise one
            if self.fused_gate_up:
                h, h_partials = self.gate_up.geglu_forward(x, self.intermediate_size)
                return self.down(h, x_partials=h_partials)
            gu = torch.cat([self.gate_proj(x), self.up_proj(x)], -1)
            shape = gu.shape
            h, h_partials = _linear.GegluFunction.apply(gu.reshape(-1, shape[-1]).contiguous())
            return self.down(h.reshape(*shape[:-1], shape[-1] // 2), x_partials=h_partials)
        I = self.intermediate_size
        flat = x.reshape(-1, x.shape[-1])
        flat, length, aligned = _pad_rows(flat)
        if flat.dtype != torch.bfloat16:
            flat = flat.to(torch.bfloat16)
        down_first = self.down._note_microbatch()
        if (self.fused_gate_up and self.down.scaling is not None
                and self.gate_up.scaling is not None):
            first = self.gate_up._note_microbatch()
            return self._delayed_forward(x, flat, length, aligned,
                                         first or self.gate_up._fp8_weight is None,
                                         down_first or self.down._fp8_weight is None)
        down_q = self.down.fp8_weight(down_first)
        if _is_mx(self.down.recipe):
            return self._mx_forward(x, flat, length, aligned, down_q)
        if self.fused_gate_up:
            first = self.gate_up._note_microbatch()
            if first or self.gate_up._fp8_weight is None:
                gs = self.gate_up.scaling
                self.gate_up._fp8_weight = _linear.quantize_gate_up(
                    self.gate_up.weight, I, split_scales=False, scaler=gs and gs.weight)
            gu_q = self.gate_up._fp8_weight
            w_gu = self.gate_up.weight
        else:
            first_g = self.gate_proj._note_microbatch()
            first_u = self.up_proj._note_microbatch()
            if first_g or first_u or self._split_cache is None:
                self._split_cache = _linear.quantize_gate_up(
                    torch.cat([self.gate_proj.weight, self.up_proj.weight], 0), I,
                    split_scales=True)
            gu_q = self._split_cache
            w_gu = _SplitGateUp.apply(self.gate_proj.weight, self.up_proj.weight)
        scaling = None
        if self.fused_gate_up and self.gate_up.scaling is not None:
            scaling = (self.gate_up.scaling, self.down.scaling)
        out = _linear.Fp8GegluMlpFunction.apply(flat, w_gu, self.down.weight, gu_q, down_q, I,
                                                not self.fused_gate_up, scaling)
        if aligned != length:
            out = out[:length]
        return out.reshape(*x.shape[:-1], out.shape[-1])


    def _delayed_forward(self, x, flat, length, aligned, new_gu, new_down):
        """'fp8_delayed' with the fused gate_up: the weights' FP8 copies, re-quantized
        where a weight changed (both in one launch when both did), cached for the next
        microbatches, and the gated MLP on them."""
        I = self.intermediate_size
        gs, dsc = self.gate_up.scaling, self.down.scaling
        if new_gu and new_down:
            wq, dq = _scaling.quantize_many([
                (gs.weight, self.gate_up.weight.detach(), True, False),
                (dsc.weight, self.down.weight.detach(), True, False)])
            self.gate_up._fp8_weight = _linear._GateUp(wq.data, None, wq.meta.view(1, 4))
            self.down._fp8_weight = dq
        elif new_gu:
            self.gate_up._fp8_weight = _linear.quantize_gate_up(
                self.gate_up.weight, I, split_scales=False, scaler=gs.weight)
        elif new_down:
            self.down._fp8_weight = _linear.quantize_weight(self.down.weight, scaler=dsc.weight)
        out = _linear.Fp8GegluMlpFunction.apply(flat, self.gate_up.weight, self.down.weight,
                                                self.gate_up._fp8_weight,
                                                self.down._fp8_weight, I, False, (gs, dsc))
        if aligned != length:
            out = out[:length]
        return out.reshape(*x.shape[:-1], out.shape[-1])

    def _mx_forward(self, x, flat, length, aligned, down_q):
        """MXFP8: blocks along K never straddle gate and up rows, so the stacked weight's
        MX copy is the two projections' copies side by side (fused or split alike)."""
        I = self.intermediate_size
        if self.fused_gate_up:
            first = self.gate_up._note_microbatch()
            if first or self.gate_up._fp8_weight is None:
                self.gate_up._fp8_weight = _linear.quantize_weight_mx(self.gate_up.weight)
            gu_q = self.gate_up._fp8_weight
            w_gu = self.gate_up.weight
        else:
            first_g = self.gate_proj._note_microbatch()
            first_u = self.up_proj._note_microbatch()
            if first_g or first_u or self._split_cache is None:
                self._split_cache = _linear.quantize_weight_mx(
                    torch.cat([self.gate_proj.weight, self.up_proj.weight], 0))
            gu_q = self._split_cache
            w_gu = _SplitGateUp.apply(self.gate_proj.weight, self.up_proj.weight)
        out = _linear.Fp8GegluMlpMxFunction.apply(flat, w_gu, self.down.weight, gu_q, down_q, I)
        if aligned != length:
            out = out[:length]
        return out.reshape(*x.shape[:-1], out.shape[-1])


class _SplitGateUp(torch.autograd.Function):
    """Stacks separate gate/up weights for the fused kernel; splits the gradient back."""

    @staticmethod
    def forward(ctx, wg, wu):
        ctx.rows = wg.shape[0]
        return torch.cat([wg, wu], 0)

    @staticmethod
    def backward(ctx, d):
        return d[:ctx.rows], d[ctx.rows:]


def _text_layers(model):
    """Every encoder and decoder text layer, in model order."""
    backbone = model.backbone
    yield from backbone.encoder.text_model.layers
    yield from backbone.decoder.layers


def _keep_or_replace(current, cls, recipe, build, message):
    """Return ``current`` if already converted with ``recipe``; else a new module."""
    if isinstance(current, cls):
        if current.bongard_recipe != recipe:
            raise ValueError(message)
        return current
    return build()


def enable_te_linear(model, *, mlp=None, attention=None):
    """Convert the MLP and/or the q/k/v/o projections of every text layer.

    Returns ``{'mlp': layers converted, 'attention': projections converted}`` (keys only
    for the kinds requested). Sets ``model.pack_multiple = 32``: the packed forward then
    hands every projection a row count that needs no padding.
    """
    if not (mlp or attention) or model.device.type != 'cuda':
        raise ValueError('TE projections require CUDA and at least one recipe')
    if any(r is not None and r not in RECIPES for r in (mlp, attention)):
        raise ValueError(f'TE recipe must be one of {RECIPES}')
    model.pack_multiple = 32
    counts = Counter()
    for layer in _text_layers(model):
        if mlp:
            layer.mlp = _keep_or_replace(
                layer.mlp, TEMLP, mlp, lambda: TEMLP(layer.mlp, mlp),
                'An existing TE MLP must retain its recipe')
            counts['mlp'] += 1
        if not attention:
            continue
        attn = layer.self_attn
        for proj in ATTENTION_PROJECTIONS:
            current = getattr(attn, proj)
            setattr(attn, proj, _keep_or_replace(
                current, TELinear, attention, lambda: TELinear([current], attention),
                'An existing TE projection must retain its recipe'))
            counts['attention'] += 1
    return dict(counts)


def present(backbone):
    """True if any module of ``backbone`` is one of this file's FP8 projections."""
    for module in backbone.modules():
        if _te_linear(module) or _te_mlp(module):
            return True
    return False


def _pop_empty_extra_state(state, key):
    if state.pop(key).numel() != 0:
        raise ValueError('TE export requires stateless quantization scaling')


def _mlp_export(prefix, module, state):
    """HF keys for one TEMLP: gate_proj/up_proj/down_proj weights, no extra state."""
    own = ['gate_up'] if module.fused_gate_up else ['gate_proj', 'up_proj']
    for sub in own + ['down']:
        _pop_empty_extra_state(state, f'{prefix}{sub}._extra_state')
    if module.fused_gate_up:
        stacked = state.pop(f'{prefix}gate_up.weight')
        halves = stacked.split(module.intermediate_size)
        state[f'{prefix}gate_proj.weight'], state[f'{prefix}up_proj.weight'] = halves
    state[f'{prefix}down_proj.weight'] = state.pop(f'{prefix}down.weight')


def restore_hf_layout(backbone, state):
    """Rewrite ``state`` (a backbone state dict) to the Hugging Face module keys.

    TEMLP weights go back to gate_proj/up_proj/down_proj; attention projections keep
    their ``weight`` key. Every ``_extra_state`` entry is removed and must be empty:
    exporting a module with stateful (delayed) scaling raises ValueError.
    """
    for name, module in backbone.named_modules():
        if _te_mlp(module):
            _mlp_export(name + '.', module, state)
        elif _te_linear(module) and name.rpartition('.')[2] in ATTENTION_PROJECTIONS:
            _pop_empty_extra_state(state, name + '._extra_state')
    return state
