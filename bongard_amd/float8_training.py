"""FP8 text GEMMs preserving the model's chosen parameter storage dtype (MI355X).

Drop-in for bongard/float8_training.py (torchao Float8Linear path): same ``RECIPES``,
``enable_float8(model, recipe, *, emulate=False) -> int`` with the same module filter and
errors, and ``TrainingLinear`` with BF16 ``F.linear`` in eval. In training the linear runs
on the gfx950 FP8 kernels with torchao 0.17.0's recipe semantics:
  * ``tensorwise`` (bongard_amd.linear.Fp8LinearFunction): dynamic per-tensor e4m3 for X
    and W, e5m2 for grad_out;
  * ``rowwise`` / ``rowwise_with_gw_hp`` (bongard_amd.linear.Fp8LinearAxiswiseFunction):
    axiswise e4m3 casts of X, W and grad_out with power-of-2 scales; the second keeps the
    weight gradient in bf16 and quantizes W tensorwise for the input gradient.

Difference from the reference, by design: ``emulate=True`` skips the device check so
modules can be converted (and their state dicts inspected) on a CPU, but a training
forward still needs the gfx950 device: the product path has no CPU emulation.
"""

from dataclasses import dataclass, replace

import torch
from torch.nn import functional as F

from . import custom_ops as _custom_ops
from . import linear as _linear

RECIPES = ("tensorwise", "rowwise", "rowwise_with_gw_hp")
_PREFIXES = ("backbone.encoder.text_model.layers.", "backbone.decoder.layers.")


@dataclass(frozen=True)
class Float8LinearConfig:
    """The fields of torchao's Float8LinearConfig that this path honours."""

    recipe: str = "tensorwise"
    emulate: bool = False
    pad_inner_dim: bool = False

    @classmethod
    def from_recipe_name(cls, recipe):
        if recipe not in RECIPES:
            raise ValueError(f"fp8 must be one of {RECIPES}")
        return cls(recipe=recipe)


def _is_gfx950(device):
    if device.type != "cuda" or not torch.cuda.is_available():
        return False
    return torch.cuda.get_device_properties(device).gcnArchName.startswith("gfx950")


class Float8Linear(torch.nn.Linear):
    """nn.Linear whose training forward/backward run in FP8 on gfx950.

    Parameters are the original ``weight`` / ``bias`` (shared with the converted module),
    so the state dict is unchanged and no scale buffers exist (tensorwise scaling is
    recomputed from the data on every call).
    """

    config: Float8LinearConfig

    @classmethod
    def from_float(cls, mod, config):
        with torch.device("meta"):
            new = cls(mod.in_features, mod.out_features, bias=False)
        new.weight = mod.weight
        new.bias = mod.bias
        new.config = config
        return new

    # Under the reference's regional compile (bongard/model.py:249-281) this forward is
    # traced: the FP8 linear is then one custom op (bongard_amd.custom_ops) in the compiled
    # graph; eager calls take the autograd function directly (less dispatch overhead).
    # Both run the same kernels, so compiled and eager results are bit-identical.
    def forward(self, inputs):
        if inputs.device.type != "cuda":
            raise RuntimeError("FP8 training forward needs the MI355X device (no CPU emulation)")
        shape = inputs.shape
        flat = inputs.reshape(-1, shape[-1])
        if flat.dtype != torch.bfloat16:
            flat = flat.to(torch.bfloat16)
        length = flat.shape[0]
        # pad_inner_dim: the wgrad GEMM reduces over tokens, so keep them a multiple of 16
        aligned = (length + 15) // 16 * 16
        if aligned != length:
            flat = F.pad(flat, (0, 0, 0, aligned - length))
        weight = self.weight if self.weight.dtype == torch.bfloat16 else self.weight.to(torch.bfloat16)
        bias = None if self.bias is None else self.bias.to(torch.bfloat16)
        if torch.compiler.is_compiling():
            out = _custom_ops.fp8_linear(flat, weight, bias, self.config.recipe)
        elif self.config.recipe == "tensorwise":
            out = _linear.Fp8LinearFunction.apply(flat, weight, bias, None)
        else:
            out = _linear.Fp8LinearAxiswiseFunction.apply(flat, weight, bias, self.config.recipe)
        if aligned != length:
            out = out[:length]
        return out.reshape(*shape[:-1], out.shape[-1])

    def extra_repr(self):
        return f"{super().extra_repr()}, recipe={self.config.recipe}"


class TrainingLinear(Float8Linear):
    """Float8Linear whose eval forward is the plain BF16 linear (FP8 only while training)."""

    def forward(self, inputs):
        if self.training:
            return super().forward(inputs)
        return F.linear(inputs, self.weight, self.bias)


def convert_to_float8_training(model, *, config, module_filter_fn):
    """Swap every selected nn.Linear for a Float8Linear sharing its parameters."""
    for parent_name, parent in list(model.named_modules()):
        for child_name, child in list(parent.named_children()):
            name = f"{parent_name}.{child_name}" if parent_name else child_name
            if module_filter_fn(child, name):
                setattr(parent, child_name, Float8Linear.from_float(child, config))
    return model


def enable_float8(model, recipe, *, emulate=False):
    """Convert the eligible text-layer linears to TrainingLinear; returns how many.

    Eligible: an nn.Linear under an encoder or decoder text layer, trainable, with in and
    out features divisible by 16. ``emulate`` only lifts the device check (see module doc).
    """
    if recipe not in RECIPES:
        raise ValueError(f"fp8 must be one of {RECIPES}")
    device = next(model.parameters()).device if not hasattr(model, "device") else model.device
    if not emulate and not _is_gfx950(device):
        raise ValueError("FP8 training requires an MI355X (gfx950) GPU")
    # Token counts vary per request, so the wgrad GEMM's reduction dim gets padded.
    config = replace(Float8LinearConfig.from_recipe_name(recipe), emulate=emulate,
                     pad_inner_dim=True)

    def eligible(module, name):
        if isinstance(module, Float8Linear):
            if module.config != config:
                raise ValueError('An already converted model must retain its FP8 recipe')
            return False
        if not isinstance(module, torch.nn.Linear) or not name.startswith(_PREFIXES):
            return False
        dims_ok = module.in_features % 16 == 0 and module.out_features % 16 == 0
        return dims_ok and module.weight.requires_grad

    convert_to_float8_training(model, config=config, module_filter_fn=eligible)
    converted = [m for m in model.modules() if isinstance(m, Float8Linear)]
    if not converted:
        raise ValueError("FP8 found no eligible trainable text Linear modules")
    for module in converted:
        module.__class__ = TrainingLinear
    return len(converted)
