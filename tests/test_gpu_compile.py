"""The compile-visible FP8 ops (bongard_amd.custom_ops) under torch.compile's default
Inductor backend.

The reference compiles each text layer (bongard/model.py:249-283) with its torchao
Float8Linear inside. Blocks of two FP8 linears are compiled with ``fullgraph=True`` (any
graph break fails the compile) for each torchao recipe: a block whose other ops round
identically compiled and eager must give the eager outputs and gradients bit for bit, and a
layer-like block (RMSNorm -> FP8 up -> GELU -> FP8 down) its eager output bit for bit (its
gradients within a bf16 ulp: Inductor fuses the norm's backward in fp32). The gated-MLP op
likewise. torch.library.opcheck checks the ops' schemas, fake implementations and autograd
registrations.
"""

import pytest
import torch
from torch import nn
from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2RMSNorm

from bongard_amd import custom_ops, float8_training, linear

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


_OPCHECK = ("test_schema", "test_autograd_registration", "test_faketensor")


@pytest.mark.parametrize("need_dx,need_dw", [(True, True), (False, False), (True, False),
                                             (False, True)])
def test_opcheck_linear_and_mlp(gpu, need_dx, need_dw):
    """Every gradient combination: without gradients the tensorwise forward quantizes x and
    W in one launch, and its outputs must still not alias one another (test_schema)."""
    g = torch.Generator(device=gpu).manual_seed(1)
    x0 = torch.randn(64, 128, device=gpu, generator=g).to(torch.bfloat16)
    w0 = (torch.randn(96, 128, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    x = x0.clone().requires_grad_(need_dx)
    w = w0.clone().requires_grad_(need_dw)
    for recipe in ("tensorwise", "rowwise", "rowwise_with_gw_hp"):
        torch.library.opcheck(torch.ops.bongard_fp8.linear.default,
                              (x, w, None, recipe, need_dx, need_dw), test_utils=_OPCHECK)
    w_gu = (torch.randn(256, 128, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    w_d = (torch.randn(128, 128, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    for split in (False, True):
        a = w_gu.clone().requires_grad_(need_dw)
        b = w_d.clone().requires_grad_(need_dw)
        torch.library.opcheck(torch.ops.bongard_fp8.geglu_mlp.default,
                              (x, a, b, 128, split, need_dx, need_dw, need_dw),
                              test_utils=_OPCHECK)


@pytest.mark.parametrize("recipe", ["tensorwise", "rowwise", "rowwise_with_gw_hp"])
def test_float8_linear_compiled_without_grad_matches_eager(gpu, recipe):
    """An eval-style compiled region (no_grad, or frozen weight and input) runs the op's
    no-gradient form: fullgraph, and bit-identical to the eager autograd function."""
    torch._dynamo.reset()
    block = _ExactBlock(256, 512, recipe).to(gpu).train()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4, 64, 256, generator=g).to(torch.bfloat16).to(gpu)
    with torch.no_grad():
        ref = block(x)
        got = torch.compile(block, fullgraph=True)(x)
    torch.cuda.synchronize()
    assert torch.equal(_bits(ref), _bits(got)), recipe
    for p in block.parameters():          # frozen weights, input without grad
        p.requires_grad_(False)
    torch._dynamo.reset()
    got = torch.compile(block, fullgraph=True)(x)
    assert torch.equal(_bits(ref), _bits(got)), f"{recipe} (frozen)"


def _fp8_linear(i, o, std, recipe):
    cfg = float8_training.Float8LinearConfig(recipe=recipe, pad_inner_dim=True)
    base = nn.Linear(i, o, bias=False).to(torch.bfloat16)
    with torch.no_grad():
        base.weight.normal_(std=std)
    m = float8_training.Float8Linear.from_float(base, cfg)
    m.__class__ = float8_training.TrainingLinear
    return m


class _ExactBlock(nn.Module):
    """Two FP8 linears joined by ops whose compiled form rounds exactly as eager does (a
    power-of-two scaling and a residual add of two bf16 values), so any difference between
    the compiled and eager runs would come from the FP8 ops."""

    def __init__(self, hidden, inter, recipe):
        super().__init__()
        torch.manual_seed(7)
        self.up = _fp8_linear(hidden, inter, 0.05, recipe)
        self.down = _fp8_linear(inter, hidden, 0.03, recipe)

    def forward(self, x):
        return self.down(self.up(x) * 2.0) + x


class _LayerBlock(_ExactBlock):
    """A layer-like region: RMSNorm -> FP8 up -> GELU -> FP8 down, residual."""

    def __init__(self, hidden, inter, recipe):
        super().__init__(hidden, inter, recipe)
        self.norm = T5Gemma2RMSNorm(hidden, eps=1e-6).to(torch.bfloat16)
        with torch.no_grad():
            self.norm.weight.normal_(std=0.1)

    def forward(self, x):
        return self.down(nn.functional.gelu(self.up(self.norm(x)), approximate="tanh")) + x


def _run(block_cls, recipe, compiled, x, dy, dev):
    block = block_cls(256, 512, recipe).to(dev).train()
    fn = torch.compile(block, fullgraph=True) if compiled else block
    xg = x.clone().requires_grad_(True)
    y = fn(xg)
    y.backward(dy)
    torch.cuda.synchronize()
    return [y.detach(), xg.grad] + [p.grad for p in block.parameters()]


@pytest.mark.parametrize("recipe", ["tensorwise", "rowwise", "rowwise_with_gw_hp"])
def test_float8_linear_in_a_fullgraph_inductor_region(gpu, recipe):
    """fullgraph=True: the FP8 linears trace without a graph break. The exact block's
    outputs and gradients equal eager bit for bit; in the layer-like block Inductor fuses
    the norm's and GELU's own arithmetic in fp32 (a bf16 rounding fewer than eager), so its
    forward output is still bit-identical and its gradients agree to within a bf16 ulp."""
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 64, 256, generator=g).to(torch.bfloat16).to(gpu)
    dy = (torch.randn(4, 64, 256, generator=g) * 1e-2).to(torch.bfloat16).to(gpu)
    eager = _run(_ExactBlock, recipe, False, x, dy, gpu)
    comp = _run(_ExactBlock, recipe, True, x, dy, gpu)
    for i, (a, b) in enumerate(zip(eager, comp)):
        assert torch.equal(_bits(a), _bits(b)), f"{recipe}: tensor {i} differs from eager"
    torch._dynamo.reset()
    eager = _run(_LayerBlock, recipe, False, x, dy, gpu)
    comp = _run(_LayerBlock, recipe, True, x, dy, gpu)
    assert torch.equal(_bits(eager[0]), _bits(comp[0])), f"{recipe}: layer output"
    for i, (a, b) in enumerate(zip(eager[1:], comp[1:])):
        ulp = torch.finfo(torch.bfloat16).eps * a.float().abs().max()
        diff = (a.float() - b.float()).abs().max()
        assert diff <= 2 * ulp, f"{recipe}: layer gradient {i} off by {diff} (ulp {ulp})"


def test_geglu_mlp_op_in_a_fullgraph_inductor_region(gpu):
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(3)
    M, K, I = 256, 256, 512
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(gpu)
    w_gu = (torch.randn(2 * I, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    w_d = (torch.randn(K, I, generator=g) * 0.014).to(torch.bfloat16).to(gpu)
    dy = (torch.randn(M, K, generator=g) * 1e-3).to(torch.bfloat16).to(gpu)

    def eager(t, a, b):
        return linear.Fp8GegluMlpFunction.apply(t * 2.0, a, b, None, None, I, False) + t

    @torch.compile(fullgraph=True)
    def compiled(t, a, b):
        return custom_ops.fp8_geglu_mlp(t * 2.0, a, b, I) + t

    results = []
    for fn in (eager, compiled):
        xg = x.clone().requires_grad_(True)
        a = w_gu.clone().requires_grad_(True)
        b = w_d.clone().requires_grad_(True)
        y = fn(xg, a, b)
        y.backward(dy)
        torch.cuda.synchronize()
        results.append((y.detach(), xg.grad, a.grad, b.grad))
    for i, (u, v) in enumerate(zip(*results)):
        assert torch.equal(_bits(u), _bits(v)), f"MLP tensor {i} differs from eager"
    with torch.no_grad():   # the inference form of the op (no saved tensors)
        assert torch.equal(_bits(compiled(x, w_gu, w_d)), _bits(results[0][0]))
