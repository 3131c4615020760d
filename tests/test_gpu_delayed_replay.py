"""'fp8_delayed' under activation checkpointing and across a save / resume.

The reference trains with non-reentrant activation checkpointing of every text layer
(bongard/model.py:124-132, 234-247), which replays each layer's forward during backward. A
delayed-scaling module must quantize the replay with the scales of the original forward
and leave its amax histories alone; and a run resumed from a state dict must continue with
the scales the uninterrupted run would use. Both are checked bit for bit: outputs,
gradients and the saved histories (``_extra_state``), over three training steps.
"""

import copy
import types

import pytest
import torch
from torch.utils.checkpoint import checkpoint
from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2MLP, T5Gemma2RMSNorm

from bongard_amd import fused_mlp, te_linear

pytestmark = pytest.mark.gpu

HIDDEN, INTER, ROWS = 256, 512, 256


def _build(kind, dev):
    cfg = types.SimpleNamespace(hidden_size=HIDDEN, intermediate_size=INTER,
                                hidden_activation="gelu_pytorch_tanh", dropout_rate=0.0)
    torch.manual_seed(3)
    mlp = T5Gemma2MLP(cfg)
    with torch.no_grad():
        mlp.gate_proj.weight.normal_(std=0.02)
        mlp.up_proj.weight.normal_(std=0.02)
        mlp.down_proj.weight.normal_(std=0.014)
    mlp = mlp.to(torch.bfloat16)
    if kind == "temlp":
        return te_linear.TEMLP(mlp, "fp8_delayed").to(dev).train()
    norm = T5Gemma2RMSNorm(HIDDEN, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.normal_(std=0.1)
    return fused_mlp.FusedMLP(mlp, norm, "fp8_delayed").to(dev).train()


def _inputs(steps):
    g = torch.Generator().manual_seed(11)
    return [((torch.randn(ROWS, HIDDEN, generator=g) * (1 + s)).to(torch.bfloat16),
             (torch.randn(ROWS, HIDDEN, generator=g) * 1e-3 * (1 + s)).to(torch.bfloat16))
            for s in range(steps)]


def _step(module, x, dy, ckpt):
    """One training step: new weight versions (as an optimizer step makes), forward,
    backward. Returns the output, the input gradient and the weight gradients."""
    with torch.no_grad():
        for p in module.parameters():
            p.mul_(1.0)
    xg = x.clone().requires_grad_(True)
    if ckpt:
        y = checkpoint(lambda t: module(t) * 1.0, xg, use_reentrant=False)
    else:
        y = module(xg) * 1.0
    y.backward(dy)
    grads = [p.grad.clone() for p in module.parameters()]
    for p in module.parameters():
        p.grad = None
    return [y.detach(), xg.grad] + grads


def _same(a, b, what):
    assert len(a) == len(b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert u.dtype == v.dtype and u.shape == v.shape, what
        assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                           v.view(torch.int16) if v.dtype == torch.bfloat16 else v), \
            f"{what}: tensor {i} differs"


def _extra(module):
    return {k: v.clone() for k, v in module.state_dict().items() if k.endswith("_extra_state")}


@pytest.mark.parametrize("kind", ["temlp", "fused"])
def test_delayed_scaling_under_activation_checkpointing(gpu, kind):
    plain, ckpt = _build(kind, gpu), _build(kind, gpu)
    for step, (x, dy) in enumerate(_inputs(3)):
        a = _step(plain, x.to(gpu), dy.to(gpu), False)
        b = _step(ckpt, x.to(gpu), dy.to(gpu), True)
        torch.cuda.synchronize()
        _same(a, b, f"{kind} step {step}: checkpointed vs plain")
        ea, eb = _extra(plain), _extra(ckpt)
        assert ea.keys() == eb.keys()
        for k in ea:
            assert torch.equal(ea[k], eb[k]), f"{kind} step {step}: {k} differs"


@pytest.mark.parametrize("kind", ["temlp", "fused"])
def test_delayed_scaling_resumes_from_state_dict(gpu, kind):
    data = _inputs(4)
    straight = _build(kind, gpu)
    ref = [_step(straight, x.to(gpu), dy.to(gpu), False) for x, dy in data]
    saved = _build(kind, gpu)
    for x, dy in data[:3]:
        _step(saved, x.to(gpu), dy.to(gpu), False)
    state = copy.deepcopy(saved.state_dict())
    after_save = _step(saved, data[3][0].to(gpu), data[3][1].to(gpu), False)
    resumed = _build(kind, gpu)
    resumed.load_state_dict(state)
    got = _step(resumed, data[3][0].to(gpu), data[3][1].to(gpu), False)
    torch.cuda.synchronize()
    _same(after_save, ref[3], f"{kind}: step 3 after saving vs uninterrupted")
    _same(got, ref[3], f"{kind}: step 3 resumed vs uninterrupted")
    for k, v in _extra(straight).items():
        assert torch.equal(_extra(resumed)[k], v), f"{kind}: {k} after the resumed step"
