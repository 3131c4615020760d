"""CPU tests of how delayed scaling recognises a checkpoint replay
(bongard_amd.scaling.checkpoint_region). The reference checkpoints every text layer with
non-reentrant torch.utils.checkpoint (bongard/model.py:124-132, 234-247), so each FP8
forward runs twice per step; the replay must be told apart from a new step even when
other saved-tensor hooks (activation offload, say) sit inside the checkpointed region."""

import pytest
import torch
from torch.utils.checkpoint import checkpoint

from bongard_amd import scaling


def _identity_hooks():
    return torch.autograd.graph.saved_tensors_hooks(lambda t: t, lambda t: t)


def test_outside_any_region():
    assert scaling.checkpoint_region() == (None, False)
    with _identity_hooks():
        assert scaling.checkpoint_region() == (None, False)


@pytest.mark.parametrize("nested", ["none", "identity", "save_on_cpu"])
def test_replay_seen_through_hooks_nested_inside_the_region(nested):
    seen = []

    def inner_hooks():
        if nested == "identity":
            return _identity_hooks()
        if nested == "save_on_cpu":
            return torch.autograd.graph.save_on_cpu()
        return _NullCtx()

    def layer(x):
        seen.append(("outer", scaling.checkpoint_region()))
        with inner_hooks():
            seen.append(("inner", scaling.checkpoint_region()))
            y = x * x            # saved through the nested hooks
        return y.sin()           # saved through checkpoint's hook: backward replays layer

    x = torch.randn(8, requires_grad=True)
    out = checkpoint(layer, x, use_reentrant=False)
    assert [s for s, _ in seen] == ["outer", "inner"]
    frame = seen[0][1][0]
    assert frame is not None
    assert seen[0][1] == (frame, False) and seen[1][1] == (frame, False)
    out.sum().backward()
    assert len(seen) == 4, "the backward replays the region once"
    assert seen[2][1] == (frame, True) and seen[3][1] == (frame, True)
    xr = x.detach().clone().requires_grad_(True)
    (xr * xr).sin().sum().backward()
    assert torch.allclose(x.grad, xr.grad)


class _NullCtx:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def test_hook_stack_restored_after_reading():
    pack = lambda t: t  # noqa: E731
    unpack = lambda t: t  # noqa: E731
    with torch.autograd.graph.saved_tensors_hooks(pack, unpack):
        with _identity_hooks():
            top = torch._C._autograd._top_saved_tensors_default_hooks(False)
            scaling.checkpoint_region()
            assert torch._C._autograd._top_saved_tensors_default_hooks(False) == top
        assert torch._C._autograd._top_saved_tensors_default_hooks(False) == (pack, unpack)
    assert torch._C._autograd._top_saved_tensors_default_hooks(False) is None


def test_nested_regions_report_the_innermost():
    seen = []

    def inner(x):
        seen.append(scaling.checkpoint_region())
        return (x * x).sin()

    def outer(x):
        seen.append(scaling.checkpoint_region())
        return checkpoint(inner, x.cos(), use_reentrant=False).exp()

    x = torch.randn(4, requires_grad=True)
    checkpoint(outer, x, use_reentrant=False).sum().backward()
    assert seen[0][0] is not None and seen[1][0] is not None
    assert seen[0][0] is not seen[1][0]
    assert seen[0][1] is False and seen[1][1] is False
    replays = [s for s in seen[2:] if s[1]]
    assert replays and all(f in (seen[0][0], seen[1][0]) for f, _ in replays)


def test_reentrant_replay_of_a_forward_role_raises():
    """Reentrant checkpointing re-runs the forward inside backward with no hook to tell
    it from a new step: a forward role refuses, a gradient role (quantized in backward by
    design) does not."""
    calls = []

    def layer(x):
        calls.append(len(calls))
        if len(calls) > 1:       # the replay, inside the backward pass
            with pytest.raises(RuntimeError, match="use_reentrant=False"):
                scaling.checkpoint_region()
            assert scaling.checkpoint_region(forward_role=False) == (None, False)
        else:
            assert scaling.checkpoint_region() == (None, False)
        return (x * x).sin()

    x = torch.randn(4, requires_grad=True)
    checkpoint(layer, x, use_reentrant=True).sum().backward()
    assert len(calls) == 2


def test_gradient_roles_inside_backward_are_not_replays():
    seen = []

    class F(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            return x * 2

        @staticmethod
        def backward(ctx, g):
            seen.append(scaling.checkpoint_region(forward_role=False))
            return g * 2

    x = torch.randn(3, requires_grad=True)
    F.apply(x).sum().backward()
    assert seen == [(None, False)]
