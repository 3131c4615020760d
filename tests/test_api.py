"""CPU tests of the drop-in module API (no GPU: surgery, state dicts, export, eval paths).

Mirrors the reference's contract: bongard/float8_training.py:27-65,
bongard/te_linear.py:41-161, bongard/fused_mlp.py:21-124 and the export call at
bongard/model.py:532-539.
"""

import types

import pytest
import torch
from torch import nn
from transformers.models.t5gemma2.modeling_t5gemma2 import T5Gemma2MLP, T5Gemma2RMSNorm

from bongard_amd import float8_training, fused_mlp, te_linear

H, I = 64, 128


def _mlp(seed):
    cfg = types.SimpleNamespace(hidden_size=H, intermediate_size=I,
                                hidden_activation="gelu_pytorch_tanh", dropout_rate=0.0)
    torch.manual_seed(seed)
    m = T5Gemma2MLP(cfg).to(torch.bfloat16)
    for p in m.parameters():
        nn.init.normal_(p, std=0.05)
    return m


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(H, 64, bias=False)
        self.k_proj = nn.Linear(H, 32, bias=False)
        self.v_proj = nn.Linear(H, 32, bias=False)
        self.o_proj = nn.Linear(64, H, bias=False)


class _Layer(nn.Module):
    def __init__(self, seed):
        super().__init__()
        self.self_attn = _Attn().to(torch.bfloat16)
        self.mlp = _mlp(seed)
        self.pre_feedforward_layernorm = T5Gemma2RMSNorm(H).to(torch.bfloat16)
        with torch.no_grad():
            self.pre_feedforward_layernorm.weight.normal_(std=0.1)


class _Model(nn.Module):
    """The module tree the reference's enable_* functions walk."""

    def __init__(self, fake_device="cuda"):
        super().__init__()
        self.backbone = nn.Module()
        self.backbone.encoder = nn.Module()
        self.backbone.encoder.text_model = nn.Module()
        self.backbone.encoder.text_model.layers = nn.ModuleList([_Layer(1), _Layer(2)])
        self.backbone.decoder = nn.Module()
        self.backbone.decoder.layers = nn.ModuleList([_Layer(3)])
        self.head = nn.Linear(H, 16)
        self._fake_device = torch.device(fake_device)

    @property
    def device(self):
        return self._fake_device


# ---- te_linear ------------------------------------------------------------------------
def test_telinear_state_dict_and_eval():
    a, b = nn.Linear(H, 32, bias=False), nn.Linear(H, 48, bias=False)
    t = te_linear.TELinear([a, b], "fp8")
    assert t.splits == [32, 48] and t.bongard_recipe == "fp8"
    assert isinstance(t.recipe, te_linear.Float8CurrentScaling)
    sd = t.state_dict()
    assert set(sd) == {"weight", "_extra_state"}
    assert sd["_extra_state"].numel() == 0
    assert torch.equal(sd["weight"], torch.cat([a.weight, b.weight]).to(torch.bfloat16))
    t.eval()
    x = torch.randn(5, H).to(torch.bfloat16)
    assert torch.equal(t(x), nn.functional.linear(x, t.weight))
    assert t.counts == {}
    t2 = te_linear.TELinear([a, b], "fp8")
    t2.load_state_dict(sd)
    assert torch.equal(t2.weight, t.weight)


def test_telinear_rejects_bias_and_builds_block_recipes():
    with pytest.raises(ValueError, match="bias-free"):
        te_linear.TELinear([nn.Linear(H, 16)], "fp8")
    with pytest.raises(ValueError, match="TE recipe must be one of"):
        te_linear.TELinear([nn.Linear(H, 16, bias=False)], "fp16")
    t = te_linear.TELinear([nn.Linear(H, 16, bias=False)], "mxfp8")
    assert t.recipe.fp8_format == "E4M3" and t.state_dict()["_extra_state"].numel() == 0
    # NVFP4 is stateless too: an empty _extra_state, so export works as for 'fp8'
    t = te_linear.TELinear([nn.Linear(H, 16, bias=False)], "nvfp4")
    assert t.recipe.fp4_format == "E2M1" and t.recipe.block_size == 16
    assert t.state_dict()["_extra_state"].numel() == 0


def test_temlp_eval_matches_hf_mlp():
    mlp = _mlp(5)
    ref = mlp
    x = torch.randn(3, 7, H).to(torch.bfloat16)
    want = ref(x)
    t = te_linear.TEMLP(mlp, "fp8").eval()
    assert t.fused_gate_up and t.intermediate_size == I
    got = t(x)
    assert torch.allclose(got.float(), want.float(), rtol=2e-2, atol=2e-3)


def test_temlp_split_env(monkeypatch):
    monkeypatch.setenv("BONGARD_TE_SPLIT_GATE_UP", "1")
    t = te_linear.TEMLP(_mlp(6), "fp8")
    assert not t.fused_gate_up and hasattr(t, "gate_proj") and hasattr(t, "up_proj")
    assert set(t.state_dict()) == {"gate_proj.weight", "gate_proj._extra_state",
                                   "up_proj.weight", "up_proj._extra_state",
                                   "down.weight", "down._extra_state"}


def test_temlp_requires_tanh_gelu():
    m = _mlp(7)
    m.config = types.SimpleNamespace(hidden_activation="gelu")
    with pytest.raises(ValueError, match="tanh GELU"):
        te_linear.TEMLP(m, "fp8")


def test_enable_te_linear_surgery_and_export_round_trip():
    model = _Model()
    hf = {k: v.clone() for k, v in model.backbone.state_dict().items()}
    counts = te_linear.enable_te_linear(model, mlp="fp8", attention="fp8")
    assert counts == {"mlp": 3, "attention": 12}
    assert model.pack_multiple == 32
    assert te_linear.present(model.backbone)
    # idempotent with the same recipe
    assert te_linear.enable_te_linear(model, mlp="fp8", attention="fp8") == counts
    layer = model.backbone.encoder.text_model.layers[0]
    assert isinstance(layer.mlp, te_linear.TEMLP)
    assert isinstance(layer.self_attn.q_proj, te_linear.TELinear)
    restored = te_linear.restore_hf_layout(model.backbone, model.backbone.state_dict())
    assert set(restored) == set(hf)
    for k in hf:
        assert torch.equal(restored[k], hf[k]), k
    # hf_state_dict covers te_linear modules too
    assert set(fused_mlp.hf_state_dict(model.backbone)) == set(hf)


def test_enable_te_linear_errors():
    with pytest.raises(ValueError, match="CUDA"):
        te_linear.enable_te_linear(_Model("cpu"), mlp="fp8")
    with pytest.raises(ValueError, match="at least one recipe"):
        te_linear.enable_te_linear(_Model())
    with pytest.raises(ValueError, match="must be one of"):
        te_linear.enable_te_linear(_Model(), mlp="fp4")
    model = _Model()
    te_linear.enable_te_linear(model, attention="fp8")
    model.backbone.decoder.layers[0].self_attn.q_proj.bongard_recipe = "mxfp8"
    with pytest.raises(ValueError, match="retain its recipe"):
        te_linear.enable_te_linear(model, attention="fp8")


def test_export_rejects_stateful_extra_state():
    model = _Model()
    te_linear.enable_te_linear(model, mlp="fp8")
    state = model.backbone.state_dict()
    key = next(k for k in state if k.endswith("down._extra_state"))
    state[key] = torch.ones(3, dtype=torch.uint8)
    with pytest.raises(ValueError, match="stateless"):
        te_linear.restore_hf_layout(model.backbone, state)


# ---- fused_mlp --------------------------------------------------------------------------
def test_fused_mlp_layout_eval_and_export():
    model = _Model()
    hf = {k: v.clone() for k, v in model.backbone.state_dict().items()}
    layer = model.backbone.encoder.text_model.layers[1]
    x = torch.randn(4, H).to(torch.bfloat16)
    want = layer.mlp(layer.pre_feedforward_layernorm(x))
    assert fused_mlp.enable_fused_mlp(model, "fp8") == 3
    assert fused_mlp.enable_fused_mlp(model, "fp8") == 3
    f = layer.mlp
    assert isinstance(layer.pre_feedforward_layernorm, nn.Identity)
    assert set(f.state_dict()) == {"layer_norm_weight", "fc1_weight", "fc2_weight", "_extra_state"}
    assert f.fc1_weight.shape == (2 * I, H) and f.fc2_weight.shape == (H, I)
    f.eval()
    assert torch.equal(f(x), want)
    # HF views share storage with the registered parameters
    assert f._hf_mlp.gate_proj.weight.data_ptr() == f.fc1_weight.data_ptr()
    assert not any(n.startswith("_hf") for n, _ in f.named_modules())
    exported = fused_mlp.hf_state_dict(model.backbone)
    assert set(exported) == set(hf)
    for k in hf:
        assert torch.equal(exported[k], hf[k]), k
    with pytest.raises(ValueError, match="CUDA"):
        fused_mlp.enable_fused_mlp(_Model("cpu"), "fp8")
    assert fused_mlp.hf_state_dict(_Model().backbone) is None


def test_fused_mlp_apply_refreshes_views():
    model = _Model()
    fused_mlp.enable_fused_mlp(model, "fp8")
    f = model.backbone.decoder.layers[0].mlp
    f.float()
    assert f._hf_mlp.up_proj.weight.dtype == torch.float32
    assert f._hf_mlp.up_proj.weight.data_ptr() == f.fc1_weight[I:].data_ptr()


# ---- float8_training ------------------------------------------------------------------
def test_enable_float8_emulate_conversion_on_cpu():
    model = _Model("cpu")
    before = {k: v.clone() for k, v in model.state_dict().items()}
    n = float8_training.enable_float8(model, "tensorwise", emulate=True)
    assert n == 3 * 7  # q, k, v, o, gate, up, down per text layer; head untouched
    assert not isinstance(model.head, float8_training.Float8Linear)
    lin = model.backbone.decoder.layers[0].mlp.up_proj
    assert isinstance(lin, float8_training.TrainingLinear)
    assert lin.config.pad_inner_dim and lin.config.emulate
    assert set(model.state_dict()) == set(before)
    lin.eval()
    x = torch.randn(2, H).to(torch.bfloat16)
    assert torch.equal(lin(x), nn.functional.linear(x, lin.weight))
    # same recipe again: nothing new, count stays
    assert float8_training.enable_float8(model, "tensorwise", emulate=True) == n
    # a training forward needs the device: no CPU emulation in the product path
    lin.train()
    with pytest.raises(RuntimeError, match="MI355X"):
        lin(x)


def test_enable_float8_errors():
    with pytest.raises(ValueError, match="must be one of"):
        float8_training.enable_float8(_Model("cpu"), "bogus", emulate=True)
    with pytest.raises(ValueError, match="MI355X"):
        float8_training.enable_float8(_Model("cpu"), "tensorwise")
    model = _Model("cpu")
    for p in model.parameters():
        p.requires_grad_(False)
    with pytest.raises(ValueError, match="no eligible"):
        float8_training.enable_float8(model, "tensorwise", emulate=True)
    model = _Model("cpu")
    float8_training.enable_float8(model, "tensorwise", emulate=True)
    model.backbone.decoder.layers[0].mlp.up_proj.config = float8_training.Float8LinearConfig(
        recipe="tensorwise")
    with pytest.raises(ValueError, match="retain its FP8 recipe"):
        float8_training.enable_float8(model, "tensorwise", emulate=True)
    # a model converted under one recipe cannot be converted again under another
    with pytest.raises(ValueError, match="retain its FP8 recipe"):
        float8_training.enable_float8(model, "rowwise", emulate=True)


@pytest.mark.parametrize("recipe", ["rowwise", "rowwise_with_gw_hp"])
def test_enable_float8_axiswise_recipes_convert(recipe):
    model = _Model("cpu")
    assert float8_training.enable_float8(model, recipe, emulate=True) == 3 * 7
    lin = model.backbone.encoder.text_model.layers[0].self_attn.q_proj
    assert isinstance(lin, float8_training.TrainingLinear) and lin.config.recipe == recipe
    assert float8_training.enable_float8(model, recipe, emulate=True) == 3 * 7


# ---- delayed scaling recipe ('fp8_delayed') ---------------------------------------------
def test_delayed_recipe_extra_state_round_trip_and_export():
    """'fp8_delayed' modules keep amax histories in _extra_state (non-empty), which load
    back through load_state_dict and make export raise as stateful scaling does."""
    lin = te_linear.TELinear([nn.Linear(H, 32, bias=False).to(torch.bfloat16)], "fp8_delayed")
    assert lin.recipe.amax_history_len == 16
    sd = lin.state_dict()
    assert sd["_extra_state"].numel() == 3 * (3 + 16 + 4)
    hist = sd["_extra_state"].clone()
    hist[3] = 2.5                                   # input role, history slot 0
    hist[1] = 1.0                                   # one amax recorded
    lin2 = te_linear.TELinear([nn.Linear(H, 32, bias=False).to(torch.bfloat16)], "fp8_delayed")
    lin2.load_state_dict({"weight": sd["weight"], "_extra_state": hist})
    assert lin2.scaling.input.recorded == 1
    assert lin2.scaling.input.state[0].item() == 2.5
    assert torch.equal(lin2.state_dict()["_extra_state"], hist)
    with pytest.raises(ValueError, match="stateless"):
        te_linear.TELinear([nn.Linear(H, 32, bias=False)], "fp8").load_state_dict(
            {"weight": sd["weight"], "_extra_state": hist})
    model = _Model()
    te_linear.enable_te_linear(model, mlp="fp8_delayed")
    with pytest.raises(ValueError, match="stateless"):
        te_linear.restore_hf_layout(model.backbone, model.backbone.state_dict())
    model = _Model()
    assert fused_mlp.enable_fused_mlp(model, "fp8_delayed") == 3
    f = model.backbone.decoder.layers[0].mlp
    assert f.state_dict()["_extra_state"].numel() == 2 * 3 * (3 + 16 + 4)
    with pytest.raises(ValueError, match="stateless"):
        fused_mlp.hf_state_dict(model.backbone)


def test_delayed_recipe_needs_fused_gate_up(monkeypatch):
    monkeypatch.setenv("BONGARD_TE_SPLIT_GATE_UP", "1")
    with pytest.raises(ValueError, match="fused gate_up"):
        te_linear.TEMLP(_mlp(4), "fp8_delayed")


def test_pack_to_32_rows_need_no_pad_copy():
    """The pack-to-32 contract (bongard/packing.py:240-246): a packed batch whose row count
    is already a multiple of 32 (filler segment included) reaches the projections as is,
    with no alignment copy; other row counts are padded with zero rows, which leave every
    amax unchanged."""
    x = torch.randn(64, 16)
    flat, length, aligned = te_linear._pad_rows(x)
    assert flat is x and length == aligned == 64
    y = torch.randn(70, 16)
    flat, length, aligned = te_linear._pad_rows(y)
    assert (length, aligned) == (70, 96) and torch.equal(flat[:70], y)
    assert bool((flat[70:] == 0).all()) and flat.abs().max() == y.abs().max()


def test_checkpoint_region_detection_on_cpu():
    """The delayed scalers tell a checkpointed region's original forward from its replay in
    backward (torch.utils.checkpoint, non-reentrant), and see neither outside a region."""
    from torch.utils.checkpoint import checkpoint

    from bongard_amd.scaling import checkpoint_region

    seen = []

    def region(t):
        seen.append(checkpoint_region())
        return (t * 2).sin()

    assert checkpoint_region() == (None, False)
    x = torch.randn(8, requires_grad=True)
    y = checkpoint(region, x, use_reentrant=False)
    y.sum().backward()
    (f0, replay0), (f1, replay1) = seen
    assert f0 is not None and replay0 is False      # the original forward names its region
    assert f1 is f0 and replay1 is True             # the replay names the same region
    seen.clear()
    y2 = checkpoint(region, x, use_reentrant=False)
    assert seen[0][0] is not f0                     # another region, another frame
    y2.sum().backward()
    region(x)                                       # a plain call: no region
    assert seen[-1] == (None, False)


def test_fp8_training_needs_feature_sizes_of_16():
    """The FP8 backward reads the forward's fp8 tensors as K-major GEMM operands, whose rows
    must be whole 16-byte multiples: training a linear or gated MLP whose feature sizes are
    not raises before any kernel runs (inference has no such bound)."""
    from bongard_amd import linear
    x = torch.zeros(32, 256, dtype=torch.bfloat16, requires_grad=True)
    w = torch.zeros(376, 256, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(ValueError, match="multiples of 16"):
        linear.Fp8LinearFunction.apply(x, w, None, None)
    w_gu = torch.zeros(2 * 512, 256, dtype=torch.bfloat16, requires_grad=True)
    w_d = torch.zeros(264, 512, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(ValueError, match="multiples of 16"):
        linear.Fp8GegluMlpFunction.apply(x, w_gu, w_d, None, None, 512, False)
