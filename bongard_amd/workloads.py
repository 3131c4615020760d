"""Seeded synthetic inputs of the five BASELINE configurations of the FP8 linear path.

Tensors are drawn on the CPU in fp32 with ``torch.Generator().manual_seed(seed)`` in the
order listed, then rounded to bf16 (RNE), so the GPU and the CPU oracle see identical
bytes. Shapes are Gemma-3-4B's text layer: hidden 2560, intermediate 10240, Q 2048,
K 1024, V 1024, O 2048 -> 2560.
"""

import torch

HIDDEN = 2560
INTERMEDIATE = 10240
Q_OUT, K_OUT, V_OUT = 2048, 1024, 1024


def _randn(gen, *shape, std=1.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


def config1(seed=1, rows=512, hidden=HIDDEN, out=2048, outliers=8):
    """c1: X [512, 2560] ~N(0,1) with 8 random columns x20; W [2048, 2560] ~N(0, 0.02)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, hidden, generator=g, dtype=torch.float32)
    idx = torch.randperm(hidden, generator=g)[:outliers]
    x[:, idx] *= 20.0
    w = torch.randn(out, hidden, generator=g, dtype=torch.float32) * 0.02
    return {"x": x.to(torch.bfloat16), "w": w.to(torch.bfloat16)}


def mlp_weights(gen, hidden=HIDDEN, inter=INTERMEDIATE):
    return {
        "w_gate": _randn(gen, inter, hidden, std=0.02),
        "w_up": _randn(gen, inter, hidden, std=0.02),
        "w_down": _randn(gen, hidden, inter, std=0.014),
    }


def config2(seed=2, rows=4096, hidden=HIDDEN, inter=INTERMEDIATE):
    """c2: gated-GELU MLP, X [4096, 2560]; W_gate/W_up [10240, 2560]; W_down [2560, 10240]."""
    g = torch.Generator().manual_seed(seed)
    x = _randn(g, rows, hidden)
    return {"x": x, **mlp_weights(g, hidden, inter)}


def attention_weights(gen, hidden=HIDDEN):
    return {
        "w_q": _randn(gen, Q_OUT, hidden, std=0.02),
        "w_k": _randn(gen, K_OUT, hidden, std=0.02),
        "w_v": _randn(gen, V_OUT, hidden, std=0.02),
        "w_o": _randn(gen, hidden, Q_OUT, std=0.02),
    }


def config3(seed=3, n_seq=8, lo=512, hi=3584, hidden=HIDDEN, inter=INTERMEDIATE):
    """c3: packed varlen encoder layer: 8 lengths ~U[512, 3584], M = sum (~16k tokens)."""
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lo, hi + 1, (n_seq,), generator=g)
    m = int(lengths.sum())
    x = _randn(g, m, hidden)
    return {"lengths": lengths, "x": x, **attention_weights(g, hidden), **mlp_weights(g, hidden, inter)}


def config4(seed=4, branches=8, tokens=64, hidden=HIDDEN, inter=INTERMEDIATE):
    """c4: decoder-branch skinny GEMMs: M = 8 x 64 = 512 rows, c3's weights."""
    g = torch.Generator().manual_seed(seed)
    x = _randn(g, branches * tokens, hidden)
    return {"x": x, **attention_weights(g, hidden), **mlp_weights(g, hidden, inter)}


def config5(seed=5, rows=8192, hidden=HIDDEN, inter=INTERMEDIATE, history=16):
    """c5: FP8 training step of c2's MLP at M=8192; grad_out ~N(0, 1e-3) (e5m2)."""
    g = torch.Generator().manual_seed(seed)
    x = _randn(g, rows, hidden)
    w = mlp_weights(g, hidden, inter)
    dy = _randn(g, rows, hidden, std=1e-3)
    return {"x": x, "dy": dy, "history": history, **w}
