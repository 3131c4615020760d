"""Writes tests/golden/fp8_golden.npz from the CPU oracle (run from the repo root).

The reference ships no fixtures for this path, so these vectors pin the oracle's own
outputs (regression) after tests/test_oracle.py has checked the oracle against known
answers, a second encoder and closed forms. Small, seeded, config-1-like cases:
  c1s: X [64, 256] bf16 ~N(0,1) with 4 outlier columns x20, W [128, 256] ~N(0, 0.02)
       -> e4m3 bytes and scales of X and W, fp32 Y = Xq.Wq^T (fp64 accumulate)
  e5m2: dY [64, 128] ~N(0, 1e-3) -> e5m2 bytes and scale
  geglu: g, u bf16 [32, 64] -> H = gelu_tanh(g) * u (torch CPU bf16 chain)
  table: e4m3 and e5m2 bytes of all 65,536 bf16 bit patterns at scale 1
"""

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import fp8_oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().with_name("fp8_golden.npz")


def bits16(t):
    return t.view(torch.int16).numpy().astype(np.uint16)


def main():
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(64, 256, generator=g)
    idx = torch.randperm(256, generator=g)[:4]
    x[:, idx] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(128, 256, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(64, 128, generator=g) * 1e-3).to(torch.bfloat16)
    gg = (torch.randn(32, 64, generator=g) * 2).to(torch.bfloat16)
    uu = torch.randn(32, 64, generator=g).to(torch.bfloat16)

    xq, xa, xs, xsi = orc.quantize(x, orc.E4M3)
    wq, wa, ws, wsi = orc.quantize(w, orc.E4M3)
    y = orc.scaled_mm(xq, xs, orc.E4M3, wq, ws, orc.E4M3)
    dq, da, ds, dsi = orc.quantize(dy, orc.E5M2)
    h = orc.geglu(gg, uu)
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    one = torch.tensor(1.0)
    np.savez_compressed(
        OUT,
        x=bits16(x), w=bits16(w), dy=bits16(dy), g=bits16(gg), u=bits16(uu),
        xq=xq.numpy(), wq=wq.numpy(), dq=dq.numpy(),
        x_meta=np.array([xa, xs, xsi], dtype=np.float32),
        w_meta=np.array([wa, ws, wsi], dtype=np.float32),
        dy_meta=np.array([da, ds, dsi], dtype=np.float32),
        y=y.numpy().astype(np.float32), h=bits16(h),
        table_e4m3=orc.cast(allb, one, orc.E4M3).numpy(),
        table_e5m2=orc.cast(allb, one, orc.E5M2).numpy(),
    )
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
