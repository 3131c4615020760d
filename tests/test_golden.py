"""Committed golden vectors (tests/golden/fp8_golden.npz, written by make_golden.py):
the CPU oracle must still reproduce them, and the GPU path must match them."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as orc

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "fp8_golden.npz")


def _bf16(name):
    return torch.from_numpy(GOLD[name].astype(np.int16)).view(torch.bfloat16)


def test_oracle_reproduces_golden():
    x, w, dy = _bf16("x"), _bf16("w"), _bf16("dy")
    xq, xa, xs, xsi = orc.quantize(x, orc.E4M3)
    wq, _, ws, _ = orc.quantize(w, orc.E4M3)
    dq, _, ds, _ = orc.quantize(dy, orc.E5M2)
    assert np.array_equal(xq.numpy(), GOLD["xq"])
    assert np.array_equal(wq.numpy(), GOLD["wq"])
    assert np.array_equal(dq.numpy(), GOLD["dq"])
    assert np.array_equal(np.array([xa, xs, xsi], dtype=np.float32), GOLD["x_meta"])
    y = orc.scaled_mm(xq, xs, orc.E4M3, wq, ws, orc.E4M3).numpy()
    assert np.array_equal(y, GOLD["y"])
    h = orc.geglu(_bf16("g"), _bf16("u"))
    assert np.array_equal(h.view(torch.int16).numpy().astype(np.uint16), GOLD["h"])
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    assert np.array_equal(orc.cast(allb, torch.tensor(1.0), orc.E4M3).numpy(), GOLD["table_e4m3"])
    assert np.array_equal(orc.cast(allb, torch.tensor(1.0), orc.E5M2).numpy(), GOLD["table_e5m2"])


@pytest.mark.gpu
def test_gpu_matches_golden(gpu):
    from bongard_amd import ops

    for name, fmt, qname, mname in (("x", 0, "xq", "x_meta"), ("w", 0, "wq", "w_meta"),
                                    ("dy", 1, "dq", "dy_meta")):
        q = ops.quantize(_bf16(name).to(gpu), fmt, transpose=True)
        torch.cuda.synchronize()
        assert np.array_equal(q.data.view(torch.uint8).cpu().numpy(), GOLD[qname]), name
        assert np.array_equal(q.data_t.view(torch.uint8).cpu().numpy(), GOLD[qname].T), name
        assert np.array_equal(q.meta[:3].cpu().numpy(), GOLD[mname]), name
    xq = ops.quantize(_bf16("x").to(gpu))
    wq = ops.quantize(_bf16("w").to(gpu))
    y = ops.gemm(xq.data, 0, xq.meta, wq.data, 0, wq.meta, out_dtype=torch.float32).cpu().numpy()
    ref = GOLD["y"]
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert np.abs(y - ref).max() <= 0.01 * rms
