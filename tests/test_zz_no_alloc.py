"""The allocation-free quantization (bf8_quantize_bf16_noalloc), called through the C ABI.

It is bf8_quantize_bf16 with the amax partials in a library-owned device array instead of
a caller workspace; its bytes (row-major and transposed copies) and meta must equal the
workspace entry point's bit for bit on two calls in a row, the second one smaller (the
array keeps the first call's partials, which the second must not read), and the oracle's.
"""

import ctypes

import pytest
import torch

from bongard_amd import _lib
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu

E4M3, E5M2, POW2 = 0, 1, 0x10


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _outputs(x, transpose):
    rows, cols = x.shape
    out = torch.empty(rows, cols, dtype=torch.uint8, device=x.device)
    out_t = torch.empty(cols, rows, dtype=torch.uint8, device=x.device) if transpose else None
    meta = torch.full((4,), float("nan"), dtype=torch.float32, device=x.device)
    return out, out_t, meta


def _noalloc(x, fmt, transpose):
    out, out_t, meta = _outputs(x, transpose)
    rows, cols = x.shape
    _lib.check(_lib.lib().bf8_quantize_bf16_noalloc(_p(x), rows, cols, fmt, _p(out), _p(out_t),
                                                    _p(meta), _stream()),
               "bf8_quantize_bf16_noalloc")
    return out, out_t, meta


def _with_workspace(x, fmt, transpose):
    L = _lib.lib()
    out, out_t, meta = _outputs(x, transpose)
    rows, cols = x.shape
    parts = torch.empty(L.bf8_amax_partials(rows * cols), dtype=torch.int32, device=x.device)
    _lib.check(L.bf8_quantize_bf16(_p(x), rows, cols, fmt, _p(out), _p(out_t), _p(meta),
                                   _p(parts), _stream()), "bf8_quantize_bf16")
    return out, out_t, meta


def test_noalloc_equals_workspace_entry_point(gpu):
    g = torch.Generator().manual_seed(91)
    big = torch.randn(4096, 2560, generator=g)
    big[17, 5] = 900.0                       # a large amax left behind in the scratch slots
    small = torch.randn(96, 160, generator=g) * 1e-3
    cases = [(big.to(torch.bfloat16), E4M3, True), (small.to(torch.bfloat16), E5M2 | POW2, False)]
    for x_cpu, fmt, transpose in cases:
        x = x_cpu.to(gpu)
        got = _noalloc(x, fmt, transpose)
        want = _with_workspace(x, fmt, transpose)
        torch.cuda.synchronize()
        assert torch.equal(got[0].cpu(), want[0].cpu()), "row-major bytes differ"
        if transpose:
            assert torch.equal(got[1].cpu(), want[1].cpu()), "transposed bytes differ"
        assert torch.equal(got[2].cpu().view(torch.int32), want[2].cpu().view(torch.int32)), \
            f"meta differs: {got[2].cpu().tolist()} vs {want[2].cpu().tolist()}"
        base = fmt & ~POW2
        rq, ra, rs, _ = orc.quantize(x_cpu, base) if not fmt & POW2 else (None, None, None, None)
        if rq is not None:
            assert torch.equal(got[0].cpu(), rq) and got[2].cpu()[1].item() == rs.item()
        else:  # the rowwise recipes' power-of-two scale: mantissa of the scale cleared
            s = orc.amax_to_scale_axiswise(orc.amax(x_cpu), base, pow2=True)
            assert got[2].cpu()[1].item() == s.item()
            assert torch.equal(got[0].cpu(), orc.cast(x_cpu, s, base))


def test_noalloc_rejects_bad_arguments(gpu):
    x = torch.randn(64, 64, device=gpu).to(torch.bfloat16)
    out, _, meta = _outputs(x, False)
    L = _lib.lib()
    assert L.bf8_quantize_bf16_noalloc(_p(x), 64, 64, 7, _p(out), None, _p(meta), _stream()) != 0
    assert b"bad fmt" in L.bf8_last_error()
    assert L.bf8_quantize_bf16_noalloc(_p(x), 64, 64, E4M3, _p(out), None, None, _stream()) != 0
