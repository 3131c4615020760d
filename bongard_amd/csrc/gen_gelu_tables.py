"""Writes gelu_tables.inc: the gated-GELU(tanh) lookup tables of the HIP kernels.

The reference applies ``F.gelu(gate, approximate='tanh') * up`` to bf16 tensors
(bongard/te_linear.py:103; HF T5Gemma2MLP) and differentiates it with autograd. On bf16
inputs torch's CPU kernels compute, per element x (all arithmetic in fp32):

  forward   a(x)  = bf16(0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))))
  backward  d(dy, x) = bf16(f32(dy) * F(x)),  F(x) = the fp32 value of
            0.5 (1 + t) + 0.5 x (1 - t^2) sqrt(2/pi) (1 + 3 * 0.044715 x^2),  t = tanh(...)

with torch's own vectorised tanh. Both depend on x alone, so a table over the bf16 inputs
reproduces them bit for bit. Outside the ranges tabulated here the values follow simple
rules, which this script verifies on all 65,536 bf16 inputs before writing anything:

  a(x):  |x| < 2^-9  -> bf16(x / 2) (round to nearest even); the table nevertheless
                        starts at 2^-16, so that gates of ordinary magnitude (the bulk
                        of a GEMM's outputs) all take the table path
         |x| >= 8    -> x (positive, +inf), -0 (negative finite), NaN (NaN, -inf)
  F(x):  |x| < 2^-25 -> 0.5
         |x| >= 8    -> 1 (positive), 0 (negative) while x^2 is finite, NaN beyond
                        (|x| >= 2^64) and for inf / NaN

Tables (bf16 magnitude bits m = bits & 0x7FFF, sign s):
  kGeluA[s * 2432 + (m - 0x3780)]  bf16 bits of a(x), 0x3780 <= m < 0x4100  (2^-16 .. 8),
                                   zero-padded to 10 KB (whole 1 KB copies into LDS)
  kGeluA32[s * 4096 + (m - 0x3780)]  the same values as fp32 bits (bf16 << 16), negative
                                   inputs from entry 4096 (byte 16384) on, zero-padded to
                                   26 KB, for kernels that multiply them as read
  kGeluF[s * 3584 + (m - 0x3300)]  fp32 bits of F(x), 0x3300 <= m < 0x4100  (2^-25 .. 8)

Run by bongard_amd/build.py before compiling (``python gen_gelu_tables.py OUT``).
"""

import sys
from pathlib import Path

A_LO, A_HI = 0x3780, 0x4100
A_PAD_BYTES = 10 * 1024
A32_PAD_BYTES = 26 * 1024
A32_NEG = 4096  # first entry of the negative inputs in kGeluA32
F_LO, F_HI = 0x3300, 0x4100


def _all_bf16():
    import torch

    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def torch_gelu_bits():
    """bf16 bits of torch's CPU gelu(x, 'tanh') for every bf16 bit pattern x (int64 [65536])."""
    import torch
    import torch.nn.functional as F

    return F.gelu(_all_bf16(), approximate="tanh").view(torch.int16).to(torch.int64) & 0xFFFF


def torch_gelu_grad_factor_bits():
    """fp32 bits of F(x) (the backward's factor, torch's fp32 formula) for every bf16 x."""
    import torch

    x = _all_bf16().float()
    f = torch.ops.aten.gelu_backward(torch.ones_like(x), x, approximate="tanh")
    return f.view(torch.int32).to(torch.int64) & 0xFFFFFFFF


def rule_gelu_bits(bits):
    """a(x) outside the table, from the rules in the module docstring (bits: int)."""
    mag, neg = bits & 0x7FFF, bits >> 15
    if mag < 0x3B00:  # |x| < 2^-9
        if mag >= 0x100:
            half = mag - 0x80
        else:  # result below the normal range: halve the integer significand, ties to even
            half = (mag >> 1) + (mag & (mag >> 1) & 1)
        return half | (neg << 15)
    if mag > 0x7F80:
        return 0xFFFF
    if not neg:
        return bits
    return 0xFFFF if mag == 0x7F80 else 0x8000


def rule_factor_bits(bits):
    """F(x) outside the table (fp32 bits)."""
    mag, neg = bits & 0x7FFF, bits >> 15
    if mag < F_LO:
        return 0x3F000000            # 0.5
    if mag >= 0x5F80:                # |x| >= 2^64 (x^2 overflows), inf, NaN
        return 0x7FC00000
    return 0x00000000 if neg else 0x3F800000


def _check_rules(a_bits, f_bits):
    bad = []
    for b in range(65536):
        m = b & 0x7FFF
        if not A_LO <= m < A_HI and rule_gelu_bits(b) != int(a_bits[b]):
            bad.append(("a", hex(b), hex(int(a_bits[b])), hex(rule_gelu_bits(b))))
        if not F_LO <= m < F_HI:
            want = rule_factor_bits(b)
            got = int(f_bits[b])
            nan_both = want == 0x7FC00000 and (got & 0x7FFFFFFF) > 0x7F800000
            if got != want and not nan_both:
                bad.append(("F", hex(b), hex(got), hex(want)))
    if bad:
        raise RuntimeError(f"gelu table rules do not hold for torch's CPU kernels: {bad[:8]}")


def tables():
    """(kGeluA, kGeluF) as lists of ints, after checking the rules."""
    a_bits = torch_gelu_bits().tolist()
    f_bits = torch_gelu_grad_factor_bits().tolist()
    _check_rules(a_bits, f_bits)
    ga = [a_bits[(s << 15) | m] for s in (0, 1) for m in range(A_LO, A_HI)]
    ga += [0] * (A_PAD_BYTES // 2 - len(ga))
    gf = [f_bits[(s << 15) | m] for s in (0, 1) for m in range(F_LO, F_HI)]
    # inside the table, a NaN factor never occurs (checked so the kernels need no patch)
    assert not any((v & 0x7FFFFFFF) > 0x7F800000 for v in gf)
    return ga, gf


def render(ga, gf):
    span = A_HI - A_LO
    ga32 = [v << 16 for v in ga[:span]] + [0] * (A32_NEG - span) + [v << 16 for v in ga[span:2 * span]]
    ga32 += [0] * (A32_PAD_BYTES // 4 - len(ga32))

    def rows(vals, fmt, per):
        return "\n".join("    " + ", ".join(fmt.format(v) for v in vals[i:i + per]) + ","
                         for i in range(0, len(vals), per))

    return (
        "// Generated by gen_gelu_tables.py from torch's CPU gelu(tanh) kernels; do not edit.\n"
        f"constexpr uint32_t kGeluALo = 0x{A_LO:04X}u, kGeluASpan = 0x{A_HI - A_LO:X}u;\n"
        f"constexpr uint32_t kGeluFLo = 0x{F_LO:04X}u, kGeluFSpan = 0x{F_HI - F_LO:X}u;\n"
        f"static __device__ const uint16_t kGeluA[{len(ga)}] __attribute__((aligned(16))) = {{\n"
        f"{rows(ga, '0x{:04X}', 12)}\n}};\n"
        f"static __device__ const uint32_t kGeluA32[{len(ga32)}] __attribute__((aligned(16))) = {{\n"
        f"{rows(ga32, '0x{:08X}u', 8)}\n}};\n"
        f"static __device__ const uint32_t kGeluF[{len(gf)}] __attribute__((aligned(16))) = {{\n"
        f"{rows(gf, '0x{:08X}u', 8)}\n}};\n")


def main(out):
    ga, gf = tables()
    text = render(ga, gf)
    out = Path(out)
    if not out.exists() or out.read_text() != text:
        out.write_text(text)
    return out


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "gelu_tables.inc")
