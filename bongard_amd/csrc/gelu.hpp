// The gated GELU(tanh) of the MLP, bit-exact with torch's CPU kernels on bf16 tensors.
//
// The reference computes h = F.gelu(gate, approximate='tanh') * up on bf16 tensors
// (bongard/te_linear.py:103; HF T5Gemma2MLP) and differentiates it with autograd:
//   a   = gelu(g)             bf16 of torch's fp32 formula (its own vectorised tanh)
//   h   = bf16(f32(a) * f32(u))
//   d_u = bf16(f32(dh) * f32(a)),  d_a = bf16(f32(dh) * f32(u))
//   d_g = bf16(f32(d_a) * F(g))    F(g): the fp32 derivative factor of torch's gelu
//                                  backward (a function of g alone)
// a and F come from tables generated from torch's CPU kernels at build time
// (gen_gelu_tables.py -> gelu_tables.inc, over 2^-16 <= |g| < 8 and 2^-25 <= |g| < 8) and
// from closed rules outside them (checked against torch on all 65,536 bf16 inputs by the
// generator). Kernels copy the tables into LDS and look them up there. NaN results are
// 0xFFFF, the bf16 NaN torch's vectorised CPU conversion writes.
#pragma once

#include "common.hpp"
#include "gelu_tables.inc"

namespace bf8 {

constexpr int kGeluABytes = (int)sizeof(kGeluA);  // 10240 (9728 used)
constexpr int kGeluA32Bytes = (int)sizeof(kGeluA32);  // 26624 (positive: 0 .., negative: 16384 ..)
constexpr int kGeluFBytes = (int)sizeof(kGeluF);  // 28672

// Index into kGeluA for the bf16 g in the low 16 bits (clamped into the table when g lies
// outside it; gelu_finish then ignores the value read).
__device__ __forceinline__ uint32_t gelu_index(uint32_t g) {
  const uint32_t mag = g & 0x7FFFu, neg = (g >> 15) & 1u;
  return min(mag - kGeluALo, kGeluASpan - 1u) + neg * kGeluASpan;
}

// a(g) from the table value t read at gelu_index(g): t inside the table, the rules outside.
__device__ __forceinline__ uint32_t gelu_finish(uint32_t g, uint32_t t) {
  const uint32_t mag = g & 0x7FFFu, neg = (g >> 15) & 1u;
  // below the table (|g| < 2^-16): bf16(g / 2); below the normal range the integer
  // significand is halved with ties to even
  const uint32_t half = mag >= 0x100u ? mag - 0x80u : (mag >> 1) + (mag & (mag >> 1) & 1u);
  // |g| >= 8: g (positive, +inf), -0 (negative finite), NaN (NaN, -inf)
  const uint32_t large = mag > 0x7F80u ? 0xFFFFu : (neg == 0u ? g & 0xFFFFu : (mag == 0x7F80u ? 0xFFFFu : 0x8000u));
  return mag - kGeluALo < kGeluASpan ? t : (mag < kGeluALo ? (half | (neg << 15)) : large);
}

// Table indices (two u16 halves) of the two bf16 values of a packed pair, for a table
// over magnitudes [LO, LO + SPAN) per sign, clamped into the table; `outside` gets a
// non-zero bit when either value lies outside it, in which case the caller finishes those
// values with the rules (gelu_finish / gelu_factor_finish) instead of taking the entries.
template <uint32_t LO, uint32_t SPAN>
__device__ __forceinline__ uint32_t table_index2(uint32_t g2, uint32_t& outside) {
  const u16x2 rel = __builtin_bit_cast(u16x2, g2 & 0x7FFF7FFFu) -
                    u16x2{(unsigned short)LO, (unsigned short)LO};
  const u16x2 cl =
      __builtin_elementwise_min(rel, u16x2{(unsigned short)(SPAN - 1), (unsigned short)(SPAN - 1)});
  outside |= __builtin_bit_cast(uint32_t, cl) ^ __builtin_bit_cast(uint32_t, rel);
  const u16x2 neg = __builtin_bit_cast(u16x2, (g2 >> 15) & 0x00010001u);
  return __builtin_bit_cast(uint32_t, cl + neg * u16x2{(unsigned short)SPAN, (unsigned short)SPAN});
}

__device__ __forceinline__ uint32_t gelu_index2(uint32_t g2, uint32_t& outside) {
  return table_index2<kGeluALo, kGeluASpan>(g2, outside);
}
__device__ __forceinline__ uint32_t gelu_factor_index2(uint32_t g2, uint32_t& outside) {
  return table_index2<kGeluFLo, kGeluFSpan>(g2, outside);
}

// Byte offsets (two u16 halves) into kGeluA32 of the two bf16 values of a packed pair,
// clamped into the table; `outside` as for table_index2. Positive inputs sit at bytes
// 4 * (m - LO), negative ones 16384 bytes further on, so the sign bit of each half, shifted
// right by one, is its offset.
__device__ __forceinline__ uint32_t gelu_addr32x2(uint32_t g2, uint32_t& outside) {
  static_assert(4 * kGeluASpan <= 16384 && sizeof(kGeluA32) >= 16384 + 4 * kGeluASpan,
                "kGeluA32 layout");
  asm volatile("" : "+v"(g2));  // keep the packed form (not the halves' sources) in view
  constexpr unsigned short lo = (unsigned short)kGeluALo, span = (unsigned short)kGeluASpan;
  const u16x2 rel = __builtin_bit_cast(u16x2, g2 & 0x7FFF7FFFu) - u16x2{lo, lo};
  const u16x2 cl = __builtin_elementwise_min(rel, u16x2{(unsigned short)(span - 1),
                                                        (unsigned short)(span - 1)});
  outside |= __builtin_bit_cast(uint32_t, cl) ^ __builtin_bit_cast(uint32_t, rel);
  return __builtin_bit_cast(uint32_t, cl << (unsigned short)2) | ((g2 >> 1) & 0x40004000u);
}

// Whether a packed pair of |bf16| keys (sign bits clear) holds a NaN.
__device__ __forceinline__ bool nan_key2(uint32_t k2) {
  return (k2 & 0xFFFFu) > 0x7F80u || (k2 >> 16) > 0x7F80u;
}

// F(g) (fp32 bits) from the table value t read at the clamped index of g: t inside the
// table; outside it 0.5 (|g| < 2^-25), and for |g| >= 8: 1 / 0 by sign while g^2 is
// finite, NaN from 2^64 on.
__device__ __forceinline__ uint32_t gelu_factor_finish(uint32_t g, uint32_t t) {
  const uint32_t mag = g & 0x7FFFu, neg = (g >> 15) & 1u;
  const uint32_t large = mag >= 0x5F80u ? 0x7FC00000u : (neg ? 0u : 0x3F800000u);
  return mag - kGeluFLo < kGeluFSpan ? t : (mag < kGeluFLo ? 0x3F000000u : large);
}

// A packed bf16 pair with each NaN half replaced by 0xFFFF.
__device__ __forceinline__ uint32_t nan_ffff_bf16x2(uint32_t w) {
  const uint32_t nan = ((w & 0x7FFF7FFFu) + 0x007F007Fu) & 0x80008000u;
  if (__builtin_expect(nan != 0, 0)) {
    if (nan & 0x8000u) w |= 0x0000FFFFu;
    if (nan & 0x80000000u) w |= 0xFFFF0000u;
  }
  return w;
}

// h = bf16(f32(a) * f32(u)) for packed pairs of a = gelu(g) and u.
__device__ __forceinline__ uint32_t geglu_mul_bf16x2(uint32_t a2, uint32_t u2) {
  return nan_ffff_bf16x2(pack_bf16x2(bf16_lo(a2) * bf16_lo(u2), bf16_hi(a2) * bf16_hi(u2)));
}

// Copies kGeluA (and kGeluF when tab_f is set) into LDS with NT threads; the caller
// synchronises the block before the first lookup.
template <int NT>
__device__ __forceinline__ void load_gelu_tables(uint16_t* tab_a, uint32_t* tab_f) {
  const uint4* sa = reinterpret_cast<const uint4*>(kGeluA);
  uint4* da = reinterpret_cast<uint4*>(tab_a);
  for (int i = threadIdx.x; i < kGeluABytes / 16; i += NT) da[i] = sa[i];
  if (tab_f) {
    const uint4* sf = reinterpret_cast<const uint4*>(kGeluF);
    uint4* df = reinterpret_cast<uint4*>(tab_f);
    for (int i = threadIdx.x; i < kGeluFBytes / 16; i += NT) df[i] = sf[i];
  }
}

}  // namespace bf8
