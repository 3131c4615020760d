// FP8 GEMM kernel for gfx950 (MI355X) on the double-rate f8f6f4 MFMA, with a dequant/bias
// epilogue (or raw fp32 split-K partials), and a gated-GELU(tanh) epilogue for the MLP
// gate/up projection. Included by the gemm_tile_*.hip files only.
//
// Semantics replace torch._scaled_mm / cuBLASLt under torchao Float8Linear
// (bongard/float8_training.py:22) and TE's FP8 GEMM under te.Linear
// (bongard/te_linear.py:73-74): C = (A8 . B8^T accumulated in fp32) * sa_inv * sb_inv
// (+ bias), "TN" layout (both operands K-contiguous, as nn.Linear weights are).
//
// Design (one workgroup = 4 wave64, block tile BM x BN, K step 128 bytes):
//  - global -> LDS by direct 16-byte buffer loads into LDS (no VGPR staging; out-of-range
//    rows/K read as zero), NS LDS stages of (BM + BN) x 128 bytes in flight;
//  - LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at c ^ ((r >> 1) & 7)
//    so that a fragment read (16 lanes = 16 rows x 16 bytes per LDS cycle on the 64-bank,
//    256 B/clk gfx950 LDS) touches every bank once;
//  - each wave owns FM x FN MFMA 32x32x64 tiles; the MFMA "A" operand is the B (weight)
//    tile, so every lane ends up holding four consecutive output columns of one row;
//  - per 64-byte K sub-step a wave issues FM*FN MFMAs with the fragment reads of the next
//    sub-step and the DMA loads of the stage after next spread evenly between them;
//  - workgroups are renumbered so that each XCD (blockIdx % 8 on MI355X) owns a
//    contiguous range of (split, tile) ids, walked in groups of kGroupM tile rows.
#pragma once

#include <type_traits>
#include <utility>

#include "gelu.hpp"
#include "gemm_kernel.hpp"

namespace bf8 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, 0>{}) .. f(...<N - 1>{}), unrolled at compile time (the
// index selects accumulator registers, so it must be a constant).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int kBK = 128;       // K bytes per LDS stage
constexpr int kNumXcd = 8;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset that always reads as zero

// LDS bytes a variant needs besides its NS pipeline stages: the gated-GELU epilogue keeps
// the fp32 gelu table (kGeluA32) there, at LDS offset 0 ahead of the stages, so that its
// byte offsets (below 64 KB) address it directly from packed 16-bit arithmetic.
template <int EPI>
constexpr int extra_lds() { return EPI == EPI_GEGLU ? kGeluA32Bytes : 0; }

// Buffer resource (4 SGPRs): base, stride 0, `bytes` valid bytes (offsets at or beyond
// read as zero), raw-buffer flags of gfx9/gfx950.
__device__ __forceinline__ i32x4 make_srd(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xFFFFu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// 16-byte-per-lane load from a buffer straight into LDS: lane l's bytes land at
// lds_addr + 16 l. Written as inline asm so that the compiler's wait-count pass does
// not serialise it against LDS reads of other stages (it cannot prove they do not
// alias); the kernel orders it with explicit vmcnt waits and barriers instead. M0 is
// set inside the same asm block, immediately before its only use.
__device__ __forceinline__ void dma16(i32x4 srd, uint32_t lds_addr, uint32_t voff,
                                      uint32_t soff) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0v), "v"(voff), "s"(srd), "s"(so)
               : "memory");
}

// 4-byte-per-lane variant (MX block scales): lane l's dword lands at lds_addr + 4 l.
__device__ __forceinline__ void dma4(i32x4 srd, uint32_t lds_addr, uint32_t voff,
                                     uint32_t soff) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(m0v), "v"(voff), "s"(srd), "s"(so)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const uint8_t*)(p));
}

// XCD-contiguous renumbering of blocks [0, nb) (block b is dispatched to XCD b % 8): the
// blocks of XCD x get positions [x*q + min(x, r), ...) with q = nb / 8, r = nb % 8.
__device__ __forceinline__ int xcd_position(int b, int nb) {
  const int x = b % kNumXcd, idx = b / kNumXcd;
  const int q = nb / kNumXcd, r = nb % kNumXcd;
  return x * q + (x < r ? x : r) + idx;
}

// (tile row, tile column, K split) of this workgroup; `tail_slot` >= 0 for a K piece of a
// tail-split schedule (its partials' slot in tail_ws).
__device__ __forceinline__ void block_coords(const GemmParams& p, int& tm, int& tn, int& split,
                                             int& tail_slot) {
  const int ntiles = p.tiles_m * p.tiles_n;
  const int b = blockIdx.x;
  tail_slot = -1;
  if (p.tail_pieces > 0) {
    if (b < p.full_tiles) {  // whole tiles, one round per 256 workgroups
      walk_tile(p.tiles_m, p.tiles_n, xcd_position(b, p.full_tiles), tm, tn);
      split = 0;
      return;
    }
    // pieces: position = piece * tails + t, so an XCD's pieces share their K range and
    // neighbouring tail tiles share operand rows (full_tiles is a multiple of 8, so
    // b - full_tiles is on the same XCD as b)
    const int tails = ntiles - p.full_tiles;
    const int pos = xcd_position(b - p.full_tiles, tails * p.tail_pieces);
    const int t = pos % tails;
    split = pos / tails;
    walk_tile(p.tiles_m, p.tiles_n, p.full_tiles + t, tm, tn);
    tail_slot = t * p.tail_pieces + split;
    return;
  }
  int id = xcd_position(b, ntiles * p.splits);
  split = id / ntiles;
  id -= split * ntiles;
  walk_tile(p.tiles_m, p.tiles_n, id, tm, tn);
}

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <int FA, int FB>
__device__ __forceinline__ v16f mfma(v8i a, v8i b, v16f c) {
  if constexpr (FA == kFmtBf16) {
    static_assert(FB == kFmtBf16, "bf16 GEMMs take two bf16 operands");
    // the 64 bytes of a sub-step are 32 bf16 K-values: two 32x32x16 MFMAs, one per
    // 16-byte half of each lane's fragment (A and B halves pair up, so every K-value
    // of the row meets its partner)
    const v8bf a0 = __builtin_bit_cast(v8bf, __builtin_shufflevector(a, a, 0, 1, 2, 3));
    const v8bf a1 = __builtin_bit_cast(v8bf, __builtin_shufflevector(a, a, 4, 5, 6, 7));
    const v8bf b0 = __builtin_bit_cast(v8bf, __builtin_shufflevector(b, b, 0, 1, 2, 3));
    const v8bf b1 = __builtin_bit_cast(v8bf, __builtin_shufflevector(b, b, 4, 5, 6, 7));
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c, 0, 0, 0);
  } else {
    // scale operands 0: plain (unscaled) f8f6f4 MFMA; FA/FB select e4m3 (0) / e5m2 (1).
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, 0, 0, 0, 0);
  }
}

// Block-scaled (MX) form: each lane supplies the E8M0 scale of the 32 K-values it holds
// (its row of the operand, K block lane >> 5 of the 64-byte sub-step), as byte OPSEL of
// its scale register; the product of the two scales multiplies that block's products.
template <int FA, int FB, int OPSEL>
__device__ __forceinline__ v16f mfma_mx(v8i a, v8i b, v16f c, uint32_t sa, uint32_t sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, OPSEL, (int)sa, OPSEL,
                                                         (int)sb);
}

// Swizzled position of logical 16-byte chunk c in tile row r (128-byte rows).
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// Reads 16 bytes of an MFMA operand fragment: 32 rows starting at `row0` of an LDS tile,
// K bytes [kk*64, kk*64+64); lane l holds row row0 + (l & 31) (two halves make the lane's
// 32 bytes). The f8f6f4 MFMA takes register bytes 0-15 of lane half h as K = 16 h + 0..15
// and bytes 16-31 as K = 32 + 16 h + 0..15 (measured on gfx950). A plain MFMA does not
// care which K the bytes are (A and B are permuted alike), so it reads the lane's 32
// contiguous bytes (l >> 5)*32 + 16*half; the block-scaled MFMA needs K blocks [0, 32)
// and [32, 64) of the sub-step to be the ones its scales describe, so `mx` reads
// 32*half + 16*(l >> 5).
__device__ __forceinline__ v4u read_half(const uint8_t* tile, int row0, int kk, int half,
                                         int lane, bool mx = false) {
  const int row = row0 + (lane & 31);
  const int c = mx ? kk * 4 + half * 2 + (lane >> 5) : kk * 4 + (lane >> 5) * 2 + half;
  return *reinterpret_cast<const v4u*>(tile + row * kBK + (swz(row, c) << 4));
}

// K-major operand tiles (the stored tensor is the operand's transpose, [K][rows]): a stage
// holds 128 K rows of 256 row bytes, and the 16-byte chunk c of K row k sits at position
// c ^ kmaj_swz(k). A lane's 16-byte DMA piece of K row k takes logical chunk
// (its position) ^ kmaj_swz(k); the XOR keeps the transposing reads below on distinct banks
// (each half-wave reads eight K rows of two adjacent chunks: even and odd positions).
__device__ __forceinline__ int kmaj_swz(int k) { return 2 * (k & 7); }

// The same 16 bytes as read_half (lane l: operand row row0 + (l & 31), K bytes kk*64 +
// (l >> 5)*32 + 16*half .. +15) from a K-major tile, as two ds_read_b64_tr_b8: in each group
// of 16 lanes, output lane j receives byte j mod 8 of the 8-byte pieces addressed by lanes
// (j >> 3) + 2 i, i = 0..7, so lane p + 2 i of group g addresses K row k0 + i, row bytes
// c0 + 8 p (c0 = row0 + 16 (g & 1)), and lane j gets K values k0 .. k0+7 of row c0 + j.
__device__ __forceinline__ v4u read_half_kmajor(const uint8_t* tile, int row0, int kk, int half,
                                                int lane) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const int g = lane >> 4, a = lane & 15;
  const int chunk = (row0 >> 4) + (g & 1);  // 16-byte chunk of the operand rows read
  v4u r;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int k = kk * 64 + (g >> 1) * 32 + 16 * half + 8 * t + (a >> 1);
    const uint8_t* src = tile + k * 256 + ((chunk ^ kmaj_swz(k)) << 4) + 8 * (a & 1);
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i*)(
            (__attribute__((address_space(3))) uint8_t*)(src)));
    r[2 * t] = (uint32_t)v[0];
    r[2 * t + 1] = (uint32_t)v[1];
  }
  return r;
}

__device__ __forceinline__ v8i join(v4u lo, v4u hi) {
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// Epilogue staging in LDS: rows of CH 16-byte chunks; chunk c of row r lives at
// c ^ (r & (CH - 1)) for power-of-two CH, else at (c + r) % CH, so that the 32 rows a
// wave writes at once spread over the banks. Lanes put 8-byte runs (4 bf16) and get
// 16-byte chunks.
template <int CH>
__device__ __forceinline__ int stage_pos(int row, int c) {
  if constexpr ((CH & (CH - 1)) == 0)
    return c ^ (row & (CH - 1));
  else
    return (c + row) % CH;
}
template <int CH>
__device__ __forceinline__ void stage_put(uint8_t* buf, int row, int col, uint2 v) {
  const int c = col >> 3, half = (col >> 2) & 1;
  *reinterpret_cast<uint2*>(buf + row * (CH * 16) + (stage_pos<CH>(row, c) << 4) + half * 8) = v;
}
template <int CH>
__device__ __forceinline__ uint4 stage_get(const uint8_t* buf, int row, int c) {
  return *reinterpret_cast<const uint4*>(buf + row * (CH * 16) + (stage_pos<CH>(row, c) << 4));
}
// The bf16 pair at columns col, col + 1 (col even) of a staged row.
template <int CH>
__device__ __forceinline__ uint32_t stage_get_pair(const uint8_t* buf, int row, int col) {
  return *reinterpret_cast<const uint32_t*>(buf + row * (CH * 16) +
                                            (stage_pos<CH>(row, col >> 3) << 4) + (col & 7) * 2);
}
// 8 bf16 to global: one 16-byte store when the row stride keeps it aligned, with the
// non-temporal hint (the output is not re-read by this kernel; measured 1-3% faster GEMMs).
__device__ __forceinline__ void store_bf16x8(uint16_t* dst, uint4 d, int64_t ld) {
  if ((ld & 7) == 0) {
    store_nt(dst, d);
  } else {
    reinterpret_cast<uint2*>(dst)[0] = make_uint2(d.x, d.y);
    reinterpret_cast<uint2*>(dst)[1] = make_uint2(d.z, d.w);
  }
}

// MX gated-GELU epilogue: the wave's staged H (ROWS rows x CH*8 bf16 columns in LDS, first
// global row gm0, first H column h0) quantized to e4m3 in blocks of 32 with the standalone
// MX quantizer's arithmetic: along rows into h8 / h8_sc (a 4-lane group per block, 8
// values a lane), and, when h8t is set, along columns into h8t / h8t_sc (a lane per
// column pair and 32-row block). C, when set, also receives the bf16 H.
template <int ROWS, int CH, bool FAST>
__device__ __forceinline__ void mx_h_epilogue(const GemmParams& p, const uint8_t* wbuf, int lane,
                                              int gm0, int h0) {
#pragma unroll 4
  for (int it = 0; it < ROWS * CH / 64; ++it) {
    const int idx = it * 64 + lane;
    const int row = idx / CH, c = idx % CH;  // lanes 4j .. 4j+3: one block of one row
    const uint4 d = stage_get<CH>(wbuf, row, c);
    // |x| keys of the 8 values as one packed 16-bit max, then the block's max over the
    // 4-lane group with DPP quad permutes ([1,0,3,2], then [2,3,0,1])
    const uint32_t k2 = pk_max_u16(pk_max_u16(d.x & 0x7FFF7FFFu, d.y & 0x7FFF7FFFu),
                                   pk_max_u16(d.z & 0x7FFF7FFFu, d.w & 0x7FFF7FFFu));
    uint32_t k = max(k2 << 16, k2 & 0xFFFF0000u);
    k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0xB1, 0xF, 0xF, true));
    k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0x4E, 0xF, 0xF, true));
    const int gm = gm0 + row;
    if (gm < p.M) {
      const int n = h0 + c * 8;
      if (p.C) store_bf16x8(reinterpret_cast<uint16_t*>(p.C) + (int64_t)gm * p.ldc + n, d, p.ldc);
      const uint32_t e = mx_exponent<BF8_E4M3>(k);
      const float mult = mx_multiplier(e);
      *reinterpret_cast<uint2*>(p.h8 + (int64_t)gm * p.I + n) =
          FAST ? quant8_bf16_finite<BF8_E4M3, false>(d, mult) : quant8_bf16<BF8_E4M3>(d, mult);
      if ((c & 3) == 0) p.h8_sc[(int64_t)gm * p.h8_sc_ld + (n >> 5)] = (uint8_t)e;
    }
  }
  if (p.h8t == nullptr) return;
  constexpr int CP = CH * 4;                 // column pairs per staged row
  constexpr int ITEMS = (ROWS / 32) * CP;    // (32-row block, column pair) items
  const int nblk = p.M >> 5;                 // M % 32 == 0 here
  const int sc_pad_end = ((p.M + 127) >> 7) << 2;
#pragma unroll 1
  for (int item = lane; item < ITEMS; item += 64) {
    const int blk = item / CP, cp = item % CP;
    const int gm = gm0 + blk * 32;
    if (gm >= p.M) continue;
    uint32_t v[32];
    uint32_t k0 = 0, k1 = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      v[i] = stage_get_pair<CH>(wbuf, blk * 32 + i, 2 * cp);
      k0 = max(k0, v[i] & 0x7FFFu);
      k1 = max(k1, (v[i] >> 16) & 0x7FFFu);
    }
    const uint32_t e0 = mx_exponent<BF8_E4M3>(k0 << 16), e1 = mx_exponent<BF8_E4M3>(k1 << 16);
    const float s0 = mx_multiplier(e0), s1 = mx_multiplier(e1);
    uint32_t q0[8], q1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a0 = bf16_lo(v[4 * j]), a1 = bf16_lo(v[4 * j + 1]);
      const float a2 = bf16_lo(v[4 * j + 2]), a3 = bf16_lo(v[4 * j + 3]);
      const float b0 = bf16_hi(v[4 * j]), b1 = bf16_hi(v[4 * j + 1]);
      const float b2 = bf16_hi(v[4 * j + 2]), b3 = bf16_hi(v[4 * j + 3]);
      if constexpr (FAST) {
        q0[j] = quant4_finite<BF8_E4M3, false>(a0 * s0, a1 * s0, a2 * s0, a3 * s0);
        q1[j] = quant4_finite<BF8_E4M3, false>(b0 * s1, b1 * s1, b2 * s1, b3 * s1);
      } else {
        q0[j] = quant4<BF8_E4M3>(a0 * s0, a1 * s0, a2 * s0, a3 * s0, a0, a1, a2, a3, s0);
        q1[j] = quant4<BF8_E4M3>(b0 * s1, b1 * s1, b2 * s1, b3 * s1, b0, b1, b2, b3, s1);
      }
    }
    const int n = h0 + 2 * cp;
    uint4* d0 = reinterpret_cast<uint4*>(p.h8t + (int64_t)n * p.M + gm);
    uint4* d1 = reinterpret_cast<uint4*>(p.h8t + (int64_t)(n + 1) * p.M + gm);
    d0[0] = make_uint4(q0[0], q0[1], q0[2], q0[3]);
    d0[1] = make_uint4(q0[4], q0[5], q0[6], q0[7]);
    d1[0] = make_uint4(q1[0], q1[1], q1[2], q1[3]);
    d1[1] = make_uint4(q1[4], q1[5], q1[6], q1[7]);
    uint8_t* r0 = p.h8t_sc + (int64_t)n * p.h8t_sc_ld;
    uint8_t* r1 = r0 + p.h8t_sc_ld;
    r0[gm >> 5] = (uint8_t)e0;
    r1[gm >> 5] = (uint8_t)e1;
    if ((gm >> 5) == nblk - 1) {
      // the column's last block also pads its scale row to whole dwords
      for (int pb = nblk; pb < sc_pad_end; ++pb) {
        r0[pb] = (uint8_t)kMxPadScale;
        r1[pb] = (uint8_t)kMxPadScale;
      }
    }
  }
}

// Tensor-scaled gated-GELU epilogue (a scale known before the GEMM, as delayed scaling
// has): the wave's staged H quantized to e4m3 with `scale` exactly as the standalone cast
// does (quant8_bf16), into h8 [M, I] and, when h8t is set, h8t = H^T [I, M] (a lane per
// column pair and 32-row block; M % 32 == 0). C, when set, also receives the bf16 H.
template <int ROWS, int CH, bool FAST>
__device__ __forceinline__ void scaled_h_epilogue(const GemmParams& p, const uint8_t* wbuf,
                                                  int lane, int gm0, int h0, float scale) {
#pragma unroll 4
  for (int it = 0; it < ROWS * CH / 64; ++it) {
    const int idx = it * 64 + lane;
    const int row = idx / CH, c = idx % CH;
    const uint4 d = stage_get<CH>(wbuf, row, c);
    const int gm = gm0 + row;
    if (gm < p.M) {
      const int n = h0 + c * 8;
      if (p.C) store_bf16x8(reinterpret_cast<uint16_t*>(p.C) + (int64_t)gm * p.ldc + n, d, p.ldc);
      *reinterpret_cast<uint2*>(p.h8 + (int64_t)gm * p.I + n) =
          FAST ? quant8_bf16_finite<BF8_E4M3, true>(d, scale) : quant8_bf16<BF8_E4M3>(d, scale);
    }
  }
  if (p.h8t == nullptr) return;
  constexpr int CP = CH * 4;
  constexpr int ITEMS = (ROWS / 32) * CP;
#pragma unroll 1
  for (int item = lane; item < ITEMS; item += 64) {
    const int blk = item / CP, cp = item % CP;
    const int gm = gm0 + blk * 32;
    if (gm >= p.M) continue;
    uint32_t q0[8], q1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = stage_get_pair<CH>(wbuf, blk * 32 + 4 * j + e, 2 * cp);
      const float a0 = bf16_lo(v[0]), a1 = bf16_lo(v[1]), a2 = bf16_lo(v[2]), a3 = bf16_lo(v[3]);
      const float b0 = bf16_hi(v[0]), b1 = bf16_hi(v[1]), b2 = bf16_hi(v[2]), b3 = bf16_hi(v[3]);
      if constexpr (FAST) {
        q0[j] = quant4_finite<BF8_E4M3, true>(a0 * scale, a1 * scale, a2 * scale, a3 * scale);
        q1[j] = quant4_finite<BF8_E4M3, true>(b0 * scale, b1 * scale, b2 * scale, b3 * scale);
      } else {
        q0[j] = quant4<BF8_E4M3>(a0 * scale, a1 * scale, a2 * scale, a3 * scale, a0, a1, a2, a3,
                                 scale);
        q1[j] = quant4<BF8_E4M3>(b0 * scale, b1 * scale, b2 * scale, b3 * scale, b0, b1, b2, b3,
                                 scale);
      }
    }
    const int n = h0 + 2 * cp;
    uint4* d0 = reinterpret_cast<uint4*>(p.h8t + (int64_t)n * p.M + gm);
    uint4* d1 = reinterpret_cast<uint4*>(p.h8t + (int64_t)(n + 1) * p.M + gm);
    d0[0] = make_uint4(q0[0], q0[1], q0[2], q0[3]);
    d0[1] = make_uint4(q0[4], q0[5], q0[6], q0[7]);
    d1[0] = make_uint4(q1[0], q1[1], q1[2], q1[3]);
    d1[1] = make_uint4(q1[4], q1[5], q1[6], q1[7]);
  }
}

// The operand fragments of one MFMA sub-step as 16-byte halves, in the order the MFMAs
// of the sub-step consume them: b0, a0 .. a(FM-1), b1 .. b(FN-1).
template <int NH>
struct Frags {
  v4u h[NH];
};

// Where the gated-GELU epilogue finds a gate value and its up partner. A wave's H columns
// come in runs of 8 (run k: H columns 8k .. 8k+7 of the wave, a lane holding 4 of them,
// register quad q of an n-subtile). Even FN: the wave's B rows are FN/2 gate subtiles then
// FN/2 up subtiles (two wave columns side by side), so run k = (subtile k/4, quad k%4)
// pairs with subtile k/4 + FN/2, same quad. Odd FN (one wave column, WN = 1): the wave's
// B rows are the tile's, gate rows [0, BN/2) then up rows [BN/2, BN), with BN/2 a multiple
// of 8 but not of 32, so run k's up rows start at BN/2 + 8k, inside subtile (BN/2+8k)/32 at
// quad ((BN/2+8k) % 32)/8; the lane half (columns 4h..4h+3 of a quad) is the same on both
// sides because BN/2 + 8k and 8k differ by a multiple of 8.
template <int FN, int BN>
struct GegluRuns {
  static constexpr bool kOdd = FN % 2 != 0;
  static constexpr int kRuns = kOdd ? BN / 16 : FN * 2;  // runs of 8 H columns per wave
  static constexpr int gate_s(int k) { return k / 4; }
  static constexpr int gate_q(int k) { return k % 4; }
  static constexpr int up_s(int k) { return kOdd ? (BN / 2 + 8 * k) / 32 : k / 4 + FN / 2; }
  static constexpr int up_q(int k) { return kOdd ? ((BN / 2 + 8 * k) % 32) / 8 : k % 4; }
};

// Threads of a workgroup of tile T.
template <class T>
constexpr int tile_threads() { return T::NW * 64 * T::KG; }

// KM: operands stored K-major (bit 0: A given as A^T [K, M], bit 1: B given as B^T [K, N]),
// read through the transposing LDS loads; eight-wave 256 x 256 linear tiles only.
template <class T, int FA, int FB, int EPI, int OUT, bool MX = false, int KM = 0>
__global__ __attribute__((amdgpu_flat_work_group_size(tile_threads<T>(), tile_threads<T>()),
                          amdgpu_waves_per_eu(T::OCC * T::KG * T::NW / 4,
                                              T::OCC * T::KG * T::NW / 4))) void
gemm_kernel(GemmParams p) {
  constexpr int BM = T::BM, BN = T::BN, FM = T::FM, FN = T::FN, WM = T::WM, NS = T::NS;
  constexpr int KG = T::KG, XB = T::XB, NW = T::NW;
  constexpr int NSB = NS + XB;  // B slots: the NS stages' B parts, then XB B-only slots
  static_assert(KG == 1 || (EPI == EPI_LINEAR && !MX), "K groups: linear epilogues only");
  constexpr int kA = BM * kBK;               // A tile bytes per stage
  // MX: each stage also holds the E8M0 block scales of its K step: one dword (4 blocks of
  // 32) per tile row, A rows at kData + 4 r, B rows at kData + 1024 + 4 r (r < 256).
  constexpr int kData = (BM + BN) * kBK;
  constexpr int kStage = kData + (MX ? 2048 : 0);  // [A tile | B tile | scales]
  constexpr int DA = BM / (8 * NW), DB = BN / (8 * NW);  // 1 KB DMA blocks per wave per stage
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "whole 1 KB blocks per wave");
  constexpr int ND = DA + DB + (MX ? 2 : 0);  // loads per wave per stage
  constexpr int NM = FM * FN;                // MFMAs per sub-step
  constexpr int NH = 2 * (FM + FN);          // 16-byte fragment halves per sub-step
  static_assert(EPI != EPI_GEGLU || FN % 2 == 0 || (T::WN == 1 && BN % 16 == 0 && BN % 64 != 0),
                "GEGLU pairs gate and up sub-tiles: even FN, or one wave column whose gate "
                "and up halves are whole runs of 8 columns");
  static_assert(!(EPI == EPI_GEGLU && MX && FN % 2 != 0), "MX GEGLU: 32-column H blocks per tile");
  static_assert(!MX || (BM <= 256 && BN <= 256), "MX scale rows: one dword per lane");
  static_assert(!MX || NW == 4, "MX scale dwords: four waves of 64 rows");
  static_assert(KM == 0 || (NW == 8 && BM == 256 && BN == 256 && EPI == EPI_LINEAR && !MX),
                "K-major operands: eight-wave 256 x 256 linear tiles");
  constexpr bool AKM = (KM & 1) != 0, BKM = (KM & 2) != 0;
  static_assert(XB == 0 || (NS == 2 && KG == 1 && !MX), "extra B slots: two stages, one K group");
  constexpr int kStageOff = extra_lds<EPI>();  // GEGLU: the gelu table, then the stages
  constexpr int kB = BN * kBK;  // B tile bytes per stage
  static_assert((KG * NS * kStage + XB * kB + extra_lds<EPI>()) * T::OCC <= 160 * 1024,
                "LDS budget");
  __shared__ __attribute__((aligned(1024)))
  uint8_t smem[KG * NS * kStage + XB * kB + extra_lds<EPI>()];

  // Dequant scales: read at the start, so their latency hides behind the first loads.
  const float sa = MX ? 1.0f : *p.a_sinv;
  float sb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) sb[s] = MX ? 1.0f : s < p.n_seg ? p.b_sinv[s * p.b_stride] : 0.0f;
  float ag = 0.0f, au = 0.0f, hs = 0.0f;
  if constexpr (EPI == EPI_GEGLU) {
    ag = MX ? 1.0f : sa * p.b_sinv[0];
    au = MX ? 1.0f : sa * p.b_sinv[p.b_stride];
    if (!MX && p.h8) hs = *p.h8_scale;  // the quantization scale of H
  }

  int tm, tn, split, tail_slot;
  block_coords(p, tm, tn, split, tail_slot);
  const int m0 = tm * BM;
  const int n0 = tn * (EPI == EPI_GEGLU ? BN / 2 : BN);  // GEGLU: n0 indexes I

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int kg = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane(t / (NW * 64));  // K group
  const int wid = (t >> 6) & (NW - 1);    // wave within the group
  const int wm = wid % WM, wn = wid / WM;
  const int wave_m0 = wm * FM * 32;

  const int ksteps = (p.K + kBK - 1) / kBK;
  // whole tiles of a tail-split schedule run every K step
  const int kps = (p.tail_pieces > 0 && tail_slot < 0) ? ksteps : p.ksteps_per_split;
  const int kbeg = split * kps;
  const int nsteps = min(kps, ksteps - kbeg);  // >= 1 by construction
  // K group kg takes the split's steps kg, kg + KG, ...: its local step ls is global step
  // kbeg + kg + KG * ls; both groups run niters local steps (the group with one step fewer
  // runs a zero-filled last one), so their barriers pair up.
  const int niters = (nsteps + KG - 1) / KG;

  // K-major operands span K rows: rows past K read as zero through the buffer's size
  const i32x4 ra = make_srd(p.A, (uint32_t)((int64_t)(AKM ? p.K : p.M) * p.lda));
  const i32x4 rb = make_srd(p.B, (uint32_t)((int64_t)(BKM ? p.K : p.N) * p.ldb));

  static_assert(ND * (NS - 1) < 64, "vmcnt holds at most 63 outstanding loads");
  // DMA: lane l of the wave's j-th 1 KB block (block j*NW + wid of the tile) covers tile
  // row blk*8 + l/8, physical chunk l%8. Its logical chunk swz(row, l%8) only depends on
  // l and wid & 1 (= blk & 1, NW even), so one K mask serves every block of the lane.
  const int lrow = lane >> 3;
  const int lchunk = (lane & 7) ^ (((wid & 1) << 2) | (lrow >> 1));
  uint32_t a_off[DA], b_off[DB];
  // K-major: lane l of 1 KB block blk covers K row blk*4 + l/16 (of the step) and 16-byte
  // position l%16 of that row's 256 bytes, holding logical chunk (l%16) ^ kmaj_swz(row)
  const int kmrow = lane >> 4;
  auto kmaj_chunk = [&](int j) { return (lane & 15) ^ kmaj_swz((j * NW + wid) * 4 + kmrow); };
#pragma unroll
  for (int j = 0; j < DA; ++j) {
    if constexpr (AKM) {
      const int am = m0 + kmaj_chunk(j) * 16;  // M % 16 == 0: whole chunks in or out
      a_off[j] = am < p.M ? (uint32_t)((int64_t)((j * NW + wid) * 4 + kmrow) * p.lda + am)
                          : kOob;
    } else {
      const int am = m0 + (j * NW + wid) * 8 + lrow;
      a_off[j] = am < p.M ? (uint32_t)((int64_t)am * p.lda + lchunk * 16) : kOob;
    }
  }
#pragma unroll
  for (int j = 0; j < DB; ++j) {
    const int r = (j * NW + wid) * 8 + lrow;
    int bn;
    bool bvalid;
    if (EPI == EPI_GEGLU) {
      const int rr = r < BN / 2 ? r : r - BN / 2;
      bn = (r < BN / 2 ? 0 : p.I) + n0 + rr;
      bvalid = n0 + rr < p.I;
    } else {
      bn = n0 + r;
      bvalid = bn < p.N;
    }
    b_off[j] = bvalid ? (uint32_t)((int64_t)bn * p.ldb + lchunk * 16) : kOob;
    if constexpr (BKM) {
      const int bc = n0 + kmaj_chunk(j) * 16;  // N % 16 == 0: whole chunks in or out
      b_off[j] = bc < p.N ? (uint32_t)((int64_t)((j * NW + wid) * 4 + kmrow) * p.ldb + bc)
                          : kOob;
    }
  }
  // MX: lane l of wave w loads the scale dword of tile row w * 64 + l (A and B), from
  // the [rows, ld] E8M0 arrays; rows outside the tile or the tensor read as zero.
  i32x4 srd_sa = {0, 0, 0, 0}, srd_sb = {0, 0, 0, 0};
  uint32_t sa_off = kOob, sb_off = kOob;
  if constexpr (MX) {
    srd_sa = make_srd(p.a_sc, (uint32_t)((int64_t)p.M * p.a_sc_ld));
    srd_sb = make_srd(p.b_sc, (uint32_t)((int64_t)p.N * p.b_sc_ld));
    const int r = wid * 64 + lane;
    if (r < BM && m0 + r < p.M) sa_off = (uint32_t)((int64_t)(m0 + r) * p.a_sc_ld);
    if (r < BN) {
      int bn;
      bool bvalid;
      if (EPI == EPI_GEGLU) {
        const int rr = r < BN / 2 ? r : r - BN / 2;
        bn = (r < BN / 2 ? 0 : p.I) + n0 + rr;
        bvalid = n0 + rr < p.I;
      } else {
        bn = n0 + r;
        bvalid = bn < p.N;
      }
      if (bvalid) sb_off = (uint32_t)((int64_t)bn * p.b_sc_ld);
    }
  }
  // A partial last K step (K % 128 != 0) must read its chunks at or beyond K as zero.
  const bool lane_ktail_dead = (p.K % kBK) != 0 && (ksteps - 1) * kBK + lchunk * 16 >= p.K;

  // Load x of a stage (x < DA: A block x, DA <= x < DA + DB: B block x - DA, then (MX)
  // the A and B scale dwords). `kill` zero-fills this lane's data (a stage past the split,
  // or the lane's chunk beyond K in the tensor's partial last step), `kill_sc` a stage past
  // the split (the scales, and K-major operands, whose rows past K read as zero anyway).
  auto dma_load = [&](int x, uint8_t* stage, uint32_t k0, bool kill, bool kill_sc,
                      uint8_t* bdst) {
    const uint32_t base = lds_addr(stage);
    if (x < DA) {
      if constexpr (AKM)
        dma16(ra, base + (x * NW + wid) * 1024, kill_sc ? kOob : a_off[x], k0 * (uint32_t)p.lda);
      else
        dma16(ra, base + (x * NW + wid) * 1024, kill ? kOob : a_off[x], k0);
    } else if (x < DA + DB) {
      if constexpr (BKM)
        dma16(rb, lds_addr(bdst) + ((x - DA) * NW + wid) * 1024,
              kill_sc ? kOob : b_off[x - DA], k0 * (uint32_t)p.ldb);
      else
        dma16(rb, lds_addr(bdst) + ((x - DA) * NW + wid) * 1024, kill ? kOob : b_off[x - DA],
              k0);
    }
    else if (x == DA + DB)
      dma4(srd_sa, base + kData + wid * 256, kill_sc ? kOob : sa_off, k0 >> 5);
    else
      dma4(srd_sb, base + kData + 1024 + wid * 256, kill_sc ? kOob : sb_off, k0 >> 5);
  };
  // Stages past this split's last step are filled with zeros (never read); the partial
  // last K step of the tensor masks lanes beyond K. (ls: the group's local step.)
  auto kstep = [&](int ls) { return kg + KG * ls; };  // the split's step of local step ls
  auto gstep = [&](int ls) { return kbeg + kstep(ls); };  // the tensor's K step
  auto stage_kill = [&](int ls) {
    return kstep(ls) >= nsteps || (gstep(ls) == ksteps - 1 && lane_ktail_dead);
  };
  auto stage_ptr = [&](int ls) { return smem + kStageOff + (kg * NS + ls % NS) * kStage; };
  // the B tile of local step ls: the B part of a stage slot, or (XB) a B-only slot
  auto b_ptr = [&](int ls) {
    if constexpr (XB == 0) {
      return stage_ptr(ls) + kA;
    } else {
      const int slot = ls % NSB;
      return slot < NS ? smem + kStageOff + slot * kStage + kA
                       : smem + kStageOff + NS * kStage + (slot - NS) * kB;
    }
  };

  // B-tile row of each of the wave's n-subtiles; GEGLU puts gate rows in the first half
  // of the B tile and the matching up rows in the second (even FN: each wave takes its
  // share of both halves; odd FN: the one wave column takes every row in order).
  int brow[FN];
#pragma unroll
  for (int s = 0; s < FN; ++s) {
    if (EPI == EPI_GEGLU && FN % 2 == 0)
      brow[s] = (s < FN / 2 ? 0 : BN / 2) + wn * (FN / 2) * 32 + (s % (FN / 2)) * 32;
    else
      brow[s] = wn * FN * 32 + s * 32;
  }
  auto read_one = [&](Frags<NH>& f, const uint8_t* stage, const uint8_t* btile, int kk, int h) {
    const int fr = h >> 1;  // 0: b0, 1..FM: a0.., FM+1..: b1..
    if (fr == 0 || fr > FM) {
      const int r0 = brow[fr == 0 ? 0 : fr - FM];
      f.h[h] = BKM ? read_half_kmajor(btile, r0, kk, h & 1, lane)
                   : read_half(btile, r0, kk, h & 1, lane, MX);
    } else {
      const int r0 = wave_m0 + (fr - 1) * 32;
      f.h[h] = AKM ? read_half_kmajor(stage, r0, kk, h & 1, lane)
                   : read_half(stage, r0, kk, h & 1, lane, MX);
    }
  };

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // MFMA x of a sub-step: n-subtile x / FM, m-subtile x % FM.
  // MX scales of the current stage (per fragment: the row's four block scales, shifted
  // so that byte 2 kk holds block 2 kk + (lane >> 5)) and of the next one.
  uint32_t scA[MX ? FM : 1], scB[MX ? FN : 1], scA_n[MX ? FM : 1], scB_n[MX ? FN : 1];
  auto read_scales = [&](const uint8_t* stage, uint32_t* sa_, uint32_t* sb_)
      __attribute__((always_inline)) {
    if constexpr (MX) {
      const uint8_t* sc = stage + kData;
      const int sh = (lane >> 5) * 8;
#pragma unroll
      for (int j = 0; j < FM; ++j)
        sa_[j] = *reinterpret_cast<const uint32_t*>(sc + (wave_m0 + j * 32 + (lane & 31)) * 4) >> sh;
#pragma unroll
      for (int i = 0; i < FN; ++i)
        sb_[i] = *reinterpret_cast<const uint32_t*>(sc + 1024 + (brow[i] + (lane & 31)) * 4) >> sh;
    }
  };
  auto mma_one = [&](const Frags<NH>& f, int x, auto kk_tag) __attribute__((always_inline)) {
    constexpr int kk = decltype(kk_tag)::value;
    const int i = x / FM, j = x % FM;
    const int hb = i == 0 ? 0 : 2 * (FM + i);
    const int ha = 2 * (1 + j);
    if constexpr (MX)
      acc[i][j] = mfma_mx<FB, FA, 2 * kk>(join(f.h[hb], f.h[hb + 1]), join(f.h[ha], f.h[ha + 1]),
                                         acc[i][j], scB[i], scA[j]);
    else
      acc[i][j] = mfma<FB, FA>(join(f.h[hb], f.h[hb + 1]), join(f.h[ha], f.h[ha + 1]), acc[i][j]);
  };

  // Pipeline (NS LDS stages, 2 MFMA sub-steps of 64 K-bytes per stage). Step ls:
  //   NM x {MFMA(ls, kk=0), reads of frags(ls, kk=1)} | wait DMA(ls+1) + barrier |
  //   NM x {MFMA(ls, kk=1), reads of frags(ls+1, kk=0), DMA loads of stage ls+NS}
  // Each MFMA consumes operands read one sub-step earlier; stage ls+NS goes into the slot
  // of stage ls, which the barrier has just released, and has about NS-1 steps to land;
  // LDS reads and texture-unit loads sit between consecutive MFMAs, so neither unit
  // (both shared by the four waves) blocks MFMA issue. sched_barrier(0) pins the order.
  // The last NS steps load nothing (their stages would lie past the split's end); their
  // mid-step wait drains every load instead (the next stage is then the last one issued,
  // or none: the trailing fragment reads of the final step go to a stale slot and are
  // never used). Prologue stages past the end are zero-filled.
  if constexpr (EPI == EPI_GEGLU) {
    // the fp32 gelu table (26 KB) into LDS ahead of the stage loads, so the prologue's wait
    // for stage 0 also covers it; wave w copies KB w, w + NW, .., below 26
    static_assert(kGeluA32Bytes == 26 * 1024, "gelu table copy assumes 26 KB");
    const i32x4 rt = make_srd(kGeluA32, (uint32_t)kGeluA32Bytes);
    const uint32_t tab = lds_addr(smem);
#pragma unroll
    for (int c = 0; c < (26 + NW - 1) / NW; ++c)
      if (wid + NW * c < 26) dma16(rt, tab + (wid + NW * c) * 1024, lane * 16, (wid + NW * c) * 1024);
  }
#pragma unroll
  for (int ls = 0; ls < NS; ++ls) {
#pragma unroll
    for (int x = 0; x < ND; ++x)
      dma_load(x, stage_ptr(ls), (uint32_t)gstep(ls) * kBK, stage_kill(ls),
               kstep(ls) >= nsteps, b_ptr(ls));
  }
  // (XB) the B tiles of steps NS .. NSB-1
#pragma unroll
  for (int ls = NS; ls < NSB; ++ls) {
#pragma unroll
    for (int x = DA; x < DA + DB; ++x)
      dma_load(x, stage_ptr(ls), (uint32_t)gstep(ls) * kBK, stage_kill(ls), kstep(ls) >= nsteps,
               b_ptr(ls));
  }
  // stage 0 landed: the NS-1 later stages (ND loads each) and the XB B tiles may still be
  // in flight
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(ND * (NS - 1) + DB * XB) : "memory");
  __syncthreads();
  Frags<NH> f0, f1;
  // same read order as the loop's second half, so that the wait counts at the loop header
  // agree on both incoming paths
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    read_one(f0, stage_ptr(0), b_ptr(0), 0, h);
    __builtin_amdgcn_sched_barrier(0);
  }
  read_scales(stage_ptr(0), scA, scB);
  auto step = [&](auto with_dma, int ls) __attribute__((always_inline)) {
    constexpr bool kDma = decltype(with_dma)::value;
    uint8_t* cur = stage_ptr(ls);
    uint8_t* nxt = stage_ptr(ls + 1);
    uint8_t* curb = b_ptr(ls);
    uint8_t* nxtb = b_ptr(ls + 1);
    __builtin_amdgcn_sched_barrier(0);
    // the first half's reads sit between its first NR MFMAs, so that they have landed
    // (their wait precedes the barrier) while the last MFMAs still run
    constexpr int NR = NM >= 8 ? NM - NM / 4 : NM;
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      mma_one(f0, x, std::integral_constant<int, 0>{});
#pragma unroll
      for (int h = x * NH / NR; h < (x + 1) * NH / NR && h < NH; ++h)
        read_one(f1, cur, curb, 1, h);
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage ls+1 landed (stages ls+2 .. ls+NS-1 may still be in flight; with XB, each
    // step's loads are A of step ls+NS then B of step ls+NSB, so the B tile of step ls+2
    // issued after A of ls+1 may be too)
    if constexpr (kDma)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(ND * (NS - 2) + DB * XB) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t kn = (uint32_t)gstep(ls + NS) * kBK;
    const bool killn = stage_kill(ls + NS);
    const bool killn_sc = kstep(ls + NS) >= nsteps;
    const uint32_t knb = (uint32_t)gstep(ls + NSB) * kBK;  // = kn without XB
    const bool killnb = stage_kill(ls + NSB);
    const bool killnb_end = kstep(ls + NSB) >= nsteps;
    read_scales(nxt, scA_n, scB_n);
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      mma_one(f1, x, std::integral_constant<int, 1>{});
#pragma unroll
      for (int h = x * NH / NM; h < (x + 1) * NH / NM; ++h) read_one(f0, nxt, nxtb, 0, h);
      if constexpr (kDma) {
#pragma unroll
        for (int d = x * ND / NM; d < (x + 1) * ND / NM; ++d) {
          if (XB == 0 || d < DA)
            dma_load(d, cur, kn, killn, killn_sc, curb);
          else
            dma_load(d, cur, knb, killnb, killnb_end, curb);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MX) {
#pragma unroll
      for (int j = 0; j < FM; ++j) scA[j] = scA_n[j];
#pragma unroll
      for (int i = 0; i < FN; ++i) scB[i] = scB_n[i];
    }
  };
  int ls = 0;
  for (; ls < niters - NS; ++ls) step(std::true_type{}, ls);
  for (; ls < niters; ++ls) step(std::false_type{}, ls);
  // Let every wave finish with the stages before the epilogue reuses the space.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if constexpr (KG == 2) {
    // group 1 hands its accumulators to group 0 through LDS (wave w of each group holds the
    // same output sub-tile; lane-major dwords, so the 64 lanes of a store hit 64 banks),
    // then leaves; group 0 adds them and runs the epilogue alone
    constexpr int kAccBytes = FN * FM * 16 * 64 * 4;  // one wave's accumulators
    static_assert(4 * kAccBytes <= KG * NS * kStage, "accumulator exchange fits the ring");
    float* xbuf = reinterpret_cast<float*>(smem + wid * kAccBytes);
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) xbuf[((i * FM + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] += xbuf[((i * FM + j) * 16 + e) * 64 + lane];
    // the epilogue's staging may overwrite other waves' exchange regions: wait for all of
    // group 0 (a barrier among its four waves; group 1 has left)
    __syncthreads();
  }

  // ---- epilogue --------------------------------------------------------------------
  if constexpr (EPI == EPI_LINEAR) {
    if (tail_slot >= 0) {
      // a K piece of a tail-split tile: raw fp32 sums of the whole BM x BN tile (rows and
      // columns past the tensor hold zeros), reduced with the other pieces later
      float* base = p.tail_ws + (int64_t)tail_slot * (BM * BN);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const int m = wave_m0 + j * 32 + (lane & 31);
            const int n = wn * FN * 32 + i * 32 + 8 * q + (lane >> 5) * 4;
            *reinterpret_cast<float4*>(base + m * BN + n) =
                make_float4(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                            acc[i][j][4 * q + 3]);
          }
      return;
    }
  }
  // acc[i][j][r]: n-subtile i, m-subtile j; row m = wave_m0 + j*32 + (lane & 31) of the
  // tile, column (within the n-subtile) 8*(r/4) + (lane >> 5)*4 + (r & 3): each lane
  // holds runs of four consecutive columns. bf16 results are staged through this wave's
  // own LDS region of the (now idle) pipeline ring and leave as 16-byte row segments.
  constexpr int ROWS = FM * 32;  // rows of the wave's output tile
  const int lrow_m = lane & 31;
  const int lcol = (lane >> 5) * 4;
  // Axiswise scales (a_vec / b_vec): the factor of element (m, n) is a_sinv[m] * b_sinv[n]
  // (either side a single value when its flag is 0), read here from global memory. Every
  // output is fma(acc, factor, bias) with one rounding, written out explicitly so that the
  // bf16 and fp32 outputs round alike (bf16 = RNE of the fp32 result).
  const bool vec = EPI == EPI_LINEAR && (p.a_vec | p.b_vec);
  float rsa[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wave_m0 + j * 32 + lrow_m;
    rsa[j] = (vec && p.a_vec) ? p.a_sinv[m < p.M ? m : p.M - 1] : sa;
  }
  auto col_factors = [&](int n, float alpha, float* cf) __attribute__((always_inline)) {
    if (vec && p.b_vec && n < p.N) {
      const float4 f = *reinterpret_cast<const float4*>(p.b_sinv + n);
      cf[0] = f.x; cf[1] = f.y; cf[2] = f.z; cf[3] = f.w;
    } else {
      const float b = vec ? (p.b_vec ? 0.0f : sb[0]) : alpha;
      cf[0] = b; cf[1] = b; cf[2] = b; cf[3] = b;
    }
  };
  if constexpr (EPI == EPI_LINEAR && OUT == BF8_OUT_BF16) {
    constexpr int CH = FN * 4;  // 16-byte chunks per staged row (FN*32 bf16)
    static_assert(NW * ROWS * CH * 16 <= NS * kStage, "per-wave staging fits the ring");
    uint8_t* wbuf = smem + wid * (ROWS * CH * 16);
    const int wave_n0 = n0 + wn * FN * 32;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = i * 32 + 8 * q + lcol;  // within the wave's columns
        const int n = wave_n0 + col;
        int seg = 0;
#pragma unroll
        for (int s2 = 0; s2 < 3; ++s2) seg += (s2 + 1 < p.n_seg && n >= p.seg_end[s2]) ? 1 : 0;
        const float alpha = sa * (seg == 0 ? sb[0] : seg == 1 ? sb[1] : seg == 2 ? sb[2] : sb[3]);
        float bias[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias && n < p.N) {
          const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + n);
          bias[0] = bf16_lo(bb.x); bias[1] = bf16_hi(bb.x);
          bias[2] = bf16_lo(bb.y); bias[3] = bf16_hi(bb.y);
        }
        if (vec) {
          float cf[4];
          col_factors(n, alpha, cf);
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            uint2 w;
            w.x = pack_bf16x2(__builtin_fmaf(acc[i][j][4 * q + 0], rsa[j] * cf[0], bias[0]),
                              __builtin_fmaf(acc[i][j][4 * q + 1], rsa[j] * cf[1], bias[1]));
            w.y = pack_bf16x2(__builtin_fmaf(acc[i][j][4 * q + 2], rsa[j] * cf[2], bias[2]),
                              __builtin_fmaf(acc[i][j][4 * q + 3], rsa[j] * cf[3], bias[3]));
            stage_put<CH>(wbuf, j * 32 + lrow_m, col, w);
          }
          continue;
        }
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          uint2 w;
          w.x = pack_bf16x2(__builtin_fmaf(acc[i][j][4 * q + 0], alpha, bias[0]),
                            __builtin_fmaf(acc[i][j][4 * q + 1], alpha, bias[1]));
          w.y = pack_bf16x2(__builtin_fmaf(acc[i][j][4 * q + 2], alpha, bias[2]),
                            __builtin_fmaf(acc[i][j][4 * q + 3], alpha, bias[3]));
          stage_put<CH>(wbuf, j * 32 + lrow_m, col, w);
        }
      }
    }
#pragma unroll 4
    for (int it = 0; it < ROWS * CH / 64; ++it) {
      const int idx = it * 64 + lane;
      const int row = idx / CH, c = idx % CH;
      const uint4 d = stage_get<CH>(wbuf, row, c);
      const int gm = m0 + wave_m0 + row;
      const int gn = wave_n0 + c * 8;
      if (gm < p.M && gn < p.N)
        store_bf16x8(reinterpret_cast<uint16_t*>(p.C) + (int64_t)gm * p.ldc + gn, d, p.ldc);
    }
  } else if constexpr (EPI == EPI_LINEAR) {
    // fp32 out; with a K split, raw partial sums into this split's slice of C
    const bool raw = p.splits > 1;
    float* cbase = reinterpret_cast<float*>(p.C) + (raw ? split * p.split_stride : 0);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * FN * 32 + i * 32 + 8 * q + lcol;
        if (n >= p.N) continue;
        int seg = 0;
#pragma unroll
        for (int s2 = 0; s2 < 3; ++s2) seg += (s2 + 1 < p.n_seg && n >= p.seg_end[s2]) ? 1 : 0;
        const float alpha =
            raw ? 1.0f : sa * (seg == 0 ? sb[0] : seg == 1 ? sb[1] : seg == 2 ? sb[2] : sb[3]);
        float bias[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias && !raw) {
          const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + n);
          bias[0] = bf16_lo(bb.x); bias[1] = bf16_hi(bb.x);
          bias[2] = bf16_lo(bb.y); bias[3] = bf16_hi(bb.y);
        }
        if (vec && !raw) {
          float cf[4];
          col_factors(n, alpha, cf);
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const int m = m0 + wave_m0 + j * 32 + lrow_m;
            if (m >= p.M) continue;
            float* c = cbase + (int64_t)m * p.ldc + n;
            *reinterpret_cast<float4*>(c) = make_float4(
                __builtin_fmaf(acc[i][j][4 * q + 0], rsa[j] * cf[0], bias[0]),
                __builtin_fmaf(acc[i][j][4 * q + 1], rsa[j] * cf[1], bias[1]),
                __builtin_fmaf(acc[i][j][4 * q + 2], rsa[j] * cf[2], bias[2]),
                __builtin_fmaf(acc[i][j][4 * q + 3], rsa[j] * cf[3], bias[3]));
          }
          continue;
        }
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const int m = m0 + wave_m0 + j * 32 + lrow_m;
          if (m >= p.M) continue;
          float* c = cbase + (int64_t)m * p.ldc + n;
          *reinterpret_cast<float4*>(c) =
              make_float4(__builtin_fmaf(acc[i][j][4 * q + 0], alpha, bias[0]),
                          __builtin_fmaf(acc[i][j][4 * q + 1], alpha, bias[1]),
                          __builtin_fmaf(acc[i][j][4 * q + 2], alpha, bias[2]),
                          __builtin_fmaf(acc[i][j][4 * q + 3], alpha, bias[3]));
        }
      }
    }
  } else {
    // Gated GELU: each run of 8 H columns pairs a gate quad with its up quad in the same
    // lane (GegluRuns). The wave owns H rows wave_m0 .. +ROWS and RUNS*8 columns of this
    // tile. Pass 0 stages H (and accumulates its amax); passes 1, 2 stage the bf16 gate /
    // up pre-activations when the caller keeps them for the backward.
    using Runs = GegluRuns<FN, BN>;
    constexpr int RUNS = Runs::kRuns;
    constexpr int CH = RUNS;  // 16-byte chunks per staged H row (8 bf16 per run)
    static_assert(NW * ROWS * CH * 16 <= NS * kStage, "per-wave staging fits the ring");
    uint8_t* wbuf = smem + kStageOff + wid * (ROWS * CH * 16);
    const int wave_h0 = n0 + wn * RUNS * 8;
    uint32_t hkeys = 0;  // packed max of the |H| bf16 keys staged by this lane
    uint32_t hmax = 0;   // the same as one fp32-bit amax key
    auto run_pass = [&](auto pass_tag) {
      constexpr int pass = decltype(pass_tag)::value;
      static_for<RUNS>([&](auto k_tag) __attribute__((always_inline)) {
        constexpr int k = decltype(k_tag)::value;
        constexpr int gs = Runs::gate_s(k), gq = Runs::gate_q(k);
        constexpr int us = Runs::up_s(k), uq = Runs::up_q(k);
        const int col = 8 * k + lcol;
        if constexpr (pass == 0) {
          // H of the run's FM rows: bf16 g, u pairs first, then all 4 FM gelu table reads
          // (independent LDS reads in flight together), then the products. Gates outside
          // the table (|g| < 2^-16 or >= 8, rare) and NaN products (from non-finite u)
          // take a wave-uniform slow path.
          uint32_t gw[2 * FM], uw[2 * FM], ad[2 * FM], ta[4 * FM], w[2 * FM];
          uint32_t outside = 0;
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            gw[2 * j] = pack_bf16x2(acc[gs][j][4 * gq] * ag, acc[gs][j][4 * gq + 1] * ag);
            gw[2 * j + 1] = pack_bf16x2(acc[gs][j][4 * gq + 2] * ag, acc[gs][j][4 * gq + 3] * ag);
            uw[2 * j] = pack_bf16x2(acc[us][j][4 * uq] * au, acc[us][j][4 * uq + 1] * au);
            uw[2 * j + 1] = pack_bf16x2(acc[us][j][4 * uq + 2] * au, acc[us][j][4 * uq + 3] * au);
          }
          // gelu(g) as fp32 from the table at LDS offset 0 (byte offsets in packed halves)
#pragma unroll
          for (int x = 0; x < 2 * FM; ++x) ad[x] = gelu_addr32x2(gw[x], outside);
#pragma unroll
          for (int x = 0; x < 2 * FM; ++x) {
            ta[2 * x] = *reinterpret_cast<const uint32_t*>(smem + (ad[x] & 0xFFFFu));
            ta[2 * x + 1] = *reinterpret_cast<const uint32_t*>(smem + (ad[x] >> 16));
          }
          if (__builtin_expect(__any(outside != 0), 0)) {
#pragma unroll
            for (int x = 0; x < 2 * FM; ++x) {
              ta[2 * x] = gelu_finish(gw[x], ta[2 * x] >> 16) << 16;
              ta[2 * x + 1] = gelu_finish(gw[x] >> 16, ta[2 * x + 1] >> 16) << 16;
            }
          }
          uint32_t bk = 0;  // packed max of the |h| keys of the run
#pragma unroll
          for (int x = 0; x < 2 * FM; ++x) {
            w[x] = pack_bf16x2(__uint_as_float(ta[2 * x]) * bf16_lo(uw[x]),
                               __uint_as_float(ta[2 * x + 1]) * bf16_hi(uw[x]));
            bk = pk_max_u16(bk, w[x] & 0x7FFF7FFFu);
          }
          if (__builtin_expect(__any(nan_key2(bk)), 0)) {
#pragma unroll
            for (int x = 0; x < 2 * FM; ++x) w[x] = nan_ffff_bf16x2(w[x]);
          }
          hkeys = pk_max_u16(hkeys, bk);
#pragma unroll
          for (int j = 0; j < FM; ++j)
            stage_put<CH>(wbuf, j * 32 + lrow_m, col, make_uint2(w[2 * j], w[2 * j + 1]));
        } else {
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            uint32_t w0, w1;  // packed bf16 pairs (columns 0-1, 2-3 of the run)
            if constexpr (pass == 1) {
              w0 = pack_bf16x2(acc[gs][j][4 * gq] * ag, acc[gs][j][4 * gq + 1] * ag);
              w1 = pack_bf16x2(acc[gs][j][4 * gq + 2] * ag, acc[gs][j][4 * gq + 3] * ag);
            } else {
              w0 = pack_bf16x2(acc[us][j][4 * uq] * au, acc[us][j][4 * uq + 1] * au);
              w1 = pack_bf16x2(acc[us][j][4 * uq + 2] * au, acc[us][j][4 * uq + 3] * au);
            }
            stage_put<CH>(wbuf, j * 32 + lrow_m, col, make_uint2(w0, w1));
          }
        }
      });
      if constexpr (pass == 0) hmax = max(hkeys << 16, hkeys & 0xFFFF0000u);
      if constexpr (pass == 0) {
        if (p.h8) {
          // every value this wave quantizes is one it staged: with none of them inf or NaN
          // (and a finite scale) no product can be NaN, so the NaN patch is skipped
          const bool finite = !__any(hmax >= 0x7F800000u) && (MX || hs < INFINITY);
          if constexpr (MX) {
            if (finite)
              mx_h_epilogue<ROWS, CH, true>(p, wbuf, lane, m0 + wave_m0, wave_h0);
            else
              mx_h_epilogue<ROWS, CH, false>(p, wbuf, lane, m0 + wave_m0, wave_h0);
          } else {
            if (finite)
              scaled_h_epilogue<ROWS, CH, true>(p, wbuf, lane, m0 + wave_m0, wave_h0, hs);
            else
              scaled_h_epilogue<ROWS, CH, false>(p, wbuf, lane, m0 + wave_m0, wave_h0, hs);
          }
          return;
        }
      }
      uint16_t* dst = pass == 0 ? reinterpret_cast<uint16_t*>(p.C) : p.GU;
      const int64_t ld = pass == 0 ? p.ldc : 2 * (int64_t)p.I;
      const int coff = pass == 2 ? p.I : 0;
#pragma unroll 4
      for (int it = 0; it < ROWS * CH / 64; ++it) {
        const int idx = it * 64 + lane;
        const int row = idx / CH, c = idx % CH;
        const uint4 d = stage_get<CH>(wbuf, row, c);
        const int gm = m0 + wave_m0 + row;
        if (gm < p.M) store_bf16x8(dst + (int64_t)gm * ld + coff + wave_h0 + c * 8, d, ld);
      }
    };
    // Eight-wave tiles store the pre-activations kept for the backward first, so their
    // stores drain while the wave computes and stages H (c5's gate/up kernel with GU:
    // 408 -> 397 us alone). Tiles with 256 accumulators a lane keep H first: the other
    // order spills 60 more bytes per lane there.
    if constexpr (NW == 8) {
      if (p.GU) {
        run_pass(std::integral_constant<int, 1>{});
        run_pass(std::integral_constant<int, 2>{});
      }
      run_pass(std::integral_constant<int, 0>{});
    } else {
      run_pass(std::integral_constant<int, 0>{});
      if (p.GU) {
        run_pass(std::integral_constant<int, 1>{});
        run_pass(std::integral_constant<int, 2>{});
      }
    }
    hmax = block_max_u32<tile_threads<T>()>(hmax);
    if (t == 0 && p.partials) p.partials[blockIdx.x] = hmax;
  }
}

// Workgroups of a launch: one per tile and K split, or for a tail-split schedule the whole
// tiles plus the tail tiles' pieces.
inline unsigned grid_blocks(const GemmParams& p) {
  const int ntiles = p.tiles_m * p.tiles_n;
  if (p.tail_pieces > 0) return (unsigned)(p.full_tiles + (ntiles - p.full_tiles) * p.tail_pieces);
  return (unsigned)(ntiles * p.splits);
}

template <class T, int EPI, int OUT>
int launch_typed(const GemmParams& p, int fa, int fb, hipStream_t s) {
  const dim3 grid(grid_blocks(p)), block(tile_threads<T>());
  if (p.kmajor) {
    // K-major operands (the training backward's dgrad and wgrad GEMMs: e5m2 gradients
    // against e4m3 weights or activations) on the eight-wave 256 x 256 tiles
    if constexpr (EPI == EPI_LINEAR && T::NW == 8 && T::BM == 256 && T::BN == 256) {
      if (fa == BF8_E5M2 && fb == BF8_E4M3 && (p.kmajor == 2 || p.kmajor == 3)) {
        if (p.kmajor == 2)
          hipLaunchKernelGGL((gemm_kernel<T, 1, 0, EPI, OUT, false, 2>), grid, block, 0, s, p);
        else
          hipLaunchKernelGGL((gemm_kernel<T, 1, 0, EPI, OUT, false, 3>), grid, block, 0, s, p);
        return launch_status("gemm_kernel(k-major)");
      }
    }
    set_error("gemm: K-major operands (layout %d) need e5m2 x e4m3 on an eight-wave 256x256 "
              "tile (got %d x %d, %dx%d)", p.kmajor, fa, fb, T::BM, T::BN);
    return BF8_EINVAL;
  }
  if (fa == kFmtBf16 || fb == kFmtBf16) {
    if constexpr (EPI == EPI_LINEAR) {
      if (fa == kFmtBf16 && fb == kFmtBf16) {
        hipLaunchKernelGGL((gemm_kernel<T, kFmtBf16, kFmtBf16, EPI, OUT>), grid, block, 0, s, p);
        return launch_status("gemm_kernel(bf16)");
      }
    }
    set_error("gemm: bf16 operands need a bf16 partner and a linear epilogue");
    return BF8_EINVAL;
  }
  if (fa == BF8_E4M3 && fb == BF8_E4M3)
    hipLaunchKernelGGL((gemm_kernel<T, 0, 0, EPI, OUT>), grid, block, 0, s, p);
  else if (fa == BF8_E5M2 && fb == BF8_E4M3)
    hipLaunchKernelGGL((gemm_kernel<T, 1, 0, EPI, OUT>), grid, block, 0, s, p);
  else if (fa == BF8_E4M3 && fb == BF8_E5M2)
    hipLaunchKernelGGL((gemm_kernel<T, 0, 1, EPI, OUT>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<T, 1, 1, EPI, OUT>), grid, block, 0, s, p);
  return launch_status("gemm_kernel");
}

}  // namespace

// The tile T with one stage fewer when the variant's stages (MX: + 2 KB of scale dwords
// each) and its extra LDS (the gelu table of the GEGLU epilogue) would overflow the LDS.
// A gated-GELU tile cut to two stages keeps a third slot for B tiles alone when it fits
// (the 256x160 tile of skinny gate/up GEMMs, whose B rows stream from HBM: B then loads
// two steps ahead).
template <class T, int EPI, bool MX>
struct FitTile {
  static constexpr int bytes(int ns, int xb = 0) {
    return (ns * ((T::BM + T::BN) * kBK + (MX ? 2048 : 0)) + xb * T::BN * kBK +
            extra_lds<EPI>()) * T::OCC;
  }
  // 256 bytes stay free for the epilogue's block reductions
  static constexpr int kLimit = 160 * 1024 - 256;
  static constexpr bool kCut = bytes(T::NS) > kLimit;
  static constexpr int kXB = (kCut && EPI == EPI_GEGLU && !MX && T::NS - 1 == 2 && T::KG == 1 &&
                              bytes(T::NS - 1, 1) <= kLimit) ? 1 : 0;
  using type = std::conditional_t<!kCut, T,
                                  GemmTile<T::WM, T::WN, T::FM, T::FN, T::NS - 1, T::OCC, T::KG,
                                           kXB>>;
  static_assert(bytes(type::NS, type::XB) <= kLimit, "stages do not fit the LDS");
};

template <class T>
int launch_gemm_tile(const GemmParams& p, int epi, int out_dtype, int fmt_a, int fmt_b,
                     hipStream_t stream, bool mx) {
  const dim3 grid(grid_blocks(p)), block(tile_threads<T>());
  if constexpr (T::XB > 0) {
    // a tile that already fills the LDS with its extra B slot: linear, non-MX only
    if (epi == EPI_GEGLU || mx) {
      set_error("gemm: tile %dx%d with an extra B slot has linear non-MX epilogues only",
                T::BM, T::BN);
      return BF8_EINVAL;
    }
    if (out_dtype == BF8_OUT_BF16)
      return launch_typed<T, EPI_LINEAR, BF8_OUT_BF16>(p, fmt_a, fmt_b, stream);
    return launch_typed<T, EPI_LINEAR, BF8_OUT_F32>(p, fmt_a, fmt_b, stream);
  } else if constexpr (T::KG != 1) {
    if (epi == EPI_GEGLU || mx) {
      set_error("gemm: tile %dx%d with two K groups has linear non-MX epilogues only", T::BM,
                T::BN);
      return BF8_EINVAL;
    }
    if (out_dtype == BF8_OUT_BF16)
      return launch_typed<T, EPI_LINEAR, BF8_OUT_BF16>(p, fmt_a, fmt_b, stream);
    return launch_typed<T, EPI_LINEAR, BF8_OUT_F32>(p, fmt_a, fmt_b, stream);
  } else {
  if (epi == EPI_GEGLU) {
    if constexpr (T::FN % 2 == 0) {
      if (mx) {
        if constexpr (T::NW == 4) {
          using TG = typename FitTile<T, EPI_GEGLU, true>::type;
          hipLaunchKernelGGL((gemm_kernel<TG, 0, 0, EPI_GEGLU, BF8_OUT_BF16, true>), grid, block,
                             0, stream, p);
          return launch_status("gemm_kernel(geglu, mx)");
        } else {
          set_error("gemm: tile %dx%d with %d waves has no MX variant", T::BM, T::BN, T::NW);
          return BF8_EINVAL;
        }
      }
      using TG = typename FitTile<T, EPI_GEGLU, false>::type;
      if (fmt_a == kFmtBf16 && fmt_b == kFmtBf16) {
        // bf16 operands (NVFP4's exactly dequantized ones): the same epilogue on the sums
        hipLaunchKernelGGL((gemm_kernel<TG, kFmtBf16, kFmtBf16, EPI_GEGLU, BF8_OUT_BF16>), grid,
                           block, 0, stream, p);
        return launch_status("gemm_kernel(geglu, bf16)");
      }
      hipLaunchKernelGGL((gemm_kernel<TG, 0, 0, EPI_GEGLU, BF8_OUT_BF16>), grid, block, 0, stream, p);
      return launch_status("gemm_kernel(geglu)");
    } else if constexpr (T::WN == 1 && T::BN % 16 == 0 && T::BN % 64 != 0) {
      // one wave column, gate and up halves of BN/2 columns: tensor-scaled only (the MX H
      // blocks of 32 columns would straddle tiles)
      if (mx) {
        set_error("gemm: tile %dx%d has no MX gated-GELU variant", T::BM, T::BN);
        return BF8_EINVAL;
      }
      using TG = typename FitTile<T, EPI_GEGLU, false>::type;
      if (fmt_a == kFmtBf16 && fmt_b == kFmtBf16) {
        hipLaunchKernelGGL((gemm_kernel<TG, kFmtBf16, kFmtBf16, EPI_GEGLU, BF8_OUT_BF16>), grid,
                           block, 0, stream, p);
        return launch_status("gemm_kernel(geglu, bf16)");
      }
      hipLaunchKernelGGL((gemm_kernel<TG, 0, 0, EPI_GEGLU, BF8_OUT_BF16>), grid, block, 0, stream, p);
      return launch_status("gemm_kernel(geglu)");
    } else {
      set_error("gemm: tile %dx%d has no gated-GELU variant", T::BM, T::BN);
      return BF8_EINVAL;
    }
  }
  if (mx) {
    if constexpr (T::NW == 4) {
      // MX block scales (e4m3 operands): each stage also holds 2 KB of scale dwords
      using TM = typename FitTile<T, EPI_LINEAR, true>::type;
      if (out_dtype == BF8_OUT_BF16)
        hipLaunchKernelGGL((gemm_kernel<TM, 0, 0, EPI_LINEAR, BF8_OUT_BF16, true>), grid, block,
                           0, stream, p);
      else
        hipLaunchKernelGGL((gemm_kernel<TM, 0, 0, EPI_LINEAR, BF8_OUT_F32, true>), grid, block,
                           0, stream, p);
      return launch_status("gemm_kernel(mx)");
    } else {
      set_error("gemm: tile %dx%d with %d waves has no MX variant", T::BM, T::BN, T::NW);
      return BF8_EINVAL;
    }
  }
  if (out_dtype == BF8_OUT_BF16) return launch_typed<T, EPI_LINEAR, BF8_OUT_BF16>(p, fmt_a, fmt_b, stream);
  return launch_typed<T, EPI_LINEAR, BF8_OUT_F32>(p, fmt_a, fmt_b, stream);
  }
}

}  // namespace bf8
