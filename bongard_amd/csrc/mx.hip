// MXFP8 quantization (OCP microscaling: blocks of 32 elements sharing one E8M0 scale) for
// gfx950, the arithmetic of TransformerEngine's MXFP8BlockScaling recipe (TE 2.19.0, the
// recipe named at bongard/te_linear.py:17,38-39 and bongard/fused_mlp.py:9,31-33).
//
// Per block of 32 bf16 values (along a row for the rowwise copy, along a column for the
// columnwise copy):
//   amax = max |x| (NaN-propagating), val = fp32(amax * fp32(1 / fp8_max)),
//   e    = E8M0 of val rounded up to a power of two (ceil; 0xFE at most; NaN -> 0xFF),
//   q    = fp8(clamp(f32(x) * 2^(127 - e), +-fp8_max)),
// so that the block's largest magnitude lands in (fp8_max / 2, fp8_max] and x ~ q * 2^(e-127).
// Scales are stored one byte per block, rows of bf8_mx_scale_ld(K) bytes (a multiple of 4;
// the bytes past the last block hold 127 = 1.0 so that the GEMM can read whole dwords).
// The columnwise copy is stored transposed ([cols, rows], blocks along rows of x), the
// K-contiguous operand layout of the TN GEMM.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"

namespace bf8 {
namespace {

constexpr int kMxNT = 256;
constexpr int kMxMaxRowBlocks = 8192;
constexpr int kMT = 64;                // columnwise tile (rows x cols)
constexpr int kMPitch = kMT + 4;
constexpr int kMaxMxTileBlocks = 2048;
// Rowwise: a 16-lane group handles 128 consecutive elements of a row (4 blocks, 4 lanes
// each, 8 elements per lane) and writes the dword of their 4 scale bytes. Grid-stride over
// (row, 128-element group) pairs; groups past the row's last block write padding scales.
// (Block blk of the nblk blocks that quantize x.)
template <int FMT>
__device__ __forceinline__ void mx_row_body(const uint16_t* __restrict__ x, int64_t rows,
                                            int64_t cols, uint8_t* __restrict__ out,
                                            uint8_t* __restrict__ sc, int64_t ld_sc,
                                            int64_t blk, int64_t nblk) {
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;                 // lane within the 16-lane group
  const int64_t groups_per_row = ld_sc / 4;  // dwords of scales per row
  const int64_t ngroups = rows * groups_per_row;
  const int64_t gstride = nblk * (kMxNT / 16);
  for (int64_t g = blk * (kMxNT / 16) + (threadIdx.x >> 4); g < ngroups; g += gstride) {
    const int64_t r = g / groups_per_row, cg = g % groups_per_row;
    const int64_t c = cg * 128 + sub * 8;
    const bool valid = c < cols;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (valid) v = *reinterpret_cast<const uint4*>(x + r * cols + c);
    uint32_t m = absmax_key8(v);
    m = max(m, (uint32_t)__shfl_xor((int)m, 1, 64));
    m = max(m, (uint32_t)__shfl_xor((int)m, 2, 64));
    const bool block_valid = valid;  // cols % 32 == 0: a block is valid iff its lanes are
    const uint32_t e = block_valid ? mx_exponent<FMT>(m) : kMxPadScale;
    if (valid) {
      const float mult = mx_multiplier(e);
      *reinterpret_cast<uint2*>(out + r * cols + c) = quant8_bf16<FMT>(v, mult);
    }
    // gather the 4 block exponents of the group (lanes 0, 4, 8, 12 of the group)
    const int base = lane & ~15;
    const uint32_t e0 = (uint32_t)__shfl((int)e, base + 0, 64);
    const uint32_t e1 = (uint32_t)__shfl((int)e, base + 4, 64);
    const uint32_t e2 = (uint32_t)__shfl((int)e, base + 8, 64);
    const uint32_t e3 = (uint32_t)__shfl((int)e, base + 12, 64);
    if (sub == 0)
      *reinterpret_cast<uint32_t*>(sc + r * ld_sc + cg * 4) = e0 | (e1 << 8) | (e2 << 16) | (e3 << 24);
  }
}

template <int FMT>
__global__ __launch_bounds__(kMxNT) void mx_row_kernel(const uint16_t* __restrict__ x,
                                                       int64_t rows, int64_t cols,
                                                       uint8_t* __restrict__ out,
                                                       uint8_t* __restrict__ sc, int64_t ld_sc) {
  mx_row_body<FMT>(x, rows, cols, out, sc, ld_sc, blockIdx.x, gridDim.x);
}

// Rowwise MX quantization of up to kMxMany tensors in one launch: tensor t owns blocks
// [first, first + blocks) and runs exactly the grid-stride loop mx_row_kernel runs for it
// alone, so its bytes and scales are unchanged; the shared launch fills the chip when one
// tensor would not and saves a launch per extra tensor.
constexpr int kMxMany = 8;

struct MxManySeg {
  const uint16_t* x;
  int64_t rows, cols;
  uint8_t* out;
  uint8_t* sc;
  int64_t ld_sc;
  int64_t first, blocks;
  int fmt;
};

struct MxManyArgs {
  MxManySeg seg[kMxMany];
  int count;
};

__global__ __launch_bounds__(kMxNT) void mx_row_many_kernel(MxManyArgs a) {
  int t = 0;
  for (int k = 1; k < a.count; ++k)
    if ((int64_t)blockIdx.x >= a.seg[k].first) t = k;
  const MxManySeg& g = a.seg[t];
  const int64_t blk = (int64_t)blockIdx.x - g.first;
  if (g.fmt == BF8_E4M3)
    mx_row_body<BF8_E4M3>(g.x, g.rows, g.cols, g.out, g.sc, g.ld_sc, blk, g.blocks);
  else
    mx_row_body<BF8_E5M2>(g.x, g.rows, g.cols, g.out, g.sc, g.ld_sc, blk, g.blocks);
}

int64_t mx_row_blocks(int64_t rows, int64_t ld_sc) {
  const int64_t groups = rows * (ld_sc / 4);
  return std::max<int64_t>(1, std::min<int64_t>((groups + kMxNT / 16 - 1) / (kMxNT / 16),
                                                kMxMaxRowBlocks));
}

// Columnwise, transposed: 64 x 64 tiles of x; each column's two 32-row blocks get their
// scales from an LDS pass over |x|; q_t [cols, rows], scales [cols, ld_sc_t].
template <int FMT>
__global__ __launch_bounds__(kMxNT) void mx_col_kernel(const uint16_t* __restrict__ x,
                                                       int64_t rows, int64_t cols,
                                                       uint8_t* __restrict__ out_t,
                                                       uint8_t* __restrict__ sc_t,
                                                       int64_t ld_sc_t) {
  __shared__ uint16_t keys[kMT][kMT + 2];       // |x| bf16 keys, [row][col]
  __shared__ float mult[2][kMT];                // per (row block, column)
  __shared__ uint32_t tile[kMT * kMPitch / 4];  // fp8 bytes, [row][col]
  uint8_t* tb = reinterpret_cast<uint8_t*>(tile);
  const int64_t tiles_c = (cols + kMT - 1) / kMT;
  const int64_t ntiles = tiles_c * ((rows + kMT - 1) / kMT);
  const int64_t nblk_rows = rows / 32;
  const int t = threadIdx.x;
  for (int64_t tile_id = blockIdx.x; tile_id < ntiles; tile_id += gridDim.x) {
    const int64_t r0 = (tile_id / tiles_c) * kMT, c0 = (tile_id % tiles_c) * kMT;
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr, c = c0 + lc;
    const bool valid = r < rows && c < cols;
    uint4 a0 = make_uint4(0u, 0u, 0u, 0u), a1 = a0;
    if (valid) {
      const uint4* src4 = reinterpret_cast<const uint4*>(x + r * cols + c);
      a0 = src4[0];
      a1 = src4[1];
    }
    {
      const uint32_t w[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        keys[lr][lc + 2 * i] = (uint16_t)(w[i] & 0x7FFFu);
        keys[lr][lc + 2 * i + 1] = (uint16_t)((w[i] >> 16) & 0x7FFFu);
      }
    }
    __syncthreads();
    if (t < 2 * kMT) {
      const int col = t & (kMT - 1), blk = t >> 6;
      uint32_t m = 0;
#pragma unroll 8
      for (int i = 0; i < 32; ++i) m = max(m, (uint32_t)keys[blk * 32 + i][col]);
      const uint32_t e = mx_exponent<FMT>(m << 16);
      mult[blk][col] = mx_multiplier(e);
      const int64_t gc = c0 + col, gb = r0 / 32 + blk;
      if (gc < cols) {
        uint8_t* srow = sc_t + gc * ld_sc_t;
        if (gb < nblk_rows) srow[gb] = (uint8_t)e;
        // the last tile row also pads the column's scale row to whole dwords
        if (blk == 1 && r0 + kMT >= rows)
          for (int64_t pb = nblk_rows; pb < ld_sc_t; ++pb) srow[pb] = (uint8_t)kMxPadScale;
      }
    }
    __syncthreads();
    {
      uint32_t q[4] = {0u, 0u, 0u, 0u};
      if (valid) {
        float s[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = mult[lr >> 5][lc + i];
        const uint4 w0 = a0, w1 = a1;
        // per-element multipliers: quantize in groups of 4 with their own factors
        const float xs[16] = {bf16_lo(w0.x), bf16_hi(w0.x), bf16_lo(w0.y), bf16_hi(w0.y),
                              bf16_lo(w0.z), bf16_hi(w0.z), bf16_lo(w0.w), bf16_hi(w0.w),
                              bf16_lo(w1.x), bf16_hi(w1.x), bf16_lo(w1.y), bf16_hi(w1.y),
                              bf16_lo(w1.z), bf16_hi(w1.z), bf16_lo(w1.w), bf16_hi(w1.w)};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t wq = quant4<FMT>(xs[4 * k] * s[4 * k], xs[4 * k + 1] * s[4 * k + 1],
                                    xs[4 * k + 2] * s[4 * k + 2], xs[4 * k + 3] * s[4 * k + 3],
                                    xs[4 * k], xs[4 * k + 1], xs[4 * k + 2], xs[4 * k + 3],
                                    s[4 * k]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float pr = xs[4 * k + e] * s[4 * k + e];
            if (__builtin_expect(pr != pr, 0))
              wq = (wq & ~(0xFFu << (8 * e))) | (nan_byte(xs[4 * k + e], s[4 * k + e]) << (8 * e));
          }
          q[k] = wq;
        }
      }
      uint32_t* dst = reinterpret_cast<uint32_t*>(tb + lr * kMPitch + lc);
      dst[0] = q[0]; dst[1] = q[1]; dst[2] = q[2]; dst[3] = q[3];
    }
    __syncthreads();
    {
      const int oc = t >> 2, orow = (t & 3) * 16;
      const int64_t tr = c0 + oc, tc = r0 + orow;
      if (tr < cols && tc < rows) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t b0 = tb[(orow + 4 * j + 0) * kMPitch + oc];
          const uint32_t b1 = tb[(orow + 4 * j + 1) * kMPitch + oc];
          const uint32_t b2 = tb[(orow + 4 * j + 2) * kMPitch + oc];
          const uint32_t b3 = tb[(orow + 4 * j + 3) * kMPitch + oc];
          w[j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        *reinterpret_cast<uint4*>(out_t + tr * rows + tc) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

int bf8_quantize_mx_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                         uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                         void* stream) {
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_quantize_mx_bf16: bad fmt %d", fmt);
  BF8_CHECK(rows >= 0 && cols >= 0, "bf8_quantize_mx_bf16: negative shape");
  BF8_CHECK((out == nullptr) == (out_scales == nullptr) &&
                (out_t == nullptr) == (out_t_scales == nullptr) && (out || out_t),
            "bf8_quantize_mx_bf16: give out with out_scales and/or out_t with out_t_scales");
  BF8_CHECK(!out || cols % 32 == 0,
            "bf8_quantize_mx_bf16: rowwise blocks need cols %% 32 == 0 (got %lld)", (long long)cols);
  BF8_CHECK(!out_t || (rows % 32 == 0 && cols % 16 == 0),
            "bf8_quantize_mx_bf16: columnwise blocks need rows %% 32 == 0 and cols %% 16 == 0 "
            "(got %lld x %lld)", (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return BF8_OK;
  BF8_CHECK(x != nullptr, "bf8_quantize_mx_bf16: x is NULL");
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 7) == 0 && ((uintptr_t)out_t & 15) == 0 &&
                ((uintptr_t)out_scales & 3) == 0,
            "bf8_quantize_mx_bf16: x, out_t 16-byte, out 8-byte, out_scales 4-byte aligned");
  hipStream_t s = as_stream(stream);
  const uint16_t* xs = (const uint16_t*)x;
  if (out) {
    const int64_t ld = bf8_mx_scale_ld(cols);
    const unsigned grid = (unsigned)mx_row_blocks(rows, ld);
    if (fmt == BF8_E4M3)
      hipLaunchKernelGGL(mx_row_kernel<BF8_E4M3>, dim3(grid), dim3(kMxNT), 0, s, xs, rows, cols,
                         out, out_scales, ld);
    else
      hipLaunchKernelGGL(mx_row_kernel<BF8_E5M2>, dim3(grid), dim3(kMxNT), 0, s, xs, rows, cols,
                         out, out_scales, ld);
    const int rc = launch_status("mx_row_kernel");
    if (rc != BF8_OK) return rc;
  }
  if (out_t) {
    const int64_t ld = bf8_mx_scale_ld(rows);
    const int64_t tiles = ((rows + kMT - 1) / kMT) * ((cols + kMT - 1) / kMT);
    const unsigned grid = (unsigned)std::min<int64_t>(tiles, kMaxMxTileBlocks);
    if (fmt == BF8_E4M3)
      hipLaunchKernelGGL(mx_col_kernel<BF8_E4M3>, dim3(grid), dim3(kMxNT), 0, s, xs, rows, cols,
                         out_t, out_t_scales, ld);
    else
      hipLaunchKernelGGL(mx_col_kernel<BF8_E5M2>, dim3(grid), dim3(kMxNT), 0, s, xs, rows, cols,
                         out_t, out_t_scales, ld);
    return launch_status("mx_col_kernel");
  }
  return BF8_OK;
}

int bf8_quantize_mx_many_bf16(int count, const void* const* x, const int64_t* rows,
                              const int64_t* cols, const int* fmt, uint8_t* const* out,
                              uint8_t* const* out_scales, void* stream) {
  BF8_CHECK(count >= 1 && count <= kMxMany,
            "bf8_quantize_mx_many_bf16: count %d outside [1, %d]", count, kMxMany);
  BF8_CHECK(x && rows && cols && fmt && out && out_scales,
            "bf8_quantize_mx_many_bf16: NULL array");
  MxManyArgs a{};
  int64_t total = 0;
  for (int t = 0; t < count; ++t) {
    BF8_CHECK(fmt[t] == BF8_E4M3 || fmt[t] == BF8_E5M2,
              "bf8_quantize_mx_many_bf16: tensor %d: bad fmt %d", t, fmt[t]);
    BF8_CHECK(rows[t] >= 0 && cols[t] >= 0, "bf8_quantize_mx_many_bf16: tensor %d: negative shape",
              t);
    BF8_CHECK(cols[t] % 32 == 0,
              "bf8_quantize_mx_many_bf16: tensor %d: rowwise blocks need cols %% 32 == 0 (got %lld)",
              t, (long long)cols[t]);
    if (rows[t] == 0 || cols[t] == 0) continue;
    BF8_CHECK(x[t] && out[t] && out_scales[t],
              "bf8_quantize_mx_many_bf16: tensor %d: x, out or out_scales is NULL", t);
    BF8_CHECK(((uintptr_t)x[t] & 15) == 0 && ((uintptr_t)out[t] & 7) == 0 &&
                  ((uintptr_t)out_scales[t] & 3) == 0,
              "bf8_quantize_mx_many_bf16: tensor %d: x 16-byte, out 8-byte, out_scales 4-byte "
              "aligned", t);
    MxManySeg& g = a.seg[a.count++];
    g.x = (const uint16_t*)x[t];
    g.rows = rows[t];
    g.cols = cols[t];
    g.out = out[t];
    g.sc = out_scales[t];
    g.ld_sc = bf8_mx_scale_ld(cols[t]);
    g.first = total;
    g.blocks = mx_row_blocks(rows[t], g.ld_sc);
    g.fmt = fmt[t];
    total += g.blocks;
  }
  if (a.count == 0) return BF8_OK;
  hipLaunchKernelGGL(mx_row_many_kernel, dim3((unsigned)total), dim3(kMxNT), 0,
                     as_stream(stream), a);
  return launch_status("mx_row_many_kernel");
}

}  // extern "C"
