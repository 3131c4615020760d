// NVFP4 block quantization for gfx950: e2m1 values in blocks of 16 with an e4m3 scale per
// block under a per-tensor fp32 scale, and the exact dequantization of such blocks to bf16.
//
// Replaces TE's NVFP4BlockScaling quantizer behind te.Linear under the 'nvfp4' recipe
// (bongard/te_linear.py:17,38; bongard/fused_mlp.py:9,32) for the part its arithmetic
// fixes without TE at hand (round to nearest even everywhere; no random Hadamard
// transform, no stochastic rounding, 1-D blocks along the GEMM's reduction dimension):
//
//   S_enc = fp32(2688 / max(f64(amax), 1e-12))       2688 = e4m3 max (448) x e2m1 max (6)
//   S_dec = fp32(1 / S_enc)
//   per block of 16 (b = max |x| over the block):
//     s    = e4m3_rne_sat(fp32(fp32(b / 6) * S_enc))  the stored block scale
//     mult = s == 0 ? 0 : fp32(S_enc / s)
//     q_i  = e2m1_rne(fp32(x_i * mult))               saturating at +-6
//   x_i ~ e2m1(q_i) * s * S_dec
//
// gfx950's block-scaled MFMA takes FP4 only with power-of-two scales per 32 values, so the
// GEMM runs on the bf16 MFMA instead: e2m1(q) * s has at most 6 significant bits and is
// exact in bf16 (bf8_dequant_nvfp4 writes it), and the GEMM epilogue applies S_dec of both
// operands. Codes: bit 3 the sign (copied from the product, so -0 is 0x8), bits 0-2 the
// magnitude index into {0, 0.5, 1, 1.5, 2, 3, 4, 6}; two codes per byte, the even element
// in the low nibble. A NaN product gives code 0 with its sign bit (unpinned: no reference
// result exists for non-finite blocks).
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace bf8 {
namespace {

constexpr int kNT = 256;
constexpr float kNvfp4Max = 6.0f;
constexpr float kNvfp4Global = 448.0f * 6.0f;
constexpr int64_t kMaxNvfp4Blocks = 2048;

// Round-to-nearest-even onto the e2m1 grid by threshold counting: each midpoint between
// neighbours rounds to the neighbour whose code is even (0.25 -> 0, 0.75 -> 1, 1.25 -> 1,
// 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4); beyond 5 everything (inf included) is 6.
__device__ __forceinline__ uint32_t e2m1_code(float p) {
  const float a = fabsf(p);
  const uint32_t m = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) +
                     (uint32_t)(a >= 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) +
                     (uint32_t)(a > 5.0f);
  return m | ((__float_as_uint(p) >> 31) << 3);
}

__device__ __forceinline__ float e2m1_value(uint32_t code) {
  const uint32_t m = code & 7u;
  // 0, 0.5 (subnormal: m / 2), then 2^(e - 1) * (1 + mantissa / 2) with e = m >> 1:
  // 1, 1.5, 2, 3, 4, 6
  const float mag = m < 2 ? 0.5f * (float)m
                          : (float)(1u << ((m >> 1) - 1)) * ((m & 1u) ? 1.5f : 1.0f);
  return (code & 8u) ? -mag : mag;
}

// e4m3 byte of v (RNE, saturating at 448; NaN as 0x7F | sign), and the fp32 value of a byte.
__device__ __forceinline__ uint32_t e4m3_byte(float v) {
  return quant4<BF8_E4M3>(v, 0.f, 0.f, 0.f, v, 0.f, 0.f, 0.f, 1.0f) & 0xFFu;
}
__device__ __forceinline__ float e4m3_value(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
}

// The block scale byte and the multiplier of a block whose max |x| is the bf16 key k.
__device__ __forceinline__ void block_scale(uint32_t key, float s_enc, uint32_t& sbyte,
                                            float& mult) {
  const float bmax = __uint_as_float(key);
  sbyte = e4m3_byte((bmax / kNvfp4Max) * s_enc);
  const float s = e4m3_value(sbyte);
  mult = s == 0.0f ? 0.0f : s_enc / s;
}

// 16 bf16 values (two uint4) -> 8 packed code bytes.
__device__ __forceinline__ uint2 pack16(const uint32_t (&w)[8], float mult) {
  uint32_t r[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = e2m1_code(bf16_lo(w[i]) * mult);
    const uint32_t hi = e2m1_code(bf16_hi(w[i]) * mult);
    r[i >> 2] |= (lo | (hi << 4)) << (8 * (i & 3));
  }
  return make_uint2(r[0], r[1]);
}

// 8 packed code bytes of a block with scale value s -> its 16 bf16 values e2m1(code) * s
// (two uint4). e2m1 x e4m3 has at most 6 significant bits: the fp32 product is exact, and so
// is its bf16 (upper half).
__device__ __forceinline__ void dequant16(uint2 c, float s, uint4& d0, uint4& d1) {
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t byte = ((i < 4 ? c.x : c.y) >> (8 * (i & 3))) & 0xFFu;
    const uint32_t lo = __float_as_uint(e2m1_value(byte & 0xFu) * s) >> 16;
    const uint32_t hi = __float_as_uint(e2m1_value(byte >> 4) * s) >> 16;
    o[i] = lo | (hi << 16);
  }
  d0 = make_uint4(o[0], o[1], o[2], o[3]);
  d1 = make_uint4(o[4], o[5], o[6], o[7]);
}

// Rowwise: blocks of 16 consecutive elements of a row; one block per thread (grid-stride).
// out [rows, cols / 2], scales [rows, cols / 16]; or, with deq set, the blocks' exact bf16
// dequantization deq [rows, cols] in their place. Block 0 publishes the meta record.
__global__ __launch_bounds__(kNT) void nvfp4_rows_kernel(const uint16_t* __restrict__ x,
                                                         int64_t rows, int64_t cols,
                                                         const uint32_t* __restrict__ partials,
                                                         int64_t np, float* __restrict__ meta,
                                                         uint8_t* __restrict__ out,
                                                         uint8_t* __restrict__ scales,
                                                         uint16_t* __restrict__ deq) {
  const float s_enc = scale_from_partials_block<kNT>(partials, np, kNvfp4Global, meta, false,
                                                     blockIdx.x == 0);
  const int64_t per_row = cols / 16;
  const int64_t nblk = rows * per_row;
  for (int64_t b = (int64_t)blockIdx.x * kNT + threadIdx.x; b < nblk;
       b += (int64_t)gridDim.x * kNT) {
    const uint4* src = reinterpret_cast<const uint4*>(x + b * 16);
    const uint4 v0 = src[0], v1 = src[1];
    const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    const uint32_t key = max(absmax_key8(v0), absmax_key8(v1));
    uint32_t sbyte;
    float mult;
    block_scale(key, s_enc, sbyte, mult);
    const uint2 c = pack16(w, mult);
    if (deq) {
      uint4 d0, d1;
      dequant16(c, e4m3_value(sbyte), d0, d1);
      uint4* dst = reinterpret_cast<uint4*>(deq + b * 16);
      dst[0] = d0;
      dst[1] = d1;
    } else {
      *reinterpret_cast<uint2*>(out + b * 8) = c;
      scales[b] = (uint8_t)sbyte;
    }
  }
}

// Columnwise: the quantization of x^T [cols, rows], blocks of 16 consecutive rows of one
// column of x. One (column, 16-row block) per thread, consecutive threads on consecutive
// columns (the loads of a row coalesce). out_t [cols, rows / 2], scales_t [cols, rows / 16].
__global__ __launch_bounds__(kNT) void nvfp4_cols_kernel(const uint16_t* __restrict__ x,
                                                         int64_t rows, int64_t cols,
                                                         const uint32_t* __restrict__ partials,
                                                         int64_t np, float* __restrict__ meta,
                                                         int publish, uint8_t* __restrict__ out_t,
                                                         uint8_t* __restrict__ scales_t) {
  const float s_enc = scale_from_partials_block<kNT>(partials, np, kNvfp4Global, meta, false,
                                                     publish && blockIdx.x == 0);
  const int64_t rblocks = rows / 16;
  const int64_t nitems = cols * rblocks;
  for (int64_t it = (int64_t)blockIdx.x * kNT + threadIdx.x; it < nitems;
       it += (int64_t)gridDim.x * kNT) {
    const int64_t rb = it / cols, c = it - rb * cols;
    uint32_t w[8];
    uint32_t key = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = x[(rb * 16 + 2 * i) * cols + c];
      const uint32_t hi = x[(rb * 16 + 2 * i + 1) * cols + c];
      w[i] = lo | (hi << 16);
      key = max(key, max((lo & 0x7FFFu) << 16, (hi & 0x7FFFu) << 16));
    }
    uint32_t sbyte;
    float mult;
    block_scale(key, s_enc, sbyte, mult);
    *reinterpret_cast<uint2*>(out_t + c * (rows / 2) + rb * 8) = pack16(w, mult);
    scales_t[c * rblocks + rb] = (uint8_t)sbyte;
  }
}

// bf16 [rows, cols] = e2m1(q) * s for every block (exact); S_dec is left to the GEMM.
__global__ __launch_bounds__(kNT) void nvfp4_dequant_kernel(const uint8_t* __restrict__ q,
                                                            const uint8_t* __restrict__ scales,
                                                            int64_t nblk,
                                                            uint16_t* __restrict__ out) {
  for (int64_t b = (int64_t)blockIdx.x * kNT + threadIdx.x; b < nblk;
       b += (int64_t)gridDim.x * kNT) {
    uint4 d0, d1;
    dequant16(*reinterpret_cast<const uint2*>(q + b * 8), e4m3_value(scales[b]), d0, d1);
    uint4* dst = reinterpret_cast<uint4*>(out + b * 16);
    dst[0] = d0;
    dst[1] = d1;
  }
}

unsigned stream_grid(int64_t items) {
  int64_t g = (items + kNT - 1) / kNT;
  if (g < 1) g = 1;
  return (unsigned)(g < kMaxNvfp4Blocks ? g : kMaxNvfp4Blocks);
}

}  // namespace
}  // namespace bf8

using namespace bf8;

// Argument checks shared by the NVFP4 quantize entry points (before anything launches).
static int nvfp4_args(const char* who, const void* x, int64_t rows, int64_t cols,
                      const uint8_t* out, const uint8_t* out_scales, const uint8_t* out_t,
                      const uint8_t* out_t_scales, const float* meta) {
  BF8_CHECK(rows >= 0 && cols >= 0, "%s: negative shape", who);
  BF8_CHECK(out || out_t, "%s: out and out_t are both NULL", who);
  BF8_CHECK(!out || (out_scales && cols % 16 == 0),
            "%s: rowwise blocks need cols %% 16 == 0 (got %lld) and scales", who,
            (long long)cols);
  BF8_CHECK(!out_t || (out_t_scales && rows % 16 == 0),
            "%s: columnwise blocks need rows %% 16 == 0 (got %lld) and scales", who,
            (long long)rows);
  BF8_CHECK(meta != nullptr, "%s: meta is NULL", who);
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 7) == 0 && ((uintptr_t)out_t & 7) == 0,
            "%s: x must be 16-byte and out, out_t 8-byte aligned", who);
  BF8_CHECK(rows * cols == 0 || x != nullptr, "%s: x is NULL", who);
  return BF8_OK;
}

// The rowwise and/or columnwise casts, the per-tensor amax reduced from np partials (maxima
// of |x| as fp32 bits) that are already written.
static int nvfp4_casts(const void* x, int64_t rows, int64_t cols, const uint32_t* partials,
                       int64_t np, uint8_t* out, uint8_t* out_scales, uint8_t* out_t,
                       uint8_t* out_t_scales, float* meta, hipStream_t s,
                       void* deq = nullptr) {
  const int64_t n = rows * cols;
  if (out || deq) {
    hipLaunchKernelGGL(nvfp4_rows_kernel, dim3(stream_grid(n / 16)), dim3(kNT), 0, s,
                       (const uint16_t*)x, rows, cols, partials, np, meta, out, out_scales,
                       (uint16_t*)deq);
    const int rc = launch_status("nvfp4_rows_kernel");
    if (rc != BF8_OK) return rc;
  }
  if (out_t) {
    hipLaunchKernelGGL(nvfp4_cols_kernel, dim3(stream_grid(n / 16)), dim3(kNT), 0, s,
                       (const uint16_t*)x, rows, cols, partials, np, meta,
                       (out || deq) ? 0 : 1, out_t, out_t_scales);
    return launch_status("nvfp4_cols_kernel");
  }
  return BF8_OK;
}

extern "C" {

int bf8_quantize_nvfp4_partials_bf16(const void* x, int64_t rows, int64_t cols,
                                     const uint32_t* partials, int64_t n_partials, uint8_t* out,
                                     uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                                     float* meta, void* stream) {
  const char* who = "bf8_quantize_nvfp4_partials_bf16";
  int rc = nvfp4_args(who, x, rows, cols, out, out_scales, out_t, out_t_scales, meta);
  if (rc != BF8_OK) return rc;
  BF8_CHECK(partials && n_partials >= 1, "%s: partials is NULL or empty", who);
  if (rows * cols == 0) return BF8_OK;
  return nvfp4_casts(x, rows, cols, partials, n_partials, out, out_scales, out_t, out_t_scales,
                     meta, as_stream(stream));
}

int bf8_quantize_nvfp4_bf16(const void* x, int64_t rows, int64_t cols, uint8_t* out,
                            uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                            float* meta, uint32_t* partials, void* stream) {
  const char* who = "bf8_quantize_nvfp4_bf16";
  int rc = nvfp4_args(who, x, rows, cols, out, out_scales, out_t, out_t_scales, meta);
  if (rc != BF8_OK) return rc;
  BF8_CHECK(partials, "%s: partials is NULL", who);
  const int64_t n = rows * cols;
  if (n == 0) return BF8_OK;
  rc = bf8_amax_bf16(x, n, partials, stream);
  if (rc != BF8_OK) return rc;
  return nvfp4_casts(x, rows, cols, partials, bf8_amax_partials(n), out, out_scales, out_t,
                     out_t_scales, meta, as_stream(stream));
}

int bf8_quantize_nvfp4_dequant_bf16(const void* x, int64_t rows, int64_t cols,
                                    uint32_t* partials, int64_t n_partials, void* deq,
                                    uint8_t* out_t, uint8_t* out_t_scales, float* meta,
                                    void* stream) {
  const char* who = "bf8_quantize_nvfp4_dequant_bf16";
  BF8_CHECK(rows >= 0 && cols >= 0, "%s: negative shape", who);
  BF8_CHECK(deq != nullptr && cols % 16 == 0,
            "%s: needs deq and cols %% 16 == 0 (got %lld)", who, (long long)cols);
  BF8_CHECK(!out_t || (out_t_scales && rows % 16 == 0),
            "%s: columnwise blocks need rows %% 16 == 0 (got %lld) and scales", who,
            (long long)rows);
  BF8_CHECK(meta != nullptr && partials != nullptr && n_partials >= 0,
            "%s: meta or partials is NULL", who);
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)deq & 15) == 0 && ((uintptr_t)out_t & 7) == 0,
            "%s: x and deq must be 16-byte and out_t 8-byte aligned", who);
  BF8_CHECK(rows * cols == 0 || x != nullptr, "%s: x is NULL", who);
  int rc = BF8_OK;
  const int64_t n = rows * cols;
  if (n == 0) return BF8_OK;
  if (n_partials == 0) {
    rc = bf8_amax_bf16(x, n, partials, stream);
    if (rc != BF8_OK) return rc;
    n_partials = bf8_amax_partials(n);
  }
  return nvfp4_casts(x, rows, cols, partials, n_partials, nullptr, nullptr, out_t, out_t_scales,
                     meta, as_stream(stream), deq);
}

int bf8_dequant_nvfp4(const uint8_t* q, const uint8_t* scales, int64_t rows, int64_t cols,
                      void* out, void* stream) {
  BF8_CHECK(rows >= 0 && cols >= 0 && cols % 16 == 0,
            "bf8_dequant_nvfp4: need cols %% 16 == 0 (got %lld)", (long long)cols);
  BF8_CHECK(((uintptr_t)q & 7) == 0 && ((uintptr_t)out & 15) == 0,
            "bf8_dequant_nvfp4: q must be 8-byte and out 16-byte aligned");
  const int64_t nblk = rows * (cols / 16);
  if (nblk == 0) return BF8_OK;
  BF8_CHECK(q && scales && out, "bf8_dequant_nvfp4: NULL pointer");
  hipLaunchKernelGGL(nvfp4_dequant_kernel, dim3(stream_grid(nblk)), dim3(kNT), 0,
                     as_stream(stream), q, scales, nblk, (uint16_t*)out);
  return launch_status("nvfp4_dequant_kernel");
}

}  // extern "C"
