// RMSNorm with zero-centred gamma fused with the amax pass of the quantization that follows
// it (FusedMLP's norm -> fc1 input), for gfx950.
//
// Replaces the norm of TE LayerNormMLP(normalization='RMSNorm', zero_centered_gamma=True)
// constructed at bongard/fused_mlp.py:25-30 and, in evaluation, HF T5Gemma2RMSNorm
// (modeling_t5gemma2.py:61-69): per row, in fp32,
//   r = 1 / sqrt(mean(x^2) + eps),  y = bf16((x * r) * (1 + gamma))
// (gamma used as is when zero_centered is 0). The sum of squares accumulates in fp64 and
// is rounded to fp32 before the mean, so the result is the correctly rounded fp32 mean of
// the squares; sqrt and the reciprocal are correctly rounded (never v_rsq_f32).
// Every block also writes the max |y| key of the rows it normalised, so the cast of y takes
// its scale from these partials (bf8_cast_partials_bf16) and y needs no separate amax pass.
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace bf8 {
namespace {

constexpr int kNormNT = 256;            // four waves, one row per wave at a time
constexpr int kMaxNormBlocks = 1024;    // amax partials stay within the cast's inline limit
constexpr int kMaxVecPerLane = 8;       // 16-byte vectors of a row per lane (cols <= 4096)

int64_t norm_blocks(int64_t rows) {
  int64_t b = (rows + 3) / 4;
  if (b < 1) b = 1;
  return b < kMaxNormBlocks ? b : kMaxNormBlocks;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per row (grid-stride over rows), the next row's loads issued before the current
// row is reduced and written. Lane l holds the row's 16-byte vectors l, l + 64, ... (V of
// them, cols = 8 * 64 * V at most).
template <int V>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ x, int64_t row,
                                         int64_t rows, int cols, int lane, uint4* xv) {
  const int nvec = cols >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * cols);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int v = lane + 64 * j;
    xv[j] = (row < rows && v < nvec) ? xr[v] : make_uint4(0u, 0u, 0u, 0u);
  }
}

template <int V>
__global__ __launch_bounds__(kNormNT) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int cols, const uint16_t* __restrict__ gamma,
    float eps, int zero_centered, uint16_t* __restrict__ y, float* __restrict__ rstd,
    uint32_t* __restrict__ partials) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nvec = cols >> 3;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t row = (int64_t)blockIdx.x * 4 + wid;
  uint4 xv[V];
  load_row<V>(x, row, rows, cols, lane, xv);
  // the lane's gamma vectors (bf16, the same for every row; the factor 1 + gamma is formed
  // per use, which keeps half the registers of holding it in fp32)
  uint4 gv[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int v = lane + 64 * j;
    gv[j] = v < nvec ? reinterpret_cast<const uint4*>(gamma)[v] : make_uint4(0u, 0u, 0u, 0u);
  }
  const float g0 = zero_centered ? 1.0f : 0.0f;
  uint32_t m = 0;
  for (; row < rows; row += stride) {
    uint4 nx[V];
    load_row<V>(x, row + stride, rows, cols, lane, nx);
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double lo = bf16_lo(w[e]), hi = bf16_hi(w[e]);
        ss = fma(lo, lo, ss);
        ss = fma(hi, hi, ss);
      }
    }
    ss = wave_sum_f64(ss);
    const float mean = __fdiv_rn((float)ss, (float)cols);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    if (rstd && lane == 0) rstd[row] = r;
    uint4* yr = reinterpret_cast<uint4*>(y + row * cols);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int v = lane + 64 * j;
      if (v < nvec) {
        const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        const uint32_t gw[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = (bf16_lo(w[e]) * r) * (g0 + bf16_lo(gw[e]));
          const float b = (bf16_hi(w[e]) * r) * (g0 + bf16_hi(gw[e]));
          o[e] = f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
        }
        const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
        m = max(m, absmax_key8(ov));
        yr[v] = ov;
      }
    }
#pragma unroll
    for (int j = 0; j < V; ++j) xv[j] = nx[j];
  }
  m = block_max_u32<kNormNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

int64_t bf8_rmsnorm_partials(int64_t rows) { return norm_blocks(rows); }

int bf8_rmsnorm_bf16(const void* x, int64_t rows, int64_t cols, const void* gamma, float eps,
                     int zero_centered, void* y, float* rstd, uint32_t* partials,
                     void* stream) {
  BF8_CHECK(rows >= 0 && cols > 0, "bf8_rmsnorm_bf16: bad shape");
  BF8_CHECK(cols % 8 == 0 && cols <= 8 * 64 * kMaxVecPerLane,
            "bf8_rmsnorm_bf16: need cols %% 8 == 0 and cols <= %d (got %lld)",
            8 * 64 * kMaxVecPerLane, (long long)cols);
  if (rows == 0) return BF8_OK;
  BF8_CHECK(x && gamma && y && partials, "bf8_rmsnorm_bf16: NULL pointer");
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)gamma & 15) == 0,
            "bf8_rmsnorm_bf16: x, y, gamma must be 16-byte aligned");
  const dim3 grid((unsigned)norm_blocks(rows)), block(kNormNT);
  hipStream_t s = as_stream(stream);
  const int nvec_lane = (int)((cols / 8 + 63) / 64);
  const uint16_t* xs = (const uint16_t*)x;
  const uint16_t* gs = (const uint16_t*)gamma;
  uint16_t* ys = (uint16_t*)y;
#define BF8_NORM(VV)                                                                      \
  hipLaunchKernelGGL(rmsnorm_kernel<VV>, grid, block, 0, s, xs, rows, (int)cols, gs, eps, \
                     zero_centered, ys, rstd, partials)
  switch (nvec_lane) {
    case 1: BF8_NORM(1); break;
    case 2: BF8_NORM(2); break;
    case 3: BF8_NORM(3); break;
    case 4: BF8_NORM(4); break;
    case 5: BF8_NORM(5); break;
    case 6: BF8_NORM(6); break;
    default: BF8_NORM(8); break;
  }
#undef BF8_NORM
  return launch_status("rmsnorm_kernel");
}

}  // extern "C"
