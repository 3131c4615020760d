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

// Backward of the norm for the bf16 gradient dy of y (autograd of the fp32 formula above):
//   n = x r,  g = f32(dy),  dn = g (z + gamma)   (z = 1 zero-centred, else 0)
//   dx = bf16(r (dn - n s / cols)),  s = sum_j dn_j n_j over the row
//   dgamma = bf16(sum over rows of g n)
// r is recomputed exactly as the forward computes it. One wave per row (grid-stride); each
// lane keeps fp32 sums of g n for its columns, the block adds its four waves' sums through
// LDS and writes one row of partials [gridDim.x, cols]; rmsnorm_dgamma_kernel adds the
// blocks' partials in block order (deterministic) and rounds to bf16.
template <int V>
__global__ __launch_bounds__(kNormNT) void rmsnorm_bwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy, int64_t rows, int cols,
    const uint16_t* __restrict__ gamma, float eps, int zero_centered, uint16_t* __restrict__ dx,
    float* __restrict__ dgamma_part) {
  __shared__ float red[4][8 * 64 * V];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nvec = cols >> 3;
  const int64_t stride = (int64_t)gridDim.x * 4;
  uint4 gv[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int v = lane + 64 * j;
    gv[j] = v < nvec ? reinterpret_cast<const uint4*>(gamma)[v] : make_uint4(0u, 0u, 0u, 0u);
  }
  const float z = zero_centered ? 1.0f : 0.0f;
  float acc[V][8];
#pragma unroll
  for (int j = 0; j < V; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wid; row < rows; row += stride) {
    uint4 xv[V], dv[V];
    load_row<V>(x, row, rows, cols, lane, xv);
    load_row<V>(dy, row, rows, cols, lane, dv);
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
    // pass 1: s and the lane's dgamma sums; pass 2 forms n and dn again for dx (cheaper
    // than keeping them in registers across the wave reduction)
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
      const uint32_t d[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
      const uint32_t gw[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float n0 = bf16_lo(w[e]) * r, n1 = bf16_hi(w[e]) * r;
        const float g0 = bf16_lo(d[e]), g1 = bf16_hi(d[e]);
        acc[j][2 * e] = fmaf(g0, n0, acc[j][2 * e]);
        acc[j][2 * e + 1] = fmaf(g1, n1, acc[j][2 * e + 1]);
        s = fmaf(g0 * (z + bf16_lo(gw[e])), n0, s);
        s = fmaf(g1 * (z + bf16_hi(gw[e])), n1, s);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    const float c = s / (float)cols;
    if (dx) {
      uint4* dxr = reinterpret_cast<uint4*>(dx + row * cols);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int v = lane + 64 * j;
        if (v < nvec) {
          const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
          const uint32_t d[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
          const uint32_t gw[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = r * (bf16_lo(d[e]) * (z + bf16_lo(gw[e])) - (bf16_lo(w[e]) * r) * c);
            const float b = r * (bf16_hi(d[e]) * (z + bf16_hi(gw[e])) - (bf16_hi(w[e]) * r) * c);
            o[e] = f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
          }
          dxr[v] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
  if (!dgamma_part) return;
  // the block's four waves: lane l of wave w holds columns 8 (l + 64 j) + e
#pragma unroll
  for (int j = 0; j < V; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wid][8 * (lane + 64 * j) + e] = acc[j][e];
  __syncthreads();
  for (int col = threadIdx.x; col < cols; col += kNormNT)
    dgamma_part[(int64_t)blockIdx.x * cols + col] =
        ((red[0][col] + red[1][col]) + red[2][col]) + red[3][col];
}

__global__ __launch_bounds__(kNormNT) void rmsnorm_dgamma_kernel(
    const float* __restrict__ part, int nblocks, int cols, uint16_t* __restrict__ dgamma) {
  const int col = blockIdx.x * kNormNT + threadIdx.x;
  if (col >= cols) return;
  float a = 0.0f;
  for (int b = 0; b < nblocks; ++b) a += part[(int64_t)b * cols + col];
  dgamma[col] = (uint16_t)f32_to_bf16_bits(a);
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

size_t bf8_rmsnorm_bwd_workspace(int64_t rows, int64_t cols) {
  return (size_t)norm_blocks(rows) * (size_t)(cols > 0 ? cols : 0) * sizeof(float);
}

int bf8_rmsnorm_bwd_bf16(const void* x, const void* dy, int64_t rows, int64_t cols,
                         const void* gamma, float eps, int zero_centered, void* dx,
                         void* dgamma, void* ws, size_t ws_bytes, void* stream) {
  BF8_CHECK(rows >= 0 && cols > 0, "bf8_rmsnorm_bwd_bf16: bad shape");
  BF8_CHECK(cols % 8 == 0 && cols <= 8 * 64 * kMaxVecPerLane,
            "bf8_rmsnorm_bwd_bf16: need cols %% 8 == 0 and cols <= %d (got %lld)",
            8 * 64 * kMaxVecPerLane, (long long)cols);
  BF8_CHECK(x && dy && gamma && (dx || dgamma), "bf8_rmsnorm_bwd_bf16: NULL pointer");
  BF8_CHECK((((uintptr_t)x | (uintptr_t)dy | (uintptr_t)gamma | (uintptr_t)dx) & 15) == 0,
            "bf8_rmsnorm_bwd_bf16: x, dy, gamma, dx must be 16-byte aligned");
  const int64_t nb = norm_blocks(rows);
  if (dgamma) {
    BF8_CHECK(ws && ws_bytes >= bf8_rmsnorm_bwd_workspace(rows, cols),
              "bf8_rmsnorm_bwd_bf16: workspace of %zu bytes, need %zu", ws_bytes,
              bf8_rmsnorm_bwd_workspace(rows, cols));
  }
  hipStream_t s = as_stream(stream);
  const int nvec_lane = (int)((cols / 8 + 63) / 64);
  const uint16_t* xs = (const uint16_t*)x;
  const uint16_t* ds = (const uint16_t*)dy;
  const uint16_t* gs = (const uint16_t*)gamma;
  uint16_t* dxs = (uint16_t*)dx;
  float* part = dgamma ? (float*)ws : nullptr;
  if (rows > 0) {
#define BF8_NORM_BWD(VV)                                                                      \
  hipLaunchKernelGGL(rmsnorm_bwd_kernel<VV>, dim3((unsigned)nb), dim3(kNormNT), 0, s, xs, ds, \
                     rows, (int)cols, gs, eps, zero_centered, dxs, part)
    switch (nvec_lane) {
      case 1: BF8_NORM_BWD(1); break;
      case 2: BF8_NORM_BWD(2); break;
      case 3: BF8_NORM_BWD(3); break;
      case 4: BF8_NORM_BWD(4); break;
      case 5: BF8_NORM_BWD(5); break;
      case 6: BF8_NORM_BWD(6); break;
      default: BF8_NORM_BWD(8); break;
    }
#undef BF8_NORM_BWD
    const int rc = launch_status("rmsnorm_bwd_kernel");
    if (rc != BF8_OK) return rc;
  }
  if (!dgamma) return BF8_OK;
  if (rows == 0) {
    BF8_CHECK(false, "bf8_rmsnorm_bwd_bf16: no rows to reduce dgamma over");
  }
  hipLaunchKernelGGL(rmsnorm_dgamma_kernel, dim3((unsigned)((cols + kNormNT - 1) / kNormNT)),
                     dim3(kNormNT), 0, s, (const float*)ws, (int)nb, (int)cols,
                     (uint16_t*)dgamma);
  return launch_status("rmsnorm_dgamma_kernel");
}

}  // extern "C"
