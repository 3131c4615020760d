// Axiswise (per-row / per-column) FP8 quantization for gfx950: torchao's AXISWISE scaling
// granularity, used by its `rowwise` and `rowwise_with_gw_hp` recipes.
//
// Replaces torchao hp_tensor_to_float8_dynamic(..., scaling_granularity=AXISWISE,
// axiswise_dim=d, round_scales_to_power_of_2=True) as reached from TrainingLinear.forward
// (bongard/float8_training.py:22, Float8Linear.forward) for recipes named at
// bongard/float8_training.py:9. For a bf16 tensor x [rows, cols]:
//   dim -1 (one scale per row):    amax_r = max_c |x[r, c]|
//   dim 0  (one scale per column): amax_c = max_r |x[r, c]|
//   scale = fp32(fp8_max / max(f64(amax), 1e-12)), rounded down to a power of two when
//   BF8_SCALE_POW2 is set; q = fp8(clamp(f32(x) * scale, +-fp8_max)).
// The per-row quantization is stored as q [rows, cols]; the per-column one is stored
// transposed, q_t [cols, rows] (row c of q_t holds column c of x, the K-contiguous layout
// the GEMM reads), each with its scale_inv vector.
//
// Kernels (bf16 x is read at most twice):
//   axis_row_kernel      one pass over x: per-row amax -> scale -> cast (row output), and
//                        per-block column amax partials (bf16 keys) for the column scales;
//   axis_col_scale_kernel the column partials -> per-column scale and scale_inv;
//   axis_col_cast_kernel  second pass over x: per-column cast through a wave-level LDS
//                        transpose.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"

namespace bf8 {
namespace {

constexpr int kAxNT = 512;              // threads of the row kernel (8 waves)
constexpr int kAxMaxCols = 16384;       // widest row the row kernel holds in registers
constexpr int kAxBlocksPartials = 512;  // row-kernel blocks when it writes column partials
constexpr int kAxBlocksPlain = 2048;    // ... when it does not
constexpr int kColNT = 256;
constexpr int kCT = 64;                 // column-cast tile (rows x cols)
constexpr int kMaxColCastBlocks = 2048;

// |x| keys of two packed bf16: clearing the sign makes the unsigned order of each half the
// order of |x| (NaN above inf).
__device__ __forceinline__ uint4 abs_keys(uint4 v) {
  return make_uint4(v.x & 0x7FFF7FFFu, v.y & 0x7FFF7FFFu, v.z & 0x7FFF7FFFu, v.w & 0x7FFF7FFFu);
}

// Quantize 8 bf16 values with one scale each.
template <int FMT>
__device__ __forceinline__ uint2 quant8_bf16_vs(uint4 v, const float* sc) {
  const float x0 = bf16_lo(v.x), x1 = bf16_hi(v.x), x2 = bf16_lo(v.y), x3 = bf16_hi(v.y);
  const float x4 = bf16_lo(v.z), x5 = bf16_hi(v.z), x6 = bf16_lo(v.w), x7 = bf16_hi(v.w);
  uint2 r;
  r.x = quant4<FMT>(x0 * sc[0], x1 * sc[1], x2 * sc[2], x3 * sc[3], x0, x1, x2, x3, sc[0]);
  r.y = quant4<FMT>(x4 * sc[4], x5 * sc[5], x6 * sc[6], x7 * sc[7], x4, x5, x6, x7, sc[4]);
  // quant4 takes one scale for the sign of a NaN product; patch lanes whose own scale is
  // the NaN source (a NaN column or row amax) with their own scale's rule.
  const float xs[8] = {x0, x1, x2, x3, x4, x5, x6, x7};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pr = xs[e] * sc[e];
    if (__builtin_expect(pr != pr, 0)) {
      uint32_t& w = e < 4 ? r.x : r.y;
      const int sh = 8 * (e & 3);
      w = (w & ~(0xFFu << sh)) | (nan_byte(xs[e], sc[e]) << sh);
    }
  }
  return r;
}

// Max of m over the TPR threads of a row group (TPR = 64: one wave; TPR = 256: four waves
// of a kAxNT / 256 group block, through LDS; every thread of the block must call it).
template <int TPR>
__device__ __forceinline__ uint32_t group_max(uint32_t m) {
  m = wave_max_u32(m);
  if constexpr (TPR == 64) {
    return m;
  } else {
    static_assert(TPR == 256, "row groups of 64 or 256 threads");
    __shared__ uint32_t red[kAxNT / 64];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = m;
    __syncthreads();
    const int base = (w / 4) * 4;
    const uint32_t r = max(max(red[base], red[base + 1]), max(red[base + 2], red[base + 3]));
    __syncthreads();
    return r;
  }
}

// Rows [blockIdx.x * strip, + strip) of x, one row per TPR-thread group at a time (strip is
// a multiple of the kAxNT / TPR groups, so every group runs the same number of steps).
// Thread tl of a group holds the row's 16-byte vectors tl, tl + TPR, ... (V of them).
// out / row_sinv: per-row quantization (NULL: skipped). colpart: per-block max |x| keys
// of each column (bf16 keys, [gridDim.x][cols]), or NULL.
template <int FMT, int TPR, int V>
__global__ __launch_bounds__(kAxNT) void axis_row_kernel(
    const uint16_t* __restrict__ x, int rows, int cols, int strip, int pow2,
    uint8_t* __restrict__ out, float* __restrict__ row_sinv, uint16_t* __restrict__ colpart) {
  constexpr int G = kAxNT / TPR;
  extern __shared__ uint4 cbuf[];  // [G - 1][cols / 8] column keys of groups 1.. (colpart)
  const int g = threadIdx.x / TPR, tl = threadIdx.x % TPR;
  const int nvec = cols >> 3;
  uint4 ck[V];
#pragma unroll
  for (int j = 0; j < V; ++j) ck[j] = make_uint4(0u, 0u, 0u, 0u);
  const int r0 = blockIdx.x * strip;
  for (int rr = g; rr < strip; rr += G) {
    const int r = r0 + rr;
    const bool valid = r < rows;
    const uint4* xr = reinterpret_cast<const uint4*>(x + (int64_t)r * cols);
    uint4 xv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int v = tl + TPR * j;
      xv[j] = (valid && v < nvec) ? xr[v] : make_uint4(0u, 0u, 0u, 0u);
    }
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < V; ++j) m = max(m, absmax_key8(xv[j]));
    m = group_max<TPR>(m);
    if (colpart) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const uint4 k = abs_keys(xv[j]);
        ck[j] = make_uint4(pk_max_u16(ck[j].x, k.x), pk_max_u16(ck[j].y, k.y),
                           pk_max_u16(ck[j].z, k.z), pk_max_u16(ck[j].w, k.w));
      }
    }
    if (valid && (out || row_sinv)) {
      float scale, sinv;
      scale_from_amax_key(m, Fp8Max<FMT>::value, pow2 != 0, scale, sinv);
      if (row_sinv && tl == 0) row_sinv[r] = sinv;
      if (out) {
        uint2* orow = reinterpret_cast<uint2*>(out + (int64_t)r * cols);
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const int v = tl + TPR * j;
          if (v < nvec) orow[v] = quant8_bf16<FMT>(xv[j], scale);
        }
      }
    }
  }
  if (!colpart) return;
  uint4* dst = reinterpret_cast<uint4*>(colpart + (int64_t)blockIdx.x * cols);
  if constexpr (G == 1) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int v = tl + TPR * j;
      if (v < nvec) dst[v] = ck[j];
    }
  } else {
    // groups 1.. hand their keys to group 0, whose threads hold the same columns
    if (g > 0) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int v = tl + TPR * j;
        if (v < nvec) cbuf[(g - 1) * nvec + v] = ck[j];
      }
    }
    __syncthreads();
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int v = tl + TPR * j;
        if (v >= nvec) continue;
        uint4 k = ck[j];
#pragma unroll
        for (int gg = 1; gg < G; ++gg) {
          const uint4 o = cbuf[(gg - 1) * nvec + v];
          k = make_uint4(pk_max_u16(k.x, o.x), pk_max_u16(k.y, o.y), pk_max_u16(k.z, o.z),
                         pk_max_u16(k.w, o.w));
        }
        dst[v] = k;
      }
    }
  }
}

// Column scales from the row kernel's partials [nblk][cols]: a block covers 64 columns
// (8 threads x 8 columns) and splits the nblk partial rows over 32 thread rows.
template <int FMT>
__global__ __launch_bounds__(kColNT) void axis_col_scale_kernel(
    const uint16_t* __restrict__ colpart, int nblk, int cols, int pow2,
    float* __restrict__ col_scale, float* __restrict__ col_sinv) {
  __shared__ uint4 red[32][8];
  const int cg = threadIdx.x & 7, rg = threadIdx.x >> 3;
  const int nvec = cols >> 3;
  const int v = blockIdx.x * 8 + cg;
  uint4 k = make_uint4(0u, 0u, 0u, 0u);
  if (v < nvec) {
    // four independent loads in flight per thread (the partial rows are a latency-bound
    // gather of ~nblk / 32 loads each)
    const uint4* src = reinterpret_cast<const uint4*>(colpart);
    uint4 k4[4] = {k, k, k, k};
    int b = rg;
    for (; b + 96 < nblk; b += 128) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint4 o = src[(int64_t)(b + 32 * u) * nvec + v];
        k4[u] = make_uint4(pk_max_u16(k4[u].x, o.x), pk_max_u16(k4[u].y, o.y),
                           pk_max_u16(k4[u].z, o.z), pk_max_u16(k4[u].w, o.w));
      }
    }
    for (; b < nblk; b += 32) {
      const uint4 o = src[(int64_t)b * nvec + v];
      k4[0] = make_uint4(pk_max_u16(k4[0].x, o.x), pk_max_u16(k4[0].y, o.y),
                         pk_max_u16(k4[0].z, o.z), pk_max_u16(k4[0].w, o.w));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      k = make_uint4(pk_max_u16(k.x, k4[u].x), pk_max_u16(k.y, k4[u].y), pk_max_u16(k.z, k4[u].z),
                     pk_max_u16(k.w, k4[u].w));
  }
  red[rg][cg] = k;
  __syncthreads();
  if (rg != 0 || v >= nvec) return;
#pragma unroll 4
  for (int i = 1; i < 32; ++i) {
    const uint4 o = red[i][cg];
    k = make_uint4(pk_max_u16(k.x, o.x), pk_max_u16(k.y, o.y), pk_max_u16(k.z, o.z),
                   pk_max_u16(k.w, o.w));
  }
  const uint32_t w[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t key = ((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) << 16;
    float scale, sinv;
    scale_from_amax_key(key, Fp8Max<FMT>::value, pow2 != 0, scale, sinv);
    col_scale[v * 8 + e] = scale;
    col_sinv[v * 8 + e] = sinv;
  }
}

// q_t [cols, rows] = per-column cast of x: one 64 x 64 tile per wave (grid-stride), loaded
// as eight 8-row x 128-byte pieces, cast with the lane's 8 column scales, staged in the
// wave's own LDS region and stored transposed (wave_transpose64_staged), as the tensorwise
// cast-transpose does with one scale per column.
template <int FMT>
__global__ __launch_bounds__(kColNT) void axis_col_cast_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols,
    const float* __restrict__ col_scale, uint8_t* __restrict__ out_t) {
  constexpr int kWaves = kColNT / 64;
  __shared__ uint32_t stage[kWaves][kWaveTileDwords];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t tiles_c = (cols + kCT - 1) / kCT;
  const int64_t ntiles = tiles_c * ((rows + kCT - 1) / kCT);
  const bool t16 = (rows & 15) == 0;
  const int ch = lane & 7;
  uint32_t* lds = stage[wid];
  for (int64_t tile_id = (int64_t)blockIdx.x * kWaves + wid; tile_id < ntiles;
       tile_id += (int64_t)gridDim.x * kWaves) {
    const int64_t r0 = (tile_id / tiles_c) * kCT, c0 = (tile_id % tiles_c) * kCT;
    const int64_t c = c0 + 8 * ch;
    const bool cv = c < cols;
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t r = r0 + 8 * k + (lane >> 3);
      v[k] = make_uint4(0u, 0u, 0u, 0u);
      if (r < rows && cv) v[k] = *reinterpret_cast<const uint4*>(x + r * cols + c);
    }
    float sc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (cv) {
      const float4 s0 = reinterpret_cast<const float4*>(col_scale + c)[0];
      const float4 s1 = reinterpret_cast<const float4*>(col_scale + c)[1];
      sc[0] = s0.x; sc[1] = s0.y; sc[2] = s0.z; sc[3] = s0.w;
      sc[4] = s1.x; sc[5] = s1.y; sc[6] = s1.z; sc[7] = s1.w;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int lr = 8 * k + (lane >> 3);
      const uint2 q = quant8_bf16_vs<FMT>(v[k], sc);
      lds[lr * kWaveTilePitch + 2 * ch] = q.x;
      lds[lr * kWaveTilePitch + 2 * ch + 1] = q.y;
    }
    uint4 tq[4];
    wave_transpose64_staged(lds, lane, tq);
    const int64_t tc = r0 + (lane >> 4) * 16;  // column of out_t (a row of x)
    if (tc < rows) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int64_t tr = c0 + 4 * (lane & 15) + cc;  // row of out_t (a column of x)
        if (tr >= cols) continue;
        uint8_t* dst = out_t + tr * rows + tc;
        if (t16 && tc + 16 <= rows) {
          *reinterpret_cast<uint4*>(dst) = tq[cc];
        } else {
          const uint32_t w[4] = {tq[cc].x, tq[cc].y, tq[cc].z, tq[cc].w};
          for (int j = 0; j < 16 && tc + j < rows; ++j)
            dst[j] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
        }
      }
    }
  }
}

struct AxisPlan {
  int tpr, v, groups, strip, blocks;
  size_t part_bytes;  // column partials, 256-byte aligned
};

AxisPlan axis_plan(int64_t rows, int64_t cols, bool colwise) {
  AxisPlan p{};
  const int64_t nvec = cols / 8;
  p.tpr = cols <= 4096 ? 64 : 256;
  const int64_t per = (nvec + p.tpr - 1) / p.tpr;
  p.v = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
  p.groups = kAxNT / p.tpr;
  const int64_t cap = colwise ? kAxBlocksPartials : kAxBlocksPlain;
  int64_t strip = (rows + cap - 1) / cap;
  strip = (strip + p.groups - 1) / p.groups * p.groups;
  if (strip < p.groups) strip = p.groups;
  p.strip = (int)strip;
  p.blocks = (int)std::max<int64_t>(1, (rows + strip - 1) / strip);
  p.part_bytes = colwise ? ((size_t)p.blocks * (size_t)cols * 2 + 255) / 256 * 256 : 0;
  return p;
}

template <int FMT, int TPR>
void launch_row(const AxisPlan& p, const uint16_t* x, int rows, int cols, int pow2, uint8_t* out,
                float* row_sinv, uint16_t* colpart, hipStream_t s) {
  const size_t lds = (colpart && p.groups > 1) ? (size_t)(p.groups - 1) * cols * 2 : 0;
  const dim3 grid((unsigned)p.blocks), block(kAxNT);
#define BF8_AXIS_ROW(VV)                                                                      \
  hipLaunchKernelGGL((axis_row_kernel<FMT, TPR, VV>), grid, block, lds, s, x, rows, cols,    \
                     p.strip, pow2, out, row_sinv, colpart)
  switch (p.v) {
    case 1: BF8_AXIS_ROW(1); break;
    case 2: BF8_AXIS_ROW(2); break;
    case 4: BF8_AXIS_ROW(4); break;
    default: BF8_AXIS_ROW(8); break;
  }
#undef BF8_AXIS_ROW
}

template <int FMT>
int run_axiswise(const uint16_t* x, int rows, int cols, int pow2, uint8_t* out, float* row_sinv,
                 uint8_t* out_t, float* col_sinv, uint8_t* ws, hipStream_t s) {
  const bool colwise = out_t != nullptr;
  const AxisPlan p = axis_plan(rows, cols, colwise);
  uint16_t* colpart = colwise ? reinterpret_cast<uint16_t*>(ws) : nullptr;
  if (p.tpr == 64)
    launch_row<FMT, 64>(p, x, rows, cols, pow2, out, row_sinv, colpart, s);
  else
    launch_row<FMT, 256>(p, x, rows, cols, pow2, out, row_sinv, colpart, s);
  int rc = launch_status("axis_row_kernel");
  if (rc != BF8_OK || !colwise) return rc;
  float* col_scale = reinterpret_cast<float*>(ws + p.part_bytes);
  hipLaunchKernelGGL(axis_col_scale_kernel<FMT>, dim3((unsigned)((cols / 8 + 7) / 8)),
                     dim3(kColNT), 0, s, colpart, p.blocks, cols, pow2, col_scale, col_sinv);
  rc = launch_status("axis_col_scale_kernel");
  if (rc != BF8_OK) return rc;
  const int64_t tiles = ((int64_t)(rows + kCT - 1) / kCT) * ((cols + kCT - 1) / kCT);
  const unsigned grid = (unsigned)std::min<int64_t>((tiles + kColNT / 64 - 1) / (kColNT / 64),
                                                    kMaxColCastBlocks);
  hipLaunchKernelGGL(axis_col_cast_kernel<FMT>, dim3(grid), dim3(kColNT), 0, s, x,
                     (int64_t)rows, (int64_t)cols, col_scale, out_t);
  return launch_status("axis_col_cast_kernel");
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

size_t bf8_axiswise_workspace(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const AxisPlan p = axis_plan(rows, cols, true);
  return p.part_bytes + (size_t)cols * 4;
}

int bf8_quantize_axiswise_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                               float* row_scale_inv, uint8_t* out_t, float* col_scale_inv,
                               void* ws, size_t ws_bytes, void* stream) {
  const int pow2 = (fmt & BF8_SCALE_POW2) ? 1 : 0;
  fmt &= ~BF8_SCALE_POW2;
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_quantize_axiswise_bf16: bad fmt %d", fmt);
  BF8_CHECK(rows >= 0 && cols >= 0 && rows < (1LL << 31),
            "bf8_quantize_axiswise_bf16: bad shape");
  BF8_CHECK(cols % 16 == 0 && cols <= kAxMaxCols,
            "bf8_quantize_axiswise_bf16: need cols %% 16 == 0 and cols <= %d (got %lld)",
            kAxMaxCols, (long long)cols);
  BF8_CHECK((out == nullptr) == (row_scale_inv == nullptr) &&
                (out_t == nullptr) == (col_scale_inv == nullptr) && (out || out_t),
            "bf8_quantize_axiswise_bf16: give out with row_scale_inv and/or out_t with "
            "col_scale_inv");
  if (rows == 0 || cols == 0) return BF8_OK;
  BF8_CHECK(x != nullptr, "bf8_quantize_axiswise_bf16: x is NULL");
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)out_t & 15) == 0,
            "bf8_quantize_axiswise_bf16: x, out, out_t must be 16-byte aligned");
  if (out_t) {
    const size_t need = bf8_axiswise_workspace(rows, cols);
    BF8_CHECK(ws && ws_bytes >= need && ((uintptr_t)ws & 255) == 0,
              "bf8_quantize_axiswise_bf16: workspace needs %zu bytes, 256-byte aligned (got %zu)",
              need, ws_bytes);
    BF8_CHECK(((uintptr_t)col_scale_inv & 15) == 0,
              "bf8_quantize_axiswise_bf16: col_scale_inv must be 16-byte aligned");
  }
  const uint16_t* xs = (const uint16_t*)x;
  hipStream_t s = as_stream(stream);
  if (fmt == BF8_E4M3)
    return run_axiswise<BF8_E4M3>(xs, (int)rows, (int)cols, pow2, out, row_scale_inv, out_t,
                                  col_scale_inv, (uint8_t*)ws, s);
  return run_axiswise<BF8_E5M2>(xs, (int)rows, (int)cols, pow2, out, row_scale_inv, out_t,
                                col_scale_inv, (uint8_t*)ws, s);
}

}  // extern "C"
