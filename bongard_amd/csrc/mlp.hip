// Backward of the gated GELU(tanh) between the MLP's gate/up and down projections.
//
// Forward (bongard/te_linear.py:103): h = bf16(bf16(gelu_tanh(g)) * u) on bf16 g, u.
// Autograd of that bf16 chain gives, per element:
//   a   = bf16(gelu_tanh(g))                 (recomputed exactly as the forward kernel)
//   d_a = bf16(dh * u)                       (mul backward, grad wrt a)
//   d_u = bf16(dh * a)                       (mul backward, grad wrt u)
//   d_g = bf16(d_a * gelu_tanh'(g))          (gelu backward, fp32 inside)
// (gelu_tanh_fwd_bwd in common.hpp). The kernel is one streaming pass (read dH, g, u;
// write d_g, d_u) that also writes per-block amax partials of |dGU|, from which the
// e5m2 cast of dGU derives its scale.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"

namespace bf8 {
namespace {

constexpr int kNT = 256;
constexpr int64_t kMaxBlocks = 2048;

int64_t bwd_blocks(int64_t M, int64_t I) {
  const int64_t vec = M * I / 8;
  int64_t b = (vec + kNT - 1) / kNT;
  if (b < 1) b = 1;
  return b < kMaxBlocks ? b : kMaxBlocks;
}


__global__ __launch_bounds__(kNT) void geglu_bwd_kernel(const uint16_t* __restrict__ dH,
                                                        const uint16_t* __restrict__ GU,
                                                        int64_t M, int64_t I,
                                                        uint16_t* __restrict__ dGU,
                                                        uint32_t* __restrict__ partials) {
  const int64_t per_row = I / 8;
  const int64_t nvec = M * per_row;
  const int64_t stride = (int64_t)gridDim.x * kNT;
  uint32_t m = 0;
  for (int64_t v = (int64_t)blockIdx.x * kNT + threadIdx.x; v < nvec; v += stride) {
    const int64_t row = v / per_row;
    const int64_t col = (v - row * per_row) * 8;
    const uint4 dh = *reinterpret_cast<const uint4*>(dH + row * I + col);
    const uint4 g = *reinterpret_cast<const uint4*>(GU + row * 2 * I + col);
    const uint4 u = *reinterpret_cast<const uint4*>(GU + row * 2 * I + I + col);
    const uint32_t dhw[4] = {dh.x, dh.y, dh.z, dh.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t dg[4], du[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t og = 0, ou = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float x = h ? bf16_hi(gw[w]) : bf16_lo(gw[w]);
        const float uu = h ? bf16_hi(uw[w]) : bf16_lo(uw[w]);
        const float d = h ? bf16_hi(dhw[w]) : bf16_lo(dhw[w]);
        float y, dydx;
        gelu_tanh_fwd_bwd(x, y, dydx);
        const float a = bf16_round(y);
        const float da = bf16_round(d * uu);
        const uint32_t bu = f32_to_bf16_bits(d * a);
        const uint32_t bg = f32_to_bf16_bits(da * dydx);
        og |= bg << (16 * h);
        ou |= bu << (16 * h);
        m = max(m, max((bg & 0x7FFFu) << 16, (bu & 0x7FFFu) << 16));
      }
      dg[w] = og;
      du[w] = ou;
    }
    *reinterpret_cast<uint4*>(dGU + row * 2 * I + col) = make_uint4(dg[0], dg[1], dg[2], dg[3]);
    *reinterpret_cast<uint4*>(dGU + row * 2 * I + I + col) = make_uint4(du[0], du[1], du[2], du[3]);
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// The geglu backward fused with its delayed-scaling cast (for 'fp8_delayed', where dGU's
// scale is known before dGU exists): the same per-element chain as geglu_bwd_kernel, the
// bf16 d_g, d_u quantized at once with the role's delayed scale, written as fp8 rows
// [M, 2I] and/or through an LDS transpose as fp8 [2I, M] (the wgrad layout), plus this
// step's amax partials of |dGU|. Tiles of 64 rows x 64 columns of I; thread t handles 16
// consecutive columns of one row for d_g and the same for d_u. Identical bytes to
// geglu_bwd_kernel followed by the delayed cast of its output.
constexpr int kTT = 64;
constexpr int kTPitch = kTT + 4;
constexpr int64_t kMaxFusedBlocks = 1024;

int64_t fused_blocks(int64_t M, int64_t I) {
  const int64_t tiles = ((M + kTT - 1) / kTT) * (I / kTT);
  return tiles < 1 ? 1 : (tiles < kMaxFusedBlocks ? tiles : kMaxFusedBlocks);
}

__device__ __forceinline__ void geglu_bwd_pair(uint32_t dhw, uint32_t gw, uint32_t uw,
                                               uint32_t& dg, uint32_t& du, uint32_t& m) {
  uint32_t og = 0, ou = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float x = h ? bf16_hi(gw) : bf16_lo(gw);
    const float uu = h ? bf16_hi(uw) : bf16_lo(uw);
    const float d = h ? bf16_hi(dhw) : bf16_lo(dhw);
    float y, dydx;
    gelu_tanh_fwd_bwd(x, y, dydx);
    const float a = bf16_round(y);
    const float da = bf16_round(d * uu);
    const uint32_t bu = f32_to_bf16_bits(d * a);
    const uint32_t bg = f32_to_bf16_bits(da * dydx);
    og |= bg << (16 * h);
    ou |= bu << (16 * h);
    m = max(m, max((bg & 0x7FFFu) << 16, (bu & 0x7FFFu) << 16));
  }
  dg = og;
  du = ou;
}

template <int FMT>
__global__ __launch_bounds__(kNT) void geglu_bwd_delayed_kernel(
    const uint16_t* __restrict__ dH, const uint16_t* __restrict__ GU, int64_t M, int64_t I,
    float* __restrict__ state, int len, int pos, const uint32_t* __restrict__ prev,
    int64_t n_prev, float* __restrict__ meta_out, uint8_t* __restrict__ out,
    uint8_t* __restrict__ out_t, uint32_t* __restrict__ partials) {
  __shared__ uint32_t tiles[2][kTT * kTPitch / 4];
  const float scale =
      delayed_scale_block<kNT>(state, len, pos, prev, n_prev, Fp8Max<FMT>::value, meta_out);
  const int64_t tiles_c = I / kTT;
  const int64_t ntiles = tiles_c * ((M + kTT - 1) / kTT);
  const int t = threadIdx.x;
  const int lr = t >> 2, lc = (t & 3) * 16;
  uint32_t m = 0;
  for (int64_t tile_id = blockIdx.x; tile_id < ntiles; tile_id += gridDim.x) {
    const int64_t r0 = (tile_id / tiles_c) * kTT, c0 = (tile_id % tiles_c) * kTT;
    const int64_t r = r0 + lr, c = c0 + lc;
    uint32_t qg[4] = {0u, 0u, 0u, 0u}, qu[4] = {0u, 0u, 0u, 0u};
    if (r < M) {
      const uint4* dh4 = reinterpret_cast<const uint4*>(dH + r * I + c);
      const uint4* g4 = reinterpret_cast<const uint4*>(GU + r * 2 * I + c);
      const uint4* u4 = reinterpret_cast<const uint4*>(GU + r * 2 * I + I + c);
#pragma unroll
      for (int hv = 0; hv < 2; ++hv) {
        const uint4 dh = dh4[hv], g = g4[hv], u = u4[hv];
        const uint32_t dhw[4] = {dh.x, dh.y, dh.z, dh.w};
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t dg[4], du[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) geglu_bwd_pair(dhw[w], gw[w], uw[w], dg[w], du[w], m);
        const uint2 a = quant8_bf16<FMT>(make_uint4(dg[0], dg[1], dg[2], dg[3]), scale);
        const uint2 b = quant8_bf16<FMT>(make_uint4(du[0], du[1], du[2], du[3]), scale);
        qg[2 * hv] = a.x; qg[2 * hv + 1] = a.y;
        qu[2 * hv] = b.x; qu[2 * hv + 1] = b.y;
      }
      if (out) {
        *reinterpret_cast<uint4*>(out + r * 2 * I + c) = make_uint4(qg[0], qg[1], qg[2], qg[3]);
        *reinterpret_cast<uint4*>(out + r * 2 * I + I + c) =
            make_uint4(qu[0], qu[1], qu[2], qu[3]);
      }
    }
    if (out_t) {
      uint8_t* tg = reinterpret_cast<uint8_t*>(tiles[0]);
      uint8_t* tu = reinterpret_cast<uint8_t*>(tiles[1]);
      uint32_t* dg_l = reinterpret_cast<uint32_t*>(tg + lr * kTPitch + lc);
      uint32_t* du_l = reinterpret_cast<uint32_t*>(tu + lr * kTPitch + lc);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        dg_l[k] = qg[k];
        du_l[k] = qu[k];
      }
      __syncthreads();
      const int oc = t >> 2, orow = (t & 3) * 16;
      const int64_t tc = r0 + orow;  // column of out_t (a row of dGU)
      if (tc < M) {
#pragma unroll
        for (int which = 0; which < 2; ++which) {
          const uint8_t* tb = which ? tu : tg;
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t b0 = tb[(orow + 4 * j + 0) * kTPitch + oc];
            const uint32_t b1 = tb[(orow + 4 * j + 1) * kTPitch + oc];
            const uint32_t b2 = tb[(orow + 4 * j + 2) * kTPitch + oc];
            const uint32_t b3 = tb[(orow + 4 * j + 3) * kTPitch + oc];
            w[j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
          }
          const int64_t tr = (which ? I : 0) + c0 + oc;  // row of out_t
          *reinterpret_cast<uint4*>(out_t + tr * M + tc) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      __syncthreads();  // the next tile reuses the LDS tiles
    }
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

int64_t bf8_geglu_bwd_partials(int64_t M, int64_t I) { return bwd_blocks(M, I); }

int bf8_geglu_bwd(const void* dH, const void* GU, int64_t M, int64_t I, void* dGU,
                  uint32_t* partials, void* stream) {
  BF8_CHECK(M >= 0 && I >= 8 && I % 8 == 0, "bf8_geglu_bwd: need I %% 8 == 0 (I=%lld)", (long long)I);
  BF8_CHECK(dH && GU && dGU && partials, "bf8_geglu_bwd: NULL pointer");
  BF8_CHECK((((uintptr_t)dH | (uintptr_t)GU | (uintptr_t)dGU) & 15) == 0,
            "bf8_geglu_bwd: pointers must be 16-byte aligned");
  const int64_t nb = bwd_blocks(M, I);
  hipLaunchKernelGGL(geglu_bwd_kernel, dim3((unsigned)nb), dim3(kNT), 0, as_stream(stream),
                     (const uint16_t*)dH, (const uint16_t*)GU, M, I, (uint16_t*)dGU, partials);
  return launch_status("geglu_bwd_kernel");
}

int64_t bf8_geglu_bwd_delayed_partials(int64_t M, int64_t I) { return fused_blocks(M, I); }

int bf8_geglu_bwd_delayed(const void* dH, const void* GU, int64_t M, int64_t I, float* state,
                          int len, int pos, const uint32_t* prev_partials, int64_t n_prev, int fmt,
                          float* meta_out, uint8_t* out, uint8_t* out_t, uint32_t* partials_out,
                          void* stream) {
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_geglu_bwd_delayed: bad fmt %d", fmt);
  BF8_CHECK(M >= 0 && I >= kTT && I % kTT == 0,
            "bf8_geglu_bwd_delayed: need I %% 64 == 0 (I=%lld)", (long long)I);
  BF8_CHECK(M % 16 == 0, "bf8_geglu_bwd_delayed: need M %% 16 == 0 (M=%lld)", (long long)M);
  BF8_CHECK(dH && GU && state && partials_out && (out || out_t),
            "bf8_geglu_bwd_delayed: NULL pointer");
  BF8_CHECK(len >= 1 && len <= 1024 && pos >= 0 && pos < len,
            "bf8_geglu_bwd_delayed: bad history length %d / slot %d", len, pos);
  BF8_CHECK(n_prev >= 0 && n_prev <= 4096 && (n_prev == 0 || prev_partials),
            "bf8_geglu_bwd_delayed: bad previous partials (%lld)", (long long)n_prev);
  BF8_CHECK((((uintptr_t)dH | (uintptr_t)GU | (uintptr_t)out | (uintptr_t)out_t) & 15) == 0,
            "bf8_geglu_bwd_delayed: pointers must be 16-byte aligned");
  if (M == 0) return BF8_OK;
  const int64_t nb = fused_blocks(M, I);
  hipStream_t s = as_stream(stream);
  const uint16_t* dh = (const uint16_t*)dH;
  const uint16_t* gu = (const uint16_t*)GU;
  if (fmt == BF8_E4M3)
    hipLaunchKernelGGL(geglu_bwd_delayed_kernel<BF8_E4M3>, dim3((unsigned)nb), dim3(kNT), 0, s,
                       dh, gu, M, I, state, len, pos, prev_partials, n_prev, meta_out, out, out_t,
                       partials_out);
  else
    hipLaunchKernelGGL(geglu_bwd_delayed_kernel<BF8_E5M2>, dim3((unsigned)nb), dim3(kNT), 0, s,
                       dh, gu, M, I, state, len, pos, prev_partials, n_prev, meta_out, out, out_t,
                       partials_out);
  return launch_status("geglu_bwd_delayed_kernel");
}

}  // extern "C"
