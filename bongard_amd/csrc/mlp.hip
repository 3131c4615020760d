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

}  // extern "C"
