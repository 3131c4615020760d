// The gated GELU(tanh) between the MLP's gate/up and down projections as elementwise
// kernels: its forward on given pre-activations, and its backward.
//
// Forward (bongard/te_linear.py:103): h = bf16(bf16(gelu_tanh(g)) * u) on bf16 g, u.
// Autograd of that bf16 chain gives, per element:
//   a   = bf16(gelu_tanh(g))                 (the forward's activation)
//   d_a = bf16(dh * u)                       (mul backward, grad wrt a)
//   d_u = bf16(dh * a)                       (mul backward, grad wrt u)
//   d_g = bf16(d_a * F(g))                   (gelu backward, fp32 factor F of g)
// a and F come from the tables of gelu.hpp, so every value is bit-identical to torch's CPU
// chain. Each kernel is one streaming pass that also writes per-block amax partials of its
// output (|H| or |dGU|), from which the following e4m3 / e5m2 cast derives its scale.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"
#include "gelu.hpp"

namespace bf8 {
namespace {

constexpr int kNT = 256;
// Every block copies the gelu tables (34 KB) into LDS first, so the streaming grids stay
// at a few blocks per CU.
constexpr int64_t kMaxBlocks = 1024;

int64_t bwd_blocks(int64_t M, int64_t I) {
  const int64_t vec = M * I / 8;
  int64_t b = (vec + kNT - 1) / kNT;
  if (b < 1) b = 1;
  return b < kMaxBlocks ? b : kMaxBlocks;
}


// The chain for 8 elements (4 packed bf16 pairs of dh, g, u): d_g, d_u as packed bf16
// pairs (NaNs 0xFFFF) and the running amax key of |d_g|, |d_u|. ta / tf: the LDS copies
// of the gelu tables; all 16 table reads are issued before any is used, gates outside the
// tables take a wave-uniform slow path.
__device__ __forceinline__ void geglu_bwd8(const uint32_t (&dhw)[4], const uint32_t (&gw)[4],
                                           const uint32_t (&uw)[4], const uint16_t* ta,
                                           const uint32_t* tf, uint32_t (&dg)[4],
                                           uint32_t (&du)[4], uint32_t& m) {
  uint32_t outside = 0, ia[4], jf[4], va[8], vf[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    ia[w] = gelu_index2(gw[w], outside);
    jf[w] = gelu_factor_index2(gw[w], outside);
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    va[2 * w] = ta[ia[w] & 0xFFFFu];
    va[2 * w + 1] = ta[ia[w] >> 16];
    vf[2 * w] = tf[jf[w] & 0xFFFFu];
    vf[2 * w + 1] = tf[jf[w] >> 16];
  }
  if (__builtin_expect(__any(outside != 0), 0)) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      va[2 * w] = gelu_finish(gw[w], va[2 * w]);
      va[2 * w + 1] = gelu_finish(gw[w] >> 16, va[2 * w + 1]);
      vf[2 * w] = gelu_factor_finish(gw[w], vf[2 * w]);
      vf[2 * w + 1] = gelu_factor_finish(gw[w] >> 16, vf[2 * w + 1]);
    }
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float d0 = bf16_lo(dhw[w]), d1 = bf16_hi(dhw[w]);
    const uint32_t a = va[2 * w] | (va[2 * w + 1] << 16);                          // bf16(gelu(g))
    const uint32_t da = pack_bf16x2(d0 * bf16_lo(uw[w]), d1 * bf16_hi(uw[w]));    // bf16(dh * u)
    du[w] = nan_ffff_bf16x2(pack_bf16x2(d0 * bf16_lo(a), d1 * bf16_hi(a)));
    dg[w] = nan_ffff_bf16x2(pack_bf16x2(bf16_lo(da) * __uint_as_float(vf[2 * w]),
                                        bf16_hi(da) * __uint_as_float(vf[2 * w + 1])));
    const uint32_t kg = dg[w] & 0x7FFF7FFFu, ku = du[w] & 0x7FFF7FFFu;
    m = max(m, max(max(kg << 16, kg & 0xFFFF0000u), max(ku << 16, ku & 0xFFFF0000u)));
  }
}

// H for 8 elements (4 packed pairs of g, u), with the table reads issued together.
__device__ __forceinline__ uint4 geglu_fwd8(uint4 g, uint4 u, const uint16_t* ta) {
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t outside = 0, ia[4], va[8], h[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) ia[w] = gelu_index2(gw[w], outside);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    va[2 * w] = ta[ia[w] & 0xFFFFu];
    va[2 * w + 1] = ta[ia[w] >> 16];
  }
  if (__builtin_expect(__any(outside != 0), 0)) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      va[2 * w] = gelu_finish(gw[w], va[2 * w]);
      va[2 * w + 1] = gelu_finish(gw[w] >> 16, va[2 * w + 1]);
    }
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) h[w] = geglu_mul_bf16x2(va[2 * w] | (va[2 * w + 1] << 16), uw[w]);
  return make_uint4(h[0], h[1], h[2], h[3]);
}

// H [M, I] = gelu(g) * u from GU [M, 2I] (gate | up), and per-block amax keys of |H|.
__global__ __launch_bounds__(kNT) void geglu_fwd_kernel(const uint16_t* __restrict__ GU,
                                                        int64_t M, int64_t I,
                                                        uint16_t* __restrict__ H,
                                                        uint32_t* __restrict__ partials) {
  __shared__ __attribute__((aligned(16))) uint16_t ta[kGeluABytes / 2];
  load_gelu_tables<kNT>(ta, nullptr);
  __syncthreads();
  const int64_t per_row = I / 8;
  const int64_t nvec = M * per_row;
  const int64_t stride = (int64_t)gridDim.x * kNT;
  uint32_t m = 0;
  for (int64_t v = (int64_t)blockIdx.x * kNT + threadIdx.x; v < nvec; v += stride) {
    const int64_t row = v / per_row;
    const int64_t col = (v - row * per_row) * 8;
    const uint4 g = *reinterpret_cast<const uint4*>(GU + row * 2 * I + col);
    const uint4 u = *reinterpret_cast<const uint4*>(GU + row * 2 * I + I + col);
    const uint4 h = geglu_fwd8(g, u, ta);
    const uint32_t k = pk_max_u16(pk_max_u16(h.x & 0x7FFF7FFFu, h.y & 0x7FFF7FFFu),
                                  pk_max_u16(h.z & 0x7FFF7FFFu, h.w & 0x7FFF7FFFu));
    m = max(m, max(k << 16, k & 0xFFFF0000u));
    *reinterpret_cast<uint4*>(H + row * I + col) = h;
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

__global__ __launch_bounds__(kNT) void geglu_bwd_kernel(const uint16_t* __restrict__ dH,
                                                        const uint16_t* __restrict__ GU,
                                                        int64_t M, int64_t I,
                                                        uint16_t* __restrict__ dGU,
                                                        uint32_t* __restrict__ partials) {
  __shared__ __attribute__((aligned(16))) uint16_t ta[kGeluABytes / 2];
  __shared__ __attribute__((aligned(16))) uint32_t tf[kGeluFBytes / 4];
  load_gelu_tables<kNT>(ta, tf);
  __syncthreads();
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
    geglu_bwd8(dhw, gw, uw, ta, tf, dg, du, m);
    *reinterpret_cast<uint4*>(dGU + row * 2 * I + col) = make_uint4(dg[0], dg[1], dg[2], dg[3]);
    *reinterpret_cast<uint4*>(dGU + row * 2 * I + I + col) = make_uint4(du[0], du[1], du[2], du[3]);
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// The geglu backward fused with its delayed-scaling cast (for 'fp8_delayed', where dGU's
// scale is known before dGU exists): the same per-element chain as geglu_bwd_kernel, the
// bf16 d_g, d_u quantized at once with the role's delayed scale, written as fp8 rows
// [M, 2I] and/or transposed as fp8 [2I, M] (the wgrad layout), plus this step's amax
// partials of |dGU|. One 64-row x 64-column tile of I per wave: the wave streams it in
// 8-row pieces (dH, g, u: 16-byte loads, four pieces in flight), stages the fp8 d_g and
// d_u bytes in its own LDS regions and reads them back transposed (wave_transpose64_staged).
// Identical bytes to geglu_bwd_kernel followed by the delayed cast of its output.
constexpr int kTT = 64;
constexpr int kFusedWaves = kNT / 64;
constexpr int64_t kMaxFusedBlocks = 512;

int64_t fused_blocks(int64_t M, int64_t I) {
  const int64_t tiles = ((M + kTT - 1) / kTT) * (I / kTT);
  const int64_t blocks = (tiles + kFusedWaves - 1) / kFusedWaves;
  return blocks < 1 ? 1 : (blocks < kMaxFusedBlocks ? blocks : kMaxFusedBlocks);
}

template <int FMT>
__global__ __launch_bounds__(kNT) void geglu_bwd_delayed_kernel(
    const uint16_t* __restrict__ dH, const uint16_t* __restrict__ GU, int64_t M, int64_t I,
    float* __restrict__ state, int len, int pos, const uint32_t* __restrict__ prev,
    int64_t n_prev, float* __restrict__ meta_out, uint8_t* __restrict__ out,
    uint8_t* __restrict__ out_t, uint32_t* __restrict__ partials) {
  __shared__ uint32_t stage[kFusedWaves][2][kWaveTileDwords];
  __shared__ __attribute__((aligned(16))) uint16_t ta[kGeluABytes / 2];
  __shared__ __attribute__((aligned(16))) uint32_t tf[kGeluFBytes / 4];
  load_gelu_tables<kNT>(ta, tf);  // the scale step below synchronises the block
  const float scale =
      delayed_scale_block<kNT>(state, len, pos, prev, n_prev, Fp8Max<FMT>::value, meta_out,
                               blockIdx.x == 0);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t tiles_c = I / kTT;
  const int64_t ntiles = tiles_c * ((M + kTT - 1) / kTT);
  const int ch = lane & 7;  // 16-byte chunk of the piece's rows
  uint32_t* lg = stage[wid][0];
  uint32_t* lu = stage[wid][1];
  uint32_t m = 0;
  for (int64_t tile_id = (int64_t)blockIdx.x * kFusedWaves + wid; tile_id < ntiles;
       tile_id += (int64_t)gridDim.x * kFusedWaves) {
    const int64_t r0 = (tile_id / tiles_c) * kTT, c0 = (tile_id % tiles_c) * kTT;
    const int64_t c = c0 + 8 * ch;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint4 dh[4], g[4], u[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t r = r0 + 32 * half + 8 * k + (lane >> 3);
        dh[k] = g[k] = u[k] = make_uint4(0u, 0u, 0u, 0u);
        if (r < M) {
          dh[k] = *reinterpret_cast<const uint4*>(dH + r * I + c);
          g[k] = *reinterpret_cast<const uint4*>(GU + r * 2 * I + c);
          u[k] = *reinterpret_cast<const uint4*>(GU + r * 2 * I + I + c);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int lr = 32 * half + 8 * k + (lane >> 3);
        const int64_t r = r0 + lr;
        const uint32_t dhw[4] = {dh[k].x, dh[k].y, dh[k].z, dh[k].w};
        const uint32_t gw[4] = {g[k].x, g[k].y, g[k].z, g[k].w};
        const uint32_t uw[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
        uint32_t dg[4], du[4];
        geglu_bwd8(dhw, gw, uw, ta, tf, dg, du, m);
        const uint2 qg = quant8_bf16<FMT>(make_uint4(dg[0], dg[1], dg[2], dg[3]), scale);
        const uint2 qu = quant8_bf16<FMT>(make_uint4(du[0], du[1], du[2], du[3]), scale);
        if (out && r < M) {
          *reinterpret_cast<uint2*>(out + r * 2 * I + c) = qg;
          *reinterpret_cast<uint2*>(out + r * 2 * I + I + c) = qu;
        }
        lg[lr * kWaveTilePitch + 2 * ch] = qg.x;
        lg[lr * kWaveTilePitch + 2 * ch + 1] = qg.y;
        lu[lr * kWaveTilePitch + 2 * ch] = qu.x;
        lu[lr * kWaveTilePitch + 2 * ch + 1] = qu.y;
      }
    }
    if (out_t) {
      const int64_t tc = r0 + (lane >> 4) * 16;  // column of out_t (a row of dGU)
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        uint4 tq[4];
        wave_transpose64_staged(which ? lu : lg, lane, tq);
        if (tc < M) {  // M % 16 == 0: whole 16-byte segments
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            const int64_t tr = (which ? I : 0) + c0 + 4 * (lane & 15) + cc;  // row of out_t
            *reinterpret_cast<uint4*>(out_t + tr * M + tc) = tq[cc];
          }
        }
      }
    }
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// geglu_bwd_delayed_kernel without the transposed output (the K-major backward reads dGU
// as it is): a grid-stride stream over 8-element vectors of [M, I], kRowVecs per thread
// per pass with all their loads issued first, so a wave writes 512 contiguous fp8 bytes of
// d_g and of d_u per vector slot. Same chain, scale, bytes and partials count.
constexpr int kRowVecs = 4;

template <int FMT>
__global__ __launch_bounds__(kNT) void geglu_bwd_delayed_rows_kernel(
    const uint16_t* __restrict__ dH, const uint16_t* __restrict__ GU, int64_t M, int64_t I,
    float* __restrict__ state, int len, int pos, const uint32_t* __restrict__ prev,
    int64_t n_prev, float* __restrict__ meta_out, uint8_t* __restrict__ out,
    uint32_t* __restrict__ partials) {
  __shared__ __attribute__((aligned(16))) uint16_t ta[kGeluABytes / 2];
  __shared__ __attribute__((aligned(16))) uint32_t tf[kGeluFBytes / 4];
  load_gelu_tables<kNT>(ta, tf);  // the scale step below synchronises the block
  const float scale =
      delayed_scale_block<kNT>(state, len, pos, prev, n_prev, Fp8Max<FMT>::value, meta_out,
                               blockIdx.x == 0);
  const int64_t per_row = I / 8;
  const int64_t nvec = M * per_row;
  const int64_t pass = (int64_t)gridDim.x * kNT * kRowVecs;
  uint32_t m = 0;
  for (int64_t v0 = (int64_t)blockIdx.x * kNT * kRowVecs + threadIdx.x; v0 < nvec; v0 += pass) {
    uint4 dh[kRowVecs], g[kRowVecs], u[kRowVecs];
    int64_t eo[kRowVecs], go[kRowVecs];  // element offsets in dH / out and in GU
#pragma unroll
    for (int j = 0; j < kRowVecs; ++j) {
      const int64_t v = v0 + (int64_t)j * kNT;
      const int64_t vv = v < nvec ? v : nvec - 1;  // loads of a clamped vector, not stored
      const int64_t row = vv / per_row;
      const int64_t col = (vv - row * per_row) * 8;
      eo[j] = row * I + col;
      go[j] = row * 2 * I + col;
      dh[j] = *reinterpret_cast<const uint4*>(dH + eo[j]);
      g[j] = *reinterpret_cast<const uint4*>(GU + go[j]);
      u[j] = *reinterpret_cast<const uint4*>(GU + go[j] + I);
    }
#pragma unroll
    for (int j = 0; j < kRowVecs; ++j) {
      const uint32_t dhw[4] = {dh[j].x, dh[j].y, dh[j].z, dh[j].w};
      const uint32_t gw[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
      const uint32_t uw[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
      uint32_t dg[4], du[4], mj = 0;
      geglu_bwd8(dhw, gw, uw, ta, tf, dg, du, mj);
      if (v0 + (int64_t)j * kNT < nvec) {
        m = max(m, mj);
        *reinterpret_cast<uint2*>(out + go[j]) =
            quant8_bf16<FMT>(make_uint4(dg[0], dg[1], dg[2], dg[3]), scale);
        *reinterpret_cast<uint2*>(out + go[j] + I) =
            quant8_bf16<FMT>(make_uint4(du[0], du[1], du[2], du[3]), scale);
      }
    }
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

int64_t bf8_geglu_partials_elementwise(int64_t M, int64_t I) { return bwd_blocks(M, I); }

int bf8_geglu_bf16(const void* GU, int64_t M, int64_t I, void* H, uint32_t* partials,
                   void* stream) {
  BF8_CHECK(M >= 0 && I >= 8 && I % 8 == 0, "bf8_geglu_bf16: need I %% 8 == 0 (I=%lld)", (long long)I);
  BF8_CHECK(GU && H && partials, "bf8_geglu_bf16: NULL pointer");
  BF8_CHECK((((uintptr_t)GU | (uintptr_t)H) & 15) == 0,
            "bf8_geglu_bf16: pointers must be 16-byte aligned");
  const int64_t nb = bwd_blocks(M, I);
  hipLaunchKernelGGL(geglu_fwd_kernel, dim3((unsigned)nb), dim3(kNT), 0, as_stream(stream),
                     (const uint16_t*)GU, M, I, (uint16_t*)H, partials);
  return launch_status("geglu_fwd_kernel");
}

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
  if (!out_t) {
    if (fmt == BF8_E4M3)
      hipLaunchKernelGGL(geglu_bwd_delayed_rows_kernel<BF8_E4M3>, dim3((unsigned)nb), dim3(kNT), 0,
                         s, dh, gu, M, I, state, len, pos, prev_partials, n_prev, meta_out, out,
                         partials_out);
    else
      hipLaunchKernelGGL(geglu_bwd_delayed_rows_kernel<BF8_E5M2>, dim3((unsigned)nb), dim3(kNT), 0,
                         s, dh, gu, M, I, state, len, pos, prev_partials, n_prev, meta_out, out,
                         partials_out);
    return launch_status("geglu_bwd_delayed_rows_kernel");
  }
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
