// FP8 GEMM for gfx950 (MI355X) on the double-rate f8f6f4 MFMA, with a dequant/bias
// epilogue and a gated-GELU(tanh) epilogue for the MLP gate/up projection.
//
// Semantics replace torch._scaled_mm / cuBLASLt under torchao Float8Linear
// (bongard/float8_training.py:22) and TE's FP8 GEMM under te.Linear
// (bongard/te_linear.py:73-74): C = (A8 . B8^T accumulated in fp32) * sa_inv * sb_inv
// (+ bias), "TN" layout (both operands K-contiguous, as nn.Linear weights are).
//
// Design (one workgroup = 4 wave64, 256 x 256 output tile, K step 128 bytes):
//  - global -> LDS through 16-byte buffer loads (out-of-range rows/K read as zero),
//    staged in VGPRs one K step ahead, double-buffered LDS (2 x 64 KB);
//  - LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at c ^ (r & 7) so
//    that the MFMA fragment reads (8 rows x 16 bytes per lane group) hit all banks;
//  - each wave owns a 128 x 128 sub-tile = 4 x 4 MFMA 32x32x64 tiles (256 fp32 acc);
//    the MFMA "A" operand is the B (weight) tile, so every lane ends up holding four
//    consecutive output columns of one row -> 8-byte bf16 / 16-byte fp32 stores;
//  - workgroups are renumbered so that each XCD (blockIdx % 8 on MI355X) owns a
//    contiguous range of tiles, walked in groups of kGroupM tile rows for L2 reuse.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"

namespace bf8 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;
constexpr int kNumXcd = 8;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset that always reads as zero
constexpr int kTileBytes = kBM * kBK;   // one operand tile per LDS stage (32 KB)

enum Epi { EPI_LINEAR = 0, EPI_GEGLU = 1 };

struct GemmParams {
  const uint8_t* A;
  const uint8_t* B;
  int64_t lda, ldb;
  int M, N, K;           // for GEGLU, N = 2I (rows of W)
  int I;                 // GEGLU intermediate size
  int tiles_m, tiles_n;  // output tiles
  const float* a_sinv;
  const float* b_sinv;
  int b_stride;
  int n_seg;
  int seg_end[4];
  const uint16_t* bias;
  void* C;
  int64_t ldc;
  uint16_t* GU;
  uint32_t* partials;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ void tile_coords(const GemmParams& p, int& tm, int& tn) {
  const int nb = p.tiles_m * p.tiles_n;
  const int b = blockIdx.x;
  // XCD-contiguous renumbering: blocks dispatched to XCD x (b % 8 == x) get ids
  // [x*q + min(x, r), ...) with q = nb / 8, r = nb % 8.
  const int x = b % kNumXcd, idx = b / kNumXcd;
  const int q = nb / kNumXcd, r = nb % kNumXcd;
  const int id = x * q + (x < r ? x : r) + idx;
  const int per_group = kGroupM * p.tiles_n;
  const int g = id / per_group;
  const int first_m = g * kGroupM;
  const int gm = min(p.tiles_m - first_m, kGroupM);
  const int in_g = id - g * per_group;
  tm = first_m + in_g % gm;
  tn = in_g / gm;
}

template <int FA, int FB>
__device__ __forceinline__ v16f mfma(v8i a, v8i b, v16f c) {
  // scale operands 0: plain (unscaled) f8f6f4 MFMA; FA/FB select e4m3 (0) / e5m2 (1).
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, 0, 0, 0, 0);
}

// Reads one MFMA operand fragment: 32 rows starting at `row0` of an LDS tile, K bytes
// [kk*64, kk*64+64): lane l holds row row0 + (l & 31), bytes (l >> 5)*32 .. +31.
__device__ __forceinline__ v8i read_frag(const uint8_t* tile, int row0, int kk, int lane) {
  const int row = row0 + (lane & 31);
  const int c = kk * 4 + (lane >> 5) * 2;
  const int sw = row & 7;
  const uint8_t* base = tile + row * kBK;
  v4u lo = *reinterpret_cast<const v4u*>(base + ((c ^ sw) << 4));
  v4u hi = *reinterpret_cast<const v4u*>(base + (((c + 1) ^ sw) << 4));
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

__device__ __forceinline__ float gelu_tanh_f32(float x) {
  // 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), evaluated in fp32 in the
  // order of PyTorch's CPU kernel for reduced-precision inputs, without FMA contraction.
#pragma clang fp contract(off)
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  float x3 = x * x * x;
  float inner = kBeta * (x + kKappa * x3);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <int FA, int FB, int EPI, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * kTileBytes];
  // stage s: A tile at smem + 2s * kTileBytes, B tile right after it.
  auto sA = [&](int s) { return smem + (2 * s) * kTileBytes; };
  auto sB = [&](int s) { return smem + (2 * s + 1) * kTileBytes; };

  int tm, tn;
  tile_coords(p, tm, tn);
  const int m0 = tm * kBM;
  const int n0 = tn * (EPI == EPI_GEGLU ? kBN / 2 : kBN);  // GEGLU: n0 indexes I

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wid = t >> 6;
  const int wm = wid & 1, wn = wid >> 1;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, (uint32_t)((int64_t)p.M * p.lda));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, (uint32_t)((int64_t)p.N * p.ldb));

  // Loader mapping: thread t moves chunk (t & 7) of rows (t >> 3) + 32 j, j = 0..7.
  const int lrow = t >> 3;
  const int lchunk = t & 7;
  const int lds_chunk = lchunk ^ (lrow & 7);
  uint32_t a_off[8], b_off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = lrow + 32 * j;
    const int am = m0 + r;
    a_off[j] = am < p.M ? (uint32_t)((int64_t)am * p.lda + lchunk * 16) : kOob;
    int bn;
    if (EPI == EPI_GEGLU)
      bn = r < 128 ? n0 + r : p.I + n0 + (r - 128);
    else
      bn = n0 + r;
    const bool bvalid = (EPI == EPI_GEGLU) ? (n0 + (r & 127) < p.I) : (bn < p.N);
    b_off[j] = bvalid ? (uint32_t)((int64_t)bn * p.ldb + lchunk * 16) : kOob;
  }

  v4u pa[8], pb[8];
  auto gload = [&](int k0) {
    const bool kvalid = k0 + lchunk * 16 < p.K;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t oa = (kvalid && a_off[j] != kOob) ? a_off[j] + k0 : kOob;
      const uint32_t ob = (kvalid && b_off[j] != kOob) ? b_off[j] + k0 : kOob;
      pa[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, oa, 0, 0);
      pb[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, ob, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = lrow + 32 * j;
      *reinterpret_cast<v4u*>(sA(buf) + r * kBK + lds_chunk * 16) = pa[j];
      *reinterpret_cast<v4u*>(sB(buf) + r * kBK + lds_chunk * 16) = pb[j];
    }
  };

  // MFMA-A rows (weight tile rows) per n-subtile, MFMA-B rows (activation rows) per m.
  int brow[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (EPI == EPI_GEGLU)
      brow[s] = (s < 2) ? wn * 64 + s * 32 : 128 + wn * 64 + (s - 2) * 32;
    else
      brow[s] = wn * 128 + s * 32;
  }

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int ksteps = (p.K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  int cur = 0;
  for (int ks = 0; ks < ksteps; ++ks) {
    const bool more = ks + 1 < ksteps;
    if (more) gload((ks + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v8i fb[4], fa[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) fb[s] = read_frag(sB(cur), brow[s], kk, lane);
#pragma unroll
      for (int s = 0; s < 4; ++s) fa[s] = read_frag(sA(cur), wm * 128 + s * 32, kk, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma<FB, FA>(fb[i], fa[j], acc[i][j]);
    }
    if (more) sstore(cur ^ 1);
    __syncthreads();
    cur ^= 1;
  }

  // ---- epilogue --------------------------------------------------------------------
  // acc[i][j][r]: n-subtile i, m-subtile j; row m = m0 + wm*128 + j*32 + (lane & 31),
  // column (within the n-subtile) 8*(r/4) + (lane >> 5)*4 + (r & 3).
  const float sa = *p.a_sinv;
  const int lrow_m = lane & 31;
  const int lcol = (lane >> 5) * 4;
  if (EPI == EPI_LINEAR) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * 128 + i * 32 + 8 * q + lcol;
        if (n >= p.N) continue;
        int seg = 0;
#pragma unroll
        for (int s = 0; s < 3; ++s) seg += (s + 1 < p.n_seg && n >= p.seg_end[s]) ? 1 : 0;
        const float alpha = sa * p.b_sinv[seg * p.b_stride];
        float bias[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
          const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + n);
          bias[0] = bf16_lo(bb.x); bias[1] = bf16_hi(bb.x);
          bias[2] = bf16_lo(bb.y); bias[3] = bf16_hi(bb.y);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = m0 + wm * 128 + j * 32 + lrow_m;
          if (m >= p.M) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e] * alpha + bias[e];
          if (OUT == BF8_OUT_BF16) {
            uint16_t* c = reinterpret_cast<uint16_t*>(p.C) + (int64_t)m * p.ldc + n;
            uint2 w;
            w.x = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
            w.y = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
            *reinterpret_cast<uint2*>(c) = w;
          } else {
            float* c = reinterpret_cast<float*>(p.C) + (int64_t)m * p.ldc + n;
            *reinterpret_cast<float4*>(c) = make_float4(v[0], v[1], v[2], v[3]);
          }
        }
      }
    }
  } else {
    // Gated GELU: acc[i] (gate) pairs with acc[i + 2] (up) for i = 0, 1.
    const float ag = sa * p.b_sinv[0];
    const float au = sa * p.b_sinv[p.b_stride];
    uint32_t hmax = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + wn * 64 + i * 32 + 8 * q + lcol;  // column of H (index into I)
        if (col >= p.I) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = m0 + wm * 128 + j * 32 + lrow_m;
          if (m >= p.M) continue;
          uint32_t hb[4], gb[4], ub[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gb[e] = f32_to_bf16_bits(acc[i][j][4 * q + e] * ag);
            ub[e] = f32_to_bf16_bits(acc[i + 2][j][4 * q + e] * au);
            const float g = __uint_as_float(gb[e] << 16);
            const float u = __uint_as_float(ub[e] << 16);
            const float gl = bf16_round(gelu_tanh_f32(g));
            hb[e] = f32_to_bf16_bits(gl * u);
            hmax = max(hmax, (hb[e] & 0x7FFFu) << 16);
          }
          uint16_t* h = reinterpret_cast<uint16_t*>(p.C) + (int64_t)m * p.ldc + col;
          *reinterpret_cast<uint2*>(h) = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
          if (p.GU) {
            uint16_t* g = p.GU + (int64_t)m * (2 * (int64_t)p.I) + col;
            *reinterpret_cast<uint2*>(g) = make_uint2(gb[0] | (gb[1] << 16), gb[2] | (gb[3] << 16));
            *reinterpret_cast<uint2*>(g + p.I) =
                make_uint2(ub[0] | (ub[1] << 16), ub[2] | (ub[3] << 16));
          }
        }
      }
    }
    hmax = block_max_u32<kThreads>(hmax);
    if (t == 0) p.partials[blockIdx.x] = hmax;
  }
}

template <int EPI, int OUT>
int launch_typed(const GemmParams& p, int fa, int fb, hipStream_t s) {
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n)), block(kThreads);
  if (fa == BF8_E4M3 && fb == BF8_E4M3)
    hipLaunchKernelGGL((gemm_kernel<0, 0, EPI, OUT>), grid, block, 0, s, p);
  else if (fa == BF8_E5M2 && fb == BF8_E4M3)
    hipLaunchKernelGGL((gemm_kernel<1, 0, EPI, OUT>), grid, block, 0, s, p);
  else if (fa == BF8_E4M3 && fb == BF8_E5M2)
    hipLaunchKernelGGL((gemm_kernel<0, 1, EPI, OUT>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<1, 1, EPI, OUT>), grid, block, 0, s, p);
  return launch_status("gemm_kernel");
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

size_t bf8_gemm_workspace(int64_t M, int64_t N, int64_t K) {
  (void)M; (void)N; (void)K;
  return 0;
}

int bf8_gemm(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b, int64_t ldb,
             int64_t M, int64_t N, int64_t K, const float* a_scale_inv,
             const float* b_scale_inv, int b_scale_stride, const int64_t* seg_ends, int n_seg,
             const void* bias, void* C, int out_dtype, int64_t ldc, void* ws, size_t ws_bytes,
             void* stream) {
  (void)ws; (void)ws_bytes;
  BF8_CHECK((fmt_a == BF8_E4M3 || fmt_a == BF8_E5M2) && (fmt_b == BF8_E4M3 || fmt_b == BF8_E5M2),
            "bf8_gemm: bad formats %d/%d", fmt_a, fmt_b);
  BF8_CHECK(out_dtype == BF8_OUT_BF16 || out_dtype == BF8_OUT_F32, "bf8_gemm: bad out_dtype");
  BF8_CHECK(M >= 0 && N >= 0 && K >= 0, "bf8_gemm: negative shape");
  BF8_CHECK(K % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && lda >= K && ldb >= K,
            "bf8_gemm: need K, lda, ldb multiples of 16 and lda, ldb >= K (K=%lld lda=%lld ldb=%lld)",
            (long long)K, (long long)lda, (long long)ldb);
  BF8_CHECK(N % 8 == 0 && ldc >= N && ldc % 4 == 0, "bf8_gemm: need N %% 8 == 0, ldc >= N, ldc %% 4 == 0");
  BF8_CHECK(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && ((uintptr_t)C & 15) == 0,
            "bf8_gemm: A, B, C must be 16-byte aligned");
  BF8_CHECK(M * lda < (1LL << 31) && N * ldb < (1LL << 31), "bf8_gemm: operand larger than 2 GiB");
  BF8_CHECK(a_scale_inv && b_scale_inv, "bf8_gemm: scale pointers are NULL");
  BF8_CHECK(n_seg >= 1 && n_seg <= 4, "bf8_gemm: n_seg must be 1..4");
  BF8_CHECK(n_seg == 1 || seg_ends, "bf8_gemm: seg_ends is NULL with n_seg > 1");
  if (M == 0 || N == 0) return BF8_OK;
  GemmParams p{};
  p.A = A; p.B = B; p.lda = lda; p.ldb = ldb;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.I = 0;
  p.tiles_m = (int)((M + kBM - 1) / kBM);
  p.tiles_n = (int)((N + kBN - 1) / kBN);
  p.a_sinv = a_scale_inv; p.b_sinv = b_scale_inv; p.b_stride = b_scale_stride;
  p.n_seg = n_seg;
  for (int s = 0; s < 4; ++s) p.seg_end[s] = (int)N;
  if (n_seg > 1) {
    for (int s = 0; s < n_seg; ++s) {
      BF8_CHECK(seg_ends[s] > (s ? seg_ends[s - 1] : 0) && seg_ends[s] % 4 == 0,
                "bf8_gemm: seg_ends must ascend in multiples of 4");
      p.seg_end[s] = (int)seg_ends[s];
    }
    BF8_CHECK(seg_ends[n_seg - 1] == N, "bf8_gemm: last seg_end must equal N");
  }
  p.bias = (const uint16_t*)bias; p.C = C; p.ldc = ldc;
  BF8_CHECK(((uintptr_t)bias & 7) == 0, "bf8_gemm: bias must be 8-byte aligned");
  hipStream_t s = as_stream(stream);
  if (K == 0) {
    BF8_CHECK(false, "bf8_gemm: K == 0 is not supported");
  }
  if (out_dtype == BF8_OUT_BF16) return launch_typed<EPI_LINEAR, BF8_OUT_BF16>(p, fmt_a, fmt_b, s);
  return launch_typed<EPI_LINEAR, BF8_OUT_F32>(p, fmt_a, fmt_b, s);
}

int64_t bf8_geglu_partials(int64_t M, int64_t I) {
  return ((M + kBM - 1) / kBM) * ((I + kBN / 2 - 1) / (kBN / 2));
}

int bf8_gemm_geglu(const uint8_t* X, int64_t ldx, const uint8_t* W, int64_t ldw, int64_t M,
                   int64_t I, int64_t K, const float* x_scale_inv, const float* w_scale_inv,
                   int w_scale_stride, void* H, int64_t ldh, void* GU, uint32_t* h_partials,
                   void* stream) {
  BF8_CHECK(M >= 1 && I >= 1 && K >= 16, "bf8_gemm_geglu: bad shape");
  BF8_CHECK(I % 128 == 0, "bf8_gemm_geglu: I must be a multiple of 128 (got %lld)", (long long)I);
  BF8_CHECK(K % 16 == 0 && ldx % 16 == 0 && ldw % 16 == 0 && ldx >= K && ldw >= K,
            "bf8_gemm_geglu: need K, ldx, ldw multiples of 16 and >= K");
  BF8_CHECK(ldh >= I && ldh % 4 == 0, "bf8_gemm_geglu: bad ldh");
  BF8_CHECK(((uintptr_t)X & 15) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)H & 15) == 0 &&
                ((uintptr_t)GU & 15) == 0,
            "bf8_gemm_geglu: X, W, H, GU must be 16-byte aligned");
  BF8_CHECK(M * ldx < (1LL << 31) && 2 * I * ldw < (1LL << 31), "bf8_gemm_geglu: operand > 2 GiB");
  BF8_CHECK(x_scale_inv && w_scale_inv && h_partials, "bf8_gemm_geglu: NULL pointer");
  GemmParams p{};
  p.A = X; p.B = W; p.lda = ldx; p.ldb = ldw;
  p.M = (int)M; p.N = (int)(2 * I); p.K = (int)K; p.I = (int)I;
  p.tiles_m = (int)((M + kBM - 1) / kBM);
  p.tiles_n = (int)(I / (kBN / 2));
  p.a_sinv = x_scale_inv; p.b_sinv = w_scale_inv; p.b_stride = w_scale_stride;
  p.n_seg = 1;
  p.C = H; p.ldc = ldh; p.GU = (uint16_t*)GU; p.partials = h_partials;
  return launch_typed<EPI_GEGLU, BF8_OUT_BF16>(p, BF8_E4M3, BF8_E4M3, as_stream(stream));
}

}  // extern "C"
