// FP8 GEMM for gfx950 (MI355X) on the double-rate f8f6f4 MFMA, with a dequant/bias
// epilogue and a gated-GELU(tanh) epilogue for the MLP gate/up projection.
//
// Semantics replace torch._scaled_mm / cuBLASLt under torchao Float8Linear
// (bongard/float8_training.py:22) and TE's FP8 GEMM under te.Linear
// (bongard/te_linear.py:73-74): C = (A8 . B8^T accumulated in fp32) * sa_inv * sb_inv
// (+ bias), "TN" layout (both operands K-contiguous, as nn.Linear weights are).
//
// Design (one workgroup = 4 wave64, 256 x 256 output tile, K step 128 bytes):
//  - global -> LDS by direct 16-byte buffer loads into LDS (no VGPR staging;
//    out-of-range rows/K read as zero), two LDS stages (2 x 64 KB);
//  - LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at c ^ ((r >> 1) & 7)
//    so that a fragment read (16 lanes = 16 rows x 16 bytes per LDS cycle on the 64-bank,
//    256 B/clk gfx950 LDS) touches every bank once;
//  - each wave owns a 128 x 128 sub-tile = 4 x 4 MFMA 32x32x64 tiles (256 fp32 acc);
//    the MFMA "A" operand is the B (weight) tile, so every lane ends up holding four
//    consecutive output columns of one row -> 8-byte bf16 / 16-byte fp32 stores;
//  - workgroups are renumbered so that each XCD (blockIdx % 8 on MI355X) owns a
//    contiguous range of tiles, walked in groups of kGroupM tile rows for L2 reuse.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "common.hpp"

namespace bf8 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kStages = 2;  // LDS pipeline depth (2 x 64 KB)
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
  uint32_t* partials;  // GEGLU: one amax key of |H| per tile
};

typedef int i32x4 __attribute__((ext_vector_type(4)));

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
  // lds_addr and soff are wave-uniform; readfirstlane puts them in SGPRs
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0v), "v"(voff), "s"(srd), "s"(so)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const uint8_t*)(p));
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

// Swizzled position of logical 16-byte chunk c in tile row r (128-byte rows).
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// Reads 16 bytes of an MFMA operand fragment: 32 rows starting at `row0` of an LDS tile,
// K bytes [kk*64, kk*64+64); lane l holds row row0 + (l & 31), bytes (l >> 5)*32 + 16*half
// .. +15 (two halves make the lane's 32 bytes).
__device__ __forceinline__ v4u read_half(const uint8_t* tile, int row0, int kk, int half,
                                         int lane) {
  const int row = row0 + (lane & 31);
  const int c = kk * 4 + (lane >> 5) * 2 + half;
  return *reinterpret_cast<const v4u*>(tile + row * kBK + (swz(row, c) << 4));
}

__device__ __forceinline__ v8i read_frag(const uint8_t* tile, int row0, int kk, int lane) {
  const int row = row0 + (lane & 31);
  const int c = kk * 4 + (lane >> 5) * 2;
  const uint8_t* base = tile + row * kBK;
  v4u lo = *reinterpret_cast<const v4u*>(base + (swz(row, c) << 4));
  v4u hi = *reinterpret_cast<const v4u*>(base + (swz(row, c + 1) << 4));
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 with round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Epilogue staging in LDS: rows of CHUNKS 16-byte chunks; chunk c of row r lives at
// c ^ (r & (CHUNKS - 1)). Lanes put 8-byte runs (4 bf16) and get 16-byte chunks.
template <int CHUNKS>
__device__ __forceinline__ void stage_put(uint8_t* buf, int row, int col, uint2 v) {
  const int c = col >> 3, half = (col >> 2) & 1;
  *reinterpret_cast<uint2*>(buf + row * (CHUNKS * 16) + ((c ^ (row & (CHUNKS - 1))) << 4) +
                            half * 8) = v;
}
template <int CHUNKS>
__device__ __forceinline__ uint4 stage_get(const uint8_t* buf, int row, int c) {
  return *reinterpret_cast<const uint4*>(buf + row * (CHUNKS * 16) +
                                         ((c ^ (row & (CHUNKS - 1))) << 4));
}
// 8 bf16 to global: one 16-byte store when the row stride keeps it aligned.
__device__ __forceinline__ void store_bf16x8(uint16_t* dst, uint4 d, int64_t ld) {
  if ((ld & 7) == 0) {
    *reinterpret_cast<uint4*>(dst) = d;
  } else {
    reinterpret_cast<uint2*>(dst)[0] = make_uint2(d.x, d.y);
    reinterpret_cast<uint2*>(dst)[1] = make_uint2(d.z, d.w);
  }
}


// Stage layout in LDS: [A tile | B tile], each kBM (= kBN) rows of kBK bytes.
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kBlocksPerTile = kTileBytes / 1024;   // 1 KB DMA blocks per operand tile
constexpr int kRowsPerBlock = 1024 / kBK;           // tile rows covered by one DMA block
constexpr int kChunksPerRow = kBK / 16;
constexpr int kDmaPerWave = kBlocksPerTile / 4;     // per operand, per wave, per stage

// Issues one stage of direct global->LDS loads (16 bytes per lane). Lane l of DMA block
// b fills LDS bytes [b*1024 + 16 l, +16): tile row b*kRowsPerBlock + l / kChunksPerRow,
// physical chunk l % kChunksPerRow, i.e. logical chunk swz(row, physical).
__device__ __forceinline__ void dma_stage(i32x4 ra, i32x4 rb, const uint32_t* a_off,
                                          const uint32_t* b_off, uint8_t* stage, int wid,
                                          uint32_t k0) {
  const uint32_t base = lds_addr(stage);
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int blk = wid * kDmaPerWave + j;
    dma16(ra, base + blk * 1024, a_off[j], k0);
    dma16(rb, base + kTileBytes + blk * 1024, b_off[j], k0);
  }
}

// One of the wave's DMA loads of a stage: x = 0..15 -> operand (x & 1: 0 = A, 1 = B),
// block j = x >> 1 of this wave.
__device__ __forceinline__ void dma_one(i32x4 ra, i32x4 rb, const uint32_t* a_off,
                                        const uint32_t* b_off, uint8_t* stage, int wid,
                                        uint32_t k0, int x) {
  const int j = x >> 1;
  const uint32_t dst = lds_addr(stage) + (wid * kDmaPerWave + j) * 1024;
  if ((x & 1) == 0)
    dma16(ra, dst, a_off[j], k0);
  else
    dma16(rb, dst + kTileBytes, b_off[j], k0);
}

// The 8 operand fragments of one MFMA sub-step as 16 halves (16 bytes each), in the order
// the MFMAs of the sub-step consume them: b0, a0, a1, a2, a3, b1, b2, b3.
struct Frags {
  v4u h[16];
};
__device__ __forceinline__ int half_b(int i) { return i == 0 ? 0 : 8 + 2 * i; }
__device__ __forceinline__ int half_a(int j) { return 2 + 2 * j; }
__device__ __forceinline__ v8i frag_of(const Frags& f, int first) {
  const v4u lo = f.h[first], hi = f.h[first + 1];
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

template <int FA, int FB, int EPI, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStageBytes];
  static_assert(kStages == 2, "the main loop below alternates two stages");

  int tm, tn;
  tile_coords(p, tm, tn);
  const int m0 = tm * kBM;
  const int n0 = tn * (EPI == EPI_GEGLU ? kBN / 2 : kBN);  // GEGLU: n0 indexes I

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wid = t >> 6;
  const int wm = wid & 1, wn = wid >> 1;

  const i32x4 ra = make_srd(p.A, (uint32_t)((int64_t)p.M * p.lda));
  const i32x4 rb = make_srd(p.B, (uint32_t)((int64_t)p.N * p.ldb));

  // Per-lane DMA source offsets (without k0) for this wave's blocks of each operand.
  const int lrow = lane / kChunksPerRow;
  const int pchunk = lane % kChunksPerRow;
  uint32_t a_off[kDmaPerWave], b_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int r = (wid * kDmaPerWave + j) * kRowsPerBlock + lrow;  // tile row
    const int c = swz(r, pchunk);                                   // logical chunk
    const int am = m0 + r;
    a_off[j] = am < p.M ? (uint32_t)((int64_t)am * p.lda + c * 16) : kOob;
    int bn;
    bool bvalid;
    if (EPI == EPI_GEGLU) {
      bn = r < 128 ? n0 + r : p.I + n0 + (r - 128);
      bvalid = n0 + (r & 127) < p.I;
    } else {
      bn = n0 + r;
      bvalid = bn < p.N;
    }
    b_off[j] = bvalid ? (uint32_t)((int64_t)bn * p.ldb + c * 16) : kOob;
  }
  // K tail (K % kBK != 0): chunks at or beyond K must read as zero; only the last stage
  // can contain them, and it gets masked offsets.
  const int ksteps = (p.K + kBK - 1) / kBK;
  const bool k_tail = (p.K % kBK) != 0;
  uint32_t a_off_t[kDmaPerWave], b_off_t[kDmaPerWave];
  if (k_tail) {
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int r = (wid * kDmaPerWave + j) * kRowsPerBlock + lrow;
      const int c = swz(r, pchunk);
      const bool cvalid = (ksteps - 1) * kBK + c * 16 < p.K;
      a_off_t[j] = cvalid ? a_off[j] : kOob;
      b_off_t[j] = cvalid ? b_off[j] : kOob;
    }
  }

  // MFMA-A rows (weight tile rows) per n-subtile, MFMA-B rows (activation rows) per m.
  int brow[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (EPI == EPI_GEGLU)
      brow[s] = (s < 2) ? wn * 64 + s * 32 : 128 + wn * 64 + (s - 2) * 32;
    else
      brow[s] = wn * 128 + s * 32;
  }

  // Row of the LDS tile where half h of the sub-step's fragments starts, and its tile.
  auto half_src = [&](int h, const uint8_t* stage, int& row0) -> const uint8_t* {
    const int fr = h >> 1;  // 0: b0, 1..4: a0..a3, 5..7: b1..b3
    if (fr == 0 || fr >= 5) {
      row0 = brow[fr == 0 ? 0 : fr - 4];
      return stage + kTileBytes;
    }
    row0 = wm * 128 + (fr - 1) * 32;
    return stage;
  };
  auto read_one = [&](Frags& f, const uint8_t* stage, int kk, int h) {
    int row0;
    const uint8_t* tile = half_src(h, stage, row0);
    f.h[h] = read_half(tile, row0, kk, h & 1, lane);
  };
  auto load_frags = [&](Frags& f, const uint8_t* stage, int kk) {
#pragma unroll
    for (int h = 0; h < 16; ++h) read_one(f, stage, kk, h);
  };

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // MFMA number x of a sub-step: n-subtile x >> 2, m-subtile x & 3.
  auto mma_one = [&](const Frags& f, int x) {
    const int i = x >> 2, j = x & 3;
    acc[i][j] = mfma<FB, FA>(frag_of(f, half_b(i)), frag_of(f, half_a(j)), acc[i][j]);
  };

  // Pipeline (2 LDS stages, 2 MFMA sub-steps of 64 K-bytes per stage). Iteration ks:
  //   16 x {MFMA(ks, kk=0), read 1/16 of frags(ks, kk=1)} | wait DMA(ks+1) + barrier |
  //   16 x {MFMA(ks, kk=1), read 1/16 of frags(ks+1, kk=0), 1 DMA load of stage ks+2}
  // Each MFMA consumes operands read one sub-step earlier; each DMA has two sub-steps
  // (~2k MFMA cycles) to land; one LDS read and one texture-unit load sit between
  // consecutive MFMAs, so neither unit (both shared by the four waves) blocks MFMA issue.
  // sched_barrier(0) pins the order. Loads past the last stage read zeros (kOob) into a
  // stage that is never read again, which keeps the loop free of branches.
  const uint32_t kend = (uint32_t)ksteps * kBK;
  auto dma = [&](int kstep, uint8_t* stage) {
    const uint32_t k0 = (uint32_t)kstep * kBK;
    if (k_tail && kstep == ksteps - 1)
      dma_stage(ra, rb, a_off_t, b_off_t, stage, wid, k0);
    else
      dma_stage(ra, rb, a_off, b_off, stage, wid, k0);
  };
  dma(0, smem);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  Frags f0, f1;
  load_frags(f0, smem, 0);
  if (ksteps > 1) dma(1, smem + kStageBytes);
  for (int ks = 0; ks < ksteps; ++ks) {
    uint8_t* cur = smem + (ks & 1) * kStageBytes;
    uint8_t* nxt = smem + ((ks & 1) ^ 1) * kStageBytes;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      mma_one(f0, x);
      read_one(f1, cur, 1, x);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // stage ks+2's DMA: zero-fill offsets past K; the K-tail stage uses masked offsets
    const uint32_t k2 = (uint32_t)(ks + 2) * kBK;
    const bool tail2 = k_tail && ks + 2 == ksteps - 1;
    const uint32_t* ao = tail2 ? a_off_t : a_off;
    const uint32_t* bo = tail2 ? b_off_t : b_off;
    const uint32_t k2s = k2 < kend ? k2 : 0x40000000u;  // beyond K: offset >= 2^30 -> OOB
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      mma_one(f1, x);
      read_one(f0, nxt, 0, x);
      dma_one(ra, rb, ao, bo, cur, wid, k2s, x);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The last iteration's zero-fill loads still target LDS: drain them, and let every wave
  // finish with the stages, before the epilogue reuses the space.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- epilogue --------------------------------------------------------------------
  // acc[i][j][r]: n-subtile i, m-subtile j; row m = wm*128 + j*32 + (lane & 31) of the
  // tile, column (within the n-subtile) 8*(r/4) + (lane >> 5)*4 + (r & 3): each lane
  // holds runs of four consecutive columns. bf16 results are staged through this wave's
  // own LDS region of the (now idle) pipeline ring and leave as 16-byte row segments,
  // 16 lanes per 256-byte row.
  const float sa = *p.a_sinv;
  const int lrow_m = lane & 31;
  const int lcol = (lane >> 5) * 4;
  if (EPI == EPI_LINEAR && OUT == BF8_OUT_BF16) {
    uint8_t* wbuf = smem + wid * (128 * 256);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = i * 32 + 8 * q + lcol;  // within the wave's 128 columns
        const int n = n0 + wn * 128 + col;
        int seg = 0;
#pragma unroll
        for (int s2 = 0; s2 < 3; ++s2) seg += (s2 + 1 < p.n_seg && n >= p.seg_end[s2]) ? 1 : 0;
        const float alpha = sa * p.b_sinv[seg * p.b_stride];
        float bias[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias && n < p.N) {
          const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + n);
          bias[0] = bf16_lo(bb.x); bias[1] = bf16_hi(bb.x);
          bias[2] = bf16_lo(bb.y); bias[3] = bf16_hi(bb.y);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint2 w;
          w.x = pack_bf16x2(acc[i][j][4 * q + 0] * alpha + bias[0], acc[i][j][4 * q + 1] * alpha + bias[1]);
          w.y = pack_bf16x2(acc[i][j][4 * q + 2] * alpha + bias[2], acc[i][j][4 * q + 3] * alpha + bias[3]);
          stage_put<16>(wbuf, j * 32 + lrow_m, col, w);
        }
      }
    }
    const int gn = n0 + wn * 128 + (lane & 15) * 8;
#pragma unroll 4
    for (int it = 0; it < 32; ++it) {
      const int row = it * 4 + (lane >> 4);
      const uint4 d = stage_get<16>(wbuf, row, lane & 15);
      const int gm = m0 + wm * 128 + row;
      if (gm < p.M && gn < p.N)
        store_bf16x8(reinterpret_cast<uint16_t*>(p.C) + (int64_t)gm * p.ldc + gn, d, p.ldc);
    }
  } else if (EPI == EPI_LINEAR) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * 128 + i * 32 + 8 * q + lcol;
        if (n >= p.N) continue;
        int seg = 0;
#pragma unroll
        for (int s2 = 0; s2 < 3; ++s2) seg += (s2 + 1 < p.n_seg && n >= p.seg_end[s2]) ? 1 : 0;
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
          float* c = reinterpret_cast<float*>(p.C) + (int64_t)m * p.ldc + n;
          *reinterpret_cast<float4*>(c) =
              make_float4(acc[i][j][4 * q + 0] * alpha + bias[0], acc[i][j][4 * q + 1] * alpha + bias[1],
                          acc[i][j][4 * q + 2] * alpha + bias[2], acc[i][j][4 * q + 3] * alpha + bias[3]);
        }
      }
    }
  } else {
    // Gated GELU: acc[i] (gate) pairs with acc[i + 2] (up) for i = 0, 1. The wave owns
    // H rows wm*128 .. +128 and columns wn*64 .. +64 of this tile (128-byte LDS rows).
    // Pass 0 stages H (and accumulates its amax); passes 1, 2 stage the bf16 gate / up
    // pre-activations when the caller keeps them for the backward.
    const float ag = sa * p.b_sinv[0];
    const float au = sa * p.b_sinv[p.b_stride];
    uint8_t* wbuf = smem + wid * (128 * 128);
    uint32_t hmax = 0;
    auto run_pass = [&](auto pass_tag) {
      constexpr int pass = decltype(pass_tag)::value;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = i * 32 + 8 * q + lcol;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float ga[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                 acc[i][j][4 * q + 3]};
            const float ua[4] = {acc[i + 2][j][4 * q], acc[i + 2][j][4 * q + 1],
                                 acc[i + 2][j][4 * q + 2], acc[i + 2][j][4 * q + 3]};
            uint32_t w0, w1;  // packed bf16 pairs (columns 0-1, 2-3 of the run)
            if constexpr (pass == 0) {
              const uint32_t g01 = pack_bf16x2(ga[0] * ag, ga[1] * ag);
              const uint32_t g23 = pack_bf16x2(ga[2] * ag, ga[3] * ag);
              const uint32_t u01 = pack_bf16x2(ua[0] * au, ua[1] * au);
              const uint32_t u23 = pack_bf16x2(ua[2] * au, ua[3] * au);
              const uint32_t l01 = pack_bf16x2(gelu_tanh_f32(bf16_lo(g01)), gelu_tanh_f32(bf16_hi(g01)));
              const uint32_t l23 = pack_bf16x2(gelu_tanh_f32(bf16_lo(g23)), gelu_tanh_f32(bf16_hi(g23)));
              w0 = pack_bf16x2(bf16_lo(l01) * bf16_lo(u01), bf16_hi(l01) * bf16_hi(u01));
              w1 = pack_bf16x2(bf16_lo(l23) * bf16_lo(u23), bf16_hi(l23) * bf16_hi(u23));
              const uint32_t a0 = w0 & 0x7FFF7FFFu, a1 = w1 & 0x7FFF7FFFu;
              hmax = max(hmax, max(max(a0 << 16, a0 & 0xFFFF0000u), max(a1 << 16, a1 & 0xFFFF0000u)));
            } else if constexpr (pass == 1) {
              w0 = pack_bf16x2(ga[0] * ag, ga[1] * ag);
              w1 = pack_bf16x2(ga[2] * ag, ga[3] * ag);
            } else {
              w0 = pack_bf16x2(ua[0] * au, ua[1] * au);
              w1 = pack_bf16x2(ua[2] * au, ua[3] * au);
            }
            stage_put<8>(wbuf, j * 32 + lrow_m, col, make_uint2(w0, w1));
          }
        }
      }
      uint16_t* dst = pass == 0 ? reinterpret_cast<uint16_t*>(p.C) : p.GU;
      const int64_t ld = pass == 0 ? p.ldc : 2 * (int64_t)p.I;
      const int coff = pass == 2 ? p.I : 0;
      const int gcol = coff + n0 + wn * 64 + (lane & 7) * 8;
#pragma unroll 4
      for (int it = 0; it < 16; ++it) {
        const int row = it * 8 + (lane >> 3);
        const uint4 d = stage_get<8>(wbuf, row, lane & 7);
        const int gm = m0 + wm * 128 + row;
        if (gm < p.M) store_bf16x8(dst + (int64_t)gm * ld + gcol, d, ld);
      }
    };
    run_pass(std::integral_constant<int, 0>{});
    if (p.GU) {
      run_pass(std::integral_constant<int, 1>{});
      run_pass(std::integral_constant<int, 2>{});
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
