// Per-tensor amax, scale and saturating bf16 -> fp8 cast kernels for gfx950.
//
// Arithmetic follows torchao's tensorwise current scaling (tensor_to_amax,
// amax_to_scale, to_fp8_saturated) as reached from bongard/float8_training.py:22 and
// TE Float8CurrentScaling (bongard/te_linear.py:38-39,73-74): amax = max|x| (exact for
// bf16), scale = fp32(fp8_max / clamp(f64(amax), 1e-12)), q = fp8_rne(clamp(f32(x) *
// scale, +-fp8_max)).
//
// Current scaling needs the whole tensor's amax before the first byte is cast, so a
// quantization is two streaming passes: amax_partials_kernel writes one max per block
// (at most kMaxAmaxBlocks, plain stores, no atomics), and the cast kernel reduces those
// partials in every block (a <= 4 KB read, overlapped with the block's first data
// loads) to the scale before it streams the data; its block 0 publishes the meta record.
// The same cast kernel consumes the per-tile partials of H written by the gate/up GEMM
// epilogue and those of dGU written by the gated-GELU backward. Streaming loads and
// stores are plain 16-byte vector accesses, several in flight per lane (the non-temporal
// hint measured up to 30% slower on gfx950 for these streams).
//
// Delayed scaling (amax history, TE DelayedScaling semantics) needs no pre-pass: the
// cast kernel derives the scale from the history (after folding in the previous step's
// amax partials) and writes this step's amax partials while it casts, so a delayed
// quantization is one streaming pass and one launch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace bf8 {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return BF8_ELAUNCH;
  }
  return BF8_OK;
}

namespace {

constexpr int kNT = 256;            // threads per block for streaming kernels
constexpr int kVecPerThread = 8;    // 16-byte loads in flight per lane (amax)
constexpr int64_t kMaxAmaxBlocks = 1024;  // 4 blocks per CU; consumers read <= 4 KB of partials
constexpr int64_t kMaxCastBlocks = 2048;  // 8 blocks per CU
// Consumers reduce up to this many partials in every block; a longer list (the gated-GELU
// GEMM writes one per tile: 5200 at M = 16.6k) is first reduced by a one-block kernel.
constexpr int64_t kMaxInlinePartials = 2048;
// Slots of the library-owned scratch of bf8_quantize_bf16_noalloc: the most amax partials
// any tensor's quantization writes.
constexpr int64_t kNoAllocSlots = kMaxAmaxBlocks;

int64_t amax_blocks(int64_t n) {
  int64_t per_block = (int64_t)kNT * kVecPerThread * 8;  // bf16 elements per block pass
  int64_t b = (n + per_block - 1) / per_block;
  if (b < 1) b = 1;
  return b < kMaxAmaxBlocks ? b : kMaxAmaxBlocks;
}

int grid_for_stream(int64_t work_items, int64_t per_block, int64_t cap) {
  int64_t b = (work_items + per_block - 1) / per_block;
  if (b < 1) b = 1;
  return (int)(b < cap ? b : cap);
}

// partials[blk] = max over the grid-stride share of |x| keys of block blk of the nblk
// blocks that read x.
__device__ __forceinline__ void amax_partials_body(const uint16_t* __restrict__ x, int64_t n,
                                                   uint32_t* __restrict__ partials,
                                                   int64_t blk, int64_t nblk) {
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const int64_t nvec = n >> 3;
  constexpr int64_t kChunk = (int64_t)kNT * kVecPerThread;  // vectors per block pass
  const int64_t stride = nblk * kChunk;
  uint32_t m = 0;
  int64_t i = blk * kChunk + threadIdx.x;
  // kVecPerThread independent 16-byte loads per lane in flight (HBM latency x bandwidth
  // needs ~32 MB in flight chip-wide), each pass of a block one contiguous 32 KB chunk,
  // also in the last, partial round: its missing loads are zero vectors (key 0), so a tail
  // never degrades to one load in flight at a time
  for (; i < nvec; i += stride) {
    uint4 v[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
      v[j] = i + j * kNT < nvec ? xv[i + j * kNT] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) m = max(m, absmax_key8(v[j]));
  }
  // scalar tail (n % 8), handled by the first block
  if (blk == 0) {
    for (int64_t j = (nvec << 3) + threadIdx.x; j < n; j += kNT)
      m = max(m, (uint32_t)(x[j] & 0x7FFFu) << 16);
  }
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) partials[blk] = m;
}

__global__ __launch_bounds__(kNT) void amax_partials_kernel(const uint16_t* __restrict__ x,
                                                            int64_t n,
                                                            uint32_t* __restrict__ partials) {
  amax_partials_body(x, n, partials, blockIdx.x, gridDim.x);
}

// One block of 1024 threads, four independent loads per thread and pass: a producer with
// thousands of partials (the gated-GELU GEMM's one per tile: 5,840 at M = 18494) is
// reduced in a few memory round trips (c3: 8.3 -> 5.0 us per call, against one block of
// 256 threads with one load each per pass).
constexpr int kScaleNT = 1024;
__global__ __launch_bounds__(kScaleNT) void scale_from_partials_kernel(
    const uint32_t* __restrict__ partials, int64_t np, float fp8_max, int pow2,
    float* __restrict__ meta) {
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < np; i += 4 * kScaleNT) {
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = i + j * kScaleNT < np ? partials[i + j * kScaleNT] : 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) m = max(m, v[j]);
  }
  m = block_max_u32<kScaleNT>(m);
  if (threadIdx.x == 0) write_meta_from_amax(m, fp8_max, meta, pow2 != 0);
}

// Where a cast kernel takes its scale from (exactly one source):
//  - `scale`: a device fp32 scalar;
//  - current scaling: `partials` (np amax partials of x or of its producer), reduced in
//    every block; block 0 publishes meta_out = {amax, scale, scale_inv, 0}; `pow2` rounds
//    that scale down to a power of two;
//  - delayed scaling: `state` (amax history [len] + meta), which first absorbs the
//    previous step's amax (`prev`, n_prev partials; none on the first step) at slot pos;
//    block 0 copies this step's meta to meta_out (if not NULL).
struct ScaleSrc {
  const float* scale;
  const uint32_t* partials;
  int64_t np;
  float* meta_out;
  float* state;
  int len, pos;
  const uint32_t* prev;
  int64_t n_prev;
  int pow2;
};

template <int FMT>
__device__ __forceinline__ float resolve_scale(const ScaleSrc& s, bool leader) {
  if (s.scale) return *s.scale;
  if (s.state)
    return delayed_scale_block<kNT>(s.state, s.len, s.pos, s.prev, s.n_prev, Fp8Max<FMT>::value,
                                    s.meta_out, leader);
  return scale_from_partials_block<kNT>(s.partials, s.np, Fp8Max<FMT>::value, s.meta_out,
                                        s.pow2 != 0, leader);
}

// Block max of the lanes' amax keys, stored as this block's partial (amax_out != NULL).
__device__ __forceinline__ void store_block_amax(uint32_t m, uint32_t* amax_out, int64_t blk) {
  if (!amax_out) return;
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) amax_out[blk] = m;
}

// Row-major cast: each lane converts 16 consecutive bf16 (two 16-byte loads) into one
// 16-byte store. n16 = number of 16-element groups; the n % 16 tail is done bytewise.
// With amax_out, each block also writes the max |x| key of the elements it cast.
// Block blk of the nblk blocks that cast x; blk == 0 leads (publishes the meta record).
template <int FMT>
__device__ __forceinline__ void cast_body(const uint16_t* __restrict__ x, int64_t n,
                                          const ScaleSrc& src, uint8_t* __restrict__ out,
                                          uint32_t* __restrict__ amax_out, int64_t blk,
                                          int64_t nblk) {
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  uint4* ov = reinterpret_cast<uint4*>(out);
  const int64_t n16 = n >> 4;
  const int64_t step = 2 * nblk * kNT;  // groups per pass of the grid
  int64_t i = blk * 2 * kNT + threadIdx.x;
  // Two 16-element groups (i, i + kNT) per lane and iteration, so each pass of a block
  // reads one contiguous 16 KB chunk; the next iteration's four loads are issued before
  // this one is converted, and the first iteration's before the scale is resolved (whose
  // partial-amax reduction then overlaps them).
  uint4 a0 = make_uint4(0u, 0u, 0u, 0u), a1 = a0, b0 = a0, b1 = a0;
  if (i < n16) { a0 = xv[2 * i]; a1 = xv[2 * i + 1]; }
  if (i + kNT < n16) { b0 = xv[2 * (i + kNT)]; b1 = xv[2 * (i + kNT) + 1]; }
  const float scale = resolve_scale<FMT>(src, blk == 0);
  uint32_t m = 0;
  for (; i < n16; i += step) {
    const uint4 c0 = a0, c1 = a1, d0 = b0, d1 = b1;
    const int64_t inext = i + step;
    if (inext < n16) { a0 = xv[2 * inext]; a1 = xv[2 * inext + 1]; }
    if (inext + kNT < n16) { b0 = xv[2 * (inext + kNT)]; b1 = xv[2 * (inext + kNT) + 1]; }
    if (amax_out) m = max(m, max(absmax_key8(c0), absmax_key8(c1)));
    const uint2 qc0 = quant8_bf16<FMT>(c0, scale), qc1 = quant8_bf16<FMT>(c1, scale);
    ov[i] = make_uint4(qc0.x, qc0.y, qc1.x, qc1.y);
    if (i + kNT < n16) {
      if (amax_out) m = max(m, max(absmax_key8(d0), absmax_key8(d1)));
      const uint2 qd0 = quant8_bf16<FMT>(d0, scale), qd1 = quant8_bf16<FMT>(d1, scale);
      ov[i + kNT] = make_uint4(qd0.x, qd0.y, qd1.x, qd1.y);
    }
  }
  if (blk == 0) {
    for (int64_t j = (n16 << 4) + threadIdx.x; j < n; j += kNT) {
      float xf = __uint_as_float((uint32_t)x[j] << 16);
      float p = xf * scale;
      out[j] = (uint8_t)(quant4<FMT>(p, 0.f, 0.f, 0.f, xf, 0.f, 0.f, 0.f, scale) & 0xFFu);
      m = max(m, (uint32_t)(x[j] & 0x7FFFu) << 16);
    }
  }
  store_block_amax(m, amax_out, blk);
}

template <int FMT>
__global__ __launch_bounds__(kNT) void cast_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                   ScaleSrc src, uint8_t* __restrict__ out,
                                                   uint32_t* __restrict__ amax_out) {
  cast_body<FMT>(x, n, src, out, amax_out, blockIdx.x, gridDim.x);
}

// Cast with a transposed copy, over kTR x 64 tiles of x, one tile per wave (grid-stride,
// so the grid and the number of amax partials stay bounded), walked in tile-row pairs
// (pair_tile) so that a block's four waves fill whole 128-byte lines of both outputs.
// Per tile:
//  - the wave loads the tile as 8-row x 128-byte pieces (kTR / 8 16-byte loads in flight
//    per lane), quantizes, stores `out` (if requested) and stages the bytes in its own LDS
//    region;
//  - per 64-row half, each lane reads back 4 columns x 16 rows (wave_transpose64_staged)
//    and stores them as four 16-byte row segments of out_t.
// rows and cols need not be multiples of the tile; cols % 16 == 0.
constexpr int kTR = 64;   // tile rows
constexpr int kTT = 64;   // tile columns
constexpr int kWavesPerBlock = kNT / 64;
// 1024 blocks (4 per CU): with a delayed scale every block first folds the previous
// step's partials into the history, so fewer, longer blocks pay for it less often
// (dY [8192, 2560] e5m2 with its transposed copy: 22.9 -> 19.5 us; the c5 training step
// 2090 -> 2068 us; interleaved A/B against 2048)
constexpr int kMaxTransposeBlocks = 1024;

// Block blk of the nblk blocks that cast x with its transposed copy; blk == 0 leads
// (publishes the meta record, pushes a delayed amax). The first tile's loads are issued
// before the scale is resolved, so a delayed or current scale's partials reduction runs
// while they are in flight.
template <int FMT>
__device__ __forceinline__ void cast_transpose_body(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, const ScaleSrc& src,
    uint8_t* __restrict__ out, uint8_t* __restrict__ out_t, uint32_t* __restrict__ amax_out,
    int64_t blk, int64_t nblk) {
  constexpr int NL = kTR / 8;  // 16-byte loads per lane
  __shared__ uint32_t stage[kWavesPerBlock][(kTR / 64) * kWaveTileDwords];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t tiles_c = (cols + kTT - 1) / kTT;
  const int64_t tile_rows = (rows + kTR - 1) / kTR;
  const int64_t ntiles = tiles_c * tile_rows;
  const bool t16 = (rows & 15) == 0;  // out_t rows 16-byte aligned
  const int ch = lane & 7;
  // load k of tile tile_id: rows 8k + (lane >> 3), 16-byte chunk lane & 7 (8 rows x 128
  // bytes each)
  auto load_tile = [&](int64_t tile_id, uint4 (&v)[NL], int64_t& r0, int64_t& c0) {
    int64_t ti, tj;
    pair_tile(tile_id, tiles_c, tile_rows, ti, tj);
    r0 = ti * kTR;
    c0 = tj * kTT;
    const int64_t c = c0 + 8 * ch;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int64_t r = r0 + 8 * k + (lane >> 3);
      v[k] = make_uint4(0u, 0u, 0u, 0u);
      if (tile_id < ntiles && r < rows && c < cols)
        v[k] = *reinterpret_cast<const uint4*>(x + r * cols + c);
    }
  };
  int64_t tile_id = blk * kWavesPerBlock + wid;
  uint4 v[NL];
  int64_t r0, c0;
  load_tile(tile_id, v, r0, c0);
  const float scale = resolve_scale<FMT>(src, blk == 0);
  uint32_t m = 0;
  for (; tile_id < ntiles; tile_id += nblk * kWavesPerBlock) {
    if (tile_id != blk * kWavesPerBlock + wid) load_tile(tile_id, v, r0, c0);
    const int64_t c = c0 + 8 * ch;
    uint32_t* lds = stage[wid];
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int lr = 8 * k + (lane >> 3);
      const int64_t r = r0 + lr;
      if (amax_out) m = max(m, absmax_key8(v[k]));
      const uint2 qq = quant8_bf16<FMT>(v[k], scale);
      if (out && r < rows && c < cols) *reinterpret_cast<uint2*>(out + r * cols + c) = qq;
      lds[lr * kWaveTilePitch + 2 * ch] = qq.x;
      lds[lr * kWaveTilePitch + 2 * ch + 1] = qq.y;
    }
#pragma unroll
    for (int h = 0; h < kTR / 64; ++h) {
      uint4 tq[4];
      wave_transpose64_staged(lds + h * kWaveTileDwords, lane, tq);
      const int64_t tc = r0 + 64 * h + (lane >> 4) * 16;  // out_t column (a row of x)
      if (tc < rows) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const int64_t tr = c0 + 4 * (lane & 15) + cc;  // out_t row (a column of x)
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
  store_block_amax(m, amax_out, blk);
}

template <int FMT>
__global__ __launch_bounds__(kNT) void cast_transpose_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, ScaleSrc src,
    uint8_t* __restrict__ out, uint8_t* __restrict__ out_t, uint32_t* __restrict__ amax_out) {
  cast_transpose_body<FMT>(x, rows, cols, src, out, out_t, amax_out, blockIdx.x, gridDim.x);
}

int64_t transpose_blocks(int64_t rows, int64_t cols) {
  const int64_t tiles = ((rows + kTR - 1) / kTR) * ((cols + kTT - 1) / kTT);
  const int64_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  return blocks < kMaxTransposeBlocks ? (blocks > 0 ? blocks : 1) : kMaxTransposeBlocks;
}

// Blocks of the row-major cast: up to kMaxCastBlocks; 512 when it writes amax partials
// (a delayed-scaling cast, whose next step's blocks each fold them into the history, so
// fewer partials and fewer folding blocks: c5 step 1915 -> 1877 us for 1024 against 2048,
// and for 512 dY's e5m2 cast [8192, 2560] 15.6 -> 14.6 us, the step 1852 -> 1849 us).
constexpr int64_t kMaxPartialCastBlocks = 512;
static_assert(kMaxPartialCastBlocks <= kMaxInlinePartials, "consumers reduce them inline");
int64_t row_cast_blocks(int64_t n, bool with_amax) {
  return grid_for_stream((n + 15) / 16, 2 * kNT, with_amax ? kMaxPartialCastBlocks : kMaxCastBlocks);
}

// ---- delayed scaling ------------------------------------------------------------------
// state layout: history[len], then meta {amax_last, scale, scale_inv, pos}; a fresh
// state is zero except scale = scale_inv = 1. The new scale is fp8_max / max(history)
// when that maximum is finite and positive, else the previous scale is kept (TE's
// default scaling-factor update with margin 0).
__global__ void delayed_begin_kernel(float* state, int len, float fp8_max) {
  if (threadIdx.x != 0) return;
  float h = 0.0f;
  bool finite = true;
  for (int i = 0; i < len; ++i) {
    float v = state[i];
    finite &= (v == v) && (fabsf(v) != INFINITY);
    h = fmaxf(h, v);
  }
  float* meta = state + len;
  if (finite && h > 0.0f) {
    const float scale = (float)((double)fp8_max / (double)h);
    meta[1] = scale;
    meta[2] = (float)(1.0 / (double)scale);
  }
}

// Only the scale step of a delayed cast (for a producer that quantizes its own output with
// the scale, as the gated-GELU GEMM does for H): push the previous step's amax, derive
// this step's scale and publish it at state + len and meta_out.
__global__ __launch_bounds__(kNT) void delayed_fold_kernel(float* state, int len, int pos,
                                                           const uint32_t* __restrict__ prev,
                                                           int64_t n_prev, float fp8_max,
                                                           float* meta_out) {
  delayed_scale_block<kNT>(state, len, pos, prev, n_prev, fp8_max, meta_out, true);
}

__global__ __launch_bounds__(kNT) void delayed_end_kernel(float* state, int len,
                                                          const uint32_t* __restrict__ partials,
                                                          int64_t np) {
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < np; i += kNT) m = max(m, partials[i]);
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) {
    float* meta = state + len;
    int pos = (int)meta[3];
    if (pos < 0 || pos >= len) pos = 0;
    const float amax = __uint_as_float(m);
    state[pos] = amax;
    meta[0] = amax;
    meta[3] = (float)((pos + 1) % len);
  }
}

// Delayed scaling with a long list of previous partials: pushes their max into slot pos
// (and meta {amax, ., ., next slot}), so the cast itself then has none to fold.
__global__ __launch_bounds__(kNT) void fold_amax_kernel(float* state, int len, int pos,
                                                        const uint32_t* __restrict__ prev,
                                                        int64_t n_prev) {
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < n_prev; i += kNT) m = max(m, prev[i]);
  m = block_max_u32<kNT>(m);
  if (threadIdx.x == 0) {
    const float amax = __uint_as_float(m);
    state[pos] = amax;
    state[len] = amax;
    state[len + 3] = (float)((pos + 1) % len);
  }
}

int launch_cast(const void* x, int64_t rows, int64_t cols, ScaleSrc src, int fmt,
                uint8_t* out, uint8_t* out_t, uint32_t* amax_out, void* stream, const char* who) {
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "%s: bad fmt %d", who, fmt);
  BF8_CHECK(!src.pow2 || (src.partials && !src.state), "%s: BF8_SCALE_POW2 needs current scaling",
            who);
  BF8_CHECK(rows >= 0 && cols >= 0, "%s: negative shape", who);
  BF8_CHECK(out || out_t, "%s: out and out_t are both NULL", who);
  BF8_CHECK(((uintptr_t)x & 15) == 0 && (!out || ((uintptr_t)out & 15) == 0),
            "%s: x and out must be 16-byte aligned", who);
  const int64_t n = rows * cols;
  if (n == 0) return BF8_OK;
  BF8_CHECK(x != nullptr, "%s: x is NULL", who);
  hipStream_t s = as_stream(stream);
  const uint16_t* xs = (const uint16_t*)x;
  if (!src.scale && !src.state && src.np > kMaxInlinePartials) {
    // current scaling from many partials: meta first, then a cast with its scale
    float* meta = src.meta_out;
    hipLaunchKernelGGL(scale_from_partials_kernel, dim3(1), dim3(kScaleNT), 0, s, src.partials,
                       src.np, fp8_max_host(fmt), src.pow2, meta);
    const int rc = launch_status("scale_from_partials_kernel");
    if (rc != BF8_OK) return rc;
    src = ScaleSrc{};
    src.scale = meta + 1;
  }
  if (src.state && src.n_prev > kMaxInlinePartials) {
    // delayed scaling after a producer with many partials: fold them in first
    hipLaunchKernelGGL(fold_amax_kernel, dim3(1), dim3(kNT), 0, s, src.state, src.len, src.pos,
                       src.prev, src.n_prev);
    const int rc = launch_status("fold_amax_kernel");
    if (rc != BF8_OK) return rc;
    src.prev = nullptr;
    src.n_prev = 0;
  }
  if (out_t == nullptr) {
    const int grid = (int)row_cast_blocks(n, amax_out != nullptr);
    if (fmt == BF8_E4M3)
      hipLaunchKernelGGL(cast_kernel<BF8_E4M3>, dim3(grid), dim3(kNT), 0, s, xs, n, src, out,
                         amax_out);
    else
      hipLaunchKernelGGL(cast_kernel<BF8_E5M2>, dim3(grid), dim3(kNT), 0, s, xs, n, src, out,
                         amax_out);
    return launch_status("cast_kernel");
  }
  BF8_CHECK(cols % 16 == 0, "%s: transposed cast needs cols %% 16 == 0 (got %lld)", who,
            (long long)cols);
  BF8_CHECK(((uintptr_t)out_t & 15) == 0, "%s: out_t must be 16-byte aligned", who);
  const dim3 grid((unsigned)transpose_blocks(rows, cols));
  if (fmt == BF8_E4M3)
    hipLaunchKernelGGL(cast_transpose_kernel<BF8_E4M3>, grid, dim3(kNT), 0, s, xs, rows, cols,
                       src, out, out_t, amax_out);
  else
    hipLaunchKernelGGL(cast_transpose_kernel<BF8_E5M2>, grid, dim3(kNT), 0, s, xs, rows, cols,
                       src, out, out_t, amax_out);
  return launch_status("cast_transpose_kernel");
}

ScaleSrc given_scale(const float* scale) {
  ScaleSrc s{};
  s.scale = scale;
  return s;
}

ScaleSrc current_scale(const uint32_t* partials, int64_t np, float* meta) {
  ScaleSrc s{};
  s.partials = partials;
  s.np = np;
  s.meta_out = meta;
  return s;
}

// ---- several tensors in two launches ------------------------------------------------
// Current-scaling quantization of up to kMaxMany bf16 tensors: one launch computes every
// tensor's amax partials, one launch casts them all. Each tensor keeps the block count,
// grid-stride order, partials and scale it has in amax_partials_kernel + cast_kernel, so
// its bytes and meta are those of its own quantization; sharing the launches fills the
// chip when a tensor alone would not, and saves two launches per extra tensor.
constexpr int kMaxMany = 8;
static_assert(kMaxAmaxBlocks <= kMaxInlinePartials, "the cast reduces a tensor's partials inline");

struct ManySeg {
  const uint16_t* x;
  int64_t n;
  uint8_t* out;
  float* meta;
  int64_t part_off;    // this tensor's partials: [part_off, part_off + amax_blocks)
  int64_t amax_first;  // first block of this tensor in the amax launch
  int64_t amax_blocks;
  int64_t cast_first;  // first block of this tensor in the cast launch
  int64_t cast_blocks;
  int fmt, pow2;
};

struct ManyArgs {
  ManySeg seg[kMaxMany];
  int count;
  uint32_t* partials;
};

// The tensor whose blocks include block b (segments in launch order).
__device__ __forceinline__ int many_segment(const ManyArgs& a, int64_t b, bool cast) {
  int t = 0;
  for (int k = 1; k < a.count; ++k)
    if (b >= (cast ? a.seg[k].cast_first : a.seg[k].amax_first)) t = k;
  return t;
}

__global__ __launch_bounds__(kNT) void amax_many_kernel(ManyArgs a) {
  const int t = many_segment(a, blockIdx.x, false);
  const ManySeg& g = a.seg[t];
  amax_partials_body(g.x, g.n, a.partials + g.part_off, (int64_t)blockIdx.x - g.amax_first,
                     g.amax_blocks);
}

__global__ __launch_bounds__(kNT) void cast_many_kernel(ManyArgs a) {
  const int t = many_segment(a, blockIdx.x, true);
  const ManySeg& g = a.seg[t];
  ScaleSrc src{};
  src.partials = a.partials + g.part_off;
  src.np = g.amax_blocks;
  src.meta_out = g.meta;
  src.pow2 = g.pow2;
  const int64_t blk = (int64_t)blockIdx.x - g.cast_first;
  if (g.fmt == BF8_E4M3)
    cast_body<BF8_E4M3>(g.x, g.n, src, g.out, nullptr, blk, g.cast_blocks);
  else
    cast_body<BF8_E5M2>(g.x, g.n, src, g.out, nullptr, blk, g.cast_blocks);
}

// ---- several delayed casts in one launch ----------------------------------------------
// Up to kMaxMany delayed-scaling casts (each with its own history, formats, optional
// transposed copy and amax partials) in one launch: tensor t runs on blocks [first,
// first + blocks) with the grid, block order and partials its own bf8_cast_delayed_bf16
// launch would have, so its bytes, meta, history and partials are those of that call.
struct DelayedSeg {
  const uint16_t* x;
  int64_t rows, cols;
  ScaleSrc src;
  int fmt;
  uint8_t* out;
  uint8_t* out_t;
  uint32_t* amax_out;
  int64_t first, blocks;
};

struct DelayedManyArgs {
  DelayedSeg seg[kMaxMany];
  int count;
};

__global__ __launch_bounds__(kNT) void cast_delayed_many_kernel(DelayedManyArgs a) {
  int t = 0;
  for (int k = 1; k < a.count; ++k)
    if ((int64_t)blockIdx.x >= a.seg[k].first) t = k;
  const DelayedSeg& g = a.seg[t];
  const int64_t blk = (int64_t)blockIdx.x - g.first;
  if (g.out_t) {
    if (g.fmt == BF8_E4M3)
      cast_transpose_body<BF8_E4M3>(g.x, g.rows, g.cols, g.src, g.out, g.out_t, g.amax_out, blk,
                                    g.blocks);
    else
      cast_transpose_body<BF8_E5M2>(g.x, g.rows, g.cols, g.src, g.out, g.out_t, g.amax_out, blk,
                                    g.blocks);
  } else {
    if (g.fmt == BF8_E4M3)
      cast_body<BF8_E4M3>(g.x, g.rows * g.cols, g.src, g.out, g.amax_out, blk, g.blocks);
    else
      cast_body<BF8_E5M2>(g.x, g.rows * g.cols, g.src, g.out, g.amax_out, blk, g.blocks);
  }
}

}  // namespace
}  // namespace bf8

// ---- library-owned scratch of bf8_quantize_bf16_noalloc ------------------------------
// The amax partials of the allocation-free quantization live in a file-scope device array
// (each GPU the library runs on holds its own copy, 4 KB, until the process ends). Host code
// must not pass `scratch` itself to a kernel (in host code the name is a stand-in, not a
// device address): the device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept in `g_scratch_ptr`.
static __device__ __align__(256) uint32_t scratch[bf8::kNoAllocSlots];

namespace bf8 {
namespace {

constexpr int kMaxDevices = 64;
uint32_t* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The device address of this GPU's `scratch` (the GPU of `stream`; the current one for the
// NULL stream), looked up on the first call for that GPU. No memory is allocated.
int noalloc_scratch(hipStream_t stream, uint32_t** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("bf8_quantize_bf16_noalloc: no device for the stream (%s)", hipGetErrorString(e));
    return BF8_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess || p == nullptr) {
      set_error("bf8_quantize_bf16_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
      return BF8_ELAUNCH;
    }
    g_scratch_ptr[dev] = static_cast<uint32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return BF8_OK;
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

const char* bf8_last_error(void) { return bf8::g_err; }
int bf8_abi_version(void) { return 18; }

int64_t bf8_amax_partials(int64_t n) { return amax_blocks(n); }

int bf8_amax_bf16(const void* x, int64_t n, uint32_t* partials, void* stream) {
  BF8_CHECK(n >= 0, "bf8_amax_bf16: n < 0");
  BF8_CHECK(partials != nullptr, "bf8_amax_bf16: partials is NULL");
  BF8_CHECK(n == 0 || x != nullptr, "bf8_amax_bf16: x is NULL");
  BF8_CHECK(((uintptr_t)x & 15) == 0, "bf8_amax_bf16: x must be 16-byte aligned");
  const int64_t nb = amax_blocks(n);
  hipLaunchKernelGGL(amax_partials_kernel, dim3((unsigned)nb), dim3(kNT), 0, as_stream(stream),
                     (const uint16_t*)x, n, partials);
  return launch_status("amax_partials_kernel");
}

int bf8_scale_from_partials(const uint32_t* partials, int64_t n_partials, int fmt, float* meta,
                            void* stream) {
  const int pow2 = (fmt & BF8_SCALE_POW2) ? 1 : 0;
  fmt &= ~BF8_SCALE_POW2;
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_scale_from_partials: bad fmt %d", fmt);
  BF8_CHECK(partials && meta, "bf8_scale_from_partials: NULL pointer");
  BF8_CHECK(n_partials >= 1, "bf8_scale_from_partials: n_partials < 1");
  hipLaunchKernelGGL(scale_from_partials_kernel, dim3(1), dim3(kScaleNT), 0, as_stream(stream),
                     partials, n_partials, fp8_max_host(fmt), pow2, meta);
  return launch_status("scale_from_partials_kernel");
}

int bf8_cast_bf16(const void* x, int64_t rows, int64_t cols, const float* scale, int fmt,
                  uint8_t* out, uint8_t* out_t, void* stream) {
  BF8_CHECK(scale != nullptr, "bf8_cast_bf16: scale is NULL");
  return launch_cast(x, rows, cols, given_scale(scale), fmt, out, out_t, nullptr, stream,
                     "bf8_cast_bf16");
}

int bf8_cast_partials_bf16(const void* x, int64_t rows, int64_t cols, const uint32_t* partials,
                           int64_t n_partials, int fmt, float* meta, uint8_t* out,
                           uint8_t* out_t, void* stream) {
  BF8_CHECK(partials && meta && n_partials >= 1, "bf8_cast_partials_bf16: bad partials or meta");
  ScaleSrc src = current_scale(partials, n_partials, meta);
  src.pow2 = (fmt & BF8_SCALE_POW2) ? 1 : 0;
  return launch_cast(x, rows, cols, src, fmt & ~BF8_SCALE_POW2, out, out_t, nullptr, stream,
                     "bf8_cast_partials_bf16");
}

int64_t bf8_cast_amax_partials(int64_t rows, int64_t cols, int transpose) {
  if (rows <= 0 || cols <= 0) return 1;
  return transpose ? transpose_blocks(rows, cols) : row_cast_blocks(rows * cols, true);
}

int bf8_cast_delayed_bf16(const void* x, int64_t rows, int64_t cols, float* state, int len,
                          int pos, const uint32_t* prev_partials, int64_t n_prev, int fmt,
                          float* meta_out, uint8_t* out, uint8_t* out_t, uint32_t* partials_out,
                          void* stream) {
  BF8_CHECK(state && len >= 1 && len <= 1024, "bf8_cast_delayed_bf16: bad state/len");
  BF8_CHECK(pos >= 0 && pos < len, "bf8_cast_delayed_bf16: pos %d outside [0, %d)", pos, len);
  BF8_CHECK(n_prev >= 0 && (n_prev == 0 || prev_partials),
            "bf8_cast_delayed_bf16: bad previous partials");
  ScaleSrc src{};
  src.state = state;
  src.len = len;
  src.pos = pos;
  src.prev = prev_partials;
  src.n_prev = n_prev;
  src.meta_out = meta_out;
  return launch_cast(x, rows, cols, src, fmt, out, out_t, partials_out, stream,
                     "bf8_cast_delayed_bf16");
}

int bf8_quantize_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                      uint8_t* out_t, float* meta, uint32_t* partials, void* stream) {
  BF8_CHECK(rows >= 0 && cols >= 0, "bf8_quantize_bf16: negative shape");
  BF8_CHECK((fmt & ~BF8_SCALE_POW2) == BF8_E4M3 || (fmt & ~BF8_SCALE_POW2) == BF8_E5M2,
            "bf8_quantize_bf16: bad fmt %d", fmt);
  // everything the cast checks, checked before the amax pass is enqueued
  BF8_CHECK(meta && (out || out_t), "bf8_quantize_bf16: meta is NULL or no output given");
  BF8_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)out_t & 15) == 0,
            "bf8_quantize_bf16: x, out and out_t must be 16-byte aligned");
  BF8_CHECK(!out_t || cols % 16 == 0,
            "bf8_quantize_bf16: transposed cast needs cols %% 16 == 0 (got %lld)", (long long)cols);
  const int64_t n = rows * cols;
  int rc = bf8_amax_bf16(x, n, partials, stream);
  if (rc) return rc;
  return bf8_cast_partials_bf16(x, rows, cols, partials, amax_blocks(n), fmt, meta, out, out_t,
                                stream);
}

int bf8_quantize_bf16_noalloc(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                              uint8_t* out_t, float* meta, void* stream) {
  BF8_CHECK(rows >= 0 && cols >= 0, "bf8_quantize_bf16_noalloc: negative shape");
  const int64_t need = amax_blocks(rows * cols);
  BF8_CHECK(need <= kNoAllocSlots,
            "bf8_quantize_bf16_noalloc: needs %lld amax slots, the library scratch holds %lld",
            (long long)need, (long long)kNoAllocSlots);
  uint32_t* partials = nullptr;
  const int rc = noalloc_scratch(as_stream(stream), &partials);
  if (rc != BF8_OK) return rc;
  // the amax pass writes every slot [0, need) that the cast then reads: nothing to clear
  return bf8_quantize_bf16(x, rows, cols, fmt, out, out_t, meta, partials, stream);
}

int64_t bf8_quantize_many_partials(int count, const int64_t* n) {
  if (count < 1 || count > kMaxMany || !n) return 0;
  int64_t total = 0;
  for (int t = 0; t < count; ++t) total += n[t] > 0 ? amax_blocks(n[t]) : 0;
  return total;
}

int bf8_quantize_many_bf16(int count, const void* const* x, const int64_t* n, const int* fmt,
                           uint8_t* const* out, float* const* meta, uint32_t* partials,
                           void* stream) {
  BF8_CHECK(count >= 1 && count <= kMaxMany, "bf8_quantize_many_bf16: count %d outside [1, %d]",
            count, kMaxMany);
  BF8_CHECK(x && n && fmt && out && meta, "bf8_quantize_many_bf16: NULL array");
  ManyArgs a{};
  a.partials = partials;
  int64_t amax_total = 0, cast_total = 0;
  for (int t = 0; t < count; ++t) {
    const int f = fmt[t] & ~BF8_SCALE_POW2;
    BF8_CHECK(f == BF8_E4M3 || f == BF8_E5M2, "bf8_quantize_many_bf16: tensor %d: bad fmt %d", t,
              fmt[t]);
    BF8_CHECK(n[t] >= 0, "bf8_quantize_many_bf16: tensor %d: n < 0", t);
    BF8_CHECK(meta[t] != nullptr, "bf8_quantize_many_bf16: tensor %d: meta is NULL", t);
    if (n[t] == 0) continue;  // as bf8_quantize_bf16: nothing cast, meta untouched
    BF8_CHECK(x[t] && out[t], "bf8_quantize_many_bf16: tensor %d: x or out is NULL", t);
    BF8_CHECK(((uintptr_t)x[t] & 15) == 0 && ((uintptr_t)out[t] & 15) == 0,
              "bf8_quantize_many_bf16: tensor %d: x and out must be 16-byte aligned", t);
    ManySeg& g = a.seg[a.count++];
    g.x = (const uint16_t*)x[t];
    g.n = n[t];
    g.out = out[t];
    g.meta = meta[t];
    g.fmt = f;
    g.pow2 = (fmt[t] & BF8_SCALE_POW2) ? 1 : 0;
    g.part_off = amax_total;
    g.amax_first = amax_total;
    g.amax_blocks = amax_blocks(n[t]);
    g.cast_first = cast_total;
    g.cast_blocks = row_cast_blocks(n[t], false);
    amax_total += g.amax_blocks;
    cast_total += g.cast_blocks;
  }
  if (a.count == 0) return BF8_OK;
  BF8_CHECK(partials != nullptr, "bf8_quantize_many_bf16: partials is NULL");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(amax_many_kernel, dim3((unsigned)amax_total), dim3(kNT), 0, s, a);
  const int rc = launch_status("amax_many_kernel");
  if (rc != BF8_OK) return rc;
  hipLaunchKernelGGL(cast_many_kernel, dim3((unsigned)cast_total), dim3(kNT), 0, s, a);
  return launch_status("cast_many_kernel");
}

int bf8_cast_delayed_many_bf16(int count, const void* const* x, const int64_t* rows,
                               const int64_t* cols, float* const* state, const int* len,
                               const int* pos, const uint32_t* const* prev_partials,
                               const int64_t* n_prev, const int* fmt, float* const* meta_out,
                               uint8_t* const* out, uint8_t* const* out_t,
                               uint32_t* const* partials_out, void* stream) {
  BF8_CHECK(count >= 1 && count <= kMaxMany,
            "bf8_cast_delayed_many_bf16: count %d outside [1, %d]", count, kMaxMany);
  BF8_CHECK(x && rows && cols && state && len && pos && prev_partials && n_prev && fmt &&
                meta_out && out && out_t && partials_out,
            "bf8_cast_delayed_many_bf16: NULL array");
  DelayedManyArgs a{};
  int64_t total = 0;
  for (int t = 0; t < count; ++t) {
    BF8_CHECK(fmt[t] == BF8_E4M3 || fmt[t] == BF8_E5M2,
              "bf8_cast_delayed_many_bf16: tensor %d: bad fmt %d", t, fmt[t]);
    BF8_CHECK(rows[t] >= 0 && cols[t] >= 0, "bf8_cast_delayed_many_bf16: tensor %d: negative shape",
              t);
    BF8_CHECK(state[t] && len[t] >= 1 && len[t] <= 1024,
              "bf8_cast_delayed_many_bf16: tensor %d: bad state/len", t);
    BF8_CHECK(pos[t] >= 0 && pos[t] < len[t],
              "bf8_cast_delayed_many_bf16: tensor %d: pos %d outside [0, %d)", t, pos[t], len[t]);
    BF8_CHECK(n_prev[t] >= 0 && n_prev[t] <= kMaxInlinePartials &&
                  (n_prev[t] == 0 || prev_partials[t]),
              "bf8_cast_delayed_many_bf16: tensor %d: bad previous partials (%lld, at most %lld)",
              t, (long long)n_prev[t], (long long)kMaxInlinePartials);
    BF8_CHECK(out[t] || out_t[t], "bf8_cast_delayed_many_bf16: tensor %d: out and out_t are NULL",
              t);
    BF8_CHECK(((uintptr_t)x[t] & 15) == 0 && ((uintptr_t)out[t] & 15) == 0 &&
                  ((uintptr_t)out_t[t] & 15) == 0,
              "bf8_cast_delayed_many_bf16: tensor %d: x, out and out_t must be 16-byte aligned", t);
    BF8_CHECK(!out_t[t] || cols[t] % 16 == 0,
              "bf8_cast_delayed_many_bf16: tensor %d: transposed cast needs cols %% 16 == 0", t);
    const int64_t n = rows[t] * cols[t];
    if (n == 0) continue;  // as bf8_cast_delayed_bf16: nothing cast, state untouched
    BF8_CHECK(x[t] != nullptr, "bf8_cast_delayed_many_bf16: tensor %d: x is NULL", t);
    DelayedSeg& g = a.seg[a.count++];
    g.x = (const uint16_t*)x[t];
    g.rows = rows[t];
    g.cols = cols[t];
    g.src = ScaleSrc{};
    g.src.state = state[t];
    g.src.len = len[t];
    g.src.pos = pos[t];
    g.src.prev = prev_partials[t];
    g.src.n_prev = n_prev[t];
    g.src.meta_out = meta_out[t];
    g.fmt = fmt[t];
    g.out = out[t];
    g.out_t = out_t[t];
    g.amax_out = partials_out[t];
    g.first = total;
    g.blocks = out_t[t] ? transpose_blocks(rows[t], cols[t])
                        : row_cast_blocks(n, partials_out[t] != nullptr);
    total += g.blocks;
  }
  if (a.count == 0) return BF8_OK;
  hipLaunchKernelGGL(cast_delayed_many_kernel, dim3((unsigned)total), dim3(kNT), 0,
                     as_stream(stream), a);
  return launch_status("cast_delayed_many_kernel");
}

int bf8_delayed_scale_begin(float* state, int len, int fmt, void* stream) {
  BF8_CHECK(state && len >= 1 && len <= 1024, "bf8_delayed_scale_begin: bad state/len");
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_delayed_scale_begin: bad fmt %d", fmt);
  hipLaunchKernelGGL(delayed_begin_kernel, dim3(1), dim3(64), 0, as_stream(stream), state, len,
                     fp8_max_host(fmt));
  return launch_status("delayed_begin_kernel");
}

int bf8_delayed_scale_fold(float* state, int len, int pos, const uint32_t* prev_partials,
                           int64_t n_prev, int fmt, float* meta_out, void* stream) {
  BF8_CHECK(state && len >= 1 && len <= 1024, "bf8_delayed_scale_fold: bad state/len");
  BF8_CHECK(pos >= 0 && pos < len, "bf8_delayed_scale_fold: pos %d outside [0, %d)", pos, len);
  BF8_CHECK(fmt == BF8_E4M3 || fmt == BF8_E5M2, "bf8_delayed_scale_fold: bad fmt %d", fmt);
  BF8_CHECK(n_prev >= 0 && (n_prev == 0 || prev_partials),
            "bf8_delayed_scale_fold: bad previous partials");
  hipLaunchKernelGGL(delayed_fold_kernel, dim3(1), dim3(kNT), 0, as_stream(stream), state, len,
                     pos, prev_partials, n_prev, fp8_max_host(fmt), meta_out);
  return launch_status("delayed_fold_kernel");
}

int bf8_delayed_scale_end(float* state, int len, const uint32_t* partials, int64_t n_partials,
                          void* stream) {
  BF8_CHECK(state && len >= 1 && len <= 1024, "bf8_delayed_scale_end: bad state/len");
  BF8_CHECK(partials && n_partials >= 1, "bf8_delayed_scale_end: bad partials");
  hipLaunchKernelGGL(delayed_end_kernel, dim3(1), dim3(kNT), 0, as_stream(stream), state, len,
                     partials, n_partials);
  return launch_status("delayed_end_kernel");
}

}  // extern "C"
