// Shared device helpers and the C-ABI error plumbing of libbongard_fp8.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/bongard_fp8.h"

namespace bf8 {

// ---- error reporting --------------------------------------------------------------
void set_error(const char* fmt, ...);

#define BF8_CHECK(cond, ...)            \
  do {                                  \
    if (!(cond)) {                      \
      ::bf8::set_error(__VA_ARGS__);    \
      return BF8_EINVAL;                \
    }                                   \
  } while (0)

// Checks the launch that was just enqueued.
int launch_status(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- format constants -------------------------------------------------------------
// OCP e4m3 (fn): max finite 448. OCP e5m2: max finite 57344.
template <int FMT>
struct Fp8Max;
template <>
struct Fp8Max<BF8_E4M3> {
  static constexpr float value = 448.0f;
};
template <>
struct Fp8Max<BF8_E5M2> {
  static constexpr float value = 57344.0f;
};

inline float fp8_max_host(int fmt) { return fmt == BF8_E4M3 ? 448.0f : 57344.0f; }

// ---- vector memory helpers (device) ----------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte loads/stores with the non-temporal hint (streamed data that is not re-read).
__device__ __forceinline__ uint4 load_nt(const void* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(void* p, uint4 v) {
  u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// ---- bit helpers (device) ---------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16 bits, round to nearest even; any NaN becomes 0x7FC0 (as torch's
// c10::BFloat16 conversion does).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_round(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 with round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32); equal
// to f32_to_bf16_bits on each value except that a NaN keeps its sign and payload bits.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// A packed bf16 pair with each NaN replaced by 0x7FC0 (torch's canonical bf16 NaN), so
// that pack_bf16x2 then gives f32_to_bf16_bits bit for bit. A half h is NaN iff
// (h & 0x7FFF) + 0x7F carries into bit 15; the low half's sum cannot reach bit 16.
__device__ __forceinline__ uint32_t canon_nan_bf16x2(uint32_t w) {
  const uint32_t nan = ((w & 0x7FFF7FFFu) + 0x007F007Fu) & 0x80008000u;
  if (__builtin_expect(nan != 0, 0)) {
    if (nan & 0x8000u) w = (w & 0xFFFF0000u) | 0x7FC0u;
    if (nan & 0x80000000u) w = (w & 0x0000FFFFu) | 0x7FC00000u;
  }
  return w;
}

// Byte for an fp32 product p = f32(x) * scale that is NaN. It follows torch's CPU
// result for clamp(x.float() * scale).to(float8): the NaN carries the scale's sign if
// the scale is NaN, else x's sign if x is NaN, else (inf * 0) the x86 default NaN, which
// is negative. Both formats encode NaN as 0x7F | sign.
__device__ __forceinline__ uint32_t nan_byte(float x, float scale) {
  uint32_t s;
  if (scale != scale)
    s = __float_as_uint(scale) >> 31;
  else if (x != x)
    s = __float_as_uint(x) >> 31;
  else
    s = 1u;
  return 0x7Fu | (s << 7);
}

// Saturating RNE conversion of four fp32 values (already multiplied by the scale) to
// four fp8 bytes packed little-endian. xs are the unscaled inputs (for NaN signs).
template <int FMT>
__device__ __forceinline__ uint32_t quant4(float p0, float p1, float p2, float p3, float x0,
                                           float x1, float x2, float x3, float scale) {
  constexpr float M = Fp8Max<FMT>::value;
  float c0 = __builtin_amdgcn_fmed3f(p0, -M, M);
  float c1 = __builtin_amdgcn_fmed3f(p1, -M, M);
  float c2 = __builtin_amdgcn_fmed3f(p2, -M, M);
  float c3 = __builtin_amdgcn_fmed3f(p3, -M, M);
  uint32_t w;
  if constexpr (FMT == BF8_E4M3) {
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c2, c3, w, true);
  } else {
    w = __builtin_amdgcn_cvt_pk_bf8_f32(c0, c1, 0, false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(c2, c3, w, true);
  }
  // NaN products are rare: patch them bytewise.
  if (__builtin_expect((p0 != p0) | (p1 != p1) | (p2 != p2) | (p3 != p3), 0)) {
    if (p0 != p0) w = (w & 0xFFFFFF00u) | nan_byte(x0, scale);
    if (p1 != p1) w = (w & 0xFFFF00FFu) | (nan_byte(x1, scale) << 8);
    if (p2 != p2) w = (w & 0xFF00FFFFu) | (nan_byte(x2, scale) << 16);
    if (p3 != p3) w = (w & 0x00FFFFFFu) | (nan_byte(x3, scale) << 24);
  }
  return w;
}

// Quantize 8 bf16 values (two packed per uint32) to 8 fp8 bytes (two uint32).
template <int FMT>
__device__ __forceinline__ uint2 quant8_bf16(uint4 v, float scale) {
  float x0 = bf16_lo(v.x), x1 = bf16_hi(v.x), x2 = bf16_lo(v.y), x3 = bf16_hi(v.y);
  float x4 = bf16_lo(v.z), x5 = bf16_hi(v.z), x6 = bf16_lo(v.w), x7 = bf16_hi(v.w);
  uint2 r;
  r.x = quant4<FMT>(x0 * scale, x1 * scale, x2 * scale, x3 * scale, x0, x1, x2, x3, scale);
  r.y = quant4<FMT>(x4 * scale, x5 * scale, x6 * scale, x7 * scale, x4, x5, x6, x7, scale);
  return r;
}

// quant4 / quant8_bf16 for inputs known to be finite with a finite scale (no product can
// be NaN): the same bytes without the NaN patch. CLAMP = false further drops the clamp,
// for callers whose products are known to lie within +-fp8_max (MX blocks of finite
// values).
template <int FMT, bool CLAMP>
__device__ __forceinline__ uint32_t quant4_finite(float p0, float p1, float p2, float p3) {
  constexpr float M = Fp8Max<FMT>::value;
  if constexpr (CLAMP) {
    p0 = __builtin_amdgcn_fmed3f(p0, -M, M);
    p1 = __builtin_amdgcn_fmed3f(p1, -M, M);
    p2 = __builtin_amdgcn_fmed3f(p2, -M, M);
    p3 = __builtin_amdgcn_fmed3f(p3, -M, M);
  }
  uint32_t w;
  if constexpr (FMT == BF8_E4M3) {
    w = __builtin_amdgcn_cvt_pk_fp8_f32(p0, p1, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(p2, p3, w, true);
  } else {
    w = __builtin_amdgcn_cvt_pk_bf8_f32(p0, p1, 0, false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(p2, p3, w, true);
  }
  return w;
}
template <int FMT, bool CLAMP>
__device__ __forceinline__ uint2 quant8_bf16_finite(uint4 v, float scale) {
  return make_uint2(quant4_finite<FMT, CLAMP>(bf16_lo(v.x) * scale, bf16_hi(v.x) * scale,
                                              bf16_lo(v.y) * scale, bf16_hi(v.y) * scale),
                    quant4_finite<FMT, CLAMP>(bf16_lo(v.z) * scale, bf16_hi(v.z) * scale,
                                              bf16_lo(v.w) * scale, bf16_hi(v.w) * scale));
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Per-half unsigned max of two packed 16-bit pairs (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  const u16x2 r = __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                            __builtin_bit_cast(u16x2, b));
  return __builtin_bit_cast(uint32_t, r);
}

// Max of |bf16| over the 8 values of v, as an fp32 bit pattern key: for non-negative
// floats the unsigned order of the bits is the numeric order, and NaN keys sort above
// +inf (as torch's NaN-propagating max does).
__device__ __forceinline__ uint32_t absmax_key8(uint4 v) {
  uint32_t a = v.x & 0x7FFF7FFFu, b = v.y & 0x7FFF7FFFu;
  uint32_t c = v.z & 0x7FFF7FFFu, d = v.w & 0x7FFF7FFFu;
  uint32_t m0 = max(max(a & 0xFFFFu, a >> 16), max(b & 0xFFFFu, b >> 16));
  uint32_t m1 = max(max(c & 0xFFFFu, c >> 16), max(d & 0xFFFFu, d >> 16));
  return max(m0, m1) << 16;
}

// ---- MXFP8 block scales (TE MXFP8BlockScaling, 32-element blocks, E8M0 bytes) -------
constexpr uint32_t kMxPadScale = 127u;  // E8M0 1.0, the padding past a row's last block

// E8M0 exponent of amax / fp8_max rounded up to a power of two (TE float_to_e8m0 on
// fp32(amax * fp32(1 / fp8_max))). key: fp32 bits of amax (>= 0 or NaN).
template <int FMT>
__device__ __forceinline__ uint32_t mx_exponent(uint32_t key) {
  constexpr float kRcp = (float)(1.0 / (double)Fp8Max<FMT>::value);
  const float amax = __uint_as_float(key);
  if (amax != amax) return 0xFFu;
  const float val = amax * kRcp;
  const uint32_t b = __float_as_uint(val);
  if (b >= 0x7F800000u) return 0xFEu;  // inf: saturate
  uint32_t e = b >> 23;
  const uint32_t man = b & 0x7FFFFFu;
  if (man != 0 && e != 0xFEu && !(e == 0 && man <= 0x400000u)) ++e;
  return e;
}

// 2^(127 - e), the factor applied to the block's values (NaN for e = 0xFF).
__device__ __forceinline__ float mx_multiplier(uint32_t e) {
  if (e == 0xFFu) return __uint_as_float(0x7FC00000u);
  if (e == 254u) return __uint_as_float(0x00400000u);  // 2^-127, subnormal
  return __uint_as_float((254u - e) << 23);
}

// ---- wave-level 64 x 64 byte transpose ------------------------------------------------
constexpr int kWaveTilePitch = 17;  // dwords per staged row (odd: conflict-free row writes)
constexpr int kWaveTileDwords = 64 * kWaveTilePitch;

// Transpose of a 64 x 64 byte tile that one wave has staged in its own LDS region (row r
// at lds + r * kWaveTilePitch dwords, kWaveTileDwords in all): lane l gets columns
// 4 (l & 15) + c, c < 4, over rows 16 (l >> 4) .. +15 as t[c] (byte i of t[c] = row
// 16 (l >> 4) + i). No barrier is needed between the wave's staging stores and these
// reads: a wave's LDS accesses complete in order.
__device__ __forceinline__ void wave_transpose64_staged(const uint32_t* lds, int lane,
                                                        uint4 (&t)[4]) {
  const int row0 = (lane >> 4) * 16, cg = lane & 15;
  uint32_t d[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = lds[(row0 + i) * kWaveTilePitch + cg];
  uint32_t c[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // 4 x 4 byte transpose of rows 4k .. 4k+3
    const uint32_t t0 = __byte_perm(d[4 * k], d[4 * k + 1], 0x5140);
    const uint32_t t1 = __byte_perm(d[4 * k], d[4 * k + 1], 0x7362);
    const uint32_t t2 = __byte_perm(d[4 * k + 2], d[4 * k + 3], 0x5140);
    const uint32_t t3 = __byte_perm(d[4 * k + 2], d[4 * k + 3], 0x7362);
    c[0][k] = __byte_perm(t0, t2, 0x5410);
    c[1][k] = __byte_perm(t0, t2, 0x7632);
    c[2][k] = __byte_perm(t1, t3, 0x5410);
    c[3][k] = __byte_perm(t1, t3, 0x7632);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) t[k] = make_uint4(c[k][0], c[k][1], c[k][2], c[k][3]);
}

// Tile t of a grid of tile rows x tiles_c tile columns, in tile-row-pair order: tiles 2j
// and 2j + 1 are one tile column of the tile rows 2i and 2i + 1 (a last, odd tile row
// alone), so the four waves of a block (four consecutive t, tiles_c even) cover a 2 x 2
// square of 64 x 64 tiles. Each 128-byte line of a transposed output (128 rows of one
// column) and of an fp8 row output (128 columns of one row) is then written by one block,
// at one time, through one L2, instead of as halves from tiles far apart in the walk.
__device__ __forceinline__ void pair_tile(int64_t t, int64_t tiles_c, int64_t tile_rows,
                                          int64_t& tr, int64_t& tcol) {
  const int64_t rp = t / (2 * tiles_c), rem = t - rp * 2 * tiles_c;
  if (2 * rp + 1 < tile_rows) {
    tr = 2 * rp + (rem & 1);
    tcol = rem >> 1;
  } else {
    tr = 2 * rp;
    tcol = rem;
  }
}

// Wavefront (64-lane) max reduction.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

// Block max reduction for blockDim.x == NT (multiple of 64). Result valid in all threads.
template <int NT>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v) {
  __shared__ uint32_t red[NT / 64];
  v = wave_max_u32(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) r = max(r, red[i]);
  __syncthreads();
  return r;
}

// ---- scale from an amax key --------------------------------------------------------
// scale = fp32(fp8_max / max(f64(amax), 1e-12)) (f64 division, correctly rounded, then one
// rounding to fp32: equal to the correctly rounded fp32 quotient since 53 >= 2 * 24 + 2);
// a NaN amax gives its quietened NaN. pow2 rounds the scale down to a power of two by
// clearing its mantissa (torchao round_scales_to_power_of_2; 0 and inf stay as they are).
// scale_inv = fp32(1 / scale), correctly rounded (exact for a power of two).
__device__ inline void scale_from_amax_key(uint32_t key, float fp8_max, bool pow2, float& scale,
                                           float& scale_inv) {
  const float amax = __uint_as_float(key);
  if (amax != amax) {
    scale = __uint_as_float(key | 0x00400000u);
    scale_inv = scale;
    return;
  }
  double a = (double)amax;
  if (a < 1e-12) a = 1e-12;
  scale = (float)((double)fp8_max / a);
  if (pow2) scale = __uint_as_float(__float_as_uint(scale) & 0xFF800000u);
  scale_inv = (float)(1.0 / (double)scale);
}

// ---- per-tensor scale from block partials, finished by the last block ---------------
// meta = {amax, scale, scale_inv, 0} (scale_from_amax_key).
__device__ inline void write_meta_from_amax(uint32_t key, float fp8_max, float* meta,
                                            bool pow2 = false) {
  float scale, scale_inv;
  scale_from_amax_key(key, fp8_max, pow2, scale, scale_inv);
  meta[0] = __uint_as_float(key);
  meta[1] = scale;
  meta[2] = scale_inv;
  meta[3] = 0.0f;
}

// Scale of a tensor from the per-block amax partials its producer wrote, computed by
// every block of the consumer (each reads the <= 2048 partials once); the leader block
// (the consumer's first block of this tensor) also publishes the meta record. Result
// valid in all threads.
template <int NT>
__device__ inline float scale_from_partials_block(const uint32_t* __restrict__ partials,
                                                  int64_t np, float fp8_max,
                                                  float* __restrict__ meta_out,
                                                  bool pow2, bool leader) {
  __shared__ float s_scale;
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < np; i += NT) m = max(m, partials[i]);
  m = block_max_u32<NT>(m);
  if (threadIdx.x == 0) {
    float meta[4];
    write_meta_from_amax(m, fp8_max, meta, pow2);
    s_scale = meta[1];
    if (meta_out && leader) {
      meta_out[0] = meta[0];
      meta_out[1] = meta[1];
      meta_out[2] = meta[2];
      meta_out[3] = meta[3];
    }
  }
  __syncthreads();
  return s_scale;
}

// Delayed scaling (TE DelayedScaling, margin 0, amax_compute_algo "max") folded into a
// consumer kernel; the block reads the partials and the history window in parallel (one
// thread walking the window's len entries serially cost every folding block len dependent
// loads: dY's delayed e5m2 cast at c5 16.2 -> 15.0 us). state = history[len], then meta {amax, scale, scale_inv, next slot}.
// Every block reduces the previous step's amax partials (n_prev of them; none on the
// first step) and forms w = max(history[i != pos], that amax), the window after the
// amax is pushed into slot pos. scale = fp32(fp8_max / f64(w)) when the window is finite
// and w > 0, else the stored scale is kept. The leader block (by default block (0,0))
// pushes the amax and publishes the meta. All blocks compute the same values, so reading
// the words the leader rewrites is harmless: slot pos is excluded, and the stored scale is
// only used when it is written back unchanged. The leader also writes {w, scale,
// scale_inv, 0} to meta_out (if any), a copy of this step's scale that later steps do not
// overwrite. Result valid in all threads.
// Order-preserving key of a float for an unsigned max (negative values below positive
// ones, -0 below +0); NaN maps to 0, below every number, so that a max over keys skips NaNs
// as fmaxf does. key_value inverts it (key 0: no number was seen).
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  if (v != v) return 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  if (k == 0u) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int NT>
__device__ inline float delayed_scale_block(float* __restrict__ state, int len, int pos,
                                            const uint32_t* __restrict__ prev, int64_t n_prev,
                                            float fp8_max, float* __restrict__ meta_out,
                                            bool leader) {
  __shared__ float s_scale;
  __shared__ uint32_t red[3][NT / 64];
  const bool have_new = n_prev > 0;
  // the previous step's partials and the history window (slot pos excluded when a new
  // amax replaces it) are read by all threads at once: the window's max as an order key,
  // its finiteness as a flag
  uint32_t m = 0, hk = 0, bad = 0;
  for (int64_t i = threadIdx.x; i < n_prev; i += NT) m = max(m, prev[i]);
  for (int i = threadIdx.x; i < len; i += NT) {
    if (have_new && i == pos) continue;
    const float v = state[i];
    bad |= (v != v) || (fabsf(v) == INFINITY) ? 1u : 0u;
    hk = max(hk, order_key(v));
  }
  m = wave_max_u32(m);
  hk = wave_max_u32(hk);
  bad = wave_max_u32(bad);
  const int wlane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (wlane == 0) {
    red[0][wv] = m;
    red[1][wv] = hk;
    red[2][wv] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
      m = max(m, red[0][i]);
      hk = max(hk, red[1][i]);
      bad = max(bad, red[2][i]);
    }
    const float amax_new = __uint_as_float(m);
    // w = the window's maximum taken as fmaxf would, from the new amax (or 0 on the
    // first step) and the history entries
    const float w = key_value(max(hk, order_key(have_new ? amax_new : 0.0f)));
    const bool finite = (!have_new || (m < 0x7F800000u)) && bad == 0u;
    float* meta = state + len;
    float scale = meta[1];
    if (finite && w > 0.0f) scale = (float)((double)fp8_max / (double)w);
    s_scale = scale;
    if (leader) {
      if (have_new) {
        state[pos] = amax_new;
        meta[0] = amax_new;
      }
      const float scale_inv = (float)(1.0 / (double)scale);
      meta[1] = scale;
      meta[2] = scale_inv;
      if (have_new) meta[3] = (float)((pos + 1) % len);
      if (meta_out) {
        meta_out[0] = w;
        meta_out[1] = scale;
        meta_out[2] = scale_inv;
        meta_out[3] = 0.0f;
      }
    }
  }
  __syncthreads();
  return s_scale;
}

}  // namespace bf8
