// Host entry points of the FP8 GEMM (bf8_gemm, bf8_gemm_geglu): argument checks, the
// choice of block tile and K split for a shape, split-K workspace sizing and the split-K
// reduction. The GEMM kernels live in gemm_kernel_impl.hpp, instantiated per tile shape
// in gemm_tile_*.hip.
//
// Semantics replace torch._scaled_mm / cuBLASLt under torchao Float8Linear
// (bongard/float8_training.py:22) and TE's FP8 GEMM under te.Linear
// (bongard/te_linear.py:73-74): C = (A8 . B8^T accumulated in fp32) * sa_inv * sb_inv
// (+ bias), both operands K-contiguous.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "gemm_kernel.hpp"

namespace bf8 {
namespace {

constexpr int kNumCus = 256;  // MI355X: 8 XCDs x 32 CUs
constexpr int kStepBytes = 128;
constexpr int kMaxSplits = 8;
constexpr int kMinStepsPerSplit = 4;

enum TileId {
  TILE_256x256 = 0,
  TILE_256x160,
  TILE_160x256,
  TILE_128x128,
  TILE_192x256,
  TILE_128x64,
  TILE_64x128,
  TILE_256x128,
  TILE_128x64k2,
  TILE_64x128k2,
  TILE_128x128k2,
  TILE_256x256w8,
  TILE_256x256w8x,
  NUM_TILES
};

struct TileInfo {
  int bm, bn, occ;
  double rate;        // modelled dense FP8 rate of one CU running this tile, TFLOP/s
  double geglu_rate;  // the same with the gated-GELU epilogue; 0: no such variant (the
                      // gated GELU pairs gate and up sub-tiles, so FN must be even)
  const char* name;
  bool mx;            // has an MX (block-scaled) variant (tiles whose stages would overflow
                      // the LDS with the scale dwords run it with one stage fewer)
};

// Rates are per-CU throughputs measured on MI355X (time per K step of one workgroup, with
// every CU busy, over the tile's FLOP per step).
constexpr TileInfo kTiles[NUM_TILES] = {
    {256, 256, 1, 9.6, 8.8, "256x256", true},
    {256, 160, 1, 9.2, 8.0, "256x160", true},
    {160, 256, 1, 9.0, 7.6, "160x256", true},
    {128, 128, 1, 8.0, 6.2, "128x128", true},
    {192, 256, 1, 9.0, 8.0, "192x256", true},
    {128, 64, 2, 6.5, 0.0, "128x64", true},
    {64, 128, 2, 6.5, 4.0, "64x128", true},
    {256, 128, 1, 0.1, 0.1, "256x128", true},
    {128, 64, 1, 0.1, 0.0, "128x64k2", false},
    {64, 128, 1, 0.1, 0.0, "64x128k2", false},
    {128, 128, 1, 0.1, 0.0, "128x128k2", false},
    {256, 256, 1, 10.0, 9.2, "256x256w8", false},
    {256, 256, 1, 10.0, 0.0, "256x256w8x", false},
};
// Whether `tile` has a gated-GELU variant for I = N / 2: tiles of 128 or 64 H columns take
// any I (a multiple of 128); the 256x160 tile (80 gate + 80 up columns, one wave column)
// needs I % 80 == 0 (its H stores are not column-masked) and has no MX variant (its MX H
// blocks of 32 columns would straddle tiles).
bool geglu_tile_ok(int tile, int64_t N, bool mx) {
  if (kTiles[tile].geglu_rate <= 0) return false;
  const int hcols = kTiles[tile].bn / 2;
  if (hcols % 64 == 0) return true;
  return !mx && (N / 2) % hcols == 0;
}

// Gated-GELU plans may not depend on K (the amax partial count is sized from M and I
// alone); they are costed at a typical 20 K steps (hidden size 2560).
constexpr int kGegluNominalSteps = 20;

struct Plan {
  int tile = TILE_256x256;
  int splits = 1;
  int kps = 0;  // K steps per split (tail split: per piece)
  int tiles_m = 0, tiles_n = 0;
  int full_tiles = 0, tail_pieces = 0;  // tail split: whole tiles, K pieces per tail tile
  size_t ws_bytes = 0;  // split-K workspace: fp32 partials [splits][M][N], or the tail
                        // tiles' pieces [tails * pieces][BM][BN]
};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

Plan make_plan(int tile, int64_t M, int64_t N, int64_t ksteps, int splits) {
  // M, N: the output's shape (split-K partials are M x N fp32 per split)
  const TileInfo& ti = kTiles[tile];
  Plan p;
  p.tile = tile;
  p.tiles_m = (int)cdiv(M, ti.bm);
  p.tiles_n = (int)cdiv(N, ti.bn);
  p.kps = (int)cdiv(ksteps, splits);
  p.splits = (int)cdiv(ksteps, p.kps);  // no empty split
  if (p.splits > 1) p.ws_bytes = (size_t)p.splits * M * N * 4;
  return p;
}

// Tail split: with T tiles filling R rounds and a partial last round of t = T mod 256
// tiles (t <= 128), the whole rounds run whole tiles and each of the t tail tiles is split
// into pieces = min(256 / t, 8) K ranges, one workgroup each, so the last round has every
// CU busy for a fraction of a tile instead of t CUs for a whole one. Valid for tiles that
// run one workgroup per CU with one K group. Returns false when it does not apply.
// Per-CU FP8 rate of a long run of K steps (no epilogue) for the tiles that take tail
// splits: the 256x256 tile, ~1.5 us per 128-byte step on MI355X with every CU busy (8192^3
// and c5's dX shape). Measured gain at c5 (interleaved A/B): dX (M=8192, N=2560,
// K=20480) 343.5 -> 341.0 us, dW_gu (M=20480, N=2560, K=8192) 338.8 -> 332.6 us against
// two rounds of 256x160 tiles; a shape with a smaller tail gains more.
constexpr double kTailStepRate256 = 11.2;
// the eight-wave 256x256 tile on the same long-K shapes (8192^3: 394.8 -> 385.4 us)
constexpr double kTailStepRate256w8 = 11.5;

// Linear GEMMs with at least this many K steps run the eight-wave tile with its third B
// slot (Tile256x256w8x): in a training step their operands come from HBM, not the MALL,
// and B loaded two steps ahead hides that (operands rotated through more than the MALL
// holds, interleaved A/B, bit-identical: c5's dW_down 197.7 -> 179.5 us, dX (K = 20480)
// 355.8 -> 337.5 us, 8192^3 423.1 -> 403.5 us); with K = 2560 (20 steps) the extra slot
// costs 1.5-2%, warm or cold.
constexpr int64_t kExtraBSlotMinSteps = 48;

bool make_tail_plan(int tile, int64_t M, int64_t N, int64_t ksteps, Plan& p) {
  const TileInfo& ti = kTiles[tile];
  if (tile != TILE_256x256 && tile != TILE_256x256w8 && tile != TILE_256x256w8x) return false;
  p = Plan{};
  p.tile = tile;
  p.tiles_m = (int)cdiv(M, ti.bm);
  p.tiles_n = (int)cdiv(N, ti.bn);
  const int64_t T = (int64_t)p.tiles_m * p.tiles_n;
  const int64_t tails = T % kNumCus;
  if (T <= kNumCus || tails == 0 || tails > kNumCus / 2) return false;
  int pieces = (int)std::min<int64_t>(kNumCus / tails, kMaxSplits);
  p.kps = (int)cdiv(ksteps, pieces);
  pieces = (int)cdiv(ksteps, p.kps);  // no empty piece
  if (pieces < 2 || p.kps < kMinStepsPerSplit) return false;
  p.full_tiles = (int)(T - tails);
  p.tail_pieces = pieces;
  p.ws_bytes = (size_t)tails * pieces * ti.bm * ti.bn * 4;
  return true;
}

// A K step never takes less than this, however little MFMA work it holds: with few
// workgroups per CU the loads of the stages in flight no longer cover their latency
// (measured at M = 512: ~520 ns per step for one workgroup per CU, ~450 ns when the tile
// is small enough for two to share the CU).
constexpr double kStepFloorNs = 520.0;
constexpr double kStepFloorNsOcc2 = 450.0;

// Modelled time (ns): rounds of co-resident workgroups, each running its K steps plus
// about two steps of pipeline fill and epilogue, plus the split-K partials' HBM round
// trip and the reduction's launch. A step costs the MFMA work of the workgroups sharing
// a CU in the busiest round, or the latency floor.
double plan_cost(const Plan& p, int64_t M, int64_t N, bool geglu, int64_t ksteps = 0) {
  const TileInfo& ti = kTiles[p.tile];
  if (p.tail_pieces > 0) {
    // whole rounds of whole tiles, one round of pieces, the pieces' partials written and
    // read back, the reduction's launch
    const double rate =
        p.tile == TILE_256x256 ? kTailStepRate256 : kTailStepRate256w8;  // w8 and w8x alike
    const double step_ns = 2.0 * ti.bm * ti.bn * kStepBytes / (rate * 1e3);
    const double rounds = (double)p.full_tiles / kNumCus;
    return rounds * (ksteps + 2) * step_ns + (p.kps + 2) * step_ns + 2.0 * p.ws_bytes / 5e3 + 5000.0;
  }
  const int64_t ctas = (int64_t)p.tiles_m * p.tiles_n * p.splits;
  const int64_t rounds = cdiv(ctas, (int64_t)kNumCus * ti.occ);
  const int64_t per_cu = std::min<int64_t>(ti.occ, cdiv(ctas, (int64_t)kNumCus));
  const double rate = geglu ? ti.geglu_rate : ti.rate;
  const double work_ns = per_cu * 2.0 * ti.bm * ti.bn * kStepBytes / (rate * 1e3);
  const double step_ns = std::max(work_ns, ti.occ > 1 ? kStepFloorNsOcc2 : kStepFloorNs);
  // A last round that only part of the CUs run, after whole rounds, steps faster than a
  // whole one (the busy CUs share the memory system and the power budget with fewer
  // others): costed as 0.35 + 0.65 f of a round for a fraction f of the workgroup slots.
  // Measured on c5's dW_down (M = 2560, N = 10240, K = 8192): one round and 56% of a
  // second of eight-wave 256x256 tiles 164 us, two rounds and 50% of a third of 256x160
  // tiles 188 us. A lone partial round (small M) is latency-bound and keeps its full cost.
  const int64_t slots = (int64_t)kNumCus * ti.occ;
  const int64_t whole = ctas / slots;
  const double frac = (double)(ctas - whole * slots) / slots;
  const double eff_rounds =
      whole >= 1 && frac > 0 ? whole + 0.35 + 0.65 * frac : (double)rounds;
  double t = eff_rounds * (p.kps + 2) * step_ns;
  if (p.splits > 1) t += 2.0 * p.splits * M * N * 4 / 5e3 + 5000.0;
  return t;
}

// Tuning override, read on every call: BONGARD_FP8_GEMM_TILE=<bm>x<bn>[:<splits>|:t]
// (e.g. "256x160:4"; ":t" the tail split, when the shape has one). Unknown values are
// ignored.
constexpr int kTailSplitOverride = -1;
bool env_override(int& tile, int& splits) {
  tile = -1;
  splits = 1;
  const char* e = std::getenv("BONGARD_FP8_GEMM_TILE");
  if (!e || !*e) return false;
  for (int i = 0; i < NUM_TILES; ++i) {
    const size_t n = std::strlen(kTiles[i].name);
    if (std::strncmp(e, kTiles[i].name, n) == 0 && (e[n] == 0 || e[n] == ':')) {
      tile = i;
      if (e[n] == ':') splits = e[n + 1] == 't' ? kTailSplitOverride : std::atoi(e + n + 1);
    }
  }
  if (splits != kTailSplitOverride) splits = splits < 1 ? 1 : (splits > kMaxSplits ? kMaxSplits : splits);
  return tile >= 0;
}

// Chooses the tile and K split for C[M, N] = A[M, K] . B[N, K]^T. GEGLU plans never split
// and depend on (M, N) only, so the per-tile amax partial count is known without K.
Plan choose_plan(int64_t M, int64_t N, int64_t K, bool geglu, size_t ws_avail, bool mx = false,
                 bool kmajor = false) {
  const int64_t ksteps = std::max<int64_t>(cdiv(K, kStepBytes), 1);
  int otile, osplits;
  if (env_override(otile, osplits) && (!geglu || geglu_tile_ok(otile, N, mx)) &&
      (!mx || kTiles[otile].mx) &&
      (!kmajor || otile == TILE_256x256w8 || otile == TILE_256x256w8x)) {
    Plan p;
    if (!geglu && osplits == kTailSplitOverride) {
      if (make_tail_plan(otile, M, N, ksteps, p) && p.ws_bytes <= ws_avail) return p;
      osplits = 1;
    }
    p = make_plan(otile, M, N, ksteps, geglu ? 1 : osplits);
    if (p.ws_bytes > ws_avail) p = make_plan(otile, M, N, ksteps, 1);
    return p;
  }
  Plan best;
  double best_cost = 0;
  bool have = false;
  for (int tile = 0; tile < NUM_TILES; ++tile) {
    if ((geglu && !geglu_tile_ok(tile, N, mx)) || (mx && !kTiles[tile].mx)) continue;
    // K-major operands: the eight-wave 256x256 tiles only
    if (kmajor && tile != TILE_256x256w8) continue;
    // the eight-wave 256x256 tile replaces the four-wave one wherever it has a variant
    // (measured faster on every large shape, same bits); MX keeps the four-wave tile
    if (!mx && tile == TILE_256x256) continue;
    // the extra-B-slot twin of the eight-wave tile is substituted below, by K
    if (tile == TILE_256x256w8x) continue;
    for (int s = 1; s <= (geglu ? 1 : kMaxSplits); ++s) {
      const Plan p = make_plan(tile, M, N, geglu ? kGegluNominalSteps : ksteps, s);
      if (p.splits != s || (s > 1 && p.kps < kMinStepsPerSplit) || p.ws_bytes > ws_avail)
        continue;
      const double c = plan_cost(p, M, N, geglu);
      if (!have || c < best_cost * 0.97) {  // prefer earlier (larger, unsplit) plans on ties
        best = p;
        best_cost = c;
        have = true;
      }
    }
    Plan tp;
    if (!geglu && make_tail_plan(tile, M, N, ksteps, tp) && tp.ws_bytes <= ws_avail) {
      const double c = plan_cost(tp, M, N, false, ksteps);
      if (!have || c < best_cost * 0.97) {
        best = tp;
        best_cost = c;
        have = true;
      }
    }
  }
  if (geglu) best.kps = (int)ksteps;
  if (!geglu && !mx && best.tile == TILE_256x256w8 && ksteps >= kExtraBSlotMinSteps)
    best.tile = TILE_256x256w8x;  // same geometry, so the plan (tiles, pieces) stands
  // A small tile that leaves one workgroup per CU (no K split) runs as its two-K-group
  // twin: two pipelines per CU take alternate K steps (measured ~10% faster at M = 512,
  // e.g. N = 4096, K = 2560: 10.5 vs 11.5 us; with more tiles than CUs the one-group tile
  // already shares each CU between two workgroups).
  if (!geglu && !mx && best.splits == 1 &&
      (int64_t)best.tiles_m * best.tiles_n <= kNumCus &&
      (best.tile == TILE_128x64 || best.tile == TILE_64x128)) {
    best.tile = best.tile == TILE_128x64 ? TILE_128x64k2 : TILE_64x128k2;
  }
  if (const char* d = std::getenv("BONGARD_FP8_GEMM_DEBUG"); d && d[0] == '1')
    std::fprintf(stderr, "bf8 plan %s%s M=%lld N=%lld K=%lld: tile %s splits %d (%d x %d tiles, tail pieces %d)\n",
                 geglu ? "geglu" : "gemm", mx ? " mx" : "", (long long)M, (long long)N, (long long)K,
                 kTiles[best.tile].name, best.splits, best.tiles_m, best.tiles_n, best.tail_pieces);
  return best;
}

// ---- K-major operands on small shapes ------------------------------------------------
// The K-major GEMM runs on the eight-wave 256x256 tiles only, which leave most CUs idle when
// the output is small (M = 512, N = 2560, K = 2048: 20 tiles; measured 30 us against 12 us
// for the row-major plan on a transposed copy of B). For a call with only B K-major whose
// plan the cost model prices well above the row-major plan plus a byte transpose of B, the
// entry point transposes B^T [K, N] into its workspace and runs the row-major plan. (The
// wgrad form, A and B K-major, measured level or faster on the same shapes, so it always
// runs K-major.)
constexpr double kTransposeBytesPerNs = 2.5e3;  // a small transpose: ~2.5 TB/s read + write
constexpr double kTransposeLaunchNs = 4000.0;
constexpr double kKmajorFallbackGain = 0.8;  // transpose only when that is 20% cheaper

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct KmajorChoice {
  Plan plan;
  bool transpose_b = false;
  size_t b_bytes = 0;  // the transposed B's share of the workspace (the plan's own follows)
};

KmajorChoice choose_kmajor(int64_t M, int64_t N, int64_t K, bool a_kmajor, size_t ws_avail) {
  KmajorChoice c;
  c.plan = choose_plan(M, N, K, false, ws_avail, false, true);
  int otile, osplits;
  if (a_kmajor || env_override(otile, osplits)) return c;  // a forced plan stays as asked
  const size_t bb = align256((size_t)N * K);
  if (ws_avail < bb) return c;
  const int64_t ksteps = std::max<int64_t>(cdiv(K, kStepBytes), 1);
  const Plan pr = choose_plan(M, N, K, false, ws_avail - bb);
  // costed as the planner costed them: the two-K-group and extra-B-slot tiles replace
  // their plain twins after the choice, on the twins' costs
  auto costed = [&](Plan q) {
    if (q.tile == TILE_128x64k2) q.tile = TILE_128x64;
    if (q.tile == TILE_64x128k2) q.tile = TILE_64x128;
    if (q.tile == TILE_256x256w8x) q.tile = TILE_256x256w8;
    return plan_cost(q, M, N, false, ksteps);
  };
  const double ck = costed(c.plan);
  const double cr = costed(pr) + 2.0 * (double)N * K / kTransposeBytesPerNs + kTransposeLaunchNs;
  if (const char* d = std::getenv("BONGARD_FP8_GEMM_DEBUG"); d && d[0] == '1')
    std::fprintf(stderr, "bf8 kmajor M=%lld N=%lld K=%lld: K-major %.0f ns, transposed B %.0f ns\n",
                 (long long)M, (long long)N, (long long)K, ck, cr);
  if (cr < kKmajorFallbackGain * ck) {
    c.plan = pr;
    c.transpose_b = true;
    c.b_bytes = bb;
  }
  return c;
}

// B^T [rows = K, cols = N] (row stride ld) -> B [N, K] (row stride K): one 64 x 64 byte tile
// per wave, staged in the wave's own LDS region and read back transposed; rows and cols are
// multiples of 16 (whole 16-byte segments). No block barrier, so a wave past the last tile
// may leave at once.
constexpr int kTransposeWaves = 4;
__global__ __launch_bounds__(kTransposeWaves * 64) void transpose_u8_kernel(
    const uint8_t* __restrict__ src, int64_t rows, int64_t cols, int64_t ld,
    uint8_t* __restrict__ dst) {
  __shared__ uint32_t stage[kTransposeWaves][kWaveTileDwords];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t tiles_c = (cols + 63) / 64;
  const int64_t t = (int64_t)blockIdx.x * kTransposeWaves + wid;
  if (t >= tiles_c * ((rows + 63) / 64)) return;
  const int64_t r0 = (t / tiles_c) * 64, c0 = (t % tiles_c) * 64;
  uint32_t* lds = stage[wid];
  const int ch = lane & 3;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = 16 * k + (lane >> 2);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r0 + row < rows && c0 + 16 * ch < cols)
      v = *reinterpret_cast<const uint4*>(src + (r0 + row) * ld + c0 + 16 * ch);
    lds[row * kWaveTilePitch + 4 * ch] = v.x;
    lds[row * kWaveTilePitch + 4 * ch + 1] = v.y;
    lds[row * kWaveTilePitch + 4 * ch + 2] = v.z;
    lds[row * kWaveTilePitch + 4 * ch + 3] = v.w;
  }
  uint4 tq[4];
  wave_transpose64_staged(lds, lane, tq);
  const int64_t orow = c0 + 4 * (lane & 15), ocol = r0 + 16 * (lane >> 4);
  if (ocol < rows) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (orow + c < cols) *reinterpret_cast<uint4*>(dst + (orow + c) * rows + ocol) = tq[c];
  }
}

int launch_tile(const Plan& pl, const GemmParams& p, int epi, int out_dtype, int fa, int fb,
                hipStream_t s, bool mx) {
  switch (pl.tile) {
    case TILE_256x256: return launch_gemm_tile<Tile256x256>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_256x160: return launch_gemm_tile<Tile256x160>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_160x256: return launch_gemm_tile<Tile160x256>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_192x256: return launch_gemm_tile<Tile192x256>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_128x64: return launch_gemm_tile<Tile128x64>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_64x128: return launch_gemm_tile<Tile64x128>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_256x128: return launch_gemm_tile<Tile256x128>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_128x64k2: return launch_gemm_tile<Tile128x64k2>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_64x128k2: return launch_gemm_tile<Tile64x128k2>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_128x128k2: return launch_gemm_tile<Tile128x128k2>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_256x256w8: return launch_gemm_tile<Tile256x256w8>(p, epi, out_dtype, fa, fb, s, mx);
    case TILE_256x256w8x: return launch_gemm_tile<Tile256x256w8x>(p, epi, out_dtype, fa, fb, s, mx);
    default: return launch_gemm_tile<Tile128x128>(p, epi, out_dtype, fa, fb, s, mx);
  }
}

struct SegEnds {
  int e[4];
};

// The epilogue of a reduced partial sum: v (8 fp32 sums for columns n .. n+7 of row m) times
// alpha(n) = a_scale_inv * b_scale_inv[segment of n] (or the axiswise factors, or 1 for MX),
// plus bias, written to C as bf16 (RNE) or fp32.
struct ReduceOut {
  const float* a_sinv;
  const float* b_sinv;
  int b_stride, n_seg;
  SegEnds seg_end;
  const uint16_t* bias;
  void* C;
  int64_t ldc;
  int a_vec, b_vec, unit;
};

template <int OUT>
__device__ __forceinline__ void reduce_store(const ReduceOut& o, float (&v)[8], int m, int n) {
  const float sa = (o.a_vec || o.unit) ? 0.0f : *o.a_sinv;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // segments change at multiples of 4 columns
    const int nh = n + 4 * h;
    int seg = 0;
#pragma unroll
    for (int s2 = 0; s2 < 3; ++s2) seg += (s2 + 1 < o.n_seg && nh >= o.seg_end.e[s2]) ? 1 : 0;
    float b4[4] = {0.f, 0.f, 0.f, 0.f};
    if (o.bias) {
      const uint2 bb = *reinterpret_cast<const uint2*>(o.bias + nh);
      b4[0] = bf16_lo(bb.x); b4[1] = bf16_hi(bb.x); b4[2] = bf16_lo(bb.y); b4[3] = bf16_hi(bb.y);
    }
    if (o.unit) {  // MX: the block scales were applied inside the MFMA
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * h + e] = v[4 * h + e] + b4[e];
      continue;
    }
    if (o.a_vec | o.b_vec) {  // axiswise: (a_sinv[m] or a_sinv[0]) * (b_sinv[n] or b_sinv[0])
      const float ra = o.a_vec ? o.a_sinv[m] : *o.a_sinv;
      float cf[4];
      if (o.b_vec) {
        const float4 f = *reinterpret_cast<const float4*>(o.b_sinv + nh);
        cf[0] = f.x; cf[1] = f.y; cf[2] = f.z; cf[3] = f.w;
      } else {
        cf[0] = cf[1] = cf[2] = cf[3] = *o.b_sinv;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * h + e] = v[4 * h + e] * (ra * cf[e]) + b4[e];
      continue;
    }
    const float alpha = sa * o.b_sinv[seg * o.b_stride];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * h + e] = v[4 * h + e] * alpha + b4[e];
  }
  if (OUT == BF8_OUT_BF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(o.C) + m * o.ldc + n;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                 (float __attribute__((ext_vector_type(2)))){v[2 * e], v[2 * e + 1]},
                 __bf16 __attribute__((ext_vector_type(2)))));
    if ((o.ldc & 7) == 0) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      reinterpret_cast<uint2*>(dst)[0] = make_uint2(w[0], w[1]);
      reinterpret_cast<uint2*>(dst)[1] = make_uint2(w[2], w[3]);
    }
  } else {
    float* dst = reinterpret_cast<float*>(o.C) + m * o.ldc + n;
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// v = P[0] + P[1] + ... + P[count-1] (8 fp32 at src + s * stride), summed in index order.
// count <= kMaxSplits. Every load is issued before the first add, so the partials come in
// one memory latency instead of one per piece.
__device__ __forceinline__ void sum_pieces(const float* src, int64_t stride, int count,
                                           float (&v)[8]) {
  float4 lo[kMaxSplits], hi[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) {
    if (s < count) {
      lo[s] = *reinterpret_cast<const float4*>(src + s * stride);
      hi[s] = *reinterpret_cast<const float4*>(src + s * stride + 4);
    }
  }
  v[0] = lo[0].x; v[1] = lo[0].y; v[2] = lo[0].z; v[3] = lo[0].w;
  v[4] = hi[0].x; v[5] = hi[0].y; v[6] = hi[0].z; v[7] = hi[0].w;
#pragma unroll
  for (int s = 1; s < kMaxSplits; ++s) {
    if (s < count) {
      v[0] += lo[s].x; v[1] += lo[s].y; v[2] += lo[s].z; v[3] += lo[s].w;
      v[4] += hi[s].x; v[5] += hi[s].y; v[6] += hi[s].z; v[7] += hi[s].w;
    }
  }
}

// C = alpha(n) * sum_s P[s] + bias(n) for the split-K partials P [splits][M][N] (fp32),
// summed in split order, so the result does not depend on which split finished first.
// Each thread does 8 columns.
template <int OUT>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ P, int splits,
                                                           int64_t stride, int M, int N,
                                                           ReduceOut o) {
  const int n8 = N >> 3;
  const int64_t total = (int64_t)M * n8;
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * 256) {
    const int m = (int)(g / n8), n = (int)(g % n8) * 8;
    const float* src = P + (int64_t)m * N + n;
    float v[8];
    sum_pieces(src, stride, splits, v);
    reduce_store<OUT>(o, v, m, n);
  }
}

// The tail tiles of a tail-split schedule: tile t (walk position full_tiles + t) is the sum
// of its pieces P[t * pieces + s] ([BM][BN] fp32 each), taken in piece order. A block covers
// 2048 outputs of one tile, 8 columns a thread.
template <int OUT>
__global__ __launch_bounds__(256) void tail_reduce_kernel(const float* __restrict__ P, int pieces,
                                                          int bm, int bn, int full_tiles,
                                                          int tiles_m, int tiles_n, int M, int N,
                                                          ReduceOut o) {
  const int per_tile = bm * bn / 2048;
  const int t = blockIdx.x / per_tile;
  const int e = (blockIdx.x % per_tile) * 256 + threadIdx.x;
  const int row = e / (bn / 8), col = (e % (bn / 8)) * 8;
  int tm, tn;
  walk_tile(tiles_m, tiles_n, full_tiles + t, tm, tn);
  const int m = tm * bm + row, n = tn * bn + col;
  if (m >= M || n >= N) return;  // N % 8 == 0: eight columns are all in or all out
  const float* src = P + (int64_t)t * pieces * bm * bn + row * bn + col;
  float v[8];
  sum_pieces(src, (int64_t)bm * bn, pieces, v);
  reduce_store<OUT>(o, v, m, n);
}

int launch_plan(const Plan& pl, GemmParams p, int epi, int out_dtype, int fa, int fb, void* ws,
                hipStream_t s, bool mx = false) {
  p.tiles_m = pl.tiles_m;
  p.tiles_n = pl.tiles_n;
  p.splits = pl.splits;
  p.ksteps_per_split = pl.kps;
  ReduceOut o;
  o.a_sinv = p.a_sinv; o.b_sinv = p.b_sinv; o.b_stride = p.b_stride; o.n_seg = p.n_seg;
  for (int i = 0; i < 4; ++i) o.seg_end.e[i] = p.seg_end[i];
  o.bias = p.bias; o.C = p.C; o.ldc = p.ldc; o.a_vec = p.a_vec; o.b_vec = p.b_vec;
  o.unit = mx ? 1 : 0;
  if (pl.tail_pieces > 0) {
    // whole tiles write C; the tail tiles' pieces write raw partials, reduced after
    p.full_tiles = pl.full_tiles;
    p.tail_pieces = pl.tail_pieces;
    p.tail_ws = static_cast<float*>(ws);
    const int rc = launch_tile(pl, p, epi, out_dtype, fa, fb, s, mx);
    if (rc != BF8_OK) return rc;
    const TileInfo& ti = kTiles[pl.tile];
    const int tails = pl.tiles_m * pl.tiles_n - pl.full_tiles;
    const unsigned blocks = (unsigned)(tails * (ti.bm * ti.bn / 2048));
    if (out_dtype == BF8_OUT_BF16)
      hipLaunchKernelGGL(tail_reduce_kernel<BF8_OUT_BF16>, dim3(blocks), dim3(256), 0, s,
                         (const float*)ws, pl.tail_pieces, ti.bm, ti.bn, pl.full_tiles,
                         pl.tiles_m, pl.tiles_n, p.M, p.N, o);
    else
      hipLaunchKernelGGL(tail_reduce_kernel<BF8_OUT_F32>, dim3(blocks), dim3(256), 0, s,
                         (const float*)ws, pl.tail_pieces, ti.bm, ti.bn, pl.full_tiles,
                         pl.tiles_m, pl.tiles_n, p.M, p.N, o);
    return launch_status("tail_reduce_kernel");
  }
  if (pl.splits == 1) return launch_tile(pl, p, epi, out_dtype, fa, fb, s, mx);
  // K split: raw fp32 partials into the workspace, then the ordered reduction
  GemmParams q = p;
  q.C = ws;
  q.ldc = p.N;
  q.split_stride = (int64_t)p.M * p.N;
  q.bias = nullptr;
  const int rc = launch_tile(pl, q, EPI_LINEAR, BF8_OUT_F32, fa, fb, s, mx);
  if (rc != BF8_OK) return rc;
  const int64_t items = (int64_t)p.M * (p.N / 8);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(items, 256), 4096);
  if (out_dtype == BF8_OUT_BF16)
    hipLaunchKernelGGL(split_reduce_kernel<BF8_OUT_BF16>, dim3(blocks), dim3(256), 0, s,
                       (const float*)ws, pl.splits, q.split_stride, p.M, p.N, o);
  else
    hipLaunchKernelGGL(split_reduce_kernel<BF8_OUT_F32>, dim3(blocks), dim3(256), 0, s,
                       (const float*)ws, pl.splits, q.split_stride, p.M, p.N, o);
  return launch_status("split_reduce_kernel");
}

int gemm_entry(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b, int64_t ldb,
               int64_t M, int64_t N, int64_t K, const float* a_scale_inv, int a_vec,
               const float* b_scale_inv, int b_vec, int b_scale_stride, const int64_t* seg_ends,
               int n_seg, const void* bias, void* C, int out_dtype, int64_t ldc, void* ws,
               size_t ws_bytes, void* stream) {
  BF8_CHECK(((fmt_a == BF8_E4M3 || fmt_a == BF8_E5M2) && (fmt_b == BF8_E4M3 || fmt_b == BF8_E5M2)) ||
                (fmt_a == kFmtBf16 && fmt_b == kFmtBf16),
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
  BF8_CHECK(((uintptr_t)bias & 7) == 0, "bf8_gemm: bias must be 8-byte aligned");
  BF8_CHECK(ws_bytes == 0 || (ws && ((uintptr_t)ws & 255) == 0),
            "bf8_gemm: workspace must be 256-byte aligned");
  if (M == 0 || N == 0) return BF8_OK;
  BF8_CHECK(K > 0, "bf8_gemm: K == 0 is not supported");
  BF8_CHECK(A && B && C, "bf8_gemm: A, B or C is NULL");
  GemmParams p{};
  p.A = A; p.B = B; p.lda = lda; p.ldb = ldb;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.I = 0;
  p.a_sinv = a_scale_inv; p.b_sinv = b_scale_inv; p.b_stride = b_scale_stride;
  p.a_vec = a_vec; p.b_vec = b_vec;
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
  const Plan pl = choose_plan(M, N, K, false, ws ? ws_bytes : 0);
  return launch_plan(pl, p, EPI_LINEAR, out_dtype, fmt_a, fmt_b, ws, as_stream(stream));
}

}  // namespace
}  // namespace bf8

using namespace bf8;

extern "C" {

size_t bf8_gemm_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return choose_plan(M, N, K, false, (size_t)-1).ws_bytes;
}

int bf8_gemm(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b, int64_t ldb,
             int64_t M, int64_t N, int64_t K, const float* a_scale_inv,
             const float* b_scale_inv, int b_scale_stride, const int64_t* seg_ends, int n_seg,
             const void* bias, void* C, int out_dtype, int64_t ldc, void* ws, size_t ws_bytes,
             void* stream) {
  return gemm_entry(A, fmt_a, lda, B, fmt_b, ldb, M, N, K, a_scale_inv, 0, b_scale_inv, 0,
                    b_scale_stride, seg_ends, n_seg, bias, C, out_dtype, ldc, ws, ws_bytes, stream);
}

size_t bf8_gemm_bf16_workspace(int64_t M, int64_t N, int64_t K) {
  return bf8_gemm_workspace(M, N, 2 * K);  // plans are made on K bytes
}

size_t bf8_gemm_kmajor_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // the larger of the two layouts' needs (the B-only call may run on a transposed B)
  const KmajorChoice b_only = choose_kmajor(M, N, K, false, (size_t)-1);
  const size_t both = choose_kmajor(M, N, K, true, (size_t)-1).plan.ws_bytes;
  return std::max(both, b_only.b_bytes + b_only.plan.ws_bytes);
}

int bf8_gemm_kmajor(const uint8_t* A, int fmt_a, int64_t lda, int a_kmajor, const uint8_t* B,
                    int fmt_b, int64_t ldb, int64_t M, int64_t N, int64_t K,
                    const float* a_scale_inv, const float* b_scale_inv, void* C, int out_dtype,
                    int64_t ldc, void* ws, size_t ws_bytes, void* stream) {
  const char* who = "bf8_gemm_kmajor";
  BF8_CHECK(fmt_a == BF8_E5M2 && fmt_b == BF8_E4M3,
            "%s: formats %d x %d (supported: e5m2 x e4m3)", who, fmt_a, fmt_b);
  BF8_CHECK(a_kmajor == 0 || a_kmajor == 1, "%s: a_kmajor must be 0 or 1", who);
  BF8_CHECK(out_dtype == BF8_OUT_BF16 || out_dtype == BF8_OUT_F32, "%s: bad out_dtype", who);
  BF8_CHECK(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", who);
  if (a_kmajor)
    BF8_CHECK(M % 16 == 0 && lda % 16 == 0 && lda >= M && K * lda < (1LL << 31),
              "%s: A^T [K, M] needs M and lda multiples of 16, lda >= M, < 2 GiB", who);
  else
    BF8_CHECK(K % 16 == 0 && lda % 16 == 0 && lda >= K && M * lda < (1LL << 31),
              "%s: A [M, K] needs K and lda multiples of 16, lda >= K, < 2 GiB", who);
  BF8_CHECK(N % 16 == 0 && ldb % 16 == 0 && ldb >= N && K * ldb < (1LL << 31),
            "%s: B^T [K, N] needs N and ldb multiples of 16, ldb >= N, < 2 GiB", who);
  BF8_CHECK(ldc >= N && ldc % 4 == 0, "%s: need ldc >= N, ldc %% 4 == 0", who);
  BF8_CHECK(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && ((uintptr_t)C & 15) == 0,
            "%s: A, B, C must be 16-byte aligned", who);
  BF8_CHECK(a_scale_inv && b_scale_inv, "%s: scale pointers are NULL", who);
  BF8_CHECK(ws_bytes == 0 || (ws && ((uintptr_t)ws & 255) == 0),
            "%s: workspace must be 256-byte aligned", who);
  if (M == 0 || N == 0) return BF8_OK;
  BF8_CHECK(K > 0, "%s: K == 0 is not supported", who);
  BF8_CHECK(A && B && C, "%s: A, B or C is NULL", who);
  GemmParams p{};
  p.A = A; p.B = B; p.lda = lda; p.ldb = ldb;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.I = 0;
  p.a_sinv = a_scale_inv; p.b_sinv = b_scale_inv;
  p.n_seg = 1;
  for (int s = 0; s < 4; ++s) p.seg_end[s] = (int)N;
  p.C = C; p.ldc = ldc;
  p.kmajor = a_kmajor ? 3 : 2;
  hipStream_t s = as_stream(stream);
  const KmajorChoice ch = choose_kmajor(M, N, K, a_kmajor != 0, ws ? ws_bytes : 0);
  if (!ch.transpose_b) return launch_plan(ch.plan, p, EPI_LINEAR, out_dtype, fmt_a, fmt_b, ws, s);
  // B^T [K, N] -> B [N, K] in the workspace, then the row-major plan on it
  uint8_t* bt = static_cast<uint8_t*>(ws);
  const int64_t tiles = ((K + 63) / 64) * ((N + 63) / 64);
  hipLaunchKernelGGL(transpose_u8_kernel, dim3((unsigned)((tiles + kTransposeWaves - 1) / kTransposeWaves)),
                     dim3(kTransposeWaves * 64), 0, s, B, K, N, ldb, bt);
  const int rc = launch_status("transpose_u8_kernel");
  if (rc != BF8_OK) return rc;
  p.B = bt;
  p.ldb = K;
  p.kmajor = 0;
  return launch_plan(ch.plan, p, EPI_LINEAR, out_dtype, fmt_a, fmt_b,
                     ch.plan.ws_bytes ? bt + ch.b_bytes : nullptr, s);
}

int bf8_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                  int64_t K, const float* a_scale_inv, const float* b_scale_inv, void* C,
                  int out_dtype, int64_t ldc, void* ws, size_t ws_bytes, void* stream) {
  BF8_CHECK(K >= 0 && lda >= 0 && ldb >= 0, "bf8_gemm_bf16: negative size");
  BF8_CHECK(K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0,
            "bf8_gemm_bf16: need K, lda, ldb multiples of 8 (K=%lld lda=%lld ldb=%lld)",
            (long long)K, (long long)lda, (long long)ldb);
  return gemm_entry((const uint8_t*)A, kFmtBf16, 2 * lda, (const uint8_t*)B, kFmtBf16, 2 * ldb,
                    M, N, 2 * K, a_scale_inv, 0, b_scale_inv, 0, 0, nullptr, 1, nullptr, C,
                    out_dtype, ldc, ws, ws_bytes, stream);
}

int bf8_gemm_axiswise(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b,
                      int64_t ldb, int64_t M, int64_t N, int64_t K, const float* a_scale_inv,
                      int a_vec, const float* b_scale_inv, int b_vec, const void* bias, void* C,
                      int out_dtype, int64_t ldc, void* ws, size_t ws_bytes, void* stream) {
  BF8_CHECK((a_vec == 0 || a_vec == 1) && (b_vec == 0 || b_vec == 1),
            "bf8_gemm_axiswise: a_vec and b_vec must be 0 or 1");
  BF8_CHECK(!b_vec || ((uintptr_t)b_scale_inv & 15) == 0,
            "bf8_gemm_axiswise: a per-column b_scale_inv must be 16-byte aligned");
  return gemm_entry(A, fmt_a, lda, B, fmt_b, ldb, M, N, K, a_scale_inv, a_vec, b_scale_inv,
                    b_vec, 0, nullptr, 1, bias, C, out_dtype, ldc, ws, ws_bytes, stream);
}


int64_t bf8_geglu_partials(int64_t M, int64_t I) {
  if (M <= 0 || I <= 0) return 0;
  const Plan pl = choose_plan(M, 2 * I, 0, true, 0);
  return (int64_t)pl.tiles_m * pl.tiles_n;
}

// The gate/up GEMM + gated GELU; h_scale set: H quantized in the epilogue (H8, H8t).
// K, ldx and ldw in bytes; fmt: BF8_E4M3 operands, or kFmtBf16 (two bytes per element)
static int geglu_entry(const char* who, const uint8_t* X, int64_t ldx, const uint8_t* W,
                       int64_t ldw, int64_t M, int64_t I, int64_t K, const float* x_scale_inv,
                       const float* w_scale_inv, int w_scale_stride, void* H, int64_t ldh,
                       const float* h_scale, uint8_t* H8, uint8_t* H8t, void* GU,
                       uint32_t* h_partials, void* stream, int fmt = BF8_E4M3) {
  BF8_CHECK(M >= 1 && I >= 1 && K >= 16, "%s: bad shape", who);
  BF8_CHECK(I % 128 == 0, "%s: I must be a multiple of 128 (got %lld)", who, (long long)I);
  BF8_CHECK(K % 16 == 0 && ldx % 16 == 0 && ldw % 16 == 0 && ldx >= K && ldw >= K,
            "%s: need K, ldx, ldw multiples of 16 and >= K", who);
  BF8_CHECK(H || H8, "%s: H is NULL", who);
  BF8_CHECK(!H || (ldh >= I && ldh % 4 == 0), "%s: bad ldh", who);
  BF8_CHECK(((uintptr_t)X & 15) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)H & 15) == 0 &&
                ((uintptr_t)GU & 15) == 0,
            "%s: X, W, H, GU must be 16-byte aligned", who);
  BF8_CHECK(M * ldx < (1LL << 31) && 2 * I * ldw < (1LL << 31), "%s: operand > 2 GiB", who);
  BF8_CHECK(X && W && x_scale_inv && w_scale_inv && h_partials, "%s: NULL pointer", who);
  if (H8) {
    BF8_CHECK(h_scale && ((uintptr_t)H8 & 7) == 0, "%s: H8 needs h_scale and 8-byte alignment",
              who);
    BF8_CHECK(M * I < (1LL << 31), "%s: H8 larger than 2 GiB", who);
  }
  BF8_CHECK(!H8t || H8, "%s: H8t needs H8", who);
  BF8_CHECK(!H8t || (M % 32 == 0 && ((uintptr_t)H8t & 15) == 0),
            "%s: H8t needs M %% 32 == 0 (got %lld) and 16-byte alignment", who, (long long)M);
  GemmParams p{};
  p.A = X; p.B = W; p.lda = ldx; p.ldb = ldw;
  p.M = (int)M; p.N = (int)(2 * I); p.K = (int)K; p.I = (int)I;
  p.a_sinv = x_scale_inv; p.b_sinv = w_scale_inv; p.b_stride = w_scale_stride;
  p.n_seg = 1;
  p.C = H; p.ldc = ldh; p.GU = (uint16_t*)GU; p.partials = h_partials;
  p.h8_scale = h_scale; p.h8 = H8; p.h8t = H8t;
  Plan pl = choose_plan(M, 2 * I, K, true, 0);
  return launch_plan(pl, p, EPI_GEGLU, BF8_OUT_BF16, fmt, fmt, nullptr, as_stream(stream));
}

int bf8_gemm_geglu(const uint8_t* X, int64_t ldx, const uint8_t* W, int64_t ldw, int64_t M,
                   int64_t I, int64_t K, const float* x_scale_inv, const float* w_scale_inv,
                   int w_scale_stride, void* H, int64_t ldh, void* GU, uint32_t* h_partials,
                   void* stream) {
  return geglu_entry("bf8_gemm_geglu", X, ldx, W, ldw, M, I, K, x_scale_inv, w_scale_inv,
                     w_scale_stride, H, ldh, nullptr, nullptr, nullptr, GU, h_partials, stream);
}

int bf8_gemm_geglu_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw, int64_t M,
                        int64_t I, int64_t K, const float* x_scale, const float* w_scale,
                        void* H, int64_t ldh, void* GU, uint32_t* h_partials, void* stream) {
  BF8_CHECK(K >= 8 && K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0,
            "bf8_gemm_geglu_bf16: need K, ldx, ldw multiples of 8 (K=%lld ldx=%lld ldw=%lld)",
            (long long)K, (long long)ldx, (long long)ldw);
  return geglu_entry("bf8_gemm_geglu_bf16", (const uint8_t*)X, 2 * ldx, (const uint8_t*)W,
                     2 * ldw, M, I, 2 * K, x_scale, w_scale, 0, H, ldh, nullptr, nullptr, nullptr,
                     GU, h_partials, stream, kFmtBf16);
}

int bf8_gemm_geglu_quant(const uint8_t* X, int64_t ldx, const uint8_t* W, int64_t ldw,
                         int64_t M, int64_t I, int64_t K, const float* x_scale_inv,
                         const float* w_scale_inv, int w_scale_stride, const float* h_scale,
                         void* H, int64_t ldh, uint8_t* H8, uint8_t* H8t, void* GU,
                         uint32_t* h_partials, void* stream) {
  BF8_CHECK(H8 != nullptr, "bf8_gemm_geglu_quant: H8 is NULL");
  return geglu_entry("bf8_gemm_geglu_quant", X, ldx, W, ldw, M, I, K, x_scale_inv, w_scale_inv,
                     w_scale_stride, H, ldh, h_scale, H8, H8t, GU, h_partials, stream);
}

// ---- MX (block-scaled) GEMMs ----------------------------------------------------------
size_t bf8_gemm_mx_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return choose_plan(M, N, K, false, (size_t)-1, true).ws_bytes;
}

int64_t bf8_mx_scale_ld(int64_t K) { return (K + 127) / 128 * 4; }

static int check_mx_operand(const char* who, const char* what, const uint8_t* q, int64_t ld,
                            const uint8_t* sc, int64_t ld_sc, int64_t rows, int64_t K) {
  BF8_CHECK(q && sc, "%s: %s or its scales are NULL", who, what);
  BF8_CHECK(ld % 16 == 0 && ld >= K && ((uintptr_t)q & 15) == 0,
            "%s: %s needs a 16-byte aligned base and row stride >= K", who, what);
  BF8_CHECK(ld_sc % 4 == 0 && ld_sc >= bf8_mx_scale_ld(K) && ((uintptr_t)sc & 3) == 0,
            "%s: %s scales need a 4-byte aligned base and row stride >= %lld", who, what,
            (long long)bf8_mx_scale_ld(K));
  BF8_CHECK(rows * ld < (1LL << 31) && rows * ld_sc < (1LL << 31), "%s: %s larger than 2 GiB",
            who, what);
  return BF8_OK;
}

int bf8_gemm_mx(const uint8_t* A, int64_t lda, const uint8_t* A_scales, int64_t lda_sc,
                const uint8_t* B, int64_t ldb, const uint8_t* B_scales, int64_t ldb_sc,
                int64_t M, int64_t N, int64_t K, const void* bias, void* C, int out_dtype,
                int64_t ldc, void* ws, size_t ws_bytes, void* stream) {
  BF8_CHECK(out_dtype == BF8_OUT_BF16 || out_dtype == BF8_OUT_F32, "bf8_gemm_mx: bad out_dtype");
  BF8_CHECK(M >= 0 && N >= 0 && K >= 0, "bf8_gemm_mx: negative shape");
  BF8_CHECK(K % 32 == 0, "bf8_gemm_mx: K must be a multiple of the 32-element block (got %lld)",
            (long long)K);
  BF8_CHECK(N % 8 == 0 && ldc >= N && ldc % 4 == 0,
            "bf8_gemm_mx: need N %% 8 == 0, ldc >= N, ldc %% 4 == 0");
  BF8_CHECK(((uintptr_t)C & 15) == 0 && ((uintptr_t)bias & 7) == 0,
            "bf8_gemm_mx: C must be 16-byte, bias 8-byte aligned");
  BF8_CHECK(ws_bytes == 0 || (ws && ((uintptr_t)ws & 255) == 0),
            "bf8_gemm_mx: workspace must be 256-byte aligned");
  if (M == 0 || N == 0) return BF8_OK;
  BF8_CHECK(K > 0, "bf8_gemm_mx: K == 0 is not supported");
  BF8_CHECK(C != nullptr, "bf8_gemm_mx: C is NULL");
  int rc = check_mx_operand("bf8_gemm_mx", "A", A, lda, A_scales, lda_sc, M, K);
  if (rc) return rc;
  rc = check_mx_operand("bf8_gemm_mx", "B", B, ldb, B_scales, ldb_sc, N, K);
  if (rc) return rc;
  GemmParams p{};
  p.A = A; p.B = B; p.lda = lda; p.ldb = ldb;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.I = 0;
  p.a_sc = A_scales; p.b_sc = B_scales; p.a_sc_ld = lda_sc; p.b_sc_ld = ldb_sc;
  p.n_seg = 1;
  for (int s = 0; s < 4; ++s) p.seg_end[s] = (int)N;
  p.bias = (const uint16_t*)bias; p.C = C; p.ldc = ldc;
  const Plan pl = choose_plan(M, N, K, false, ws ? ws_bytes : 0, true);
  return launch_plan(pl, p, EPI_LINEAR, out_dtype, BF8_E4M3, BF8_E4M3, ws, as_stream(stream),
                     true);
}

// The MX gate/up GEMM + gated GELU; H8 (with H8t) set: H quantized in the epilogue.
static int geglu_mx_entry(const char* who, const uint8_t* X, int64_t ldx, const uint8_t* X_scales,
                          int64_t ldx_sc, const uint8_t* W, int64_t ldw, const uint8_t* W_scales,
                          int64_t ldw_sc, int64_t M, int64_t I, int64_t K, void* H, int64_t ldh,
                          uint8_t* H8, uint8_t* H8_scales, int64_t ldh8_sc, uint8_t* H8t,
                          uint8_t* H8t_scales, int64_t ldh8t_sc, void* GU, void* stream) {
  BF8_CHECK(M >= 1 && I >= 1 && K >= 32, "%s: bad shape", who);
  BF8_CHECK(I % 128 == 0, "%s: I must be a multiple of 128 (got %lld)", who, (long long)I);
  BF8_CHECK(K % 32 == 0, "%s: K must be a multiple of 32", who);
  BF8_CHECK(H || H8, "%s: H is NULL", who);
  BF8_CHECK(!H || (ldh >= I && ldh % 4 == 0), "%s: bad ldh", who);
  BF8_CHECK(((uintptr_t)H & 15) == 0 && ((uintptr_t)GU & 15) == 0,
            "%s: H, GU must be 16-byte aligned", who);
  if (H8) {
    BF8_CHECK(H8_scales && ldh8_sc >= I / 32 && ((uintptr_t)H8 & 7) == 0,
              "%s: H8 needs 8-byte alignment and scales with row stride >= I / 32", who);
    BF8_CHECK(M * I < (1LL << 31), "%s: H8 larger than 2 GiB", who);
  }
  BF8_CHECK(!H8t || H8, "%s: H8t needs H8", who);
  if (H8t) {
    BF8_CHECK(M % 32 == 0, "%s: H8t blocks along M need M %% 32 == 0 (got %lld)", who,
              (long long)M);
    BF8_CHECK(H8t_scales && ldh8t_sc >= bf8_mx_scale_ld(M) && ((uintptr_t)H8t & 15) == 0,
              "%s: H8t needs 16-byte alignment and scales with row stride >= %lld", who,
              (long long)bf8_mx_scale_ld(M));
  }
  int rc = check_mx_operand(who, "X", X, ldx, X_scales, ldx_sc, M, K);
  if (rc) return rc;
  rc = check_mx_operand(who, "W", W, ldw, W_scales, ldw_sc, 2 * I, K);
  if (rc) return rc;
  GemmParams p{};
  p.A = X; p.B = W; p.lda = ldx; p.ldb = ldw;
  p.M = (int)M; p.N = (int)(2 * I); p.K = (int)K; p.I = (int)I;
  p.a_sc = X_scales; p.b_sc = W_scales; p.a_sc_ld = ldx_sc; p.b_sc_ld = ldw_sc;
  p.n_seg = 1;
  p.C = H; p.ldc = ldh; p.GU = (uint16_t*)GU; p.partials = nullptr;
  p.h8 = H8; p.h8_sc = H8_scales; p.h8_sc_ld = ldh8_sc;
  p.h8t = H8t; p.h8t_sc = H8t_scales; p.h8t_sc_ld = ldh8t_sc;
  Plan pl = choose_plan(M, 2 * I, K, true, 0, true);
  return launch_plan(pl, p, EPI_GEGLU, BF8_OUT_BF16, BF8_E4M3, BF8_E4M3, nullptr,
                     as_stream(stream), true);
}

int bf8_gemm_geglu_mx(const uint8_t* X, int64_t ldx, const uint8_t* X_scales, int64_t ldx_sc,
                      const uint8_t* W, int64_t ldw, const uint8_t* W_scales, int64_t ldw_sc,
                      int64_t M, int64_t I, int64_t K, void* H, int64_t ldh, void* GU,
                      void* stream) {
  return geglu_mx_entry("bf8_gemm_geglu_mx", X, ldx, X_scales, ldx_sc, W, ldw, W_scales, ldw_sc,
                        M, I, K, H, ldh, nullptr, nullptr, 0, nullptr, nullptr, 0, GU, stream);
}

int bf8_gemm_geglu_mx_quant(const uint8_t* X, int64_t ldx, const uint8_t* X_scales,
                            int64_t ldx_sc, const uint8_t* W, int64_t ldw,
                            const uint8_t* W_scales, int64_t ldw_sc, int64_t M, int64_t I,
                            int64_t K, void* H, int64_t ldh, uint8_t* H8, uint8_t* H8_scales,
                            int64_t ldh8_sc, uint8_t* H8t, uint8_t* H8t_scales,
                            int64_t ldh8t_sc, void* GU, void* stream) {
  BF8_CHECK(H8 != nullptr, "bf8_gemm_geglu_mx_quant: H8 is NULL");
  return geglu_mx_entry("bf8_gemm_geglu_mx_quant", X, ldx, X_scales, ldx_sc, W, ldw, W_scales,
                        ldw_sc, M, I, K, H, ldh, H8, H8_scales, ldh8_sc, H8t, H8t_scales,
                        ldh8t_sc, GU, stream);
}

}  // extern "C"
