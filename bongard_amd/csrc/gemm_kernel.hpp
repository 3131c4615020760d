// Shared declarations of the FP8 GEMM: launch parameters, block-tile shapes and the
// per-tile launchers (each instantiated in its own gemm_tile_*.hip translation unit so
// that the tile variants compile in parallel).
#pragma once

#include "common.hpp"

namespace bf8 {

enum GemmEpi { EPI_LINEAR = 0, EPI_GEGLU = 1 };

// Operand format of a bf16 GEMM (both operands bf16: 64 K-values per 128-byte step, so K,
// lda and ldb are passed in bytes); the FP8 formats are BF8_E4M3 (0) and BF8_E5M2 (1).
constexpr int kFmtBf16 = 2;

struct GemmParams {
  const uint8_t* A;  // [M, K] row-major, row stride lda bytes
  const uint8_t* B;  // [N, K] row-major (nn.Linear weight layout), row stride ldb bytes
  int64_t lda, ldb;
  int M, N, K;           // for GEGLU, N = 2I (rows of [W_gate; W_up])
  int I;                 // GEGLU intermediate size
  int tiles_m, tiles_n;  // output tiles
  int splits;            // K splits per output tile (LINEAR only; 1 = none)
  int ksteps_per_split;  // 128-byte K steps per split
  const float* a_sinv;    // a_vec: one per row of A (M), else a single value
  const float* b_sinv;    // b_vec: one per row of B (N), else n_seg values b_stride apart
  int a_vec, b_vec;       // LINEAR only
  const uint8_t* a_sc;    // MX: E8M0 block scales [M, a_sc_ld] (byte k/32 of row m)
  const uint8_t* b_sc;    // MX: [N, b_sc_ld]
  int64_t a_sc_ld, b_sc_ld;
  int b_stride;
  int n_seg;
  int seg_end[4];
  const uint16_t* bias;
  void* C;
  int64_t ldc;
  uint16_t* GU;
  uint32_t* partials;     // GEGLU: one amax key of |H| per tile
  // GEGLU with H quantized in the epilogue (C, the bf16 H, may then be NULL). h8: e4m3
  // [M, I]; h8t (optional, needs M % 32 == 0): e4m3 H^T [I, M]. MX: E8M0 block scales
  // h8_sc [M, h8_sc_ld] (blocks along I) and h8t_sc [I, h8t_sc_ld] (blocks along M);
  // otherwise one scale, read from the device word h8_scale.
  const float* h8_scale;
  uint8_t* h8;
  uint8_t* h8_sc;
  uint8_t* h8t;
  uint8_t* h8t_sc;
  int64_t h8_sc_ld, h8t_sc_ld;
  int64_t split_stride;   // splits > 1: C is fp32 [splits][M][ldc], raw sums, this many
                          // elements apart (a reduce kernel applies scales and bias)
  // Tail-split schedule (tail_pieces > 0, linear epilogues, splits == 1): workgroups
  // [0, full_tiles) take whole tiles, walk positions 0 .. full_tiles-1, and write C; the
  // others take one of tail_pieces K pieces (ksteps_per_split steps each) of a tile at walk
  // position full_tiles + t and write its raw fp32 sums to tail_ws[t * tail_pieces + piece]
  // ([BM][BN] each), which tail_reduce_kernel adds in piece order.
  int full_tiles, tail_pieces;
  float* tail_ws;
  // Operand layout (linear epilogues of the eight-wave 256 x 256 tiles): 0 = A [M, K] and
  // B [N, K]; 2 = B given as B^T [K, N] (row stride ldb >= N); 3 = A as A^T [K, M] as well.
  int kmajor;
};

constexpr int kGroupM = 8;  // tile rows walked together (the tile order of a launch)

// Tile (tm, tn) at position id of the tile walk: groups of kGroupM tile rows, each group
// walked with the tile row changing fastest.
__host__ __device__ inline void walk_tile(int tiles_m, int tiles_n, int id, int& tm, int& tn) {
  const int per_group = kGroupM * tiles_n;
  const int g = id / per_group;
  const int first_m = g * kGroupM;
  const int gm = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  const int in_g = id - g * per_group;
  tm = first_m + in_g % gm;
  tn = in_g / gm;
}

// A workgroup is KG groups of NW = WM x WN wave64s (four, or eight: two per SIMD); the
// waves of a group are arranged WM x WN and each owns FM x FN MFMA tiles of 32 x 32
// outputs, so the block tile is (WM*FM*32) x (WN*FN*32). Each group has its own NS LDS
// stages of (BM + BN) x 128 bytes in flight; with KG = 2 the groups take alternate K steps
// and add their accumulators before the epilogue (two pipelines per CU for the short K
// loops of skinny GEMMs). OCC workgroups share a CU (the register budget per wave is
// 512 / (OCC * KG * NW / 4) VGPRs, LDS 160 KB / OCC).
template <int WM_, int WN_, int FM_, int FN_, int NS_, int OCC_, int KG_ = 1, int XB_ = 0>
struct GemmTile {
  static constexpr int WM = WM_, WN = WN_, FM = FM_, FN = FN_, NS = NS_, OCC = OCC_, KG = KG_;
  // XB extra LDS slots for B tiles only: B (the operand streamed from HBM in the skinny
  // gated-GELU GEMM) then loads NS + XB - 1 steps ahead, A NS - 1
  static constexpr int XB = XB_;
  static constexpr int BM = WM * FM * 32, BN = WN * FN * 32;
  static constexpr int NW = WM * WN;  // waves per K group
  static_assert(NW == 4 || (NW == 8 && KG == 1 && OCC == 1),
                "four waves per group, or eight (two per SIMD) in a lone one-group workgroup");
  static_assert(KG == 1 || KG == 2, "one or two K groups");
  static_assert(NS >= 2 && KG * NS * (BM + BN) * 128 * OCC <= 160 * 1024, "LDS budget");
};

using Tile256x256 = GemmTile<2, 2, 4, 4, 2, 1>;
using Tile256x160 = GemmTile<4, 1, 2, 5, 3, 1>;
using Tile160x256 = GemmTile<1, 4, 5, 2, 3, 1>;
using Tile128x128 = GemmTile<2, 2, 2, 2, 4, 1>;
using Tile192x256 = GemmTile<2, 2, 3, 4, 2, 1>;
using Tile128x64 = GemmTile<2, 2, 2, 1, 3, 2>;
using Tile64x128 = GemmTile<2, 2, 1, 2, 3, 2>;
using Tile256x128 = GemmTile<2, 2, 4, 2, 3, 1>;
// eight waves, two per SIMD, each with 128 accumulators of the 256 x 256 tile: while one
// wave of a SIMD waits (LDS reads, the epilogue's dependency chains) the other issues
using Tile256x256w8 = GemmTile<2, 4, 4, 2, 2, 1>;
// the same with a third B slot in the 32 KB its stages leave free (B loads two steps
// ahead): for long-K linear GEMMs whose operands come from HBM rather than the MALL
using Tile256x256w8x = GemmTile<2, 4, 4, 2, 2, 1, 1, 1>;
// two K groups (skinny GEMMs): 8 waves, alternate K steps
using Tile128x64k2 = GemmTile<2, 2, 2, 1, 3, 1, 2>;
using Tile64x128k2 = GemmTile<2, 2, 1, 2, 3, 1, 2>;
using Tile128x128k2 = GemmTile<2, 2, 2, 2, 2, 1, 2>;

// Enqueues the GEMM for tile shape T (EPI_GEGLU: e4m3 x e4m3, bf16 H). Returns a BF8_*
// status; the host entry points have validated p.
template <class T>
int launch_gemm_tile(const GemmParams& p, int epi, int out_dtype, int fmt_a, int fmt_b,
                     hipStream_t stream, bool mx);

}  // namespace bf8
