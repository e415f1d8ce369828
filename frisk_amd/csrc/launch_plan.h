// Launch planning of the GEMM and attention kernels on gfx950: which kernel,
// workgroup tile, wave grid, K split and attention workgroup shape a request
// runs with.  Host-only C++ without HIP, so that two consumers share one
// decision: the C-ABI (capi.hip, gemm.hip, the launchers) follows it for
// every call that names no variant, and the layout target of the IR
// (frisk_amd/ir: F.frisk.gemm_launch_plan / attn_launch_plan) reports it as
// the launch contract of a whole-matrix GEMM or an attention program, which
// execute() then requests explicitly.  The reference makes the matching
// decision at compile time, in its SM90 layout target's MMA binding
// (lib/Dialect/Frisk/Target/SM90/SM90LayoutTarget.cpp:171-481).
//
// Every estimate here is in seconds of one launch, from rates measured on
// MI355X with operands streaming from HBM (the measurements are cited where
// each rule is applied).
#pragma once

#include <algorithm>
#include <cstdint>

namespace frisk {
namespace plan {

// Element codes: frisk_dtype of include/frisk_hip.h.
constexpr int kF32 = 0, kF16 = 1, kBF16 = 2, kE4M3 = 3, kI8 = 4, kI32 = 5;
inline int dtype_bytes(int t) {
  return t == kF16 || t == kBF16 ? 2 : t == kE4M3 || t == kI8 ? 1 : 4;
}

// A GEMM request as the planner sees it (sizes in elements).  tile /
// wave_m / wave_n / slices: a requested variant (0: the library chooses).
struct GemmShape {
  int in = kBF16, out = kBF16;
  int64_t m = 0, n = 0, k = 0;
  bool trans_a = false, trans_b = false;
  int tile = 0, wave_m = 0, wave_n = 0, slices = 0;
};

// Small-M rows this many or fewer can run on the small-M kernel.
#ifndef FRISK_SKINNY_MAX_M
#define FRISK_SKINNY_MAX_M 128
#endif
constexpr int64_t kSkinnyMaxM = FRISK_SKINNY_MAX_M;
// Small-M rows this many or fewer stay on the small-M kernel when split;
// more (up to its limit) run split on 128x128 tiles, which share each X
// tile across the workgroup's waves through LDS.
constexpr int64_t kSkinnySplitMaxM = 64;
// Split-K arrival words per tile of the in-launch slice sum (gemm_common.h
// splitk_tree) and the most slices summed that way on 128x128 tiles.
constexpr int kTreeWords = 64;
constexpr int kTreeMaxSlices = 2;

// Workspace of a split summed inside the GEMM launch: an f32 partial tile
// per (tile, slice) of bt x bt outputs, then kTreeWords 64-bit arrival
// words per tile.
inline int64_t split_tree_bytes(int64_t tiles, int64_t slices, int bt) {
  return tiles * slices * (int64_t)bt * bt * 4 + tiles * kTreeWords * 8;
}

// ---------------------------------------------------------------------------
// Split-K of the LDS-staged MFMA kernels (bf16/f16/f32): `slices` slices of
// kb_slice bytes of K whose f32 partials (and arrival words) take
// workspace_bytes; slices == 1 runs unsplit.  big: the slices run on
// 256x256 tiles instead of 128x128.
// ---------------------------------------------------------------------------
struct SplitPlan {
  int slices;
  int64_t kb_slice;
  int64_t workspace_bytes;
  bool big;
};

// A 128x128-tile workgroup computes about 2.5 TFLOP/s on its CU with
// operands from HBM, a 256x256-tile one about 4.7; the f32 partials are
// written and read back at about 3.5 TB/s plus one launch.
constexpr double kRate128 = 2.5e12, kRate256 = 4.7e12, kPartialBw = 3.5e12, kLaunch = 3e-6;
inline double rounds(int64_t wgs, int64_t slots) { return (double)((wgs + slots - 1) / slots); }
inline double partial_cost(const GemmShape& g, int64_t slices) {
  return slices > 1 ? ((double)slices * g.m * g.n * 4 + (double)g.m * g.n * 2) / kPartialBw + kLaunch
                    : 0.0;
}
// The f32 partials of a split (slices x M x N x 4 bytes) stay within
// (M + N) x K x esize bytes: the bytes of A and B.  Measured with operands
// from HBM, us, a quarter of A + B -> all of it: 256x4096x4096 27.4 -> 23.1
// (2 -> 4 slices), 512x4096x4096 41.8 -> 28.5 (8 slices of 256x256 tiles
// -> 2 of 128x128); 128x4096x4096 19.3 either way (4 -> 8 slices).
constexpr int64_t kSplitCap = 4;
// Bytes of K per pipeline stage of the 128x128 kernel in grids of more
// than one workgroup per CU (gemm_128.h).
constexpr int64_t kRow = 64;

inline SplitPlan split_plan(const GemmShape& g, int cus) {
  const int64_t kb = g.k * dtype_bytes(g.in);  // bytes of K per row
  SplitPlan p{1, kb, 0, false};
  // bf16 / f16 / f32 only (the partials carry no fp8 scale, and int8 sums
  // stay exact in one pass); the slice sum reads rows of 4 floats.
  if ((g.in != kBF16 && g.in != kF16 && g.in != kF32) || g.n % 4 != 0) return p;
  // Grids of at least CUs / 2 256x256 tiles run unsplit on them.
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  if (tiles256 >= cus / 2) return p;
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  // 128x128 tiles.  Split only grids that leave CUs without a tile, each
  // slice at least 8 stages, and the f32 partials at most the bytes of A
  // and B (kSplitCap).  Grids of at most half as many tiles as CUs take
  // slices up to one workgroup per CU, on 128-byte stages (the launch picks
  // them when slices fit one workgroup per CU); larger grids take slices up
  // to two workgroups per CU on 64-byte stages.  Measured on the projection
  // sweep: M = 128 runs 1.6-4.8x faster than on the unsplit small-M
  // kernel; with operands from HBM, 128 x 4096 x 14336 323 -> 416 TFLOP/s
  // and 128 x 14336 x 4096 334 -> 373 on 128-byte stages (one workgroup
  // per CU) against 64-byte ones (two); M = 1024, N = 4096 (256 tiles) runs
  // 1.3x slower split in two.
  if (tiles < cus) {
    const bool deep = 2 * tiles <= cus;
    const int64_t row = deep ? 128 : kRow;  // bytes of K per stage
    int64_t slices = deep ? cus / tiles : (2 * (int64_t)cus + tiles - 1) / tiles;
    if (g.in == kF32) {
      // fp32 runs the MFMA 16x slower per byte of operand than bf16: the
      // K loop, not the partials' traffic, sets the time, so slices of 4
      // stages and no cap on the partials (1024^3: 64 tiles in 4 slices,
      // 32.4 -> 70.2 TFLOP/s).
      slices = std::min<int64_t>(slices, kb / (4 * row));
    } else {
      slices = std::min<int64_t>(slices, kb / (8 * row));
      slices = std::min<int64_t>(slices, (g.m + g.n) * kb / (kSplitCap * g.m * g.n));
    }
    slices = std::min<int64_t>(slices, 64);
    if (slices >= 2) {
      const int64_t chunks = (kb + row - 1) / row;  // slices start on stage boundaries
      p.kb_slice = ((chunks + slices - 1) / slices) * row;
      p.slices = (int)((kb + p.kb_slice - 1) / p.kb_slice);
      if (p.slices < 2) p = SplitPlan{1, kb, 0, false};
    }
  }
  // 256x256 tiles split over K, for M past the small-M range, when the
  // estimate says they end sooner (by 20%) than the 128x128 choice above:
  // a 256-tile workgroup does twice the work per CU cycle, the split buys
  // back the parallelism, the partials cost their traffic.  Slices of at
  // least 8 stages (8 x 128 B of K).  Measured, operands from HBM:
  // 768x4096x4096 61.4 -> 46.0 us, 640x4096x8192 83.5 -> 62.4,
  // 384x4096x14336 78.2 -> 68.1, 1024x4096x14336 141 -> 116 (the 128x128
  // choice -> this one).  (The rates are those of bf16 / f16; f32 keeps
  // the 128x128 split.)
  if (g.m > kSkinnyMaxM && g.in != kF32) {
    const double flop128 = 2.0 * 128 * 128 * (double)(p.kb_slice / 2);
    const double t128 = rounds(tiles * p.slices, cus) * flop128 / kRate128 + partial_cost(g, p.slices);
    double best = 0.0;
    int64_t best_s = 0;
    for (int64_t sl = 2; sl <= 16 && kb / sl >= 1024; ++sl) {
      const int64_t kb_slice = ((kb + 127) / 128 + sl - 1) / sl * 128;
      const double t = rounds(tiles256 * sl, cus) * 2.0 * 256 * 256 * (double)(kb_slice / 2) / kRate256 +
                       partial_cost(g, sl);
      if (best_s == 0 || t < best) {
        best = t;
        best_s = sl;
      }
    }
    if (best_s > 0 && best < 0.8 * t128) {
      p.kb_slice = ((kb + 127) / 128 + best_s - 1) / best_s * 128;
      p.slices = (int)((kb + p.kb_slice - 1) / p.kb_slice);
      p.big = p.slices > 1;
      if (!p.big) p = SplitPlan{1, kb, 0, false};
    }
  }
  p.workspace_bytes = p.slices <= 1 ? 0
                     : !p.big && p.slices <= kTreeMaxSlices ? split_tree_bytes(tiles, p.slices, 128)
                                                            : (int64_t)p.slices * g.m * g.n * 4;
  return p;
}

// A requested variant with `slices` K slices (tile 256 or 128 with the 2x2
// wave grid, bf16/f16/f32): the slices start on stage boundaries as the
// library's own split would place them.
inline SplitPlan requested_split(const GemmShape& g, int cus) {
  const int64_t kb = g.k * dtype_bytes(g.in);
  SplitPlan p{1, kb, 0, false};
  if (g.slices <= 1) return p;
  const bool big = g.tile == 256;
  const int64_t tiles = big ? ((g.m + 255) / 256) * ((g.n + 255) / 256)
                            : ((g.m + 127) / 128) * ((g.n + 127) / 128);
  const int64_t row = big || tiles * g.slices <= cus ? 128 : kRow;
  const int64_t chunks = (kb + row - 1) / row;
  p.kb_slice = ((chunks + g.slices - 1) / g.slices) * row;
  p.slices = (int)((kb + p.kb_slice - 1) / p.kb_slice);
  if (p.slices < 2) return SplitPlan{1, kb, 0, false};
  p.big = big;
  p.workspace_bytes = !big && p.slices <= kTreeMaxSlices ? split_tree_bytes(tiles, p.slices, 128)
                                                         : (int64_t)p.slices * g.m * g.n * 4;
  return p;
}

// The launch of the LDS-staged MFMA kernels: 256x256 tiles (big) or
// 128x128, and the K slices (1: unsplit) of kb_slice bytes; `workspace` =
// a large enough workspace is at hand.
struct MfmaChoice {
  bool big;
  int slices;
  int64_t kb_slice;
};

inline MfmaChoice mfma_choice(const GemmShape& g, int cus, bool workspace) {
  const int64_t kb = g.k * dtype_bytes(g.in);
  if (g.tile) {
    // A requested variant runs on the tile it names, split only when the
    // request names slices (and a workspace is at hand).
    const SplitPlan r = requested_split(g, cus);
    if (workspace && r.slices > 1) return MfmaChoice{g.tile == 256, r.slices, r.kb_slice};
    return MfmaChoice{g.tile == 256, 1, kb};
  }
  const SplitPlan p = split_plan(g, cus);
  if (workspace && p.slices > 1) return MfmaChoice{p.big, p.slices, p.kb_slice};
  // 256x256 tiles (4 waves of 128x128, one workgroup per CU) when there are
  // at least half as many as CUs; otherwise 128x128 tiles (4 waves of 64x64,
  // two workgroups per CU), which keep more CUs busy (measured on the
  // projection sweep: M=1024, N=4096 runs 2x faster on 128x128 tiles,
  // N=14336 (224 big tiles) runs faster on 256x256).
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  return MfmaChoice{tiles256 >= cus / 2, 1, kb};
}

// Bytes of K per row per pipeline stage of the library's own unsplit
// 128x128 launch: 128 when its grid is at most one workgroup per CU, else
// 64 (two workgroups per CU fit in LDS).
inline int stage_bytes_128(const GemmShape& g, int cus) {
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  return tiles <= cus ? 128 : 64;
}

// ---------------------------------------------------------------------------
// Small-M kernel (M <= kSkinnyMaxM, bf16/f16, A [M, K], B [N, K]): TM x TN
// 16x16 atoms per workgroup (4 waves), `slices` K slices of
// steps_per_slice 64-byte k-steps, and the f32 workspace the slices'
// partial tiles need (0 without split-K).
// ---------------------------------------------------------------------------
inline bool skinny_supported(const GemmShape& g) {
  const bool type_ok = (g.in == kBF16 && (g.out == kBF16 || g.out == kF32)) ||
                       (g.in == kF16 && (g.out == kF16 || g.out == kF32));
  return type_ok && g.m <= kSkinnyMaxM && !g.trans_a && g.trans_b;
}

struct SkinnyPlan {
  int tm, tn, slices, steps_per_slice;
  int64_t workspace_bytes;
};

inline SkinnyPlan skinny_plan(const GemmShape& g, int cus, bool split) {
  SkinnyPlan p;
  p.tm = g.m <= 16 ? 1 : g.m <= 32 ? 2 : g.m <= 64 ? 4 : 8;
  p.tn = g.n >= 8192 ? 2 : 1;  // 32-column tiles once N alone gives >= 256 of them
  const int64_t kb = g.k * 2;   // bf16 / f16
  const int64_t steps = (kb + 63) / 64;
  p.steps_per_slice = (int)steps;
  p.slices = 1;
  p.workspace_bytes = 0;
  // Below 64 MiB of W the unsplit kernel ends before a second launch pays
  // (16 x 4096 x 4096: 10.5 us unsplit, 12.7 us split).
  // (The slice sum reads rows of 4 floats, so N % 4 != 0 runs unsplit too.)
  if (!split || g.n * kb < ((int64_t)64 << 20) || g.n % 4 != 0) {
    // 32 < M <= 64 with under 64 MiB of W: 32x32 tiles instead of 64x16,
    // the same workgroup count with a fifth fewer operand loads per k-step
    // (64 x 4096 x 4096, operands from HBM: 24.1 -> 19.6 us).
    if (g.n * kb < ((int64_t)64 << 20) && p.tm == 4 && p.tn == 1) p.tm = p.tn = 2;
    return p;
  }
  // Split-K with wider column tiles when the unsplit grid would stream X
  // from L2 many times over: 64 columns per tile (32 at TM = 8, for
  // registers); slices until the grid has one workgroup per CU (with the
  // double-buffered batches, measured 4-9% faster than two per CU on most
  // projection shapes, and 30% faster than four), each slice at least
  // 4 waves x U k-steps, the f32 partials at most a quarter of the bytes of
  // W (S.M.N.4 <= N.K.2 / 4).
  const int tn = p.tm <= 4 ? 4 : 2;
  const int64_t tiles = ((g.n + 16 * tn - 1) / (16 * tn)) * ((g.m + 16 * p.tm - 1) / (16 * p.tm));
  // Wide tiles that alone fill most CUs in one round need no split: the
  // second launch would cost more than the idle CUs (16 x 14336 x 4096:
  // 224 tiles, 28.8 us unsplit against 31.6 us in two slices; 64 x 14336 x
  // 4096: 43.2 against 49.9 us).
  if (tiles * 20 >= (int64_t)cus * 17 && tiles <= cus) {
    p.tn = tn;
    return p;
  }
  // One 16-row block whose unsplit tiles (16 or 32 columns) fill the CUs in
  // whole rounds, with at most 128 MiB of W: no partials and no second
  // launch.  Operands from HBM, us, split -> unsplit: 16x4096x14336 30.8 ->
  // 29.4, 8x4096x14336 29.6 -> 25.0, 1x4096x14336 28.3 -> 22.6, 16x4096x8192
  // 19.7 -> 17.5, 16x8192x8192 31.2 -> 29.3; with more W the split stays
  // ahead (16x8192x14336 53.0 against 54.7, 16x4096x28672 54.9 against
  // 56.0), and so it does when the tiles leave a partial round (16x5120x14336
  // 49.4 against 53.4, 16x2048x16384 20.7 against 31.0).
  if (p.tm == 1 && cus > 0 && g.n * kb <= ((int64_t)128 << 20) &&
      ((g.n + 16 * p.tn - 1) / (16 * p.tn)) % cus == 0)
    return p;
  const int64_t min_steps = 4 * (p.tm + tn <= 10 ? 4 : 2);
  int64_t slices = ((int64_t)cus + tiles - 1) / tiles;
  slices = std::min<int64_t>(slices, steps / min_steps);
  slices = std::min<int64_t>(slices, kb / (16 * g.m));
  slices = std::min<int64_t>(slices, 64);
  if (slices >= 2) {
    p.tn = tn;
    p.steps_per_slice = (int)((steps + slices - 1) / slices);
    p.slices = (int)((steps + p.steps_per_slice - 1) / p.steps_per_slice);
    p.workspace_bytes = (int64_t)p.slices * g.m * g.n * 4;
  }
  return p;
}

// ---------------------------------------------------------------------------
// Kernel family and the whole launch.
// ---------------------------------------------------------------------------
enum class Route { Skinny, Mfma, Generic };

// `matrix_cores`: the operands meet the MFMA kernels' conditions (16-byte
// aligned bases and pitches, whole 16-byte pieces of K in a K-contiguous
// operand, buffer reach below 2^31 bytes), checked by the C-ABI.
inline Route route_of(const GemmShape& g, bool matrix_cores) {
  if (!matrix_cores) return Route::Generic;
  if (g.tile) return Route::Mfma;
  return skinny_supported(g) ? Route::Skinny : Route::Mfma;
}

// Workspace bytes of the split the launch follows (0: none).
inline int64_t workspace_bytes(const GemmShape& g, Route r, int cus) {
  if (r == Route::Skinny) {
    if (g.m > kSkinnySplitMaxM) return split_plan(g, cus).workspace_bytes;
    return skinny_plan(g, cus, true).workspace_bytes;
  }
  if (r == Route::Mfma) return g.tile ? requested_split(g, cus).workspace_bytes
                                      : split_plan(g, cus).workspace_bytes;
  return 0;
}

enum class Kernel { Generic, Skinny, W4, T128 };
enum class SliceSum { None, InLaunch, SecondLaunch };

// The launch a request makes: frisk_gemm_plan reports it; the IR's layout
// target gives it as the launch contract of a whole-matrix GEMM.
struct GemmLaunch {
  Kernel kernel;
  int tile_m, tile_n;
  int wave_m, wave_n;      // wave grid (MFMA kernels)
  int stage_bytes;         // K bytes per LDS stage (MFMA kernels)
  int slices;
  int64_t kb_slice;
  SliceSum slice_sum;
  int64_t workspace_bytes;  // of the split that runs (0: unsplit)
  bool requested;
};

// `workspace`: bytes the call provides (the split runs when it covers the
// plan's workspace_bytes).
inline GemmLaunch launch_of(const GemmShape& g, Route r, int cus, int64_t workspace) {
  GemmLaunch L{};
  const int64_t need = workspace_bytes(g, r, cus);
  const bool ws = need > 0 && workspace >= need;
  L.requested = g.tile != 0;
  if (r == Route::Generic) {
    L.kernel = Kernel::Generic;
    L.tile_m = L.tile_n = 64;
    L.slices = 1;
    L.kb_slice = g.k * dtype_bytes(g.in);
    return L;
  }
  if (r == Route::Skinny && !(ws && g.m > kSkinnySplitMaxM)) {
    const SkinnyPlan p = skinny_plan(g, cus, ws);
    L.kernel = Kernel::Skinny;
    L.tile_m = 16 * p.tm;
    L.tile_n = 16 * p.tn;
    L.wave_m = L.wave_n = 1;
    L.stage_bytes = 64;
    L.slices = p.slices;
    L.kb_slice = (int64_t)p.steps_per_slice * 64;
    L.slice_sum = p.slices > 1 ? SliceSum::SecondLaunch : SliceSum::None;
    L.workspace_bytes = p.slices > 1 ? p.workspace_bytes : 0;
    return L;
  }
  const MfmaChoice c = mfma_choice(g, cus, ws);
  L.kernel = c.big ? Kernel::W4 : Kernel::T128;
  L.tile_m = L.tile_n = c.big ? 256 : 128;
  L.wave_m = c.big || !g.tile ? 2 : (g.wave_m ? g.wave_m : 2);
  L.wave_n = c.big || !g.tile ? 2 : (g.wave_n ? g.wave_n : 2);
  const int64_t tiles128 = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  // The 2x2 grid runs the library's own stage depth whether requested or
  // not (both depths sum K in the same order); the other grids take 64-byte
  // stages.
  L.stage_bytes = c.big ? 128
                  : c.slices > 1 ? (tiles128 * c.slices <= cus && c.kb_slice % 128 == 0 ? 128 : 64)
                  : g.tile && !(L.wave_m == 2 && L.wave_n == 2) ? 64
                                                                 : stage_bytes_128(g, cus);
  L.slices = c.slices;
  L.kb_slice = c.kb_slice;
  L.slice_sum = c.slices <= 1 ? SliceSum::None
                : !c.big && c.slices <= kTreeMaxSlices ? SliceSum::InLaunch
                                                       : SliceSum::SecondLaunch;
  L.workspace_bytes = c.slices > 1 ? need : 0;
  return L;
}

// The LDS swizzle of an operand's stage tile in the MFMA kernels
// (gemm_tile.h OpTile::swz), in the layout target's notation: chunk c of
// row r is stored at the given chunk.  K-major rows hold stage_bytes of K
// and take the target's own proposals (proposeLdsSwizzle); M/N-major k-rows
// of row_bytes are read by transposing (or, 32-bit, four single-dword)
// reads, which the proposer does not model.
inline const char* lds_swizzle(bool mn_major, int esize, int stage_bytes, int row_bytes) {
  if (!mn_major) return stage_bytes == 128 ? "c ^ ((r >> 1) & 7)" : "c ^ ((r >> 2) & 3)";
  if (esize == 4) return "c ^ (((r >> 2) & 1) << 3)";
  if (esize == 2) return "c ^ ((r & 3) << 2)";
  return row_bytes >= 256 ? "c ^ ((r & 7) << 1)" : "c ^ (((r >> 1) & 3) << 1)";
}

// ---------------------------------------------------------------------------
// Attention workgroup shape: 8 waves x 32 queries (one K/V tile feeds 256
// queries) unless 4 waves finish sooner.  A CU runs one 8-wave workgroup or
// two 4-wave ones at a time (two waves per SIMD), so in units of one 8-wave
// workgroup's run: 8 waves take ceil(w8 / CUs); 4 waves take one unit per
// 2 CUs workgroups, and a last round of at most one workgroup per CU about
// 0.6 (one wave per SIMD runs each wave faster).  Measured non-causal:
// b4 h32 s4096 d128 1030 vs 1012 TFLOP/s (8 kept); b8 h8 s1024 d64 657 vs
// 635 (8 kept); b2 h32 s1025 d64 366 vs 475 and b1 h16 s2048 d128 618 vs
// 839 (4 chosen).  Causal b4 h32 s4096 d128 (workgroups of paired query
// blocks): 979-989 vs 944 (8 kept).  Below head_dim 128 the kernel takes
// about 150 VGPRs, three waves per SIMD, so 4-wave workgroups share a CU
// three at a time and the rule above undercounts them: measured (us, 4 vs
// 8 waves) b2 h32 s1025 d64 33.9 vs 45.8 (causal 34.2 vs 37.6), b4 h32
// s4096 d64 617 vs 630 (causal 336 vs 348), b8 h8 s1024 d64 causal 22.6
// vs 33.4, ties elsewhere; only s256 causal favoured 8 (11.6 vs 12.8).
// Head_dim 64 and below always take 4 waves.  Both shapes give every query
// the same arithmetic, so the choice changes no result bit.
// ---------------------------------------------------------------------------
inline int attn_waves(int64_t batch_heads, int64_t seq_q, int64_t head_dim, bool causal, int cus) {
  if (head_dim <= 64) return 4;
  auto workgroups = [&](int64_t bm) {
    const int64_t q = (seq_q + bm - 1) / bm;
    return batch_heads * (causal ? (q + 1) / 2 : q);
  };
  const int64_t w8 = workgroups(256), w4 = workgroups(128);
  const double t8 = (double)((w8 + cus - 1) / cus);
  const int64_t rest4 = w4 % (2 * (int64_t)cus);
  const double t4 = (double)(w4 / (2 * (int64_t)cus)) + (rest4 == 0 ? 0.0 : rest4 <= cus ? 0.6 : 1.0);
  return t4 < t8 ? 4 : 8;
}

}  // namespace plan
}  // namespace frisk
