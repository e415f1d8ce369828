// GEMM dispatch for gfx950 (MI355X): the generic fallback kernel, the
// split-K planner and the choice between the LDS-staged MFMA kernels
// (gemm_w4.h: 256x256 tiles; gemm_128.h: 128x128 tiles), both of which take
// every storage order of A and B.
//
// Semantics follow frisk.gemm (include/Dialect/Frisk/IR/FriskOps.td:252-292):
// C = op(A).op(B) when clear_accum, else C += op(A).op(B).
//
#include <algorithm>

#include "common.h"

#include "gemm_common.h"
#include "kernels.h"

namespace frisk {

// ---------------------------------------------------------------------------
// Generic kernel: any layout, any supported type, any shape.  64x64 output
// tile per 256 threads (4x4 per thread), K in steps of 16 through LDS with
// operands converted to the accumulator type on load.
// ---------------------------------------------------------------------------
template <Elt IN, Elt OUT>
__global__ __launch_bounds__(256) void gemm_generic(const void* __restrict__ A,
                                                    const void* __restrict__ B,
                                                    void* __restrict__ C, int M, int N, int K,
                                                    int64_t lda, int64_t ldb, int64_t ldc,
                                                    int trans_a, int trans_b, float scale,
                                                    int accumulate) {
  using Acc = typename std::conditional<IN == Elt::I8, int32_t, float>::type;
  __shared__ Acc as[16][65];
  __shared__ Acc bs[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
  Acc acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 64 * 16; e += 256) {
      const int kk = e & 15, rr = e >> 4;
      const int gm = row0 + rr, gn = col0 + rr, gk = k0 + kk;
      Acc va = 0, vb = 0;
      if (gm < M && gk < K) {
        const int64_t ia = trans_a ? (int64_t)gk * lda + gm : (int64_t)gm * lda + gk;
        if constexpr (IN == Elt::I8) va = ((const int8_t*)A)[ia];
        else va = load_as_f32<IN>(A, ia);
      }
      if (gn < N && gk < K) {
        const int64_t ib = trans_b ? (int64_t)gn * ldb + gk : (int64_t)gk * ldb + gn;
        if constexpr (IN == Elt::I8) vb = ((const int8_t*)B)[ib];
        else vb = load_as_f32<IN>(B, ib);
      }
      as[kk][rr] = va;
      bs[kk][rr] = vb;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      Acc a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = as[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gm = row0 + ty + 16 * i, gn = col0 + tx + 16 * j;
      if (gm >= M || gn >= N) continue;
      const int64_t ic = (int64_t)gm * ldc + gn;
      if constexpr (OUT == Elt::I32) {
        int32_t* p = (int32_t*)C + ic;
        *p = accumulate ? *p + acc[i][j] : acc[i][j];
      } else {
        float v = (float)acc[i][j] * scale;
        if (accumulate) v += load_as_f32<OUT>(C, ic);
        store_from_f32<OUT>(C, ic, v);
      }
    }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <Elt IN, Elt OUT>
static hipError_t launch_generic(const GemmArgs& g, hipStream_t stream) {
  dim3 grid((unsigned)((g.n + 63) / 64), (unsigned)((g.m + 63) / 64));
  hipLaunchKernelGGL((gemm_generic<IN, OUT>), grid, dim3(256), 0, stream, g.a, g.b, g.c,
                     (int)g.m, (int)g.n, (int)g.k, g.lda, g.ldb, g.ldc, g.trans_a, g.trans_b,
                     g.scale, g.accumulate);
  return hipGetLastError();
}

#define FRISK_PAIR(i, o) (((int)(i) << 8) | (int)(o))

// Time estimates (seconds) of the split choices, from rates measured on
// MI355X with operands streaming from HBM: a 128x128-tile workgroup
// computes about 2.5 TFLOP/s on its CU, a 256x256-tile one about 4.7; the
// f32 partials are written and read back at about 3.5 TB/s plus one launch.
namespace {
constexpr double kRate128 = 2.5e12, kRate256 = 4.7e12, kPartialBw = 3.5e12, kLaunch = 3e-6;
double rounds(int64_t wgs, int64_t slots) { return (double)((wgs + slots - 1) / slots); }
double partial_cost(const GemmArgs& g, int64_t slices) {
  return slices > 1 ? ((double)slices * g.m * g.n * 4 + (double)g.m * g.n * 2) / kPartialBw + kLaunch
                    : 0.0;
}
}  // namespace

// The f32 partials of a split (slices x M x N x 4 bytes) stay within
// 2 x (M + N) x K x 2 / FRISK_SPLIT_CAP bytes: the bytes of A and B.
// Measured with operands from HBM, us, a quarter of A + B (16) -> all of it
// (4): 256x4096x4096 27.4 -> 23.1 (2 -> 4 slices), 512x4096x4096 41.8 ->
// 28.5 (8 slices of 256x256 tiles -> 2 of 128x128); 128x4096x4096 19.3
// either way (4 -> 8 slices).
#ifndef FRISK_W4_SPLIT
#define FRISK_W4_SPLIT 1
#endif
#ifndef FRISK_SPLIT_CAP
#define FRISK_SPLIT_CAP 4
#endif
// Bytes of K per pipeline stage of the 128x128-tile kernel (gemm_128.h).
constexpr int64_t kRow = 64;

SplitPlan gemm_split_plan(const GemmArgs& g, int cus) {
  const int64_t kb = g.k * elt_bytes(g.in);  // bytes of K per row
  SplitPlan p{1, kb, 0, false};
  // bf16 / f16 / f32 only (the partials carry no fp8 scale, and int8 sums
  // stay exact in one pass); the slice sum reads rows of 4 floats.
  if ((g.in != Elt::BF16 && g.in != Elt::F16 && g.in != Elt::F32) || g.n % 4 != 0) return p;
  // Grids of at least CUs / 2 256x256 tiles run unsplit on them.
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  if (tiles256 >= cus / 2) return p;
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  // 128x128 tiles.  Split only grids that leave CUs without a tile, each
  // slice at least 8 stages, and the f32 partials at most the bytes of A
  // and B (FRISK_SPLIT_CAP).  Grids of at
  // most half as many tiles as CUs take slices up to one workgroup per CU,
  // on 128-byte stages (the launch picks them when slices fit one
  // workgroup per CU); larger grids take slices up to two workgroups per
  // CU on 64-byte stages.  Measured on the projection sweep: M = 128 runs
  // 1.6-4.8x faster than on the unsplit small-M kernel; with operands from
  // HBM, 128 x 4096 x 14336 323 -> 416 TFLOP/s and 128 x 14336 x 4096
  // 334 -> 373 on 128-byte stages (one workgroup per CU) against 64-byte
  // ones (two); M = 1024, N = 4096 (256 tiles) runs 1.3x slower split in
  // two.
  if (tiles < cus) {
    const bool deep = 2 * tiles <= cus;
    const int64_t row = deep ? 128 : kRow;  // bytes of K per stage
    int64_t slices = deep ? cus / tiles : (2 * (int64_t)cus + tiles - 1) / tiles;
    if (g.in == Elt::F32) {
      // fp32 runs the MFMA 16x slower per byte of operand than bf16: the
      // K loop, not the partials' traffic, sets the time, so slices of 4
      // stages and no cap on the partials (1024^3: 64 tiles in 4 slices).
      slices = std::min<int64_t>(slices, kb / (4 * row));
    } else {
      slices = std::min<int64_t>(slices, kb / (8 * row));
      slices = std::min<int64_t>(slices, (g.m + g.n) * kb / (FRISK_SPLIT_CAP * g.m * g.n));
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
  // 512 x 4096 x 4096 53.1 -> 44.1 us, 768 x 2048 x 4096 51.4 -> 38.1,
  // 1024 x 4096 x 14336 179.5 -> 133.3 (estimated ratios 0.66-0.69);
  // 1024 x 4096 x 4096 stays on 128x128 tiles (57.6 us split against 54.4)
  // and 256 x 4096 x 4096 on its 128x128 split (34.9 us on 256x256 tiles
  // against 33.2; estimated ratio 0.84).
  // (The rates are those of bf16 / f16; f32 keeps the 128x128 split.)
  if (g.m > kSkinnyMaxM && FRISK_W4_SPLIT && g.in != Elt::F32) {
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

MfmaChoice gemm_mfma_choice(const GemmArgs& g, int cus, bool workspace) {
  // A requested variant runs unsplit on the tile it names.
  if (g.tile) return MfmaChoice{g.tile == 256, 1, g.k * elt_bytes(g.in)};
  const SplitPlan p = gemm_split_plan(g, cus);
  if (workspace && p.slices > 1) return MfmaChoice{p.big, p.slices, p.kb_slice};
  // 256x256 tiles (4 waves of 128x128, one workgroup per CU) when there are
  // at least half as many as CUs; otherwise 128x128 tiles (4 waves of 64x64,
  // two workgroups per CU), which keep more CUs busy (measured on the
  // projection sweep: M=1024, N=4096 runs 2x faster on 128x128 tiles,
  // N=14336 (224 big tiles) runs faster on 256x256).
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  return MfmaChoice{tiles256 >= cus / 2, 1, g.k * elt_bytes(g.in)};
}

namespace {

// One storage order: AM = A stored [K, M] (trans_a), BM = B stored [K, N]
// (not trans_b).
template <bool AM, bool BM>
hipError_t run_layout(const GemmArgs& g, hipStream_t s, const MfmaChoice& c, void* ws) {
  if (c.slices > 1) {
    if (c.big) return gemm_w4_split_layout<AM, BM>(g, c.slices, c.kb_slice, ws, s);
    return gemm_128_split_layout<AM, BM>(g, c.slices, c.kb_slice, ws, s);
  }
  if (c.big) return gemm_w4_layout<AM, BM>(g, s);
  if (g.tile == 128) return gemm_128_grid_layout<AM, BM>(g, s);
  return gemm_128_layout<AM, BM>(g, s);
}

}  // namespace

hipError_t gemm_mfma(const GemmArgs& g, hipStream_t s, void* workspace, int64_t workspace_bytes) {
  const int cus = device_cus();
  const bool ws = !g.tile && workspace && workspace_bytes >= gemm_split_plan(g, cus).workspace_bytes;
  const MfmaChoice c = gemm_mfma_choice(g, cus, ws);
  void* tree_ws = c.slices > 1 ? workspace : nullptr;
  switch ((g.trans_a ? 2 : 0) | (g.trans_b ? 0 : 1)) {
    case 0: return run_layout<false, false>(g, s, c, tree_ws);  // A [M,K], B [N,K]
    case 1: return run_layout<false, true>(g, s, c, tree_ws);   // A [M,K], B [K,N]
    case 2: return run_layout<true, false>(g, s, c, tree_ws);   // A [K,M], B [N,K]
    default: return run_layout<true, true>(g, s, c, tree_ws);   // A [K,M], B [K,N]
  }
}

hipError_t gemm_generic_any(const GemmArgs& g, hipStream_t s) {
  switch (FRISK_PAIR(g.in, g.out)) {
    case FRISK_PAIR(Elt::F32, Elt::F32): return launch_generic<Elt::F32, Elt::F32>(g, s);
    case FRISK_PAIR(Elt::BF16, Elt::BF16): return launch_generic<Elt::BF16, Elt::BF16>(g, s);
    case FRISK_PAIR(Elt::BF16, Elt::F32): return launch_generic<Elt::BF16, Elt::F32>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F16): return launch_generic<Elt::F16, Elt::F16>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F32): return launch_generic<Elt::F16, Elt::F32>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::BF16): return launch_generic<Elt::E4M3, Elt::BF16>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F16): return launch_generic<Elt::E4M3, Elt::F16>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F32): return launch_generic<Elt::E4M3, Elt::F32>(g, s);
    case FRISK_PAIR(Elt::I8, Elt::I32): return launch_generic<Elt::I8, Elt::I32>(g, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace frisk
