// GEMM dispatch for gfx950 (MI355X): the generic fallback kernel and the
// launch of the LDS-staged MFMA kernels (gemm_w4.h: 256x256 tiles;
// gemm_128.h: 128x128 tiles), both of which take every storage order of A
// and B, as the launch planner (launch_plan.h) decides.
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
  // A requested 2x2 grid runs as the library's own 128x128 launch (its
  // stage depth); the other grids run 64-byte stages.
  if (g.tile == 128 && !(g.wave_m == 2 && g.wave_n == 2)) return gemm_128_grid_layout<AM, BM>(g, s);
  return gemm_128_layout<AM, BM>(g, s);
}

}  // namespace

// The launch follows plan::mfma_choice (launch_plan.h): the library's own
// choice, or the requested variant with the K slices it names.
hipError_t gemm_mfma(const GemmArgs& g, hipStream_t s, void* workspace, int64_t workspace_bytes) {
  const int cus = device_cus();
  const int64_t need = plan::workspace_bytes(shape_of(g), plan::Route::Mfma, cus);
  const bool ws = workspace && need > 0 && workspace_bytes >= need;
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
