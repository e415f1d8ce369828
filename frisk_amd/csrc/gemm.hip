// MFMA GEMM kernels for gfx950 (MI355X): the 128x128-tile kernel, the
// generic fallback and the launch policy.  The 256x256-tile kernel lives in
// gemm4w.hip.
//
// Semantics follow frisk.gemm (include/Dialect/Frisk/IR/FriskOps.td:252-292):
// C = op(A).op(B) when clear_accum, else C += op(A).op(B).  The reference
// lowers one 64xN tile of that op to SM90 wgmma text
// (benchmark/layout/execution/backend.py:383-431); here the whole problem is
// tiled for CDNA4:
//
//  * 128x128 output tile per 256-thread workgroup (4 waves, 2x2), each wave
//    owning a 64x64 sub-tile as 2x2 v_mfma 32x32 accumulators; two
//    workgroups share a CU.
//  * K is consumed in stages of 64 bytes per row (32 bf16/f16, 64 fp8/i8),
//    loaded by LDS-DMA (buffer_load_dwordx4 ... lds: no VGPRs stage the
//    data) into kStages rotating LDS slots, one barrier per stage.
//  * LDS rows are 4 chunks of 16 B, chunk c of row r stored at chunk
//    c ^ swz(r); the XOR spreads the 32 rows of a fragment read over distinct
//    bank groups.  swz is an F2-linear map of the row bits (a GF(2) layout in
//    the sense of the reference's bit-linear shared layouts,
//    SM90GemmConstraints.cpp:106-150).
//  * The epilogue stages each 32-row f32 slice of a wave through LDS so the
//    global stores are row-contiguous 16 B per lane.
//
// Operand contract of the fast kernel: A is [M, K] and B is [N, K] (both
// K-contiguous, i.e. trans_a == 0, trans_b == 1), K*esize % 16 == 0, 16 B
// aligned rows; the generic kernel covers every other layout and type.

#include <algorithm>

#include "common.h"

#include "gemm_common.h"
#include "kernels.h"

namespace frisk {

// ---------------------------------------------------------------------------
// Tiling.  Each stage holds 64 bytes of K per row (32 bf16/f16, 64 fp8/i8)
// for the BT A rows and BT B rows (2 x 8 KiB at BT = 128).  kStages rotate
// through LDS; a stage is filled by LDS-DMA (buffer_load_dwordx4 ... lds),
// so no VGPRs stage the data and the loads of kStages-2 stages are in
// flight while one stage is multiplied.
//
// LDS row = 4 chunks of 16 B.  Chunk c of row r is stored at physical chunk
// c ^ swz(r), swz(r) = (r >> 2) & 3.  A 32x32 MFMA fragment read has lanes
// 0-31 read one logical chunk of 32 consecutive rows (lanes 32-63 the next
// chunk).  gfx950 serves ds_read_b128 at 256 B/clk (64 banks of 4 B, 16
// lanes per cycle); under this map the 16 rows of a lane group cover the 16
// distinct 16 B bank groups of a 256 B line ((r & 3) picks the quarter,
// swz the chunk), and rocprofv3 counts SQ_LDS_BANK_CONFLICT = 0 for it,
// where ((r >> 1) ^ (r >> 3)) & 3 measured 2-way conflicts and no swizzle
// 4-way.  swz is linear over GF(2) in the row bits (a bit-linear shared
// layout); the DMA side applies it by choosing which chunk a lane fetches.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }

constexpr int kRow = 64;  // bytes of K per row per stage
#ifndef FRISK_GEMM_STAGES
#define FRISK_GEMM_STAGES 4
#endif
constexpr int kStages = FRISK_GEMM_STAGES;
// LDS bytes of a BT x BT tile pipeline: kStages stages of (A, B) tiles.
constexpr int lds_bytes(int bt) { return kStages * 2 * bt * kRow; }
static_assert(2 * lds_bytes(128) <= 160 * 1024, "two 128x128 workgroups per CU");

// One workgroup per BT x BT output tile; WM x WN waves tile it, each wave
// owning a (BT/WM) x (BT/WN) sub-tile as TM x TN 32x32 accumulators.
//
// Split-K: blockIdx.y is a K slice of kb_slice bytes; the slice's A and B
// columns start kb_slice * y bytes in, and its output is the tile of C
// c_slice_bytes * y bytes further (the f32 partial of that slice).
template <Elt IN, Elt OUT, int BT, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_tn(const char* __restrict__ A,
                                                             const char* __restrict__ B,
                                                             void* __restrict__ C, int M, int N,
                                                             int Kb, int64_t lda_b, int64_t ldb_b,
                                                             int64_t ldc, float scale,
                                                             int accumulate, int kb_slice,
                                                             int64_t c_slice_bytes) {
  // The body is device code only; the host pass just needs the kernel stub.
#if defined(__HIP_DEVICE_COMPILE__)
  A += (int64_t)blockIdx.y * kb_slice;
  B += (int64_t)blockIdx.y * kb_slice;
  Kb = min(Kb - (int)blockIdx.y * kb_slice, kb_slice);
  C = (char*)C + (int64_t)blockIdx.y * c_slice_bytes;
  using Op = Mfma32<IN>;
  using Acc = typename Op::Acc;
  using AccS = typename std::conditional<IN == Elt::I8, int32_t, float>::type;
  constexpr int kWaves = WM * WN;
  constexpr int kBM = BT, kBN = BT;
  constexpr int kTileBytes = BT * kRow;  // one operand, one stage
  constexpr int kStageBytes = 2 * kTileBytes;
  constexpr int kLdsBytes = lds_bytes(BT);
  constexpr int TM = kBM / WM / 32, TN = kBN / WN / 32;
  constexpr int kStepChunks = Op::kBytes / 16;  // 16 B chunks per row per MFMA
  constexpr int kLaneChunks = kStepChunks / 2;  // chunks per lane per MFMA
  constexpr int kSteps = kRow / Op::kBytes;     // MFMA k-steps per stage (2 or 1)
  constexpr int kBlocks = kTileBytes / 1024 / kWaves;  // 1 KiB DMA blocks per wave per operand
  constexpr int kLoads = 2 * kBlocks;                  // DMA loads per lane per stage
  constexpr int kFragReads = (TM + TN) * kLaneChunks;  // ds_read_b128 per lane per k-step

  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, half = lane >> 5;

  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of_block<4>(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int row0 = tm * kBM, col0 = tn * kBN;

  // ---- LDS-DMA mapping ----------------------------------------------------
  // DMA instruction i of wave w writes the 1 KiB block of rows
  // (kBlocks w + i) * 16 .. +16 of a tile; lane L lands at row +L/4,
  // physical chunk L%4, so it fetches logical chunk (L%4) ^ swz(row) of that
  // row.  Loads are raw buffer loads based at the tile's first row: an
  // offset past num_records returns zeros, which zero-fills the K tail
  // without branches.
  const char* a_base = A + (int64_t)row0 * lda_b;
  const char* b_base = B + (int64_t)col0 * ldb_b;
  const int64_t a_left = (int64_t)(M - 1 - row0) * lda_b + Kb;
  const int64_t b_left = (int64_t)(N - 1 - col0) * ldb_b + Kb;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a_base, (short)0, (int)min(a_left, (int64_t)0x7fffffff), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)b_base, (short)0, (int)min(b_left, (int64_t)0x7fffffff), 0x00020000);
  uint32_t a_off[kBlocks], b_off[kBlocks];
  int kmax[kBlocks];
#pragma unroll
  for (int i = 0; i < kBlocks; ++i) {
    const int r = (kBlocks * wave + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ swz(r);
    // Rows past the matrix edge are clamped: they only feed output rows or
    // columns that are never stored.
    a_off[i] = (uint32_t)(min(r, M - 1 - row0) * lda_b) + c * 16;
    b_off[i] = (uint32_t)(min(r, N - 1 - col0) * ldb_b) + c * 16;
    kmax[i] = Kb - c * 16;  // the chunk is live while kb < kmax
  }
  auto issue_stage = [&](int stage, int slot) {
    const int kb = stage * kRow;
    char* dst = smem + slot * kStageBytes + wave * kBlocks * 1024;
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      const bool live = kb < kmax[i];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr_t)(dst + i * 1024), 16,
                                               live ? a_off[i] + kb : 0x80000000u, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_ptr_t)(dst + kTileBytes + i * 1024), 16,
                                               live ? b_off[i] + kb : 0x80000000u, 0, 0, 0);
    }
  };

  // ---- fragment reads -----------------------------------------------------
  int fa_off[TM], fb_off[TN], fa_sw[TM], fb_sw[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int r = wm * (32 * TM) + t * 32 + l32;
    fa_off[t] = r * kRow;
    fa_sw[t] = swz(r);
  }
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int r = wn * (32 * TN) + t * 32 + l32;
    fb_off[t] = kTileBytes + r * kRow;
    fb_sw[t] = swz(r);
  }
  using Frag = Frags<TM, TN, kLaneChunks>;
  auto load_frags = [&](int slot, int s, Frag& f) {
    const char* base = smem + slot * kStageBytes;
#pragma unroll
    for (int j = 0; j < kLaneChunks; ++j) {
      const int chunk = s * kStepChunks + half * kLaneChunks + j;
#pragma unroll
      for (int t = 0; t < TM; ++t)
        f.a[t][j] = *(const i32x4*)(base + fa_off[t] + ((chunk ^ fa_sw[t]) << 4));
#pragma unroll
      for (int t = 0; t < TN; ++t)
        f.b[t][j] = *(const i32x4*)(base + fb_off[t] + ((chunk ^ fb_sw[t]) << 4));
    }
  };

  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{};
  auto mfma_rows = [&](const Frag& f, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = Op::run(f.a[i], f.b[j], acc[i][j]);
  };

  // ---- pipeline -----------------------------------------------------------
  // Stage kt lives in slot kt % kStages.  Before the second half of the last
  // k-step of stage kt a barrier (after waiting for this lane's loads of
  // stage kt+1) makes stage kt+1 readable and proves every wave is done
  // with slot (kt-1) % kStages, which then receives stage kt+kStages-1.
  // Every iteration issues exactly kLoads loads (stages past the end reload
  // the last stage into a slot nobody reads), so vmcnt bookkeeping is static.
  const int nk = (Kb + kRow - 1) / kRow;
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) issue_stage(min(st, nk - 1), st);
  FRISK_WAIT_VMCNT(kLoads * (kStages - 2));
  __builtin_amdgcn_s_barrier();

  Frag fr[2];
  load_frags(0, 0, fr[0]);
  // Drain every LGKM operation issued so far (the prologue's fragment reads
  // and the scalar loads of the epilogue's kernel arguments).  With scalar
  // loads still pending at the loop entry the LGKM counter is unordered, and
  // the compiler then waits for lgkmcnt(0) at the top of every iteration,
  // i.e. for the fragment read it has just issued.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  int slot = 0;
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < kSteps) {
        load_frags(slot, s + 1, fr[nxt]);
        mfma_rows(fr[cur], 0, TM);
        // Fragment reads first, each under one MFMA.
#pragma unroll
        for (int i = 0; i < kFragReads; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
        __builtin_amdgcn_sched_barrier(0);
      } else {
        mfma_rows(fr[cur], 0, TM / 2);
        __builtin_amdgcn_sched_barrier(0);
        FRISK_WAIT_VMCNT(kLoads * (kStages - 3));
        __builtin_amdgcn_s_barrier();
        const int nslot = slot + 1 == kStages ? 0 : slot + 1;
        const int fslot = slot == 0 ? kStages - 1 : slot - 1;
        issue_stage(min(kt + kStages - 1, nk - 1), fslot);
        load_frags(nslot, 0, fr[kSteps & 1 ? nxt : 0]);
        mfma_rows(fr[cur], TM / 2, TM);
        // DMA issue and next-stage fragment reads interleaved with the
        // remaining MFMAs.
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (LDS-DMA)
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
        __builtin_amdgcn_sched_barrier(0);
        slot = nslot;
      }
    }
    if constexpr (kSteps == 1) fr[0] = fr[1];
  }
  // Drain the trailing DMA loads before the stage buffers are reused.
  FRISK_WAIT_VMCNT(0);
  __syncthreads();

  // Epilogue: per wave, stage a 32 x (32 TN) slice (one accumulator row
  // block) as 32-bit values, then each lane stores 8 consecutive columns.
  // The MFMA 32x32 accumulator holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32]
  // in element r.
  constexpr int kPitch = 32 * TN + 4;
  static_assert(kWaves * 32 * kPitch * 4 <= kLdsBytes, "epilogue staging fits in the stage buffers");
  AccS* stage = (AccS*)(smem + wave * (32 * kPitch * 4));
  constexpr int kGroups = 32 * TN / 8;  // 8-column groups per staged row
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = 8 * (r >> 2) + 4 * half + (r & 3);
        stage[rr * kPitch + j * 32 + l32] = acc[i][j][r];
      }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 32 * kGroups / 64; ++it) {
      const int q = it * 64 + lane;
      const int rr = q / kGroups, g = q % kGroups;
      const int gr = row0 + wm * (32 * TM) + i * 32 + rr;
      const int gc = col0 + wn * (32 * TN) + g * 8;
      if (gr < M && gc < N) {
        AccS v[8];
        *(i32x4*)&v[0] = *(const i32x4*)&stage[rr * kPitch + g * 8];
        *(i32x4*)&v[4] = *(const i32x4*)&stage[rr * kPitch + g * 8 + 4];
        store8<OUT>(C, (int64_t)gr * ldc + gc, v, accumulate != 0, scale);
      }
    }
    __syncthreads();
  }
#endif  // __HIP_DEVICE_COMPILE__
}

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
template <Elt IN, Elt OUT, int BT, int WM, int WN>
static hipError_t launch_tn_cfg(const GemmArgs& g, hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = lds_bytes(BT);
  auto kern = gemm_mfma_tn<IN, OUT, BT, WM, WN>;
  // Thread-safe one-time opt-in to more than 64 KiB of dynamic LDS.
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + BT - 1) / BT) * ((g.n + BT - 1) / BT));
  const int kb = (int)(g.k * kEsz);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), kLds, stream, (const char*)g.a,
                     (const char*)g.b, g.c, (int)g.m, (int)g.n, kb, g.lda * kEsz, g.ldb * kEsz,
                     g.ldc, g.scale, g.accumulate, kb, (int64_t)0);
  return hipGetLastError();
}

// Split-K on 128x128 tiles: f32 partial tiles of each K slice into
// `partial` ([slices][M][N]), then their sum in slice order into C.
template <Elt IN, Elt OUT>
static hipError_t launch_tn_split(const GemmArgs& g, const TnSplitPlan& p, float* partial,
                                  hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = lds_bytes(128);
  auto kern = gemm_mfma_tn<IN, Elt::F32, 128, 2, 2>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + 127) / 128) * ((g.n + 127) / 128));
  hipLaunchKernelGGL(kern, dim3(tiles, p.slices), dim3(256), kLds, stream, (const char*)g.a,
                     (const char*)g.b, (void*)partial, (int)g.m, (int)g.n, (int)(g.k * kEsz),
                     g.lda * kEsz, g.ldb * kEsz, g.n, 1.0f, 0, (int)p.kb_slice,
                     (int64_t)g.m * g.n * 4);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return gemm_splitk_sum(partial, p.slices, g, stream);
}

// 256x256 tiles (gemm4w.hip: 4 waves of 128x128, one workgroup per CU)
// when there are at least half as many as CUs; otherwise 128x128 tiles
// (4 waves of 64x64, two workgroups per CU), which keep more CUs busy
// (measured on the projection sweep: M=1024, N=4096 runs 2x faster on
// 128x128 tiles, N=14336 (224 big tiles) runs faster on 256x256).
template <Elt IN, Elt OUT>
static hipError_t launch_tn(const GemmArgs& g, hipStream_t stream, int cus, float* partial,
                            const TnSplitPlan& p) {
  if constexpr (IN == Elt::BF16 || IN == Elt::F16) {
    if (partial && p.big) return gemm_tn_w4_split(g, p.slices, p.kb_slice, partial, stream);
    if (partial) return launch_tn_split<IN, OUT>(g, p, partial, stream);
  }
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  if (tiles256 >= cus / 2) return gemm_tn_w4(g, stream);
  return launch_tn_cfg<IN, OUT, 128, 2, 2>(g, stream);
}

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

TnSplitPlan gemm_tn_split_plan(const GemmArgs& g, int cus) {
  TnSplitPlan p{1, g.k * 2, 0, false};
  if ((g.in != Elt::BF16 && g.in != Elt::F16) || g.trans_a || !g.trans_b) return p;
  // Grids of at least CUs / 2 256x256 tiles run unsplit on them.
  const int64_t tiles256 = ((g.m + 255) / 256) * ((g.n + 255) / 256);
  if (tiles256 >= cus / 2) return p;
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  const int64_t kb = g.k * 2;
  // 128x128 tiles.  Split only grids that leave CUs without a tile: slices
  // until two workgroups per CU, each slice at least 8 stages (8 x 64 B of
  // K), and the f32 partials at most a quarter of the bytes of A and B
  // (their second pass then costs little).  Measured on the projection
  // sweep: M = 128 runs 1.6-4.8x faster than on the unsplit small-M kernel
  // (17.0 us at N = K = 4096 with 4 slices, against 24.0 with 16); M = 1024,
  // N = 4096 (256 tiles) runs 1.3x slower split in two.
  if (tiles < cus) {
    int64_t slices = (2 * (int64_t)cus + tiles - 1) / tiles;
    slices = std::min<int64_t>(slices, kb / (8 * kRow));
    slices = std::min<int64_t>(slices, (g.m + g.n) * kb / (16 * g.m * g.n));
    slices = std::min<int64_t>(slices, 64);
    if (slices >= 2) {
      const int64_t chunks = (kb + kRow - 1) / kRow;  // slices start on stage boundaries
      p.kb_slice = ((chunks + slices - 1) / slices) * kRow;
      p.slices = (int)((kb + p.kb_slice - 1) / p.kb_slice);
      if (p.slices < 2) p = TnSplitPlan{1, kb, 0, false};
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
  if (g.m > kSkinnyMaxM) {
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
      if (!p.big) p = TnSplitPlan{1, kb, 0, false};
    }
  }
  p.workspace_bytes = p.slices > 1 ? (int64_t)p.slices * g.m * g.n * 4 : 0;
  return p;
}

hipError_t gemm_tn_mfma(const GemmArgs& g, hipStream_t s, void* workspace,
                        int64_t workspace_bytes) {
  const int cus = device_cus();
  TnSplitPlan p = gemm_tn_split_plan(g, cus);
  float* partial = p.slices > 1 && workspace && workspace_bytes >= p.workspace_bytes
                       ? (float*)workspace : nullptr;
  switch (FRISK_PAIR(g.in, g.out)) {
    case FRISK_PAIR(Elt::BF16, Elt::BF16): return launch_tn<Elt::BF16, Elt::BF16>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::BF16, Elt::F32): return launch_tn<Elt::BF16, Elt::F32>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::F16, Elt::F16): return launch_tn<Elt::F16, Elt::F16>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::F16, Elt::F32): return launch_tn<Elt::F16, Elt::F32>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::E4M3, Elt::BF16): return launch_tn<Elt::E4M3, Elt::BF16>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::E4M3, Elt::F16): return launch_tn<Elt::E4M3, Elt::F16>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::E4M3, Elt::F32): return launch_tn<Elt::E4M3, Elt::F32>(g, s, cus, partial, p);
    case FRISK_PAIR(Elt::I8, Elt::I32): return launch_tn<Elt::I8, Elt::I32>(g, s, cus, partial, p);
    default: return hipErrorInvalidValue;
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
