// 128x128-tile MFMA GEMM for gfx950 (MI355X): the kernel for grids too small
// for the 256x256 tiles of gemm_w4.h, and the split-K slices of medium M.
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
//  * K is consumed in stages of KROW bytes per row, loaded by LDS-DMA
//    (buffer_load_dwordx4 ... lds: no VGPRs stage the data) into kStages
//    rotating LDS slots, one barrier per stage.  KROW = 64 (32 bf16/f16,
//    64 fp8/i8; 64 KiB of LDS, two workgroups per CU) or 128 (one whole
//    128-byte line per row segment, 128 KiB, one workgroup per CU).  A row
//    segment of 64 bytes is half a cache line, whose other half the next
//    stage fetches again; with operands streamed from HBM that costs the
//    single-workgroup grids most (1024 x 4096 x 4096 bf16, operands not in
//    any cache: 668 -> 846 TFLOP/s with 128-byte stages).
//  * Operand tiles, their XOR swizzles and the fragment reads for either
//    storage order of A and B (template flags AM / BM, MN-major when set)
//    are those of gemm_tile.h.  For the K-major 64 B rows the swizzle is
//    swz(r) = (r >> 2) & 3: a 32x32 fragment read has lanes 0-31 read one
//    logical chunk of 32 consecutive rows; the 16 rows of a 16-lane cycle
//    then cover the 16 distinct 16 B bank groups of a 256 B line, and
//    rocprofv3 counts SQ_LDS_BANK_CONFLICT = 0 for it, where
//    ((r >> 1) ^ (r >> 3)) & 3 measured 2-way conflicts and no swizzle 4-way.
//  * The epilogue stages each 32-row f32 slice of a wave through LDS so the
//    global stores are row-contiguous 16 B per lane.
//
// gemm_128_a*b*.hip instantiate one layout each.
#pragma once

#include <algorithm>

#include "common.h"
#include "gemm_common.h"
#include "gemm_tile.h"
#include "kernels.h"

namespace frisk {

namespace g128 {

#ifndef FRISK_GEMM_STAGES
#define FRISK_GEMM_STAGES 4
#endif
constexpr int kStages = FRISK_GEMM_STAGES;
// LDS bytes of a BT x BT tile pipeline: kStages stages of (A, B) tiles of
// krow bytes of K per row.
constexpr int lds_bytes(int bt, int krow) { return kStages * 2 * bt * krow; }
// LDS bytes of one workgroup with a WM x WN wave grid: the pipeline, or the
// epilogue's staging (each wave 32 rows of 32 TN + 4 32-bit values) when
// that is larger (the 4x1 grid).
constexpr int lds_bytes_grid(int bt, int wm, int wn, int krow) {
  const int epi = wm * wn * 32 * (bt / wn + 4) * 4;
  return lds_bytes(bt, krow) > epi ? lds_bytes(bt, krow) : epi;
}
static_assert(2 * lds_bytes_grid(128, 4, 1, 64) <= 160 * 1024, "two 128x128 workgroups per CU");
static_assert(lds_bytes_grid(128, 4, 1, 128) <= 160 * 1024, "one 128x128 workgroup per CU");

}  // namespace g128

// One workgroup per BT x BT output tile; WM x WN waves tile it, each wave
// owning a (BT/WM) x (BT/WN) sub-tile as TM x TN 32x32 accumulators.
//
// Split-K: blockIdx.y is a K slice of kb_slice bytes; the slice's A and B
// start kb_slice bytes of K further per slice.  With TREE the slices of a
// tile sum through `tree` (splitk_tree, gemm_common.h) and the one holding
// the total writes C; otherwise a slice's output is the tile of C
// c_slice_bytes * y bytes further (the f32 partial of that slice).
template <Elt IN, Elt OUT, bool AM, bool BM, int BT, int WM, int WN, int KROW, bool TREE = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_128(const char* __restrict__ A,
                                                              const char* __restrict__ B,
                                                              void* __restrict__ C, int M, int N,
                                                              int Kb, int64_t lda_b, int64_t ldb_b,
                                                              int64_t ldc, float scale,
                                                              int accumulate, int kb_slice,
                                                              int64_t c_slice_bytes,
                                                              SplitTree tree) {
  // The body is device code only; the host pass just needs the kernel stub.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int kRow = KROW, kStages = g128::kStages;
  using TA = OpTile<IN, AM, BT, kRow>;
  using TB = OpTile<IN, BM, BT, kRow>;
  A += TA::slice_shift((int64_t)blockIdx.y * kb_slice, lda_b);
  B += TB::slice_shift((int64_t)blockIdx.y * kb_slice, ldb_b);
  Kb = min(Kb - (int)blockIdx.y * kb_slice, kb_slice);
  C = (char*)C + (int64_t)blockIdx.y * c_slice_bytes;
  using Op = Mfma32<IN>;
  using Acc = typename Op::Acc;
  using AccS = typename std::conditional<IN == Elt::I8, int32_t, float>::type;
  constexpr int kWaves = WM * WN;
  constexpr int kBM = BT, kBN = BT;
  constexpr int kTileBytes = BT * kRow;  // one operand, one stage
  constexpr int kStageBytes = 2 * kTileBytes;
  constexpr int kLdsBytes = g128::lds_bytes_grid(BT, WM, WN, KROW);
  constexpr int TM = kBM / WM / 32, TN = kBN / WN / 32;
  constexpr int kLaneChunks = TA::kLaneChunks;         // 16 B pieces per lane per MFMA
  constexpr int kSteps = kRow / Op::kBytes;            // MFMA k-steps per stage (1 to 4)
  constexpr int kBlocks = kTileBytes / 1024 / kWaves;  // 1 KiB DMA blocks per wave per operand
  constexpr int kLoads = 2 * kBlocks;                  // DMA loads per lane per stage
  constexpr int kFragReads =                           // LDS reads per lane per k-step
      (TM * TA::kReadsPerChunk + TN * TB::kReadsPerChunk) * kLaneChunks;

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

  // ---- LDS-DMA mapping (gemm_tile.h) --------------------------------------
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)TA::origin(A, row0, lda_b), (short)0,
      (int)min(TA::records(M, row0, Kb, lda_b), (int64_t)0x7fffffff), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)TB::origin(B, col0, ldb_b), (short)0,
      (int)min(TB::records(N, col0, Kb, ldb_b), (int64_t)0x7fffffff), 0x00020000);
  typename TA::template Dma<kBlocks> da;
  typename TB::template Dma<kBlocks> db;
#pragma unroll
  for (int i = 0; i < kBlocks; ++i) {
    TA::dma_setup(da, i, kBlocks * wave + i, lane, M, row0, Kb, lda_b);
    TB::dma_setup(db, i, kBlocks * wave + i, lane, N, col0, Kb, ldb_b);
  }
  TA::dma_adv(da, lda_b);
  TB::dma_adv(db, ldb_b);
  auto issue_stage = [&](int stage, int slot) {
    char* dst = smem + slot * kStageBytes + wave * kBlocks * 1024;
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr_t)(dst + i * 1024), 16,
                                               TA::offset(da, i, stage), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_ptr_t)(dst + kTileBytes + i * 1024), 16,
                                               TB::offset(db, i, stage), 0, 0, 0);
    }
  };

  // ---- fragment reads -----------------------------------------------------
  // K-major operands share one Frag (tile 0's) across their tiles.
  typename TA::Frag fa[TA::kSharedFrag ? 1 : TM];
  typename TB::Frag fb[TB::kSharedFrag ? 1 : TN];
#pragma unroll
  for (int t = 0; t < (TA::kSharedFrag ? 1 : TM); ++t) fa[t] = TA::frag(wm * (32 * TM) + t * 32, lane);
#pragma unroll
  for (int t = 0; t < (TB::kSharedFrag ? 1 : TN); ++t) fb[t] = TB::frag(wn * (32 * TN) + t * 32, lane);
  using Frag = Frags<TM, TN, kLaneChunks>;
  auto load_frags = [&](int slot, int s, Frag& f) {
    const char* base = smem + slot * kStageBytes;
#pragma unroll
    for (int t = 0; t < TM; ++t)
      TA::read(base, fa[TA::kSharedFrag ? 0 : t], s, f.a[t], TA::tile_off(t * 32));
#pragma unroll
    for (int t = 0; t < TN; ++t)
      TB::read(base + kTileBytes, fb[TB::kSharedFrag ? 0 : t], s, f.b[t], TB::tile_off(t * 32));
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
  // block) as 32-bit values, then each lane stores 8 consecutive columns
  // (the ragged last group of a row one element at a time).  The MFMA 32x32
  // accumulator holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] in element r.
  constexpr int kPitch = 32 * TN + 4;
  static_assert(kWaves * 32 * kPitch * 4 <= kLdsBytes, "epilogue staging fits in the stage buffers");
  // The split-K tree's LDS flag sits in the last 16 bytes, past the staging.
  static_assert(!TREE || kWaves * 32 * kPitch * 4 <= kLdsBytes - 16, "room for the tree's flag");
  if constexpr (TREE)
    if (!splitk_tree<kWaves>(acc, tree, blockIdx.x, blockIdx.y, (int*)(smem + kLdsBytes - 16)))
      return;
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
        if (gc + 8 <= N) store8<OUT>(C, (int64_t)gr * ldc + gc, v, accumulate != 0, scale);
        else store_n<OUT>(C, (int64_t)gr * ldc + gc, v, N - gc, accumulate != 0, scale);
      }
    }
    __syncthreads();
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <Elt IN, Elt OUT, bool AM, bool BM, int WM = 2, int WN = 2, int KROW = 64>
static hipError_t launch_128(const GemmArgs& g, hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g128::lds_bytes_grid(128, WM, WN, KROW);
  auto kern = gemm_mfma_128<IN, OUT, AM, BM, 128, WM, WN, KROW>;
  // Thread-safe one-time opt-in to more than 64 KiB of dynamic LDS.
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + 127) / 128) * ((g.n + 127) / 128));
  const int kb = (int)(g.k * kEsz);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), kLds, stream, (const char*)g.a,
                     (const char*)g.b, g.c, (int)g.m, (int)g.n, kb, g.lda * kEsz, g.ldb * kEsz,
                     g.ldc, g.scale, g.accumulate, kb, (int64_t)0, SplitTree{});
  return hipGetLastError();
}

// Split-K on 128x128 tiles, grid (tiles, slices).  Up to kTreeMaxSlices
// slices sum inside the launch (splitk_tree: partials and arrival words in
// the workspace `ws`, split_tree_bytes), and the last slice of each tile
// writes C.  More slices write f32 partial tiles to `ws` ([slices][M][N])
// and gemm_splitk_sum adds them in slice order in a second launch: the
// tree's levels are a serial chain of partial writes, arrivals and reads at
// memory latency, which two or more levels take longer than a second launch
// (operands from HBM, us, second launch -> tree: 128x14336x4096 (2 slices)
// 39.6 -> 36.9, 256x4096x4096 (2) 27.3 -> 26.6; 128x4096x4096 (4) 19.3 ->
// 20.9, 128x4096x14336 (8) 38.0 -> 42.5).  bf16 / f16 inputs, scale 1.
template <Elt IN, Elt OUT, bool AM, bool BM, int KROW, bool TREE>
static hipError_t launch_128_split_k(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                     hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g128::lds_bytes_grid(128, 2, 2, KROW);
  auto kern = gemm_mfma_128<IN, OUT, AM, BM, 128, 2, 2, KROW, TREE>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  if constexpr (TREE) {
    const SplitTree tree = split_tree_at(ws, tiles, slices, 128);
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, slices), dim3(256), kLds, stream,
                       (const char*)g.a, (const char*)g.b, g.c, (int)g.m, (int)g.n,
                       (int)(g.k * kEsz), g.lda * kEsz, g.ldb * kEsz, g.ldc, 1.0f, g.accumulate,
                       (int)kb_slice, (int64_t)0, tree);
    return hipGetLastError();
  } else {
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, slices), dim3(256), kLds, stream,
                       (const char*)g.a, (const char*)g.b, ws, (int)g.m, (int)g.n,
                       (int)(g.k * kEsz), g.lda * kEsz, g.ldb * kEsz, g.n, 1.0f, 0, (int)kb_slice,
                       (int64_t)g.m * g.n * 4, SplitTree{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return gemm_splitk_sum((const float*)ws, slices, g, stream);
  }
}

template <Elt IN, bool AM, bool BM, int KROW>
static hipError_t launch_128_split_out(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                       hipStream_t stream) {
  if (slices > kTreeMaxSlices)
    return launch_128_split_k<IN, Elt::F32, AM, BM, KROW, false>(g, slices, kb_slice, ws, stream);
  if constexpr (IN == Elt::F32) {
    if (g.out != Elt::F32) return hipErrorInvalidValue;
    return launch_128_split_k<IN, Elt::F32, AM, BM, KROW, true>(g, slices, kb_slice, ws, stream);
  }
  switch (g.out) {
    case Elt::BF16: return launch_128_split_k<IN, Elt::BF16, AM, BM, KROW, true>(g, slices, kb_slice, ws, stream);
    case Elt::F16: return launch_128_split_k<IN, Elt::F16, AM, BM, KROW, true>(g, slices, kb_slice, ws, stream);
    case Elt::F32: return launch_128_split_k<IN, Elt::F32, AM, BM, KROW, true>(g, slices, kb_slice, ws, stream);
    default: return hipErrorInvalidValue;
  }
}

template <Elt IN, bool AM, bool BM>
static hipError_t launch_128_split(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                   hipStream_t stream) {
  const int64_t tiles = ((g.m + 127) / 128) * ((g.n + 127) / 128);
  if (tiles * slices <= device_cus() && kb_slice % 128 == 0)
    return launch_128_split_out<IN, AM, BM, 128>(g, slices, kb_slice, ws, stream);
  return launch_128_split_out<IN, AM, BM, 64>(g, slices, kb_slice, ws, stream);
}

template <bool AM, bool BM>
hipError_t gemm_128_split_layout(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                 hipStream_t s) {
  if (g.in == Elt::BF16) return launch_128_split<Elt::BF16, AM, BM>(g, slices, kb_slice, ws, s);
  if (g.in == Elt::F16) return launch_128_split<Elt::F16, AM, BM>(g, slices, kb_slice, ws, s);
  if (g.in == Elt::F32) return launch_128_split<Elt::F32, AM, BM>(g, slices, kb_slice, ws, s);
  return hipErrorInvalidValue;
}

#define FRISK_PAIR(i, o) (((int)(i) << 8) | (int)(o))

template <bool AM, bool BM, int KROW>
static hipError_t gemm_128_pairs(const GemmArgs& g, hipStream_t s) {
  switch (FRISK_PAIR(g.in, g.out)) {
    case FRISK_PAIR(Elt::BF16, Elt::BF16): return launch_128<Elt::BF16, Elt::BF16, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::BF16, Elt::F32): return launch_128<Elt::BF16, Elt::F32, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F16): return launch_128<Elt::F16, Elt::F16, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F32): return launch_128<Elt::F16, Elt::F32, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::BF16): return launch_128<Elt::E4M3, Elt::BF16, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F16): return launch_128<Elt::E4M3, Elt::F16, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F32): return launch_128<Elt::E4M3, Elt::F32, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::I8, Elt::I32): return launch_128<Elt::I8, Elt::I32, AM, BM, 2, 2, KROW>(g, s);
    case FRISK_PAIR(Elt::F32, Elt::F32): return launch_128<Elt::F32, Elt::F32, AM, BM, 2, 2, KROW>(g, s);
    default: return hipErrorInvalidValue;
  }
}

// The library's own 128x128 launch: 128-byte stages when the grid is at
// most one workgroup per CU, 64-byte stages (two workgroups per CU)
// otherwise.  Both sum K in the same order, so the choice changes no bit.
template <bool AM, bool BM>
hipError_t gemm_128_layout(const GemmArgs& g, hipStream_t s) {
  if (gemm_128_stage_bytes(g, device_cus()) == 128) return gemm_128_pairs<AM, BM, 128>(g, s);
  return gemm_128_pairs<AM, BM, 64>(g, s);
}

template <bool AM, bool BM, int WM, int WN>
static hipError_t gemm_128_typed(const GemmArgs& g, hipStream_t s) {
  switch (FRISK_PAIR(g.in, g.out)) {
    case FRISK_PAIR(Elt::BF16, Elt::BF16): return launch_128<Elt::BF16, Elt::BF16, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::BF16, Elt::F32): return launch_128<Elt::BF16, Elt::F32, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F16): return launch_128<Elt::F16, Elt::F16, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F32): return launch_128<Elt::F16, Elt::F32, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::BF16): return launch_128<Elt::E4M3, Elt::BF16, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F16): return launch_128<Elt::E4M3, Elt::F16, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F32): return launch_128<Elt::E4M3, Elt::F32, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::I8, Elt::I32): return launch_128<Elt::I8, Elt::I32, AM, BM, WM, WN>(g, s);
    case FRISK_PAIR(Elt::F32, Elt::F32): return launch_128<Elt::F32, Elt::F32, AM, BM, WM, WN>(g, s);
    default: return hipErrorInvalidValue;
  }
}

template <bool AM, bool BM>
hipError_t gemm_128_grid_layout(const GemmArgs& g, hipStream_t s) {
  const int wm = g.wave_m ? g.wave_m : 2, wn = g.wave_n ? g.wave_n : 2;
  if (wm == 2 && wn == 2) return gemm_128_typed<AM, BM, 2, 2>(g, s);
  if (wm == 4 && wn == 1) return gemm_128_typed<AM, BM, 4, 1>(g, s);
  if (wm == 1 && wn == 4) return gemm_128_typed<AM, BM, 1, 4>(g, s);
  if (wm == 2 && wn == 1) return gemm_128_typed<AM, BM, 2, 1>(g, s);
  if (wm == 1 && wn == 2) return gemm_128_typed<AM, BM, 1, 2>(g, s);
  return hipErrorInvalidValue;
}

#undef FRISK_PAIR

}  // namespace frisk
