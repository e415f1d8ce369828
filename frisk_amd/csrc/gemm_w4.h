// Large-tile MFMA GEMM for gfx950: one 256x256 output tile per workgroup of
// four waves, one wave per SIMD, each wave owning a 128x128 sub-tile as 4x4
// accumulators of the 32x32 MFMA (256 accumulator registers per lane, held
// in AGPRs; the files that instantiate it are compiled without the
// VGPR-form MFMA option).
//
// Semantics: frisk.gemm (include/Dialect/Frisk/IR/FriskOps.td:252-292),
// C[m, n] = scale * sum_k op(A)[m, k] op(B)[k, n] (+ C when accumulating).
// AM / BM select the storage order of A and B (MN-major: A stored [K, M],
// i.e. trans_a; B stored [K, N], i.e. not trans_b); gemm_tile.h stages
// either order into LDS and reads fragments in one common k order, so the
// pipeline below is the same for all four layouts.  gemm_w4_a*b*.hip
// instantiate one layout each.
//
// Why four waves of 128x128 rather than eight of 128x64: per k-step a wave
// reads (TM + TN) fragments for TM * TN MFMAs, so the 128x128 sub-tile
// halves LDS read traffic per flop (8 reads per 16 MFMAs instead of 6 per
// 8), and with KR = 128 bytes of K per stage (64 bf16) the MFMA time between
// two workgroup barriers is 64 MFMAs = 2048 cycles.  A 128-byte row segment
// is one whole cache line: with 64-byte stages every line is fetched from L2
// twice (rocprofv3: TCP_TCC_READ_REQ halves from 1.34e8 to 6.7e7 at 8192^3).
// Two 64 KiB stages fill 128 KiB of the 160 KiB LDS.  With a single wave per
// SIMD nothing else can fill a stall, so every fragment read and DMA issue
// is placed between MFMAs explicitly (sched_group_barrier).

#pragma once

#include "common.h"
#include "gemm_common.h"
#include "gemm_tile.h"
#include "kernels.h"

namespace frisk {

// Bytes of K per row per stage (64 or 128), LDS stages, and the number of
// k-steps that issue DMA (0: the default below).
#ifndef FRISK_G4_KR
#define FRISK_G4_KR 128
#endif
#ifndef FRISK_G4_STAGES
#define FRISK_G4_STAGES 2
#endif
#ifndef FRISK_G4_PARTS
#define FRISK_G4_PARTS 0
#endif

namespace g4 {

constexpr int kBT = 256;
constexpr int kThreads = 256;

constexpr int lds_bytes(int kr, int stages) { return stages * 2 * kBT * kr; }

}  // namespace g4

template <Elt IN, Elt OUT, bool AM, bool BM, int KR, int S>
__global__ __launch_bounds__(g4::kThreads) void gemm_w4_kernel(
    const char* __restrict__ A, const char* __restrict__ B, void* __restrict__ C, int M, int N,
    int Kb, int64_t lda_b, int64_t ldb_b, int64_t ldc, float scale, int accumulate, int kb_slice,
    int64_t c_slice_bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
  using TA = OpTile<IN, AM, g4::kBT, KR>;
  using TB = OpTile<IN, BM, g4::kBT, KR>;
  A += TA::slice_shift((int64_t)blockIdx.y * kb_slice, lda_b);
  B += TB::slice_shift((int64_t)blockIdx.y * kb_slice, ldb_b);
  Kb = min(Kb - (int)blockIdx.y * kb_slice, kb_slice);
  C = (char*)C + (int64_t)blockIdx.y * c_slice_bytes;
  using Op = Mfma32<IN>;
  using Acc = typename Op::Acc;
  using AccS = typename std::conditional<IN == Elt::I8, int32_t, float>::type;
  constexpr int BT = g4::kBT;
  constexpr int TM = 4, TN = 4;                 // 32x32 atoms per wave
  constexpr int kTileBytes = BT * KR;           // one operand, one stage
  constexpr int kStageBytes = 2 * kTileBytes;
  constexpr int kLaneChunks = TA::kLaneChunks;  // 16 B pieces per lane per MFMA
  constexpr int kSteps = KR / Op::kBytes;       // MFMA k-steps per stage
  constexpr int kBlocks = kTileBytes / 1024 / 4;  // DMA blocks per wave per operand
  constexpr int kLoads = 2 * kBlocks;             // DMA loads per lane per stage
  // LDS read instructions per lane per k-step (two per 16 B of an MN-major
  // operand, one of a K-major one).
  constexpr int kFragReads =
      (TM * TA::kReadsPerChunk + TN * TB::kReadsPerChunk) * kLaneChunks;
  static_assert(S >= 2 && kSteps >= 1, "pipeline shape");

  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, half = lane >> 5;

  const int tiles_m = (M + BT - 1) / BT, tiles_n = (N + BT - 1) / BT;
  int tm, tn;
  tile_of_block<4>(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int row0 = tm * BT, col0 = tn * BT;

  // ---- LDS-DMA mapping ----------------------------------------------------
  // DMA instruction i of wave w fills 1 KiB block (kBlocks w + i) of each
  // operand tile (gemm_tile.h): an offset past num_records reads zeros,
  // which covers the K tail, the edges and the stages past the last one
  // without branches (and without memory traffic).
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
  // The DMA of a stage goes out in kParts parts, one in each of the first
  // kParts k-steps of an iteration; part p covers blocks
  // [p kBlocks / kParts, (p+1) kBlocks / kParts).  With three or more slots
  // every k-step issues a part.  With two, the stage being loaded is the
  // very next one, so only the first half of the k-steps issue DMA and the
  // loads issued last still have two k-steps of MFMAs to land (spreading
  // over one, two or three k-steps measured within 4% of each other).
  constexpr int kParts = FRISK_G4_PARTS > 0 ? (FRISK_G4_PARTS < kSteps ? FRISK_G4_PARTS : kSteps)
                         : (S >= 3 ? kSteps : (kSteps >= 2 ? kSteps / 2 : 1));
  static_assert(kBlocks >= kParts, "DMA parts");
  // Workgroups start their K walk at a per-XCD offset: stage kt of the loop
  // holds K stage (kt + krot) mod nk.  The workgroups of one XCD share A and
  // B rows through that XCD's L2 and keep one offset, so the sharing is
  // unchanged; the eight XCDs stop requesting the same 128-byte column of
  // every row at once (8192^3 bf16: 1190 -> 1280 TFLOP/s, neutral at 4096^3).
  // Loop stages past the last one stay past it and read nothing.
  const int nk_all = (Kb + KR - 1) / KR;
  const int krot = __builtin_amdgcn_readfirstlane((int)(blockIdx.x % 8) * nk_all / 8);
  auto issue_part = [&](int stage, int slot, auto part) {
    constexpr int p = decltype(part)::value;
    int phys = stage + krot;
    if (phys >= nk_all) phys -= nk_all;
    if (stage >= nk_all) phys = stage;
    char* dst = smem + slot * kStageBytes + wave * kBlocks * 1024;
#pragma unroll
    for (int i = p * kBlocks / kParts; i < (p + 1) * kBlocks / kParts; ++i) {
      uint32_t oa = TA::offset(da, i, phys);
      uint32_t ob = TB::offset(db, i, phys);
      // Keep the selects as selects: otherwise the backend may turn them
      // into branches around two copies of each load.
      asm("" : "+v"(oa));
      asm("" : "+v"(ob));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr_t)(dst + i * 1024), 16, oa, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_ptr_t)(dst + kTileBytes + i * 1024), 16, ob,
                                               0, 0, 0);
    }
  };

  // ---- fragment reads -----------------------------------------------------
  typename TA::Frag fa[TM];
  typename TB::Frag fb[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) fa[t] = TA::frag(wm * (32 * TM) + t * 32, lane);
#pragma unroll
  for (int t = 0; t < TN; ++t) fb[t] = TB::frag(wn * (32 * TN) + t * 32, lane);
  using Frag = Frags<TM, TN, kLaneChunks>;
  auto load_frags = [&](int slot, int s, Frag& f) {
    const char* base = smem + slot * kStageBytes;
#pragma unroll
    for (int t = 0; t < TM; ++t) TA::read(base, fa[t], s, f.a[t]);
#pragma unroll
    for (int t = 0; t < TN; ++t) TB::read(base + kTileBytes, fb[t], s, f.b[t]);
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
  // Stage kt lives in slot kt % S.  In the last k-step of stage kt, after
  // half of its MFMAs, each wave waits for its own loads of stage kt+1 and
  // for its LDS reads; a workgroup barrier then publishes stage kt+1 and
  // proves that every wave is done with slot kt % S.  That slot receives
  // stage kt+S, whose DMA is spread over the first kParts k-steps of
  // iteration kt+1.  Stage kt+1 is issued during iteration kt+2-S and S-2
  // newer stages may be in flight at the wait.  Every iteration issues
  // exactly kLoads loads (past the last stage they are zero-reads without
  // memory traffic), so the vmcnt bookkeeping is static.
  const int nk = (Kb + KR - 1) / KR;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    static_for<0, kParts>([&](auto p) { issue_part(st, st, p); });
  FRISK_WAIT_VMCNT(kLoads * (S - 2));
  __builtin_amdgcn_s_barrier();

  Frag fr[2];
  load_frags(0, 0, fr[0]);
  // Drain every LGKM operation issued so far (these fragment reads and the
  // scalar loads of the epilogue's kernel arguments): with scalar loads
  // pending at the loop entry the LGKM counter is unordered, and the
  // compiler would then wait for lgkmcnt(0) at the top of every iteration.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  int slot = 0, fslot = S - 1;  // slots of stage kt and of stage kt+S-1
  constexpr int kMf = TM * TN;
  constexpr int kHalf = kMf / 2;
  for (int kt = 0; kt < nk; ++kt) {
    static_for<0, kSteps>([&](auto step) {
      constexpr int s = decltype(step)::value;
      constexpr int cur = s & 1, nxt = cur ^ 1;
      constexpr bool dma = s < kParts;
      constexpr int nload = dma ? 2 * ((s + 1) * kBlocks / kParts - s * kBlocks / kParts) : 0;
      if constexpr (s + 1 < kSteps) {
        // Program order: fragment reads, then DMA (the compiler keeps LDS
        // reads and LDS-DMA writes in order, as it cannot tell slots apart).
        load_frags(slot, s + 1, fr[nxt]);
        if constexpr (dma) issue_part(kt + S - 1, fslot, step);
        mfma_rows(fr[cur], 0, TM);
        if constexpr (dma) {
          // Fragment reads under the first half of the MFMAs, DMA under the
          // second half.
          constexpr int kDsG = kFragReads < kHalf ? kFragReads : kHalf;
          constexpr int kDsPer = (kFragReads + kDsG - 1) / kDsG;
          constexpr int kVmPer = (nload + (kMf - kDsG) - 1) / (kMf - kDsG);
          static_for<0, kDsG>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x100, kDsPer, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
          });
          static_for<0, (nload + kVmPer - 1) / kVmPer>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x010, kVmPer, 0);  // VMEM (LDS-DMA)
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
          });
        } else {
          static_for<0, kFragReads>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          });
        }
        __builtin_amdgcn_sched_barrier(0);
      } else {
        if constexpr (dma) {
          issue_part(kt + S - 1, fslot, step);
          mfma_rows(fr[cur], 0, TM / 2);
          constexpr int kVmPer = (nload + kHalf - 1) / kHalf;
          static_for<0, (nload + kVmPer - 1) / kVmPer>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x010, kVmPer, 0);  // VMEM (LDS-DMA)
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
          });
        } else {
          mfma_rows(fr[cur], 0, TM / 2);
        }
        __builtin_amdgcn_sched_barrier(0);
        // vmcnt <= kLoads (S-2) and lgkmcnt = 0.
        __builtin_amdgcn_s_waitcnt((((kLoads * (S - 2)) & 15) | (((kLoads * (S - 2)) >> 4) << 14) |
                                    (7 << 4)));
        __builtin_amdgcn_s_barrier();
        const int nslot = slot + 1 == S ? 0 : slot + 1;
        load_frags(nslot, 0, fr[kSteps & 1 ? nxt : 0]);
        mfma_rows(fr[cur], TM / 2, TM);
        constexpr int kDsPer = (kFragReads + kHalf - 1) / kHalf;
        static_for<0, kHalf>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x100, kDsPer, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
        });
        __builtin_amdgcn_sched_barrier(0);
        fslot = slot;
        slot = nslot;
      }
    });
    if constexpr (kSteps == 1) fr[0] = fr[1];
  }
  // Drain the trailing DMA loads before the stage buffers are reused.
  FRISK_WAIT_VMCNT(0);
  __syncthreads();

  // Epilogue: per wave, stage a 32 x 128 slice (one accumulator row block)
  // as 32-bit values, then each lane stores 8 consecutive columns.  The
  // 32x32 accumulator holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] in
  // element r.
  constexpr int kPitch = 32 * TN + 4;
  static_assert(4 * 32 * kPitch * 4 <= g4::lds_bytes(KR, S), "epilogue staging fits in LDS");
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

template <Elt IN, Elt OUT, bool AM, bool BM>
static hipError_t launch_w4(const GemmArgs& g, hipStream_t stream) {
  constexpr int KR = FRISK_G4_KR, S = FRISK_G4_STAGES;
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g4::lds_bytes(KR, S);
  static_assert(kLds <= 160 * 1024, "LDS budget of one CU");
  auto kern = gemm_w4_kernel<IN, OUT, AM, BM, KR, S>;
  // Thread-safe one-time opt-in to more than 64 KiB of dynamic LDS.
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + g4::kBT - 1) / g4::kBT) * ((g.n + g4::kBT - 1) / g4::kBT));
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(g4::kThreads), kLds, stream, (const char*)g.a,
                     (const char*)g.b, g.c, (int)g.m, (int)g.n, (int)(g.k * kEsz),
                     g.lda * kEsz, g.ldb * kEsz, g.ldc, g.scale, g.accumulate,
                     (int)(g.k * kEsz), (int64_t)0);
  return hipGetLastError();
}

// Split-K: f32 partials of each K slice into `partial` ([slices][M][N]),
// then their sum in slice order into C (bf16 / f16 inputs, scale 1).
template <Elt IN, bool AM, bool BM>
static hipError_t launch_w4_split(const GemmArgs& g, int slices, int64_t kb_slice, float* partial,
                                  hipStream_t stream) {
  constexpr int KR = FRISK_G4_KR, S = FRISK_G4_STAGES;
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g4::lds_bytes(KR, S);
  auto kern = gemm_w4_kernel<IN, Elt::F32, AM, BM, KR, S>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + g4::kBT - 1) / g4::kBT) * ((g.n + g4::kBT - 1) / g4::kBT));
  hipLaunchKernelGGL(kern, dim3(tiles, slices), dim3(g4::kThreads), kLds, stream, (const char*)g.a,
                     (const char*)g.b, (void*)partial, (int)g.m, (int)g.n, (int)(g.k * kEsz),
                     g.lda * kEsz, g.ldb * kEsz, g.n, 1.0f, 0, (int)kb_slice,
                     (int64_t)g.m * g.n * 4);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return gemm_splitk_sum(partial, slices, g, stream);
}

template <bool AM, bool BM>
hipError_t gemm_w4_split_layout(const GemmArgs& g, int slices, int64_t kb_slice, float* partial,
                                hipStream_t s) {
  if (g.in == Elt::BF16) return launch_w4_split<Elt::BF16, AM, BM>(g, slices, kb_slice, partial, s);
  if (g.in == Elt::F16) return launch_w4_split<Elt::F16, AM, BM>(g, slices, kb_slice, partial, s);
  return hipErrorInvalidValue;
}

#define FRISK_PAIR(i, o) (((int)(i) << 8) | (int)(o))

template <bool AM, bool BM>
hipError_t gemm_w4_layout(const GemmArgs& g, hipStream_t s) {
  switch (FRISK_PAIR(g.in, g.out)) {
    case FRISK_PAIR(Elt::BF16, Elt::BF16): return launch_w4<Elt::BF16, Elt::BF16, AM, BM>(g, s);
    case FRISK_PAIR(Elt::BF16, Elt::F32): return launch_w4<Elt::BF16, Elt::F32, AM, BM>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F16): return launch_w4<Elt::F16, Elt::F16, AM, BM>(g, s);
    case FRISK_PAIR(Elt::F16, Elt::F32): return launch_w4<Elt::F16, Elt::F32, AM, BM>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::BF16): return launch_w4<Elt::E4M3, Elt::BF16, AM, BM>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F16): return launch_w4<Elt::E4M3, Elt::F16, AM, BM>(g, s);
    case FRISK_PAIR(Elt::E4M3, Elt::F32): return launch_w4<Elt::E4M3, Elt::F32, AM, BM>(g, s);
    case FRISK_PAIR(Elt::I8, Elt::I32): return launch_w4<Elt::I8, Elt::I32, AM, BM>(g, s);
    default: return hipErrorInvalidValue;
  }
}

#undef FRISK_PAIR

}  // namespace frisk
