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
// Five 32 KiB operand-tile slots fill the 160 KiB LDS as a ring (below).
// With a single wave per SIMD nothing else can fill a stall, so every
// fragment read and DMA issue is placed between MFMAs explicitly
// (sched_group_barrier).

#pragma once

#include "common.h"
#include "gemm_common.h"
#include "gemm_tile.h"
#include "kernels.h"

namespace frisk {

// Bytes of K per row per stage (64 or 128).
#ifndef FRISK_G4_KR
#define FRISK_G4_KR 128
#endif
// MFMA output tile (32: v_mfma_*_32x32x*, 16: v_mfma_*_16x16x*).
#ifndef FRISK_G4_ATOM
#define FRISK_G4_ATOM 32
#endif

namespace g4 {

constexpr int kBT = 256;
constexpr int kThreads = 256;

constexpr int kRing = 5;  // operand-tile slots of the LDS ring
constexpr int lds_bytes(int kr) { return kRing * kBT * kr; }

// Load q of an iteration (B(kt+1) blocks 0..nb-1, then A(kt+2) blocks) goes
// out beside MFMA pos(q) of the iteration's t MFMAs: evenly spread, the last
// beside the last MFMA.
constexpr int load_pos(int q, int nb, int t) { return (q + 1) * t / (2 * nb) - 1; }
// Loads placed beside MFMAs [g0, g1) of the iteration.
constexpr int loads_in(int nb, int t, int g0, int g1) {
  int c = 0;
  for (int q = 0; q < 2 * nb; ++q) c += load_pos(q, nb, t) >= g0 && load_pos(q, nb, t) < g1;
  return c;
}
// A loads placed before MFMA g (all B loads are older than every A load).
constexpr int a_loads_before(int nb, int t, int g) {
  int c = 0;
  for (int q = nb; q < 2 * nb; ++q) c += load_pos(q, nb, t) < g;
  return c;
}

}  // namespace g4

// Epilogue of 16-bit outputs, one pass: each wave rounds its 128x128
// sub-tile (32x32 atoms) to OUT in registers and stages it in its own
// 32 KiB of LDS, then stores whole 256-byte row pieces.  Accumulator
// elements 8p .. 8p+7 of lane L hold columns 16p + 4h .. +3 and
// 16p + 8 + 4h .. +3 (h = L / 32) of row L % 32; one v_permlane32_swap per
// packed pair hands lane L the 8 consecutive columns 16p + 8h .. +7, so each
// lane writes one 16-byte chunk per atom and p.  Staged row R keeps chunk c
// at c ^ (R & 15): the 16 lanes of a write (16 rows, one chunk) and of a
// read (one row, 16 chunks) touch every bank once.  Each output is
// acc * scale (+ C when accumulating, read as f32 before the rounding),
// rounded once to nearest even, as in the f32-staged path; each wave reads
// back only what it wrote, so no workgroup barrier is needed.
template <Elt OUT, bool ACCUMULATE, bool SCALED, int TM, int TN>
__device__ __forceinline__ void epilogue16(const f32x16 (&acc)[TM][TN], float scale, int lane,
                                           char* stage, int r0, int c0, int M, int N, int64_t ldc,
                                           void* C) {
  constexpr int kPitch = 256;
  auto at = [](int R, int c) { return R * kPitch + ((c ^ (R & 15)) << 4); };
  const int half = lane >> 5;
  // C[r0 + R][c0 + c .. c + 3] as f32 (0 outside the matrix).
  auto old4 = [&](int R, int c, float* o) {
    const int gr = r0 + R, gc = c0 + c;
    const uint16_t* src = (const uint16_t*)C + (int64_t)gr * ldc + gc;
    i32x2 w = {0, 0};
    if (gr < M && gc + 4 <= N) {
      w = *(const i32x2*)src;
    } else if (gr < M) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (gc + k < N) w[k >> 1] |= (int)((uint32_t)src[k] << (16 * (k & 1)));
    }
    const uint16_t* e = (const uint16_t*)&w;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] += load_as_f32<OUT>(e, k);
  };
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      static_for<0, 2>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        // Read from the AGPRs one element at a time: used by VALU code
        // directly, the compiler copies all 256 accumulators to VGPRs at
        // once and spills.
        float f[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(f[k]) : "a"(acc[i][j][8 * p + k]));
          if constexpr (SCALED) f[k] *= scale;  // x * 1 == x: skipped for scale 1
        }
        const int R = i * 32 + (lane & 31);
        if constexpr (ACCUMULATE) {
          old4(R, j * 32 + 16 * p + 4 * half, f);
          old4(R, j * 32 + 16 * p + 8 + 4 * half, f + 4);
        }
        const uint32_t x0 = pack_f32x2<OUT>(f[0], f[1]), x1 = pack_f32x2<OUT>(f[2], f[3]);
        const uint32_t y0 = pack_f32x2<OUT>(f[4], f[5]), y1 = pack_f32x2<OUT>(f[6], f[7]);
        // Lanes 0-31 keep x and take the partner's x; lanes 32-63 take the
        // partner's y and keep y.
        const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
        const i32x4 w = {(int)s0[0], (int)s1[0], (int)s0[1], (int)s1[1]};
        *(i32x4*)(stage + at(R, 4 * j + 2 * p + half)) = w;
        // One atom's conversions at a time.
        __builtin_amdgcn_sched_barrier(0);
      });
#pragma unroll
  for (int it = 0; it < TM * 32 * 16 / 64; ++it) {
    if (it % 8 == 0) __builtin_amdgcn_sched_barrier(0);
    const int q = it * 64 + lane, rr = q >> 4, g = q & 15;
    const i32x4 v = *(const i32x4*)(stage + at(rr, g));
    const int gr = r0 + rr, gc = c0 + 8 * g;
    if (gr < M && gc < N) {
      uint16_t* dst = (uint16_t*)C + (int64_t)gr * ldc + gc;
      if (gc + 8 <= N) {
        __builtin_nontemporal_store(v, (i32x4*)dst);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (gc + k < N) dst[k] = (uint16_t)((uint32_t)v[k >> 1] >> (16 * (k & 1)));
      }
    }
  }
}

template <Elt IN, Elt OUT, bool AM, bool BM, int KR, int ATOM>
__global__ __launch_bounds__(g4::kThreads) void gemm_w4_kernel(
    const char* __restrict__ A, const char* __restrict__ B, void* __restrict__ C, int M, int N,
    int Kb, int64_t lda_b, int64_t ldb_b, int64_t ldc, float scale, int accumulate, int kb_slice,
    int64_t c_slice_bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
  using TA = OpTile<IN, AM, g4::kBT, KR, ATOM>;
  using TB = OpTile<IN, BM, g4::kBT, KR, ATOM>;
  A += TA::slice_shift((int64_t)blockIdx.y * kb_slice, lda_b);
  B += TB::slice_shift((int64_t)blockIdx.y * kb_slice, ldb_b);
  Kb = min(Kb - (int)blockIdx.y * kb_slice, kb_slice);
  C = (char*)C + (int64_t)blockIdx.y * c_slice_bytes;
  using Op = MfmaAtom<IN, ATOM>;
  using Acc = typename Op::Acc;
  using AccS = typename std::conditional<IN == Elt::I8, int32_t, float>::type;
  constexpr int BT = g4::kBT;
  constexpr int TM = 128 / ATOM, TN = 128 / ATOM;  // atoms per wave (128x128 sub-tile)
  constexpr int kAccN = sizeof(Acc) / 4;           // accumulator elements per lane
  constexpr int kTileBytes = BT * KR;           // one operand, one stage
  constexpr int kLaneChunks = TA::kLaneChunks;  // 16 B pieces per lane per MFMA
  constexpr int kSteps = KR / Op::kBytes;       // MFMA k-steps per stage
  constexpr int kBlocks = kTileBytes / 1024 / 4;  // DMA blocks per wave per operand
  static_assert(kSteps >= 2, "a stage holds at least two MFMA k-steps");

  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

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
  // Every stage before nk_full holds KR whole bytes of K, so a lane live in
  // the last of them is live in all: a_full / b_full are the stage-invariant
  // lane offsets of those stages, and the stage base goes in the scalar
  // offset.  The steady-state iterations (below) issue exactly that, with no
  // VALU work (bf16 4096^3 +1.1-2.1%, 8192^3 +1.7-2.4%, int8 +0.6-0.9%, fp8
  // within noise).  The other iterations: with four or more k-steps per
  // stage, one VALU select per load between a_full and a_tail (the partial
  // stage nk_full, when KR does not divide K, keeps only its live chunks)
  // and a zero-length range past the last stage; with two k-steps (fp8),
  // per-lane offsets (the select form measured 1.3% slower there).
  constexpr bool kScalarStage = kSteps >= 4;
  const int nk_full = Kb / KR;
  uint32_t a_full[kBlocks], a_tail[kBlocks], b_full[kBlocks], b_tail[kBlocks];
#pragma unroll
  for (int i = 0; i < kBlocks; ++i) {
    a_full[i] = (nk_full - 1) * TA::kStep < da.lim[i] ? da.off[i] : 0x80000000u;
    b_full[i] = (nk_full - 1) * TB::kStep < db.lim[i] ? db.off[i] : 0x80000000u;
    if constexpr (kScalarStage) {
      a_tail[i] = nk_full * TA::kStep < da.lim[i] ? da.off[i] : 0x80000000u;
      b_tail[i] = nk_full * TB::kStep < db.lim[i] ? db.off[i] : 0x80000000u;
    }
  }
  const __amdgpu_buffer_rsrc_t rsa_none = __builtin_amdgcn_make_buffer_rsrc(
      (void*)TA::origin(A, row0, lda_b), (short)0, 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb_none = __builtin_amdgcn_make_buffer_rsrc(
      (void*)TB::origin(B, col0, ldb_b), (short)0, 0, 0x00020000);
  // Workgroups start their K walk at a per-XCD offset: stage kt of the loop
  // holds K stage (kt + krot) mod nk.  The workgroups of one XCD share A and
  // B rows through that XCD's L2 and keep one offset, so the sharing is
  // unchanged; the eight XCDs stop requesting the same 128-byte column of
  // every row at once (8192^3 bf16: 1190 -> 1280 TFLOP/s, neutral at 4096^3).
  // Loop stages past the last one stay past it and read nothing.
  const int nk_all = (Kb + KR - 1) / KR;
  const int krot = __builtin_amdgcn_readfirstlane((int)(blockIdx.x % 8) * nk_all / 8);
  auto phys_of = [&](int stage) {
    int phys = stage + krot;
    if (phys >= nk_all) phys -= nk_all;
    return stage >= nk_all ? stage : phys;
  };
  // issue() sends part p of np of one operand tile: blocks
  // [p kBlocks / np, (p+1) kBlocks / np).  `fast`: the steady state, where
  // the stage is a whole one inside K (no partial stage exists and the stage
  // is not past the last): every lane's offset is its stage-invariant one
  // and the stage base is the scalar offset, so a load is issued with no
  // VALU work at all.
  auto issue = [&](auto op, int stage, int slot, auto part, auto parts, auto fast) {
    constexpr int p = decltype(part)::value, np = decltype(parts)::value;
    constexpr bool is_a = decltype(op)::value;
    const int phys = phys_of(stage);
    char* dst = smem + slot * kTileBytes + wave * kBlocks * 1024;
    if constexpr (decltype(fast)::value) {
      const uint32_t soff = (uint32_t)phys * (is_a ? da.adv : db.adv);
#pragma unroll
      for (int i = p * kBlocks / np; i < (p + 1) * kBlocks / np; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? rsa : rsb, (lds_ptr_t)(dst + i * 1024), 16,
                                                 is_a ? a_full[i] : b_full[i],
                                                 __builtin_amdgcn_readfirstlane(soff), 0, 0);
    } else if constexpr (kScalarStage) {
      const bool past = phys >= nk_all, tail = phys == nk_full;
      const uint32_t soff = past ? 0u : (uint32_t)phys * (is_a ? da.adv : db.adv);
      const __amdgpu_buffer_rsrc_t rs = is_a ? (past ? rsa_none : rsa) : (past ? rsb_none : rsb);
#pragma unroll
      for (int i = p * kBlocks / np; i < (p + 1) * kBlocks / np; ++i) {
        uint32_t o = is_a ? (tail ? a_tail[i] : a_full[i]) : (tail ? b_tail[i] : b_full[i]);
        asm("" : "+v"(o));  // a v_cndmask, not a branch around two loads
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(dst + i * 1024), 16, o,
                                                 __builtin_amdgcn_readfirstlane(soff), 0, 0);
      }
    } else {
#pragma unroll
      for (int i = p * kBlocks / np; i < (p + 1) * kBlocks / np; ++i) {
        uint32_t o = is_a ? TA::offset(da, i, phys) : TB::offset(db, i, phys);
        // Keep the select a select: otherwise the backend may turn it into a
        // branch around two copies of the load.
        asm("" : "+v"(o));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? rsa : rsb, (lds_ptr_t)(dst + i * 1024),
                                                 16, o, 0, 0, 0);
      }
    }
  };
  using OpA = std::true_type;
  using OpB = std::false_type;

  // ---- fragment reads -----------------------------------------------------
  // K-major operands share one Frag (tile 0's) across their tiles.
  typename TA::Frag fa[TA::kSharedFrag ? 1 : TM];
  typename TB::Frag fb[TB::kSharedFrag ? 1 : TN];
#pragma unroll
  for (int t = 0; t < (TA::kSharedFrag ? 1 : TM); ++t) fa[t] = TA::frag(wm * 128 + t * ATOM, lane);
#pragma unroll
  for (int t = 0; t < (TB::kSharedFrag ? 1 : TN); ++t) fb[t] = TB::frag(wn * 128 + t * ATOM, lane);
  using Frag = Frags<TM, TN, kLaneChunks>;
  auto load_frags = [&](int aslot, int bslot, int s, Frag& f) {
    const char* abase = smem + aslot * kTileBytes;
    const char* bbase = smem + bslot * kTileBytes;
#pragma unroll
    for (int t = 0; t < TM; ++t)
      TA::read(abase, fa[TA::kSharedFrag ? 0 : t], s, f.a[t], TA::tile_off(t * ATOM));
#pragma unroll
    for (int t = 0; t < TN; ++t)
      TB::read(bbase, fb[TB::kSharedFrag ? 0 : t], s, f.b[t], TB::tile_off(t * ATOM));
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
      for (int j = 0; j < TN; ++j) acc[i][j] = Op::run(f.b[j], f.a[i], acc[i][j]);
  };

  // ---- pipeline -----------------------------------------------------------
  // LDS ring of five operand-tile slots: tile t (A of stage t/2 when t is
  // even, B of stage (t-1)/2 when odd) lives in slot t % 5.  Iteration kt
  // reads A(kt) and B(kt) and issues B(kt+1), then A(kt+2); their slots
  // held A(kt-1) and B(kt-1), which every wave finished reading before the
  // barrier that ended iteration kt-1.  In the last k-step, after half of
  // its MFMAs, each wave waits for its LDS reads and for all but the
  // A(kt+2) loads it has issued so far (kInFlight), which leaves A(kt+1)
  // (issued an iteration earlier) and B(kt+1) landed; the workgroup barrier
  // then publishes them.
  // The iteration's 2 kBlocks loads (B(kt+1) blocks, then A(kt+2) blocks)
  // go out one beside every (kSteps kMf) / (2 kBlocks)-th MFMA over the
  // whole iteration (g4::load_pos), the A loads of the last k-step's second
  // half after its barrier, so the load rate never bunches up (TA
  // address-FIFO-full cycles; bit-identical, bf16 +0.4-0.8%, int8 +0.5%,
  // fp8 within noise against B over the first k-steps' second halves and A
  // over the rest's).  Every iteration issues the same loads (past the last
  // stage they are zero-reads without memory traffic), so the vmcnt
  // bookkeeping is static.  Measured against two 64 KiB stages written
  // whole per iteration (4096^3 bf16 / 4096x8192x8192 fp8 / 8192^3 bf16):
  // +2% / +7% / +4%.
  const int nk = (Kb + KR - 1) / KR;
  using Slow = std::false_type;
  using Whole = std::integral_constant<int, 0>;
  using One = std::integral_constant<int, 1>;
  issue(OpA{}, 0, 0, Whole{}, One{}, Slow{});
  issue(OpB{}, 0, 1, Whole{}, One{}, Slow{});
  issue(OpA{}, 1, 2, Whole{}, One{}, Slow{});
  FRISK_WAIT_VMCNT(kBlocks);
  __builtin_amdgcn_s_barrier();

  Frag fr[2];
  load_frags(0, 1, 0, fr[0]);
  // Drain every LGKM operation issued so far (these fragment reads and the
  // scalar loads of the epilogue's kernel arguments): with scalar loads
  // pending at the loop entry the LGKM counter is unordered, and the
  // compiler would then wait for lgkmcnt(0) at the top of every iteration.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  int a_rd = 0, b_rd = 1, b_wr = 3, a_wr = 4;  // slots of A(kt), B(kt), B(kt+1), A(kt+2)
  auto adv = [](int x) { return x >= 3 ? x - 3 : x + 2; };  // (x + 2) mod 5
  constexpr int kMf = TM * TN;
  constexpr int kHalf = kMf / 2;
  // Fragment unit u (of kUnits per k-step) is read beside MFMA
  // u kHalf / kUnits of the half k-step that reads.
  constexpr int kUnits = TM + TN;
  static_assert(kHalf % kUnits == 0, "fragment units spread evenly over a half step");
  constexpr int kUnitGap = kHalf / kUnits;
  // The loads that may still be in flight at the last k-step's barrier: the
  // A(kt+2) loads issued before it (every B(kt+1) load is older).
  constexpr int kT = kSteps * kMf;
  constexpr int kInFlight = g4::a_loads_before(kBlocks, kT, kT - kHalf);
  // Fragment unit u of k-step s: A tile u (u < TM) or B tile u - TM.
  auto read_unit = [&](int aslot, int bslot, int s, Frag& f, int u) {
    if (u < TM) TA::read(smem + aslot * kTileBytes, fa[TA::kSharedFrag ? 0 : u], s, f.a[u],
                         TA::tile_off(u * ATOM));
    else TB::read(smem + bslot * kTileBytes, fb[TB::kSharedFrag ? 0 : u - TM], s, f.b[u - TM],
                  TB::tile_off((u - TM) * ATOM));
  };
  auto iteration = [&](int kt, auto fast) {
    static_for<0, kSteps>([&](auto step) {
      constexpr int s = decltype(step)::value;
      constexpr int cur = s & 1, nxt = cur ^ 1;
      constexpr bool last = s + 1 == kSteps;
      auto load = [&](auto qc) {
        constexpr int q = decltype(qc)::value;
        if constexpr (q < kBlocks)
          issue(OpB{}, kt + 1, b_wr, std::integral_constant<int, q>{},
                std::integral_constant<int, kBlocks>{}, fast);
        else
          issue(OpA{}, kt + 2, a_wr, std::integral_constant<int, q - kBlocks>{},
                std::integral_constant<int, kBlocks>{}, fast);
      };
      // Program order = issue order: beside MFMA m, a fragment unit (first
      // half of a k-step, or the next stage's in the second half of the
      // last k-step), then the loads placed at m.
      auto emit = [&](auto mc, int aslot, int bslot, int rs, Frag& f) {
        constexpr int m = decltype(mc)::value;
        constexpr int h = last ? m - kHalf : m;  // position in the reading half
        if constexpr (h >= 0 && h < kHalf && h % kUnitGap == 0)
          read_unit(aslot, bslot, rs, f, h / kUnitGap);
        static_for<0, 2 * kBlocks>([&](auto qc) {
          if constexpr (g4::load_pos(decltype(qc)::value, kBlocks, kT) == s * kMf + m) load(qc);
        });
      };
      auto groups = [&](auto m0, auto m1) {
        static_for<decltype(m0)::value, decltype(m1)::value>([&](auto mc) {
          constexpr int m = decltype(mc)::value;
          constexpr int h = last ? m - kHalf : m;
          constexpr int u = h / kUnitGap;
          if constexpr (h >= 0 && h < kHalf && h % kUnitGap == 0) {
            constexpr int nds = (u < TM ? TA::kReadsPerChunk : TB::kReadsPerChunk) * kLaneChunks;
            __builtin_amdgcn_sched_group_barrier(0x100, nds, 0);  // DS read
          }
          constexpr int nvm = g4::loads_in(kBlocks, kT, s * kMf + m, s * kMf + m + 1);
          if constexpr (nvm > 0) __builtin_amdgcn_sched_group_barrier(0x010, nvm, 0);  // LDS-DMA
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        });
      };
      if constexpr (!last) {
        static_for<0, kMf>([&](auto mc) { emit(mc, a_rd, b_rd, s + 1, fr[nxt]); });
        mfma_rows(fr[cur], 0, TM);
        groups(std::integral_constant<int, 0>{}, std::integral_constant<int, kMf>{});
        __builtin_amdgcn_sched_barrier(0);
      } else {
        const int na = adv(a_rd), nb = adv(b_rd);
        static_for<0, kHalf>([&](auto mc) { emit(mc, na, nb, 0, fr[kSteps & 1 ? nxt : 0]); });
        mfma_rows(fr[cur], 0, TM / 2);
        groups(std::integral_constant<int, 0>{}, std::integral_constant<int, kHalf>{});
        __builtin_amdgcn_sched_barrier(0);
        // vmcnt <= kInFlight (this wave's A(kt+2) loads so far) and lgkmcnt = 0.
        __builtin_amdgcn_s_waitcnt(((kInFlight & 15) | ((kInFlight >> 4) << 14) | (7 << 4)));
        __builtin_amdgcn_s_barrier();
        static_for<kHalf, kMf>([&](auto mc) { emit(mc, na, nb, 0, fr[kSteps & 1 ? nxt : 0]); });
        mfma_rows(fr[cur], TM / 2, TM);
        groups(std::integral_constant<int, kHalf>{}, std::integral_constant<int, kMf>{});
        __builtin_amdgcn_sched_barrier(0);
        a_rd = na;
        b_rd = nb;
        b_wr = adv(b_wr);
        a_wr = adv(a_wr);
      }
    });
  };
  // Iterations whose loads (stages kt + 1 and kt + 2) are whole stages
  // inside K take the fast issue; the last two, and every iteration when K
  // ends in a partial stage, take the general one.
  const int nk_fast = Kb % KR == 0 ? max(nk - 2, 0) : 0;
  int kt = 0;
  for (; kt < nk_fast; ++kt) iteration(kt, std::true_type{});
  for (; kt < nk; ++kt) iteration(kt, Slow{});
  // Drain the trailing DMA loads before the stage buffers are reused.
  FRISK_WAIT_VMCNT(0);
  __syncthreads();

  // Epilogue.  The MFMAs take the B fragment as their first operand, so
  // accumulator element r of lane L in atom (i, j) is output row
  // i ATOM + L % ATOM, column j ATOM + Op::acc_row(r, L) of the wave's
  // 128x128 sub-tile, and elements 4q .. 4q+3 are four consecutive columns.
  // 16-bit outputs of 32x32 atoms round in registers and stage once
  // (epilogue16).  Otherwise each wave stages half of its sub-tile at a time
  // in LDS by rows as 32-bit values, one 16-byte write of four accumulators
  // straight from the AGPRs per column group, then stores row pieces,
  // consecutive lanes on consecutive pieces: 8 outputs (16 bytes) per lane
  // for 16-bit outputs through store8, 4 (16 bytes) for 32-bit ones through
  // store4; both scale, accumulate and convert.  Staged row R keeps 16-byte
  // chunk c at c ^ (R & 15) ^ (c >> 4): the writes of 16 lanes (16 rows, one
  // column group) and each read of 16 lanes (one row; chunks 2g or 2g+1, or
  // g) touch every bank once.  (16-bit outputs staged that way, in two
  // passes of f32: bf16 4096^3 -0.4-1.3%, fp8 -0.2-0.7%, bit-identical.)
  if constexpr (EltInfo<OUT>::bytes == 2 && ATOM == 32) {
    char* stage = smem + wave * (128 * 256);
    const int r0 = row0 + wm * 128, c0 = col0 + wn * 128;
    if (accumulate)
      epilogue16<OUT, true, true>(acc, scale, lane, stage, r0, c0, M, N, ldc, C);
    else if (scale == 1.0f)
      epilogue16<OUT, false, false>(acc, scale, lane, stage, r0, c0, M, N, ldc, C);
    else
      epilogue16<OUT, false, true>(acc, scale, lane, stage, r0, c0, M, N, ldc, C);
    return;
  }
  {
    constexpr int kOut = EltInfo<OUT>::bytes == 2 ? 8 : 4;  // outputs per lane per store
    constexpr int kPPR = 128 / kOut;         // pieces per staged row
    constexpr int kPassTM = TM / 2;          // atom rows per pass
    constexpr int kRows = kPassTM * ATOM;
    constexpr int kPitch = 128 * 4;
    static_assert(4 * kRows * kPitch <= g4::lds_bytes(KR), "epilogue staging fits in LDS");
    static_assert(kRows * kPPR % 64 == 0, "whole store rounds");
    char* stage = smem + wave * (kRows * kPitch);
    auto chunk_at = [](int R, int c) { return R * kPitch + ((c ^ (R & 15) ^ (c >> 4)) << 4); };
#pragma unroll
    for (int ps = 0; ps < TM / kPassTM; ++ps) {
#pragma unroll
      for (int ii = 0; ii < kPassTM; ++ii) {
        const int i = ps * kPassTM + ii;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          static_for<0, kAccN / 4>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            const int R = ii * ATOM + lane % ATOM;
            const int col = j * ATOM + Op::acc_row(4 * q, lane);
            // Elements 4q .. 4q+3 as one 4-vector, a subregister of the
            // accumulator tuple.  (Assembled element by element, the
            // backend copied element 4q into all four lanes of the vector.)
            const auto a4 = __builtin_shufflevector(acc[i][j], acc[i][j], 4 * q, 4 * q + 1, 4 * q + 2,
                                                    4 * q + 3);
            *(i32x4*)(stage + chunk_at(R, col / 4)) = __builtin_bit_cast(i32x4, a4);
          });
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < kRows * kPPR / 64; ++it) {
        const int qq = it * 64 + lane;
        const int rr = qq / kPPR, g = qq % kPPR;
        const int gr = row0 + wm * 128 + ps * kRows + rr;
        const int gc = col0 + wn * 128 + g * kOut;
        AccS e[kOut];
#pragma unroll
        for (int h = 0; h < kOut / 4; ++h)
          *(i32x4*)&e[4 * h] = *(const i32x4*)(stage + chunk_at(rr, g * (kOut / 4) + h));
        if (gr < M && gc < N) {
          const int64_t idx = (int64_t)gr * ldc + gc;
          if (gc + kOut <= N) {
            if constexpr (kOut == 8) store8<OUT>(C, idx, e, accumulate != 0, scale);
            else store4<OUT>(C, idx, e, accumulate != 0, scale);
          } else {
            store_n<OUT>(C, idx, e, N - gc, accumulate != 0, scale);
          }
        }
      }
      __syncthreads();
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <Elt IN, Elt OUT, bool AM, bool BM>
static hipError_t launch_w4(const GemmArgs& g, hipStream_t stream) {
  constexpr int KR = FRISK_G4_KR;
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g4::lds_bytes(KR);
  static_assert(kLds <= 160 * 1024, "LDS budget of one CU");
  auto kern = gemm_w4_kernel<IN, OUT, AM, BM, KR, FRISK_G4_ATOM>;
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

// Split-K: f32 partials of each K slice into the workspace `ws`
// ([slices][M][N]), then their sum in slice order into C (bf16 / f16
// inputs, scale 1).  (Summed inside the launch through splitk_tree instead,
// the 256x256 kernel spills registers and the tree's serial levels cost
// more than the second launch: 1024x4096x14336 in 4 slices 120 -> 174 us.)
template <Elt IN, bool AM, bool BM>
static hipError_t launch_w4_split(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                  hipStream_t stream) {
  constexpr int KR = FRISK_G4_KR;
  constexpr int kEsz = EltInfo<IN>::bytes;
  constexpr int kLds = g4::lds_bytes(KR);
  auto kern = gemm_w4_kernel<IN, Elt::F32, AM, BM, KR, FRISK_G4_ATOM>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  const int tiles = (int)(((g.m + g4::kBT - 1) / g4::kBT) * ((g.n + g4::kBT - 1) / g4::kBT));
  hipLaunchKernelGGL(kern, dim3(tiles, slices), dim3(g4::kThreads), kLds, stream, (const char*)g.a,
                     (const char*)g.b, ws, (int)g.m, (int)g.n, (int)(g.k * kEsz),
                     g.lda * kEsz, g.ldb * kEsz, g.n, 1.0f, 0, (int)kb_slice,
                     (int64_t)g.m * g.n * 4);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return gemm_splitk_sum((const float*)ws, slices, g, stream);
}

template <bool AM, bool BM>
hipError_t gemm_w4_split_layout(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                hipStream_t s) {
  if (g.in == Elt::BF16) return launch_w4_split<Elt::BF16, AM, BM>(g, slices, kb_slice, ws, s);
  if (g.in == Elt::F16) return launch_w4_split<Elt::F16, AM, BM>(g, slices, kb_slice, ws, s);
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
    case FRISK_PAIR(Elt::F32, Elt::F32): return launch_w4<Elt::F32, Elt::F32, AM, BM>(g, s);
    default: return hipErrorInvalidValue;
  }
}

#undef FRISK_PAIR

}  // namespace frisk
