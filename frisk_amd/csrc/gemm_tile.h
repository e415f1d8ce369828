// Operand tiles of the LDS-staged MFMA GEMM kernels (gemm_w4.h: 256x256
// tiles, gemm_128.h: 128x128 tiles): how one operand of one pipeline stage
// is copied from global memory into LDS and how the MFMA fragments are read
// back, for either storage order of the operand.
//
// frisk.gemm takes A as [M, K] or, with transA, stored [K, M]; B as [K, N]
// or, with transB, stored [N, K] (ffi/ir.cpp:335-337; the builder's default
// is transA = transB = false, and the reference's own GEMM tile program
// tmp/ir.mlir:2-16 keeps B as [K, N]).  Per operand that is one of:
//
//  * K-major (A with trans_a == 0, B with trans_b == 1): the stage tile is
//    BT rows (M or N indices) of KR bytes of K.  A lane's MFMA operand is 16
//    contiguous bytes of one row: one ds_read_b128.
//  * MN-major (A with trans_a == 1, B with trans_b == 0): the stage tile is
//    KR / esize k-rows of BT * esize bytes, each a contiguous piece of one
//    stored row.  A lane's MFMA operand is a run of consecutive k of one
//    column of that tile, delivered by the gfx950 transposing LDS reads.
//    Inside each group of 16 lanes,
//      ds_read_b64_tr_b16: lane j receives element j%4 of the 8 B that lanes
//                          4e + j/4 (e = 0..3) address,
//      ds_read_b64_tr_b8:  lane j receives byte j%8 of the 8 B that lanes
//                          2e + j/8 (e = 0..7) address
//    (pinned on the device by frisk_probe_lds_transpose).  So when lane
//    4e + q addresses k-row k0 + e at columns c0 + 4q .. +3 (16-bit), lane j
//    receives column c0 + j at k0 .. k0+3; two reads (k0 and k0 + 4) give
//    the 8 consecutive k of a 16-bit operand.  For 8-bit types lane 2e + b
//    addresses k-row k0 + e at columns c0 + 8b .. +7 and lane j receives 8
//    consecutive k of column c0 + j; 2 (i8) or 4 (fp8) reads give 16 or 32.
//    The k order equals the K-major ds_read_b128's, so A and B fragments
//    agree whatever the storage order of either.  32-bit types have no
//    transposing read: lane L reads its 4 consecutive k (k-rows 4 (L / 32)
//    .. +3 of a step's 8) at column L % 32 with four ds_read_b32.
//
// LDS swizzles (16 B chunk c of tile row r is stored at chunk c ^ swz(r)).
// A read is conflict-free when the lanes served together hit distinct banks
// (64 banks of 4 B: a 256 B window).
//  * K-major: a ds_read_b128 has 16 lanes per cycle reading one logical
//    chunk of 16 consecutive rows; swz sends them to 16 distinct chunks of
//    the window (rocprofv3 SQ_LDS_BANK_CONFLICT = 0 for both maps).  Both
//    are the layout target's own proposals (proposeLdsSwizzle,
//    frisk_amd/ir/layout.cpp): c ^ ((r >> 2) & 3) for 64-byte rows,
//    c ^ ((r >> 1) & 7) for 128-byte rows; frisk_gemm_plan reports them and
//    execute() checks them against the proposal.  (The 128-byte rows used
//    c ^ (r & 7) ^ ((r >> 3) & 1) before: bit-identical results, timings
//    within 1% on bf16 / fp8 / int8 at 4096^3 and 8192^3.)
//  * MN-major 16-bit (rows of 512 or 256 B): 32 lanes read 4 k-rows (e) x
//    64 B; swz(r) = (r & 3) << 2 moves row e to the 64 B quarter
//    (c / 4) ^ e, four distinct quarters.
//  * MN-major 8-bit, 256 B rows: 32 lanes read 8 k-rows x 32 B;
//    swz(r) = (r & 7) << 1 gives each row its own 32 B pair of chunks.
//  * MN-major 8-bit, 128 B rows: two rows share a window (r & 1 picks the
//    half); swz(r) = ((r >> 1) & 3) << 1 separates the four pairs of rows.
//  * MN-major 32-bit (rows of 512 or 1024 B): a ds_read_b32 has lanes 0-31
//    on 128 contiguous bytes of k-row e and lanes 32-63 on k-row 4 + e;
//    swz(r) = ((r >> 2) & 1) << 3 moves the second row 128 B over, onto the
//    other 32 banks.
// Every swizzle is an XOR of row bits into chunk bits, i.e. a GF(2)-linear
// shared layout, and only reads row bits below 3, which k-row bases
// (multiples of 8) never change.
#pragma once

#include "common.h"
#include "gemm_common.h"

namespace frisk {

template <Elt IN, bool MN, int BT, int KR, int ATOM = 32>
struct OpTile {
  using Op = MfmaAtom<IN, ATOM>;
  static constexpr int kEsz = EltInfo<IN>::bytes;
  static constexpr int kRB = MN ? BT * kEsz : KR;  // bytes per LDS row
  static constexpr int kRows = MN ? KR / kEsz : BT;
  static constexpr int kKS = KR / kEsz;            // k per stage
  static constexpr int kChunks = kRB / 16;         // 16 B chunks per LDS row
  static constexpr int kRowsPerBlock = 1024 / kRB; // rows per 1 KiB DMA block
  static constexpr int kBytes = BT * KR;           // the tile, one stage
  static constexpr int kGroups = 64 / ATOM;        // lane groups sharing one operand row
  static constexpr int kStepChunks = Op::kBytes / 16;
  static constexpr int kLaneChunks = kStepChunks / kGroups;
  static constexpr int kLaneK = Op::kBytes / kGroups / kEsz;  // k per lane per MFMA
  static constexpr int kReadsPerChunk = MN ? (kEsz == 4 ? 4 : 2) : 1;  // LDS reads per 16 B
  static_assert(kRows * kRB == kBytes && kRowsPerBlock >= 1, "tile geometry");
  static_assert(!MN || kRB >= 128, "MN-major rows of at least 128 B");
  static_assert(ATOM == 32 || ATOM == 16, "MFMA atom");
  static_assert(kEsz != 4 || ATOM == 32, "32-bit operands on 32x32 atoms");
  static_assert(KR % Op::kBytes == 0, "whole MFMA k-steps per stage");

  // For 16x16 atoms the 32 lanes served together by a transposing read
  // come from two lane groups, i.e. k-rows e and kLaneK + e (8 + e for
  // 16-bit types), so the M/N-major swizzles also fold in that row bit.
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (!MN) {
      if constexpr (KR == 128) return (r >> 1) & 7;
      else return (r >> 2) & 3;  // KR == 64
    } else if constexpr (kEsz == 4) {
      return ((r >> 2) & 1) << 3;
    } else if constexpr (kEsz == 2) {
      if constexpr (ATOM == 32) return (r & 3) << 2;
      else return ((r & 3) | (((r >> 3) & 1) << 2)) << 1;
    } else if constexpr (kRB >= 256) {
      if constexpr (ATOM == 32) return (r & 7) << 1;
      else return (r & 7) | (((r / kLaneK) & 1) << 3);
    } else {
      if constexpr (ATOM == 32) return ((r >> 1) & 3) << 1;
      else return ((r >> 1) & 3) | (((r / kLaneK) & 1) << 2);
    }
  }

  // ---- LDS-DMA ------------------------------------------------------------
  // One buffer_load ... lds instruction fills a 1 KiB block of the tile:
  // lane L lands in block row L / kChunks at physical chunk L % kChunks, so
  // it fetches logical chunk (L % kChunks) ^ swz(row).  Loads are raw buffer
  // loads based at the tile's origin; the offset 0x80000000 lies past every
  // range and reads zeros.
  //  K-major: tile origin = row0 of the operand; rows past the edge are
  //    clamped (they only feed outputs that are never stored); a chunk is
  //    live while its K bytes exist.
  //  MN-major: tile origin = column row0 of every k-row; chunks starting
  //    past the edge and k-rows past K read zeros.
  // Stage `phys` (in units of KR bytes of K) loads at off + phys * adv while
  // phys * step < lim.
  template <int NB>
  struct Dma {
    uint32_t off[NB];
    int lim[NB];
    uint32_t adv;
  };
  static constexpr int kStep = MN ? kKS : KR;

  // Global origin of the tile and the number of bytes addressable from it.
  __device__ static __forceinline__ const char* origin(const char* X, int row0, int64_t ld_b) {
    return MN ? X + (int64_t)row0 * kEsz : X + (int64_t)row0 * ld_b;
  }
  __device__ static __forceinline__ int64_t records(int extent, int row0, int Kb, int64_t ld_b) {
    if constexpr (MN) return (int64_t)(Kb / kEsz - 1) * ld_b + (int64_t)(extent - row0) * kEsz;
    else return (int64_t)(extent - 1 - row0) * ld_b + Kb;
  }

  // Block `blk` (tile-relative, 1 KiB each) of lane `lane`.
  template <int NB>
  __device__ static __forceinline__ void dma_setup(Dma<NB>& d, int i, int blk, int lane, int extent,
                                                   int row0, int Kb, int64_t ld_b) {
    const int r = blk * kRowsPerBlock + lane / kChunks;
    const int c = (lane % kChunks) ^ swz(r);
    if constexpr (MN) {
      d.off[i] = (uint32_t)(r * ld_b) + c * 16;
      const bool col_ok = (row0 + c * (16 / kEsz)) < extent;
      d.lim[i] = col_ok ? Kb / kEsz - r : 0;
    } else {
      d.off[i] = (uint32_t)(min(r, extent - 1 - row0) * ld_b) + c * 16;
      d.lim[i] = Kb - c * 16;
    }
  }
  template <int NB>
  __device__ static __forceinline__ void dma_adv(Dma<NB>& d, int64_t ld_b) {
    d.adv = MN ? (uint32_t)(kKS * ld_b) : (uint32_t)KR;
  }
  template <int NB>
  __device__ static __forceinline__ uint32_t offset(const Dma<NB>& d, int i, int phys) {
    uint32_t o = d.off[i] + (uint32_t)phys * d.adv;
    // Materialise the live offset in every lane, so that the select stays a
    // v_cndmask: otherwise the backend turns it into exec-masked code, whose
    // EXEC writes split the scheduling regions the pipeline relies on.
    asm("" : "+v"(o));
    return phys * kStep < d.lim[i] ? o : 0x80000000u;
  }
  // Bytes to advance the operand pointer by for a K slice starting kb bytes in.
  __device__ static __forceinline__ int64_t slice_shift(int64_t kb, int64_t ld_b) {
    return MN ? (kb / kEsz) * ld_b : kb;
  }

  // ---- fragment reads ------------------------------------------------------
  // Fragment of the 32 tile rows r0 .. r0+31 (r0 a multiple of 32) for lane
  // `lane`: a byte offset from the operand's stage base (plus, K-major, the
  // row's swizzle XOR the lane half's first chunk: the chunk index
  // s * kStepChunks + half * kLaneChunks + j has disjoint bit fields, so
  // XOR-ing the half in once equals adding it).
  struct Frag {
    int off, sw;
  };
  // K-major swizzles repeat every 16 rows, so tiles at r0 = 16 i share one
  // swizzle and differ by the constant r0 * KR: tile_off() adds it, and the
  // kernels keep one Frag for all K-major tiles.
  static constexpr bool kSharedFrag = !MN;
  __device__ static __forceinline__ constexpr int tile_off(int r0) { return MN ? 0 : r0 * KR; }
  __device__ static __forceinline__ Frag frag(int r0, int lane) {
    if constexpr (!MN) {
      const int row = r0 + lane % ATOM, grp = lane / ATOM;
      return Frag{row * KR, swz(lane % 16) ^ (grp * kLaneChunks)};
    } else {
      // 16-lane group G of the wave covers columns r0 + 16 dg (dg < ATOM/16)
      // at this lane group's K share kg.
      const int G = lane >> 4, dg = G % (ATOM / 16), kg = G / (ATOM / 16);
      if constexpr (kEsz == 4) {
        // Lane L: k-rows 4 (L / 32) .. +3 at column r0 + L % 32 (one
        // swizzle for the four rows: it reads row bit 2 only).
        const int col = r0 + (lane & 31), row = kLaneK * (lane >> 5);
        return Frag{row * kRB + (((col >> 2) ^ swz(row)) << 4) + 4 * (col & 3), 0};
      } else if constexpr (kEsz == 2) {
        // Lane 16G + 4e + q: k-row kLaneK kg + e, columns r0 + 16 dg + 4q.
        const int e = (lane >> 2) & 3, q = lane & 3;
        const int row = kLaneK * kg + e;
        const int chunk = ((r0 + 16 * dg) >> 3) + (q >> 1);
        return Frag{row * kRB + ((chunk ^ swz(row)) << 4) + 8 * (q & 1), 0};
      } else {
        // Lane 16G + 2e + b: k-row kLaneK kg + e, columns r0 + 16 dg + 8b.
        const int e = (lane >> 1) & 7, b = lane & 1;
        const int row = kLaneK * kg + e;
        const int chunk = (r0 + 16 * dg) >> 4;
        return Frag{row * kRB + ((chunk ^ swz(row)) << 4) + 8 * b, 0};
      }
    }
  }
  // The lane's operand of MFMA k-step s (Op::kBytes of K per row); `off` is
  // tile_off() of the tile when f is a shared (tile 0) Frag.
  __device__ static __forceinline__ void read(const char* base, const Frag& f, int s,
                                              i32x4 (&out)[kLaneChunks], int off = 0) {
    if constexpr (!MN) {
#pragma unroll
      for (int j = 0; j < kLaneChunks; ++j) {
        const int chunk = s * kStepChunks + j;
        out[j] = *(const i32x4*)(base + off + f.off + ((chunk ^ f.sw) << 4));
      }
    } else if constexpr (kEsz == 4) {
      static_assert(kLaneChunks == 1, "32-bit operand: 4 k per lane");
      const char* p = base + f.off + s * (Op::kBytes / 4) * kRB;
      out[0] = i32x4{*(const int*)p, *(const int*)(p + kRB), *(const int*)(p + 2 * kRB),
                     *(const int*)(p + 3 * kRB)};
    } else if constexpr (kEsz == 2) {
      static_assert(kLaneChunks == 1, "16-bit operand: 8 k per lane");
      const char* p = base + f.off + s * (Op::kBytes / 2) * kRB;
      const s16x4 lo = lds_read_tr16(p);
      const s16x4 hi = lds_read_tr16(p + 4 * kRB);
      const i32x2 a = __builtin_bit_cast(i32x2, lo), b = __builtin_bit_cast(i32x2, hi);
      out[0] = i32x4{a[0], a[1], b[0], b[1]};
    } else {
      const char* p = base + f.off + s * Op::kBytes * kRB;
#pragma unroll
      for (int j = 0; j < kLaneChunks; ++j) {
        const i32x2 a = lds_read_tr8(p + 16 * j * kRB);
        const i32x2 b = lds_read_tr8(p + (16 * j + 8) * kRB);
        out[j] = i32x4{a[0], a[1], b[0], b[1]};
      }
    }
  }
};

// Stores the first n (< 8) of 8 consecutive outputs at C[idx ..] one
// element at a time: the ragged last column group of a row.
template <Elt OUT, typename AccS>
__device__ inline void store_n(void* c, int64_t idx, const AccS* v, int n, bool accumulate,
                               float scale) {
  for (int e = 0; e < n; ++e) {
    if constexpr (OUT == Elt::I32) {
      int32_t* p = (int32_t*)c + idx + e;
      *p = accumulate ? *p + (int32_t)v[e] : (int32_t)v[e];
    } else {
      float f = (float)v[e] * scale;
      if (accumulate) f += load_as_f32<OUT>(c, idx + e);
      store_from_f32<OUT>(c, idx + e, f);
    }
  }
}

}  // namespace frisk
