// Pieces shared by the MFMA GEMM kernels (gemm.hip, gemm4w.hip): MFMA
// wrappers, the vmcnt-only wait, the 8-element epilogue store and the
// fragment bundle.
#pragma once

#include "common.h"
#include "kernels.h"

namespace frisk {

// ---------------------------------------------------------------------------
// MFMA wrappers.  kBytes = bytes of one operand row consumed by one 32x32
// MFMA; every lane supplies kBytes/2 of them (lanes 0-31 and 32-63 split the
// row), as i32x4 chunks.  A and B fragments use the same (lane, byte) -> k
// assignment, so the k order inside an instruction never matters.
// ---------------------------------------------------------------------------
template <Elt E> struct Mfma32;

template <> struct Mfma32<Elt::BF16> {
  static constexpr int kBytes = 32;
  using Acc = f32x16;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                   __builtin_bit_cast(bf16x8, b[0]), c, 0, 0, 0);
  }
};

template <> struct Mfma32<Elt::F16> {
  static constexpr int kBytes = 32;
  using Acc = f32x16;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]),
                                                  __builtin_bit_cast(f16x8, b[0]), c, 0, 0, 0);
  }
};

#ifndef FRISK_F8_SCALE
#define FRISK_F8_SCALE 0
#endif
template <> struct Mfma32<Elt::E4M3> {
  static constexpr int kBytes = 64;
  using Acc = f32x16;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    const i32x8 av = {a[0][0], a[0][1], a[0][2], a[0][3], a[1][0], a[1][1], a[1][2], a[1][3]};
    const i32x8 bv = {b[0][0], b[0][1], b[0][2], b[0][3], b[1][0], b[1][1], b[1][2], b[1][3]};
    // Format 0 = fp8 e4m3 for both operands.  Scale operands 0 select the
    // form without block scales (v_mfma_f32_32x32x64_f8f6f4: 8 bytes of
    // code instead of 16 and no scale register read per MFMA), whose
    // products are the unscaled ones that unit E8M0 scales (127 = 2^0)
    // give; the parity tests hold the products to the oracle.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, FRISK_F8_SCALE, 0,
                                                           FRISK_F8_SCALE);
  }
};

template <> struct Mfma32<Elt::I8> {
  static constexpr int kBytes = 32;
  using Acc = i32x16;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[0], c, 0, 0, 0);
  }
};

// fp32 on the matrix cores: v_mfma_f32_32x32x2_f32 takes one k per lane
// half (lanes 0-31 k = 0, lanes 32-63 k = 1), so the 16 bytes (4 floats) a
// lane holds per k-step feed four of them, float j of every lane in
// instruction j.  A and B assign k alike, so the 8 k of a k-step pair up;
// the products are exact and the sums fp32 (dense peak 157.3 TFLOP/s).
template <> struct Mfma32<Elt::F32> {
  static constexpr int kBytes = 32;
  using Acc = f32x16;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    const f32x4 av = __builtin_bit_cast(f32x4, a[0]);
    const f32x4 bv = __builtin_bit_cast(f32x4, b[0]);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], bv[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1], bv[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[2], bv[2], c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(av[3], bv[3], c, 0, 0, 0);
  }
};

// The 16x16 atoms: kBytes = bytes of one operand row consumed by one MFMA;
// every lane supplies kBytes/4 of them (four lane groups of 16 split the
// row), so a lane's share is the same 16 B (32 B for fp8) as with 32x32.
template <Elt E> struct Mfma16x;

template <> struct Mfma16x<Elt::BF16> {
  static constexpr int kBytes = 64;
  using Acc = f32x4;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                   __builtin_bit_cast(bf16x8, b[0]), c, 0, 0, 0);
  }
};

template <> struct Mfma16x<Elt::F16> {
  static constexpr int kBytes = 64;
  using Acc = f32x4;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a[0]),
                                                  __builtin_bit_cast(f16x8, b[0]), c, 0, 0, 0);
  }
};

template <> struct Mfma16x<Elt::E4M3> {
  static constexpr int kBytes = 128;
  using Acc = f32x4;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    const i32x8 av = {a[0][0], a[0][1], a[0][2], a[0][3], a[1][0], a[1][1], a[1][2], a[1][3]};
    const i32x8 bv = {b[0][0], b[0][1], b[0][2], b[0][3], b[1][0], b[1][1], b[1][2], b[1][3]};
    // Format 0 = fp8 e4m3 for both operands, no block scales (as above).
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 0, 0, 0, FRISK_F8_SCALE, 0,
                                                            FRISK_F8_SCALE);
  }
};

template <> struct Mfma16x<Elt::I8> {
  static constexpr int kBytes = 64;
  using Acc = i32x4;
  __device__ static inline Acc run(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a[0], b[0], c, 0, 0, 0);
  }
};

// The MFMA of an ATOM x ATOM output tile (32 or 16).  Lane L of a wave holds
// operand row L % ATOM and the (L / ATOM)-th of the 64 / ATOM equal K pieces
// of the instruction; accumulator element r of lane L holds output
// (acc_row(r, L), L % ATOM).
template <Elt E, int ATOM> struct MfmaAtom;
template <Elt E> struct MfmaAtom<E, 32> : Mfma32<E> {
  __device__ static inline int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
};
template <Elt E> struct MfmaAtom<E, 16> : Mfma16x<E> {
  __device__ static inline int acc_row(int r, int lane) { return 4 * (lane >> 4) + r; }
};

// s_waitcnt with only the vector-memory counter limited to n (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
#define FRISK_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Two f32 values as a packed pair of 16-bit outputs (lo in bits 0-15): one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, round to nearest even.
template <Elt OUT>
__device__ inline uint32_t pack_f32x2(float lo, float hi) {
  static_assert(OUT == Elt::BF16 || OUT == Elt::F16, "16-bit output");
  if constexpr (OUT == Elt::BF16) {
    return f32x2_to_bf16x2_bits(lo, hi);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 h = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, h);
  }
}

// Stores 8 consecutive outputs (scaled, optionally added to what C holds)
// at C[idx ..].  16-bit outputs go out as one nontemporal 16 B store per
// lane, whole 128-byte lines per 8 lanes: with every tile's epilogue landing
// at once, streaming them past the caches measured 2-3% faster end to end
// (bf16 4096^3, 8192^3).  32-bit outputs take two 16 B stores per lane,
// each covering half of every 32-byte sector; as nontemporal stores those
// cost a quarter of the int8 4096^3 throughput, so they stay ordinary.
template <Elt OUT, typename AccS>
__device__ inline void store8(void* c, int64_t idx, const AccS* v, bool accumulate, float scale) {
  if constexpr (OUT == Elt::I32) {
    int32_t* p = (int32_t*)c + idx;
    i32x4 lo = {(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
    i32x4 hi = {(int)v[4], (int)v[5], (int)v[6], (int)v[7]};
    if (accumulate) {
      lo += *(const i32x4*)p;
      hi += *(const i32x4*)(p + 4);
    }
    *(i32x4*)p = lo;
    *(i32x4*)(p + 4) = hi;
  } else if constexpr (OUT == Elt::F32) {
    float* p = (float*)c + idx;
    f32x4 lo = {v[0] * scale, v[1] * scale, v[2] * scale, v[3] * scale};
    f32x4 hi = {v[4] * scale, v[5] * scale, v[6] * scale, v[7] * scale};
    if (accumulate) {
      lo += *(const f32x4*)p;
      hi += *(const f32x4*)(p + 4);
    }
    *(f32x4*)p = lo;
    *(f32x4*)(p + 4) = hi;
  } else {
    uint16_t* p = (uint16_t*)c + idx;
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = v[i] * scale;
    if (accumulate) {
      const i32x4 old = *(const i32x4*)p;
      const uint16_t* o = (const uint16_t*)&old;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (OUT == Elt::BF16) f[i] += bf16_bits_to_f32(o[i]);
        else f[i] += (float)__builtin_bit_cast(_Float16, o[i]);
      }
    }
    i32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (int)pack_f32x2<OUT>(f[2 * i], f[2 * i + 1]);
    __builtin_nontemporal_store(r, (i32x4*)p);
  }
}

// Stores 4 consecutive outputs (scaled, optionally added to what C holds)
// at C[idx ..]: one 16-byte store of a 32-bit output, one 8-byte store of a
// 16-bit one.
template <Elt OUT, typename AccS>
__device__ inline void store4(void* c, int64_t idx, const AccS* v, bool accumulate, float scale) {
  if constexpr (OUT == Elt::I32) {
    int32_t* p = (int32_t*)c + idx;
    i32x4 r = {(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
    if (accumulate) r += *(const i32x4*)p;
    *(i32x4*)p = r;
  } else if constexpr (OUT == Elt::F32) {
    float* p = (float*)c + idx;
    f32x4 r = {v[0] * scale, v[1] * scale, v[2] * scale, v[3] * scale};
    if (accumulate) r += *(const f32x4*)p;
    *(f32x4*)p = r;
  } else {
    uint16_t* p = (uint16_t*)c + idx;
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = v[i] * scale;
    if (accumulate) {
      const i32x2 old = *(const i32x2*)p;
      const uint16_t* o = (const uint16_t*)&old;
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] += load_as_f32<OUT>(o, i);
    }
    const i32x2 r = {(int)pack_f32x2<OUT>(f[0], f[1]), (int)pack_f32x2<OUT>(f[2], f[3])};
    *(i32x2*)p = r;
  }
}

// ---------------------------------------------------------------------------
// Split-K summed inside the GEMM launch.  Every K slice of an output tile
// keeps its f32 sum in registers; the slices of a tile combine in a fixed
// binary tree over slice indices: at level L the subtree of slices
// [2g 2^L, (2g+1) 2^L) meets the subtree [(2g+1) 2^L, (2g+2) 2^L).  Each of
// the two workgroups writes its subtree's sum to the partial slot of the
// subtree's first slice and arrives at the meeting's word; the second to
// arrive reads the other sum, adds it and goes up a level, the first one is
// done.  The workgroup holding the whole sum at the root runs the
// epilogue into C.  Floating-point addition is commutative, so the result
// depends on the tree alone, not on which workgroup arrives second: the
// same inputs give the same bits on every call.  Partials are stored in
// fragment order (lane-contiguous 16-byte pieces of the accumulators), so
// both their writes and reads are whole 1 KiB rows per wave instruction.
//
// Arrival words (64 bits, one per meeting, 64 per tile): 0 or any value but
// kTreeArrived reads as "nobody has arrived"; the first arrival writes
// kTreeArrived, the second writes 0 back.  Every call therefore leaves each
// word it used at 0, whatever the workspace held before (a never-used
// workspace holds kTreeArrived in a word with probability 2^-64), and
// nothing has to be cleared between calls.
// ---------------------------------------------------------------------------
struct SplitTree {
  float* partial;                // [tiles][slices][waves][chunks][64 lanes] f32x4
  unsigned long long* arrivals;  // [tiles][kTreeWords]
  int slices;
};
constexpr unsigned long long kTreeArrived = 0x5A17C0DE00000001ull;
// The tree of `tiles` tiles of bt x bt outputs in `slices` slices over a
// workspace of split_tree_bytes (kernels.h): the partials, then the words.
inline SplitTree split_tree_at(void* ws, int64_t tiles, int slices, int bt) {
  const int64_t partial_bytes = tiles * slices * (int64_t)bt * bt * 4;
  return SplitTree{(float*)ws, (unsigned long long*)((char*)ws + partial_bytes), slices};
}
// Meeting word of level L, group g: levels take 32, 16, 8, ... words.
__device__ __host__ constexpr int tree_word(int level, int group) {
  return kTreeWords - (kTreeWords >> level) + group;
}

// An accumulator tile from its f32x4 pieces in element order (whole-vector
// shuffles: no per-element inserts into the accumulator tuple).
template <typename Acc, int N>
__device__ inline Acc join_chunks(const f32x4 (&v)[N]) {
  if constexpr (N == 1) {
    return v[0];
  } else {
    static_assert(N == 4, "f32x4 or f32x16 accumulators");
    typedef float f32x8_ __attribute__((ext_vector_type(8)));
    const f32x8_ lo = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
    const f32x8_ hi = __builtin_shufflevector(v[2], v[3], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  }
}

// Sums the accumulators of this workgroup's slice with its tile's other
// slices; true for the one workgroup per tile that then holds the total
// (every thread of a workgroup gets the same answer).  `flag` is a word of
// LDS no other wave writes until the next workgroup barrier after the call.
//
// Coherence without cache-wide operations: partials are written and read
// with device-scope (SC1) buffer accesses, which the memory system keeps
// coherent across the XCDs' L2 caches on their own, and the arrival is a
// device-scope atomic.  A writer waits for its stores to be acknowledged
// (vmcnt 0) before the workgroup barrier that precedes the arrival; a
// reader issues its loads after the barrier that follows it.  Agent-scope
// fences would order the same accesses but write back and invalidate the
// whole L2 of the XCD, which every other workgroup's operand tiles then
// miss (measured: M = 128, N = K = 4096 split 4 ways 19.4 -> 41 us).
template <int kWaves, typename Acc, int TM, int TN>
__device__ inline bool splitk_tree(Acc (&acc)[TM][TN], const SplitTree& t, int tile, int slice,
                                   int* flag) {
  constexpr int kChunks = sizeof(Acc) / 16;  // f32x4 pieces per accumulator tile
  constexpr int kQ = TM * TN * kChunks;       // per lane
  constexpr int kSlotBytes = kWaves * kQ * 64 * 16;
  constexpr int kSC1 = 0x10;                  // device-scope cache policy of a buffer access
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The tile's partial slots: [slices][waves][chunks][64 lanes] x 16 bytes.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(t.partial + (int64_t)tile * t.slices * (kSlotBytes / 4)), (short)0,
      t.slices * kSlotBytes, 0x00020000);
  const int lane_off = (wave * kQ * 64 + lane) * 16;
  for (int level = 0; (1 << level) < t.slices; ++level) {
    const int span = 1 << level;
    const int group = slice >> (level + 1);
    const int right = (2 * group + 1) * span;
    if (right >= t.slices) continue;  // no right subtree at this level: go up alone
    const int mine = (slice >> level) << level;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        static_for<0, kChunks>([&](auto cc) {
          constexpr int c = decltype(cc)::value;
          const f32x4 v =
              __builtin_shufflevector(acc[i][j], acc[i][j], 4 * c, 4 * c + 1, 4 * c + 2, 4 * c + 3);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), rs,
                                                 lane_off + ((i * TN + j) * kChunks + c) * 1024,
                                                 mine * kSlotBytes, kSC1);
        });
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0): the stores are acknowledged
    __syncthreads();
    if (tid == 0) {
      unsigned long long* w = t.arrivals + (int64_t)tile * kTreeWords + tree_word(level, group);
      unsigned long long old = 0;
      int second = 0;
      // Two workgroups meet at a word, so after one failed exchange (the
      // other arrival changed the word) the next succeeds: four attempts
      // always end.
      for (int attempt = 0; attempt < 4; ++attempt) {
        second = old == kTreeArrived;
        if (__hip_atomic_compare_exchange_strong(w, &old, second ? 0ull : kTreeArrived,
                                                 __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
          break;
      }
      *(volatile int*)flag = second;
    }
    __syncthreads();
    if (!*(volatile int*)flag) return false;
    const int other = mine == right ? mine - span : right;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        f32x4 v[kChunks];
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
          v[c] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rs, lane_off + ((i * TN + j) * kChunks + c) * 1024, other * kSlotBytes, kSC1));
        acc[i][j] += join_chunks<Acc>(v);
      }
  }
  return true;
}

// MFMA operand fragments of one k-step: TM A tiles and TN B tiles.
template <int TM, int TN, int LC>
struct Frags {
  i32x4 a[TM][LC];
  i32x4 b[TN][LC];
};

}  // namespace frisk
