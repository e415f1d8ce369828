// Tile-op kernels for gfx950 on [rows, cols] tensors in HBM: the reduction
// of frisk.reduce / frisk.reduce_tensor, the element-converting copy of
// frisk.copy (and of arith.truncf / arith.extf before a tile_store) and
// frisk.fill.  All three are HBM-bound; each moves its bytes once.
//
// Reduction order.  The reference fixes one association for sums, the
// canonical_fiber_tree_v1 (lib/Dialect/Frisk/Analysis/
// ReductionLayoutProof.cpp:108-140, op contract include/Dialect/Frisk/IR/
// FriskLayoutOps.td:17-30): the inputs of one output, in order, are combined
// pairwise, adjacent nodes first, and an odd last node is carried up to the
// next level.  That tree is the complete binary tree over the index padded
// to a power of two with an identity element (-0.0 for sum: x + -0.0 == x
// for every x, +0.0 included; -inf for max; +inf for min), so one level of
// the tree is a pairwise combine along one bit of the reduced index.  The
// kernels put the low index bits on the elements of a 16-byte vector, the
// next ones on lanes and the high ones on registers or on a binary counter
// over chunks, and evaluate the levels in order: the result is bit-exact
// with the sequential definition whatever the split.  Here the inputs are
// ordered by their logical index along the reduced axis (the leaf order of
// any layout whose owners walk that axis in ascending carrier order).
//
// Arithmetic.  Sums are rounded to the element type after every addition:
// an f32 addition of two f16 (bf16) values rounded to f16 (bf16) is the
// correctly rounded f16 (bf16) sum, since f32 carries at least 2p + 2 bits.
// max / min propagate NaN and order -0.0 below +0.0 (arith.maximumf /
// minimumf), so their result is always one of the inputs.  NaN results are
// quiet NaNs with an unspecified payload.

#include "common.h"
#include "kernels.h"

namespace frisk {

namespace tile {

constexpr int kThreads = 256;

// ---- combine -------------------------------------------------------------
template <Elt E> __device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<Elt::F32>(float x) { return x; }
template <> __device__ __forceinline__ float round_to<Elt::F16>(float x) {
  return (float)(_Float16)x;
}
template <> __device__ __forceinline__ float round_to<Elt::BF16>(float x) {
  return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

template <int KIND> __device__ __forceinline__ float identity();
template <> __device__ __forceinline__ float identity<kReduceSum>() { return -0.0f; }
template <> __device__ __forceinline__ float identity<kReduceMax>() { return -__builtin_inff(); }
template <> __device__ __forceinline__ float identity<kReduceMin>() { return __builtin_inff(); }

// Symmetric in its operands (bitwise, NaN payloads aside), so a lane
// exchange can evaluate one tree node on both partners.
template <Elt E, int KIND>
__device__ __forceinline__ float combine(float a, float b) {
  if constexpr (KIND == kReduceSum) {
    return round_to<E>(a + b);
  } else {
    if (a != a || b != b) return a + b;  // quiet NaN
    const uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
    if (a == b)  // equal values; for +-0 the sign decides
      return __builtin_bit_cast(float, KIND == kReduceMax ? (ua & ub) : (ua | ub));
    if constexpr (KIND == kReduceMax) return a > b ? a : b;
    else return a < b ? a : b;
  }
}

// Binary counter over a sequence of complete, equally sized subtrees: after
// push(k, x) for k = 0..n-1, level l holds the block of 2^l subtrees for
// every set bit l of n, and finish(n) combines them from the smallest
// (rightmost) block up, which is the canonical tree over the sequence.
template <Elt E, int KIND, int L>
struct Counter {
  float lvl[L];
  // Straight-line over the levels (predicated, static indices) so that the
  // levels stay in registers.
  __device__ __forceinline__ void push(uint32_t k, float x) {
    bool carry = true;
#pragma unroll
    for (int l = 0; l < L; ++l) {
      const bool merge = carry && ((k >> l) & 1u);
      if (carry && !merge) lvl[l] = x;
      if (merge) x = combine<E, KIND>(lvl[l], x);
      carry = merge;
    }
  }
  __device__ __forceinline__ float finish(uint32_t n) const {
    float t = identity<KIND>();
    bool have = false;
#pragma unroll
    for (int l = 0; l < L; ++l) {
      if ((n >> l) & 1u) {
        t = have ? combine<E, KIND>(lvl[l], t) : lvl[l];
        have = true;
      }
    }
    return t;
  }
};

template <Elt E> __device__ __forceinline__ float load_elt(const void* p, int64_t i) {
  return load_as_f32<E>(p, i);
}

// The pairwise tree over V consecutive elements starting at column c (the
// lowest log2(V) levels); columns at or past `cols` are the identity.
template <Elt E, int KIND, int V>
__device__ __forceinline__ float slot_tree(const void* row, int64_t c, int64_t cols, bool vec_ok) {
  float x[V];
  if (vec_ok && c + V <= cols) {
    if constexpr (E == Elt::F32) {
      static_assert(V == 4, "f32 slot");
      const f32x4 v = *(const f32x4*)((const float*)row + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = v[i];
    } else {
      static_assert(V == 8, "16-bit slot");
      const i32x4 v = *(const i32x4*)((const uint16_t*)row + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = (uint32_t)v[i];
        if constexpr (E == Elt::BF16) {
          x[2 * i] = bf16_bits_to_f32((uint16_t)(w & 0xffffu));
          x[2 * i + 1] = bf16_bits_to_f32((uint16_t)(w >> 16));
        } else {
          x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
          x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) x[i] = c + i < cols ? load_elt<E>(row, c + i) : identity<KIND>();
  }
#pragma unroll
  for (int w = 1; w < V; w <<= 1)
#pragma unroll
    for (int i = 0; i < V; i += 2 * w) x[i] = combine<E, KIND>(x[i], x[i + w]);
  return x[0];
}

}  // namespace tile

// ---- axis 1: reduce along the contiguous dimension ---------------------------
// A row is split into chunks of S = LPR * R * V columns.  Within a chunk,
// column c = k S + (r LPR + lane) V + e: vector elements e are the lowest
// index bits, then the LPR lanes of the row's lane group, then the R
// registers.  Loads are coalesced across lanes for each r.  Chunk roots
// (complete subtrees of S columns, the last one padded) go through a binary
// counter.  A wave holds 64 / LPR rows.
template <Elt E, int KIND, int R>
__global__ __launch_bounds__(tile::kThreads) void reduce_rows_kernel(
    const void* __restrict__ src, int64_t ld, int64_t rows, int64_t cols, void* __restrict__ dst,
    int64_t dst_stride, int clear, int lpr_log2, int vec_ok, uint32_t chunks) {
  using namespace tile;
  constexpr int V = 16 / EltInfo<E>::bytes;
  const int lane = threadIdx.x & 63;
  const int lpr = 1 << lpr_log2;
  const int lr = lane & (lpr - 1);
  const int64_t row =
      ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * (64 >> lpr_log2) +
      (lane >> lpr_log2);
  const bool live = row < rows;
  const char* rp = (const char*)src + (live ? row : 0) * ld * EltInfo<E>::bytes;
  const int64_t span = live ? cols : 0;  // dead rows load nothing
  const int64_t S = (int64_t)lpr * R * V;

  Counter<E, KIND, 24> ctr;
  // Every lane runs the same trip count: the lane exchanges need the whole
  // wave.
  for (uint32_t k = 0; k < chunks; ++k) {
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      v[r] = slot_tree<E, KIND, V>(rp, (int64_t)k * S + ((int64_t)r * lpr + lr) * V, span,
                                   vec_ok != 0);
    for (int j = 0; j < lpr_log2; ++j) {
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = combine<E, KIND>(v[r], __shfl_xor(v[r], 1 << j, 64));
    }
#pragma unroll
    for (int w = 1; w < R; w <<= 1)
#pragma unroll
      for (int r = 0; r < R; r += 2 * w) v[r] = combine<E, KIND>(v[r], v[r + w]);
    ctr.push(k, v[0]);
  }
  float res = ctr.finish(chunks);
  if (live && lr == 0) {
    if (!clear) res = combine<E, KIND>(load_as_f32<E>(dst, row * dst_stride), res);
    store_from_f32<E>(dst, row * dst_stride, res);
  }
}

// ---- axis 0: reduce across rows -------------------------------------------------
// A workgroup of 1024 threads owns CVB slots of 4 adjacent columns; its
// 1024 / CVB row groups each take an aligned block of B = 2^b_log2 rows
// (B >= 8).  The grid has one workgroup per column strip only, so the large
// workgroup is what keeps enough loads in flight (16 waves per CU).  A thread walks
// its block eight rows at a time: the eight-row subtree is built in
// registers and pushed into a binary counter.  The block roots (complete
// subtrees; an empty block is the identity) are combined in LDS by the
// pairwise tree over the row groups.
constexpr int kColThreads = 1024;

template <Elt E, int KIND>
__global__ __launch_bounds__(kColThreads) void reduce_cols_kernel(
    const void* __restrict__ src, int64_t ld, int64_t rows, int64_t cols, void* __restrict__ dst,
    int64_t dst_stride, int clear, int cvb_log2, int b_log2, int vec_ok) {
  using namespace tile;
  constexpr int kEsz = EltInfo<E>::bytes;
  __shared__ float part[kColThreads * 4];
  const int tid = threadIdx.x;
  const int cvb = 1 << cvb_log2;
  const int cs = tid & (cvb - 1), g = tid >> cvb_log2;
  const int groups = kColThreads >> cvb_log2;
  const int64_t c0 = ((int64_t)blockIdx.x * cvb + cs) * 4;
  const int64_t r0 = (int64_t)g << b_log2;
  const int64_t r1 = min(rows, r0 + ((int64_t)1 << b_log2));
  const bool full = vec_ok && c0 + 4 <= cols;

  Counter<E, KIND, 18> ctr[4];
  uint32_t n8 = 0;
  for (int64_t i0 = r0; i0 < r1; i0 += 8, ++n8) {
    float x[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = i0 + i;
      const char* rp = (const char*)src + r * ld * kEsz;
      if (r < r1 && full) {
        if constexpr (E == Elt::F32) {
          const f32x4 v = *(const f32x4*)((const float*)rp + c0);
#pragma unroll
          for (int j = 0; j < 4; ++j) x[i][j] = v[j];
        } else {
          const uint2 v = *(const uint2*)((const uint16_t*)rp + c0);
          const uint32_t w[2] = {v.x, v.y};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
            x[i][j] = E == Elt::BF16 ? bf16_bits_to_f32(h)
                                     : (float)__builtin_bit_cast(_Float16, h);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          x[i][j] = r < r1 && c0 + j < cols ? load_as_f32<E>(rp, c0 + j) : identity<KIND>();
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int w = 1; w < 8; w <<= 1)
#pragma unroll
        for (int i = 0; i < 8; i += 2 * w) x[i][j] = combine<E, KIND>(x[i][j], x[i + w][j]);
      ctr[j].push(n8, x[0][j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    part[(g * cvb + cs) * 4 + j] = n8 ? ctr[j].finish(n8) : identity<KIND>();
  __syncthreads();
  // The pairwise tree over the row groups, one level at a time across the
  // workgroup: at level w group g (a multiple of 2w) takes in group g + w.
  // The same combines as a serial walk, so the same bits; serially, one
  // group's threads spent about 60 us on 128 groups' chains of dependent
  // LDS accesses (33 x 777 f16).
  for (int w = 1; w < groups; w <<= 1) {
    if ((g & (2 * w - 1)) == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        part[(g * cvb + cs) * 4 + j] = combine<E, KIND>(part[(g * cvb + cs) * 4 + j],
                                                        part[((g + w) * cvb + cs) * 4 + j]);
    }
    __syncthreads();
  }
  if (g == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + j;
      if (c < cols) {
        float res = part[cs * 4 + j];
        if (!clear) res = combine<E, KIND>(load_as_f32<E>(dst, c * dst_stride), res);
        store_from_f32<E>(dst, c * dst_stride, res);
      }
    }
  }
}

// ---- axis 0 in two passes ----------------------------------------------------------
// Pass 1: workgroup (strip, block) reduces rows [block B, (block + 1) B) of a
// strip of 4 * SPS columns (SPS = 2^sps_log2 <= 256 four-column slots, one
// per lane along the columns, so a row segment of up to 4 KiB is read
// contiguously by the whole workgroup); the 256 / SPS row groups each take
// B / groups consecutive rows.  Group roots are combined by the pairwise
// tree over the groups in LDS, and the block root (a complete subtree of B
// rows; the last block padded) goes to the workspace as
// partial[block][column].  Pass 2 combines the partials of each column in
// block order through a binary counter.
template <Elt E, int KIND>
__global__ __launch_bounds__(tile::kThreads) void reduce_cols_blocks_kernel(
    const void* __restrict__ src, int64_t ld, int64_t rows, int64_t cols, int sps_log2,
    int b_log2, float* __restrict__ partial, int vec_ok) {
  using namespace tile;
  constexpr int kEsz = EltInfo<E>::bytes;
  __shared__ float part[kThreads * 4];
  const int tid = threadIdx.x;
  const int sps = 1 << sps_log2;
  const int cs = tid & (sps - 1), g = tid >> sps_log2;
  const int groups = kThreads >> sps_log2;
  const int64_t c0 = ((int64_t)blockIdx.x * sps + cs) * 4;
  const int64_t gb = ((int64_t)1 << b_log2) / groups;  // rows per group, >= 8
  const int64_t r0 = ((int64_t)blockIdx.y << b_log2) + g * gb;
  const int64_t r1 = min(rows, r0 + gb);
  // Four-element vector loads need the source and its rows aligned to them
  // (element-aligned views such as x[:, 1:] take element loads).
  const bool full = vec_ok && c0 + 4 <= cols;

  // gb <= 2^12 (cols_split), so a group pushes at most 2^9 eight-row subtrees.
  Counter<E, KIND, 10> ctr[4];
  uint32_t n8 = 0;
  for (int64_t i0 = r0; i0 < r1; i0 += 8, ++n8) {
    float x[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = i0 + i;
      const char* rp = (const char*)src + r * ld * kEsz;
      if (r < r1 && full) {
        if constexpr (E == Elt::F32) {
          const f32x4 v = *(const f32x4*)((const float*)rp + c0);
#pragma unroll
          for (int j = 0; j < 4; ++j) x[i][j] = v[j];
        } else {
          const uint2 v = *(const uint2*)((const uint16_t*)rp + c0);
          const uint32_t w[2] = {v.x, v.y};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
            x[i][j] = E == Elt::BF16 ? bf16_bits_to_f32(h) : (float)__builtin_bit_cast(_Float16, h);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          x[i][j] = r < r1 && c0 + j < cols ? load_as_f32<E>(rp, c0 + j) : identity<KIND>();
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int w = 1; w < 8; w <<= 1)
#pragma unroll
        for (int i = 0; i < 8; i += 2 * w) x[i][j] = combine<E, KIND>(x[i][j], x[i + w][j]);
      ctr[j].push(n8, x[0][j]);
    }
  }
  if (groups == 1) {  // no exchange needed
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c0 + j < cols)
        partial[(int64_t)blockIdx.y * cols + c0 + j] = n8 ? ctr[j].finish(n8) : identity<KIND>();
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) part[(g * sps + cs) * 4 + j] = n8 ? ctr[j].finish(n8) : identity<KIND>();
  __syncthreads();
  // The pairwise tree over the row groups, a level at a time (as in
  // reduce_cols_kernel).
  for (int w = 1; w < groups; w <<= 1) {
    if ((g & (2 * w - 1)) == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        part[(g * sps + cs) * 4 + j] =
            combine<E, KIND>(part[(g * sps + cs) * 4 + j], part[((g + w) * sps + cs) * 4 + j]);
    }
    __syncthreads();
  }
  if (g == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c0 + j < cols) partial[(int64_t)blockIdx.y * cols + c0 + j] = part[cs * 4 + j];
  }
}

template <Elt E, int KIND>
__global__ __launch_bounds__(tile::kThreads) void reduce_cols_final_kernel(
    const float* __restrict__ partial, int64_t cols, uint32_t blocks, void* __restrict__ dst,
    int64_t dst_stride, int clear) {
  using namespace tile;
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  Counter<E, KIND, 24> ctr;
  uint32_t b = 0;
  for (; b + 8 <= blocks; b += 8) {  // eight loads in flight, then their pushes
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = partial[(int64_t)(b + i) * cols + c];
#pragma unroll
    for (int i = 0; i < 8; ++i) ctr.push(b + i, v[i]);
  }
  for (; b < blocks; ++b) ctr.push(b, partial[(int64_t)b * cols + c]);
  float res = ctr.finish(blocks);
  if (!clear) res = combine<E, KIND>(load_as_f32<E>(dst, c * dst_stride), res);
  store_from_f32<E>(dst, c * dst_stride, res);
}

// ---- any axis, permuted leaf order ------------------------------------------------
// The tree over 2^nb leaves in which leaf position p holds reduced index
// sum_j bit_j(p) << order[j] (the fiber order of a distributed layout whose
// reduced-axis bits sit on single carrier bits, sorted by carrier).  One
// thread per output walks the positions in order through a binary counter;
// threads of a wave take consecutive outputs.  Used for tile-sized
// reductions whose fibers are not in ascending index order.
struct LeafOrder {
  uint8_t bit[32];
};

template <Elt E, int KIND>
__global__ __launch_bounds__(tile::kThreads) void reduce_perm_kernel(
    const void* __restrict__ src, int64_t ld, int64_t outputs, int axis, int nb, LeafOrder order,
    void* __restrict__ dst, int64_t dst_stride, int clear) {
  using namespace tile;
  const int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (o >= outputs) return;
  Counter<E, KIND, 32> ctr;
  const uint32_t n = 1u << nb;
  for (uint32_t p = 0; p < n; ++p) {
    int64_t idx = 0;
    for (int j = 0; j < nb; ++j) idx |= (int64_t)((p >> j) & 1u) << order.bit[j];
    const int64_t off = axis == 1 ? o * ld + idx : idx * ld + o;
    ctr.push(p, load_as_f32<E>(src, off));
  }
  float res = ctr.finish(n);
  if (!clear) res = combine<E, KIND>(load_as_f32<E>(dst, o * dst_stride), res);
  store_from_f32<E>(dst, o * dst_stride, res);
}

// ---- copy with element conversion ------------------------------------------------
namespace tile {

// f32 -> OCP e4m3fn, round to nearest even; magnitudes that round past 448
// (above 464) and NaN become NaN (S.1111.111): the format has no infinity.
__device__ __forceinline__ uint8_t f32_to_e4m3_bits(float f) {
  const uint8_t s = (__builtin_bit_cast(uint32_t, f) >> 24) & 0x80u;
  const float a = __builtin_fabsf(f);
  if (!(a <= 464.0f)) return s | 0x7fu;  // NaN, +-inf, overflow
  if (a < 0.015625f) {                   // below 2^-6: multiples of 2^-9
    return s | (uint8_t)__builtin_rintf(a * 512.0f);  // 8 -> 0x08, the least normal
  }
  int e;
  const float m = __builtin_frexpf(a, &e);  // a = m 2^e, m in [0.5, 1)
  int q = (int)__builtin_rintf((m * 2.0f - 1.0f) * 8.0f);
  int ef = e - 1 + 7;
  if (q == 8) {
    q = 0;
    ++ef;
  }
  return s | (uint8_t)((ef << 3) | q);
}

template <Elt D> __device__ __forceinline__ void put(void* p, int64_t i, float v);
template <> __device__ __forceinline__ void put<Elt::F32>(void* p, int64_t i, float v) {
  ((float*)p)[i] = v;
}
template <> __device__ __forceinline__ void put<Elt::F16>(void* p, int64_t i, float v) {
  ((_Float16*)p)[i] = (_Float16)v;
}
template <> __device__ __forceinline__ void put<Elt::BF16>(void* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}
template <> __device__ __forceinline__ void put<Elt::E4M3>(void* p, int64_t i, float v) {
  ((uint8_t*)p)[i] = f32_to_e4m3_bits(v);
}

// Eight elements as raw bits, for vector loads and stores of 8 * esize bytes.
template <int BYTES> struct Raw8;
template <> struct Raw8<1> { using T = uint2; };
template <> struct Raw8<2> { using T = i32x4; };
template <> struct Raw8<4> { using T = i32x8; };
template <> struct Raw8<8> { using T = i32x16; };

template <Elt E> __device__ __forceinline__ float elt_of(const void* raw, int i) {
  return load_as_f32<E>(raw, i);
}

template <Elt D> __device__ __forceinline__ void convert8(const float* x, void* raw) {
#pragma unroll
  for (int i = 0; i < 8; ++i) put<D>(raw, i, x[i]);
}

constexpr int kSlots = 4;  // 8-element slots per thread

}  // namespace tile

// Slot s of row r holds columns [8 s, 8 s + 8).  Thread t of block x works
// on slots (x kSlots + u) 256 + t, u < kSlots, of rows y, y + gridDim.y, ...
template <Elt S, Elt D>
__global__ __launch_bounds__(tile::kThreads) void copy_convert_kernel(
    const void* __restrict__ src, int64_t ld_src, void* __restrict__ dst, int64_t ld_dst,
    int64_t rows, int64_t cols, int vec_ok) {
  using namespace tile;
  constexpr int kSe = EltInfo<S>::bytes, kDe = EltInfo<D>::bytes;
  using SRaw = typename Raw8<kSe>::T;
  using DRaw = typename Raw8<kDe>::T;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const char* sp = (const char*)src + r * ld_src * kSe;
    char* dp = (char*)dst + r * ld_dst * kDe;
    SRaw in[kSlots];
    // Loads first, conversions and stores after: kSlots loads in flight.
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int64_t c = ((int64_t)(blockIdx.x * kSlots + u) * kThreads + threadIdx.x) * 8;
      if (vec_ok && c + 8 <= cols) in[u] = *(const SRaw*)(sp + c * kSe);
    }
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int64_t c = ((int64_t)(blockIdx.x * kSlots + u) * kThreads + threadIdx.x) * 8;
      if (c >= cols) continue;
      float x[8];
      if (vec_ok && c + 8 <= cols) {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = elt_of<S>(&in[u], i);
        DRaw out;
        convert8<D>(x, &out);
        *(DRaw*)(dp + c * kDe) = out;
      } else {
        for (int i = 0; i < 8 && c + i < cols; ++i) put<D>(dp, c + i, load_as_f32<S>(sp, c + i));
      }
    }
  }
}

// Same-type copy of BYTES-wide elements (any dtype), same slot scheme.
template <int BYTES>
__global__ __launch_bounds__(tile::kThreads) void copy_raw_kernel(
    const void* __restrict__ src, int64_t ld_src, void* __restrict__ dst, int64_t ld_dst,
    int64_t rows, int64_t cols, int vec_ok) {
  using namespace tile;
  using Raw = typename Raw8<BYTES>::T;
  using Word = typename std::conditional<
      BYTES == 1, uint8_t,
      typename std::conditional<BYTES == 2, uint16_t,
                                typename std::conditional<BYTES == 4, uint32_t,
                                                          uint64_t>::type>::type>::type;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const Word* sp = (const Word*)((const char*)src + r * ld_src * BYTES);
    Word* dp = (Word*)((char*)dst + r * ld_dst * BYTES);
    Raw in[kSlots];
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int64_t c = ((int64_t)(blockIdx.x * kSlots + u) * kThreads + threadIdx.x) * 8;
      if (vec_ok && c + 8 <= cols) in[u] = *(const Raw*)(sp + c);
    }
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int64_t c = ((int64_t)(blockIdx.x * kSlots + u) * kThreads + threadIdx.x) * 8;
      if (c >= cols) continue;
      if (vec_ok && c + 8 <= cols) {
        *(Raw*)(dp + c) = in[u];
      } else {
        for (int i = 0; i < 8 && c + i < cols; ++i) dp[c + i] = sp[c + i];
      }
    }
  }
}

// Fill with a BYTES-wide bit pattern, same slot scheme.
template <int BYTES>
__global__ __launch_bounds__(tile::kThreads) void fill_kernel(void* __restrict__ dst, int64_t ld,
                                                              int64_t rows, int64_t cols,
                                                              uint64_t bits, int vec_ok) {
  using namespace tile;
  using Raw = typename Raw8<BYTES>::T;
  using Word = typename std::conditional<
      BYTES == 1, uint8_t,
      typename std::conditional<BYTES == 2, uint16_t,
                                typename std::conditional<BYTES == 4, uint32_t,
                                                          uint64_t>::type>::type>::type;
  Raw pat;
  Word* pw = (Word*)&pat;
#pragma unroll
  for (int i = 0; i < 8; ++i) pw[i] = (Word)bits;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    Word* dp = (Word*)((char*)dst + r * ld * BYTES);
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int64_t c = ((int64_t)(blockIdx.x * kSlots + u) * kThreads + threadIdx.x) * 8;
      if (c >= cols) continue;
      if (vec_ok && c + 8 <= cols) {
        *(Raw*)(dp + c) = pat;
      } else {
        for (int i = 0; i < 8 && c + i < cols; ++i) dp[c + i] = (Word)bits;
      }
    }
  }
}

// ---- launchers ------------------------------------------------------------------------

namespace {

int ilog2(int64_t x) {
  int l = 0;
  while (((int64_t)1 << l) < x) ++l;
  return l;
}

bool aligned(const void* p, int64_t ld_bytes, int a) {
  return ((uintptr_t)p % a) == 0 && ld_bytes % a == 0;
}

}  // namespace

ColsSplit cols_split(int64_t rows, int64_t cols) {
  // One round of workgroups: pass 1 holds about 104 VGPRs, so 4 workgroups
  // of 256 threads are resident per CU and 1024 fill the 256 CUs.  A sweep
  // on 8192 x 16384 f32 (strips of 64 .. 1024 columns, row blocks of 8 ..
  // 2^16 rows) peaked at exactly 1024 workgroups (4.0 TB/s; 2048 gave 3.7,
  // 512 gave 2.6) with strips of 64 or 128 columns, whose 16 or 8 row groups
  // keep each thread on a long run of rows.
  ColsSplit sp;
  const int64_t slots = (cols + 3) / 4;
  sp.sps_log2 = ilog2(slots) < 5 ? ilog2(slots) : 5;
  const int g_log2 = 8 - sp.sps_log2;  // log2 of the row groups
  sp.strips = (slots + ((int64_t)1 << sp.sps_log2) - 1) >> sp.sps_log2;
  const int64_t want_blocks = sp.strips >= 1024 ? 1 : 1024 / sp.strips;
  sp.b_log2 = ilog2((rows + want_blocks - 1) / want_blocks);
  if (sp.b_log2 < 3 + g_log2) sp.b_log2 = 3 + g_log2;
  if (sp.b_log2 > 12 + g_log2) sp.b_log2 = 12 + g_log2;
  sp.blocks = (rows + ((int64_t)1 << sp.b_log2) - 1) >> sp.b_log2;
  return sp;
}

namespace {

template <Elt E, int KIND>
hipError_t reduce_typed(const ReduceArgs& a, hipStream_t s) {
  constexpr int kEsz = EltInfo<E>::bytes;
  if (a.order_bits > 0) {
    LeafOrder ord;
    for (int j = 0; j < 32; ++j) ord.bit[j] = j < a.order_bits ? a.order[j] : 0;
    const int64_t outputs = a.axis == 1 ? a.rows : a.cols;
    const dim3 grid((unsigned)((outputs + tile::kThreads - 1) / tile::kThreads));
    hipLaunchKernelGGL((reduce_perm_kernel<E, KIND>), grid, dim3(tile::kThreads), 0, s, a.src,
                       a.ld, outputs, a.axis, a.order_bits, ord, a.dst, a.dst_stride, a.clear);
    return hipGetLastError();
  }
  if (a.axis == 1) {
    constexpr int V = 16 / kEsz;
    const int64_t slots = (a.cols + V - 1) / V;
    const int pl = ilog2(slots);  // log2 of the padded slot count
    const int lpr_log2 = pl < 6 ? pl : 6;
    const int r_log2 = pl - 6 > 3 ? 3 : (pl > 6 ? pl - 6 : 0);
    const int64_t S = ((int64_t)1 << (lpr_log2 + r_log2)) * V;
    const uint32_t chunks = (uint32_t)((a.cols + S - 1) / S);
    const int vec_ok = aligned(a.src, a.ld * kEsz, 16);
    const int64_t rows_per_block = (int64_t)(tile::kThreads / 64) << (6 - lpr_log2);
    const dim3 grid((unsigned)((a.rows + rows_per_block - 1) / rows_per_block));
#define FRISK_ROWS(R)                                                                        \
  hipLaunchKernelGGL((reduce_rows_kernel<E, KIND, R>), grid, dim3(tile::kThreads), 0, s, a.src, \
                     a.ld, a.rows, a.cols, a.dst, a.dst_stride, a.clear, lpr_log2, vec_ok, chunks)
    switch (r_log2) {
      case 0: FRISK_ROWS(1); break;
      case 1: FRISK_ROWS(2); break;
      case 2: FRISK_ROWS(4); break;
      default: FRISK_ROWS(8); break;
    }
#undef FRISK_ROWS
  } else if (a.workspace) {
    const ColsSplit sp = cols_split(a.rows, a.cols);
    const int vec_ok = aligned(a.src, a.ld * kEsz, 4 * kEsz);
    hipLaunchKernelGGL((reduce_cols_blocks_kernel<E, KIND>), dim3(sp.strips, sp.blocks),
                       dim3(tile::kThreads), 0, s, a.src, a.ld, a.rows, a.cols, sp.sps_log2,
                       sp.b_log2, (float*)a.workspace, vec_ok);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((reduce_cols_final_kernel<E, KIND>),
                       dim3((unsigned)((a.cols + tile::kThreads - 1) / tile::kThreads)),
                       dim3(tile::kThreads), 0, s, (const float*)a.workspace, a.cols,
                       (uint32_t)sp.blocks, a.dst, a.dst_stride, a.clear);
  } else {
    const int64_t slots = (a.cols + 3) / 4;
    // Widest column strip (best coalescing) that still yields >= 1024
    // workgroups; at least 8 slots (128 B of f32 per row) when there are
    // that many columns.
    int cvb_log2 = 6;
    while (cvb_log2 > 3 && (slots + (1 << cvb_log2) - 1) >> cvb_log2 < 1024) --cvb_log2;
    const int pl = ilog2(slots);
    if (pl < cvb_log2) cvb_log2 = pl;
    const int groups = kColThreads >> cvb_log2;
    int b_log2 = ilog2((a.rows + groups - 1) / groups);
    if (b_log2 < 3) b_log2 = 3;
    const int vec_ok = aligned(a.src, a.ld * kEsz, 4 * kEsz);
    const dim3 grid((unsigned)((slots + (1 << cvb_log2) - 1) >> cvb_log2));
    hipLaunchKernelGGL((reduce_cols_kernel<E, KIND>), grid, dim3(kColThreads), 0, s, a.src,
                       a.ld, a.rows, a.cols, a.dst, a.dst_stride, a.clear, cvb_log2, b_log2,
                       vec_ok);
  }
  return hipGetLastError();
}

template <Elt E>
hipError_t reduce_kind(const ReduceArgs& a, hipStream_t s) {
  switch (a.kind) {
    case kReduceSum: return reduce_typed<E, kReduceSum>(a, s);
    case kReduceMax: return reduce_typed<E, kReduceMax>(a, s);
    case kReduceMin: return reduce_typed<E, kReduceMin>(a, s);
    default: return hipErrorInvalidValue;
  }
}

dim3 slot_grid(int64_t rows, int64_t cols) {
  const int64_t per_block = (int64_t)tile::kThreads * tile::kSlots * 8;
  return dim3((unsigned)((cols + per_block - 1) / per_block),
              (unsigned)(rows < 65535 ? rows : 65535));
}

template <Elt S, Elt D>
hipError_t copy_typed(const CopyArgs& a, hipStream_t s) {
  constexpr int kSe = EltInfo<S>::bytes, kDe = EltInfo<D>::bytes;
  const int vec_ok = aligned(a.src, a.ld_src * kSe, 8 * kSe < 16 ? 8 * kSe : 16) &&
                     aligned(a.dst, a.ld_dst * kDe, 8 * kDe < 16 ? 8 * kDe : 16);
  hipLaunchKernelGGL((copy_convert_kernel<S, D>), slot_grid(a.rows, a.cols),
                     dim3(tile::kThreads), 0, s, a.src, a.ld_src, a.dst, a.ld_dst, a.rows, a.cols,
                     vec_ok);
  return hipGetLastError();
}

template <Elt S>
hipError_t copy_from(const CopyArgs& a, hipStream_t s) {
  switch (a.dst_t) {
    case Elt::F32: return copy_typed<S, Elt::F32>(a, s);
    case Elt::F16: return copy_typed<S, Elt::F16>(a, s);
    case Elt::BF16: return copy_typed<S, Elt::BF16>(a, s);
    case Elt::E4M3: return copy_typed<S, Elt::E4M3>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <int BYTES>
hipError_t copy_raw(const CopyArgs& a, hipStream_t s) {
  const int va = 8 * BYTES < 16 ? 8 * BYTES : 16;
  const int vec_ok = aligned(a.src, a.ld_src * BYTES, va) && aligned(a.dst, a.ld_dst * BYTES, va);
  hipLaunchKernelGGL((copy_raw_kernel<BYTES>), slot_grid(a.rows, a.cols), dim3(tile::kThreads), 0,
                     s, a.src, a.ld_src, a.dst, a.ld_dst, a.rows, a.cols, vec_ok);
  return hipGetLastError();
}

template <int BYTES>
hipError_t fill_bytes(const FillArgs& a, hipStream_t s) {
  const int va = 8 * BYTES < 16 ? 8 * BYTES : 16;
  const int vec_ok = aligned(a.dst, a.ld * BYTES, va);
  hipLaunchKernelGGL((fill_kernel<BYTES>), slot_grid(a.rows, a.cols), dim3(tile::kThreads), 0, s,
                     a.dst, a.ld, a.rows, a.cols, a.bits, vec_ok);
  return hipGetLastError();
}

}  // namespace

hipError_t tile_reduce(const ReduceArgs& a, hipStream_t s) {
  switch (a.dtype) {
    case Elt::F32: return reduce_kind<Elt::F32>(a, s);
    case Elt::F16: return reduce_kind<Elt::F16>(a, s);
    case Elt::BF16: return reduce_kind<Elt::BF16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t tile_copy(const CopyArgs& a, hipStream_t s) {
  if (a.src_t == a.dst_t) {
    switch (a.esize) {
      case 1: return copy_raw<1>(a, s);
      case 2: return copy_raw<2>(a, s);
      case 4: return copy_raw<4>(a, s);
      case 8: return copy_raw<8>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (a.src_t) {
    case Elt::F32: return copy_from<Elt::F32>(a, s);
    case Elt::F16: return copy_from<Elt::F16>(a, s);
    case Elt::BF16: return copy_from<Elt::BF16>(a, s);
    case Elt::E4M3: return copy_from<Elt::E4M3>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t tile_fill(const FillArgs& a, hipStream_t s) {
  switch (a.esize) {
    case 1: return fill_bytes<1>(a, s);
    case 2: return fill_bytes<2>(a, s);
    case 4: return fill_bytes<4>(a, s);
    case 8: return fill_bytes<8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace frisk
