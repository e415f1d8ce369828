// Shared device-side helpers for the gfx950 kernels: vector types, element
// conversions and the XCD-aware tile order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

namespace frisk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Element kinds the kernels are templated on (mirrors frisk_dtype).
enum class Elt : int { F32 = 0, F16 = 1, BF16 = 2, E4M3 = 3, I8 = 4, I32 = 5, F64 = 6 };

template <Elt E> struct EltInfo;
template <> struct EltInfo<Elt::F32> { using T = float; static constexpr int bytes = 4; };
template <> struct EltInfo<Elt::F16> { using T = _Float16; static constexpr int bytes = 2; };
template <> struct EltInfo<Elt::BF16> { using T = __bf16; static constexpr int bytes = 2; };
template <> struct EltInfo<Elt::E4M3> { using T = uint8_t; static constexpr int bytes = 1; };
template <> struct EltInfo<Elt::I8> { using T = int8_t; static constexpr int bytes = 1; };
template <> struct EltInfo<Elt::I32> { using T = int32_t; static constexpr int bytes = 4; };
// Element bytes of a runtime element kind.
inline int elt_bytes(Elt e) {
  switch (e) {
    case Elt::F16: case Elt::BF16: return 2;
    case Elt::E4M3: case Elt::I8: return 1;
    case Elt::F64: return 8;
    default: return 4;
  }
}

// OCP float8 e4m3fn -> f32, from the format definition: 1 sign, 4 exponent
// (bias 7), 3 mantissa bits, no infinities, S.1111.111 is NaN.
__device__ __host__ inline float e4m3_to_f32(uint8_t x) {
  const uint32_t s = x >> 7, e = (x >> 3) & 15u, m = x & 7u;
  float mag;
  if (e == 15u && m == 7u) {
    mag = __builtin_nanf("");
  } else if (e == 0u) {
    mag = (float)m * (1.0f / 512.0f);  // m * 2^-3 * 2^-6
  } else {
    mag = __builtin_ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  }
  return s ? -mag : mag;
}

// Calls f(std::integral_constant<int, i>) for i = I .. N-1, so that the body
// can use i in constant expressions (builtin arguments, array bounds).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Round-to-nearest-even f32 -> bf16 bit pattern (NaN stays a quiet NaN):
// gfx950's v_cvt_pk_bf16_f32.  (Written out in integer arithmetic, the NaN
// test compiled to exec-masked branches around every conversion, which made
// the GEMM epilogue a sixth of the 4096^3 kernel.)
__device__ inline uint16_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two f32 values as one packed pair of bf16 (lo in bits 0-15), one
// v_cvt_pk_bf16_f32.
__device__ inline uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ inline float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

template <Elt E> __device__ inline float load_as_f32(const void* p, int64_t i);
template <> __device__ inline float load_as_f32<Elt::F32>(const void* p, int64_t i) {
  return ((const float*)p)[i];
}
template <> __device__ inline float load_as_f32<Elt::F16>(const void* p, int64_t i) {
  return (float)((const _Float16*)p)[i];
}
template <> __device__ inline float load_as_f32<Elt::BF16>(const void* p, int64_t i) {
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
template <> __device__ inline float load_as_f32<Elt::E4M3>(const void* p, int64_t i) {
  return e4m3_to_f32(((const uint8_t*)p)[i]);
}

template <Elt E> __device__ inline void store_from_f32(void* p, int64_t i, float v);
template <> __device__ inline void store_from_f32<Elt::F32>(void* p, int64_t i, float v) {
  ((float*)p)[i] = v;
}
template <> __device__ inline void store_from_f32<Elt::F16>(void* p, int64_t i, float v) {
  ((_Float16*)p)[i] = (_Float16)v;
}
template <> __device__ inline void store_from_f32<Elt::BF16>(void* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}

// Maps a linear block id to a (tile_m, tile_n) pair.  Consecutive block ids
// are dispatched round-robin over the 8 XCDs of an MI355X, each with its own
// L2; the remap hands every XCD a contiguous run of tile ids, and the
// grouped raster makes that run a GROUP_M-tall patch that shares A rows and
// B columns inside one L2.
template <int GROUP_M>
__device__ inline void tile_of_block(int pid, int nblocks, int tiles_m, int tiles_n, int& tm,
                                     int& tn) {
  constexpr int kXcds = 8;
  if (nblocks % kXcds == 0) pid = (pid % kXcds) * (nblocks / kXcds) + pid / kXcds;
  const int per_group = GROUP_M * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * GROUP_M;
  const int rows = min(tiles_m - first_m, GROUP_M);
  const int in_group = pid % per_group;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// Compute units of the current device (cached per device; 256 if the
// query fails).
inline int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Transposing LDS reads through a restrict pointer.  The intrinsics carry
// no pointer information of their own beyond the address, and without an
// alias scope the waitcnt insertion makes every one of them wait for all
// LDS-DMA loads in flight (vmcnt(0)), although those write another buffer
// (the GEMM's next stage slot, attention's next K/V block): a stall of the
// whole memory latency in the middle of the loop.  The scope of the
// restrict parameter lets them issue like plain ds_read_b128 loads.  The
// true dependency (a buffer's DMA before its first read) is ordered by the
// kernels themselves: each wave waits for its own DMA (vmcnt) and a
// workgroup barrier follows, before any wave reads the buffer.
__device__ __forceinline__ s16x4 lds_read_tr16(const char* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
}
__device__ __forceinline__ i32x2 lds_read_tr8(const char* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)p);
}

}  // namespace frisk
