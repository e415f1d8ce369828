// MFMA fragment-layout probe: runs one MFMA atom per k0 on index-encoded
// operands so the host can read back which (row, column) of the product each
// accumulator register of each lane holds.
//
// Operands follow the fragment maps the GEMM and attention kernels use: lane
// L supplies row (or column) L % M of the atom at k = (K / (64 / M)) (L / M)
// + e for its e-th element.  With A[i][k0] = i, A[i][k1] = S, B[k0][j] = 1,
// B[k1][j] = j (k1 = k0 + 1 mod K, S = 64 for bf16 / 32 for i8), every
// product element equals i + S j, which encodes its own coordinates exactly
// (the values are exact in bf16 / i8 and in the f32 / i32 accumulators).
// Sweeping k0 over all K values also checks that A and B slots are paired
// consistently for every k.

#include "common.h"
#include "kernels.h"

namespace frisk {

namespace {

__device__ inline __bf16 as_bf16(float v) {
  return __builtin_bit_cast(__bf16, f32_to_bf16_bits(v));
}

template <int M, int K>
__global__ __launch_bounds__(64) void probe_bf16(float* out) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int kPer = M * K / 64;  // elements per lane
  constexpr int kAcc = M * M / 64;  // accumulators per lane
  const int lane = threadIdx.x;
  const int mn = lane % M;
  for (int k0 = 0; k0 < K; ++k0) {
    const int k1 = (k0 + 1) % K;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int k = kPer * (lane / M) + e;
      a[e] = as_bf16(k == k0 ? (float)mn : (k == k1 ? 64.0f : 0.0f));
      b[e] = as_bf16(k == k0 ? 1.0f : (k == k1 ? (float)mn : 0.0f));
    }
    if constexpr (M == 32) {
      f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, f32x16{}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < kAcc; ++r) out[(k0 * 64 + lane) * kAcc + r] = c[r];
    } else {
      f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, f32x4{}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < kAcc; ++r) out[(k0 * 64 + lane) * kAcc + r] = c[r];
    }
  }
#endif
}

__global__ __launch_bounds__(64) void probe_i8_32(float* out) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int K = 32, kPer = 16;
  const int lane = threadIdx.x;
  const int mn = lane % 32;
  for (int k0 = 0; k0 < K; ++k0) {
    const int k1 = (k0 + 1) % K;
    int8_t a[kPer], b[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int k = kPer * (lane / 32) + e;
      a[e] = (int8_t)(k == k0 ? mn : (k == k1 ? 32 : 0));
      b[e] = (int8_t)(k == k0 ? 1 : (k == k1 ? mn : 0));
    }
    const i32x4 av = __builtin_bit_cast(i32x4, a);
    const i32x4 bv = __builtin_bit_cast(i32x4, b);
    i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, i32x16{}, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) out[(k0 * 64 + lane) * 16 + r] = (float)c[r];
  }
#endif
}

// Transposing LDS reads: LDS holds the identity pattern (16-bit element e
// holds e; for the 8-bit read byte address a holds a, written as two passes
// of its low and high byte), every lane addresses the 8 bytes at lane * 8,
// and the lane's returned elements are recorded: the LDS element id (16-bit)
// or byte address (8-bit) each one came from.
__global__ __launch_bounds__(64) void probe_tr16(uint16_t* out) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ uint16_t lds[256];
  const int lane = threadIdx.x;
  for (int i = lane; i < 256; i += 64) lds[i] = (uint16_t)i;
  __syncthreads();
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)((__attribute__((address_space(3))) char*)lds + lane * 8));
#pragma unroll
  for (int e = 0; e < 4; ++e) out[lane * 4 + e] = (uint16_t)v[e];
#endif
}

__global__ __launch_bounds__(64) void probe_tr8(uint16_t* out) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ uint8_t lds[512];
  typedef int i32x2 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
  const int lane = threadIdx.x;
  uint16_t got[8] = {};
  for (int pass = 0; pass < 2; ++pass) {
    for (int i = lane; i < 512; i += 64) lds[i] = (uint8_t)(pass ? i >> 8 : i & 255);
    __syncthreads();
    const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (lds_i32x2*)((__attribute__((address_space(3))) char*)lds + lane * 8));
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) got[e] |= (uint16_t)(((v[e >> 2] >> (8 * (e & 3))) & 255) << (8 * pass));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) out[lane * 8 + e] = got[e];
#endif
}

}  // namespace

hipError_t lds_transpose_probe(int bits, uint16_t* out, hipStream_t stream) {
  if (bits == 16) hipLaunchKernelGGL(probe_tr16, dim3(1), dim3(64), 0, stream, out);
  else if (bits == 8) hipLaunchKernelGGL(probe_tr8, dim3(1), dim3(64), 0, stream, out);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

int mfma_probe_floats(int atom) {
  switch (atom) {
    case 0: return 16 * 64 * 16;  // bf16 32x32x16
    case 1: return 32 * 64 * 4;   // bf16 16x16x32
    case 2: return 32 * 64 * 16;  // i8 32x32x32
    default: return 0;
  }
}

hipError_t mfma_layout_probe(int atom, float* out, hipStream_t stream) {
  switch (atom) {
    case 0: hipLaunchKernelGGL((probe_bf16<32, 16>), dim3(1), dim3(64), 0, stream, out); break;
    case 1: hipLaunchKernelGGL((probe_bf16<16, 32>), dim3(1), dim3(64), 0, stream, out); break;
    case 2: hipLaunchKernelGGL(probe_i8_32, dim3(1), dim3(64), 0, stream, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace frisk
