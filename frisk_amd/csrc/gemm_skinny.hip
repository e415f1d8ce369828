// Small-M (skinny) MFMA GEMM for gfx950: Y[M, N] = X[M, K] . W[N, K]^T with
// M <= 128, the memory-bound regime of the projection sweep (BASELINE
// configs[2], M in {16, 128}), where the 256x256-tile kernel would launch
// only N/256 workgroups.
//
//  * One workgroup per (16 TM) x (16 TN) output tile, so N/16 (or N/32)
//    workgroups stream W.  The 4 waves split K (wave w takes k-steps
//    w, w+4, ...) and their partial accumulators are summed through LDS at
//    the end.
//  * Operands go straight from global memory into MFMA registers (no LDS):
//    v_mfma_f32_16x16x32_{bf16,f16} wants lane l to hold 16 contiguous bytes
//    of row l%16 at k-offset 8*(l/16), i.e. 16 B per lane and 64 B per row
//    per load instruction.  U k-steps are loaded ahead of their MFMAs to keep
//    enough bytes in flight to cover HBM latency.
//  * W rows and the K tail are bounds-checked by raw buffer loads (offsets
//    past num_records read zeros); X rows past M are clamped (their outputs
//    are not stored).
//  * Roofline: HBM-bound; algorithmic bytes = M.K.2 + N.K.2 + M.N.2.

#include "common.h"
#include "kernels.h"

namespace frisk {

namespace {

typedef float f32x4_ __attribute__((ext_vector_type(4)));

template <Elt E> struct Mfma16;
template <> struct Mfma16<Elt::BF16> {
  __device__ static inline f32x4_ run(i32x4 a, i32x4 b, f32x4_ c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<Elt::F16> {
  __device__ static inline f32x4_ run(i32x4 a, i32x4 b, f32x4_ c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyUnroll = 4;  // k-steps loaded ahead per wave

}  // namespace

template <Elt IN, Elt OUT, int TM, int TN>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny_kernel(
    const char* __restrict__ A, const char* __restrict__ B, void* __restrict__ C, int M, int N,
    int Kb, int64_t lda_b, int64_t ldb_b, int64_t ldc, int accumulate) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int U = kSkinnyUnroll;
  __shared__ float red[kSkinnyWaves][TM * TN * 4][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, quad = lane >> 4;
  const int m0 = blockIdx.y * 16 * TM, n0 = blockIdx.x * 16 * TN;

  const char* a_base = A + (int64_t)m0 * lda_b;
  const char* b_base = B + (int64_t)n0 * ldb_b;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a_base, (short)0,
      (int)min((int64_t)(M - 1 - m0) * lda_b + Kb, (int64_t)0x7fffffff), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)b_base, (short)0,
      (int)min((int64_t)(N - 1 - n0) * ldb_b + Kb, (int64_t)0x7fffffff), 0x00020000);
  uint32_t a_off[TM], b_off[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) a_off[t] = (uint32_t)(min(t * 16 + l16, M - 1 - m0) * lda_b) + quad * 16;
#pragma unroll
  for (int t = 0; t < TN; ++t) b_off[t] = (uint32_t)((t * 16 + l16) * ldb_b) + quad * 16;
  // W rows past N are not clamped: the buffer range check zero-fills the
  // last tile's missing rows.

  f32x4_ acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_{0, 0, 0, 0};

  const int nsteps = (Kb + 63) / 64;  // 64 B of K per MFMA k-step
  const int kmax = Kb - quad * 16;    // this lane's 16 B chunk is live while kb < kmax
  for (int s0 = wave; s0 < nsteps; s0 += kSkinnyWaves * U) {
    i32x4 av[U][TM], bv[U][TN];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = (s0 + kSkinnyWaves * u) * 64;
      const bool live = kb < kmax;
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(rsb, live ? b_off[t] + kb : 0x80000000u,
                                                         0, 0);
#pragma unroll
      for (int t = 0; t < TM; ++t)
        av[u][t] = __builtin_amdgcn_raw_buffer_load_b128(rsa, live ? a_off[t] + kb : 0x80000000u,
                                                         0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma16<IN>::run(av[u][i], bv[u][j], acc[i][j]);
  }

  // Sum the 4 waves' partial tiles.  The 16x16 accumulator holds
  // D[4*(lane/16) + r][lane%16] in element r.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][(i * TN + j) * 4 + r][lane] = acc[i][j][r];
  __syncthreads();
  constexpr int kElems = TM * TN * 4 * 64;
  for (int e = tid; e < kElems; e += 64 * kSkinnyWaves) {
    const int idx = e >> 6, ln = e & 63;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) v += red[w][idx][ln];
    const int tile = idx >> 2, r = idx & 3;
    const int i = tile / TN, j = tile % TN;
    const int row = m0 + i * 16 + 4 * (ln >> 4) + r;
    const int col = n0 + j * 16 + (ln & 15);
    if (row < M && col < N) {
      const int64_t o = (int64_t)row * ldc + col;
      if (accumulate) v += load_as_f32<OUT>(C, o);
      store_from_f32<OUT>(C, o, v);
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <Elt IN, Elt OUT, int TM, int TN>
static hipError_t launch_skinny(const GemmArgs& g, hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  dim3 grid((unsigned)((g.n + 16 * TN - 1) / (16 * TN)), (unsigned)((g.m + 16 * TM - 1) / (16 * TM)));
  hipLaunchKernelGGL((gemm_skinny_kernel<IN, OUT, TM, TN>), grid, dim3(64 * kSkinnyWaves), 0,
                     stream, (const char*)g.a, (const char*)g.b, g.c, (int)g.m, (int)g.n,
                     (int)(g.k * kEsz), g.lda * kEsz, g.ldb * kEsz, g.ldc, g.accumulate);
  return hipGetLastError();
}

template <Elt IN, Elt OUT, int TN>
static hipError_t skinny_by_m(const GemmArgs& g, hipStream_t s) {
  if (g.m <= 16) return launch_skinny<IN, OUT, 1, TN>(g, s);
  if (g.m <= 32) return launch_skinny<IN, OUT, 2, TN>(g, s);
  if (g.m <= 64) return launch_skinny<IN, OUT, 4, TN>(g, s);
  return launch_skinny<IN, OUT, 8, TN>(g, s);
}

// 32-column tiles once N alone gives >= 256 of them (measured: better for
// N = 14336, worse for N = 4096).
template <Elt IN, Elt OUT>
static hipError_t skinny_by_n(const GemmArgs& g, hipStream_t s) {
  if (g.n >= 8192) return skinny_by_m<IN, OUT, 2>(g, s);
  return skinny_by_m<IN, OUT, 1>(g, s);
}

bool gemm_skinny_supported(const GemmArgs& g) {
  const bool type_ok = (g.in == Elt::BF16 && (g.out == Elt::BF16 || g.out == Elt::F32)) ||
                       (g.in == Elt::F16 && (g.out == Elt::F16 || g.out == Elt::F32));
  return type_ok && g.m <= kSkinnyMaxM && !g.trans_a && g.trans_b;
}

hipError_t gemm_skinny(const GemmArgs& g, hipStream_t s) {
  switch (((int)g.in << 8) | (int)g.out) {
    case ((int)Elt::BF16 << 8) | (int)Elt::BF16: return skinny_by_n<Elt::BF16, Elt::BF16>(g, s);
    case ((int)Elt::BF16 << 8) | (int)Elt::F32: return skinny_by_n<Elt::BF16, Elt::F32>(g, s);
    case ((int)Elt::F16 << 8) | (int)Elt::F16: return skinny_by_n<Elt::F16, Elt::F16>(g, s);
    case ((int)Elt::F16 << 8) | (int)Elt::F32: return skinny_by_n<Elt::F16, Elt::F32>(g, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace frisk
