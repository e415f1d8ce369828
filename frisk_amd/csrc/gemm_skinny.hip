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
//    per load instruction.  Batches of U k-steps are double-buffered: batch
//    b+1 is loaded while batch b is multiplied (operands from HBM:
//    64x4096x4096 33.0 -> 24.5 us, 16x4096x4096 13.9 -> 11.9 us).
//  * A batch of kSkinnyWaves * U k-steps gives wave w the k-step pairs
//    (2w, 2w+1), (2w+8, 2w+9), ...: the two 64 B halves of each 128 B line
//    are loaded by one wave back to back (the per-workgroup rotation is
//    even, so pairs stay aligned).  Operands from HBM, TFLOP/s, against
//    interleaving single k-steps over the waves: 16x4096x4096 45.4 -> 47.8,
//    16x14336x4096 65.4 -> 68.0, 16x4096x14336 60.3 -> 61.7.
//  * W rows and the K tail are bounds-checked by raw buffer loads (offsets
//    past num_records read zeros); X rows past M are clamped (their outputs
//    are not stored).
//  * Each workgroup starts its K walk at its own step (and wraps around), so
//    the workgroups streaming different W columns do not all request the
//    same X cache lines at once (128x4096x4096: 52.7 -> 39.0 us).
//  * Split-K (when the caller provides a workspace): blockIdx.z picks a
//    slice of the k-steps, each workgroup writes its f32 partial tile to
//    workspace[slice][M][N], and gemm_splitk_sum_kernel adds the slices in
//    slice order (deterministic) and converts.  Wider column tiles then cut
//    the number of times X is streamed from L2 (every workgroup reads the
//    X rows of its K range), and the slices restore the parallelism.
//  * Roofline: HBM-bound; algorithmic bytes = M.K.2 + N.K.2 + M.N.2.

#include <algorithm>

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

// k-steps loaded ahead per wave: as many as the load registers allow
// (U (TM + TN) 4 VGPRs beside the TM TN 4 accumulator VGPRs).
// A single 16 x 16 tile per workgroup loads 8 k-steps ahead: its 128 KiB
// of W at N = K = 4096 are then half in flight at once (16 x 4096 x 4096,
// operands from HBM: 11.4 -> 10.5 us; 12 or 16 k-steps ran 4% and 13% slower,
// and the wider tiles measured no change with 8).
template <int TM, int TN> constexpr int skinny_unroll() {
  return TM + TN <= 2 ? 8 : TM + TN <= 10 ? 4 : 2;
}

}  // namespace

template <Elt IN, Elt OUT, int TM, int TN>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny_kernel(
    const char* __restrict__ A, const char* __restrict__ B, void* __restrict__ C, int M, int N,
    int Kb, int64_t lda_b, int64_t ldb_b, int64_t ldc, int accumulate, int steps_per_slice,
    float* __restrict__ partial) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int U = skinny_unroll<TM, TN>();
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

  // This workgroup's k-steps (64 B of K each): [s_begin, s_begin + nsteps),
  // walked from a per-workgroup offset `rot`.
  const int all_steps = (Kb + 63) / 64;
  const int s_begin = blockIdx.z * steps_per_slice;
  const int nsteps = min(all_steps - s_begin, steps_per_slice);
  const int rot = (int)(((unsigned)blockIdx.x * 5u + (unsigned)blockIdx.y * 3u) % (unsigned)nsteps) & ~1;
  const int kmax = Kb - quad * 16;    // this lane's 16 B chunk is live while kb < kmax
  // Batches of U k-steps, double-buffered: the loads of batch b+1 are in
  // flight while batch b is multiplied, so a workgroup pays one memory
  // latency per slice instead of one per batch.  Batches past the end load
  // nothing (zero reads) and add zero products.
  static_assert(U % 2 == 0, "k-step pairs");
  auto load = [&](int b0, i32x4 (&av)[U][TM], i32x4 (&bv)[U][TN]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = b0 + 2 * wave + (u & 1) + 2 * kSkinnyWaves * (u >> 1);
      int sr = st + rot;
      if (sr >= nsteps) sr -= nsteps;
      const int kb = (s_begin + sr) * 64;
      const bool live = st < nsteps && kb < kmax;
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(rsb, live ? b_off[t] + kb : 0x80000000u,
                                                         0, 0);
#pragma unroll
      for (int t = 0; t < TM; ++t)
        av[u][t] = __builtin_amdgcn_raw_buffer_load_b128(rsa, live ? a_off[t] + kb : 0x80000000u,
                                                         0, 0);
    }
  };
  auto mul = [&](const i32x4 (&av)[U][TM], const i32x4 (&bv)[U][TN]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma16<IN>::run(av[u][i], bv[u][j], acc[i][j]);
  };
  constexpr int kBatch = kSkinnyWaves * U;
  i32x4 a0[U][TM], b0[U][TN], a1[U][TM], b1[U][TN];
  load(0, a0, b0);
  for (int s0 = 0; s0 < nsteps; s0 += 2 * kBatch) {
    load(s0 + kBatch, a1, b1);
    mul(a0, b0);
    if (s0 + kBatch >= nsteps) break;
    load(s0 + 2 * kBatch, a0, b0);
    mul(a1, b1);
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
      if (partial) {
        partial[((int64_t)blockIdx.z * M + row) * N + col] = v;
      } else {
        const int64_t o = (int64_t)row * ldc + col;
        if (accumulate) v += load_as_f32<OUT>(C, o);
        store_from_f32<OUT>(C, o, v);
      }
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// C[row, 4c .. 4c+3] (+)= sum over slices z = 0, 1, ... of
// partial[z][row][4c .. 4c+3], added in slice order.  N is a multiple of 4.
template <Elt OUT>
__global__ __launch_bounds__(256) void gemm_splitk_sum_kernel(const float* __restrict__ partial,
                                                              int slices, int M, int N,
                                                              void* __restrict__ C, int64_t ldc,
                                                              int accumulate) {
  const int64_t quads = (int64_t)N / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * quads) return;
  const int row = (int)(idx / quads), col = (int)(idx % quads) * 4;
  f32x4 sum = *(const f32x4*)(partial + (int64_t)row * N + col);
#pragma unroll 8
  for (int z = 1; z < slices; ++z) sum += *(const f32x4*)(partial + ((int64_t)z * M + row) * N + col);
  const int64_t o = (int64_t)row * ldc + col;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = sum[e];
    if (accumulate) v += load_as_f32<OUT>(C, o + e);
    store_from_f32<OUT>(C, o + e, v);
  }
}

namespace {

template <Elt IN, Elt OUT, int TM, int TN>
hipError_t launch_skinny(const GemmArgs& g, const SkinnyPlan& p, float* partial,
                         hipStream_t stream) {
  constexpr int kEsz = EltInfo<IN>::bytes;
  dim3 grid((unsigned)((g.n + 16 * TN - 1) / (16 * TN)), (unsigned)((g.m + 16 * TM - 1) / (16 * TM)),
            (unsigned)(partial ? p.slices : 1));
  const int steps = partial ? p.steps_per_slice : (int)((g.k * kEsz + 63) / 64);
  hipLaunchKernelGGL((gemm_skinny_kernel<IN, OUT, TM, TN>), grid, dim3(64 * kSkinnyWaves), 0,
                     stream, (const char*)g.a, (const char*)g.b, g.c, (int)g.m, (int)g.n,
                     (int)(g.k * kEsz), g.lda * kEsz, g.ldb * kEsz, g.ldc, g.accumulate, steps,
                     partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !partial) return e;
  return gemm_splitk_sum(partial, p.slices, g, stream);
}

template <Elt IN, Elt OUT, int TN>
hipError_t skinny_by_m(const GemmArgs& g, const SkinnyPlan& p, float* partial, hipStream_t s) {
  switch (p.tm) {
    case 1: return launch_skinny<IN, OUT, 1, TN>(g, p, partial, s);
    case 2: return launch_skinny<IN, OUT, 2, TN>(g, p, partial, s);
    case 4: return launch_skinny<IN, OUT, 4, TN>(g, p, partial, s);
    default: return launch_skinny<IN, OUT, 8, TN>(g, p, partial, s);
  }
}

template <Elt IN, Elt OUT>
hipError_t skinny_by_n(const GemmArgs& g, const SkinnyPlan& p, float* partial, hipStream_t s) {
  switch (p.tn) {
    case 1: return skinny_by_m<IN, OUT, 1>(g, p, partial, s);
    case 2: return skinny_by_m<IN, OUT, 2>(g, p, partial, s);
    default: return skinny_by_m<IN, OUT, 4>(g, p, partial, s);
  }
}

}  // namespace

hipError_t gemm_splitk_sum(const float* partial, int slices, const GemmArgs& g, hipStream_t s) {
  const int64_t threads = g.m * (g.n / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  switch (g.out) {
    case Elt::BF16:
      hipLaunchKernelGGL((gemm_splitk_sum_kernel<Elt::BF16>), grid, dim3(256), 0, s, partial,
                         slices, (int)g.m, (int)g.n, g.c, g.ldc, g.accumulate);
      break;
    case Elt::F16:
      hipLaunchKernelGGL((gemm_splitk_sum_kernel<Elt::F16>), grid, dim3(256), 0, s, partial,
                         slices, (int)g.m, (int)g.n, g.c, g.ldc, g.accumulate);
      break;
    case Elt::F32:
      hipLaunchKernelGGL((gemm_splitk_sum_kernel<Elt::F32>), grid, dim3(256), 0, s, partial,
                         slices, (int)g.m, (int)g.n, g.c, g.ldc, g.accumulate);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t gemm_skinny(const GemmArgs& g, hipStream_t s, void* workspace, int64_t workspace_bytes) {
  SkinnyPlan p = gemm_skinny_plan(g, device_cus(), true);
  float* partial = nullptr;
  if (p.slices > 1) {
    if (workspace && workspace_bytes >= p.workspace_bytes)
      partial = (float*)workspace;
    else
      p = gemm_skinny_plan(g, 0, false);
  }
  switch (((int)g.in << 8) | (int)g.out) {
    case ((int)Elt::BF16 << 8) | (int)Elt::BF16: return skinny_by_n<Elt::BF16, Elt::BF16>(g, p, partial, s);
    case ((int)Elt::BF16 << 8) | (int)Elt::F32: return skinny_by_n<Elt::BF16, Elt::F32>(g, p, partial, s);
    case ((int)Elt::F16 << 8) | (int)Elt::F16: return skinny_by_n<Elt::F16, Elt::F16>(g, p, partial, s);
    case ((int)Elt::F16 << 8) | (int)Elt::F32: return skinny_by_n<Elt::F16, Elt::F32>(g, p, partial, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace frisk
