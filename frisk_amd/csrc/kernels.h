// Host-side launcher interface between the C-ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "launch_plan.h"


namespace frisk {

// A validated GEMM request (sizes in elements).
struct GemmArgs {
  Elt in, out;
  int64_t m, n, k;
  int trans_a, trans_b;
  const void* a;
  int64_t lda;
  const void* b;
  int64_t ldb;
  void* c;
  int64_t ldc;
  float scale;  // scale_a * scale_b
  int accumulate;
  // Requested kernel variant (0: the library chooses): 256 or 128 tiles,
  // the 128x128 kernel's wave grid, and K slices of a 2x2-grid variant.
  int tile = 0, wave_m = 0, wave_n = 0, slices = 0;
};

// The request as the launch planner (launch_plan.h) sees it.
inline plan::GemmShape shape_of(const GemmArgs& g) {
  plan::GemmShape s;
  s.in = (int)g.in;
  s.out = (int)g.out;
  s.m = g.m;
  s.n = g.n;
  s.k = g.k;
  s.trans_a = g.trans_a != 0;
  s.trans_b = g.trans_b != 0;
  s.tile = g.tile;
  s.wave_m = g.wave_m;
  s.wave_n = g.wave_n;
  s.slices = g.slices;
  return s;
}

using plan::kTreeMaxSlices;
using plan::kTreeWords;
using plan::split_tree_bytes;
using SplitPlan = plan::SplitPlan;
using MfmaChoice = plan::MfmaChoice;
using SkinnyPlan = plan::SkinnyPlan;
inline SplitPlan gemm_split_plan(const GemmArgs& g, int cus) { return plan::split_plan(shape_of(g), cus); }
inline MfmaChoice gemm_mfma_choice(const GemmArgs& g, int cus, bool workspace) {
  return plan::mfma_choice(shape_of(g), cus, workspace);
}
// LDS-staged MFMA GEMM, any storage order of A and B; the caller checked 16 B
// aligned operands with 16 B row pitches, K * esize % 16 == 0 for every
// K-major operand and a 16 B row pitch of C.  With a workspace of at least
// the plan's bytes (16-byte aligned) the planned split runs; otherwise the
// unsplit kernels.
hipError_t gemm_mfma(const GemmArgs& g, hipStream_t s, void* workspace, int64_t workspace_bytes);
// C (+)= the sum over slices of partial[slice][M][N] (f32, added in slice
// order), converted to C's type; N is a multiple of 4.
hipError_t gemm_splitk_sum(const float* partial, int slices, const GemmArgs& g, hipStream_t s);
// The kernels of one storage order (AM: A stored [K, M]; BM: B stored
// [K, N]), instantiated in gemm_w4_a*b*.hip (256x256 tiles) and
// gemm_128_a*b*.hip (128x128 tiles).  The split variants run `slices` K
// slices of kb_slice bytes in one launch, summed into C through the
// workspace `ws` of split_tree_bytes.
template <bool AM, bool BM> hipError_t gemm_w4_layout(const GemmArgs& g, hipStream_t s);
template <bool AM, bool BM>
hipError_t gemm_w4_split_layout(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                hipStream_t s);
template <bool AM, bool BM> hipError_t gemm_128_layout(const GemmArgs& g, hipStream_t s);
// Bytes of K per row per pipeline stage of gemm_128_layout's launch
// (plan::stage_bytes_128).
inline int gemm_128_stage_bytes(const GemmArgs& g, int cus) {
  return plan::stage_bytes_128(shape_of(g), cus);
}
// The 128x128 kernel with the wave grid g.wave_m x g.wave_n (2x2, 4x1, 1x4,
// 2x1 or 1x2), 64-byte stages.
template <bool AM, bool BM> hipError_t gemm_128_grid_layout(const GemmArgs& g, hipStream_t s);
template <bool AM, bool BM>
hipError_t gemm_128_split_layout(const GemmArgs& g, int slices, int64_t kb_slice, void* ws,
                                 hipStream_t s);
// Any layout / shape; LDS-tiled FMA kernel.
hipError_t gemm_generic_any(const GemmArgs& g, hipStream_t s);
// Small-M kernel (plan::skinny_supported: M <= kSkinnyMaxM, bf16/f16,
// trans_a == 0, trans_b == 1, 16 B aligned K-contiguous rows);
// memory-bound regime.
using plan::kSkinnyMaxM;
inline bool gemm_skinny_supported(const GemmArgs& g) { return plan::skinny_supported(shape_of(g)); }
inline SkinnyPlan gemm_skinny_plan(const GemmArgs& g, int cus, bool split) {
  return plan::skinny_plan(shape_of(g), cus, split);
}
// Split-K runs when `workspace` holds at least the plan's workspace_bytes
// (16-byte aligned); otherwise the unsplit kernel runs.
hipError_t gemm_skinny(const GemmArgs& g, hipStream_t s, void* workspace, int64_t workspace_bytes);

// A validated attention request.
struct AttnArgs {
  Elt dtype;  // Q/K/V
  Elt out;    // O: dtype or F32
  int64_t batch, heads, seq_q, seq_k, head_dim;
  int causal;
  float sm_scale;
  const void* q;
  int64_t q_sb, q_sh, q_ss;
  const void* k;
  int64_t k_sb, k_sh, k_ss;  // k_ss: between keys, or with k_dmajor between head_dim rows
  int k_dmajor;              // K stored [batch, heads, head_dim, seq]
  int waves = 0;             // waves per workgroup (4 or 8); 0: plan::attn_waves
  const void* v;
  int64_t v_sb, v_sh, v_ss;
  void* o;
  int64_t o_sb, o_sh, o_ss;
  float* lse;
};

hipError_t attn_fwd_d128(const AttnArgs& a, hipStream_t s);
hipError_t attn_fwd_d64(const AttnArgs& a, hipStream_t s);
hipError_t attn_fwd_d32(const AttnArgs& a, hipStream_t s);
hipError_t attn_fwd_d16(const AttnArgs& a, hipStream_t s);
inline hipError_t attn_fwd(const AttnArgs& a, hipStream_t s) {
  switch (a.head_dim) {
    case 128: return attn_fwd_d128(a, s);
    case 64: return attn_fwd_d64(a, s);
    case 32: return attn_fwd_d32(a, s);
    case 16: return attn_fwd_d16(a, s);
    default: return hipErrorInvalidValue;
  }
}

// Tile ops (tileops.hip).  Reduction kinds of frisk.reduce_tensor.
constexpr int kReduceSum = 0, kReduceMax = 1, kReduceMin = 2;

// A validated reduction of a [rows, cols] tensor (element strides) along
// `axis`; dtype F32, F16 or BF16 for source and destination.
struct ReduceArgs {
  Elt dtype;
  int kind, axis, clear;
  int64_t rows, cols;
  const void* src;
  int64_t ld;
  void* dst;
  int64_t dst_stride;
  // Leaf order: 0 = ascending index; else the reduced extent is
  // 2^order_bits and tree level j combines along index bit order[j].
  int order_bits;
  uint8_t order[32];
  // Axis 0 only: f32 scratch of cols_split(rows, cols).blocks * cols
  // elements for the two-pass kernels, or null for the single pass.
  void* workspace;
};
hipError_t tile_reduce(const ReduceArgs& a, hipStream_t s);

// Two-pass axis-0 geometry: strips of 4 * 2^sps_log2 columns x row blocks
// of 2^b_log2 rows.
struct ColsSplit {
  int64_t strips, blocks;
  int sps_log2, b_log2;
};
ColsSplit cols_split(int64_t rows, int64_t cols);

// A validated copy of a [rows, cols] tensor; src_t == dst_t copies raw
// elements of `esize` bytes, otherwise both are F32, F16, BF16 or E4M3.
struct CopyArgs {
  Elt src_t, dst_t;
  int esize;
  int64_t rows, cols;
  const void* src;
  int64_t ld_src;
  void* dst;
  int64_t ld_dst;
};
hipError_t tile_copy(const CopyArgs& a, hipStream_t s);

// Fill a [rows, cols] tensor of `esize`-byte elements with a bit pattern.
struct FillArgs {
  int esize;
  uint64_t bits;
  int64_t rows, cols;
  void* dst;
  int64_t ld;
};
hipError_t tile_fill(const FillArgs& a, hipStream_t s);

// MFMA fragment-layout probe (probe.hip): atom 0 = bf16 32x32x16,
// 1 = bf16 16x16x32, 2 = i8 32x32x32; `out` holds mfma_probe_floats(atom)
// floats.
int mfma_probe_floats(int atom);
hipError_t mfma_layout_probe(int atom, float* out, hipStream_t stream);
// Transposing LDS read probe (probe.hip): bits 16 = ds_read_b64_tr_b16
// (256 outputs), 8 = ds_read_b64_tr_b8 (512 outputs).
hipError_t lds_transpose_probe(int bits, uint16_t* out, hipStream_t stream);

}  // namespace frisk
