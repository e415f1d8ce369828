/*
 * frisk_hip.h — C-ABI of the MI355X (gfx950) GEMM, attention and tile-op
 * kernels.
 *
 * The reference (guoqiao7/frisk) has no execute entry in its FFI: the
 * pass/execute bindings are commented out at ffi/ffi.h:14 and ffi/ffi.cpp:6,
 * and the only GPU path is the out-of-process harness
 * benchmark/layout/execution/run_execution.py:23-95 (frisk-opt -> JSON ->
 * Triton).  These entry points are what that FFI would bind for the GEMM and
 * attention tile programs and the tile ops around them:
 *
 *   frisk_gemm      <- the semantics of frisk.gemm
 *                      (include/Dialect/Frisk/IR/FriskOps.td:252-292;
 *                      shape/type contract lib/Dialect/Frisk/IR/
 *                      LegacyImportSemantics.cpp:11-46, extended to
 *                      int8->int32 and fp8-e4m3->f32/bf16/f16),
 *                      replacing the wgmma emission of
 *                      benchmark/layout/execution/backend.py:383-431.
 *   frisk_attn_fwd  <- the attention tile program (tmp/ir.mlir:89-157,
 *                      benchmark/layout/execution/tiled_attention.py:210-728),
 *                      with online softmax instead of three passes.
 *   frisk_reduce    <- frisk.reduce (include/Dialect/Frisk/IR/FriskOps.td:
 *                      425-453; clear/merge lowering LegacyFragmentNormalization
 *                      .cpp:522-555) and frisk.reduce_tensor (FriskLayoutOps.td:
 *                      17-30) in the canonical_fiber_tree_v1 order
 *                      (lib/Dialect/Frisk/Analysis/ReductionLayoutProof.cpp:
 *                      108-140).
 *   frisk_copy      <- frisk.copy (FriskOps.td:351-397) of a whole tile,
 *                      including the element-type change of a fragment stored
 *                      to global memory (tmp/ir.mlir:154).
 *   frisk_fill      <- frisk.fill (FriskOps.td:400-422; builder ffi/ir.cpp:
 *                      439-454).
 *
 * Conventions: plain pointers and sizes only; every pointer is a device
 * pointer owned by the caller; `stream` is a hipStream_t (NULL = the null
 * stream).  Calls are stream-ordered and reentrant.  Every entry returns 0
 * on success or a negative FRISK_E* code; a failed call launches nothing and
 * writes no output, and frisk_last_error() (thread-local) describes why.
 */
#ifndef FRISK_HIP_H
#define FRISK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FRISK_ABI_VERSION 7

/* Element types (the dtype strings of ffi/ir.cpp:399-411 plus bf16/i8/i32). */
typedef enum frisk_dtype {
  FRISK_F32 = 0,
  FRISK_F16 = 1,
  FRISK_BF16 = 2,
  FRISK_E4M3 = 3, /* OCP float8 e4m3fn */
  FRISK_I8 = 4,
  FRISK_I32 = 5,
  FRISK_F64 = 6
} frisk_dtype;

/* Error codes. */
#define FRISK_OK 0
#define FRISK_EINVAL (-1)   /* bad shape, stride, dtype combination or pointer */
#define FRISK_EUNSUP (-2)   /* valid request this build has no kernel for */
#define FRISK_EHIP (-3)     /* the HIP runtime reported an error */

/*
 * C[m, n] = op(A)[m, k] . op(B)[k, n]   (clear_accum != 0)
 * C[m, n] += op(A)[m, k] . op(B)[k, n]  (clear_accum == 0)
 *
 * op(A) = A (stored [m, k], row stride lda)        when trans_a == 0
 *       = A^T (A stored [k, m], row stride lda)    when trans_a != 0
 * op(B) = B (stored [k, n], row stride ldb)        when trans_b == 0
 *       = B^T (B stored [n, k], row stride ldb)    when trans_b != 0
 * C is stored [m, n] with row stride ldc.  Strides are in elements.
 *
 * Type contract (a_type must equal b_type):
 *   f32  x f32  -> f32
 *   f16  x f16  -> f16 | f32        (f32 accumulation)
 *   bf16 x bf16 -> bf16 | f32       (f32 accumulation)
 *   e4m3 x e4m3 -> bf16 | f16 | f32 (f32 accumulation, then * scale_a*scale_b)
 *   i8   x i8   -> i32              (exact int32 accumulation)
 * scale_a/scale_b are the per-tensor dequantisation factors of fp8 inputs
 * and must be 1.0 for every other type.
 *
 * workspace / workspace_bytes: optional device scratch (16-byte aligned)
 * owned by the caller.  A small-M bf16/f16/f32 GEMM given at least
 * frisk_gemm_workspace_size() bytes splits K over the whole GPU (f32
 * partial tiles, added in a fixed order, so the result does not depend on
 * timing); without it, or when the size is 0, the unsplit kernels run.
 * Two slices are summed inside the GEMM launch, through partials and
 * arrival words in the workspace; its contents before the call do not
 * matter, and nothing needs clearing between calls.  Calls that share a
 * workspace must not overlap.
 */
typedef struct frisk_gemm_desc {
  int64_t m, n, k;
  int32_t trans_a, trans_b;
  int32_t a_type, b_type, c_type; /* frisk_dtype */
  int32_t clear_accum;
  const void* a;
  int64_t lda;
  const void* b;
  int64_t ldb;
  void* c;
  int64_t ldc;
  float scale_a, scale_b;
  void* workspace; /* optional, may be NULL */
  int64_t workspace_bytes;
  /* Optional kernel variant; all zero: the library chooses.  tile = 256:
   * the 256x256 kernel (four waves in a 2x2 grid); tile = 128: the 128x128
   * kernel with a wave_m x wave_n wave grid, one of 2x2, 4x1, 1x4 (256
   * threads) or 2x1, 1x2 (128 threads), 0x0 meaning 2x2.  A requested
   * variant runs unsplit, or with slices > 1 in that many K slices (2x2
   * grid, bf16/f16/f32, N % 4 == 0; placed on stage boundaries as the
   * library's own split; it needs the workspace frisk_gemm_workspace_size
   * reports for the request, and runs unsplit without it).  It returns
   * FRISK_EUNSUP when the descriptor does not meet the matrix-core
   * conditions below.  variant_flags must be 0.  This is how a tile
   * program's instruction contract (its #frisk.mma_contract: MFMA atom and
   * wave grid of the workgroup tile) and the launch contract layout
   * inference gives a whole-matrix GEMM select the kernel that runs. */
  int32_t tile, wave_m, wave_n, variant_flags;
  int32_t slices; /* K slices of a requested variant; 0 or 1: unsplit */
} frisk_gemm_desc;

int frisk_gemm(const frisk_gemm_desc* desc, void* stream);

/* Every storage order of A and B runs on the matrix cores (f32/bf16/f16/fp8/
 * i8; f32 on v_mfma_f32_32x32x2_f32) when the operands have 16-byte aligned
 * bases and row pitches, K * esize is a multiple of 16 for an operand stored
 * K-contiguous (A without trans_a, B with trans_b), C's row pitch is a
 * multiple of 16 bytes, and every buffer a tile addresses spans less than
 * 2^31 bytes; anything else runs a correct but slower generic kernel. */

/* frisk_gemm without any device allocation by the library or the caller:
 * no hipMalloc, hipFree or allocating library routine is called.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  It runs the same kernels as frisk_gemm given a workspace of
 * frisk_gemm_workspace_size(desc) bytes, with the split-K partials in a
 * device array of FRISK_GEMM_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends.  desc->workspace must be NULL
 * and workspace_bytes 0.  A GEMM whose split needs more scratch than that is
 * rejected with FRISK_EUNSUP (call frisk_gemm with a workspace instead).
 * Calls on one GPU share that array: calls that overlap in time on one GPU
 * (different streams, or host threads) race on it and must be serialised by
 * the caller; calls ordered on one stream are safe.  The first call on a
 * device looks the array up there (hipGetSymbolAddress): make it outside
 * graph capture (one warm-up call), then capture freely. */
#define FRISK_GEMM_NOALLOC_SCRATCH_BYTES (64ll << 20)
int frisk_gemm_noalloc(const frisk_gemm_desc* desc, void* stream);

/* Workspace bytes that make frisk_gemm(desc) split K (0: none is used), or
 * a negative FRISK_E* code for an invalid descriptor.  Pointers in desc are
 * not read.  No counterpart in the reference (its GEMM ops take no
 * scratch); callers that have none keep calling frisk_gemm unchanged. */
int64_t frisk_gemm_workspace_size(const frisk_gemm_desc* desc);

/* The launch frisk_gemm(desc) makes, as one line of JSON written to buf
 * (len bytes including the terminating NUL): "kernel" (gemm_w4 = 256x256
 * tiles, gemm_128 = 128x128 tiles, gemm_skinny = small M, gemm_generic),
 * "tile_m"/"tile_n", the MFMA "atom", "waves" and "wave_tile" (the wave
 * grid and each wave's sub-tile), "stage_bytes" (K bytes per LDS stage),
 * "a_major"/"b_major" ("k" = K-contiguous storage, "m"/"n" otherwise), the
 * LDS fragment read of each operand ("lds_read_a"/"lds_read_b":
 * ds_read_b128, or ds_read_b64_tr_b16 / _tr_b8 for an M/N-major operand),
 * "slices" (split-K), "slice_sum" ("none", "in_launch": summed by the GEMM
 * kernel itself, "second_launch": by a slice-sum kernel) and
 * "workspace_bytes".  desc->workspace_bytes is taken
 * as the workspace a call would pass; pointers are never read, but when all
 * of a, b and c are given their alignment counts as in frisk_gemm (so a
 * requested variant the tensors cannot run is refused here too).  No
 * counterpart in the reference, whose execution packet records the chosen
 * instruction contract instead (ExportExecution.cpp:46-295): this reports
 * the contract of the kernel the C-ABI selects, for layout checks and
 * tests. */
int frisk_gemm_plan(const frisk_gemm_desc* desc, char* buf, int64_t len);

/*
 * Flash-attention forward over [batch, heads, seq, head_dim] tensors:
 *   O[b,h,i,:] = softmax_j(sm_scale * Q[b,h,i,:].K[b,h,j,:]) . V[b,h,j,:]
 * with j <= i (plus seq_k - seq_q) when causal != 0.  Q/K/V are bf16 or f16
 * (one dtype); O is that dtype or f32 (o_dtype; the reference's tiled
 * attention writes f32 O, tiled_attention.py:658-683).  head_dim is 16, 32,
 * 64 or 128.  The softmax statistics are f32.  Strides are in elements; the
 * innermost (head_dim) stride is 1.  lse, if non-NULL, receives the f32
 * natural-log row log-sum-exp of the scaled scores, laid out
 * [batch, heads, seq_q] contiguous.
 *
 * k_transposed = 1 takes K stored [batch, heads, head_dim, seq_k] with unit
 * key stride (the layout of the reference's FA tile program, K as
 * memref<1x32x128x4096>, tmp/ir.mlir:89-92); k_stride_s is then the stride
 * between head_dim rows (at least seq_k), and seq_k must be even (odd:
 * FRISK_EUNSUP).  The kernel reads it in place.
 */
typedef struct frisk_attn_desc {
  int64_t batch, heads, seq_q, seq_k, head_dim;
  int32_t dtype; /* frisk_dtype: FRISK_BF16 or FRISK_F16 */
  int32_t causal;
  float sm_scale;
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_s;
  const void* k;
  int64_t k_stride_b, k_stride_h, k_stride_s;
  const void* v;
  int64_t v_stride_b, v_stride_h, v_stride_s;
  void* o;
  int64_t o_stride_b, o_stride_h, o_stride_s;
  float* lse;
  int32_t o_dtype;      /* frisk_dtype: equal to dtype, or FRISK_F32 */
  int32_t k_transposed; /* 0: K [b, h, seq_k, head_dim]; 1: K [b, h, head_dim, seq_k] */
  /* Waves per workgroup (32 queries each): 0, the library chooses (the
   * launch contract layout inference gives an attention program); 4 or 8
   * (8 needs head_dim 128).  The result bits do not depend on it. */
  int32_t waves;
} frisk_attn_desc;

int frisk_attn_fwd(const frisk_attn_desc* desc, void* stream);

/* Reduction kinds (frisk.reduce "add"/"max"/"min", reduce_tensor "sum"/...). */
typedef enum frisk_reduce_kind {
  FRISK_REDUCE_SUM = 0,
  FRISK_REDUCE_MAX = 1,
  FRISK_REDUCE_MIN = 2
} frisk_reduce_kind;

/*
 * Reduction of src[rows, cols] (row stride ld_src) along `axis`:
 *   axis 1:  dst[r * dst_stride] = reduce over c of src[r, c]   (rows outputs)
 *   axis 0:  dst[c * dst_stride] = reduce over r of src[r, c]   (cols outputs)
 * clear == 0 merges with the destination's old value:
 *   dst = combine(dst, reduction)   (frisk.reduce with clear = false).
 * dtype is f32, f16 or bf16 for both src and dst, and every combine is done
 * in it: a sum is rounded to dtype after each addition.  Sums associate as
 * the canonical pairwise tree over the reduced index in ascending order
 * (adjacent pairs first, an odd last node carried up), so results are
 * deterministic and independent of the launch shape.  max / min propagate
 * NaN and order -0.0 below +0.0.  src and dst must not overlap; pointers are
 * element-aligned.  Limits: rows, cols < 2^31; axis 0 needs rows < 2^23.
 *
 * leaf_order_bits > 0 selects another leaf order, that of a distributed
 * layout whose reduced-axis bits sit on single carrier bits (the fibers of
 * canonical_fiber_tree_v1, ReductionLayoutProof.cpp:119-124): the reduced
 * extent must be 2^leaf_order_bits, leaf_order[0..bits) is a permutation of
 * 0..bits-1, and leaf position p holds reduced index
 * sum_j ((p >> j) & 1) << leaf_order[j].  This path runs one thread per
 * output and is meant for tile-sized reductions.
 *
 * workspace / workspace_bytes: optional device scratch (16-byte aligned)
 * owned by the caller.  An axis-0 reduction of many rows with at least
 * frisk_reduce_workspace_size() bytes splits the rows over the whole GPU
 * in two passes (same tree, same result); without it, or when the size is
 * 0, one pass runs.  Calls that share a workspace must not overlap.
 */
typedef struct frisk_reduce_desc {
  int64_t rows, cols;
  int32_t dtype; /* frisk_dtype: FRISK_F32, FRISK_F16 or FRISK_BF16 */
  int32_t kind;  /* frisk_reduce_kind */
  int32_t axis;  /* 0 or 1 */
  int32_t clear;
  const void* src;
  int64_t ld_src;
  void* dst;
  int64_t dst_stride;
  int32_t leaf_order_bits; /* 0: ascending index order */
  uint8_t leaf_order[32];
  void* workspace;         /* optional, may be NULL */
  int64_t workspace_bytes;
} frisk_reduce_desc;

int frisk_reduce(const frisk_reduce_desc* desc, void* stream);

/* Workspace bytes that make frisk_reduce(desc) take its two-pass path (0:
 * none is used), or a negative FRISK_E* code for an invalid descriptor.
 * Pointers in desc are not read. */
int64_t frisk_reduce_workspace_size(const frisk_reduce_desc* desc);

/*
 * dst[r, c] = convert(src[r, c]) for a [rows, cols] tile (row strides
 * ld_src, ld_dst in elements).  Equal types copy the elements unchanged (any
 * frisk_dtype).  Otherwise src_type and dst_type are f32, f16, bf16 or e4m3:
 * widening is exact and narrowing rounds to nearest even (arith.truncf);
 * f16 and bf16 overflow to infinity, e4m3 (no infinity) to NaN.  src and dst
 * must not overlap.
 */
typedef struct frisk_copy_desc {
  int64_t rows, cols;
  int32_t src_type, dst_type; /* frisk_dtype */
  const void* src;
  int64_t ld_src;
  void* dst;
  int64_t ld_dst;
} frisk_copy_desc;

int frisk_copy(const frisk_copy_desc* desc, void* stream);

/*
 * dst[r, c] = value for a [rows, cols] tile (row stride ld).  For float
 * dtypes `value` is rounded to nearest even in dtype (e4m3: values past 464
 * in magnitude become NaN); for i8 / i32 it must be an integer in range.
 */
typedef struct frisk_fill_desc {
  int64_t rows, cols;
  int32_t dtype; /* frisk_dtype */
  double value;
  void* dst;
  int64_t ld;
} frisk_fill_desc;

int frisk_fill(const frisk_fill_desc* desc, void* stream);

/* Description of the last failure on the calling thread ("" if none). */
const char* frisk_last_error(void);

/* FRISK_ABI_VERSION of the loaded library. */
int frisk_abi_version(void);

/* MFMA fragment-layout probe.  No counterpart in the reference, whose SM90
 * fragment maps are pinned by golden rows (SM90MmaLayoutProofTest.cpp:10-82);
 * this one pins the CDNA4 maps the kernels use on the device itself.  Runs
 * one atom (0 = v_mfma_f32_32x32x16_bf16, 1 = v_mfma_f32_16x16x32_bf16,
 * 2 = v_mfma_i32_32x32x32_i8) for every k0 in [0, K) on operands with
 * A[i][k0] = i, A[i][k0+1] = S, B[k0][j] = 1, B[k0+1][j] = j (S = 64, or 32
 * for i8) and writes accumulator register r of lane L for k0 to
 * out[(k0 * 64 + L) * R + r] (R = 16, 4, 16), i.e. the value i + S j of the
 * element it holds.  `out` is a device buffer of at least K * 64 * R floats
 * (16384, 8192 and 32768). */
int frisk_probe_mfma_layout(int atom, float* out, int64_t out_floats, void* stream);

/* Transposing LDS read probe: LDS holds the identity pattern, every lane of
 * one wave addresses the 8 bytes at lane * 8 through ds_read_b64_tr_b16
 * (bits 16: out[lane * 4 + e] = the 16-bit element id returned as element
 * e, 256 values) or ds_read_b64_tr_b8 (bits 8: out[lane * 8 + e] = the byte
 * address returned as byte e, 512 values).  Pins the lane map the GEMM
 * kernels assume for M/N-major operands.  No counterpart in the reference
 * (SM90 has no such instruction). */
int frisk_probe_lds_transpose(int bits, uint16_t* out, int64_t out_elems, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FRISK_HIP_H */
