/*
 * frisk_hip.h — C-ABI of the MI355X (gfx950) GEMM and attention kernels.
 *
 * The reference (guoqiao7/frisk) has no execute entry in its FFI: the
 * pass/execute bindings are commented out at ffi/ffi.h:14 and ffi/ffi.cpp:6,
 * and the only GPU path is the out-of-process harness
 * benchmark/layout/execution/run_execution.py:23-95 (frisk-opt -> JSON ->
 * Triton).  These entry points are what that FFI would bind for the GEMM and
 * attention tile programs:
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

#define FRISK_ABI_VERSION 2

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
} frisk_gemm_desc;

int frisk_gemm(const frisk_gemm_desc* desc, void* stream);

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
  int32_t o_dtype; /* frisk_dtype: equal to dtype, or FRISK_F32 */
} frisk_attn_desc;

int frisk_attn_fwd(const frisk_attn_desc* desc, void* stream);

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

#ifdef __cplusplus
}
#endif

#endif /* FRISK_HIP_H */
