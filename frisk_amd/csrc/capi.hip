// C-ABI of libfrisk_hip.so: request validation and kernel dispatch.
//
// Validation mirrors the reference's GEMM contract
// (lib/Dialect/Frisk/IR/LegacyImportSemantics.cpp:11-46: positive M/N/K, A and
// B of one element type, C equal to it or f32 for f16/bf16) widened to the
// int8->int32 and fp8->{f32,bf16,f16} pairs; a request that fails it returns
// FRISK_EINVAL before anything is launched, so outputs are never partially
// written ("validate before publish", PassPipelines.cpp:128-208).

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/frisk_hip.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FRISK_EHIP, "%s: %s", what, hipGetErrorString(e));
}

const char* dtype_name(int t) {
  switch (t) {
    case FRISK_F32: return "f32";
    case FRISK_F16: return "f16";
    case FRISK_BF16: return "bf16";
    case FRISK_E4M3: return "e4m3";
    case FRISK_I8: return "i8";
    case FRISK_I32: return "i32";
    case FRISK_F64: return "f64";
    default: return "?";
  }
}

int esize(int t) {
  switch (t) {
    case FRISK_F32: case FRISK_I32: return 4;
    case FRISK_F16: case FRISK_BF16: return 2;
    case FRISK_E4M3: case FRISK_I8: return 1;
    case FRISK_F64: return 8;
    default: return 0;
  }
}

bool gemm_pair_ok(int in, int out) {
  switch (in) {
    case FRISK_F32: return out == FRISK_F32;
    case FRISK_F16: return out == FRISK_F16 || out == FRISK_F32;
    case FRISK_BF16: return out == FRISK_BF16 || out == FRISK_F32;
    case FRISK_E4M3: return out == FRISK_BF16 || out == FRISK_F16 || out == FRISK_F32;
    case FRISK_I8: return out == FRISK_I32;
    default: return false;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

const char* frisk_last_error(void) { return g_last_error.c_str(); }

int frisk_abi_version(void) { return FRISK_ABI_VERSION; }

int frisk_gemm(const frisk_gemm_desc* d, void* stream) {
  g_last_error.clear();
  if (!d) return fail(FRISK_EINVAL, "frisk_gemm: null descriptor");
  if (d->m <= 0 || d->n <= 0 || d->k <= 0)
    return fail(FRISK_EINVAL, "legacy-gemm-shape: M, N, and K must be positive (got %lld, %lld, %lld)",
                (long long)d->m, (long long)d->n, (long long)d->k);
  if (d->a_type != d->b_type)
    return fail(FRISK_EINVAL, "legacy-gemm-type: A and B must have the same element type (%s vs %s)",
                dtype_name(d->a_type), dtype_name(d->b_type));
  if (!gemm_pair_ok(d->a_type, d->c_type))
    return fail(FRISK_EINVAL, "legacy-gemm-type: unsupported A/B -> C element types %s -> %s",
                dtype_name(d->a_type), dtype_name(d->c_type));
  if (!d->a || !d->b || !d->c) return fail(FRISK_EINVAL, "frisk_gemm: null operand pointer");
  const int64_t a_cols = d->trans_a ? d->m : d->k;
  const int64_t b_cols = d->trans_b ? d->k : d->n;
  if (d->lda < a_cols || d->ldb < b_cols || d->ldc < d->n)
    return fail(FRISK_EINVAL, "frisk_gemm: leading dimension too small (lda %lld < %lld, ldb %lld < %lld or ldc %lld < %lld)",
                (long long)d->lda, (long long)a_cols, (long long)d->ldb, (long long)b_cols,
                (long long)d->ldc, (long long)d->n);
  const bool fp8 = d->a_type == FRISK_E4M3;
  if (!fp8 && (d->scale_a != 1.0f || d->scale_b != 1.0f))
    return fail(FRISK_EINVAL, "frisk_gemm: scale_a/scale_b apply to fp8 inputs only");
  if (d->m > INT32_MAX / 2 || d->n > INT32_MAX / 2 || d->k > INT32_MAX / 16)
    return fail(FRISK_EUNSUP, "frisk_gemm: dimension beyond the 32-bit index range of the kernels");
  if (d->a_type == FRISK_I8 && d->k > 133152)
    // |sum| <= K * 127 * 128 must stay below 2^31 for exact int32 results.
    return fail(FRISK_EUNSUP, "frisk_gemm: int8 K=%lld could overflow the int32 accumulator",
                (long long)d->k);

  frisk::GemmArgs g;
  g.in = (frisk::Elt)d->a_type;
  g.out = (frisk::Elt)d->c_type;
  g.m = d->m; g.n = d->n; g.k = d->k;
  g.trans_a = d->trans_a != 0; g.trans_b = d->trans_b != 0;
  g.a = d->a; g.lda = d->lda;
  g.b = d->b; g.ldb = d->ldb;
  g.c = d->c; g.ldc = d->ldc;
  g.scale = fp8 ? d->scale_a * d->scale_b : 1.0f;
  g.accumulate = d->clear_accum ? 0 : 1;

  const int ies = esize(d->a_type), oes = esize(d->c_type);
  const bool mfma_type = d->a_type != FRISK_F32;
  const bool tn = !g.trans_a && g.trans_b;
  const bool vec_ok = (d->k * ies) % 16 == 0 && (d->lda * ies) % 16 == 0 &&
                      (d->ldb * ies) % 16 == 0 && aligned16(d->a) && aligned16(d->b) &&
                      aligned16(d->c) && (d->ldc * oes) % 16 == 0 && d->n % 8 == 0;
  hipError_t e;
  if (mfma_type && tn && vec_ok && frisk::gemm_skinny_supported(g))
    e = frisk::gemm_skinny(g, (hipStream_t)stream);
  else if (mfma_type && tn && vec_ok) e = frisk::gemm_tn_mfma(g, (hipStream_t)stream);
  else e = frisk::gemm_generic_any(g, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_gemm launch");
  return FRISK_OK;
}

int frisk_attn_fwd(const frisk_attn_desc* d, void* stream) {
  g_last_error.clear();
  if (!d) return fail(FRISK_EINVAL, "frisk_attn_fwd: null descriptor");
  if (d->batch <= 0 || d->heads <= 0 || d->seq_q <= 0 || d->seq_k <= 0 || d->head_dim <= 0)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: sizes must be positive");
  if (d->dtype != FRISK_BF16 && d->dtype != FRISK_F16)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: dtype must be bf16 or f16 (got %s)",
                dtype_name(d->dtype));
  if (d->o_dtype != d->dtype && d->o_dtype != FRISK_F32)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: o_dtype must be the input dtype or f32 (got %s)",
                dtype_name(d->o_dtype));
  if (d->head_dim != 16 && d->head_dim != 32 && d->head_dim != 64 && d->head_dim != 128)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: head_dim %lld not supported (16, 32, 64, 128)",
                (long long)d->head_dim);
  if (!d->q || !d->k || !d->v || !d->o) return fail(FRISK_EINVAL, "frisk_attn_fwd: null tensor");
  if (!aligned16(d->q) || !aligned16(d->k) || !aligned16(d->v) || !aligned16(d->o))
    return fail(FRISK_EINVAL, "frisk_attn_fwd: Q/K/V/O must be 16-byte aligned");
  const int64_t strides[12] = {d->q_stride_b, d->q_stride_h, d->q_stride_s,
                               d->k_stride_b, d->k_stride_h, d->k_stride_s,
                               d->v_stride_b, d->v_stride_h, d->v_stride_s,
                               d->o_stride_b, d->o_stride_h, d->o_stride_s};
  for (int i = 0; i < 12; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return fail(FRISK_EINVAL, "frisk_attn_fwd: strides must be non-negative multiples of 8 elements");
  if (d->q_stride_s < d->head_dim || d->k_stride_s < d->head_dim ||
      d->v_stride_s < d->head_dim || d->o_stride_s < d->head_dim)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: sequence stride smaller than head_dim");
  if (!(d->sm_scale > 0.0f) || !__builtin_isfinite(d->sm_scale))
    return fail(FRISK_EINVAL, "frisk_attn_fwd: sm_scale must be positive and finite");
  if (d->seq_q > INT32_MAX / 2 || d->seq_k > INT32_MAX / 2 || d->batch * d->heads > INT32_MAX / 2)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: sizes beyond the 32-bit index range");

  frisk::AttnArgs a;
  a.dtype = (frisk::Elt)d->dtype;
  a.out = (frisk::Elt)d->o_dtype;
  a.batch = d->batch; a.heads = d->heads; a.seq_q = d->seq_q; a.seq_k = d->seq_k;
  a.head_dim = d->head_dim;
  a.causal = d->causal != 0;
  a.sm_scale = d->sm_scale;
  a.q = d->q; a.q_sb = d->q_stride_b; a.q_sh = d->q_stride_h; a.q_ss = d->q_stride_s;
  a.k = d->k; a.k_sb = d->k_stride_b; a.k_sh = d->k_stride_h; a.k_ss = d->k_stride_s;
  a.v = d->v; a.v_sb = d->v_stride_b; a.v_sh = d->v_stride_h; a.v_ss = d->v_stride_s;
  a.o = d->o; a.o_sb = d->o_stride_b; a.o_sh = d->o_stride_h; a.o_ss = d->o_stride_s;
  a.lse = d->lse;
  hipError_t e = frisk::attn_fwd(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_attn_fwd launch");
  return FRISK_OK;
}

int frisk_probe_mfma_layout(int atom, float* out, int64_t out_floats, void* stream) {
  const int need = frisk::mfma_probe_floats(atom);
  if (need == 0) return fail(FRISK_EINVAL, "mfma-probe: unknown atom %d (0, 1 or 2)", atom);
  if (!out) return fail(FRISK_EINVAL, "mfma-probe: null output");
  if (out_floats < need)
    return fail(FRISK_EINVAL, "mfma-probe: atom %d writes %d floats, buffer holds %lld", atom, need,
                (long long)out_floats);
  hipError_t e = frisk::mfma_layout_probe(atom, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "mfma-probe launch");
  return FRISK_OK;
}

}  // extern "C"
