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

#include <algorithm>
#include <cmath>
#include <mutex>
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

// Resets the calling thread's HIP error state before a launch, so that the
// hipGetLastError() after it reports that launch only, not a failure left
// behind by an unrelated earlier HIP call.
void clear_stale_error() { (void)hipGetLastError(); }

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

// Bit pattern of `v` rounded to nearest even in a float format with `mant`
// explicit mantissa bits, `ebits` exponent bits (bias 2^(ebits-1) - 1) and
// `max_finite`; without infinities (e4m3fn) overflow and NaN give the
// all-ones NaN.  Mirrors how a fill value becomes a FloatAttr of the tile's
// element type (ffi/ir.cpp:439-454).
uint64_t float_bits(double v, int mant, int ebits, double max_finite, bool has_inf) {
  const int bias = (1 << (ebits - 1)) - 1, emin = 1 - bias;
  const uint64_t sign = std::signbit(v) ? 1ull << (mant + ebits) : 0;
  const uint64_t emask = (1ull << ebits) - 1;
  const uint64_t nan = has_inf ? (emask << mant) | (1ull << (mant - 1)) : (emask << mant) | ((1ull << mant) - 1);
  if (std::isnan(v)) return nan;
  double a = std::fabs(v);
  if (std::isinf(a)) return has_inf ? sign | (emask << mant) : sign | nan;
  if (a == 0.0) return sign;
  int e2;
  std::frexp(a, &e2);
  const int e = std::max(e2 - 1, emin);
  const double q = std::ldexp(1.0, e - mant);
  const double r = std::nearbyint(a / q) * q;  // ties to even
  if (r > max_finite) return has_inf ? sign | (emask << mant) : sign | nan;
  int re;
  std::frexp(r, &re);
  if (re - 1 < emin) return sign | (uint64_t)(r / std::ldexp(1.0, emin - mant));  // subnormal
  const uint64_t field = (uint64_t)(re - 1 + bias);
  const uint64_t frac = (uint64_t)((r / std::ldexp(1.0, re - 1) - 1.0) * std::ldexp(1.0, mant));
  return sign | (field << mant) | frac;
}

bool fill_bits(int dtype, double v, uint64_t* out) {
  switch (dtype) {
    case FRISK_F64: { uint64_t b; memcpy(&b, &v, 8); *out = b; return true; }
    case FRISK_F32: *out = float_bits(v, 23, 8, 3.4028234663852886e38, true); return true;
    case FRISK_F16: *out = float_bits(v, 10, 5, 65504.0, true); return true;
    case FRISK_BF16: *out = float_bits(v, 7, 8, 3.3895313892515355e38, true); return true;
    case FRISK_E4M3: *out = float_bits(v, 3, 4, 448.0, false); return true;
    case FRISK_I8:
      if (!(v == std::floor(v) && v >= -128.0 && v <= 127.0)) return false;
      *out = (uint8_t)(int8_t)v;
      return true;
    case FRISK_I32:
      if (!(v == std::floor(v) && v >= -2147483648.0 && v <= 2147483647.0)) return false;
      *out = (uint32_t)(int32_t)v;
      return true;
    default: return false;
  }
}

}  // namespace

extern "C" {

const char* frisk_last_error(void) { return g_last_error.c_str(); }

int frisk_abi_version(void) { return FRISK_ABI_VERSION; }

}  // extern "C"

namespace {

// Which kernel family a GEMM descriptor goes to (launch_plan.h).
using GemmRoute = frisk::plan::Route;

// Rows of the largest operand tile a GEMM kernel addresses from one buffer
// base (the 256x256 tiles).
constexpr int64_t kMaxTileRows = 256;

// Checks of frisk_gemm / frisk_gemm_workspace_size / frisk_gemm_plan, the
// kernel arguments and the route; 0 or an error code.  With ptrs == false
// the operand pointers are not required; when all three are given their
// alignment still counts (they are never read).
int check_gemm(const frisk_gemm_desc* d, const char* fn, bool ptrs, frisk::GemmArgs& g,
               GemmRoute& route) {
  if (!d) return fail(FRISK_EINVAL, "%s: null descriptor", fn);
  if (d->m <= 0 || d->n <= 0 || d->k <= 0)
    return fail(FRISK_EINVAL, "legacy-gemm-shape: M, N, and K must be positive (got %lld, %lld, %lld)",
                (long long)d->m, (long long)d->n, (long long)d->k);
  if (d->a_type != d->b_type)
    return fail(FRISK_EINVAL, "legacy-gemm-type: A and B must have the same element type (%s vs %s)",
                dtype_name(d->a_type), dtype_name(d->b_type));
  if (!gemm_pair_ok(d->a_type, d->c_type))
    return fail(FRISK_EINVAL, "legacy-gemm-type: unsupported A/B -> C element types %s -> %s",
                dtype_name(d->a_type), dtype_name(d->c_type));
  if (ptrs && (!d->a || !d->b || !d->c)) return fail(FRISK_EINVAL, "%s: null operand pointer", fn);
  const int64_t a_cols = d->trans_a ? d->m : d->k;
  const int64_t b_cols = d->trans_b ? d->k : d->n;
  if (d->lda < a_cols || d->ldb < b_cols || d->ldc < d->n)
    return fail(FRISK_EINVAL, "%s: leading dimension too small (lda %lld < %lld, ldb %lld < %lld or ldc %lld < %lld)",
                fn, (long long)d->lda, (long long)a_cols, (long long)d->ldb, (long long)b_cols,
                (long long)d->ldc, (long long)d->n);
  const bool fp8 = d->a_type == FRISK_E4M3;
  if (!fp8 && (d->scale_a != 1.0f || d->scale_b != 1.0f))
    return fail(FRISK_EINVAL, "%s: scale_a/scale_b apply to fp8 inputs only", fn);
  if (d->m > INT32_MAX / 2 || d->n > INT32_MAX / 2 || d->k > INT32_MAX / 16)
    return fail(FRISK_EUNSUP, "%s: dimension beyond the 32-bit index range of the kernels", fn);
  if (d->a_type == FRISK_I8 && d->k > INT32_MAX / (128 * 128))
    // Every product of two int8 values has |a b| <= 128 * 128 = 2^14, so
    // K <= (2^31 - 1) / 2^14 = 131071 keeps every int32 sum exact.
    return fail(FRISK_EUNSUP, "%s: int8 K=%lld could overflow the int32 accumulator (K <= 131071)",
                fn, (long long)d->k);
  if (d->workspace_bytes < 0) return fail(FRISK_EINVAL, "%s: negative workspace_bytes", fn);

  g.in = (frisk::Elt)d->a_type;
  g.out = (frisk::Elt)d->c_type;
  g.m = d->m; g.n = d->n; g.k = d->k;
  g.trans_a = d->trans_a != 0; g.trans_b = d->trans_b != 0;
  g.a = d->a; g.lda = d->lda;
  g.b = d->b; g.ldb = d->ldb;
  g.c = d->c; g.ldc = d->ldc;
  g.scale = fp8 ? d->scale_a * d->scale_b : 1.0f;
  g.accumulate = d->clear_accum ? 0 : 1;

  // The MFMA kernels stage 16 B pieces of operand rows: 16 B aligned bases
  // and row pitches, and for an operand stored K-major (A not transposed, B
  // transposed) whole 16 B pieces of K; the epilogue stores 16 B per lane
  // into C rows.  Their buffer loads take 32-bit offsets from one tile
  // origin: a K-major operand reaches (rows - 1) pitches plus K, an MN-major
  // one (K - 1) pitches plus a tile row; beyond 2^31 - 1 bytes the generic
  // kernel (64-bit indexing) runs instead.
  const int ies = esize(d->a_type), oes = esize(d->c_type);
  const bool a_kmajor = !g.trans_a, b_kmajor = g.trans_b;
  // Pointers are never dereferenced here; when a query (ptrs == false)
  // passes them anyway, their alignment takes part as in the call.
  const bool have_ptrs = d->a && d->b && d->c;
  const bool aligned = !(ptrs || have_ptrs) || (aligned16(d->a) && aligned16(d->b) && aligned16(d->c));
  const bool k_pieces = (!a_kmajor && !b_kmajor) || (d->k * ies) % 16 == 0;
  const bool vec_ok = aligned && k_pieces && (d->lda * ies) % 16 == 0 &&
                      (d->ldb * ies) % 16 == 0 && (d->ldc * oes) % 16 == 0;
  auto reach = [&](bool kmajor, int64_t ld) {
    return kmajor ? (kMaxTileRows - 1) * ld * ies + d->k * ies
                  : (d->k - 1) * ld * ies + kMaxTileRows * ies;
  };
  const bool offsets_ok = reach(a_kmajor, d->lda) <= INT32_MAX && reach(b_kmajor, d->ldb) <= INT32_MAX;
  const bool matrix_cores = vec_ok && offsets_ok;  // every type pair, f32 included, has MFMA kernels

  // A requested kernel variant: the named tile and wave grid, unsplit or in
  // the K slices the request names.
  if (d->slices < 0 || d->slices > 64)
    return fail(FRISK_EINVAL, "%s: slices %d outside 0..64", fn, (int)d->slices);
  if (d->slices > 1 && !d->tile)
    return fail(FRISK_EINVAL, "%s: slices name a split of a requested variant (set tile)", fn);
  if (d->tile || d->wave_m || d->wave_n || d->variant_flags) {
    const int wm = d->wave_m ? d->wave_m : 2, wn = d->wave_n ? d->wave_n : 2;
    const bool grid_pair = (d->wave_m == 0) == (d->wave_n == 0);
    const bool ok256 = d->tile == 256 && wm == 2 && wn == 2;
    const bool ok128 = d->tile == 128 && ((wm == 2 && wn == 2) || (wm == 4 && wn == 1) ||
                                          (wm == 1 && wn == 4) || (wm == 2 && wn == 1) ||
                                          (wm == 1 && wn == 2));
    if (d->variant_flags != 0 || !grid_pair || !(ok256 || ok128))
      return fail(FRISK_EINVAL,
                  "%s: no kernel variant tile=%d wave grid %dx%d (flags %d): 256 with 2x2, or 128 "
                  "with 2x2, 4x1, 1x4, 2x1 or 1x2",
                  fn, (int)d->tile, (int)d->wave_m, (int)d->wave_n, (int)d->variant_flags);
    if (!matrix_cores)
      return fail(FRISK_EUNSUP,
                  "%s: the %dx%d-tile variant runs on the matrix cores only: "
                  "16-byte aligned operands and row pitches, whole 16-byte pieces of K in a "
                  "K-contiguous operand, operand reach below 2^31 bytes",
                  fn, (int)d->tile, (int)d->tile);
    if (d->slices > 1 && !(wm == 2 && wn == 2 &&
                           (d->a_type == FRISK_BF16 || d->a_type == FRISK_F16 ||
                            d->a_type == FRISK_F32) && d->n % 4 == 0))
      return fail(FRISK_EUNSUP,
                  "%s: a split variant needs the 2x2 wave grid, bf16/f16/f32 inputs and N %% 4 "
                  "== 0 (got %dx%d, %s, N %lld)",
                  fn, wm, wn, dtype_name(d->a_type), (long long)d->n);
    g.tile = d->tile;
    g.wave_m = wm;
    g.wave_n = wn;
    g.slices = d->slices;
  }
  route = frisk::plan::route_of(frisk::shape_of(g), matrix_cores);
  return 0;
}

using frisk::plan::kSkinnySplitMaxM;

// Workspace bytes of the split-K plan frisk_gemm follows (0: none).
int64_t gemm_workspace(const frisk::GemmArgs& g, GemmRoute route) {
  return frisk::plan::workspace_bytes(frisk::shape_of(g), route, frisk::device_cus());
}

// K bytes per lane row of one MFMA atom (the atom's k times the element size).
int atom_k_bytes(frisk::Elt in) {
  switch (in) {
    case frisk::Elt::BF16:
    case frisk::Elt::F16: return 32;  // 32x32x16
    case frisk::Elt::E4M3: return 64;  // 32x32x64
    case frisk::Elt::I8: return 32;  // 32x32x32
    case frisk::Elt::F32: return 32;  // four 32x32x2 per 8 k
    default: return 0;
  }
}

const char* mfma_atom(frisk::Elt in) {
  switch (in) {
    case frisk::Elt::BF16: return "v_mfma_f32_32x32x16_bf16";
    case frisk::Elt::F16: return "v_mfma_f32_32x32x16_f16";
    case frisk::Elt::E4M3: return "v_mfma_f32_32x32x64_f8f6f4";
    case frisk::Elt::I8: return "v_mfma_i32_32x32x32_i8";
    case frisk::Elt::F32: return "v_mfma_f32_32x32x2_f32";
    default: return "";
  }
}

// Launches a validated GEMM on its route with an optional split-K scratch.
int launch_gemm(const frisk::GemmArgs& g, GemmRoute route, void* ws, int64_t ws_bytes,
                void* stream, const char* fn) {
  clear_stale_error();
  hipError_t e;
  if (route == GemmRoute::Skinny && ws && g.m > kSkinnySplitMaxM) {
    e = frisk::gemm_mfma(g, (hipStream_t)stream, ws, ws_bytes);
  } else if (route == GemmRoute::Skinny) {
    e = frisk::gemm_skinny(g, (hipStream_t)stream, ws, ws_bytes);
  } else if (route == GemmRoute::Mfma) {
    e = frisk::gemm_mfma(g, (hipStream_t)stream, ws, ws_bytes);
  } else {
    e = frisk::gemm_generic_any(g, (hipStream_t)stream);
  }
  if (e != hipSuccess) return fail(FRISK_EHIP, "%s launch: %s", fn, hipGetErrorString(e));
  return FRISK_OK;
}

}  // namespace

extern "C" {

int64_t frisk_gemm_workspace_size(const frisk_gemm_desc* d) {
  g_last_error.clear();
  frisk::GemmArgs g;
  GemmRoute route;
  const int rc = check_gemm(d, "frisk_gemm_workspace_size", false, g, route);
  if (rc) return rc;
  return gemm_workspace(g, route);
}

int frisk_gemm_plan(const frisk_gemm_desc* d, char* buf, int64_t len) {
  g_last_error.clear();
  frisk::GemmArgs g;
  GemmRoute route;
  const int rc = check_gemm(d, "frisk_gemm_plan", false, g, route);
  if (rc) return rc;
  if (!buf || len <= 0) return fail(FRISK_EINVAL, "frisk_gemm_plan: no output buffer");
  const frisk::plan::GemmLaunch L =
      frisk::plan::launch_of(frisk::shape_of(g), route, frisk::device_cus(), d->workspace_bytes);
  const int ies = esize(d->a_type);
  const char* a_major = g.trans_a ? "m" : "k";
  const char* b_major = g.trans_b ? "k" : "n";
  auto lds_read = [&](bool mn) {
    return !mn ? "ds_read_b128"
           : ies == 4 ? "ds_read_b32"
           : ies == 2 ? "ds_read_b64_tr_b16" : "ds_read_b64_tr_b8";
  };
  const char* slice_sum = L.slice_sum == frisk::plan::SliceSum::InLaunch ? "in_launch"
                          : L.slice_sum == frisk::plan::SliceSum::SecondLaunch ? "second_launch"
                                                                              : "none";
  int n = 0;
  if (L.kernel == frisk::plan::Kernel::Generic) {
    n = snprintf(buf, (size_t)len,
                 "{\"kernel\": \"gemm_generic\", \"tile_m\": 64, \"tile_n\": 64, \"atom\": \"fma\", "
                 "\"a_major\": \"%s\", \"b_major\": \"%s\", \"slices\": 1, \"slice_sum\": \"none\", "
                 "\"workspace_bytes\": 0}",
                 a_major, b_major);
  } else if (L.kernel == frisk::plan::Kernel::Skinny) {
    n = snprintf(buf, (size_t)len,
                 "{\"kernel\": \"gemm_skinny\", \"tile_m\": %d, \"tile_n\": %d, "
                 "\"atom\": \"v_mfma_f32_16x16x32_%s\", \"waves\": [1, 1], \"a_major\": \"k\", "
                 "\"b_major\": \"k\", \"slices\": %d, \"slice_sum\": \"%s\", "
                 "\"workspace_bytes\": %lld}",
                 L.tile_m, L.tile_n, d->a_type == FRISK_BF16 ? "bf16" : "f16", L.slices, slice_sum,
                 (long long)L.workspace_bytes);
  } else {
    const bool big = L.kernel == frisk::plan::Kernel::W4;
    const int tile = L.tile_m, wm = L.wave_m, wn = L.wave_n;
    // The workgroup tile's instruction contract in the solver's syntax
    // (#frisk.mma_contract): the 256x256 kernel feeds the B fragment as the
    // MFMA's first operand (swapped), the 128x128 kernel does not.
    const char* policy = wm == wn ? "Square" : wn == 1 ? "FullRow" : "FullCol";
    n = snprintf(buf, (size_t)len,
                 "{\"kernel\": \"%s\", \"tile_m\": %d, \"tile_n\": %d, \"atom\": \"%s\", "
                 "\"waves\": [%d, %d], \"wave_tile\": [%d, %d], \"stage_bytes\": %d, "
                 "\"a_major\": \"%s\", \"b_major\": \"%s\", \"lds_read_a\": \"%s\", "
                 "\"lds_read_b\": \"%s\", \"lds_swizzle_a\": \"%s\", \"lds_swizzle_b\": \"%s\", "
                 "\"slices\": %d, \"slice_sum\": \"%s\", \"workspace_bytes\": %lld, "
                 "\"requested\": %s, \"mma_contract\": \"{atom = \\\"%s\\\", wave_grid = [%d, %d], "
                 "repeats = [%d, %d, %d], policy = \\\"%s\\\", swapped = %s}\"}",
                 big ? "gemm_w4" : "gemm_128", tile, tile, mfma_atom(g.in), wm, wn, tile / wm,
                 tile / wn, L.stage_bytes, a_major, b_major, lds_read(g.trans_a), lds_read(!g.trans_b),
                 frisk::plan::lds_swizzle(g.trans_a, ies, L.stage_bytes, tile * ies),
                 frisk::plan::lds_swizzle(!g.trans_b, ies, L.stage_bytes, tile * ies), L.slices,
                 slice_sum, (long long)L.workspace_bytes, L.requested ? "true" : "false",
                 mfma_atom(g.in), wm, wn, tile / wm / 32, tile / wn / 32,
                 L.stage_bytes / atom_k_bytes(g.in), policy, big ? "true" : "false");
  }
  if (n < 0 || n >= len)
    return fail(FRISK_EINVAL, "frisk_gemm_plan: buffer of %lld bytes is too small", (long long)len);
  return FRISK_OK;
}

int frisk_gemm(const frisk_gemm_desc* d, void* stream) {
  g_last_error.clear();
  frisk::GemmArgs g;
  GemmRoute route;
  const int rc = check_gemm(d, "frisk_gemm", true, g, route);
  if (rc) return rc;
  void* ws = nullptr;
  int64_t ws_bytes = 0;
  if (d->workspace) {
    const int64_t need = gemm_workspace(g, route);
    if (need > 0) {
      if (d->workspace_bytes < need)
        return fail(FRISK_EINVAL, "frisk_gemm: workspace of %lld bytes, this GEMM takes %lld",
                    (long long)d->workspace_bytes, (long long)need);
      if ((uintptr_t)d->workspace % 16)
        return fail(FRISK_EINVAL, "frisk_gemm: workspace must be 16-byte aligned");
      ws = d->workspace;
      ws_bytes = d->workspace_bytes;
    }
  }
  return launch_gemm(g, route, ws, ws_bytes, stream, "frisk_gemm");
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
  if (d->k_transposed != 0 && d->k_transposed != 1)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: k_transposed must be 0 or 1 (got %d)",
                (int)d->k_transposed);
  const bool kt = d->k_transposed != 0;
  if (d->q_stride_s < d->head_dim || (!kt && d->k_stride_s < d->head_dim) ||
      d->v_stride_s < d->head_dim || d->o_stride_s < d->head_dim)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: sequence stride smaller than head_dim");
  if (kt && d->k_stride_s < d->seq_k)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: transposed K needs a head_dim row stride of at "
                              "least seq_k (got %lld < %lld)",
                (long long)d->k_stride_s, (long long)d->seq_k);
  // The loads of a transposed K stop at its last key with 4-byte
  // granularity (a buffer range check zeroes each dword that extends past
  // the end), so with an odd seq_k the last key of the last head_dim row
  // would share a zeroed dword with the element after it.
  if (d->waves != 0 && d->waves != 4 && d->waves != 8)
    return fail(FRISK_EINVAL, "frisk_attn_fwd: waves must be 0, 4 or 8 (got %d)", (int)d->waves);
  if (d->waves == 8 && d->head_dim != 128)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: 8-wave workgroups run head_dim 128 only (got %lld)",
                (long long)d->head_dim);
  if (kt && d->seq_k % 2 != 0)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: transposed K needs an even seq_k (got %lld)",
                (long long)d->seq_k);
  if (!(d->sm_scale > 0.0f) || !__builtin_isfinite(d->sm_scale))
    return fail(FRISK_EINVAL, "frisk_attn_fwd: sm_scale must be positive and finite");
  if (d->seq_q > INT32_MAX / 2 || d->seq_k > INT32_MAX / 2 || d->batch * d->heads > INT32_MAX / 2)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: sizes beyond the 32-bit index range");
  // K and V are read through buffer loads with 32-bit offsets from the
  // head's first row: the last key row (with a transposed K, the last
  // head_dim row of seq_k keys) must end within 2^31 - 1 bytes.
  const int64_t k_reach = kt ? (d->head_dim - 1) * d->k_stride_s * 2 + d->seq_k * 2
                             : (d->seq_k - 1) * d->k_stride_s * 2 + d->head_dim * 2;
  const int64_t kv_reach = std::max(k_reach, (d->seq_k - 1) * d->v_stride_s * 2 + d->head_dim * 2);
  if (kv_reach > INT32_MAX)
    return fail(FRISK_EUNSUP, "frisk_attn_fwd: K/V rows span %lld bytes of one head, beyond the "
                              "2^31 - 1 bytes the kernel addresses",
                (long long)kv_reach);

  frisk::AttnArgs a;
  a.dtype = (frisk::Elt)d->dtype;
  a.out = (frisk::Elt)d->o_dtype;
  a.batch = d->batch; a.heads = d->heads; a.seq_q = d->seq_q; a.seq_k = d->seq_k;
  a.head_dim = d->head_dim;
  a.causal = d->causal != 0;
  a.sm_scale = d->sm_scale;
  a.q = d->q; a.q_sb = d->q_stride_b; a.q_sh = d->q_stride_h; a.q_ss = d->q_stride_s;
  a.k = d->k; a.k_sb = d->k_stride_b; a.k_sh = d->k_stride_h; a.k_ss = d->k_stride_s;
  a.k_dmajor = kt ? 1 : 0;
  a.waves = d->waves;
  a.v = d->v; a.v_sb = d->v_stride_b; a.v_sh = d->v_stride_h; a.v_ss = d->v_stride_s;
  a.o = d->o; a.o_sb = d->o_stride_b; a.o_sh = d->o_stride_h; a.o_ss = d->o_stride_s;
  a.lse = d->lse;
  clear_stale_error();
  hipError_t e = frisk::attn_fwd(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_attn_fwd launch");
  return FRISK_OK;
}

}  // extern "C"

namespace {

// Checks of frisk_reduce / frisk_reduce_workspace_size; 0 or an error code.
int check_reduce(const frisk_reduce_desc* d, const char* fn) {
  if (!d) return fail(FRISK_EINVAL, "%s: null descriptor", fn);
  if (d->rows <= 0 || d->cols <= 0)
    return fail(FRISK_EINVAL, "%s: rows and cols must be positive (got %lld, %lld)", fn,
                (long long)d->rows, (long long)d->cols);
  if (d->dtype != FRISK_F32 && d->dtype != FRISK_F16 && d->dtype != FRISK_BF16)
    return fail(FRISK_EINVAL, "%s: dtype must be f32, f16 or bf16 (got %s)", fn,
                dtype_name(d->dtype));
  if (d->kind != FRISK_REDUCE_SUM && d->kind != FRISK_REDUCE_MAX && d->kind != FRISK_REDUCE_MIN)
    return fail(FRISK_EINVAL, "%s: unknown reduction kind %d", fn, d->kind);
  if (d->axis != 0 && d->axis != 1)
    return fail(FRISK_EINVAL, "%s: axis must be 0 or 1 (got %d)", fn, d->axis);
  if (d->ld_src < d->cols || d->dst_stride < 1)
    return fail(FRISK_EINVAL, "%s: ld_src %lld < cols %lld or dst_stride %lld < 1", fn,
                (long long)d->ld_src, (long long)d->cols, (long long)d->dst_stride);
  if (d->rows >= ((int64_t)1 << 31) || d->cols >= ((int64_t)1 << 31) ||
      (d->axis == 0 && d->rows >= ((int64_t)1 << 23)))
    return fail(FRISK_EUNSUP, "%s: size beyond the kernels' limits (rows, cols < 2^31; "
                              "axis 0 rows < 2^23)", fn);
  const int64_t extent = d->axis == 1 ? d->cols : d->rows;
  if (d->leaf_order_bits < 0 || d->leaf_order_bits > 30)
    return fail(FRISK_EINVAL, "%s: leaf_order_bits %d outside 0..30", fn, d->leaf_order_bits);
  if (d->leaf_order_bits > 0) {
    if (extent != ((int64_t)1 << d->leaf_order_bits))
      return fail(FRISK_EINVAL, "%s: a leaf order of %d bits needs a reduced extent of %lld "
                                "(got %lld)",
                  fn, d->leaf_order_bits, (long long)1 << d->leaf_order_bits, (long long)extent);
    uint32_t seen = 0;
    for (int j = 0; j < d->leaf_order_bits; ++j) {
      const int b = d->leaf_order[j];
      if (b >= d->leaf_order_bits || (seen >> b) & 1u)
        return fail(FRISK_EINVAL, "%s: leaf_order is not a permutation of 0..%d", fn,
                    d->leaf_order_bits - 1);
      seen |= 1u << b;
    }
  }
  if (d->workspace_bytes < 0) return fail(FRISK_EINVAL, "%s: negative workspace_bytes", fn);
  return FRISK_OK;
}

// Bytes of workspace the two-pass axis-0 kernels take (0: single pass).
int64_t reduce_workspace(const frisk_reduce_desc* d) {
  if (d->axis != 0 || d->leaf_order_bits > 0 || d->rows < 256) return 0;
  const frisk::ColsSplit sp = frisk::cols_split(d->rows, d->cols);
  return sp.blocks * d->cols * (int64_t)sizeof(float);
}

}  // namespace

extern "C" {

int64_t frisk_reduce_workspace_size(const frisk_reduce_desc* d) {
  g_last_error.clear();
  const int rc = check_reduce(d, "frisk_reduce_workspace_size");
  return rc ? rc : reduce_workspace(d);
}

int frisk_reduce(const frisk_reduce_desc* d, void* stream) {
  g_last_error.clear();
  const int rc = check_reduce(d, "frisk_reduce");
  if (rc) return rc;
  if (!d->src || !d->dst) return fail(FRISK_EINVAL, "frisk_reduce: null tensor");
  const int es = esize(d->dtype);
  if ((uintptr_t)d->src % es || (uintptr_t)d->dst % es)
    return fail(FRISK_EINVAL, "frisk_reduce: pointers must be element-aligned");
  const int64_t need = reduce_workspace(d);
  void* ws = nullptr;
  if (d->workspace && need > 0) {
    if (d->workspace_bytes < need)
      return fail(FRISK_EINVAL, "frisk_reduce: workspace of %lld bytes, this reduction takes %lld",
                  (long long)d->workspace_bytes, (long long)need);
    if ((uintptr_t)d->workspace % 16)
      return fail(FRISK_EINVAL, "frisk_reduce: workspace must be 16-byte aligned");
    ws = d->workspace;
  }
  frisk::ReduceArgs a;
  a.order_bits = d->leaf_order_bits;
  for (int j = 0; j < 32; ++j) a.order[j] = j < d->leaf_order_bits ? d->leaf_order[j] : 0;
  a.workspace = ws;
  a.dtype = (frisk::Elt)d->dtype;
  a.kind = d->kind;
  a.axis = d->axis;
  a.clear = d->clear != 0;
  a.rows = d->rows; a.cols = d->cols;
  a.src = d->src; a.ld = d->ld_src;
  a.dst = d->dst; a.dst_stride = d->dst_stride;
  clear_stale_error();
  hipError_t e = frisk::tile_reduce(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_reduce launch");
  return FRISK_OK;
}

int frisk_copy(const frisk_copy_desc* d, void* stream) {
  g_last_error.clear();
  if (!d) return fail(FRISK_EINVAL, "frisk_copy: null descriptor");
  if (d->rows <= 0 || d->cols <= 0)
    return fail(FRISK_EINVAL, "frisk_copy: rows and cols must be positive (got %lld, %lld)",
                (long long)d->rows, (long long)d->cols);
  const int ses = esize(d->src_type), des = esize(d->dst_type);
  if (!ses || !des)
    return fail(FRISK_EINVAL, "frisk_copy: unknown element type %d -> %d", d->src_type,
                d->dst_type);
  auto convertible = [](int t) {
    return t == FRISK_F32 || t == FRISK_F16 || t == FRISK_BF16 || t == FRISK_E4M3;
  };
  if (d->src_type != d->dst_type && !(convertible(d->src_type) && convertible(d->dst_type)))
    return fail(FRISK_EINVAL, "frisk_copy: no conversion %s -> %s (f32, f16, bf16, e4m3)",
                dtype_name(d->src_type), dtype_name(d->dst_type));
  if (!d->src || !d->dst) return fail(FRISK_EINVAL, "frisk_copy: null tensor");
  if ((uintptr_t)d->src % ses || (uintptr_t)d->dst % des)
    return fail(FRISK_EINVAL, "frisk_copy: pointers must be element-aligned");
  if (d->ld_src < d->cols || d->ld_dst < d->cols)
    return fail(FRISK_EINVAL, "frisk_copy: row stride smaller than cols");
  if (d->rows >= ((int64_t)1 << 40) || d->cols >= ((int64_t)1 << 40))
    return fail(FRISK_EUNSUP, "frisk_copy: size beyond the kernels' limits");
  frisk::CopyArgs a;
  a.src_t = (frisk::Elt)d->src_type;
  a.dst_t = (frisk::Elt)d->dst_type;
  a.esize = ses;
  a.rows = d->rows; a.cols = d->cols;
  a.src = d->src; a.ld_src = d->ld_src;
  a.dst = d->dst; a.ld_dst = d->ld_dst;
  if (a.rows > 1 && a.ld_src == a.cols && a.ld_dst == a.cols) {  // contiguous: one long row
    a.cols *= a.rows;
    a.ld_src = a.ld_dst = a.cols;
    a.rows = 1;
  }
  clear_stale_error();
  hipError_t e = frisk::tile_copy(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_copy launch");
  return FRISK_OK;
}

int frisk_fill(const frisk_fill_desc* d, void* stream) {
  g_last_error.clear();
  if (!d) return fail(FRISK_EINVAL, "frisk_fill: null descriptor");
  if (d->rows <= 0 || d->cols <= 0)
    return fail(FRISK_EINVAL, "frisk_fill: rows and cols must be positive (got %lld, %lld)",
                (long long)d->rows, (long long)d->cols);
  const int es = esize(d->dtype);
  if (!es) return fail(FRISK_EINVAL, "frisk_fill: unknown element type %d", d->dtype);
  if (!d->dst) return fail(FRISK_EINVAL, "frisk_fill: null tensor");
  if ((uintptr_t)d->dst % es) return fail(FRISK_EINVAL, "frisk_fill: pointer must be element-aligned");
  if (d->ld < d->cols) return fail(FRISK_EINVAL, "frisk_fill: row stride smaller than cols");
  if (d->rows >= ((int64_t)1 << 40) || d->cols >= ((int64_t)1 << 40))
    return fail(FRISK_EUNSUP, "frisk_fill: size beyond the kernels' limits");
  uint64_t bits = 0;
  if (!fill_bits(d->dtype, d->value, &bits))
    return fail(FRISK_EINVAL, "frisk_fill: value %g is not representable as %s", d->value,
                dtype_name(d->dtype));
  frisk::FillArgs a;
  a.esize = es;
  a.bits = bits;
  a.rows = d->rows; a.cols = d->cols;
  a.dst = d->dst; a.ld = d->ld;
  if (a.rows > 1 && a.ld == a.cols) {
    a.cols *= a.rows;
    a.ld = a.cols;
    a.rows = 1;
  }
  clear_stale_error();
  hipError_t e = frisk::tile_fill(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "frisk_fill launch");
  return FRISK_OK;
}

int frisk_probe_mfma_layout(int atom, float* out, int64_t out_floats, void* stream) {
  g_last_error.clear();
  const int need = frisk::mfma_probe_floats(atom);
  if (need == 0) return fail(FRISK_EINVAL, "mfma-probe: unknown atom %d (0, 1 or 2)", atom);
  if (!out) return fail(FRISK_EINVAL, "mfma-probe: null output");
  if (out_floats < need)
    return fail(FRISK_EINVAL, "mfma-probe: atom %d writes %d floats, buffer holds %lld", atom, need,
                (long long)out_floats);
  clear_stale_error();
  hipError_t e = frisk::mfma_layout_probe(atom, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "mfma-probe launch");
  return FRISK_OK;
}

int frisk_probe_lds_transpose(int bits, uint16_t* out, int64_t out_elems, void* stream) {
  g_last_error.clear();
  if (bits != 8 && bits != 16)
    return fail(FRISK_EINVAL, "lds-transpose-probe: bits must be 8 or 16 (got %d)", bits);
  if (!out) return fail(FRISK_EINVAL, "lds-transpose-probe: null output");
  const int64_t need = bits == 16 ? 256 : 512;
  if (out_elems < need)
    return fail(FRISK_EINVAL, "lds-transpose-probe: %d-bit read writes %lld values, buffer holds %lld",
                bits, (long long)need, (long long)out_elems);
  clear_stale_error();
  hipError_t e = frisk::lds_transpose_probe(bits, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "lds-transpose-probe launch");
  return FRISK_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free GEMM.  frisk_gemm_noalloc runs exactly what frisk_gemm
// runs with a workspace of frisk_gemm_workspace_size() bytes, but its
// split-K partials live in `scratch`, a file-scope device array: the call
// allocates nothing.  Each GPU the library runs on holds its own copy of the
// array until the process ends.  In host code the name `scratch` is only a
// host-side stand-in: its device address on the current GPU comes from
// hipGetSymbolAddress, taken once per device and kept in g_scratch, and only
// that address is ever passed to a kernel.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kNoAllocScratchBytes = FRISK_GEMM_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device

// The current device's address of `scratch` (resolved on first use).
int scratch_address(void** out, const char* fn) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FRISK_EHIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FRISK_EUNSUP, "%s: device %d beyond the %d this library tracks", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FRISK_EHIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return FRISK_OK;
}

}  // namespace

extern "C" {

int frisk_gemm_noalloc(const frisk_gemm_desc* d, void* stream) {
  g_last_error.clear();
  frisk::GemmArgs g;
  GemmRoute route;
  const int rc = check_gemm(d, "frisk_gemm_noalloc", true, g, route);
  if (rc) return rc;
  if (d->workspace || d->workspace_bytes)
    return fail(FRISK_EINVAL, "frisk_gemm_noalloc: takes no workspace (its scratch is the "
                              "library's own); pass workspace = NULL, workspace_bytes = 0");
  const int64_t need = gemm_workspace(g, route);
  if (need > kNoAllocScratchBytes)
    return fail(FRISK_EUNSUP, "frisk_gemm_noalloc: this GEMM splits K over %lld bytes of partials, "
                              "beyond the %lld-byte scratch; call frisk_gemm with a workspace",
                (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int src = scratch_address(&ws, "frisk_gemm_noalloc");
    if (src) return src;
  }
  return launch_gemm(g, route, ws, need > 0 ? kNoAllocScratchBytes : 0, stream, "frisk_gemm_noalloc");
}

}  // extern "C"
