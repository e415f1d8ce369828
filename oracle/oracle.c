/*
 * oracle.c -- fp64 CPU restatement of the GEMM and attention path.
 * TEST INFRASTRUCTURE ONLY: linked by tests/ and timed by bench.py's
 * cpu_baseline leg; the product library never calls it.
 *
 * oracle_gemm_f64: C = op(A).op(B) in double, the textbook product that
 *   frisk.gemm denotes (include/Dialect/Frisk/IR/FriskOps.td:252-292; shapes
 *   from ffi/ir.cpp:335-337).  OpenMP over output rows.
 * oracle_attn_f64: one (batch, head) slice of softmax attention in double
 *   with a stable softmax (benchmark/layout/execution/
 *   tail_attention_reference.py:81-114), optional causal mask
 *   (key j visible to query i iff j <= i + sk - sq) and natural-log LSE.
 *   OpenMP over query rows.
 * oracle_attn_rows_f64: the same for a subset of a head's query rows.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

int oracle_gemm_f64(int64_t m, int64_t n, int64_t k, const double* a, int64_t lda, int trans_a,
                    const double* b, int64_t ldb, int trans_b, double* c, int64_t ldc,
                    int threads) {
  if (m <= 0 || n <= 0 || k <= 0) return -1;
  set_threads(threads);
#pragma omp parallel
  {
    double* arow = (double*)malloc(sizeof(double) * (size_t)k);
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      for (int64_t t = 0; t < k; ++t) arow[t] = trans_a ? a[t * lda + i] : a[i * lda + t];
      double* crow = c + i * ldc;
      if (trans_b) {
        /* B stored [n, k]: dot products along contiguous k. */
        for (int64_t j = 0; j < n; ++j) {
          const double* brow = b + j * ldb;
          double s = 0.0;
          for (int64_t t = 0; t < k; ++t) s += arow[t] * brow[t];
          crow[j] = s;
        }
      } else {
        /* B stored [k, n]: rank-1 row updates along contiguous n. */
        for (int64_t j = 0; j < n; ++j) crow[j] = 0.0;
        for (int64_t t = 0; t < k; ++t) {
          const double av = arow[t];
          const double* brow = b + t * ldb;
          for (int64_t j = 0; j < n; ++j) crow[j] += av * brow[j];
        }
      }
    }
    free(arow);
  }
  return 0;
}

/* Row i of one head (query qi, keys/values [0, end)) into oi / *lse_i; s
 * is scratch of sk doubles. */
static void attn_row(const double* qi, const double* k, const double* v, int64_t end, int64_t d,
                     double scale, double* s, double* oi, double* lse_i) {
  for (int64_t x = 0; x < d; ++x) oi[x] = 0.0;
  if (end <= 0) {
    if (lse_i) *lse_i = -INFINITY;
    return;
  }
  double mx = -INFINITY;
  for (int64_t j = 0; j < end; ++j) {
    const double* kj = k + j * d;
    double acc = 0.0;
    for (int64_t x = 0; x < d; ++x) acc += qi[x] * kj[x];
    s[j] = acc * scale;
    if (s[j] > mx) mx = s[j];
  }
  double den = 0.0;
  for (int64_t j = 0; j < end; ++j) {
    const double e = exp(s[j] - mx);
    den += e;
    const double* vj = v + j * d;
    for (int64_t x = 0; x < d; ++x) oi[x] += e * vj[x];
  }
  for (int64_t x = 0; x < d; ++x) oi[x] /= den;
  if (lse_i) *lse_i = log(den) + mx;
}

int oracle_attn_f64(int64_t sq, int64_t sk, int64_t d, const double* q, const double* k,
                    const double* v, int causal, double scale, double* o, double* lse,
                    int threads) {
  if (sq <= 0 || sk <= 0 || d <= 0) return -1;
  set_threads(threads);
  const int64_t diag = sk - sq;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)sk);
#pragma omp for schedule(dynamic, 16)
    for (int64_t i = 0; i < sq; ++i) {
      int64_t end = sk;
      if (causal) end = i + diag + 1 < sk ? i + diag + 1 : sk;
      attn_row(q + i * d, k, v, end, d, scale, s, o + i * d, lse ? lse + i : NULL);
    }
    free(s);
  }
  return 0;
}

/* The same arithmetic for a subset of the sq query rows of one head: row
 * rows[r] (its causal mask from that index) into o[r] / lse[r]; q holds all
 * sq rows.  A sampled check of a full-size head at a fraction of the cost. */
int oracle_attn_rows_f64(int64_t sq, int64_t sk, int64_t d, const int64_t* rows, int64_t nrows,
                         const double* q, const double* k, const double* v, int causal,
                         double scale, double* o, double* lse, int threads) {
  if (sq <= 0 || sk <= 0 || d <= 0 || nrows < 0) return -1;
  for (int64_t r = 0; r < nrows; ++r)
    if (rows[r] < 0 || rows[r] >= sq) return -1;
  set_threads(threads);
  const int64_t diag = sk - sq;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)sk);
#pragma omp for schedule(dynamic, 4)
    for (int64_t r = 0; r < nrows; ++r) {
      const int64_t i = rows[r];
      int64_t end = sk;
      if (causal) end = i + diag + 1 < sk ? i + diag + 1 : sk;
      attn_row(q + i * d, k, v, end, d, scale, s, o + r * d, lse ? lse + r : NULL);
    }
    free(s);
  }
  return 0;
}
