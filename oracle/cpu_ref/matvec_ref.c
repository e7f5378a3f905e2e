/*
 * CPU restatement of the reference's fused forward matvec — TEST/BASELINE
 * INFRASTRUCTURE ONLY (used by tests/ and the cpu_baseline leg of bench.py).
 *
 * Follows caspbian/mojogp mojogp/codegen_engine/emit/gpu_kernel.py:151-260:
 * one output row i at a time, for every column j the kernel value is formed
 * from per-dimension differences (diff_d / l_d), guarded as in
 * codegen_engine/passes/numerical_stability.py:29-41,62-85 (sqrt(max(x,1e-20)),
 * Matern r carrying +1e-20, expressions.py:197-240; exp(max(x,-20)) for the
 * Matern-5/2 exponent, no clamp on the RBF exponent, as the reference's
 * generated code has them), and
 * accumulated in fp32 as acc[c] += k * v[c*n + j]; the row is written as
 * out[c*n + i] = acc[c] + noise * v[c*n + i].  Rows are spread over OpenMP
 * threads; the arithmetic per row is the reference's sequential order.
 *
 * Pinned by tests/test_cpu_ref.py against oracle/kernels.py (float64), which
 * is itself pinned against scikit-learn and closed forms.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#define MAX_DIM 64
#define MAX_COLS 64

static inline float kval(int kind, float r2, float os) {
  if (kind == 0) return os * expf(-0.5f * r2);  /* RBF: not clamped */
  float x = r2 + 1e-20f;
  if (x < 1e-20f) x = 1e-20f;
  const float r = sqrtf(x);
  const float s5r = 2.2360679774997896f * r;
  float a = -s5r;
  if (a < -20.0f) a = -20.0f;
  return os * (1.0f + s5r + (5.0f / 3.0f) * r * r) * expf(a);
}

/* out[c*nrows + (i-row0)] for rows [row0, row0+nrows).  Returns 0 or -1. */
int ref_forward_matvec_rows(int kind, int ard, int d, int64_t n, const float* X,
                            const float* params, float noise, const float* V,
                            int ncols, int64_t row0, int64_t nrows, float* out) {
  if (d < 1 || d > MAX_DIM || ncols < 1 || ncols > MAX_COLS) return -1;
  float inv_ls[MAX_DIM];
  for (int k = 0; k < d; ++k) inv_ls[k] = 1.0f / (ard ? params[k] : params[0]);
  const float os = params[ard ? d : 1];
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t ii = 0; ii < nrows; ++ii) {
    const int64_t i = row0 + ii;
    float xi[MAX_DIM];
    float acc[MAX_COLS];
    for (int k = 0; k < d; ++k) xi[k] = X[i * d + k];
    for (int c = 0; c < ncols; ++c) acc[c] = 0.0f;
    for (int64_t j = 0; j < n; ++j) {
      const float* xj = X + j * d;
      float r2 = 0.0f;
      for (int k = 0; k < d; ++k) {
        const float df = (xi[k] - xj[k]) * inv_ls[k];
        r2 += df * df;
      }
      const float kv = kval(kind, r2, os);
      for (int c = 0; c < ncols; ++c) acc[c] += kv * V[(int64_t)c * n + j];
    }
    for (int c = 0; c < ncols; ++c)
      out[(int64_t)c * nrows + ii] = acc[c] + noise * V[(int64_t)c * n + i];
  }
  return 0;
}

int ref_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
