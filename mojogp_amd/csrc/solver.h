// Device building blocks of the solvers: batched CG vector kernels, probe RNG,
// pivoted-Cholesky steps, Woodbury apply, gradient traces, Lanczos helpers.
// All reductions are deterministic (fixed partition, fixed order, fp64).
#pragma once

#include "provider.h"

namespace mgp {

// Number of row chunks per column used by the two-stage reductions.
int reduction_chunks(int64_t n);
// Row chunks of the batched CG's dot partials (~256 rows each, <= 2048): the
// CG vector kernels and the Woodbury apply run one workgroup per chunk.
int cg_chunks(int64_t n);
// Rows per chunk of those kernels: ceil(n / nb) rounded up to a multiple of 4,
// so 16-byte vector accesses never straddle a chunk (trailing chunks may be
// empty and then contribute zero partials).
__host__ __device__ inline int64_t cg_chunk_rows(int64_t n, int64_t nb) {
  return (((n + nb - 1) / nb) + 3) & ~(int64_t)3;
}

// part[c*nb + b] = sum_{i in chunk b} a[c*n+i] * b[c*n+i]   (fp64)
void coldot_partial(const float* a, const float* b, int64_t n, int ncols, int nb,
                    double* part, hipStream_t st);
// out[c] = sum_b part[c*nb + b] (fixed order); optionally sqrt.
void coldot_finalize(const double* part, int nb, int ncols, double* out, hipStream_t st);

// ---------------------------------------------------------------- batched CG
// Per-column scalars live in one device block (CGScalars).
struct CGScalars {
  float* rz_old;   // [C] r.z of the current iteration
  float* rz_next;  // [C] r.z of the next one (the caller swaps the two)
  float* alpha;    // [C]
  float* beta;     // [C]
  float* hist_alpha;  // [max_tridiag][C]
  float* hist_beta;   // [max_tridiag][C]
  int* done;       // [1] device stop flag (single-rhs solves)
};

// alpha = safe(rz_old / pAp) from the pAp partials (cg_solver.mojo:181-209),
// stored in s.alpha; x += alpha p, r -= alpha Ap with the reference skip rules
// (cg_solver.mojo:138-179); writes rr partials (r.r) for every column.
void cg_update(float* x, float* r, const float* p, const float* Ap, int64_t n,
               int ncols, int nb, const double* pap_part, CGScalars s, double* rr_part,
               hipStream_t st);
// beta = safe(rz_new / rz_old) from the rz partials, s.rz_next = rz_new
// (cg_solver.mojo:211-255), alpha / beta into the history slot `iter` when
// iter < max_tridiag, then p = z + beta p (cg_solver.mojo:108-136).  The
// caller swaps s.rz_old and s.rz_next before the next iteration.
void cg_pupdate(float* p, const float* z, int64_t n, int ncols, int nb, const double* rz_part,
                CGScalars s, int iter, int max_tridiag, hipStream_t st);
// mean_c sqrt(rr_c) into *out (cg_solver.mojo:446-543)
void cg_mean_resnorm(const double* rr_part, int nb, int ncols, float* out,
                     hipStream_t st);

// ---------------------------------------------------------------- vectors
void fill(float* x, int64_t count, float v, hipStream_t st);
void copy(float* dst, const float* src, int64_t count, hipStream_t st);
// y = a - b
void sub(float* y, const float* a, const float* b, int64_t count, hipStream_t st);
// y[i] = x[i] - s
void sub_scalar(float* y, const float* x, float s, int64_t count, hipStream_t st);
// columns c: x[c*n+i] *= scale[c] (or /= when divide)
void scale_columns(float* x, const float* scale, int64_t n, int ncols, bool divide,
                   hipStream_t st);
// norms[c] = ||x_c||; x_c /= norms[c]   (pivoted_cholesky.mojo:1818-1907)
void normalize_columns(float* x, int64_t n, int ncols, float* norms, double* part,
                       hipStream_t st);

// Counter-hash Gaussian draws: out[i] for i < len with the reference's integer
// hash and Box-Muller transform (pivoted_cholesky.mojo:51-86).
void gaussian(float* out, int64_t len, uint64_t seed, hipStream_t st);

// ---------------------------------------------------------------- precond
struct PivotState;  // device-side pivot bookkeeping

// Pivot selection and stopping rules of the reference's unified builder
// (pivoted_cholesky.mojo:2104-2444):
//   method 0 greedy     pivot = argmax residual diagonal (lowest index on ties);
//                       stop when sum|diag|/diag_value < error_tol
//   method 1 rpcholesky pivot sampled proportionally to the positive residual
//                       diagonal with a host xorshift64 stream; same stop rule
//   method 2 nystrom    rpcholesky sampling; stop when sum|diag| <
//                       adaptive_tol * n * noise (after the first pivot)
// Every method stops when the largest residual falls below 1e-10.
struct PivotOptions {
  int method = 0;
  float error_tol = 0.f;
  float adaptive_tol = 0.01f;
  uint64_t seed = 42;
};

// Pivoted Cholesky of K into L [rank][n] (column-major by pivot); returns the
// realized rank.  Greedy with error_tol = 0 runs without host round trips;
// the other cases read the pivot statistics (and, when sampling, the residual
// diagonal) back to the host once per pivot, as the reference does.
int pivoted_cholesky(Provider& pv, int rank, const PivotOptions& o, float* L,
                     hipStream_t st);
// The same builder over the full Kronecker operator os (B (x) K) + D of a
// base provider (build_pivoted_cholesky_precond_unified over
// KroneckerDirectProvider, kronecker_direct_provider.mojo:182-209, 338-386,
// 511-553): N = n T entries, task-blocked; column p is the forward product of
// the unit vector e_p minus noise_min at the pivot (os_B[:, t_p] (x) K[:, j_p]
// plus task_noise[t_p] - noise_min at p); the residual diagonal starts at
// os_B[s][s] (the provider reports a base diagonal of 1) and the stop rule
// uses max_s os_B[s][s] and noise_min.  osB_dev / task_noise_dev: device
// [T][T] and [T]; L: [rank][N].
int pivoted_cholesky_kron(Provider& base, int T, const float* osB_dev,
                          const std::vector<float>& osB, const float* task_noise_dev,
                          float noise_min, int rank, const PivotOptions& o, float* L,
                          hipStream_t st);

// M = L^T L (k x k, fp64) for the first k columns.
// M = L^T diag(wt) L when wt (device [n]) is given.
void syrk_ltl(const float* L, int64_t n, int k, double* M_dev, hipStream_t st,
              const float* wt = nullptr);
// M[a][b] = La_a . Lb_b (ka x kb, fp64 on the device) for factors [k][n].
void cross_ltl(const float* La, int ka, const float* Lb, int kb, int64_t n, double* M_dev,
               hipStream_t st);


// out = (v - L u)/noise with u = Minv (L^T v) for ncols columns (Woodbury,
// pivoted_cholesky.mojo:1646-1771).  Optionally writes dot partials of
// dotv . out (for r.z) over nb row chunks, dot_part[c*nb + b].  out and dotv
// may alias v.
struct WoodburyWork {
  DevBuf<float> wpart;   // [nbw][C][k] row-chunk partials of L^T v
  DevBuf<float> wsum;    // [C][k]
  DevBuf<float> u;       // [C][k]
};
// With dinv (device [n], per-row 1/d_i of a diagonal D): u = Minv L^T D^-1 v and
// out = D^-1 (v - L u), Minv = (I + L^T D^-1 L)^-1.
void woodbury_apply(const float* L, int64_t n, int k, const float* Minv, float noise,
                    const float* v, int ncols, float* out, WoodburyWork& w,
                    const float* dotv, int nb, double* dot_part, hipStream_t st,
                    const float* dinv = nullptr);
// out[c*n + i] = sum_kk L[kk*n+i] * zr[c*k + kk] + s * zn[c*n + i]  (zn may be null)
// ds (device [n], optional): per-row sqrt(d_i) in place of s.
void low_rank_sample(const float* L, int64_t n, int k, const float* zr,
                     const float* zn, float s, int ncols, float* out, hipStream_t st,
                     const float* ds = nullptr);

// out[c][kk] = L_kk . V_c for ncols columns (L [k][n], V [ncols][n]).
void lt_matmul(const float* L, int64_t n, int k, const float* V, int ncols, float* out,
               WoodburyWork& w, hipStream_t st);
// out[c][i] = sum_kk L[kk][i] Z[c][kk] for ncols columns.
void l_matmul(const float* L, int64_t n, int k, const float* Z, int ncols, float* out,
              hipStream_t st);
// The same with column c = b gT + j of Z read in place from a blocked vector:
// Z[c][kk] = z[b gK + goff + j k + kk] (the LMC preconditioner's per-latent
// slice of each probe's coefficients, without a gathered copy).
void l_matmul_gather(const float* L, int64_t n, int k, const float* z, int gT, int gK, int goff,
                     int ncols, float* out, hipStream_t st);

// ---------------------------------------------------------------- gradients
// g[p] = sum_{a,b} dK_p[a,b] * sum_c Lf[c*n+a] Rf[c*n+b]  for every kernel
// parameter p (engine layout), fp64 result on the host.
void gradient_traces(const Provider& pv, const float* Lf, const float* Rf, int ncols,
                     double* g_host, hipStream_t st);

// ---------------------------------------------------------------- Lanczos
// out[j] = Q_j . w for j < nvec (Q [nvec][n]), fp64 via partials.
void multi_dot(const float* Q, int nvec, const float* w, int64_t n, double* part,
               int nb, double* out, hipStream_t st);
// w -= sum_j coef[j] Q_j
void multi_axpy(const float* Q, int nvec, const double* coef, float* w, int64_t n,
                hipStream_t st);
// S[c*n + i] = sum_k Q[k*n + i] * T[k*r + c]  (n x r times r x r)
void gemm_nr_rr(const float* Q, const float* T, int64_t n, int r, float* S,
                hipStream_t st);
// var[j] = max(diag_j - sum_k V[k*m + j]^2, 1e-10) with diag_j = diag_vec[j]
// (device, optional) or diag (jit_prediction.mojo:211-233)
void love_variance(const float* V, int64_t m, int r, float diag, float* var,
                   hipStream_t st, const float* diag_vec = nullptr);

}  // namespace mgp
