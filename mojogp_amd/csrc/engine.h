// Host orchestration of the exact-GP algorithms on one provider: batched CG
// with Lanczos tridiagonals, pivoted-Cholesky preconditioner, one BBMM
// (NLL + gradients) evaluation, the Adam training loop and prediction.
//
// Reference counterparts (caspbian/mojogp):
//   batched_cg_unified        kernels/combined_inv_quad_logdet.mojo:81-449
//   bbmm_with_precond         kernels/combined_inv_quad_logdet.mojo:452-1140
//   build_pivoted_cholesky_precond_unified  kernels/pivoted_cholesky.mojo:2104-2444
//   train_jit_with_provider   kernels/jit/jit_training.mojo:274-1008
//   prediction                kernels/jit/jit_prediction.mojo:681-1350
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "solver.h"

namespace mgp {

struct Precond {
  int rank = 0;        // 0 = no preconditioner
  float noise = 0.f;   // noise at construction (used by apply, log-det, probes)
  DevBuf<float> L;     // [rank][n]
  DevBuf<float> Minv;  // (L^T L + max(noise,1e-6) I)^{-1}, row-major fp32
                       // (diagonal noise D: (I + L^T D^-1 L)^-1)
  float logdet = 0.f;  // log|L L^T + noise I| (or log|L L^T + D|)
  WoodburyWork work;
  // Diagonal noise D from the provider's noise vector (pivoted_cholesky.mojo:
  // 1209-1240, 1346-1520, 2060-2095): per-row 1/d_i and sqrt(d_i).
  bool vec = false;
  DevBuf<float> dinv, dsqrt;
  const float* dinv_ptr() const { return vec ? dinv.ptr : nullptr; }
  const float* dsqrt_ptr() const { return vec ? dsqrt.ptr : nullptr; }
};

// Pivot options of the training loop for a precond_method (greedy: no trace
// stop; rpcholesky / nystrom: error_tol 1e-3; adaptive_tol 0.01; seed 42).
PivotOptions training_pivot_options(int method);
void build_precond(Provider& pv, int rank, const PivotOptions& po, Precond& P);
// Scalar-noise Woodbury pieces (Minv, log|P|) of P = L L^T + P.noise I for a
// factor already in P.L ([k][n]).
void precond_from_factor(Precond& P, int64_t n, int k, hipStream_t st);

struct CGWork {
  DevBuf<float> x, r, z, p, Ap;  // [C][n]
  DevBuf<float> scal;            // rz_old | alpha | beta   (3*C)
  DevBuf<float> hist_a, hist_b;  // [max_tridiag][C]
  DevBuf<double> part_a, part_b, part_c;  // [C][nb]: pAp, r.z, r.r partials
  DevBuf<float> resn;            // [1]
  DevBuf<int> done;
  CGScalars scalars(int ncols);
};

struct CGResult {
  int iterations = 0;
  bool converged = false;
  int tridiag_size = 0;
  double loop_ms = 0.0;  // wall time of the iteration loop (device work synced)
  std::vector<std::vector<float>> diag, offdiag;  // per column
};

// A symmetric positive definite operator on device vectors of length n for
// mBCG: matvec(V, C, out) = A V for C columns ([C][n]); precond (optional)
// writes z = P^{-1} r for C columns plus the fixed-chunk partials of the
// column dots r.z over the nb chunks the CG passes (cg_chunks(n)).
struct CGOperator {
  int64_t n = 0;
  hipStream_t st = nullptr;
  std::function<void(const float*, int, float*)> matvec;
  // precond(r, ncols, z, rz_part, nb): z = P^-1 r and, when rz_part is set,
  // the partials rz_part[c*nb + b] of r . z over nb row chunks.
  std::function<void(const float*, int, float*, double*, int)> precond;
};

// Solves A X = rhs for `ncols` columns (device rhs [C][n]) by the reference's
// preconditioned mBCG (combined_inv_quad_logdet.mojo:81-449); the solution
// stays in w.x (normalised-RHS scale, as given).
CGResult batched_cg(const CGOperator& op, const float* rhs, int ncols, int max_iter,
                    int max_tridiag, float tol, CGWork& w, bool warm_start);
// The single-output system (K + noise I) with the pivoted-Cholesky Woodbury
// preconditioner P (null or rank 0: none).
CGResult batched_cg(Provider& pv, Precond* P, const float* rhs, int ncols, int max_iter,
                    int max_tridiag, float tol, CGWork& w, bool warm_start);

struct BBMMWork {
  CGWork cg;
  DevBuf<float> probes, zr, zn, rhs, sol, lf, rf, ycopy;
  DevBuf<float> probe_norms, rhs_norms;
  DevBuf<double> part;
  bool has_x = false;
};

struct BBMMResult {
  float nll = 0.f, inv_quad = 0.f, logdet = 0.f;
  std::vector<float> grads;  // kernel params then noise
  int cg_iterations = 0;
  bool converged = false;
  double cg_loop_ms = 0.0;
  const float* alpha_dev = nullptr;  // sol column 0 (valid until next call)
};

BBMMResult bbmm_step(Provider& pv, Precond& P, bool use_precond, const float* y_c,
                     int num_probes, int max_cg, int max_tridiag, float tol,
                     int iteration, bool recycle, BBMMWork& w);

struct TrainOptions {
  int max_iterations = 100;
  float learning_rate = 0.01f;
  int num_probes = 10;
  int max_cg_iter = 100;
  float cg_tol = 1e-2f;
  int precond_rank = 10;
  bool verbose = false;
  bool use_cosine_lr = false;
  bool use_preconditioner = true;
  int max_tridiag_iter = 30;
  float precond_rebuild_threshold = 0.5f;
  int precond_method = 0;
  float init_mean = 0.f;
  bool enable_early_stopping = false;
  int early_stop_patience = 10;
  float early_stop_tol = 1e-4f;
  bool learn_noise = true;
  float noise_floor = 1e-6f;
  float noise_regularization = 0.01f;
  int progress_interval = 1;
  uint64_t nan_inject_mask = 0;  // tests: bit i forces the NLL of iteration i to NaN
};

struct ProgressEvent {
  const char* phase;
  int current, total;
  float nll, best_nll;
  int cg_iter;
  double iter_ms;
  float noise, mean;
  int precond_rank, precond_rebuild_count;
  bool converged;
};

struct TrainResult {
  std::vector<float> params;
  float noise = 0.f, mean = 0.f, final_nll = 0.f;
  int iterations = 0;
  bool converged = false;
  std::vector<float> nll_history;
  std::vector<double> iter_times_ms;
  std::vector<int> cg_iterations_history, precond_rank_history, precond_rebuild_steps;
  int precond_build_count = 0;
  double precond_build_total_ms = 0.0;
  std::vector<float> alpha;  // best-NLL alpha (empty if none)
  // Learned noise modes: the final per-point variances [n] and, for the
  // linear mode, the raw function weights [1 + d] (intercept first).
  std::vector<float> learned_noise, noise_fn_params;
};

TrainResult train(Provider& pv, const float* y_host, const std::vector<float>& init_params,
                  float init_noise, const TrainOptions& o,
                  const std::function<void(const ProgressEvent&)>& progress);

// ---------------------------------------------------------------- prediction
struct PredictState {
  DevBuf<float> alpha;  // [n]
  DevBuf<float> root;   // [rank][n]
  int rank = 0;
  bool has_alpha = false;
};

// alpha = (K + noise I)^{-1} (y - mean) by unpreconditioned CG with the
// reference's stop rule (relative residual < tol, pAp guard).
int solve_alpha(Provider& pv, const float* y_host, float mean, int max_iter, float tol,
                PredictState& ps);
// X = A^{-1} B for C device columns [C][n], each column an independent
// unpreconditioned CG from x0 = 0 with the stop rules of solve_alpha
// (solve_single_rhs_deterministic_host_jit, jit_prediction.mojo:681-765, run
// once per column there).  Finished columns freeze while the rest go on.
// Returns the number of operator applications.
int solve_columns(const CGOperator& op, const float* B, int C, int max_iter, float tol,
                  float* X);
// Lanczos inverse root S (S S^T ~ (K + noise I)^{-1}), rank r.
void lanczos_inv_root(Provider& pv, int r, PredictState& ps);
// solve_alpha followed by lanczos_inv_root with the same results; where the
// provider's products are column independent the two run side by side, one
// two-column product per iteration while both are active.  alpha_s is the
// time until alpha is done, root_s the rest.  Returns solve_alpha's count.
int solve_alpha_and_root(Provider& pv, const float* y_host, float mean, int max_iter, float tol,
                         int rank, PredictState& ps, double* alpha_s, double* root_s);

struct PredictTimes {
  double alpha_s = 0, love_root_s = 0, mean_s = 0, variance_s = 0, total_s = 0;
};

// Exact predictive variance options and statistics
// (predict_variance_exact_jit, jit_prediction.mojo:1357-1789).
struct ExactVarianceOptions {
  int max_cg_iter = 300;
  float cg_tol = 1e-3f;
  int precond_rank = 10;   // Nystrom pivoted-Cholesky preconditioner; 0 = none
  int block_cols = 0;      // 0: all columns when materialized, else <= 512
};
struct ExactVarianceStats {
  int block_cols = 0, block_count = 0, cg_total_iterations = 0, cg_max_iterations = 0;
  int precond_rank = 0;
};

// var[j] = k(x*_j, x*_j) - K(X, x*_j)^T (K + noise I)^{-1} K(X, x*_j), clamped
// at 1e-10, for the packed test set pv.test (device output var_dev[m]).
void exact_variance(Provider& pv, int64_t m, const ExactVarianceOptions& o, float* var_dev,
                    ExactVarianceStats& stats);

// mean[m] (+ var[m]: variance_method 1 LOVE, 2 exact) for test inputs.
void predict_from_state(Provider& pv, const PredictState& ps, const float* Xs_host,
                        int64_t m, float mean, int variance_method, float* mean_out,
                        float* var_out, PredictTimes& t,
                        const ExactVarianceOptions* exact = nullptr,
                        ExactVarianceStats* exact_stats = nullptr);

}  // namespace mgp
