// Linear Model of Coregionalization (LMC) on gfx950: the structured operator
// K_full = sum_s A_s (x) K_s + D over task-blocked vectors, its
// Sum-of-Kronecker Woodbury preconditioner, one BBMM evaluation with the
// kernel / A_s / per-task-noise gradients, the Adam training loop and mean
// prediction.
//
// Reference (caspbian/mojogp):
//   operator + gradients     kernels/jit/jit_lmc.mojo:131-540, kernels/lmc_provider.mojo:45-268
//   preconditioner           kernels/lmc_preconditioner.mojo:143-719
//   A_s / noise gradients    kernels/jit/jit_lmc.mojo:582-696
//   training loop            kernels/jit/jit_lmc.mojo:699-1529
//   prediction (mean, var)   kernels/jit/jit_engine_lmc_bindings.mojo:1102-1396
//
// Layouts: a task-blocked vector is [T][n] (index t*n + i); C of them are
// [C][T][n].  A_s and C_s = chol(A_s) are row-major T x T.
#pragma once

#include <memory>
#include <vector>

#include "engine.h"

namespace mgp {

struct LMCModel {
  int R = 0, T = 0;
  int64_t n = 0;
  std::vector<Provider*> prov;  // R latent providers (noise 0), not owned
  std::vector<float> A;         // [R][T][T]
  std::vector<float> noise;     // [T]
  std::vector<float> fixed;     // [T][n] fixed observation noise, or empty
  hipStream_t st = nullptr;     // every latent provider runs on this stream
  DevBuf<float> A_dev, noise_dev, fixed_dev, tmp;

  int64_t size() const { return n * T; }
  bool has_fixed() const { return !fixed.empty(); }
  // noise_t + mean_i fixed[t][i]: the diagonal the preconditioner assumes
  // (jit_lmc.mojo:882-888).
  std::vector<float> precond_noise() const;
  void upload();  // A, noise (and fixed noise) to the device after changing them
  // out = (sum_s A_s (x) K_s + D) V for C task-blocked columns.
  void forward(const float* V, int C, float* out);
  // out = K_s V for `cols` plain columns of length n (noise 0).
  void latent_forward(int s, const float* V, int cols, float* out);
};

// Runs every latent provider of an LMC model on one stream for the guard's
// lifetime (restores the providers' own streams afterwards).
struct LMCStreamGuard {
  LMCModel& m;
  std::vector<hipStream_t> saved;
  explicit LMCStreamGuard(LMCModel& model);
  ~LMCStreamGuard();
};

// P = sum_s (A_s (x) L_s L_s^T) + D with A_s = C_s C_s^T and L_s the rank-r_s
// pivoted-Cholesky factor of K_s; applied by Woodbury with the inner matrix
// M = I + U^T D^-1 U (U = [C_s (x) L_s]_s) inverted once and applied in fp64.
struct LMCPrecond {
  virtual ~LMCPrecond() = default;
  int R = 0, T = 0, K = 0;  // K = sum_s r_s T
  int64_t n = 0;
  std::vector<int> rank, off;          // per latent: r_s, offset of (s, 0, 0) in K
  std::vector<std::unique_ptr<DevBuf<float>>> L;  // per latent [r_s][n]
  std::vector<float> Cs;               // [R][T][T]
  std::vector<float> noise;            // [T]
  DevBuf<float> Cs_dev, dinv, dsqrt;
  DevBuf<double> Minv;  // [K][K], fp64
  float logdet = 0.f;
  // work
  DevBuf<float> w, Y, zk, Z, out_l, res;
  DevBuf<double> yk;
  WoodburyWork lt_work;

  bool active() const { return K > 0; }
  void build(LMCModel& m, int precond_rank, const PivotOptions& po);
  // z = P^{-1} r for C task-blocked columns; rz_part gets the column-dot
  // partials of r.z (fixed chunking of n*T).
  // z = P^-1 r; with rz_part, the partials rz_part[c*nb + b] of r . z.
  virtual void apply(const float* r, int C, float* z, double* rz_part, int nb, hipStream_t st);
  // N(0, P) probes: D^{1/2} eps + U w (counter-hash Gaussians, seeds
  // seed + 1000000 and seed).
  virtual void sample(float* out, int C, uint64_t seed, hipStream_t st);
};

// ICM (Kronecker) preconditioner P = os (B' (x) L L^T) + D (x) I_n with
// B' = B + 1e-6 D (the jitter D^{-1/2} B D^{-1/2} + 1e-6 I of the reference)
// and L the rank-r pivoted-Cholesky factor of the base kernel at noise 0
// (kernels/kronecker_preconditioner.mojo:140-400).  It is applied through the
// LMC Woodbury path with U = D^{1/2} (x) L and the inner matrix replaced by
// (Q~ (x) V) diag(C^-1) (Q~ (x) V)^T, where L^T L = V Sigma V^T,
// D^{-1/2} B D^{-1/2} + 1e-6 I = Q~ Lambda~ Q~^T (Jacobi, fp64) and
// C^-1[j][i] = 1 / (1/(os lambda_j) + sigma_i); log|P| = n sum_t log noise_t +
// sum_{j,i} log(1 + os lambda_j sigma_i).  Probes are
// D^{1/2} z_noise + (C_B (x) L) z_rank with C_B = sqrt(os) D^{1/2} Q~ Lambda~^{1/2},
// z_noise = gaussian(C*n*T, seed + 12345) ([C][T][n]) and
// z_rank = gaussian(C*r*T, seed) at index (t*C + c)*r + k (:629-730).
struct KronPrecond : LMCPrecond {
  std::vector<float> Cb;             // [T][T] probe factor C_B
  std::vector<float> sigma, lambda;  // eigenvalues of L^T L and of B~ (ascending)
  DevBuf<float> Cb_dev, zraw;
  // m: one-latent model over the base kernel (its A and noise are not read).
  void build_kron(LMCModel& m, int precond_rank, const PivotOptions& po, float os,
                  const std::vector<float>& B, const std::vector<float>& noise_t);
  void sample(float* out, int C, uint64_t seed, hipStream_t st) override;
};

struct LMCWork {
  CGWork cg;
  DevBuf<float> probes, probe_norms, rhs_norms, rhs, sol, lf, rf, rfm, krf, zr, zn, facs;
  DevBuf<double> part;
  bool has_x = false;
};

struct LMCEval {
  float nll = 0.f, inv_quad = 0.f, logdet = 0.f;
  std::vector<float> kernel_grads;  // sum_s P_s (per-latent engine layout)
  std::vector<float> G_A;           // [R][T][T]
  std::vector<float> noise_grads;   // [T]
  std::vector<float> alpha;         // [T][n] (host copy of the solution)
  int cg_iterations = 0;
  bool converged = false;
  double cg_loop_ms = 0.0;  // wall time of the mBCG iteration loop
};

// One BBMM evaluation of the LMC marginal likelihood at the model's current
// parameters (y_c: device, task-blocked, mean removed).
LMCEval lmc_bbmm(LMCModel& m, LMCPrecond* P, const float* y_c, int num_probes, int max_cg,
                 int max_tridiag, float tol, int iteration, bool recycle, LMCWork& w);

struct LMCTrainOptions {
  int max_iterations = 100;
  float learning_rate = 0.05f;
  int num_probes = 10;
  int max_cg_iter = 200;
  int max_tridiag_iter = 30;
  float cg_tol = 1.0f;
  int precond_rank = 15;
  int precond_method = 0;
  float precond_rebuild_threshold = 0.5f;
  float early_stop_tol = 1e-4f;
  int early_stop_patience = 15;
};

struct LMCTrainResult {
  std::vector<std::vector<float>> params;  // per latent (constrained)
  std::vector<float> A, L, var_diag;       // [R][T][T], [R][T][T], [R][T]
  std::vector<float> noise, mean;          // [T]
  std::vector<float> alpha;                // [T][n]
  std::vector<float> nll_history;
  std::vector<double> iter_times_ms;
  float final_nll = 0.f;
  int iterations = 0;
  bool converged = false;
  int precond_rebuild_count = 0;
};

LMCTrainResult lmc_train(LMCModel& m, const float* y_blocked_host,
                         const std::vector<std::vector<float>>& init_params,
                         const std::vector<std::vector<char>>& trainable,
                         const std::vector<float>& init_noise,
                         const std::vector<float>& init_mean, const LMCTrainOptions& o);

// Mixed continuous x categorical LMC (train_lmc_mixed_jit,
// kernels/jit/jit_lmc_mixed.mojo:684-1557): the parametrisation and Adam of
// lmc_train plus, for every latent whose kernel tree has categorical leaves,
// their raw correlation parameters (cat_kinds[s]: one kind per categorical
// leaf in tree order; init_cat_raw[s]: their raw parameters, concatenated)
// with Adam moments of their own and the shared step count.  The loop's own
// rules: a NaN NLL ends the run; the best-NLL evaluation is the only snapshot;
// after iteration 20 every evaluation not below the best NLL counts toward
// the patience (the improving one included); the preconditioner is rebuilt
// when a kernel parameter, a constrained categorical parameter, an entry of
// A_s or a task noise moved by more than the threshold since the last build.
// Every parameter is trained (no masks).
struct LMCMixedResult : LMCTrainResult {
  std::vector<std::vector<float>> cat_raw;  // best raw categorical parameters per latent
};

LMCMixedResult lmc_train_mixed(LMCModel& m, const float* y_blocked_host,
                               const std::vector<std::vector<float>>& init_params,
                               const std::vector<std::vector<int>>& cat_kinds,
                               const std::vector<std::vector<float>>& init_cat_raw,
                               const std::vector<float>& init_noise,
                               const std::vector<float>& init_mean, const LMCTrainOptions& o);

// out[c][t][i] = sum_s sum_t' A_s[t][t'] (K_s(X*, X) alpha_{c,t'})[i] for C
// task-blocked columns alpha [C][T][n] (test inputs already packed into every
// latent provider's `test`); out is a device array [C][T][mtest].
void lmc_cross_mix(LMCModel& m, const float* alpha_dev, int C, int64_t mtest, float* out_dev);

// mean[i][t] = sum_s sum_t' A_s[t][t'] (K_s(X*, X) alpha_t')[i] + mean_t
// (predict_lmc_python, jit_engine_lmc_bindings.mojo:1102-1396); out_host [m][T].
void lmc_predict_mean(LMCModel& m, const float* alpha_dev, int64_t mtest,
                      const std::vector<float>& mean, float* out_host);

// Exact joint posterior variance [m][T] (host): for every test point i and
// output task t, beta = K_full^{-1} r_{i,t} with r_{i,t} the joint cross
// covariance column (r[t'][j] = sum_s A_s[t'][t] k_s(x_j, x*_i)), then
// var = sum_s A_s[t][t] os_s - r . beta + noise_t, clamped at 1e-10
// (_predict_lmc_full_exact_variance_backend, multi_output_gp.py:4360-4515,
// which runs one solve per (i, t)); here `block` test points (0: 512) share
// each block solve.  Returns the number of operator applications.
int lmc_exact_variance(LMCModel& m, int64_t mtest, int max_cg, float tol, int block,
                       float* var_host);

// Pathwise correction for S residuals [S][T][n] (device): beta_c = K_full^{-1}
// r_c by per-column CG (max_cg, relative tolerance tol) and correction
// [S][m][T] (host) = sum_s A_s (x) K_s(X*, X) beta_c
// (sample_lmc_pathwise_python, jit_engine_lmc_bindings.mojo:599-797, which
// runs one sample per call).  Returns the number of operator applications.
int lmc_pathwise_correction(LMCModel& m, const float* resid_dev, int S, int64_t mtest,
                            int max_cg, float tol, float* corr_host);

}  // namespace mgp
