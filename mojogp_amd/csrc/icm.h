// Intrinsic Coregionalization Model (ICM) multi-output GP on gfx950:
// K_full = os (B (x) K_X) + D over task-blocked vectors, B = W W^T +
// diag(softplus(raw_v)), trained with BBMM under the Kronecker
// preconditioner, and predicted per eigen-task of os B.
//
// Reference (caspbian/mojogp):
//   training loop            kernels/jit/jit_multi_output.mojo:130-817
//   task covariance          kernels/task_covariance.mojo:168-307
//   Kronecker operator       kernels/jit/fused_kronecker_provider.mojo:97-330
//   preconditioner           kernels/kronecker_preconditioner.mojo:140-730
//   bindings                 kernels/jit/jit_engine_multi_output_bindings.mojo:57-712
//
// The operator, BBMM evaluation and preconditioner apply are the LMC ones
// (lmc.h) with one latent and mixing matrix os B; only the task covariance
// parameterisation, the Kronecker preconditioner and the update rules are
// ICM-specific.
#pragma once

#include <functional>
#include <vector>

#include "lmc.h"

namespace mgp {

// W [T][R] of the reference's TaskCovariance: 0.1 + 0.4 u with u from a
// 31-bit LCG over seed ^ (i * 2654435761).
std::vector<float> icm_init_w(int T, int R, int seed = 42);
// B = W W^T + diag(softplus(raw_v)) accumulated in fp64, stored fp32.
std::vector<float> icm_task_b(const std::vector<float>& W, const std::vector<float>& raw_v,
                              int T, int R);

struct ICMTrainOptions {
  int max_iterations = 100;
  float learning_rate = 0.05f;
  int task_rank = -1;  // -1: full rank T
  int num_probes = 10;
  int max_cg_iter = 200;
  int max_tridiag_iter = 30;
  float cg_tol = 1e-2f;
  int precond_rank = 15;
  int precond_method = 0;
  float precond_rebuild_threshold = 0.5f;
  bool use_cosine_lr = false;
  int early_stop_patience = 15;
  float early_stop_tol = 1e-4f;
  int progress_interval = 1;
};

struct ICMTrainResult {
  std::vector<float> params;  // base kernel (constrained)
  float outputscale = 0.f;
  std::vector<float> noise, mean;  // [T]
  std::vector<float> B;            // [T][T], without the outputscale
  std::vector<float> alpha;        // [T][n]
  std::vector<float> nll_history;
  std::vector<int> cg_iterations_history;
  std::vector<double> iter_times_ms;
  float final_nll = 0.f;
  int iterations = 0, task_rank = 0, precond_rebuild_count = 0;
  bool converged = false;
};

// base: the base-kernel provider (its own params are overwritten each
// iteration; noise 0).  fixed: [T][n] fixed per-sample-task noise replacing
// the learned per-task noise (noise mode 1: no preconditioner, noise frozen),
// or empty.
ICMTrainResult icm_train(Provider& base, int T, const float* y_blocked_host,
                         const std::vector<float>& init_params, const std::vector<char>& trainable,
                         const std::vector<float>& init_noise, float init_outputscale,
                         const std::vector<float>& init_mean, const std::vector<float>& fixed,
                         const ICMTrainOptions& o,
                         const std::function<void(const ProgressEvent&)>& progress);

// Mixed continuous x categorical ICM (train_multi_output_mixed_jit,
// kernels/jit/jit_multi_output_mixed.mojo:477-1148): base is a kernel-tree
// provider with categorical leaves (cat_kinds: one per leaf in tree order;
// init_cat_raw: their raw parameters).  The evaluation is the single-output
// BBMM of the full operator os (B (x) K) + D with the single-output probe
// streams, preconditioned by a pivoted Cholesky of that operator
// (pivoted_cholesky_kron) with the smallest task noise; the categorical raw
// parameters train by Adam moments of their own on
// (-0.5 a^T dK a + (0.5/P) sum_j u_j^T dK zn_j) times the transform's chain
// derivative, dK = os (B (x) dK_X), neither divided by nT nor clipped; the
// kernel, outputscale, noise and W gradients are unclipped (G_B at +-10, the
// mean gradient at +-100); no NaN handling; rebuild when a kernel
// parameter, a constrained categorical parameter, the outputscale, a task
// noise or an entry of B moved by more than the threshold (after iteration
// 0); best-NLL snapshot; early stop on early_stop_patience evaluations not
// below the best by early_stop_tol.  Every parameter is trained.
struct ICMMixedResult : ICMTrainResult {
  std::vector<float> cat_raw;  // best raw categorical parameters
};
ICMMixedResult icm_train_mixed(Provider& base, int T, const float* y_blocked_host,
                               const std::vector<float>& init_params,
                               const std::vector<float>& init_noise, float init_outputscale,
                               const std::vector<float>& init_mean,
                               const std::vector<int>& cat_kinds,
                               const std::vector<float>& init_cat_raw,
                               const ICMTrainOptions& o,
                               const std::function<void(const ProgressEvent&)>& progress);

// Prediction from the rotated posterior state (predict_multi_output_python,
// jit_engine_multi_output_bindings.mojo:329-549): for each eigen-task s,
// mean[i][t] += Q[t][s] scale_s (K(X*, X) alpha_rot[s])[i] and, when
// scale_s > 1e-8, var[i][t] += Q[t][s]^2 scale_s v_s[i] with v_s the
// single-output LOVE (variance_method 1) or exact (2) variance at noise
// noise / scale_s.  alpha_rot: host [T][n]; outputs [m][T].
void icm_predict(Provider& pv, int T, const float* alpha_rot, const float* Q,
                 const float* scales, const float* Xs_host, int64_t m, float noise,
                 int variance_method, int max_cg_iter, float cg_tol, int precond_rank,
                 int lanczos_rank, float* mean_out, float* var_out);

}  // namespace mgp
