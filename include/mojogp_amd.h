/*
 * mojogp_amd — C ABI of the MI355X (gfx950) exact-GP engine.
 *
 * Drop-in boundary for the reference's two native modules (caspbian/mojogp):
 *   - the generated kernel module (init_provider / materialize /
 *     destroy_provider and the fn-pointer table it returns),
 *     mojogp/codegen_engine/emit/fn_ptr_module.py:998-1211, 1120-1166;
 *   - the engine module (train / predict / prediction cache /
 *     benchmark_provider_ops), mojogp/kernels/jit/jit_engine_bindings.mojo:1750-1775.
 *
 * Conventions
 *   - Every function returns 0 on success or a non-zero status; the message is
 *     available from mgp_last_error() (per thread).
 *   - Arrays are host pointers unless the name ends in _device.  Matrices of
 *     right-hand sides are column-major [ncols][n] (element c*n + i), as in the
 *     reference (fn_ptr_module.py:391-491).  Inputs X are row-major [n][d].
 *   - Every call is synchronous on return.  Each provider owns one HIP stream;
 *     a handle must not be used from two threads at once.
 *   - Kernel kinds: 0 = RBF, 1 = Matern-5/2, 2 = Matern-1/2, 3 = Matern-3/2.  Parameter layout (engine layout,
 *     mojogp/kernel.py:494-509): isotropic [lengthscale, outputscale];
 *     ARD [ls_0 .. ls_{d-1}, outputscale].
 */
#ifndef MOJOGP_AMD_H
#define MOJOGP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MGP_API __attribute__((visibility("default")))

/* Status codes. */
#define MGP_OK 0
#define MGP_ERR_INVALID 1
#define MGP_ERR_HIP 2
#define MGP_ERR_NUMERIC 3
#define MGP_ERR_INTERNAL 4

/* Copies the calling thread's last error message into buf (NUL terminated,
 * truncated to len-1 bytes); returns the full message length.
 * Replaces the Python exceptions raised by the reference's `raises` functions
 * (jit_engine_bindings.mojo:163-164, 479-480). */
MGP_API int mgp_last_error(char* buf, size_t len);
MGP_API const char* mgp_version(void);
MGP_API int mgp_device_count(int* out);

/* ---- Provider (kernel module) ------------------------------------------ */

/* Creates a device-resident provider for training inputs X[n][d].
 * Replaces init_provider(X, params, noise) (fn_ptr_module.py:998-1168). */
MGP_API int mgp_init_provider(int kind, int ard, int d, int64_t n,
                              const float* X, const float* params, int nparams,
                              float noise, void** out_handle);
/* Provider for a composite kernel tree: sums, products and scales of RBF,
 * Matern-1/2, 3/2, 5/2, RQ, periodic, linear, polynomial and categorical
 * leaves, each leaf on a subset of the input dimensions.
 * spec[spec_len] = [d, nparams, nleaves, nnodes,
 *   per leaf (tree order): code (0 RBF, 1 M52, 2 M12, 3 M32, 4 RQ,
 *   5 periodic, 6 categorical, 7 linear, 8 polynomial), ard, ndim, p0,
 *   [degree: polynomial leaves only], dims[ndim],
 *   per node (children first, root last): code (0 leaf: a = leaf index;
 *   1 sum / 2 product: a, b = child nodes; 3 scale: a = child node,
 *   b = index of the scale factor in params), a, b].
 * Leaf parameters start at p0: [ls | ls_0..ls_{q-1}], (alpha | period), os;
 * linear [var | var_0..], os; polynomial [var | var_0..], degree, offset, os.
 * Categorical leaves: ard = number of levels L, ndim = 1 (the column holding
 * the level code), p0 = offset of their L x L table after the parameters
 * (mgp_set_categorical_tables / mgp_set_categorical_params).
 * At most 8 leaves, 16 nodes, 48 parameters, d <= 32, 64 leaf dimensions.
 * Replaces init_provider of a generated composite module (the kernel
 * expression tree of codegen_engine/expressions.py:474-648 compiled per
 * tree, parameter layout mojogp/kernel.py:528-568).  The provider reports
 * kind -1; products are evaluated per pair from raw inputs (VALU). */
MGP_API int mgp_init_provider_tree(const int* spec, int spec_len, int d, int64_t n,
                                   const float* X, const float* params, int nparams,
                                   float noise, void** out_handle);
/* Learned per-point noise for mgp_train (the provider noise modes 2-4 of
 * init_provider, fn_ptr_module.py:297-327, trained as
 * jit_training.mojo:41-228, 352-960): mode 2 one variance per point, 3 one
 * per group (group_ids[n] in [0, num_groups)), 4 softplus(w0 + w . x) + floor
 * on the raw inputs; 0 clears.  Needs a noise vector set first
 * (mgp_set_noise_vector: the initial variances).  Training starts every raw
 * value at inv_softplus(init_noise - noise_floor) (mode 4: the intercept;
 * weights 0), learns them with their own Adam moments and leaves the final
 * vector on the provider. */
MGP_API int mgp_set_learned_noise(void* handle, int mode, const int* group_ids,
                                  int num_groups);
/* Replaces destroy_provider(info) (fn_ptr_module.py:1183-1195). */
MGP_API int mgp_destroy_provider(void* handle);

/* Select the materialized route: hold the dense K on the device as a scaled
 * two-term fp16 split (4 bytes per entry, like fp32), fill its symmetric half
 * and refill it on every parameter update (the full matrix is filled on the
 * first product wider than 16 columns); forward products then run on the
 * hand-written fp16 matrix-core kernels (three part products, fp32/fp64
 * accumulation) plus the noise term.  Replaces materialize(info) /
 * _do_materialize (fn_ptr_module.py:363-384, 1168-1181). */
MGP_API int mgp_materialize(void* handle);
/* Replace the impl_update_params / impl_update_noise / impl_get_noise /
 * impl_get_diagonal_value fn pointers (fn_ptr_module.py:651-703). */
MGP_API int mgp_update_params(void* handle, const float* params, int nparams);
MGP_API int mgp_update_noise(void* handle, float noise);

/* Fixed per-point observation-noise variances noise_vec[n] (finite, > 0), or
 * NULL to return to the scalar noise: the operator becomes K + diag(noise_vec)
 * (the scalar noise is then ignored) and preconditioners are built for
 * L L^T + diag(noise_vec).  Replaces init_provider(X, params, noise,
 * observation_noise, noise_mode=1) (fn_ptr_module.py:998-1168, noise modes
 * :297-327). */
MGP_API int mgp_set_noise_vector(void* handle, const float* noise_vec);
MGP_API int mgp_get_noise(void* handle, float* out);
MGP_API int mgp_get_diagonal_value(void* handle, float* out);

/* The reference's non-raising provider fn pointers with their exact
 * signatures (UpdateNoiseFn fn(Int, Float32), GetFloatFn fn(Int) -> Float32,
 * GetIntFn fn(Int) -> Int, GetPtrFn fn(Int) -> Float32*;
 * erased_provider.mojo:43-50; implementations impl_update_noise ..
 * impl_get_noise_vector_ptr, impl_get_diagonal_value, fn_ptr_module.py:
 * 666-696): their addresses are the provider dict's update_noise, get_noise,
 * get_noise_mode, get_noise_vector_ptr and get_diagonal_value entries
 * (fn_ptr_module.py:1120-1166), callable through ctypes as the reference's
 * Python does (update_noise: CFUNCTYPE(None, c_ssize_t, c_float),
 * _multi_output_backend.py:166-183).  handle = the provider_ptr value.
 * They return no status: a failure is recorded for mgp_last_error and they
 * return NaN / -1 / NULL (update_noise leaves the noise unchanged).
 * get_noise_mode: 0 scalar, 1 fixed vector, 2-4 learned; get_noise_vector_ptr:
 * the device array of per-point noise, NULL in mode 0. */
MGP_API void mgp_fn_update_noise(intptr_t handle, float noise);
MGP_API float mgp_fn_get_noise(intptr_t handle);
MGP_API intptr_t mgp_fn_get_noise_mode(intptr_t handle);
MGP_API float* mgp_fn_get_noise_vector_ptr(intptr_t handle);
MGP_API float mgp_fn_get_diagonal_value(intptr_t handle);
/* Shape of a provider (the n / dim / num_gradient_params / is_ard keys of the
 * reference's provider dict, fn_ptr_module.py:1120-1166). */
MGP_API int mgp_provider_info(void* handle, int64_t* n, int* d, int* nparams,
                              int* kind, int* ard);

/* out = (K + noise I) V.  Replaces the forward_matvec fn pointer
 * (impl_forward_matvec, fn_ptr_module.py:391-491). */
MGP_API int mgp_forward_matvec(void* handle, const float* V, int ncols,
                               float* out);
/* Same with device-resident V/out (no PCIe copies). */
MGP_API int mgp_forward_matvec_device(void* handle, const float* V_device,
                                      int ncols, float* out_device);
/* Same as mgp_forward_matvec_device, allocating nothing: no hipMalloc, no
 * hipFree, no allocating library call.  No counterpart in the reference; it
 * is for callers that cannot allocate (tight serving loops, harnesses that
 * forbid hipMalloc).  The work runs eagerly on the provider's own stream and
 * ends in a stream synchronize, so it is not recorded into a caller's HIP
 * graph.  Its work buffers (packed right-hand sides, column maxima, split
 * partial sums) live in one fixed 64 MiB device array per GPU, held until the
 * process ends; split partials that do not fit reduce the split count.  A
 * call whose packed right-hand sides alone exceed the array (about
 * 4 n min(ncols, 64) bytes: n up to ~1M at 16 columns, ~260k at 64) fails
 * with MGP_ERR_INVALID.  Serves the single-kernel matrix-free route only (not
 * kernel trees or materialized providers), always on the one-sided tile
 * kernel: the symmetric kernel's transposed partial sums (n^2/16 bytes) do
 * not fit a fixed array, so above the automatic symmetric threshold
 * (n >= 24065) this call is slower than mgp_forward_matvec_device (config 3:
 * ~22.8 ms against ~16.9 ms) and agrees with it to the product rounding, not
 * bit for bit.  Every call on a GPU shares that GPU's array; a per-device
 * lock, held until the call's stream has drained, makes overlapping calls
 * (other threads, other providers) run one after another. */
MGP_API int mgp_forward_matvec_device_noalloc(void* handle, const float* V_device,
                                              int ncols, float* out_device);
/* (K + noise I) V from per-dimension differences (no Gram form, no MFMA):
 * an independent device cross-check of mgp_forward_matvec.  No reference
 * counterpart; kept for parity tests. */
MGP_API int mgp_direct_matvec(void* handle, const float* V, int ncols,
                              float* out);
/* out[c*m + i] = sum_j k(Xs_i, X_j) V[c*n + j].  Replaces the cross_matvec fn
 * pointer (impl_cross_matvec, fn_ptr_module.py:576-626). */
MGP_API int mgp_cross_matvec(void* handle, const float* Xs, int64_t m,
                             const float* V, int ncols, float* out);
/* diag k(x_i, x_i).  Replace extract_diagonal / extract_diagonal_test
 * (fn_ptr_module.py:628-649). */
MGP_API int mgp_extract_diagonal(void* handle, float* out);
MGP_API int mgp_extract_diagonal_test(void* handle, const float* Xs, int64_t m,
                                      float* out);

/* out[p][c][i] = sum_j dk(x_i, x_j)/dtheta_p V[c][j] for the P engine
 * parameters [l | l_0..l_{d-1}, os] (out is [P][ncols][n]).  Replaces the
 * fused_gradient_matvec / gradient_matvec fn pointers (fn_ptr_module.py:
 * 493-541; kernels gpu_kernel.py:382-484, 878-975). */
MGP_API int mgp_gradient_matvec(void* handle, const float* V, int ncols, float* out);

/* out[p] = sum_{a,b} dK_p[a,b] sum_c Lf[c*n+a] Rf[c*n+b] for every kernel
 * parameter p (engine layout), Lf and Rf host [ncols][n], out host [P].  The
 * trace routine of mgp_bbmm_eval's gradient step (the matrix-core trace where
 * its route applies, MGP_GRAD_MFMA as there, else the pair loop) on
 * caller-given weight columns, in place of the reference's per-parameter
 * fused_gradient_matvec + kernel_dot_*_vs_strided pair
 * (combined_inv_quad_logdet.mojo:715-800).  Internal to the reference (no
 * exported counterpart); exposed for at-size parity tests. */
MGP_API int mgp_gradient_trace(void* handle, const float* Lf, const float* Rf,
                               int ncols, double* out);

/* Isolated timing of provider ops.  Replaces benchmark_provider_ops(info, rhs,
 * num_cols, op_code, repeats, warmup) (jit_engine_bindings.mojo:439-572);
 * op 0 forward matvec, 1 fused gradient products, 2 gradient products + the
 * per-(parameter, column) dots <rhs_c, out_pc>, 3 the dots alone.
 * times_ms[repeats] gets per-call host wall times, tile_ms_avg the mean
 * HIP-event duration of the fused tile kernel (op 0), and out_or_null (if
 * non-null) the last output ([ncols][n] for op 0, [P][ncols][n] otherwise). */
MGP_API int mgp_benchmark_provider_ops(void* handle, const float* rhs,
                                       int ncols, int op, int repeats,
                                       int warmup, double* times_ms,
                                       double* tile_ms_avg, float* out_or_null);

/* ---- Engine: training --------------------------------------------------- */

/* Mirrors the 23 positional arguments of the reference's engine.train()
 * after the provider/y/params/noise (jit_engine_bindings.mojo:123-250; order
 * fixed by mojogp/gp.py:1665-1691). */
typedef struct mgp_train_opts {
  int max_iterations;
  float learning_rate;
  int num_probes;
  int max_cg_iter;
  float cg_tol;
  int precond_rank;
  int verbose;
  int use_cosine_lr;
  int use_preconditioner;
  int max_tridiag_iter;
  float precond_rebuild_threshold;
  int precond_method; /* 0 greedy, 1 rpcholesky, 2 nystrom */
  float init_mean;
  int enable_early_stopping;
  int early_stop_patience;
  float early_stop_tol;
  int learn_noise;
  float noise_floor;
  float noise_regularization;
  int progress_interval;
  /* Forced-failure switch for tests of the NaN recovery (no counterpart in
   * the reference's arguments): bit i set treats the evaluated NLL of
   * iteration i (i < 64) as NaN, which runs the recovery path of
   * jit_training.mojo:605-685.  0 in normal use. */
  unsigned long long nan_inject_mask;
} mgp_train_opts_t;

/* Progress event (the reference's event dict, jit_progress.mojo:22-65). */
typedef struct mgp_progress {
  const char* phase; /* "start" "iteration" "nan" "early_stop" "complete" */
  int current;
  int total;
  double nll;
  double best_nll;
  int cg_iter;       /* -1: absent */
  double iter_ms;    /* < 0: absent */
  double noise;      /* < 0: absent */
  double mean;
  int precond_rank;
  int precond_rebuild_count;
  int converged;
} mgp_progress_t;
typedef void (*mgp_progress_cb)(const mgp_progress_t* event, void* user);

/* Result of mgp_train (the reference's result dict,
 * jit_engine_bindings.mojo:336-432).  Array members are caller-allocated:
 * params[nparams], the histories [max_iterations], cached_alpha[n]; any may be
 * NULL.  The *_len members receive the number of entries written. */
typedef struct mgp_train_result {
  float* params;
  float* nll_history;
  double* iter_times_ms;
  int* cg_iterations_history;
  int* precond_rank_history;
  int* precond_rebuild_steps;
  float* cached_alpha;
  float final_nll;
  float noise;
  float mean;
  int iterations;
  int converged;
  int history_len;
  int cg_history_len;
  int rank_history_len;
  int rebuild_steps_len;
  int precond_build_count;
  double precond_build_total_ms;
  int has_alpha;
  /* Learned noise modes (mgp_set_learned_noise): the final per-point
   * variances [n] and, for mode 4, the raw linear-function weights [1 + d]
   * (intercept first).  Caller-allocated, may be NULL. */
  float* learned_noise;
  float* noise_fn_params;
  int has_learned_noise;
  int noise_fn_len;
} mgp_train_result_t;

/* Adam training of the kernel hyperparameters, noise and constant mean with
 * preconditioned mBCG / SLQ.  Replaces engine.train() (train_python,
 * jit_engine_bindings.mojo:123-432 -> train_jit_with_provider,
 * jit_training.mojo:274-1008).  cb may be NULL. */
MGP_API int mgp_train(void* handle, const float* y, const float* init_params,
                      int nparams, float init_noise,
                      const mgp_train_opts_t* opts, mgp_progress_cb cb,
                      void* user, mgp_train_result_t* out);

/* Mixed continuous x categorical training of a kernel-tree provider whose
 * spec has categorical leaves (code 6): split Adam as in train_mixed
 * (jit_engine_bindings.mojo:1241-1460, jit_mixed.mojo:428-909): continuous
 * parameters, noise and mean from BBMM, categorical raw parameters
 * (cat_kinds[ncat] per categorical leaf in tree order: 0 GD, 1 CR, 2 EHH,
 * 3 HH, 4 FE; ncat_params raw values in that order) from
 * -0.5 alpha^T dK alpha + (0.5/S) sum_s (K^-1 z_s)^T dK zn_s.  Writes the
 * best raw categorical parameters to cat_raw_out[ncat_params] and leaves the
 * provider at the best state. */
MGP_API int mgp_train_mixed(void* handle, const float* y, const float* init_params,
                            int nparams, float init_noise, const int* cat_kinds, int ncat,
                            const float* init_cat_raw, int ncat_params,
                            const mgp_train_opts_t* opts, mgp_progress_cb cb, void* user,
                            mgp_train_result_t* out, float* cat_raw_out);
/* Categorical correlation tables of a tree provider from raw parameters
 * (same layout as mgp_train_mixed; replaces the mixed prediction's
 * categorical_prediction_params + update_correlation_matrices,
 * mojogp/kernel.py:132-174). */
MGP_API int mgp_set_categorical_params(void* handle, const int* cat_kinds, int ncat,
                                       const float* raw, int nraw);
/* Raw correlation tables (tree.table_size entries, leaf p0 offsets). */
MGP_API int mgp_set_categorical_tables(void* handle, const float* tables, int size);

/* One BBMM evaluation at the provider's current hyperparameters: NLL per
 * sample, y^T K^-1 y, log|K| (SLQ) and gradients[nparams + 1] (kernel
 * params, then noise) of the reference's bbmm_with_precond
 * (combined_inv_quad_logdet.mojo:452-1140) with probe seed
 * iteration*104729+42 and a greedy preconditioner of precond_rank (0: none);
 * cg_loop_ms receives the wall time of the mBCG iteration loop.
 * Internal to the reference (no exported counterpart); exposed for
 * teacher-forced parity tests. */
MGP_API int mgp_bbmm_eval(void* handle, const float* y, float mean,
                          int num_probes, int max_cg_iter, int max_tridiag_iter,
                          float cg_tol, int iteration, int precond_rank,
                          float* nll, float* inv_quad, float* logdet,
                          float* grads, int* cg_iterations,
                          float* precond_logdet, double* cg_loop_ms);
/* Counter-hash Gaussian draws of kernel_gpu_gaussian
 * (pivoted_cholesky.mojo:51-86), computed on the device. */
MGP_API int mgp_gaussian(int64_t len, uint64_t seed, float* out);
/* Pivoted Cholesky factor L[rank][n] (column-major, realised rank in
 * rank_out) and log|L L^T + noise I| of build_pivoted_cholesky_precond_unified
 * (pivoted_cholesky.mojo:2104-2444).  method: 0 greedy, 1 rpcholesky,
 * 2 nystrom; error_tol / adaptive_tol / seed as the reference's arguments
 * (training uses error_tol 0 for greedy, 1e-3 otherwise; adaptive_tol 0.01,
 * seed 42). */
MGP_API int mgp_pivoted_cholesky(void* handle, int rank, int method, float error_tol,
                                 float adaptive_tol, uint64_t seed, float* L_out,
                                 int* rank_out, float* logdet);

/* ---- Engine: prediction ------------------------------------------------- */

typedef struct mgp_predict_opts {
  float mean;          /* learned constant mean */
  int variance_method; /* 0 mean only, 1 LOVE, 2 exact */
  int max_cg_iter;
  float cg_tol;
  int precond_rank;
  int lanczos_rank;
  int exact_block_cols;
} mgp_predict_opts_t;

typedef struct mgp_predict_info {
  double alpha_time_s;
  double mean_time_s;
  double variance_time_s;
  double total_time_s;
  double love_root_time_s;
  int alpha_cache_used;
  int love_root_cache_used;
  int alpha_cg_iterations;
  /* exact variance (variance_method 2): block width, CG blocks, CG
   * iterations (total / max per block), realised preconditioner rank */
  int exact_block_cols;
  int exact_cg_block_count;
  int exact_cg_total_iterations;
  int exact_cg_max_iterations;
  int exact_precond_rank;
} mgp_predict_info_t;

/* Predictive mean (and variance) at Xs[m][d].  alpha_in / root_in are the
 * optional cached alpha [n] and LOVE root [lanczos_rank][n]; alpha_out /
 * root_out (optional) receive what was computed.  The provider must already
 * hold the trained params/noise.  Replaces engine.predict()
 * (predict_python, jit_engine_bindings.mojo:944-1235). */
MGP_API int mgp_predict(void* handle, const float* y, const float* Xs,
                        int64_t m, const mgp_predict_opts_t* opts,
                        const float* alpha_in, const float* root_in,
                        float* mean_out, float* var_out, float* alpha_out,
                        float* root_out, mgp_predict_info_t* info);

/* Device-resident alpha (+ LOVE root) reused across predictions.  Replace
 * prepare_prediction_cache / predict_with_cache / destroy_prediction_cache
 * (jit_engine_bindings.mojo:636-942, PredictionCacheJIT :72-121). */
MGP_API int mgp_prepare_prediction_cache(void* handle, const float* y,
                                         const mgp_predict_opts_t* opts,
                                         const float* alpha_in,
                                         void** cache_out,
                                         mgp_predict_info_t* info);
MGP_API int mgp_predict_with_cache(void* handle, void* cache, const float* Xs,
                                   int64_t m, int variance_method,
                                   float* mean_out, float* var_out,
                                   mgp_predict_info_t* info);
MGP_API int mgp_destroy_prediction_cache(void* cache);

/* ---- Multi-output LMC ---------------------------------------------------- */
/* An LMC model is R latent providers (mgp_init_provider with noise 0, all
 * over the same training inputs X[n][d]) with mixing matrices A[R][T][T]
 * (row-major), per-task noise[T] and optional fixed observation noise
 * fixed_noise[T][n] (NULL: none).  Task-blocked vectors are [T][n]
 * (index t*n + i); C of them are [C][T][n]. */

/* out = (sum_s A_s (x) K_s + diag(noise_t) + diag(fixed)) V for C task-blocked
 * columns.  Replaces JITLMCGradientAdapter.forward_matvec
 * (kernels/jit/jit_lmc.mojo:275-330) with kernel_lmc_accumulate_batched /
 * kernel_lmc_add_noise_batched / kernel_lmc_add_fixed_noise_batched
 * (kernels/lmc_provider.mojo:113-170). */
MGP_API int mgp_lmc_forward_matvec(void* const* providers, int R, int T,
                                   const float* A, const float* noise,
                                   const float* fixed_noise, const float* V,
                                   int C, float* out);

/* The positional options of the reference's train_lmc()
 * (jit_engine_lmc_bindings.mojo:365-390). */
typedef struct mgp_lmc_train_opts {
  int max_iterations;
  float learning_rate;
  int num_probes;
  int max_cg_iter;
  float cg_tol;
  int precond_rank;    /* 0: no preconditioner */
  int precond_method;  /* 0 greedy, 1 rpcholesky, 2 nystrom */
  float precond_rebuild_threshold;
  int max_tridiag_iter;
  float early_stop_tol;
  int early_stop_patience;
} mgp_lmc_train_opts_t;

/* Result of mgp_lmc_train (the reference's result dict,
 * jit_engine_lmc_bindings.mojo:533-585).  Caller-allocated arrays (any may be
 * NULL): params[sum_s P_s] (per latent, concatenated), A[R][T][T],
 * L[R][T][T], var_diag[R][T], noise[T], mean[T], alpha[T][n] (task-blocked),
 * nll_history / iter_times_ms [max_iterations]. */
typedef struct mgp_lmc_train_result {
  float* params;
  float* A;
  float* L;
  float* var_diag;
  float* noise;
  float* mean;
  float* alpha;
  float* nll_history;
  double* iter_times_ms;
  int history_len;
  float final_nll;
  int iterations;
  int converged;
  int precond_rebuild_count;
} mgp_lmc_train_result_t;

/* Joint Adam training of the latent kernel parameters, A_s = L_s L_s^T +
 * diag(var_diag_s), per-task noise and per-task mean by BBMM on the T*n joint
 * system with the sum-of-Kronecker Woodbury preconditioner.  y_blocked [T][n];
 * init_params / trainable: per latent, concatenated.  The providers end with
 * the best parameters.  Replaces train_lmc() (train_lmc_python,
 * jit_engine_lmc_bindings.mojo:365-597 -> train_lmc_jit,
 * kernels/jit/jit_lmc.mojo:699-1529; preconditioner
 * kernels/lmc_preconditioner.mojo:143-589). */
MGP_API int mgp_lmc_train(void* const* providers, int R, int T,
                          const float* y_blocked, const float* init_params,
                          const int* trainable, const float* init_noise,
                          const float* fixed_noise, const float* init_mean,
                          const mgp_lmc_train_opts_t* opts,
                          mgp_lmc_train_result_t* out);

/* Mixed continuous x categorical LMC: mgp_lmc_train plus the raw correlation
 * parameters of the categorical leaves of each kernel-tree latent, trained by
 * their own Adam moments on (-0.5 alpha^T dK alpha + (0.5/P) sum_j
 * u_j^T dK zn_j) / (nT) with dK = A_s (x) dK_s (every parameter trained, no
 * masks).  cat_counts[R]: categorical leaves per latent; cat_kinds: their
 * kinds (0 GD, 1 CR, 2 EHH, 3 HH, 4 FE) in tree order, concatenated over the
 * latents; init_cat_raw[ncat_params]: their raw parameters in the same order.
 * Outputs (either may be NULL): cat_raw_out[ncat_params] the best raw values,
 * cat_params_out[ncat_params] their constrained values (the reference's
 * cat_params_per_latent).  The loop stops at the first NaN NLL, keeps the
 * best-NLL state only, counts after iteration 20 every evaluation not below
 * the best toward the patience, and rebuilds the preconditioner when a kernel
 * parameter, a constrained categorical parameter, an entry of A_s or a task
 * noise moved by more than the threshold.  Replaces train_lmc_mixed()
 * (train_lmc_mixed_python, jit_engine_lmc_bindings.mojo:54-360 ->
 * train_lmc_mixed_jit, kernels/jit/jit_lmc_mixed.mojo:684-1557). */
MGP_API int mgp_lmc_train_mixed(void* const* providers, int R, int T,
                                const float* y_blocked, const float* init_params,
                                const float* init_noise, const float* fixed_noise,
                                const float* init_mean, const int* cat_counts,
                                const int* cat_kinds, const float* init_cat_raw,
                                int ncat_params, const mgp_lmc_train_opts_t* opts,
                                mgp_lmc_train_result_t* out, float* cat_raw_out,
                                float* cat_params_out);

/* One BBMM evaluation of the LMC marginal likelihood at fixed A / noise /
 * kernel parameters (y_c: task-blocked, mean removed): NLL per joint entry,
 * y^T K^-1 y, log|K|, kernel gradients [sum_s P_s], dNLL/dA [R][T][T],
 * dNLL/dnoise [T], alpha [T][n].  The body of one iteration of train_lmc_jit
 * (jit_lmc.mojo:1132-1212 with _compute_A_and_noise_gradients_jit
 * :582-696); internal there, exposed for teacher-forced parity tests.
 * cg_loop_ms (optional) gets the wall time of the mBCG iteration loop. */
MGP_API int mgp_lmc_bbmm_eval(void* const* providers, int R, int T,
                              const float* A, const float* noise,
                              const float* fixed_noise, const float* y_c,
                              int num_probes, int max_cg_iter,
                              int max_tridiag_iter, float cg_tol, int iteration,
                              int precond_rank, int precond_method, float* nll,
                              float* inv_quad, float* logdet,
                              float* kernel_grads, float* grad_A,
                              float* noise_grads, float* alpha_out,
                              int* cg_iterations, float* precond_logdet,
                              double* cg_loop_ms);

/* Device-resident timing of the structured product (inputs uploaded once):
 * times_ms[repeats] gets the HIP-event duration of each product on the
 * models' stream after `warmup` untimed ones; out (optional) the last result.
 * The LMC counterpart of benchmark_provider_ops op 0
 * (jit_engine_bindings.mojo:439-572); no reference export of its own. */
MGP_API int mgp_lmc_benchmark_forward(void* const* providers, int R, int T,
                                      const float* A, const float* noise,
                                      const float* V, int C, int repeats,
                                      int warmup, double* times_ms, float* out);

/* Predictive mean [m][T] (and variance [m][T], latent variances [R][m]) at
 * Xs[m][d] from the task-blocked alpha [T][n].  variance_method 0 mean only,
 * 1 LOVE (rank lanczos_rank), 2 exact; each latent's variance is computed
 * with its provider noise set to the average task noise, mixed by
 * sum_t' A_s[t][t']^2 and the task noise added.  Replaces predict_lmc()
 * (predict_lmc_python, jit_engine_lmc_bindings.mojo:1102-1394). */
MGP_API int mgp_lmc_predict(void* const* providers, int R, int T,
                            const float* A, const float* alpha,
                            const float* mean, const float* noise,
                            const float* Xs, int64_t m, int variance_method,
                            int max_cg_iter, float cg_tol, int precond_rank,
                            int lanczos_rank, float* mean_out, float* var_out,
                            float* latent_var_out);

/* Exact joint posterior variance [m][T] of the LMC model (observation noise
 * included): per test point and output task, one CG solve of K_full against
 * the joint cross-covariance column (unpreconditioned, per-column stop
 * ||r|| / ||b|| < cg_tol), var = sum_s A_s[t][t] os_s - r . beta + noise_t,
 * clamped at 1e-10.  block_points test points (0: 512) share one block solve.
 * Replaces _predict_lmc_full_exact_variance_backend
 * (mojogp/multi_output_gp.py:4360-4515), which issues one
 * sample_lmc_pathwise() solve per (point, task). */
MGP_API int mgp_lmc_exact_variance(void* const* providers, int R, int T,
                                   const float* A, const float* noise,
                                   const float* fixed_noise, const float* Xs,
                                   int64_t m, int max_cg_iter, float cg_tol,
                                   int block_points, float* var_out,
                                   int* cg_iterations);

/* Pathwise correction for S residuals [S][T][n]: beta = K_full^-1 r by
 * unpreconditioned CG per column (stop: ||r|| / ||b|| < cg_tol, pAp guard),
 * correction [S][m][T] = sum_s A_s (x) K_s(Xs, X) beta.  Replaces
 * sample_lmc_pathwise() (sample_lmc_pathwise_python,
 * jit_engine_lmc_bindings.mojo:599-797), which handles one sample per call;
 * here all S samples share each structured product.  cg_iterations receives
 * the number of joint-operator applications. */
MGP_API int mgp_lmc_pathwise_correction(void* const* providers, int R, int T,
                                        const float* A, const float* noise,
                                        const float* fixed_noise,
                                        const float* residual, int S,
                                        const float* Xs, int64_t m,
                                        int max_cg_iter, float cg_tol,
                                        float* correction_out,
                                        int* cg_iterations);

/* ------------------------------------------------------------------ ICM
 * Intrinsic Coregionalization Model: K_full = os (B (x) K_X) + D with
 * B = W W^T + diag(softplus(raw_v)) over one base-kernel provider (created
 * with noise 0).  Task-blocked vectors are [T][n]. */

/* Training options of mgp_icm_train (train_multi_output arguments 8-21,
 * jit_engine_multi_output_bindings.mojo:57-84). */
typedef struct mgp_icm_train_opts {
  int max_iterations;
  float learning_rate;
  int task_rank;       /* rank R of W; -1: T */
  int num_probes;
  int max_cg_iter;
  float cg_tol;
  int precond_rank;    /* 0: no preconditioner */
  int precond_method;  /* 0 greedy, 1 rpcholesky, 2 nystrom */
  float precond_rebuild_threshold;
  int max_tridiag_iter;
  int early_stop_patience;
  float early_stop_tol; /* 0 disables early stopping */
  int use_cosine_lr;
  int progress_interval;
} mgp_icm_train_opts_t;

/* Result of mgp_icm_train (the reference's result dict,
 * jit_engine_multi_output_bindings.mojo:241-320).  Caller-allocated arrays
 * (any may be NULL): params[P], noise[T], mean[T], B[T][T] (without the
 * outputscale), alpha[T][n], nll_history / cg_iterations_history /
 * iter_times_ms [max_iterations]. */
typedef struct mgp_icm_train_result {
  float* params;
  float* noise;
  float* mean;
  float* B;
  float* alpha;
  float* nll_history;
  int* cg_iterations_history;
  double* iter_times_ms;
  int history_len;
  float outputscale;
  float final_nll;
  int iterations;
  int converged;
  int task_rank;
  int precond_rebuild_count;
} mgp_icm_train_result_t;

/* Adam training of the base-kernel parameters, the ICM outputscale, per-task
 * noise, W, raw_v and per-task means by BBMM on the T*n joint system with the
 * Kronecker preconditioner; y_blocked [T][n]; fixed_noise [T][n] (or NULL)
 * replaces the per-task noise and disables the preconditioner.  The provider
 * ends with the best parameters.  Replaces train_multi_output()
 * (train_multi_output_python, jit_engine_multi_output_bindings.mojo:57-326 ->
 * train_multi_output_jit, kernels/jit/jit_multi_output.mojo:130-817). */
MGP_API int mgp_icm_train(void* provider, int T, const float* y_blocked,
                          const float* init_params, const int* trainable,
                          const float* init_noise, float init_outputscale,
                          const float* init_mean, const float* fixed_noise,
                          const mgp_icm_train_opts_t* opts, mgp_progress_cb cb,
                          void* user, mgp_icm_train_result_t* out);

/* Mixed continuous x categorical ICM on a kernel-tree provider with
 * categorical leaves: mgp_icm_train's parameters (every one trained, no
 * fixed noise) plus the raw correlation parameters of the leaves, trained by
 * Adam moments of their own on (-0.5 a^T dK a + (0.5/P) sum_j u_j^T dK zn_j)
 * times the transform's chain derivative with dK = os (B (x) dK_X), neither
 * divided by nT nor clipped.  The evaluation is the single-output BBMM of the
 * full operator os (B (x) K) + D preconditioned by a pivoted Cholesky of that
 * operator (columns from unit-vector products, a base diagonal of 1, the
 * smallest task noise).  cat_kinds[ncat]: the leaves' kinds (0 GD, 1 CR,
 * 2 EHH, 3 HH, 4 FE) in tree order; init_cat_raw[ncat_params]: their raw
 * parameters; cat_raw_out[ncat_params] (may be NULL): the best raw values.
 * The provider ends with the best parameters and tables.  Replaces
 * train_multi_output_mixed() (train_multi_output_mixed_python,
 * jit_engine_multi_output_bindings.mojo:953-1200 ->
 * train_multi_output_mixed_jit, kernels/jit/jit_multi_output_mixed.mojo:477-1148). */
MGP_API int mgp_icm_train_mixed(void* provider, int T, const float* y_blocked,
                                const float* init_params, const float* init_noise,
                                float init_outputscale, const float* init_mean,
                                const int* cat_kinds, int ncat, const float* init_cat_raw,
                                int ncat_params, const mgp_icm_train_opts_t* opts,
                                mgp_progress_cb cb, void* user, mgp_icm_train_result_t* out,
                                float* cat_raw_out);

/* Mean [m][T] (and variance [m][T] for variance_method 1 LOVE / 2 exact)
 * from the rotated posterior state: alpha_rot [T][n] (eigen-task s's
 * weights in row s), Q [T][T] row-major and scales[T] the eigenvectors and
 * eigenvalues of os B; variance of eigen-task s at noise / scales[s].  The
 * provider's parameters must already be set.  Replaces predict_multi_output()
 * (predict_multi_output_python, jit_engine_multi_output_bindings.mojo:329-549). */
MGP_API int mgp_icm_predict(void* provider, int T, const float* alpha_rot,
                            const float* Q, const float* scales, const float* Xs,
                            int64_t m, float noise, int variance_method,
                            int max_cg_iter, float cg_tol, int precond_rank,
                            int lanczos_rank, float* mean_out, float* var_out);

/* One BBMM evaluation of the ICM marginal likelihood at fixed parameters
 * (y_c task-blocked, mean removed): NLL per joint entry, y^T K^-1 y, log|K|,
 * base-kernel gradients [P], dNLL/d(os), dNLL/dB [T][T] (os times the
 * mixing gradient, before the reference's +-10 clip), dNLL/dnoise [T] and
 * alpha [T][n], under a Kronecker preconditioner of precond_rank (0: none).
 * The body of one iteration of train_multi_output_jit
 * (jit_multi_output.mojo:406-598); internal there, exposed for parity tests. */
MGP_API int mgp_icm_bbmm_eval(void* provider, int T, float outputscale, const float* B,
                              const float* noise, const float* fixed_noise,
                              const float* y_c, int num_probes, int max_cg_iter,
                              int max_tridiag_iter, float cg_tol, int iteration,
                              int precond_rank, int precond_method, float* nll,
                              float* inv_quad, float* logdet, float* kernel_grads,
                              float* grad_outputscale, float* grad_B,
                              float* noise_grads, float* alpha_out,
                              int* cg_iterations, float* precond_logdet);

/* The Kronecker preconditioner on its own: builds it from the base provider,
 * applies P^-1 to C task-blocked columns rhs [C][T][n] -> solved, draws
 * num_probes N(0, P) probes with the given seed -> probes [num_probes][T][n],
 * and returns log|P| and the factor rank.  KroneckerPreconditioner
 * (kernels/kronecker_preconditioner.mojo:140-730); internal there, exposed
 * for parity tests. */
MGP_API int mgp_kron_precond(void* provider, int T, float outputscale, const float* B,
                             const float* noise, int precond_rank, int precond_method,
                             const float* rhs, int C, float* solved, int num_probes,
                             uint64_t seed, float* probes, float* logdet, int* rank_out);

/* Initial W [T][R] of the task covariance (TaskCovariance.__init__,
 * kernels/task_covariance.mojo:168-210).  Host-only. */
MGP_API int mgp_icm_task_covariance_init(int T, int R, int seed, float* W);

/* Prior draws through a stationary random-Fourier-feature map, fp64:
 * out[k][i] = sqrt(os) sum_f weights[k][f] sqrt(2/F)
 *             cos(sum_q X[i][q] / lengthscales[q] * W[f][q] + phase[f]).
 * Replaces sample_prior_values over the RBF / Matern feature map
 * (mojogp/pathwise_prior.py:37-47, 130-160); W, phase and weights are drawn
 * by the caller. */
MGP_API int mgp_rff_prior_values(const float* X, int64_t n, int d,
                                 const double* lengthscales, const double* W,
                                 const double* phase, int F, double outputscale,
                                 const double* weights, int K, float* out);

/* Streaming device copy of `bytes` repeated `repeats` times; ms_avg gets the
 * mean duration of one copy.  Used only to calibrate HBM byte counters
 * (FETCH_SIZE / WRITE_SIZE) against a kernel of known traffic.  No reference
 * counterpart. */
MGP_API int mgp_calibration_copy(int64_t bytes, int repeats, double* ms_avg);

/* Pipe-throughput probe for the tile kernel's instruction-cost model: out[0]
 * shader clock (GHz), then cycles per wave-instruction per SIMD of out[1]
 * v_exp_f32, out[2] v_fma_f32, out[3] v_mfma_f32_16x16x32_f16, out[4] the same
 * MFMA interleaved with VALU work of the same waves (4 MFMA + 16 FMA per
 * iteration, FMA cycles subtracted), out[5] the compute-unit count.
 * nout >= 6.  Measurement hook; no reference counterpart. */
MGP_API int mgp_pipe_probe(double* out, int nout);

#ifdef __cplusplus
}
#endif

#endif /* MOJOGP_AMD_H */
