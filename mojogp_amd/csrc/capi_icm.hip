// C entry points of the ICM (Kronecker) multi-output engine (declarations
// and the reference interface each replaces are in include/mojogp_amd.h).
#include <cmath>
#include <cstring>

#include "host_numerics.h"
#include "icm.h"
#include "mojogp_amd.h"

using namespace mgp;

namespace {

Provider* provider_of(void* h) { return checked_provider(h); }

template <class T>
int copy_to(T* dst, const std::vector<T>& src) {
  if (dst && !src.empty()) std::memcpy(dst, src.data(), src.size() * sizeof(T));
  return (int)src.size();
}

// One-latent LMC model over the base provider with A = os B.
void icm_model(LMCModel& m, Provider* pv, int T, float os, const float* B, const float* noise,
               const float* fixed) {
  if (T < 1 || !B || !noise) throw Error(ST_INVALID, "need T >= 1, B and noise");
  m.R = 1;
  m.T = T;
  m.n = pv->n;
  m.prov.push_back(pv);
  m.st = pv->st;
  m.A.resize((size_t)T * T);
  for (int i = 0; i < T * T; ++i) m.A[i] = os * B[i];
  m.noise.assign(noise, noise + T);
  if (fixed) m.fixed.assign(fixed, fixed + (size_t)m.n * T);
}

ICMTrainOptions icm_options(const mgp_icm_train_opts_t* opts) {
  ICMTrainOptions o;
  o.max_iterations = opts->max_iterations;
  o.learning_rate = opts->learning_rate;
  o.task_rank = opts->task_rank;
  o.num_probes = opts->num_probes;
  o.max_cg_iter = opts->max_cg_iter;
  o.cg_tol = opts->cg_tol;
  o.precond_rank = opts->precond_rank;
  o.precond_method = opts->precond_method;
  o.precond_rebuild_threshold = opts->precond_rebuild_threshold;
  o.max_tridiag_iter = opts->max_tridiag_iter;
  o.early_stop_patience = opts->early_stop_patience;
  o.early_stop_tol = opts->early_stop_tol;
  o.use_cosine_lr = opts->use_cosine_lr != 0;
  o.progress_interval = opts->progress_interval;
  if (o.num_probes < 0 || o.max_cg_iter < 1 || o.max_tridiag_iter < 0)
    throw Error(ST_INVALID, "bad CG settings");
  return o;
}

std::function<void(const ProgressEvent&)> icm_progress(mgp_progress_cb cb, void* user) {
  if (!cb) return {};
  return [cb, user](const ProgressEvent& e) {
    mgp_progress_t p;
    p.phase = e.phase;
    p.current = e.current;
    p.total = e.total;
    p.nll = e.nll;
    p.best_nll = e.best_nll;
    p.cg_iter = e.cg_iter;
    p.iter_ms = e.iter_ms;
    p.noise = e.noise;
    p.mean = e.mean;
    p.precond_rank = e.precond_rank;
    p.precond_rebuild_count = e.precond_rebuild_count;
    p.converged = e.converged ? 1 : 0;
    cb(&p, user);
  };
}

void put_icm_result(const ICMTrainResult& r, mgp_icm_train_result_t* out) {
  copy_to(out->params, r.params);
  copy_to(out->noise, r.noise);
  copy_to(out->mean, r.mean);
  copy_to(out->B, r.B);
  copy_to(out->alpha, r.alpha);
  out->history_len = copy_to(out->nll_history, r.nll_history);
  copy_to(out->cg_iterations_history, r.cg_iterations_history);
  copy_to(out->iter_times_ms, r.iter_times_ms);
  out->outputscale = r.outputscale;
  out->final_nll = r.final_nll;
  out->iterations = r.iterations;
  out->converged = r.converged ? 1 : 0;
  out->task_rank = r.task_rank;
  out->precond_rebuild_count = r.precond_rebuild_count;
}

}  // namespace

extern "C" {

int mgp_icm_train(void* provider, int T, const float* y_blocked, const float* init_params,
                  const int* trainable, const float* init_noise, float init_outputscale,
                  const float* init_mean, const float* fixed_noise,
                  const mgp_icm_train_opts_t* opts, mgp_progress_cb cb, void* user,
                  mgp_icm_train_result_t* out) {
  return guarded([&] {
    Provider* pv = provider_of(provider);
    if (!y_blocked || !init_params || !trainable || !init_noise || !init_mean || !opts || !out)
      throw Error(ST_INVALID, "null argument");
    if (T < 1) throw Error(ST_INVALID, "num_tasks must be >= 1");
    const int P = pv->nparams;
    const ICMTrainOptions o = icm_options(opts);
    std::vector<float> ip(init_params, init_params + P);
    std::vector<char> tm(P);
    for (int p = 0; p < P; ++p) tm[p] = trainable[p] != 0;
    std::vector<float> noise0(init_noise, init_noise + T), mean0(init_mean, init_mean + T);
    std::vector<float> fixed;
    if (fixed_noise) fixed.assign(fixed_noise, fixed_noise + (size_t)pv->n * T);
    ICMTrainResult r = icm_train(*pv, T, y_blocked, ip, tm, noise0, init_outputscale, mean0,
                                 fixed, o, icm_progress(cb, user));
    put_icm_result(r, out);
  });
}

int mgp_icm_train_mixed(void* provider, int T, const float* y_blocked, const float* init_params,
                        const float* init_noise, float init_outputscale, const float* init_mean,
                        const int* cat_kinds, int ncat, const float* init_cat_raw,
                        int ncat_params, const mgp_icm_train_opts_t* opts, mgp_progress_cb cb,
                        void* user, mgp_icm_train_result_t* out, float* cat_raw_out) {
  return guarded([&] {
    Provider* pv = provider_of(provider);
    if (!y_blocked || !init_params || !init_noise || !init_mean || !opts || !out)
      throw Error(ST_INVALID, "null argument");
    if (T < 1) throw Error(ST_INVALID, "num_tasks must be >= 1");
    if (ncat < 1 || !cat_kinds) throw Error(ST_INVALID, "cat_kinds must name every categorical leaf");
    if (ncat_params < 0 || (ncat_params > 0 && !init_cat_raw))
      throw Error(ST_INVALID, "init_cat_raw must hold ncat_params values");
    const int P = pv->nparams;
    const ICMTrainOptions o = icm_options(opts);
    std::vector<float> ip(init_params, init_params + P);
    std::vector<float> noise0(init_noise, init_noise + T), mean0(init_mean, init_mean + T);
    std::vector<int> kinds(cat_kinds, cat_kinds + ncat);
    std::vector<float> raw0(init_cat_raw, init_cat_raw + ncat_params);
    ICMMixedResult r = icm_train_mixed(*pv, T, y_blocked, ip, noise0, init_outputscale, mean0,
                                       kinds, raw0, o, icm_progress(cb, user));
    put_icm_result(r, out);
    copy_to(cat_raw_out, r.cat_raw);
  });
}

int mgp_icm_predict(void* provider, int T, const float* alpha_rot, const float* Q,
                    const float* scales, const float* Xs, int64_t m, float noise,
                    int variance_method, int max_cg_iter, float cg_tol, int precond_rank,
                    int lanczos_rank, float* mean_out, float* var_out) {
  return guarded([&] {
    Provider* pv = provider_of(provider);
    if (!alpha_rot || !Q || !scales || !Xs || !mean_out) throw Error(ST_INVALID, "null argument");
    if (!(noise >= 0.0f)) throw Error(ST_INVALID, "noise must be >= 0");
    icm_predict(*pv, T, alpha_rot, Q, scales, Xs, m, noise, variance_method, max_cg_iter, cg_tol,
                precond_rank, lanczos_rank, mean_out, var_out);
  });
}

int mgp_icm_bbmm_eval(void* provider, int T, float outputscale, const float* B,
                      const float* noise, const float* fixed_noise, const float* y_c,
                      int num_probes, int max_cg_iter, int max_tridiag_iter, float cg_tol,
                      int iteration, int precond_rank, int precond_method, float* nll,
                      float* inv_quad, float* logdet, float* kernel_grads, float* grad_outputscale,
                      float* grad_B, float* noise_grads, float* alpha_out, int* cg_iterations,
                      float* precond_logdet) {
  return guarded([&] {
    Provider* pv = provider_of(provider);
    if (!y_c || num_probes < 0 || max_cg_iter < 1) throw Error(ST_INVALID, "bad arguments");
    LMCModel m;
    icm_model(m, pv, T, outputscale, B, noise, fixed_noise);
    m.upload();
    DevBuf<float> yd;
    yd.ensure((size_t)m.size());
    MGP_HIP_CHECK(hipMemcpyAsync(yd.ptr, y_c, m.size() * sizeof(float), hipMemcpyHostToDevice,
                                 m.st));
    KronPrecond Pk;
    std::vector<float> Bv(B, B + (size_t)T * T), nv(noise, noise + T);
    if (precond_rank > 0)
      Pk.build_kron(m, precond_rank, training_pivot_options(precond_method), outputscale, Bv, nv);
    LMCWork w;
    LMCEval ev = lmc_bbmm(m, precond_rank > 0 ? &Pk : nullptr, yd.ptr, num_probes, max_cg_iter,
                          max_tridiag_iter, cg_tol, iteration, false, w);
    if (nll) *nll = ev.nll;
    if (inv_quad) *inv_quad = ev.inv_quad;
    if (logdet) *logdet = ev.logdet;
    copy_to(kernel_grads, ev.kernel_grads);
    double gos = 0.0;
    for (int i = 0; i < T * T; ++i) gos += (double)B[i] * (double)ev.G_A[i];
    if (grad_outputscale) *grad_outputscale = (float)gos;
    if (grad_B)
      for (int i = 0; i < T * T; ++i) grad_B[i] = outputscale * ev.G_A[i];
    copy_to(noise_grads, ev.noise_grads);
    copy_to(alpha_out, ev.alpha);
    if (cg_iterations) *cg_iterations = ev.cg_iterations;
    if (precond_logdet) *precond_logdet = Pk.active() ? Pk.logdet : 0.0f;
  });
}

int mgp_kron_precond(void* provider, int T, float outputscale, const float* B,
                     const float* noise, int precond_rank, int precond_method, const float* rhs,
                     int C, float* solved, int num_probes, uint64_t seed, float* probes,
                     float* logdet, int* rank_out) {
  return guarded([&] {
    Provider* pv = provider_of(provider);
    if (precond_rank < 1 || C < 0 || num_probes < 0) throw Error(ST_INVALID, "bad arguments");
    LMCModel m;
    icm_model(m, pv, T, outputscale, B, noise, nullptr);
    KronPrecond Pk;
    std::vector<float> Bv(B, B + (size_t)T * T), nv(noise, noise + T);
    Pk.build_kron(m, precond_rank, training_pivot_options(precond_method), outputscale, Bv, nv);
    if (rank_out) *rank_out = Pk.active() ? Pk.rank[0] : 0;
    if (logdet) *logdet = Pk.logdet;
    if (!Pk.active()) throw Error(ST_NUMERIC, "pivoted Cholesky returned rank 0");
    const size_t N = (size_t)m.size();
    if (C > 0 && rhs && solved) {
      DevBuf<float> dr, dz;
      dr.ensure(N * C);
      dz.ensure(N * C);
      MGP_HIP_CHECK(hipMemcpyAsync(dr.ptr, rhs, N * C * sizeof(float), hipMemcpyHostToDevice, m.st));
      Pk.apply(dr.ptr, C, dz.ptr, nullptr, 0, m.st);
      MGP_HIP_CHECK(hipMemcpyAsync(solved, dz.ptr, N * C * sizeof(float), hipMemcpyDeviceToHost,
                                   m.st));
    }
    if (num_probes > 0 && probes) {
      DevBuf<float> dp;
      dp.ensure(N * num_probes);
      Pk.sample(dp.ptr, num_probes, seed, m.st);
      MGP_HIP_CHECK(hipMemcpyAsync(probes, dp.ptr, N * num_probes * sizeof(float),
                                   hipMemcpyDeviceToHost, m.st));
    }
    MGP_HIP_CHECK(hipStreamSynchronize(m.st));
  });
}

int mgp_icm_task_covariance_init(int T, int R, int seed, float* W) {
  return guarded([&] {
    if (T < 1 || R < 1 || !W) throw Error(ST_INVALID, "bad arguments");
    std::vector<float> w = icm_init_w(T, R, seed);
    std::memcpy(W, w.data(), w.size() * sizeof(float));
  });
}

}  // extern "C"
