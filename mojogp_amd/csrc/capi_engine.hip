// C ABI: training, prediction and the prediction cache.  Declarations (with
// the reference interface each entry point replaces) are in
// include/mojogp_amd.h.
#include <chrono>
#include <cstring>
#include <mutex>
#include <set>

#include "engine.h"
#include "mixed.h"
#include "mojogp_amd.h"

using namespace mgp;

namespace {

Provider* as_provider(void* h) { return checked_provider(h); }

struct PredictionCache {
  Provider* owner = nullptr;
  PredictState state;
  float mean = 0.f;
  int variance_method = 0;
  ExactVarianceOptions exact;
};

// Live prediction-cache handles.  The reference passes the raw pointer as an
// int (jit_engine_bindings.mojo:111-121); here every handle is checked
// against this set, so a destroyed or foreign handle is an error, not a
// use-after-free.
std::mutex g_cache_mu;
std::set<PredictionCache*> g_caches;

PredictionCache* live_cache(void* h) {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  auto* c = static_cast<PredictionCache*>(h);
  MGP_REQUIRE(h != nullptr && g_caches.count(c) != 0,
              "unknown or destroyed prediction cache handle");
  return c;
}

ExactVarianceOptions exact_options(const mgp_predict_opts_t& o) {
  ExactVarianceOptions e;
  e.max_cg_iter = o.max_cg_iter;
  e.cg_tol = o.cg_tol;
  e.precond_rank = o.precond_rank;
  e.block_cols = o.exact_block_cols;
  return e;
}

void fill_exact_info(mgp_predict_info_t* info, const ExactVarianceStats& es) {
  if (!info) return;
  info->exact_block_cols = es.block_cols;
  info->exact_cg_block_count = es.block_count;
  info->exact_cg_total_iterations = es.cg_total_iterations;
  info->exact_cg_max_iterations = es.cg_max_iterations;
  info->exact_precond_rank = es.precond_rank;
}

TrainOptions to_options(const mgp_train_opts_t* o) {
  MGP_REQUIRE(o != nullptr, "null train options");
  TrainOptions t;
  t.max_iterations = o->max_iterations;
  t.learning_rate = o->learning_rate;
  t.num_probes = o->num_probes;
  t.max_cg_iter = o->max_cg_iter;
  t.cg_tol = o->cg_tol;
  t.precond_rank = o->precond_rank;
  t.verbose = o->verbose != 0;
  t.use_cosine_lr = o->use_cosine_lr != 0;
  t.use_preconditioner = o->use_preconditioner != 0;
  t.max_tridiag_iter = o->max_tridiag_iter;
  t.precond_rebuild_threshold = o->precond_rebuild_threshold;
  t.precond_method = o->precond_method;
  t.init_mean = o->init_mean;
  t.enable_early_stopping = o->enable_early_stopping != 0;
  t.early_stop_patience = o->early_stop_patience;
  t.early_stop_tol = o->early_stop_tol;
  t.learn_noise = o->learn_noise != 0;
  t.noise_floor = o->noise_floor;
  t.noise_regularization = o->noise_regularization;
  t.progress_interval = o->progress_interval;
  t.nan_inject_mask = o->nan_inject_mask;
  return t;
}

template <class T>
int copy_out(T* dst, const std::vector<T>& src) {
  if (dst && !src.empty()) std::memcpy(dst, src.data(), src.size() * sizeof(T));
  return (int)src.size();
}

using Clock = std::chrono::steady_clock;
double since(Clock::time_point t0) {
  return std::chrono::duration<double>(Clock::now() - t0).count();
}

// Computes alpha (or uploads alpha_in) and, for LOVE, the inverse root.
void prepare_state(Provider& pv, const float* y, const mgp_predict_opts_t& o,
                   const float* alpha_in, const float* root_in, PredictState& ps,
                   mgp_predict_info_t* info) {
  auto t0 = Clock::now();
  if (!alpha_in && o.variance_method == 1 && !root_in) {
    // Both solves: side by side where the products allow it.
    MGP_REQUIRE(y != nullptr, "training targets are required to solve for alpha");
    MGP_REQUIRE(o.lanczos_rank >= 1, "lanczos_rank must be >= 1 for LOVE variance");
    double a_s = 0.0, r_s = 0.0;
    const int its = solve_alpha_and_root(pv, y, o.mean, o.max_cg_iter, o.cg_tol,
                                         o.lanczos_rank, ps, &a_s, &r_s);
    if (info) {
      info->alpha_cg_iterations = its;
      info->alpha_time_s = a_s;
      info->love_root_time_s = r_s;
    }
    return;
  }
  if (alpha_in) {
    ps.alpha.ensure(pv.n);
    MGP_HIP_CHECK(hipMemcpy(ps.alpha.ptr, alpha_in, pv.n * sizeof(float), hipMemcpyHostToDevice));
    ps.has_alpha = true;
    if (info) info->alpha_cache_used = 1;
  } else {
    MGP_REQUIRE(y != nullptr, "training targets are required to solve for alpha");
    const int its = solve_alpha(pv, y, o.mean, o.max_cg_iter, o.cg_tol, ps);
    if (info) info->alpha_cg_iterations = its;
  }
  if (info) info->alpha_time_s = since(t0);
  if (o.variance_method == 1) {
    auto t1 = Clock::now();
    MGP_REQUIRE(o.lanczos_rank >= 1, "lanczos_rank must be >= 1 for LOVE variance");
    if (root_in) {
      ps.root.ensure((size_t)o.lanczos_rank * pv.n);
      MGP_HIP_CHECK(hipMemcpy(ps.root.ptr, root_in, (size_t)o.lanczos_rank * pv.n * sizeof(float),
                              hipMemcpyHostToDevice));
      ps.rank = o.lanczos_rank;
      if (info) info->love_root_cache_used = 1;
    } else {
      lanczos_inv_root(pv, o.lanczos_rank, ps);
    }
    if (info) info->love_root_time_s = since(t1);
  }
}

}  // namespace

extern "C" {

int mgp_train(void* handle, const float* y, const float* init_params, int nparams,
              float init_noise, const mgp_train_opts_t* opts, mgp_progress_cb cb, void* user,
              mgp_train_result_t* out) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(y && init_params && out, "null argument");
    MGP_REQUIRE(nparams == pv->nparams, "wrong number of initial parameters");
    TrainOptions o = to_options(opts);
    std::function<void(const ProgressEvent&)> progress;
    if (cb) {
      progress = [cb, user](const ProgressEvent& e) {
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
    std::vector<float> ip(init_params, init_params + nparams);
    TrainResult r = train(*pv, y, ip, init_noise, o, progress);
    copy_out(out->params, r.params);
    out->final_nll = r.final_nll;
    out->noise = r.noise;
    out->mean = r.mean;
    out->iterations = r.iterations;
    out->converged = r.converged ? 1 : 0;
    out->history_len = copy_out(out->nll_history, r.nll_history);
    copy_out(out->iter_times_ms, r.iter_times_ms);
    out->cg_history_len = copy_out(out->cg_iterations_history, r.cg_iterations_history);
    out->rank_history_len = copy_out(out->precond_rank_history, r.precond_rank_history);
    out->rebuild_steps_len = copy_out(out->precond_rebuild_steps, r.precond_rebuild_steps);
    out->precond_build_count = r.precond_build_count;
    out->precond_build_total_ms = r.precond_build_total_ms;
    out->has_alpha = r.alpha.empty() ? 0 : 1;
    copy_out(out->cached_alpha, r.alpha);
    out->has_learned_noise = r.learned_noise.empty() ? 0 : 1;
    copy_out(out->learned_noise, r.learned_noise);
    out->noise_fn_len = copy_out(out->noise_fn_params, r.noise_fn_params);
  });
}

int mgp_set_categorical_params(void* handle, const int* cat_kinds, int ncat, const float* raw,
                               int nraw) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(ncat >= 0 && (ncat == 0 || cat_kinds), "null categorical kinds");
    set_categorical_raw(*pv, std::vector<int>(cat_kinds, cat_kinds + ncat), raw, nraw);
  });
}

int mgp_train_mixed(void* handle, const float* y, const float* init_params, int nparams,
                    float init_noise, const int* cat_kinds, int ncat, const float* init_cat_raw,
                    int ncat_params, const mgp_train_opts_t* opts, mgp_progress_cb cb,
                    void* user, mgp_train_result_t* out, float* cat_raw_out) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(y && init_params && out && cat_kinds && init_cat_raw, "null argument");
    MGP_REQUIRE(nparams == pv->nparams, "wrong number of initial parameters");
    TrainOptions o = to_options(opts);
    std::function<void(const ProgressEvent&)> progress;
    if (cb) {
      progress = [cb, user](const ProgressEvent& e) {
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
    MixedTrainResult r = train_mixed(*pv, y, std::vector<float>(init_params, init_params + nparams),
                                     init_noise, std::vector<int>(cat_kinds, cat_kinds + ncat),
                                     std::vector<float>(init_cat_raw, init_cat_raw + ncat_params),
                                     o, progress);
    copy_out(out->params, r.base.params);
    out->final_nll = r.base.final_nll;
    out->noise = r.base.noise;
    out->mean = r.base.mean;
    out->iterations = r.base.iterations;
    out->converged = r.base.converged ? 1 : 0;
    out->history_len = copy_out(out->nll_history, r.base.nll_history);
    copy_out(out->iter_times_ms, r.base.iter_times_ms);
    out->cg_history_len = copy_out(out->cg_iterations_history, r.base.cg_iterations_history);
    out->rank_history_len = 0;
    out->rebuild_steps_len = 0;
    out->precond_build_count = r.base.precond_build_count;
    out->precond_build_total_ms = 0.0;
    out->has_alpha = 0;
    out->has_learned_noise = 0;
    out->noise_fn_len = 0;
    copy_out(cat_raw_out, r.cat_raw);
  });
}

int mgp_bbmm_eval(void* handle, const float* y, float mean, int num_probes, int max_cg_iter,
                  int max_tridiag_iter, float cg_tol, int iteration, int precond_rank,
                  float* nll, float* inv_quad, float* logdet, float* grads,
                  int* cg_iterations, float* precond_logdet, double* cg_loop_ms) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(y && nll && grads, "null argument");
    const int64_t n = pv->n;
    Precond P;
    build_precond(*pv, precond_rank, training_pivot_options(0), P);
    DevBuf<float> yc;
    yc.ensure(n);
    MGP_HIP_CHECK(hipMemcpyAsync(yc.ptr, y, n * sizeof(float), hipMemcpyHostToDevice, pv->st));
    sub_scalar(yc.ptr, yc.ptr, mean, n, pv->st);
    BBMMWork w;
    BBMMResult r = bbmm_step(*pv, P, precond_rank > 0, yc.ptr, num_probes, max_cg_iter,
                             max_tridiag_iter, cg_tol, iteration, false, w);
    *nll = r.nll;
    if (inv_quad) *inv_quad = r.inv_quad;
    if (logdet) *logdet = r.logdet;
    if (cg_iterations) *cg_iterations = r.cg_iterations;
    if (precond_logdet) *precond_logdet = P.logdet;
    if (cg_loop_ms) *cg_loop_ms = r.cg_loop_ms;
    std::memcpy(grads, r.grads.data(), r.grads.size() * sizeof(float));
  });
}

int mgp_gaussian(int64_t len, uint64_t seed, float* out) {
  return guarded([&] {
    MGP_REQUIRE(len >= 1 && out, "bad arguments");
    DevBuf<float> d;
    d.ensure(len);
    gaussian(d.ptr, len, seed, nullptr);
    MGP_HIP_CHECK(hipMemcpy(out, d.ptr, len * sizeof(float), hipMemcpyDeviceToHost));
  });
}

int mgp_pivoted_cholesky(void* handle, int rank, int method, float error_tol,
                         float adaptive_tol, uint64_t seed, float* L_out, int* rank_out,
                         float* logdet) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    Precond P;
    PivotOptions po;
    po.method = method;
    po.error_tol = error_tol;
    po.adaptive_tol = adaptive_tol;
    po.seed = seed;
    build_precond(*pv, rank, po, P);
    if (rank_out) *rank_out = P.rank;
    if (logdet) *logdet = P.logdet;
    if (L_out && P.rank > 0)
      MGP_HIP_CHECK(hipMemcpy(L_out, P.L.ptr, (size_t)P.rank * pv->n * sizeof(float),
                              hipMemcpyDeviceToHost));
  });
}

int mgp_predict(void* handle, const float* y, const float* Xs, int64_t m,
                const mgp_predict_opts_t* opts, const float* alpha_in, const float* root_in,
                float* mean_out, float* var_out, float* alpha_out, float* root_out,
                mgp_predict_info_t* info) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(opts && Xs && mean_out, "null argument");
    MGP_REQUIRE(m >= 1, "need at least one test point");
    MGP_REQUIRE(opts->variance_method >= 0 && opts->variance_method <= 2,
                "variance_method must be 0 (mean), 1 (LOVE) or 2 (exact)");
    MGP_REQUIRE(opts->variance_method == 0 || var_out, "variance output is null");
    if (info) std::memset(info, 0, sizeof(*info));
    auto t0 = Clock::now();
    PredictState ps;
    prepare_state(*pv, y, *opts, alpha_in, root_in, ps, info);
    PredictTimes t;
    const ExactVarianceOptions eo = exact_options(*opts);
    ExactVarianceStats es;
    predict_from_state(*pv, ps, Xs, m, opts->mean, opts->variance_method, mean_out, var_out, t,
                       &eo, &es);
    if (opts->variance_method == 2) fill_exact_info(info, es);
    if (alpha_out && !alpha_in)
      MGP_HIP_CHECK(hipMemcpy(alpha_out, ps.alpha.ptr, pv->n * sizeof(float), hipMemcpyDeviceToHost));
    if (root_out && opts->variance_method == 1 && !root_in)
      MGP_HIP_CHECK(hipMemcpy(root_out, ps.root.ptr, (size_t)ps.rank * pv->n * sizeof(float),
                              hipMemcpyDeviceToHost));
    if (info) {
      info->mean_time_s = t.mean_s;
      info->variance_time_s = t.variance_s;
      info->total_time_s = since(t0);
    }
  });
}

int mgp_prepare_prediction_cache(void* handle, const float* y, const mgp_predict_opts_t* opts,
                                 const float* alpha_in, void** cache_out,
                                 mgp_predict_info_t* info) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    MGP_REQUIRE(opts && cache_out, "null argument");
    *cache_out = nullptr;
    if (info) std::memset(info, 0, sizeof(*info));
    auto* c = new PredictionCache();
    try {
      c->owner = pv;
      c->mean = opts->mean;
      c->variance_method = opts->variance_method;
      c->exact = exact_options(*opts);
      prepare_state(*pv, y, *opts, alpha_in, nullptr, c->state, info);
    } catch (...) {
      delete c;
      throw;
    }
    {
      std::lock_guard<std::mutex> lk(g_cache_mu);
      g_caches.insert(c);
    }
    *cache_out = c;
  });
}

int mgp_predict_with_cache(void* handle, void* cache, const float* Xs, int64_t m,
                           int variance_method, float* mean_out, float* var_out,
                           mgp_predict_info_t* info) {
  return guarded([&] {
    Provider* pv = as_provider(handle);
    auto* c = live_cache(cache);
    MGP_REQUIRE(c->owner == pv, "prediction cache belongs to another provider");
    MGP_REQUIRE(variance_method != 1 || c->state.rank > 0,
                "cache holds no LOVE root; prepare it with variance_method=1");
    if (info) std::memset(info, 0, sizeof(*info));
    auto t0 = Clock::now();
    PredictTimes t;
    ExactVarianceStats es;
    predict_from_state(*pv, c->state, Xs, m, c->mean, variance_method, mean_out, var_out, t,
                       &c->exact, &es);
    if (variance_method == 2) fill_exact_info(info, es);
    if (info) {
      info->alpha_cache_used = 1;
      info->love_root_cache_used = variance_method == 1;
      info->mean_time_s = t.mean_s;
      info->variance_time_s = t.variance_s;
      info->total_time_s = since(t0);
    }
  });
}

int mgp_destroy_prediction_cache(void* cache) {
  return guarded([&] {
    auto* c = live_cache(cache);
    {
      std::lock_guard<std::mutex> lk(g_cache_mu);
      g_caches.erase(c);
    }
    delete c;
  });
}

}  // extern "C"
