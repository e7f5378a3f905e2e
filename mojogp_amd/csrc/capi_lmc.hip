// C entry points of the LMC multi-output engine (declarations and the
// reference interface each replaces are in include/mojogp_amd.h).
#include <cmath>
#include <cstring>
#include <string>

#include "lmc.h"
#include "mixed.h"
#include "mojogp_amd.h"

using namespace mgp;

namespace {

void init_model(LMCModel& m, void* const* providers, int R, int T) {
  if (providers == nullptr || R < 1 || T < 1) throw Error(ST_INVALID, "need >= 1 latent and task");
  m.R = R;
  m.T = T;
  for (int s = 0; s < R; ++s) {
    if (providers[s] == nullptr) throw Error(ST_INVALID, "null latent provider");
    m.prov.push_back(checked_provider(providers[s]));
  }
  m.n = m.prov[0]->n;
  for (Provider* p : m.prov)
    if (p->n != m.n) throw Error(ST_INVALID, "latent providers must share the training inputs");
  m.st = m.prov[0]->st;
}

void set_fixed(LMCModel& m, const float* fixed) {
  m.fixed.clear();
  if (fixed) m.fixed.assign(fixed, fixed + (size_t)m.n * m.T);
}

void set_mixing(LMCModel& m, const float* A, const float* noise) {
  if (!A || !noise) throw Error(ST_INVALID, "A and noise are required");
  m.A.assign(A, A + (size_t)m.R * m.T * m.T);
  m.noise.assign(noise, noise + m.T);
  for (int t = 0; t < m.T; ++t)
    if (!std::isfinite(m.noise[t]) || m.noise[t] < 0.0f)
      throw Error(ST_INVALID, "task noise must be finite and >= 0");
}

LMCTrainOptions train_options(const mgp_lmc_train_opts_t* opts) {
  LMCTrainOptions o;
  o.max_iterations = opts->max_iterations;
  o.learning_rate = opts->learning_rate;
  o.num_probes = opts->num_probes;
  o.max_cg_iter = opts->max_cg_iter;
  o.max_tridiag_iter = opts->max_tridiag_iter;
  o.cg_tol = opts->cg_tol;
  o.precond_rank = opts->precond_rank;
  o.precond_method = opts->precond_method;
  o.precond_rebuild_threshold = opts->precond_rebuild_threshold;
  o.early_stop_tol = opts->early_stop_tol;
  o.early_stop_patience = opts->early_stop_patience;
  return o;
}

void put_result(const LMCTrainResult& r, const mgp_lmc_train_opts_t* opts,
                mgp_lmc_train_result_t* out) {
  auto put = [](float* dst, const std::vector<float>& v) {
    if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(float));
  };
  if (out->params) {
    size_t q = 0;
    for (const auto& ps : r.params)
      for (float v : ps) out->params[q++] = v;
  }
  put(out->A, r.A);
  put(out->L, r.L);
  put(out->var_diag, r.var_diag);
  put(out->noise, r.noise);
  put(out->mean, r.mean);
  put(out->alpha, r.alpha);
  const int hl = (int)std::min<size_t>(r.nll_history.size(), (size_t)opts->max_iterations);
  if (out->nll_history)
    for (int i = 0; i < hl; ++i) out->nll_history[i] = r.nll_history[i];
  if (out->iter_times_ms)
    for (int i = 0; i < (int)std::min<size_t>(r.iter_times_ms.size(), (size_t)opts->max_iterations); ++i)
      out->iter_times_ms[i] = r.iter_times_ms[i];
  out->history_len = hl;
  out->final_nll = r.final_nll;
  out->iterations = r.iterations;
  out->converged = r.converged ? 1 : 0;
  out->precond_rebuild_count = r.precond_rebuild_count;
}

}  // namespace

extern "C" {

int mgp_lmc_forward_matvec(void* const* providers, int R, int T, const float* A,
                           const float* noise, const float* fixed_noise, const float* V, int C,
                           float* out) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!V || !out || C < 1) throw Error(ST_INVALID, "bad arguments");
    set_mixing(m, A, noise);
    set_fixed(m, fixed_noise);
    LMCStreamGuard guard(m);
    m.upload();
    const size_t tot = (size_t)m.size() * C;
    DevBuf<float> dv, dout;
    dv.ensure(tot);
    dout.ensure(tot);
    MGP_HIP_CHECK(hipMemcpyAsync(dv.ptr, V, tot * sizeof(float), hipMemcpyHostToDevice, m.st));
    m.forward(dv.ptr, C, dout.ptr);
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout.ptr, tot * sizeof(float), hipMemcpyDeviceToHost, m.st));
    MGP_HIP_CHECK(hipStreamSynchronize(m.st));
  });
}

int mgp_lmc_train(void* const* providers, int R, int T, const float* y_blocked,
                  const float* init_params, const int* trainable, const float* init_noise,
                  const float* fixed_noise, const float* init_mean,
                  const mgp_lmc_train_opts_t* opts, mgp_lmc_train_result_t* out) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    set_fixed(m, fixed_noise);
    if (!y_blocked || !init_params || !trainable || !init_noise || !init_mean || !opts || !out)
      throw Error(ST_INVALID, "null argument");
    std::vector<std::vector<float>> ip(R);
    std::vector<std::vector<char>> tm(R);
    int off = 0;
    for (int s = 0; s < R; ++s) {
      const int P = m.prov[s]->nparams;
      ip[s].assign(init_params + off, init_params + off + P);
      for (int q = 0; q < P; ++q) tm[s].push_back(trainable[off + q] ? 1 : 0);
      off += P;
    }
    const LMCTrainOptions o = train_options(opts);
    std::vector<float> noise(init_noise, init_noise + T), mean(init_mean, init_mean + T);
    LMCTrainResult r = lmc_train(m, y_blocked, ip, tm, noise, mean, o);
    put_result(r, opts, out);
  });
}

int mgp_lmc_train_mixed(void* const* providers, int R, int T, const float* y_blocked,
                        const float* init_params, const float* init_noise,
                        const float* fixed_noise, const float* init_mean, const int* cat_counts,
                        const int* cat_kinds, const float* init_cat_raw, int ncat_params,
                        const mgp_lmc_train_opts_t* opts, mgp_lmc_train_result_t* out,
                        float* cat_raw_out, float* cat_params_out) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    set_fixed(m, fixed_noise);
    if (!y_blocked || !init_params || !init_noise || !init_mean || !cat_counts || !opts || !out)
      throw Error(ST_INVALID, "null argument");
    if (ncat_params < 0 || (ncat_params > 0 && !init_cat_raw))
      throw Error(ST_INVALID, "init_cat_raw must hold ncat_params values");
    std::vector<std::vector<float>> ip(R), craw(R);
    std::vector<std::vector<int>> ck(R);
    std::vector<std::vector<CatLeafRef>> leaves(R);
    int off = 0, koff = 0, roff = 0;
    for (int s = 0; s < R; ++s) {
      Provider& pv = *m.prov[s];
      ip[s].assign(init_params + off, init_params + off + pv.nparams);
      off += pv.nparams;
      const int cc = cat_counts[s];
      if (cc < 0) throw Error(ST_INVALID, "cat_counts must be >= 0");
      if (cc == 0) continue;
      if (!cat_kinds) throw Error(ST_INVALID, "cat_kinds is required with categorical leaves");
      if (!pv.is_tree) throw Error(ST_INVALID, "categorical leaves need a kernel-tree latent");
      ck[s].assign(cat_kinds + koff, cat_kinds + koff + cc);
      koff += cc;
      leaves[s] = cat_leaves(pv, ck[s]);
      int K = 0;
      for (const auto& c : leaves[s]) K += c.nparam;
      if (roff + K > ncat_params)
        throw Error(ST_INVALID, "ncat_params is smaller than the categorical leaves need");
      craw[s].assign(init_cat_raw + roff, init_cat_raw + roff + K);
      roff += K;
    }
    if (roff != ncat_params)
      throw Error(ST_INVALID, "ncat_params must equal the categorical leaves' parameter count (" +
                                  std::to_string(roff) + ")");
    const LMCTrainOptions o = train_options(opts);
    std::vector<float> noise(init_noise, init_noise + T), mean(init_mean, init_mean + T);
    LMCMixedResult r = lmc_train_mixed(m, y_blocked, ip, ck, craw, noise, mean, o);
    put_result(r, opts, out);
    int q = 0;
    std::vector<double> th;
    for (int s = 0; s < R; ++s)
      for (const auto& c : leaves[s]) {
        th.resize((size_t)c.nparam);
        cat_constrain(c.kind, c.L, r.cat_raw[s].data() + c.param_off, c.nparam, th.data(),
                      nullptr);
        for (int k = 0; k < c.nparam; ++k, ++q) {
          if (cat_raw_out) cat_raw_out[q] = r.cat_raw[s][(size_t)(c.param_off + k)];
          if (cat_params_out) cat_params_out[q] = (float)th[(size_t)k];
        }
      }
  });
}

int mgp_lmc_predict(void* const* providers, int R, int T, const float* A, const float* alpha,
                    const float* mean, const float* noise, const float* Xs, int64_t mtest,
                    int variance_method, int max_cg_iter, float cg_tol, int precond_rank,
                    int lanczos_rank, float* mean_out, float* var_out, float* latent_var_out) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!A || !alpha || !mean || !Xs || !mean_out || mtest < 1)
      throw Error(ST_INVALID, "bad arguments");
    if (variance_method < 0 || variance_method > 2)
      throw Error(ST_INVALID, "variance_method must be 0, 1 or 2");
    if (variance_method != 0 && (!var_out || !noise))
      throw Error(ST_INVALID, "variance needs noise and an output array");
    std::vector<float> zeros(T, 0.0f);
    set_mixing(m, A, noise ? noise : zeros.data());
    LMCStreamGuard guard(m);
    m.upload();
    const int d = m.prov[0]->d;
    DevBuf<float> dx, da;
    dx.ensure((size_t)mtest * d);
    da.ensure((size_t)m.size());
    MGP_HIP_CHECK(hipMemcpyAsync(dx.ptr, Xs, (size_t)mtest * d * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    MGP_HIP_CHECK(hipMemcpyAsync(da.ptr, alpha, (size_t)m.size() * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    for (Provider* p : m.prov) {
      if (p->d != d) throw Error(ST_INVALID, "latent providers must share the input dimension");
      p->pack(dx.ptr, mtest, p->test);
    }
    std::vector<float> mv(mean, mean + T);
    lmc_predict_mean(m, da.ptr, mtest, mv, mean_out);
    if (variance_method == 0) return;
    if (variance_method == 1 && lanczos_rank < 1)
      throw Error(ST_INVALID, "lanczos_rank must be >= 1 for LOVE variance");
    // Per-latent variance with the provider noise set to the average task
    // noise, mixed by sum_t' A_s[t][t']^2, plus the task noise
    // (jit_engine_lmc_bindings.mojo:1196-1390).
    float avg = 0.0f;
    for (int t = 0; t < T; ++t) avg += m.noise[t];
    avg /= (float)T;
    std::memset(var_out, 0, (size_t)mtest * T * sizeof(float));
    DevBuf<float> vs;
    vs.ensure((size_t)mtest);
    std::vector<float> hv((size_t)mtest);
    for (int s = 0; s < R; ++s) {
      Provider& pv = *m.prov[s];
      const float saved = pv.noise;
      pv.noise = avg;
      try {
        if (variance_method == 1) {
          PredictState ps;
          lanczos_inv_root(pv, lanczos_rank, ps);
          DevBuf<float> V;
          V.ensure((size_t)ps.rank * mtest);
          pv.cross(pv.test, ps.root.ptr, ps.rank, V.ptr);
          love_variance(V.ptr, mtest, ps.rank, pv.kdiag(), vs.ptr, m.st);
        } else {
          ExactVarianceOptions eo;
          eo.max_cg_iter = max_cg_iter;
          eo.cg_tol = cg_tol;
          eo.precond_rank = precond_rank;
          ExactVarianceStats es;
          exact_variance(pv, mtest, eo, vs.ptr, es);
        }
      } catch (...) {
        pv.noise = saved;
        throw;
      }
      pv.noise = saved;
      MGP_HIP_CHECK(hipMemcpyAsync(hv.data(), vs.ptr, mtest * sizeof(float), hipMemcpyDeviceToHost,
                                   m.st));
      MGP_HIP_CHECK(hipStreamSynchronize(m.st));
      if (latent_var_out) std::memcpy(latent_var_out + (size_t)s * mtest, hv.data(), mtest * sizeof(float));
      for (int t = 0; t < T; ++t) {
        float w = 0.0f;
        for (int tp = 0; tp < T; ++tp) {
          const float a = m.A[(size_t)s * T * T + t * T + tp];
          w += a * a;
        }
        for (int64_t i = 0; i < mtest; ++i) var_out[(size_t)i * T + t] += w * hv[(size_t)i];
      }
    }
    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < mtest; ++i) var_out[(size_t)i * T + t] += m.noise[t];
  });
}

int mgp_lmc_bbmm_eval(void* const* providers, int R, int T, const float* A, const float* noise,
                      const float* fixed_noise, const float* y_c, int num_probes, int max_cg_iter,
                      int max_tridiag_iter, float cg_tol, int iteration, int precond_rank,
                      int precond_method, float* nll, float* inv_quad, float* logdet,
                      float* kernel_grads, float* grad_A, float* noise_grads, float* alpha_out,
                      int* cg_iterations, float* precond_logdet, double* cg_loop_ms) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!y_c || num_probes < 0 || max_cg_iter < 1) throw Error(ST_INVALID, "bad arguments");
    set_mixing(m, A, noise);
    set_fixed(m, fixed_noise);
    LMCStreamGuard guard(m);
    m.upload();
    DevBuf<float> yd;
    yd.ensure((size_t)m.size());
    MGP_HIP_CHECK(hipMemcpyAsync(yd.ptr, y_c, (size_t)m.size() * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    LMCPrecond P;
    PivotOptions po = training_pivot_options(precond_method);
    if (precond_rank > 0) P.build(m, precond_rank, po);
    LMCWork w;
    LMCEval ev = lmc_bbmm(m, precond_rank > 0 ? &P : nullptr, yd.ptr, num_probes, max_cg_iter,
                          max_tridiag_iter, cg_tol, iteration, false, w);
    if (nll) *nll = ev.nll;
    if (inv_quad) *inv_quad = ev.inv_quad;
    if (logdet) *logdet = ev.logdet;
    if (kernel_grads) std::memcpy(kernel_grads, ev.kernel_grads.data(), ev.kernel_grads.size() * sizeof(float));
    if (grad_A) std::memcpy(grad_A, ev.G_A.data(), ev.G_A.size() * sizeof(float));
    if (noise_grads) std::memcpy(noise_grads, ev.noise_grads.data(), ev.noise_grads.size() * sizeof(float));
    if (alpha_out) std::memcpy(alpha_out, ev.alpha.data(), ev.alpha.size() * sizeof(float));
    if (cg_iterations) *cg_iterations = ev.cg_iterations;
    if (precond_logdet) *precond_logdet = P.active() ? P.logdet : 0.0f;
    if (cg_loop_ms) *cg_loop_ms = ev.cg_loop_ms;
  });
}

int mgp_lmc_benchmark_forward(void* const* providers, int R, int T, const float* A,
                              const float* noise, const float* V, int C, int repeats, int warmup,
                              double* times_ms, float* out) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!V || !times_ms || C < 1 || repeats < 1 || warmup < 0) throw Error(ST_INVALID, "bad arguments");
    set_mixing(m, A, noise);
    LMCStreamGuard guard(m);
    m.upload();
    const size_t tot = (size_t)m.size() * C;
    DevBuf<float> dv, dout;
    dv.ensure(tot);
    dout.ensure(tot);
    MGP_HIP_CHECK(hipMemcpyAsync(dv.ptr, V, tot * sizeof(float), hipMemcpyHostToDevice, m.st));
    for (int i = 0; i < warmup; ++i) m.forward(dv.ptr, C, dout.ptr);
    hipEvent_t e0, e1;
    MGP_HIP_CHECK(hipEventCreate(&e0));
    MGP_HIP_CHECK(hipEventCreate(&e1));
    for (int i = 0; i < repeats; ++i) {
      MGP_HIP_CHECK(hipEventRecord(e0, m.st));
      m.forward(dv.ptr, C, dout.ptr);
      MGP_HIP_CHECK(hipEventRecord(e1, m.st));
      MGP_HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0.0f;
      MGP_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      times_ms[i] = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (out)
      MGP_HIP_CHECK(hipMemcpyAsync(out, dout.ptr, tot * sizeof(float), hipMemcpyDeviceToHost, m.st));
    MGP_HIP_CHECK(hipStreamSynchronize(m.st));
  });
}

int mgp_lmc_exact_variance(void* const* providers, int R, int T, const float* A,
                           const float* noise, const float* fixed_noise, const float* Xs,
                           int64_t mtest, int max_cg_iter, float cg_tol, int block_points,
                           float* var_out, int* cg_iterations) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!Xs || !var_out || mtest < 1 || max_cg_iter < 1) throw Error(ST_INVALID, "bad arguments");
    set_mixing(m, A, noise);
    set_fixed(m, fixed_noise);
    LMCStreamGuard guard(m);
    m.upload();
    const int d = m.prov[0]->d;
    DevBuf<float> dx;
    dx.ensure((size_t)mtest * d);
    MGP_HIP_CHECK(hipMemcpyAsync(dx.ptr, Xs, (size_t)mtest * d * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    for (Provider* p : m.prov) {
      if (p->d != d) throw Error(ST_INVALID, "latent providers must share the input dimension");
      p->pack(dx.ptr, mtest, p->test);
    }
    const int its = lmc_exact_variance(m, mtest, max_cg_iter, cg_tol, block_points, var_out);
    if (cg_iterations) *cg_iterations = its;
  });
}

int mgp_lmc_pathwise_correction(void* const* providers, int R, int T, const float* A,
                                const float* noise, const float* fixed_noise,
                                const float* residual, int S, const float* Xs, int64_t mtest,
                                int max_cg_iter, float cg_tol, float* correction_out,
                                int* cg_iterations) {
  return guarded([&] {
    LMCModel m;
    init_model(m, providers, R, T);
    if (!residual || !Xs || !correction_out || S < 1 || mtest < 1 || max_cg_iter < 1)
      throw Error(ST_INVALID, "bad arguments");
    set_mixing(m, A, noise);
    set_fixed(m, fixed_noise);
    LMCStreamGuard guard(m);
    m.upload();
    const int d = m.prov[0]->d;
    DevBuf<float> dx, dr;
    dx.ensure((size_t)mtest * d);
    dr.ensure((size_t)m.size() * S);
    MGP_HIP_CHECK(hipMemcpyAsync(dx.ptr, Xs, (size_t)mtest * d * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    MGP_HIP_CHECK(hipMemcpyAsync(dr.ptr, residual, (size_t)m.size() * S * sizeof(float),
                                 hipMemcpyHostToDevice, m.st));
    for (Provider* p : m.prov) {
      if (p->d != d) throw Error(ST_INVALID, "latent providers must share the input dimension");
      p->pack(dx.ptr, mtest, p->test);
    }
    const int its = lmc_pathwise_correction(m, dr.ptr, S, mtest, max_cg_iter, cg_tol,
                                            correction_out);
    if (cg_iterations) *cg_iterations = its;
  });
}

}  // extern "C"
