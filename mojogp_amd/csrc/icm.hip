// ICM multi-output training loop and rotated-state prediction (reference
// files listed in icm.h).
#include "icm.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>

#include "host_numerics.h"
#include "mixed.h"
#include "tree.h"

namespace mgp {

namespace {

using Clock = std::chrono::steady_clock;

void require(bool ok, const char* msg) {
  if (!ok) throw Error(ST_INVALID, msg);
}

float sigmoidf(float x) { return 1.0f / (1.0f + std::exp(-x)); }

float max_rel_change(const std::vector<float>& prev, const std::vector<float>& cur) {
  float r = 0.0f;
  for (size_t i = 0; i < prev.size(); ++i)
    r = std::max(r, std::fabs(cur[i] - prev[i]) / (std::fabs(prev[i]) + 1e-8f));
  return r;
}

}  // namespace

std::vector<float> icm_init_w(int T, int R, int seed) {
  std::vector<float> W((size_t)T * R);
  for (int i = 0; i < T * R; ++i) {
    uint64_t state = (uint64_t)(int64_t)seed ^ ((uint64_t)i * 2654435761ull);
    state = (state * 1103515245ull + 12345ull) & 0x7FFFFFFFull;
    const float u = (float)state / (float)0x7FFFFFFF;
    W[i] = 0.1f + u * 0.4f;
  }
  return W;
}

std::vector<float> icm_task_b(const std::vector<float>& W, const std::vector<float>& raw_v, int T,
                              int R) {
  std::vector<float> B((size_t)T * T);
  for (int i = 0; i < T; ++i)
    for (int j = 0; j < T; ++j) {
      double s = 0.0;
      for (int k = 0; k < R; ++k) s += (double)W[(size_t)i * R + k] * (double)W[(size_t)j * R + k];
      if (i == j) s += (double)softplus(raw_v[i]);
      B[(size_t)i * T + j] = (float)s;
    }
  return B;
}

ICMTrainResult icm_train(Provider& base, int T, const float* y_blocked_host,
                         const std::vector<float>& init_params, const std::vector<char>& trainable,
                         const std::vector<float>& init_noise, float init_outputscale,
                         const std::vector<float>& init_mean, const std::vector<float>& fixed,
                         const ICMTrainOptions& o,
                         const std::function<void(const ProgressEvent&)>& progress) {
  const int P = base.nparams;
  require(T >= 1, "num_tasks must be >= 1");
  require((int)init_params.size() == P && (int)trainable.size() == P,
          "initial params / trainable mask length does not match the provider");
  require((int)init_noise.size() == T && (int)init_mean.size() == T, "per-task arrays mismatch");
  require(o.max_iterations >= 1, "max_iterations must be >= 1");
  require(init_outputscale > 0.0f, "initial outputscale must be > 0");
  const int R = o.task_rank < 0 ? T : o.task_rank;
  require(R >= 1 && R <= T, "task_rank must be in [1, num_tasks] or -1");
  const int64_t n = base.n, nT = n * T;
  const bool fixed_vec = !fixed.empty();
  require(!fixed_vec || (int64_t)fixed.size() == nT, "fixed noise must have T*n entries");
  for (float v : init_noise) require(std::isfinite(v) && v > 0.0f, "task noise must be > 0");

  LMCModel m;
  m.R = 1;
  m.T = T;
  m.n = n;
  m.prov.push_back(&base);
  m.st = base.st;
  if (fixed_vec) m.fixed = fixed;  // replaces the per-task noise in the operator
  hipStream_t st = m.st;

  // Raw (unconstrained) state (jit_multi_output.mojo:168-200).
  std::vector<float> raw_p(P), raw_noise(T), raw_mean(init_mean);
  for (int p = 0; p < P; ++p) raw_p[p] = inv_softplus(init_params[p]);
  float raw_os = inv_softplus(init_outputscale);
  for (int t = 0; t < T; ++t) raw_noise[t] = inv_softplus(init_noise[t]);
  std::vector<float> W = icm_init_w(T, R), raw_v(T, 0.0f);

  const int total_adam = P + 1 + T + T * R + T + T;
  std::vector<float> madam(total_adam, 0.0f), vadam(total_adam, 0.0f);
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  int t_step = 1;

  bool use_pre = o.precond_rank > 0 && !fixed_vec;
  const int prank = fixed_vec ? 0 : o.precond_rank;
  const PivotOptions po = training_pivot_options(o.precond_method);

  auto constrained = [&](const std::vector<float>& raw) {
    std::vector<float> out(raw.size());
    for (size_t i = 0; i < raw.size(); ++i) out[i] = softplus(raw[i]);
    return out;
  };
  auto set_params = [&](const std::vector<float>& p) {
    base.params = p;
    base.noise = 0.0f;
    base.refresh_coords();
  };

  // Initial Kronecker preconditioner at the initial parameters (:277-315).
  std::vector<float> cur_p = constrained(raw_p);
  float os = softplus(raw_os);
  std::vector<float> cur_noise = constrained(raw_noise);
  std::vector<float> B = icm_task_b(W, raw_v, T, R);
  set_params(cur_p);
  KronPrecond Pk;
  if (use_pre) Pk.build_kron(m, prank, po, os, B, cur_noise);
  std::vector<float> last_p = cur_p, last_noise = cur_noise, last_B = B;
  float last_os = os;

  ICMTrainResult res;
  res.task_rank = R;
  float best_nll = 1e30f, best_nll_seen = 1e30f;
  bool has_best = false;
  int patience = 0;
  std::vector<float> best_p = raw_p, best_noise = raw_noise, best_mean = raw_mean, best_B = B;
  float best_os = raw_os;
  std::vector<float> best_alpha((size_t)nT, 0.0f);

  std::vector<float> y_orig(y_blocked_host, y_blocked_host + nT), yh((size_t)nT);
  DevBuf<float> ydev;
  ydev.ensure(nT);
  LMCWork work;

  auto adam = [&](int idx, float g, float lr) {
    madam[idx] = b1 * madam[idx] + (1.0f - b1) * g;
    vadam[idx] = b2 * vadam[idx] + (1.0f - b2) * g * g;
    const float mh = madam[idx] / (1.0f - pow_float32(b1, t_step));
    const float vh = vadam[idx] / (1.0f - pow_float32(b2, t_step));
    return -lr * mh / (std::sqrt(vh) + eps);
  };
  auto rebuild_precond = [&]() {
    Pk.build_kron(m, prank, po, os, B, cur_noise);
    ++res.precond_rebuild_count;
    last_p = cur_p;
    last_os = os;
    last_noise = cur_noise;
    last_B = B;
  };
  auto emit = [&](const char* phase, int current, float nll, int cg_iter, double ms) {
    if (!progress) return;
    ProgressEvent e{};
    e.phase = phase;
    e.current = current;
    e.total = o.max_iterations;
    e.nll = nll;
    e.best_nll = best_nll_seen;
    e.cg_iter = cg_iter;
    e.iter_ms = ms;
    e.noise = T > 0 ? softplus(raw_noise[0]) : 0.0f;
    e.mean = T > 0 ? raw_mean[0] : 0.0f;
    e.precond_rank = use_pre ? (Pk.rank.empty() ? 0 : Pk.rank[0]) : 0;
    e.precond_rebuild_count = res.precond_rebuild_count;
    e.converged = res.converged;
    progress(e);
  };
  emit("start", 0, 0.0f, -1, -1.0);

  for (int it = 0; it < o.max_iterations; ++it) {
    const auto t0 = Clock::now();
    res.iterations = it + 1;
    cur_p = constrained(raw_p);
    set_params(cur_p);
    os = softplus(raw_os);
    cur_noise = constrained(raw_noise);
    B = icm_task_b(W, raw_v, T, R);
    // Operator os (B (x) K) + D (per-task noise, or the fixed vector in noise mode 1).
    m.A.resize((size_t)T * T);
    for (int i = 0; i < T * T; ++i) m.A[i] = os * B[i];
    m.noise = fixed_vec ? std::vector<float>(T, 0.0f) : cur_noise;
    m.upload();

    bool rebuild = false;
    if (it > 0) {
      float mr = max_rel_change(last_p, cur_p);
      mr = std::max(mr, std::fabs(os - last_os) / (std::fabs(last_os) + 1e-8f));
      mr = std::max(mr, max_rel_change(last_noise, cur_noise));
      mr = std::max(mr, max_rel_change(last_B, B));
      rebuild = mr > o.precond_rebuild_threshold;
    }
    if (rebuild) rebuild_precond();

    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < n; ++i)
        yh[(size_t)t * n + i] = y_orig[(size_t)t * n + i] - raw_mean[t];
    MGP_HIP_CHECK(hipMemcpyAsync(ydev.ptr, yh.data(), nT * sizeof(float), hipMemcpyHostToDevice, st));

    LMCEval ev = lmc_bbmm(m, use_pre ? &Pk : nullptr, ydev.ptr, o.num_probes, o.max_cg_iter,
                          o.max_tridiag_iter, o.cg_tol, it, it > 0 && !rebuild, work);
    bool cg_ok = ev.cg_iterations < o.max_cg_iter;
    if (!cg_ok && use_pre) {
      // Rebuild at the current parameters and retry without recycling (:430-465).
      rebuild_precond();
      ev = lmc_bbmm(m, &Pk, ydev.ptr, o.num_probes, o.max_cg_iter, o.max_tridiag_iter, o.cg_tol,
                    it, false, work);
      cg_ok = ev.cg_iterations < o.max_cg_iter;
    }
    const float nll = ev.nll;
    res.nll_history.push_back(nll);
    res.cg_iterations_history.push_back(ev.cg_iterations);
    if (!cg_ok) {
      res.iter_times_ms.push_back(
          std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
      if (!has_best) {
        best_nll_seen = nll;
        best_p = raw_p;
        best_os = raw_os;
        best_noise = raw_noise;
        best_mean = raw_mean;
        best_B = B;
        best_alpha = ev.alpha;
        has_best = true;
      }
      break;
    }
    if (nll < best_nll_seen) {
      best_nll_seen = nll;
      best_p = raw_p;
      best_os = raw_os;
      best_noise = raw_noise;
      best_mean = raw_mean;
      best_B = B;
      best_alpha = ev.alpha;
      has_best = true;
    }

    // Task-covariance gradient G_B = clip(os * dNLL/dA) (:520-560): the LMC
    // evaluation's dNLL/dA for A = os B is 0.5 (-a_s^T K a_t + tr) / nT.
    std::vector<float> GB((size_t)T * T);
    double gos = 0.0;
    for (int i = 0; i < T * T; ++i) {
      gos += (double)B[i] * (double)ev.G_A[i];
      float g = os * ev.G_A[i];
      GB[i] = g > 10.0f ? 10.0f : (g < -10.0f ? -10.0f : g);
    }
    const float lr = o.use_cosine_lr ? cosine_lr(o.learning_rate, it, o.max_iterations)
                                     : o.learning_rate;
    int ai = 0;
    for (int p = 0; p < P; ++p) {
      if (trainable[p]) {
        float g = ev.kernel_grads[p];
        if (!std::isfinite(g)) g = 0.0f;
        raw_p[p] += adam(ai, g * sigmoidf(raw_p[p]), lr);
      }
      ++ai;
    }
    {
      float g = (float)gos;
      if (!std::isfinite(g)) g = 0.0f;
      raw_os += adam(ai, g * sigmoidf(raw_os), lr);
      ++ai;
    }
    for (int t = 0; t < T; ++t) {
      if (!fixed_vec) raw_noise[t] += adam(ai, ev.noise_grads[t] * sigmoidf(raw_noise[t]), lr);
      ++ai;
    }
    // W rows updated in place in order, as the reference's loop (:626-640).
    for (int s = 0; s < T; ++s)
      for (int r = 0; r < R; ++r) {
        float gw = 0.0f;
        for (int t = 0; t < T; ++t) gw += GB[(size_t)s * T + t] * W[(size_t)t * R + r];
        W[(size_t)s * R + r] += adam(ai, 2.0f * gw, lr);
        ++ai;
      }
    for (int t = 0; t < T; ++t) {
      raw_v[t] += adam(ai, GB[(size_t)t * T + t] * sigmoidf(raw_v[t]), lr);
      ++ai;
    }
    for (int t = 0; t < T; ++t) {
      double acc = 0.0;
      for (int64_t i = 0; i < n; ++i) acc -= ev.alpha[(size_t)t * n + i];
      const float g = clip_gradient((float)acc / (float)nT);
      raw_mean[t] += adam(ai, g, lr);
      ++ai;
    }
    ++t_step;
    const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
    res.iter_times_ms.push_back(ms);
    const int every = std::max(o.progress_interval, 1);
    if ((it + 1) % every == 0 || it + 1 == o.max_iterations)
      emit("iteration", it + 1, nll, ev.cg_iterations, ms);
    if (o.early_stop_tol > 0.0f) {
      if (nll < best_nll - o.early_stop_tol) {
        best_nll = nll;
        patience = 0;
      } else if (++patience >= o.early_stop_patience) {
        res.converged = true;
        emit("early_stop", it + 1, nll, ev.cg_iterations, ms);
        break;
      }
    }
  }

  res.params = constrained(best_p);
  res.outputscale = softplus(best_os);
  res.noise = constrained(best_noise);
  res.mean = best_mean;
  res.B = best_B;
  res.alpha = best_alpha;
  res.final_nll = best_nll_seen;
  emit("complete", res.iterations, best_nll_seen, -1, -1.0);
  // Leave the provider at the returned parameters.
  set_params(res.params);
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return res;
}

// ------------------------------------------------------------------ mixed categorical
namespace {
// P = L L^T + noise I over the full n T system with the single-output
// Woodbury and probe streams (L z_rank with z_rank from seed, plus
// sqrt(noise) z_noise from seed + 1000000).
struct FullPivotPrecond : LMCPrecond {
  Precond P;
  DevBuf<float> zr, zn;
  int64_t N = 0;
  void apply(const float* r, int C, float* z, double* rz_part, int nb,
             hipStream_t st) override {
    woodbury_apply(P.L.ptr, N, P.rank, P.Minv.ptr, P.noise, r, C, z, P.work,
                   rz_part ? r : nullptr, nb, rz_part, st);
  }
  void sample(float* out, int C, uint64_t seed, hipStream_t st) override {
    float* a = zr.ensure((size_t)P.rank * C);
    float* b = zn.ensure((size_t)N * C);
    gaussian(a, (int64_t)P.rank * C, seed, st);
    gaussian(b, N * C, seed + 1000000ull, st);
    low_rank_sample(P.L.ptr, N, P.rank, a, b, std::sqrt(P.noise), C, out, st);
  }
};

__global__ void k_copy_cols(float* __restrict__ dst, const float* __restrict__ src,
                            int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) dst[i] = src[i];
}

// out[c][t][i] = sum_j M[t][j] in[c][j][i]
__global__ void k_mix_tasks(float* __restrict__ out, const float* __restrict__ in,
                            const float* __restrict__ M, int64_t n, int T, int C) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nT = n * T;
  if (idx >= nT * C) return;
  const int64_t c = idx / nT, rem = idx - c * nT;
  const int t = (int)(rem / n);
  const int64_t i = rem - (int64_t)t * n;
  const float* col = in + c * nT + i;
  float s = 0.0f;
  for (int j = 0; j < T; ++j) s = fmaf(M[t * T + j], col[(int64_t)j * n], s);
  out[idx] = s;
}
}  // namespace

ICMMixedResult icm_train_mixed(Provider& base, int T, const float* y_blocked_host,
                               const std::vector<float>& init_params,
                               const std::vector<float>& init_noise, float init_outputscale,
                               const std::vector<float>& init_mean,
                               const std::vector<int>& cat_kinds,
                               const std::vector<float>& init_cat_raw,
                               const ICMTrainOptions& o,
                               const std::function<void(const ProgressEvent&)>& progress) {
  const int P = base.nparams;
  require(T >= 1, "num_tasks must be >= 1");
  require((int)init_params.size() == P, "initial params length does not match the provider");
  require((int)init_noise.size() == T && (int)init_mean.size() == T, "per-task arrays mismatch");
  require(o.max_iterations >= 1, "max_iterations must be >= 1");
  require(o.num_probes >= 0, "num_probes must be >= 0");
  require(init_outputscale > 0.0f, "initial outputscale must be > 0");
  const int R = o.task_rank < 0 ? T : o.task_rank;
  require(R >= 1 && R <= T, "task_rank must be in [1, num_tasks] or -1");
  require(base.is_tree && base.tree.ncat > 0, "mixed training needs categorical tree leaves");
  for (float v : init_noise) require(std::isfinite(v) && v > 0.0f, "task noise must be > 0");
  const std::vector<CatLeafRef> cl = cat_leaves(base, cat_kinds);
  int KC = 0;
  for (const auto& c : cl) KC += c.nparam;
  require((int)init_cat_raw.size() == KC, "categorical parameter count does not match the leaves");
  for (float v : init_cat_raw) require(std::isfinite(v), "categorical parameters must be finite");
  const int64_t n = base.n, nT = n * T;

  LMCModel m;
  m.R = 1;
  m.T = T;
  m.n = n;
  m.prov.push_back(&base);
  m.st = base.st;
  hipStream_t st = m.st;

  // Raw state (jit_multi_output_mixed.mojo:517-575).
  std::vector<float> raw_p(P), raw_noise(T), raw_mean(init_mean), rcat(init_cat_raw);
  for (int p = 0; p < P; ++p) raw_p[p] = inv_softplus(init_params[p]);
  float raw_os = inv_softplus(init_outputscale);
  for (int t = 0; t < T; ++t) raw_noise[t] = inv_softplus(init_noise[t]);
  std::vector<float> W = icm_init_w(T, R), raw_v(T, 0.0f);
  const int total_adam = P + 1 + T + T * R + T + T;
  std::vector<float> madam(total_adam, 0.0f), vadam(total_adam, 0.0f);
  std::vector<float> mcat((size_t)KC, 0.0f), vcat((size_t)KC, 0.0f);
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  int t_step = 1;

  auto constrained = [&](const std::vector<float>& raw) {
    std::vector<float> out(raw.size());
    for (size_t i = 0; i < raw.size(); ++i) out[i] = softplus(raw[i]);
    return out;
  };
  auto constrained_cat = [&]() {
    std::vector<float> out;
    std::vector<double> th;
    for (const auto& c : cl) {
      th.resize((size_t)c.nparam);
      cat_constrain(c.kind, c.L, rcat.data() + c.param_off, c.nparam, th.data(), nullptr);
      for (double v : th) out.push_back((float)v);
    }
    return out;
  };
  auto set_state = [&](const std::vector<float>& p, float os, const std::vector<float>& B,
                       const std::vector<float>& noise) {
    base.params = p;
    base.noise = 0.0f;
    set_categorical_raw(base, cat_kinds, rcat.data(), KC);  // tables + refresh
    m.A.resize((size_t)T * T);
    for (int i = 0; i < T * T; ++i) m.A[i] = os * B[i];
    m.noise = noise;
    m.upload();
  };

  const bool use_pre = o.precond_rank > 0;
  const PivotOptions po = training_pivot_options(o.precond_method);
  FullPivotPrecond FP;
  FP.R = 1;
  FP.T = T;
  FP.n = n;
  FP.N = nT;
  auto build = [&]() {
    const float nmin = *std::min_element(m.noise.begin(), m.noise.end());
    const int rank = (int)std::min<int64_t>(o.precond_rank, nT);
    MGP_REQUIRE(rank <= 1000, "preconditioner rank must be <= 1000");
    FP.P.noise = nmin;
    const int k = pivoted_cholesky_kron(base, T, m.A_dev.ptr, m.A, m.noise_dev.ptr, nmin, rank,
                                        po, FP.P.L.ensure((size_t)rank * nT), st);
    precond_from_factor(FP.P, nT, k, st);
    FP.K = k;
    FP.logdet = FP.P.logdet;
  };

  // Initial preconditioner: the given kernel parameters, round-tripped
  // outputscale and noise (:566-611).
  float os = softplus(raw_os);
  std::vector<float> cur_noise = constrained(raw_noise);
  std::vector<float> B = icm_task_b(W, raw_v, T, R);
  set_state(init_params, os, B, cur_noise);
  if (use_pre) build();
  std::vector<float> last_p = init_params, last_cat = constrained_cat(), last_noise = cur_noise,
                     last_B = B;
  float last_os = os;

  ICMMixedResult res;
  res.task_rank = R;
  float best_nll = 1e30f, best_seen = 1e30f;
  int patience = 0;
  std::vector<float> best_p = raw_p, best_noise = raw_noise, best_mean = raw_mean,
                     best_cat = rcat, best_B = B;
  float best_os = raw_os;
  std::vector<float> best_alpha((size_t)nT, 0.0f);

  std::vector<float> y_orig(y_blocked_host, y_blocked_host + nT), yh((size_t)nT);
  DevBuf<float> ydev, rfc, rfm;
  ydev.ensure(nT);
  LMCWork work;
  std::vector<double> G((size_t)base.tree.table_size);
  const float no_clip = std::numeric_limits<float>::infinity();

  auto adam = [&](float* mm, float* vv, int idx, float g, float lr) {
    mm[idx] = b1 * mm[idx] + (1.0f - b1) * g;
    vv[idx] = b2 * vv[idx] + (1.0f - b2) * g * g;
    const float mh = mm[idx] / (1.0f - pow_float32(b1, t_step));
    const float vh = vv[idx] / (1.0f - pow_float32(b2, t_step));
    return -lr * mh / (std::sqrt(vh) + eps);
  };
  auto emit = [&](const char* phase, int current, float nll, int cg_iter, double ms) {
    if (!progress) return;
    ProgressEvent e{};
    e.phase = phase;
    e.current = current;
    e.total = o.max_iterations;
    e.nll = nll;
    e.best_nll = best_seen;
    e.cg_iter = cg_iter;
    e.iter_ms = ms;
    e.noise = softplus(raw_noise[0]);
    e.mean = raw_mean[0];
    e.precond_rank = use_pre ? FP.K : 0;
    e.precond_rebuild_count = res.precond_rebuild_count;
    e.converged = res.converged;
    progress(e);
  };
  emit("start", 0, 0.0f, -1, -1.0);

  for (int it = 0; it < o.max_iterations; ++it) {
    const auto t0 = Clock::now();
    res.iterations = it + 1;
    const std::vector<float> cur_p = constrained(raw_p);
    const std::vector<float> cur_cat = constrained_cat();
    os = softplus(raw_os);
    cur_noise = constrained(raw_noise);
    B = icm_task_b(W, raw_v, T, R);
    set_state(cur_p, os, B, cur_noise);

    bool rebuild = false;
    if (it > 0) {
      float mr = max_rel_change(last_p, cur_p);
      mr = std::max(mr, max_rel_change(last_cat, cur_cat));
      mr = std::max(mr, std::fabs(os - last_os) / (std::fabs(last_os) + 1e-8f));
      mr = std::max(mr, max_rel_change(last_noise, cur_noise));
      mr = std::max(mr, max_rel_change(last_B, B));
      rebuild = mr > o.precond_rebuild_threshold;
    }
    if (rebuild) {
      if (use_pre) build();
      ++res.precond_rebuild_count;
      last_p = cur_p;
      last_cat = cur_cat;
      last_os = os;
      last_noise = cur_noise;
      last_B = B;
    }

    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < n; ++i)
        yh[(size_t)t * n + i] = y_orig[(size_t)t * n + i] - raw_mean[t];
    MGP_HIP_CHECK(hipMemcpyAsync(ydev.ptr, yh.data(), nT * sizeof(float), hipMemcpyHostToDevice, st));
    LMCEval ev = lmc_bbmm(m, use_pre ? &FP : nullptr, ydev.ptr, o.num_probes, o.max_cg_iter,
                          o.max_tridiag_iter, o.cg_tol, it, it > 0 && !rebuild, work);
    const float nll = ev.nll;
    res.nll_history.push_back(nll);
    res.cg_iterations_history.push_back(ev.cg_iterations);
    if (nll < best_seen) {
      best_seen = nll;
      best_p = raw_p;
      best_os = raw_os;
      best_noise = raw_noise;
      best_mean = raw_mean;
      best_cat = rcat;
      best_B = B;
      best_alpha = ev.alpha;
    }
    // G_B = clip(os dNLL/dA) for A = os B; dNLL/d(os) = sum B o dNLL/dA
    // (jit_multi_output_mixed.mojo:815-860).
    std::vector<float> GB((size_t)T * T);
    double gos = 0.0;
    for (int i = 0; i < T * T; ++i) {
      gos += (double)B[i] * (double)ev.G_A[i];
      const float g = os * ev.G_A[i];
      GB[i] = g > 10.0f ? 10.0f : (g < -10.0f ? -10.0f : g);
    }
    const float lr = o.use_cosine_lr ? cosine_lr(o.learning_rate, it, o.max_iterations)
                                     : o.learning_rate;
    // Categorical gradients (:887-960): the evaluation's left factors with
    // Rf = [alpha | unit probes] mixed by os B, one tree pass for every entry.
    {
      const int C = 1 + o.num_probes;
      float* rf = rfc.ensure((size_t)nT * C);
      hipLaunchKernelGGL(k_copy_cols, dim3((unsigned)ceil_div(nT, 256)), dim3(256), 0, st, rf,
                         work.sol.ptr, nT);
      if (o.num_probes > 0)
        hipLaunchKernelGGL(k_copy_cols, dim3((unsigned)ceil_div(nT * o.num_probes, 256)),
                           dim3(256), 0, st, rf + nT, work.probes.ptr, nT * o.num_probes);
      float* rm = rfm.ensure((size_t)nT * C);
      hipLaunchKernelGGL(k_mix_tasks, dim3((unsigned)ceil_div(nT * C, 256)), dim3(256), 0, st,
                         rm, rf, m.A_dev.ptr, n, T, C);
      MGP_HIP_CHECK(hipGetLastError());
      tree_cat_grad_tables(base.tree, base.tparams.ptr, base.train.z.ptr, n, work.lf.ptr, rm,
                           C * T, G.data(), base.tree_gws, st);
      std::vector<float> gc((size_t)KC);
      cat_raw_gradients(cl, rcat.data(), G, 1.0, no_clip, gc.data());
      for (int k = 0; k < KC; ++k) rcat[(size_t)k] += adam(mcat.data(), vcat.data(), k, gc[(size_t)k], lr);
    }
    int ai = 0;
    for (int p = 0; p < P; ++p, ++ai)
      raw_p[p] += adam(madam.data(), vadam.data(), ai, ev.kernel_grads[p] * sigmoidf(raw_p[p]), lr);
    {
      float g = (float)gos;
      if (!std::isfinite(g)) g = 0.0f;
      raw_os += adam(madam.data(), vadam.data(), ai, g * sigmoidf(raw_os), lr);
      ++ai;
    }
    for (int t = 0; t < T; ++t, ++ai)
      raw_noise[t] += adam(madam.data(), vadam.data(), ai, ev.noise_grads[t] * sigmoidf(raw_noise[t]), lr);
    for (int s = 0; s < T; ++s)
      for (int r = 0; r < R; ++r, ++ai) {
        float gw = 0.0f;
        for (int t = 0; t < T; ++t) gw += GB[(size_t)s * T + t] * W[(size_t)t * R + r];
        W[(size_t)s * R + r] += adam(madam.data(), vadam.data(), ai, 2.0f * gw, lr);
      }
    for (int t = 0; t < T; ++t, ++ai)
      raw_v[t] += adam(madam.data(), vadam.data(), ai, GB[(size_t)t * T + t] * sigmoidf(raw_v[t]), lr);
    for (int t = 0; t < T; ++t, ++ai) {
      float g = 0.0f;
      for (int64_t i = 0; i < n; ++i) g -= ev.alpha[(size_t)t * n + i];
      raw_mean[t] += adam(madam.data(), vadam.data(), ai, clip_gradient(g / (float)nT), lr);
    }
    ++t_step;
    const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
    res.iter_times_ms.push_back(ms);
    const int every = std::max(o.progress_interval, 1);
    if ((it + 1) % every == 0 || it + 1 == o.max_iterations)
      emit("iteration", it + 1, nll, ev.cg_iterations, ms);
    if (o.early_stop_tol > 0.0f) {
      if (nll < best_nll - o.early_stop_tol) {
        best_nll = nll;
        patience = 0;
      } else if (++patience >= o.early_stop_patience) {
        res.converged = true;
        emit("early_stop", it + 1, nll, ev.cg_iterations, ms);
        break;
      }
    }
  }

  res.params = constrained(best_p);
  res.outputscale = softplus(best_os);
  res.noise = constrained(best_noise);
  res.mean = best_mean;
  res.B = best_B;
  res.alpha = best_alpha;
  res.cat_raw = best_cat;
  res.final_nll = best_seen;
  emit("complete", res.iterations, best_seen, -1, -1.0);
  // Leave the provider at the returned state (noise 0, best tables).
  rcat = best_cat;
  base.params = res.params;
  base.noise = 0.0f;
  set_categorical_raw(base, cat_kinds, rcat.data(), KC);
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return res;
}

void icm_predict(Provider& pv, int T, const float* alpha_rot, const float* Q,
                 const float* scales, const float* Xs_host, int64_t m, float noise,
                 int variance_method, int max_cg_iter, float cg_tol, int precond_rank,
                 int lanczos_rank, float* mean_out, float* var_out) {
  require(T >= 1 && m >= 1, "need >= 1 task and test point");
  require(variance_method >= 0 && variance_method <= 2, "variance_method must be 0, 1 or 2");
  require(variance_method == 0 || var_out, "variance needs an output array");
  require(variance_method != 1 || lanczos_rank >= 1, "lanczos_rank must be >= 1 for LOVE");
  const int64_t n = pv.n;
  hipStream_t st = pv.st;
  DevBuf<float> dx, da, cr;
  dx.ensure((size_t)m * pv.d);
  da.ensure((size_t)n * T);
  cr.ensure((size_t)m * T);
  MGP_HIP_CHECK(hipMemcpyAsync(dx.ptr, Xs_host, (size_t)m * pv.d * sizeof(float),
                               hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipMemcpyAsync(da.ptr, alpha_rot, (size_t)n * T * sizeof(float),
                               hipMemcpyHostToDevice, st));
  pv.pack(dx.ptr, m, pv.test);
  // All T eigen-task cross products in one launch: cr[s][i] = (K(X*, X) alpha_rot[s])[i].
  pv.cross(pv.test, da.ptr, T, cr.ptr);
  std::vector<float> hc((size_t)m * T);
  MGP_HIP_CHECK(hipMemcpyAsync(hc.data(), cr.ptr, hc.size() * sizeof(float),
                               hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  std::memset(mean_out, 0, (size_t)m * T * sizeof(float));
  for (int s = 0; s < T; ++s)
    for (int t = 0; t < T; ++t) {
      const float w = Q[(size_t)t * T + s] * scales[s];
      for (int64_t i = 0; i < m; ++i) mean_out[(size_t)i * T + t] += w * hc[(size_t)s * m + i];
    }
  if (variance_method == 0) return;
  std::memset(var_out, 0, (size_t)m * T * sizeof(float));
  DevBuf<float> vs;
  vs.ensure((size_t)m);
  std::vector<float> hv((size_t)m);
  const float saved = pv.noise;
  for (int s = 0; s < T; ++s) {
    if (!(scales[s] > 1e-8f)) continue;
    pv.noise = noise / scales[s];
    try {
      if (variance_method == 1) {
        PredictState ps;
        lanczos_inv_root(pv, lanczos_rank, ps);
        DevBuf<float> V;
        V.ensure((size_t)ps.rank * m);
        pv.cross(pv.test, ps.root.ptr, ps.rank, V.ptr);
        love_variance(V.ptr, m, ps.rank, pv.kdiag(), vs.ptr, st);
      } else {
        ExactVarianceOptions eo;
        eo.max_cg_iter = max_cg_iter;
        eo.cg_tol = cg_tol;
        eo.precond_rank = precond_rank;
        ExactVarianceStats es;
        exact_variance(pv, m, eo, vs.ptr, es);
      }
    } catch (...) {
      pv.noise = saved;
      throw;
    }
    MGP_HIP_CHECK(hipMemcpyAsync(hv.data(), vs.ptr, m * sizeof(float), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    for (int t = 0; t < T; ++t) {
      const float q = Q[(size_t)t * T + s];
      const float w = q * q * scales[s];
      for (int64_t i = 0; i < m; ++i) var_out[(size_t)i * T + t] += w * hv[(size_t)i];
    }
  }
  pv.noise = saved;
}

}  // namespace mgp
