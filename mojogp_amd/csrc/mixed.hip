// Mixed continuous x categorical training: categorical correlation tables
// (host, fp64) and the split-Adam training loop over a kernel tree whose
// categorical leaves look up those tables.
//
// Reference: kernels/categorical_kernel.mojo (GD, CR, EHH, HH, FE tables),
// kernels/jit/jit_categorical_params.mojo (raw -> constrained transforms),
// kernels/jit/jit_mixed.mojo:428-909 (train_mixed_jit).
#include "mixed.h"

#include <algorithm>
#include <chrono>
#include <cmath>

#include "host_numerics.h"
#include "solver.h"

namespace mgp {

namespace {
constexpr double kHalfLogEps = -13.815510558;  // log(1e-12) / 2
constexpr double kPiD = 3.14159265358979323846;

bool is_angle(int kind, int L, int k) {
  return kind == CAT_EHH || kind == CAT_HH || (kind == CAT_FE && k < L * (L - 1) / 2);
}

double sigm(double x) { return 1.0 / (1.0 + std::exp(-x)); }

// Hypersphere factor row k of C and its derivative with respect to angle
// (k, j): C[k][c] = cos(t_c) prod_{m<c} sin(t_m) (c < k), C[k][k] = prod sin.
void hyper_factor(const double* ang, int L, std::vector<double>& C) {
  C.assign((size_t)L * L, 0.0);
  C[0] = 1.0;
  int idx = 0;
  for (int k = 1; k < L; ++k) {
    double s = 1.0;
    for (int c = 0; c < k; ++c) {
      const double t = ang[idx++];
      C[(size_t)k * L + c] = std::cos(t) * s;
      s *= std::sin(t);
    }
    C[(size_t)k * L + k] = s;
  }
}

// dC[k][c] / d t_{k, j} for c = 0..k (row k only).
void hyper_row_derivative(const double* ang, int L, int k, int j, std::vector<double>& dr) {
  dr.assign((size_t)L, 0.0);
  const double* t = ang + k * (k - 1) / 2;
  for (int c = j; c <= k; ++c) {
    double v = (c < k) ? (c == j ? -std::sin(t[c]) : std::cos(t[c])) : 1.0;
    for (int m = 0; m < c; ++m) v *= (m == j) ? std::cos(t[m]) : std::sin(t[m]);
    dr[(size_t)c] = v;
  }
}
}  // namespace

int cat_num_params(int kind, int L) {
  switch (kind) {
    case CAT_GD: return 1;
    case CAT_CR: return L;
    case CAT_EHH:
    case CAT_HH: return L * (L - 1) / 2;
    case CAT_FE: return L * (L + 1) / 2;
    default: throw Error(ST_INVALID, "categorical kind must be 0 (GD) .. 4 (FE)");
  }
}

void cat_constrain(int kind, int L, const float* raw, int K, double* theta, double* chain) {
  for (int k = 0; k < K; ++k) {
    const float r = raw[k];
    if (is_angle(kind, L, k)) {
      const double s = sigm((double)r);
      theta[k] = s * kPiD;
      if (chain) chain[k] = s * (1.0 - s) * kPiD;
    } else {
      theta[k] = (double)softplus(r);
      if (chain) chain[k] = (double)softplus_derivative(r);
    }
  }
}

void cat_correlation(int kind, int L, const double* th, double* R,
                     std::vector<double>* dR) {
  const int K = cat_num_params(kind, L);
  const size_t LL = (size_t)L * L;
  for (size_t e = 0; e < LL; ++e) R[e] = 0.0;
  if (dR) dR->assign((size_t)K * LL, 0.0);
  auto at = [L](int a, int b) { return (size_t)a * L + b; };
  if (kind == CAT_GD || kind == CAT_CR) {
    for (int a = 0; a < L; ++a)
      for (int b = 0; b < L; ++b) {
        if (a == b) {
          R[at(a, b)] = 1.0;
          continue;
        }
        const double x = kind == CAT_GD ? th[0] : th[a] + th[b];
        const double r = std::exp(-x);
        R[at(a, b)] = r;
        if (!dR) continue;
        if (kind == CAT_GD) {
          (*dR)[at(a, b)] = -r;
        } else {
          (*dR)[(size_t)a * LL + at(a, b)] += -r;
          (*dR)[(size_t)b * LL + at(a, b)] += -r;
        }
      }
    return;
  }
  const int na = L * (L - 1) / 2;
  std::vector<double> C, D(LL, 0.0);
  hyper_factor(th, L, C);
  for (int a = 0; a < L; ++a)
    for (int b = 0; b < L; ++b) {
      double s = 0.0;
      for (int c = 0; c <= std::min(a, b); ++c) s += C[at(a, c)] * C[at(b, c)];
      D[at(a, b)] = s;
    }
  const double* dg = th + na;  // FE diagonal parameters
  for (int a = 0; a < L; ++a)
    for (int b = 0; b < L; ++b) {
      if (kind == CAT_HH) R[at(a, b)] = D[at(a, b)];
      else if (a == b) R[at(a, b)] = 1.0;
      else if (kind == CAT_EHH) R[at(a, b)] = std::exp(kHalfLogEps * (1.0 - D[at(a, b)]));
      else R[at(a, b)] = std::exp(-(dg[a] + dg[b] + kHalfLogEps * (D[at(a, b)] - 1.0)));
    }
  if (!dR) return;
  std::vector<double> dr;
  int idx = 0;
  for (int k = 1; k < L; ++k)
    for (int j = 0; j < k; ++j, ++idx) {
      hyper_row_derivative(th, L, k, j, dr);
      double* out = dR->data() + (size_t)idx * LL;
      for (int b = 0; b < L; ++b) {
        double s = 0.0;  // dD[k][b] = sum_c dC[k][c] C[b][c]
        for (int c = 0; c <= std::min(k, b); ++c) s += dr[(size_t)c] * C[at(b, c)];
        if (b == k) s *= 2.0;
        for (int pass = 0; pass < (b == k ? 1 : 2); ++pass) {
          const int a0 = pass == 0 ? k : b, b0 = pass == 0 ? b : k;
          if (kind == CAT_HH) out[at(a0, b0)] = s;
          else if (a0 != b0) out[at(a0, b0)] = -kHalfLogEps * R[at(a0, b0)] * s;
        }
      }
    }
  if (kind == CAT_FE)
    for (int k = 0; k < L; ++k) {
      double* out = dR->data() + (size_t)(na + k) * LL;
      for (int a = 0; a < L; ++a)
        for (int b = 0; b < L; ++b)
          if (a != b) out[at(a, b)] = -R[at(a, b)] * ((a == k ? 1.0 : 0.0) + (b == k ? 1.0 : 0.0));
    }
}

std::vector<CatLeafRef> cat_leaves(const Provider& pv, const std::vector<int>& kinds) {
  std::vector<CatLeafRef> out;
  int po = 0, i = 0;
  for (int l = 0; l < pv.tree.nleaves; ++l) {
    const TreeLeaf& lf = pv.tree.leaf[l];
    if (lf.kind != KIND_CAT) continue;
    MGP_REQUIRE(i < (int)kinds.size(), "one categorical kind per categorical leaf");
    const int K = cat_num_params(kinds[(size_t)i], lf.ard);
    out.push_back({kinds[(size_t)i], lf.ard, lf.p0, po, K});
    po += K;
    ++i;
  }
  MGP_REQUIRE(i == (int)kinds.size(), "one categorical kind per categorical leaf");
  return out;
}

void cat_raw_gradients(const std::vector<CatLeafRef>& cl, const float* rcat,
                       const std::vector<double>& G, double scale, float clipv, float* out) {
  std::vector<double> th, chain, R, dR;
  for (const CatLeafRef& c : cl) {
    th.resize((size_t)c.nparam);
    chain.resize((size_t)c.nparam);
    R.resize((size_t)c.L * c.L);
    cat_constrain(c.kind, c.L, rcat + c.param_off, c.nparam, th.data(), chain.data());
    cat_correlation(c.kind, c.L, th.data(), R.data(), &dR);
    const size_t LL = (size_t)c.L * c.L;
    for (int k = 0; k < c.nparam; ++k) {
      double s = 0.0;
      for (size_t e = 0; e < LL; ++e) s += dR[(size_t)k * LL + e] * G[(size_t)c.table_off + e];
      float g = (float)(s * scale);
      g = g > clipv ? clipv : (g < -clipv ? -clipv : g);
      out[c.param_off + k] = g * (float)chain[(size_t)k];
    }
  }
}

namespace {
void write_tables(Provider& pv, const std::vector<CatLeafRef>& cl, const std::vector<float>& raw) {
  std::vector<double> th, R;
  for (const CatLeafRef& c : cl) {
    th.resize((size_t)c.nparam);
    R.resize((size_t)c.L * c.L);
    cat_constrain(c.kind, c.L, raw.data() + c.param_off, c.nparam, th.data(), nullptr);
    cat_correlation(c.kind, c.L, th.data(), R.data(), nullptr);
    for (size_t e = 0; e < R.size(); ++e) pv.cat_tables[(size_t)c.table_off + e] = (float)R[e];
  }
}

// sum_i x_i (fp64 partials in a fixed order).
float sum_f(const float* x, const float* ones, int64_t n, DevBuf<double>& part, hipStream_t st) {
  const int nb = reduction_chunks(n);
  double* pp = part.ensure((size_t)nb + 1);
  coldot_partial(x, ones, n, 1, nb, pp, st);
  coldot_finalize(pp, nb, 1, pp + nb, st);
  double h = 0.0;
  MGP_HIP_CHECK(hipMemcpyAsync(&h, pp + nb, sizeof(double), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return (float)h;
}

__global__ void k_copy_f(float* __restrict__ dst, const float* __restrict__ src, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}
}  // namespace

void set_categorical_raw(Provider& pv, const std::vector<int>& kinds, const float* raw,
                         int nraw) {
  MGP_REQUIRE(pv.is_tree, "categorical parameters need a kernel-tree provider");
  const auto cl = cat_leaves(pv, kinds);
  int total = 0;
  for (const auto& c : cl) total += c.nparam;
  MGP_REQUIRE(nraw == total, "expected " + std::to_string(total) + " categorical parameters");
  write_tables(pv, cl, std::vector<float>(raw, raw + nraw));
  pv.refresh_coords();
}

MixedTrainResult train_mixed(Provider& pv, const float* y_host,
                             const std::vector<float>& init_params, float init_noise,
                             const std::vector<int>& cat_kinds,
                             const std::vector<float>& init_cat_raw, const TrainOptions& o,
                             const std::function<void(const ProgressEvent&)>& progress) {
  MGP_REQUIRE(pv.is_tree && pv.tree.ncat > 0, "mixed training needs categorical tree leaves");
  const int64_t n = pv.n;
  const int P = pv.nparams;
  hipStream_t st = pv.st;
  MGP_REQUIRE((int)init_params.size() == P, "initial params size mismatch");
  MGP_REQUIRE(o.max_iterations >= 1, "max_iterations must be >= 1");
  const auto cl = cat_leaves(pv, cat_kinds);
  int KC = 0;
  for (const auto& c : cl) KC += c.nparam;
  MGP_REQUIRE((int)init_cat_raw.size() == KC, "initial categorical parameter count mismatch");

  DevBuf<float> y, yc, rfc;
  y.ensure(n);
  yc.ensure(n);
  MGP_HIP_CHECK(hipMemcpyAsync(y.ptr, y_host, n * sizeof(float), hipMemcpyHostToDevice, st));

  std::vector<float> raw(P + 1), rcat(init_cat_raw);
  for (int q = 0; q < P; ++q) raw[q] = inv_softplus(init_params[q]);
  raw[P] = inv_softplus(init_noise);
  float raw_mean = o.init_mean;
  std::vector<float> m_(P + 1, 0.f), v_(P + 1, 0.f), mc(KC, 0.f), vc(KC, 0.f);
  float m_mean = 0.f, v_mean = 0.f;
  int adam_t = 0, cat_t = 0;
  std::vector<float> best_raw(raw), best_cat(rcat);
  float best_raw_mean = raw_mean, best_nll_seen = 1e30f, best_nll = 1e30f;
  int no_improve = 0;
  float lr = o.learning_rate;
  std::vector<float> last_rebuild(init_params);
  float last_rebuild_noise = init_noise;

  MixedTrainResult res;
  Precond Pc;
  BBMMWork work;
  const int precond_rank = o.use_preconditioner ? o.precond_rank : 0;
  std::vector<float> params(init_params);
  pv.params = params;
  write_tables(pv, cl, rcat);
  pv.refresh_coords();
  pv.noise = init_noise;
  auto rebuild = [&]() {
    build_precond(pv, precond_rank, training_pivot_options(o.precond_method), Pc);
    res.base.precond_build_count += 1;
  };
  rebuild();
  auto emit = [&](const char* phase, int cur, float nll, float bnll, int cgi, double ms,
                  float noise, float mean, bool conv) {
    if (!progress) return;
    ProgressEvent e{phase, cur, o.max_iterations, nll, bnll, cgi, ms, noise, mean, Pc.rank, 0,
                    conv};
    progress(e);
  };
  emit("start", 0, 0.f, 0.f, -1, -1.0, -1.f, 0.f, false);

  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  std::vector<double> G((size_t)pv.tree.table_size), th, chain, R;
  std::vector<double> dR;
  int actual = 0;
  for (int it = 0; it < o.max_iterations; ++it) {
    const auto t_iter = std::chrono::steady_clock::now();
    actual = it + 1;
    for (int q = 0; q < P; ++q) params[q] = softplus(raw[q]);
    const float noise = softplus(raw[P]);
    pv.params = params;
    write_tables(pv, cl, rcat);
    pv.refresh_coords();
    pv.noise = noise;
    if (it > 0) {
      float max_rel = 0.f;
      for (int q = 0; q < P; ++q)
        max_rel = std::max(max_rel, std::fabs(params[q] - last_rebuild[q]) /
                                        std::max(std::fabs(last_rebuild[q]), 1e-8f));
      max_rel = std::max(max_rel, std::fabs(noise - last_rebuild_noise) /
                                      std::max(std::fabs(last_rebuild_noise), 1e-8f));
      if (max_rel > o.precond_rebuild_threshold) {
        rebuild();
        last_rebuild = params;
        last_rebuild_noise = noise;
      }
    }
    sub_scalar(yc.ptr, y.ptr, raw_mean, n, st);
    BBMMResult r = bbmm_step(pv, Pc, o.use_preconditioner, yc.ptr, o.num_probes, o.max_cg_iter,
                             o.max_tridiag_iter, o.cg_tol, it, it > 0, work);
    const float nll = r.nll;
    res.base.cg_iterations_history.push_back(r.cg_iterations);
    if (nll != nll) {  // jit_mixed.mojo:651-673: halve the rate, skip the step
      lr *= 0.5f;
      emit("nan", actual, nll, best_nll_seen, r.cg_iterations, -1.0, noise, raw_mean, false);
      continue;
    }
    if (nll < best_nll_seen) {
      best_nll_seen = nll;
      best_raw = raw;
      best_cat = rcat;
      best_raw_mean = raw_mean;
    }
    const float lr_eff = o.use_cosine_lr ? cosine_lr(o.learning_rate, it, o.max_iterations) : lr;
    // continuous parameters and noise
    for (int q = 0; q <= P; ++q) {
      const float gr = clip_gradient(r.grads[q]) * softplus_derivative(raw[q]);
      m_[q] = b1 * m_[q] + (1.0f - b1) * gr;
      v_[q] = b2 * v_[q] + (1.0f - b2) * gr * gr;
    }
    adam_t += 1;
    {
      const float bc1 = 1.0f - pow_float32(b1, adam_t), bc2 = 1.0f - pow_float32(b2, adam_t);
      for (int q = 0; q <= P; ++q) {
        const float nr = raw[q] - lr_eff * (m_[q] / bc1) / (std::sqrt(v_[q] / bc2) + eps);
        raw[q] = std::max(-20.0f, std::min(20.0f, nr));
      }
    }
    // constant mean
    {
      DevBuf<float> ones;
      ones.ensure(n);
      fill(ones.ptr, n, 1.0f, st);
      const float s = sum_f(r.alpha_dev, ones.ptr, n, work.part, st);
      const float mg = clip_gradient(-s / (float)n);
      m_mean = b1 * m_mean + (1.0f - b1) * mg;
      v_mean = b2 * v_mean + (1.0f - b2) * mg * mg;
      const float mh = m_mean / (1.0f - pow_float32(b1, adam_t));
      const float vh = v_mean / (1.0f - pow_float32(b2, adam_t));
      raw_mean -= lr_eff * mh / (std::sqrt(vh) + eps);
      if (raw_mean != raw_mean || raw_mean > 1000.0f || raw_mean < -1000.0f) raw_mean = o.init_mean;
    }
    // categorical parameters (jit_mixed.mojo:720-797): dNLL/dtheta_k =
    // -0.5 alpha^T dK_k alpha + (0.5/S) sum_s (K^-1 z_s)^T dK_k zn_s with the
    // unit-norm probes zn_s, not divided by n; one tree pass gives the
    // per-entry sums G, then sum_e dR_k[e] G[e].
    {
      const int C = 1 + o.num_probes;
      float* rf = rfc.ensure((size_t)C * n);
      hipLaunchKernelGGL(k_copy_f, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, rf,
                         r.alpha_dev, n);
      if (o.num_probes > 0)
        hipLaunchKernelGGL(k_copy_f, dim3((unsigned)ceil_div((int64_t)o.num_probes * n, 256)),
                           dim3(256), 0, st, rf + n, work.probes.ptr, (int64_t)o.num_probes * n);
      MGP_HIP_CHECK(hipGetLastError());
      tree_cat_grad_tables(pv.tree, pv.tparams.ptr, pv.train.z.ptr, n, work.lf.ptr, rf, C,
                           G.data(), pv.tree_gws, st);
      std::vector<float> gc((size_t)KC), chain_f((size_t)KC);
      for (const auto& c : cl) {
        th.resize((size_t)c.nparam);
        chain.resize((size_t)c.nparam);
        R.resize((size_t)c.L * c.L);
        cat_constrain(c.kind, c.L, rcat.data() + c.param_off, c.nparam, th.data(), chain.data());
        cat_correlation(c.kind, c.L, th.data(), R.data(), &dR);
        const size_t LL = (size_t)c.L * c.L;
        for (int k = 0; k < c.nparam; ++k) {
          double s = 0.0;
          for (size_t e = 0; e < LL; ++e) s += dR[(size_t)k * LL + e] * G[(size_t)c.table_off + e];
          gc[(size_t)(c.param_off + k)] = clip_gradient((float)s);
          chain_f[(size_t)(c.param_off + k)] = (float)chain[(size_t)k];
        }
      }
      cat_t += 1;
      const float bc1 = 1.0f - pow_float32(b1, cat_t), bc2 = 1.0f - pow_float32(b2, cat_t);
      for (int k = 0; k < KC; ++k) {
        const float gr = gc[(size_t)k] * chain_f[(size_t)k];
        mc[(size_t)k] = b1 * mc[(size_t)k] + (1.0f - b1) * gr;
        vc[(size_t)k] = b2 * vc[(size_t)k] + (1.0f - b2) * gr * gr;
        const float nr = rcat[(size_t)k] -
                         lr_eff * (mc[(size_t)k] / bc1) / (std::sqrt(vc[(size_t)k] / bc2) + eps);
        rcat[(size_t)k] = std::max(-20.0f, std::min(20.0f, nr));
      }
    }
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_iter).count();
    res.base.iter_times_ms.push_back(ms);
    res.base.nll_history.push_back(nll);
    {
      const int cur = it + 1;
      const int iv = std::max(1, o.progress_interval);
      if (cur <= 1 || cur >= o.max_iterations || cur % iv == 0)
        emit("iteration", actual, nll, best_nll_seen, r.cg_iterations, ms, noise, raw_mean, false);
    }
    if (o.enable_early_stopping) {
      if (nll < best_nll - o.early_stop_tol) {
        best_nll = nll;
        no_improve = 0;
      } else if (++no_improve >= o.early_stop_patience) {
        res.base.converged = true;
        break;
      }
    }
  }
  res.base.params.resize(P);
  for (int q = 0; q < P; ++q) res.base.params[q] = softplus(best_raw[q]);
  res.base.noise = softplus(best_raw[P]);
  res.base.mean = best_raw_mean;
  res.base.final_nll = best_nll_seen;
  res.base.iterations = actual;
  res.cat_raw = best_cat;
  // leave the provider at the best state (prediction reuses it)
  pv.params = res.base.params;
  write_tables(pv, cl, best_cat);
  pv.refresh_coords();
  pv.noise = res.base.noise;
  emit("complete", actual, best_nll_seen, best_nll_seen, -1, -1.0, res.base.noise,
       res.base.mean, res.base.converged);
  return res;
}

}  // namespace mgp
