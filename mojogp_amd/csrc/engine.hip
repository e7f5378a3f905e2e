// Host orchestration of training and prediction (see engine.h).
#include "engine.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <limits>

#include "host_numerics.h"

namespace mgp {

namespace {

constexpr float kPi = 3.14159265358979323846f;

using Clock = std::chrono::steady_clock;
double secs_since(Clock::time_point t0) {
  return std::chrono::duration<double>(Clock::now() - t0).count();
}

// dinv[i] = 1 / d[i], dsqrt[i] = sqrt(d[i])
__global__ void k_recip_sqrt(const float* __restrict__ d, int64_t n, float* __restrict__ dinv,
                             float* __restrict__ dsqrt) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dinv[i] = 1.0f / d[i];
  dsqrt[i] = sqrtf(d[i]);
}

// One wave per column (grid = ncols, 64 threads); fixed-order fp64 sum.
__global__ void k_part_to_float(const double* __restrict__ part, int nb, int ncols,
                                float* __restrict__ out) {
  const int c = blockIdx.x, lane = threadIdx.x;
  double s = 0.0;
  for (int b = lane; b < nb; b += 64) s += part[(int64_t)c * nb + b];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) out[c] = (float)s;
}

void part_to_float(const double* part, int nb, int ncols, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_part_to_float, dim3((unsigned)std::max(ncols, 1)), dim3(64), 0, st, part,
                     nb, ncols, out);
  MGP_HIP_CHECK(hipGetLastError());
}

// --------------------------------------------------- single right-hand-side CG
// Scalars: s[0] rr_old, s[1] initial residual norm, s[2] alpha, s[3] beta.
__global__ void k_a1_init(const double* __restrict__ part, int nb, float* s, int* done) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[b];
  const float rr = (float)acc;
  float init = sqrtf(rr);
  if (init < 1e-20f) init = 1.0f;
  s[0] = rr;
  s[1] = init;
  *done = 0;
}

__global__ void k_a1_alpha(const double* __restrict__ part, int nb, float* s, int* done) {
  if (threadIdx.x != 0 || blockIdx.x != 0 || *done) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[b];
  const float pap = (float)acc;
  if (pap != pap || pap < 1e-10f) {
    *done = 1;
    return;
  }
  const float a = s[0] / pap;
  if (a != a) {
    *done = 1;
    return;
  }
  s[2] = a;
}

__global__ void k_a1_update(float* __restrict__ x, float* __restrict__ r,
                            const float* __restrict__ p, const float* __restrict__ Ap,
                            int64_t n, int nb, const float* __restrict__ s,
                            const int* __restrict__ done, double* __restrict__ rr_part) {
  __shared__ double sm[4];
  if (*done) return;  // uniform
  const float a = s[2];
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  double acc = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    x[i] += a * p[i];
    const float ri = r[i] - a * Ap[i];
    r[i] = ri;
    acc += (double)ri * (double)ri;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += sm[w];
    rr_part[blockIdx.x] = t;
  }
}

__global__ void k_a1_beta(const double* __restrict__ part, int nb, float tol, float* s,
                          int* done) {
  if (threadIdx.x != 0 || blockIdx.x != 0 || *done) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[b];
  const float rr_new = (float)acc;
  if (sqrtf(rr_new) / s[1] < tol) {
    *done = 1;
    return;
  }
  const float rr_old = s[0];
  float beta = 0.0f;
  if (rr_old >= 1e-20f) {
    beta = rr_new / (rr_old + 1e-20f);
    if (beta < 0.0f || beta != beta) beta = 0.0f;
  }
  s[3] = beta;
  s[0] = rr_new;
}

__global__ void k_a1_pupdate(float* __restrict__ p, const float* __restrict__ r, int64_t n,
                             const float* __restrict__ s, const int* __restrict__ done) {
  if (*done) return;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = r[i] + s[3] * p[i];
}

// ---------------------------------------- independent single-RHS CG per column
// Column c keeps s[4c + 0..3] = rr_old, initial norm, alpha, beta and done[c];
// done[C] = every column finished.  One thread per column for the scalars.
__global__ void k_mc_init(const double* __restrict__ part, int nb, int C, float* s, int* done) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[(int64_t)c * nb + b];
  const float rr = (float)acc;
  float init = sqrtf(rr);
  if (init < 1e-20f) init = 1.0f;
  s[4 * c + 0] = rr;
  s[4 * c + 1] = init;
  done[c] = 0;
}

__global__ void k_mc_alpha(const double* __restrict__ part, int nb, int C, float* s, int* done) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C || done[c]) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[(int64_t)c * nb + b];
  const float pap = (float)acc;
  if (pap != pap || pap < 1e-10f) {
    done[c] = 1;
    return;
  }
  const float a = s[4 * c] / pap;
  if (a != a) {
    done[c] = 1;
    return;
  }
  s[4 * c + 2] = a;
}

// grid (nb, C): x += a p, r -= a Ap on chunk b of column c; rr partials.
__global__ void k_mc_update(float* __restrict__ x, float* __restrict__ r,
                            const float* __restrict__ p, const float* __restrict__ Ap, int64_t n,
                            int nb, const float* __restrict__ s, const int* __restrict__ done,
                            double* __restrict__ rr_part) {
  __shared__ double sm[4];
  const int c = blockIdx.y;
  if (done[c]) return;  // uniform per block
  const float a = s[4 * c + 2];
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const int64_t base = (int64_t)c * n;
  double acc = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    x[base + i] += a * p[base + i];
    const float ri = r[base + i] - a * Ap[base + i];
    r[base + i] = ri;
    acc += (double)ri * (double)ri;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += sm[w];
    rr_part[(int64_t)c * nb + blockIdx.x] = t;
  }
}

__global__ void k_mc_beta(const double* __restrict__ part, int nb, int C, float tol, float* s,
                          int* done) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C || done[c]) return;
  double acc = 0.0;
  for (int b = 0; b < nb; ++b) acc += part[(int64_t)c * nb + b];
  const float rr_new = (float)acc;
  if (sqrtf(rr_new) / s[4 * c + 1] < tol) {
    done[c] = 1;
    return;
  }
  const float rr_old = s[4 * c];
  float beta = 0.0f;
  if (rr_old >= 1e-20f) {
    beta = rr_new / (rr_old + 1e-20f);
    if (beta < 0.0f || beta != beta) beta = 0.0f;
  }
  s[4 * c + 3] = beta;
  s[4 * c] = rr_new;
}

__global__ void k_mc_pupdate(float* __restrict__ p, const float* __restrict__ r, int64_t n, int C,
                             const float* __restrict__ s, const int* __restrict__ done) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * C) return;
  const int c = (int)(idx / n);
  if (done[c]) return;
  p[idx] = r[idx] + s[4 * c + 3] * p[idx];
}

__global__ void k_mc_alldone(int C, int* done) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int all = 1;
  for (int c = 0; c < C; ++c) all &= done[c] != 0;
  done[C] = all;
}

// Lanczos three-term recurrence: w -= a v (+ b vprev).
__global__ void k_three_term(float* __restrict__ w, const float* __restrict__ v,
                             const float* __restrict__ vprev, float a, float b, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float x = w[i] - a * v[i];
  if (vprev) x -= b * vprev[i];
  w[i] = x;
}

__global__ void k_scale_into(float* __restrict__ dst, const float* __restrict__ src, float inv,
                             int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i] / inv;
}

__global__ void k_add_scalar(float* __restrict__ y, float s, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += s;
}

inline dim3 g1(int64_t n) { return dim3((unsigned)std::max<int64_t>(1, ceil_div(n, 256))); }

float dot_f(const float* a, const float* b, int64_t n, DevBuf<double>& part, hipStream_t st) {
  const int nb = reduction_chunks(n);
  double* pp = part.ensure((size_t)nb + 1);
  coldot_partial(a, b, n, 1, nb, pp, st);
  coldot_finalize(pp, nb, 1, pp + nb, st);
  double h = 0.0;
  MGP_HIP_CHECK(hipMemcpyAsync(&h, pp + nb, sizeof(double), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return (float)h;
}

}  // namespace

CGScalars CGWork::scalars(int ncols) {
  CGScalars s;
  s.rz_old = scal.ptr;
  s.rz_next = scal.ptr + ncols;
  s.alpha = scal.ptr + 2 * ncols;
  s.beta = scal.ptr + 3 * ncols;
  s.hist_alpha = hist_a.ptr;
  s.hist_beta = hist_b.ptr;
  s.done = done.ptr;
  return s;
}

// ------------------------------------------------------------------ precond
PivotOptions training_pivot_options(int method) {
  PivotOptions o;
  o.method = method;
  o.error_tol = method == 0 ? 0.0f : 1e-3f;  // jit_training.mojo:476-478
  return o;
}

void build_precond(Provider& pv, int rank, const PivotOptions& po, Precond& P) {
  P.vec = pv.has_noise_vec;
  P.noise = P.vec ? 1e-6f : pv.noise;
  if (rank <= 0) {
    P.rank = 0;
    P.logdet = 0.f;
    return;
  }
  MGP_REQUIRE(rank <= 1000, "preconditioner rank must be <= 1000");
  const int64_t n = pv.n;
  hipStream_t st = pv.st;
  P.L.ensure((size_t)rank * n);
  const int k = pivoted_cholesky(pv, rank, po, P.L.ptr, st);
  P.rank = k;
  if (P.vec) {
    // P = L L^T + D: M = I + L^T D^-1 L, log|P| = sum log d_i + log|M|.
    hipLaunchKernelGGL(k_recip_sqrt, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st,
                       pv.noise_vec.ptr, n,
                       P.dinv.ensure(n), P.dsqrt.ensure(n));
    MGP_HIP_CHECK(hipGetLastError());
    DevBuf<double> Md;
    Md.ensure((size_t)k * k);
    syrk_ltl(P.L.ptr, n, k, Md.ptr, st, P.dinv.ptr);
    std::vector<double> M((size_t)k * k);
    MGP_HIP_CHECK(hipMemcpy(M.data(), Md.ptr, M.size() * sizeof(double), hipMemcpyDeviceToHost));
    for (int i = 0; i < k; ++i) M[(size_t)i * k + i] += 1.0;
    std::vector<double> inv;
    if (!spd_inverse(M, k, inv)) throw Error(ST_NUMERIC, "preconditioner core matrix is singular");
    std::vector<float> invf(inv.begin(), inv.end());
    P.Minv.ensure(invf.size());
    MGP_HIP_CHECK(hipMemcpy(P.Minv.ptr, invf.data(), invf.size() * sizeof(float),
                            hipMemcpyHostToDevice));
    std::vector<float> d((size_t)n);
    MGP_HIP_CHECK(hipMemcpy(d.data(), pv.noise_vec.ptr, (size_t)n * sizeof(float),
                            hipMemcpyDeviceToHost));
    double ld = 0.0;
    for (int64_t i = 0; i < n; ++i) ld += std::log((double)d[(size_t)i]);
    P.logdet = (float)(ld + logdet_spd(M, k));
    return;
  }
  precond_from_factor(P, n, k, st);
}

void precond_from_factor(Precond& P, int64_t n, int k, hipStream_t st) {
  P.rank = k;
  P.vec = false;
  DevBuf<double> Md;
  Md.ensure((size_t)k * k);
  syrk_ltl(P.L.ptr, n, k, Md.ptr, st);
  std::vector<double> M((size_t)k * k);
  MGP_HIP_CHECK(hipMemcpy(M.data(), Md.ptr, M.size() * sizeof(double), hipMemcpyDeviceToHost));
  const double eff = std::max((double)P.noise, 1e-6);
  std::vector<double> A(M), inv;
  for (int i = 0; i < k; ++i) A[(size_t)i * k + i] += eff;
  if (!spd_inverse(A, k, inv)) throw Error(ST_NUMERIC, "preconditioner core matrix is singular");
  std::vector<float> invf(inv.begin(), inv.end());
  P.Minv.ensure(invf.size());
  MGP_HIP_CHECK(hipMemcpy(P.Minv.ptr, invf.data(), invf.size() * sizeof(float),
                          hipMemcpyHostToDevice));
  std::vector<double> B((size_t)k * k);
  for (size_t q = 0; q < B.size(); ++q) B[q] = M[q] / (double)P.noise;
  for (int i = 0; i < k; ++i) B[(size_t)i * k + i] += 1.0;
  P.logdet = (float)n * std::log(P.noise) + (float)logdet_spd(B, k);
}

// ------------------------------------------------------------------ batched CG
CGResult batched_cg(Provider& pv, Precond* P, const float* rhs, int C, int max_iter,
                    int max_tridiag, float tol, CGWork& w, bool warm_start) {
  CGOperator op;
  op.n = pv.n;
  op.st = pv.st;
  op.matvec = [&pv](const float* V, int ncols, float* out) { pv.forward(V, ncols, out); };
  if (P && P->rank > 0) {
    op.precond = [&pv, P](const float* r, int ncols, float* z, double* rz_part, int nb) {
      woodbury_apply(P->L.ptr, pv.n, P->rank, P->Minv.ptr, P->noise, r, ncols, z, P->work, r,
                     nb, rz_part, pv.st, P->dinv_ptr());
    };
  }
  return batched_cg(op, rhs, C, max_iter, max_tridiag, tol, w, warm_start);
}

CGResult batched_cg(const CGOperator& op, const float* rhs, int C, int max_iter,
                    int max_tridiag, float tol, CGWork& w, bool warm_start) {
  const int64_t n = op.n;
  hipStream_t st = op.st;
  const int nb = cg_chunks(n);
  const bool pre = (bool)op.precond;
  const size_t nc = (size_t)n * C;
  float* x = w.x.ptr;  // caller ensured capacity (warm start keeps contents)
  float* r = w.r.ensure(nc);
  float* z = pre ? w.z.ensure(nc) : r;
  float* p = w.p.ensure(nc);
  float* Ap = w.Ap.ensure(nc);
  w.scal.ensure((size_t)4 * C);
  const int mt = std::max(max_tridiag, 1);
  w.hist_a.ensure((size_t)mt * C);
  w.hist_b.ensure((size_t)mt * C);
  double* pa = w.part_a.ensure((size_t)C * nb);
  double* pb = w.part_b.ensure((size_t)C * nb);
  double* prr = w.part_c.ensure((size_t)C * nb);
  w.resn.ensure(1);
  w.done.ensure(1);
  CGScalars s = w.scalars(C);

  if (warm_start) {
    copy(r, rhs, nc, st);
    op.matvec(x, C, Ap);
    sub(r, r, Ap, nc, st);
  } else {
    fill(x, nc, 0.0f, st);
    copy(r, rhs, nc, st);
  }
  if (pre) {
    op.precond(r, C, z, pb, nb);
  } else {
    coldot_partial(r, r, n, C, nb, pb, st);
  }
  copy(p, z, nc, st);
  part_to_float(pb, nb, C, s.rz_old, st);

  CGResult res;
  int tridiag_size = 0;
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  const auto t_loop = Clock::now();
  for (int iter = 0; iter < max_iter; ++iter) {
    res.iterations = iter + 1;
    op.matvec(p, C, Ap);
    coldot_partial(p, Ap, n, C, nb, pa, st);
    cg_update(x, r, p, Ap, n, C, nb, pa, s, prr, st);  // alpha from pAp; r.r partials
    if (pre) op.precond(r, C, z, pb, nb);
    // beta from the r.z partials (r.r without a preconditioner), p update
    cg_pupdate(p, z, n, C, nb, pre ? pb : prr, s, iter, max_tridiag, st);
    std::swap(s.rz_old, s.rz_next);
    if (iter < max_tridiag) tridiag_size = iter + 1;
    if (iter >= 10 && (((iter + 1) % 10) == 0 || iter == max_iter - 1)) {
      cg_mean_resnorm(prr, nb, C, w.resn.ptr, st);
      float mean_res = 0.f;
      MGP_HIP_CHECK(hipMemcpyAsync(&mean_res, w.resn.ptr, sizeof(float),
                                   hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
      if (mean_res < tol && iter >= max_tridiag - 1) {
        res.converged = true;
        break;
      }
    }
  }
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  res.loop_ms = secs_since(t_loop) * 1e3;
  res.tridiag_size = tridiag_size;
  res.diag.assign(C, {});
  res.offdiag.assign(C, {});
  if (tridiag_size > 0) {
    std::vector<float> ha((size_t)tridiag_size * C), hb((size_t)tridiag_size * C);
    MGP_HIP_CHECK(hipMemcpyAsync(ha.data(), s.hist_alpha, ha.size() * sizeof(float),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipMemcpyAsync(hb.data(), s.hist_beta, hb.size() * sizeof(float),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    // GPyTorch tridiagonal conventions (combined_inv_quad_logdet.mojo:356-424):
    // 1/alpha := 1 for alpha < 1e-10; negative beta clamps to 0; building stops
    // for every column once the largest off-diagonal falls below 1e-6.
    auto recip = [](float a) { return a < 1e-10f ? 1.0f : 1.0f / a; };
    for (int k = 0; k < tridiag_size; ++k) {
      float max_off = 0.0f;
      for (int c = 0; c < C; ++c) {
        const float ak = ha[(size_t)k * C + c];
        float dv = recip(ak);
        if (k > 0) {
          const float bk = hb[(size_t)(k - 1) * C + c];
          const float apr = recip(ha[(size_t)(k - 1) * C + c]);
          dv = dv + bk * apr;
          const float bc = bk < 0.0f ? 0.0f : bk;
          const float off = std::sqrt(bc) * apr;
          res.offdiag[c].push_back(off);
          if (off > max_off) max_off = off;
        }
        res.diag[c].push_back(dv);
      }
      if (k > 0 && max_off < 1e-6f) break;
    }
  }
  return res;
}

// ------------------------------------------------------------------ BBMM
BBMMResult bbmm_step(Provider& pv, Precond& P, bool use_precond, const float* y_c, int T,
                     int max_cg, int max_tridiag, float tol, int iteration, bool recycle,
                     BBMMWork& w) {
  const int64_t n = pv.n;
  hipStream_t st = pv.st;
  const int C = 1 + T;
  const size_t nT = (size_t)n * T, nC = (size_t)n * C;
  const bool pre = use_precond && P.rank > 0;
  const uint64_t seed = (uint64_t)((int64_t)iteration * 104729 + 42);

  float* probes = w.probes.ensure(std::max<size_t>(nT, 1));
  float* pn = w.probe_norms.ensure(std::max(T, 1));
  float* rn = w.rhs_norms.ensure(C);
  double* part = w.part.ensure((size_t)std::max(C, 1) * reduction_chunks(n) + 64);
  if (T > 0) {
    if (pre) {
      float* zr = w.zr.ensure((size_t)P.rank * T);
      float* zn = w.zn.ensure(nT);
      gaussian(zr, (int64_t)P.rank * T, seed, st);
      gaussian(zn, (int64_t)nT, seed + 1000000ull, st);
      low_rank_sample(P.L.ptr, n, P.rank, zr, zn, std::sqrt(P.noise), T, probes, st,
                      P.dsqrt_ptr());
    } else {
      gaussian(probes, (int64_t)nT, seed, st);
    }
    normalize_columns(probes, n, T, pn, part, st);
  }
  // RHS [y | Z_norm], every column normalised (GPyTorch linear_cg convention).
  float* rhs = w.rhs.ensure(nC);
  copy(rhs, y_c, n, st);
  if (T > 0) copy(rhs + n, probes, nT, st);
  normalize_columns(rhs, n, C, rn, part, st);

  const bool warm = recycle && iteration > 0 && w.has_x && w.cg.x.count >= nC;
  if (!warm) w.cg.x.ensure(nC);
  if (warm && C > 1) fill(w.cg.x.ptr + n, (int64_t)n * (C - 1), 0.0f, st);
  CGResult cg = batched_cg(pv, pre ? &P : nullptr, rhs, C, max_cg, max_tridiag, tol, w.cg, warm);
  w.has_x = true;

  float* sol = w.sol.ensure(nC);
  copy(sol, w.cg.x.ptr, nC, st);
  scale_columns(sol, rn, n, C, false, st);

  BBMMResult out;
  out.cg_iterations = cg.iterations;
  out.converged = cg.converged;
  out.cg_loop_ms = cg.loop_ms;
  out.alpha_dev = sol;
  out.inv_quad = dot_f(y_c, sol, n, w.part, st);

  float logdet = 0.0f;
  if (cg.tridiag_size > 0) {
    std::vector<std::vector<float>> pd(cg.diag.begin() + 1, cg.diag.end());
    std::vector<std::vector<float>> po(cg.offdiag.begin() + 1, cg.offdiag.end());
    logdet = slq_logdet(pd, po, n);
    if (pre) logdet += P.logdet;
  }
  out.logdet = logdet;
  const float constant = 0.5f * (float)n * std::log(2.0f * kPi);
  out.nll = (0.5f * out.inv_quad + 0.5f * logdet + constant) / (float)n;

  // Gradient factors: Lf = [-alpha/2 | (0.5/T) U], Rf = [alpha | P^-1 Z].
  std::vector<float> norms(std::max(T, 1), 1.0f);
  if (T > 0)
    MGP_HIP_CHECK(hipMemcpyAsync(norms.data(), pn, T * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  std::vector<float> lfac(C), rfac(C);
  lfac[0] = -0.5f;
  rfac[0] = 1.0f;
  for (int j = 0; j < T; ++j) {
    lfac[1 + j] = (0.5f / (float)T) * norms[j];
    rfac[1 + j] = norms[j];
  }
  DevBuf<float> facs;
  facs.ensure(2 * (size_t)C);
  MGP_HIP_CHECK(hipMemcpyAsync(facs.ptr, lfac.data(), C * sizeof(float), hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipMemcpyAsync(facs.ptr + C, rfac.data(), C * sizeof(float), hipMemcpyHostToDevice, st));
  float* lf = w.lf.ensure(nC);
  float* rf = w.rf.ensure(nC);
  copy(lf, sol, nC, st);
  scale_columns(lf, facs.ptr, n, C, false, st);
  copy(rf, sol, n, st);
  if (T > 0) {
    copy(rf + n, probes, nT, st);
    scale_columns(rf + n, facs.ptr + C + 1, n, T, false, st);
    if (pre)
      woodbury_apply(P.L.ptr, n, P.rank, P.Minv.ptr, P.noise, rf + n, T, rf + n, P.work,
                     nullptr, 0, nullptr, st, P.dinv_ptr());
  }
  const int np = pv.nparams;
  std::vector<double> g(np, 0.0);
  gradient_traces(pv, lf, rf, C, g.data(), st);
  out.grads.resize(np + 1);
  for (int q = 0; q < np; ++q) {
    float gq = (float)(g[q] / (double)n);
    if (!std::isfinite(gq)) gq = 0.0f;
    out.grads[q] = gq;
  }
  // Noise: dK/dsigma^2 = I  ->  sum_c Lf_c . Rf_c / n.
  const int nb = reduction_chunks(n);
  coldot_partial(lf, rf, n, C, nb, part, st);
  coldot_finalize(part, nb, C, part + (size_t)C * nb, st);
  std::vector<double> dots(C);
  MGP_HIP_CHECK(hipMemcpyAsync(dots.data(), part + (size_t)C * nb, C * sizeof(double),
                               hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  double tot = 0.0;
  for (int c = 0; c < C; ++c) tot += dots[c];
  float gn = (float)(tot / (double)n);
  if (!std::isfinite(gn)) gn = 0.0f;
  out.grads[np] = gn;
  return out;
}

// ------------------------------------------------------------------ learned noise
namespace {
// out[i] = sum_c Lf[c][i] Rf[c][i]: with Lf = [-alpha/2 | (0.5/T) U] and
// Rf = [alpha | P^-1 Z] this is 0.5 (diag(K^-1) estimate_i - alpha_i^2), the
// per-point derivative of n * NLL with respect to noise variance i.
__global__ void k_row_dots(const float* __restrict__ lf, const float* __restrict__ rf, int64_t n,
                           int C, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  double s = 0.0;
  for (int c = 0; c < C; ++c) s += (double)lf[(int64_t)c * n + i] * (double)rf[(int64_t)c * n + i];
  out[i] = (float)s;
}

// Learned per-point noise state of the reference's noise modes 2-4
// (jit_training.mojo:41-228, 352-437, 699-812, 919-960): raw values on the
// host (one per point, one per group, or the 1 + d weights of a linear
// function of the raw inputs), their own Adam moments, a best-NLL snapshot.
// The noise vector noise_i = softplus(raw_i) + floor is rebuilt and uploaded
// from this state; gradients come from the per-point row dots of the BBMM
// gradient factors.
struct LearnedNoise {
  int mode = 0;
  int64_t n = 0;
  int d = 0;
  float floor = 1e-6f, reg = 0.f, target = 0.f;
  std::vector<float> raw, m, v, best_raw, best_m, best_v, vec, Xh, rd;
  const std::vector<int>* groups = nullptr;
  DevBuf<float> rd_dev;

  void init(Provider& pv, float init_noise, const TrainOptions& o) {
    mode = pv.learned_noise_mode;
    if (mode == 0) return;
    MGP_REQUIRE(mode >= 2 && mode <= 4, "learned noise mode must be 2, 3 or 4");
    MGP_REQUIRE(pv.has_noise_vec, "learned noise needs an initial noise vector");
    n = pv.n;
    d = pv.d;
    floor = o.noise_floor;
    reg = o.noise_regularization;
    target = std::max(init_noise, floor);
    size_t S = (size_t)n;
    if (mode == 3) {
      MGP_REQUIRE(pv.num_noise_groups >= 1 && (int64_t)pv.noise_groups.size() == n,
                  "learned grouped noise needs group ids");
      S = (size_t)pv.num_noise_groups;
      groups = &pv.noise_groups;
    }
    if (mode == 4) {
      S = (size_t)d + 1;
      Xh.resize((size_t)n * d);
      MGP_HIP_CHECK(hipMemcpyAsync(Xh.data(), pv.X.ptr, Xh.size() * sizeof(float),
                                   hipMemcpyDeviceToHost, pv.st));
      MGP_HIP_CHECK(hipStreamSynchronize(pv.st));
    }
    const float r0 = inv_softplus(std::max(init_noise - floor, 1e-8f));
    raw.assign(S, mode == 4 ? 0.0f : r0);
    raw[0] = r0;
    m.assign(S, 0.0f);
    v.assign(S, 0.0f);
    best_raw = raw;
    best_m = m;
    best_v = v;
    vec.resize((size_t)n);
    MGP_HIP_CHECK(hipMemcpyAsync(vec.data(), pv.noise_vec.ptr, (size_t)n * sizeof(float),
                                 hipMemcpyDeviceToHost, pv.st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv.st));
  }

  float linear_raw(int64_t i) const {
    float r = raw[0];
    for (int j = 0; j < d; ++j) r += raw[(size_t)j + 1] * Xh[(size_t)i * d + j];
    return r;
  }

  void apply(Provider& pv) {
    for (int64_t i = 0; i < n; ++i) {
      if (mode == 2) {
        vec[(size_t)i] = softplus(raw[(size_t)i]) + floor;
      } else if (mode == 3) {
        const int g = (*groups)[(size_t)i];
        if (g >= 0 && g < (int)raw.size()) vec[(size_t)i] = softplus(raw[(size_t)g]) + floor;
      } else {
        vec[(size_t)i] = softplus(linear_raw(i)) + floor;
      }
    }
    pv.load_noise_vector(vec.data());
  }

  void snapshot() {
    best_raw = raw;
    best_m = m;
    best_v = v;
  }
  void restore() {
    raw = best_raw;
    m = best_m;
    v = best_v;
  }

  // d/dnoise of the noise regulariser reg * log(noise / target)^2 / (2 count).
  double reg_grad(float noise, double count) const {
    if (!(reg > 0.f)) return 0.0;
    return (double)reg * std::log((double)noise / (double)target) / ((double)noise * count);
  }

  void step(Provider& pv, const float* lf, const float* rf, int C, float lr, int t) {
    rd.resize((size_t)n);
    rd_dev.ensure((size_t)n);
    hipLaunchKernelGGL(k_row_dots, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, pv.st, lf, rf,
                       n, C, rd_dev.ptr);
    MGP_HIP_CHECK(hipGetLastError());
    MGP_HIP_CHECK(hipMemcpyAsync(rd.data(), rd_dev.ptr, (size_t)n * sizeof(float),
                                 hipMemcpyDeviceToHost, pv.st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv.st));
    const double dn = (double)n;
    std::vector<double> g(raw.size(), 0.0);
    if (mode == 2) {
      for (int64_t i = 0; i < n; ++i) {
        const float ri = raw[(size_t)i];
        const float ni = softplus(ri) + floor;
        g[(size_t)i] = ((double)rd[(size_t)i] / dn + reg_grad(ni, dn)) * softplus_derivative(ri);
      }
    } else if (mode == 3) {
      const int G = (int)raw.size();
      for (int64_t i = 0; i < n; ++i) {
        const int gi = (*groups)[(size_t)i];
        if (gi >= 0 && gi < G) g[(size_t)gi] += (double)rd[(size_t)i] / dn;
      }
      for (int k = 0; k < G; ++k) {
        const float ng = softplus(raw[(size_t)k]) + floor;
        g[(size_t)k] = (g[(size_t)k] + reg_grad(ng, (double)G)) * softplus_derivative(raw[(size_t)k]);
      }
    } else {
      for (int64_t i = 0; i < n; ++i) {
        const float ri = linear_raw(i);
        const float ni = softplus(ri) + floor;
        const double gr = ((double)rd[(size_t)i] / dn + reg_grad(ni, dn)) * softplus_derivative(ri);
        g[0] += gr;
        for (int j = 0; j < d; ++j) g[(size_t)j + 1] += gr * Xh[(size_t)i * d + j];
      }
      if (reg > 0.f)
        for (int j = 1; j <= d; ++j) g[(size_t)j] += (double)reg * raw[(size_t)j] / std::max(d, 1);
    }
    // Adam on the raw values (kernel_adam_update_vector): non-finite or
    // |g| > 1e6 gradients count as 0; no clamp of the raw values.
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float bp1 = pow_float32(b1, t), bp2 = pow_float32(b2, t);
    for (size_t k = 0; k < raw.size(); ++k) {
      float gk = (float)g[k];
      if (gk != gk || gk > 1e6f || gk < -1e6f) gk = 0.0f;
      m[k] = b1 * m[k] + (1.0f - b1) * gk;
      v[k] = b2 * v[k] + (1.0f - b2) * gk * gk;
      const float mh = m[k] / (1.0f - bp1), vh = v[k] / (1.0f - bp2);
      raw[k] -= lr * mh / (std::sqrt(vh) + eps);
    }
  }
};
}  // namespace

// ------------------------------------------------------------------ training
TrainResult train(Provider& pv, const float* y_host, const std::vector<float>& init_params,
                  float init_noise, const TrainOptions& o,
                  const std::function<void(const ProgressEvent&)>& progress) {
  const int64_t n = pv.n;
  const int P = pv.nparams;
  hipStream_t st = pv.st;
  MGP_REQUIRE((int)init_params.size() == P, "initial params size mismatch");
  MGP_REQUIRE(o.max_iterations >= 1, "max_iterations must be >= 1");
  MGP_REQUIRE(o.num_probes >= 0, "num_probes must be >= 0");

  DevBuf<float> y, yc;
  y.ensure(n);
  yc.ensure(n);
  MGP_HIP_CHECK(hipMemcpyAsync(y.ptr, y_host, n * sizeof(float), hipMemcpyHostToDevice, st));

  std::vector<float> raw(P + 1);
  for (int q = 0; q < P; ++q) raw[q] = inv_softplus(init_params[q]);
  raw[P] = inv_softplus(init_noise);
  float raw_mean = o.init_mean;
  std::vector<float> m_(P + 1, 0.f), v_(P + 1, 0.f);
  float m_mean = 0.f, v_mean = 0.f;
  int adam_t = 0;

  std::vector<float> best_raw(raw), best_m(P + 1, 0.f), best_v(P + 1, 0.f);
  float best_raw_mean = raw_mean, best_m_mean = 0.f, best_v_mean = 0.f;
  int best_t = 0;
  float best_nll_seen = 1e30f, best_nll = 1e30f;
  std::vector<float> best_alpha;
  int no_improve = 0;
  float lr = o.learning_rate;

  std::vector<float> last_rebuild(init_params);
  float last_rebuild_noise = init_noise;

  TrainResult res;
  Precond Pc;
  BBMMWork work;
  LearnedNoise ln;
  ln.init(pv, init_noise, o);
  if (ln.mode) ln.apply(pv);
  const int precond_rank = o.use_preconditioner ? o.precond_rank : 0;
  auto rebuild = [&]() {
    auto t0 = Clock::now();
    build_precond(pv, precond_rank, training_pivot_options(o.precond_method), Pc);
    res.precond_build_total_ms += secs_since(t0) * 1e3;
    res.precond_build_count += 1;
  };
  rebuild();

  auto emit = [&](const char* phase, int cur, float nll, float bnll, int cgi, double ms,
                  float noise, float mean, bool conv) {
    if (!progress) return;
    ProgressEvent e{phase, cur, o.max_iterations, nll, bnll, cgi, ms, noise, mean,
                    Pc.rank, std::max(0, res.precond_build_count - 1), conv};
    progress(e);
  };
  emit("start", 0, 0.f, 0.f, -1, -1.0, -1.f, 0.f, false);

  std::vector<float> params(P);
  int actual = 0;
  for (int it = 0; it < o.max_iterations; ++it) {
    auto t_iter = Clock::now();
    actual = it + 1;
    for (int q = 0; q < P; ++q) params[q] = softplus(raw[q]);
    const float noise = o.learn_noise ? softplus(raw[P]) : 0.0f;
    if (ln.mode) ln.apply(pv);
    pv.params = params;
    pv.refresh_coords();
    pv.noise = noise;

    if (it > 0) {
      float max_rel = 0.f;
      for (int q = 0; q < P; ++q)
        max_rel = std::max(max_rel, std::fabs(params[q] - last_rebuild[q]) /
                                        std::max(std::fabs(last_rebuild[q]), 1e-8f));
      if (o.learn_noise)
        max_rel = std::max(max_rel, std::fabs(noise - last_rebuild_noise) /
                                        std::max(std::fabs(last_rebuild_noise), 1e-8f));
      if (ln.mode) max_rel = o.precond_rebuild_threshold + 1.0f;  // the vector moves every step
      if (max_rel > o.precond_rebuild_threshold) {
        rebuild();
        res.precond_rebuild_steps.push_back(it);
        last_rebuild = params;
        last_rebuild_noise = noise;
      }
    }
    res.precond_rank_history.push_back(Pc.rank);

    sub_scalar(yc.ptr, y.ptr, raw_mean, n, st);
    BBMMResult r = bbmm_step(pv, Pc, o.use_preconditioner, yc.ptr, o.num_probes, o.max_cg_iter,
                             o.max_tridiag_iter, o.cg_tol, it, it > 0, work);
    const bool forced_nan = it < 64 && ((o.nan_inject_mask >> it) & 1ull);
    const float nll = forced_nan ? std::numeric_limits<float>::quiet_NaN() : r.nll;
    res.cg_iterations_history.push_back(r.cg_iterations);

    if (nll != nll) {
      // NaN recovery (jit_training.mojo:605-685): halve LR, restore the best
      // snapshot, rebuild the preconditioner, skip the update.
      lr *= 0.5f;
      raw = best_raw;
      m_ = best_m;
      v_ = best_v;
      m_mean = best_m_mean;
      v_mean = best_v_mean;
      adam_t = best_t;
      raw_mean = best_raw_mean;
      for (int q = 0; q < P; ++q) params[q] = softplus(raw[q]);
      last_rebuild = params;
      const float rn = o.learn_noise ? softplus(raw[P]) : 0.0f;
      pv.params = params;
      pv.refresh_coords();
      pv.noise = rn;
      last_rebuild_noise = rn;
      if (ln.mode) {
        ln.restore();
        ln.apply(pv);
      }
      rebuild();
      res.precond_rebuild_steps.push_back(it);
      if (o.verbose) std::printf("  NaN NLL detected at iteration %d - halving LR to %g\n", it, lr);
      emit("nan", actual, nll, best_nll_seen, r.cg_iterations, secs_since(t_iter) * 1e3, rn,
           raw_mean, false);
      continue;
    }

    if (nll < best_nll_seen) {
      best_nll_seen = nll;
      best_raw = raw;
      best_raw_mean = raw_mean;
      best_m = m_;
      best_v = v_;
      best_m_mean = m_mean;
      best_v_mean = v_mean;
      best_t = adam_t;
      if (ln.mode) ln.snapshot();
      best_alpha.resize(n);
      MGP_HIP_CHECK(hipMemcpyAsync(best_alpha.data(), r.alpha_dev, n * sizeof(float),
                                   hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
    }

    const float lr_eff = o.use_cosine_lr ? cosine_lr(o.learning_rate, it, o.max_iterations) : lr;
    std::vector<float> grads(P + 1);
    for (int q = 0; q < P; ++q) grads[q] = r.grads[q];
    grads[P] = o.learn_noise ? r.grads[P] : 0.0f;

    // Adam (training_utils.mojo:214-316): moments on raw parameters through the
    // softplus chain rule, bias correction, raw clamp to [-20, 20].
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    for (int q = 0; q <= P; ++q) {
      const float gr = clip_gradient(grads[q]) * softplus_derivative(raw[q]);
      m_[q] = b1 * m_[q] + (1.0f - b1) * gr;
      v_[q] = b2 * v_[q] + (1.0f - b2) * gr * gr;
    }
    adam_t += 1;
    const float bc1 = 1.0f - pow_float32(b1, adam_t), bc2 = 1.0f - pow_float32(b2, adam_t);
    for (int q = 0; q <= P; ++q) {
      const float mh = m_[q] / bc1, vh = v_[q] / bc2;
      float nr = raw[q] - lr_eff * mh / (std::sqrt(vh) + eps);
      raw[q] = std::max(-20.0f, std::min(20.0f, nr));
    }
    if (ln.mode) ln.step(pv, work.lf.ptr, work.rf.ptr, 1 + o.num_probes, lr_eff, adam_t);
    // Constant mean: gradient -sum(alpha)/n, its own Adam moments.
    {
      DevBuf<float> ones;
      ones.ensure(n);
      fill(ones.ptr, n, 1.0f, st);
      const float s = dot_f(ones.ptr, r.alpha_dev, n, work.part, st);
      float mg = clip_gradient(-s / (float)n);
      m_mean = b1 * m_mean + (1.0f - b1) * mg;
      v_mean = b2 * v_mean + (1.0f - b2) * mg * mg;
      const float mh = m_mean / (1.0f - pow_float32(b1, adam_t));
      const float vh = v_mean / (1.0f - pow_float32(b2, adam_t));
      raw_mean -= lr_eff * mh / (std::sqrt(vh) + eps);
    }
    if (raw_mean != raw_mean || raw_mean > 1000.0f || raw_mean < -1000.0f) raw_mean = o.init_mean;
    if (o.verbose && (it % 10 == 0 || it == o.max_iterations - 1))
      std::printf("Iter %d : NLL = %g , noise = %g , mean = %g\n", it, nll, noise, raw_mean);

    const double ms = secs_since(t_iter) * 1e3;
    res.iter_times_ms.push_back(ms);
    res.nll_history.push_back(nll);
    {
      const int cur = it + 1;
      const int iv = std::max(1, o.progress_interval);
      const bool due = cur <= 1 || cur >= o.max_iterations || cur % iv == 0;
      if (due) emit("iteration", actual, nll, best_nll_seen, r.cg_iterations, ms, noise, raw_mean, false);
    }
    if (o.enable_early_stopping) {
      if (nll < best_nll - o.early_stop_tol) {
        best_nll = nll;
        no_improve = 0;
      } else if (++no_improve >= o.early_stop_patience) {
        res.converged = true;
        emit("early_stop", actual, nll, best_nll_seen, r.cg_iterations, ms, noise, raw_mean, true);
        break;
      }
    }
  }

  raw = best_raw;
  raw_mean = best_raw_mean;
  if (ln.mode) {
    ln.raw = ln.best_raw;
    ln.apply(pv);
    res.learned_noise = ln.vec;
    if (ln.mode == 4) res.noise_fn_params = ln.raw;
  }
  res.params.resize(P);
  for (int q = 0; q < P; ++q) res.params[q] = softplus(raw[q]);
  res.noise = o.learn_noise ? softplus(raw[P]) : 0.0f;
  res.mean = raw_mean;
  res.final_nll = best_nll_seen;
  res.iterations = actual;
  res.alpha = std::move(best_alpha);
  emit("complete", actual, best_nll_seen, best_nll_seen, -1, -1.0, res.noise, res.mean,
       res.converged);
  return res;
}

// ------------------------------------------------------------------ prediction
namespace {

// Unpreconditioned single-column CG for alpha = (K + noise I)^-1 (y - mean),
// one iteration per step() after the caller has formed Ap = A p.  p and Ap
// may live in a caller's product buffer (shared products with the Lanczos
// root); the stop flag is read every 4 iterations, as the reference's host
// solver checks its residual (solve_single_rhs_deterministic_host_jit).
struct AlphaSolve {
  Provider& pv;
  int64_t n;
  hipStream_t st;
  int nb, max_iter;
  float tol;
  DevBuf<float> r, pbuf, Apbuf, s;
  DevBuf<double> part;
  DevBuf<int> done;
  float *x, *p, *Ap;
  int it = 0;
  bool finished = false;

  AlphaSolve(Provider& pv_, const float* y_host, float mean, int max_iter_, float tol_,
             PredictState& ps, float* p_ext = nullptr, float* Ap_ext = nullptr)
      : pv(pv_), n(pv_.n), st(pv_.st), nb(reduction_chunks(pv_.n)), max_iter(max_iter_),
        tol(tol_) {
    x = ps.alpha.ensure(n);
    r.ensure(n);
    p = p_ext ? p_ext : pbuf.ensure(n);
    Ap = Ap_ext ? Ap_ext : Apbuf.ensure(n);
    s.ensure(4);
    part.ensure((size_t)2 * nb);
    done.ensure(1);
    MGP_HIP_CHECK(hipMemcpyAsync(r.ptr, y_host, n * sizeof(float), hipMemcpyHostToDevice, st));
    sub_scalar(r.ptr, r.ptr, mean, n, st);
    fill(x, n, 0.0f, st);
    copy(p, r.ptr, n, st);
    coldot_partial(r.ptr, r.ptr, n, 1, nb, part.ptr, st);
    hipLaunchKernelGGL(k_a1_init, dim3(1), dim3(64), 0, st, part.ptr, nb, s.ptr, done.ptr);
    finished = max_iter <= 0;
  }
  void step() {
    coldot_partial(p, Ap, n, 1, nb, part.ptr, st);
    hipLaunchKernelGGL(k_a1_alpha, dim3(1), dim3(64), 0, st, part.ptr, nb, s.ptr, done.ptr);
    hipLaunchKernelGGL(k_a1_update, dim3(nb), dim3(256), 0, st, x, r.ptr, p, Ap, n, nb, s.ptr,
                       done.ptr, part.ptr + nb);
    hipLaunchKernelGGL(k_a1_beta, dim3(1), dim3(64), 0, st, part.ptr + nb, nb, tol, s.ptr,
                       done.ptr);
    hipLaunchKernelGGL(k_a1_pupdate, g1(n), dim3(256), 0, st, p, r.ptr, n, s.ptr, done.ptr);
    MGP_HIP_CHECK(hipGetLastError());
    if ((it & 3) == 3 || it == max_iter - 1) {
      int dh = 0;
      MGP_HIP_CHECK(hipMemcpyAsync(&dh, done.ptr, sizeof(int), hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
      if (dh) {  // iterations reported as the index of the stopping one
        finished = true;
        return;
      }
    }
    if (++it >= max_iter) finished = true;
  }
};

}  // namespace

int solve_alpha(Provider& pv, const float* y_host, float mean, int max_iter, float tol,
                PredictState& ps) {
  AlphaSolve a(pv, y_host, mean, max_iter, tol, ps);
  while (!a.finished) {
    pv.forward(a.p, 1, a.Ap);
    a.step();
  }
  MGP_HIP_CHECK(hipStreamSynchronize(pv.st));
  ps.has_alpha = true;
  return a.it;
}

int solve_columns(const CGOperator& op, const float* B, int C, int max_iter, float tol,
                  float* X) {
  MGP_REQUIRE(C >= 1 && C <= 65535, "solve_columns needs 1..65535 columns");
  const int64_t n = op.n;
  hipStream_t st = op.st;
  const int nb = reduction_chunks(n);
  const size_t nc = (size_t)n * C;
  DevBuf<float> r, p, Ap, s;
  DevBuf<double> part;
  DevBuf<int> done;
  r.ensure(nc);
  p.ensure(nc);
  Ap.ensure(nc);
  s.ensure((size_t)4 * C);
  part.ensure((size_t)2 * nb * C);
  done.ensure((size_t)C + 1);
  const dim3 gc((unsigned)ceil_div(C, 64));
  copy(r.ptr, B, (int64_t)nc, st);
  copy(p.ptr, B, (int64_t)nc, st);
  fill(X, (int64_t)nc, 0.0f, st);
  coldot_partial(r.ptr, r.ptr, n, C, nb, part.ptr, st);
  hipLaunchKernelGGL(k_mc_init, gc, dim3(64), 0, st, part.ptr, nb, C, s.ptr, done.ptr);
  int it = 0;
  for (; it < max_iter; ++it) {
    op.matvec(p.ptr, C, Ap.ptr);
    coldot_partial(p.ptr, Ap.ptr, n, C, nb, part.ptr, st);
    hipLaunchKernelGGL(k_mc_alpha, gc, dim3(64), 0, st, part.ptr, nb, C, s.ptr, done.ptr);
    hipLaunchKernelGGL(k_mc_update, dim3(nb, C), dim3(256), 0, st, X, r.ptr, p.ptr, Ap.ptr, n,
                       nb, s.ptr, done.ptr, part.ptr + (size_t)nb * C);
    hipLaunchKernelGGL(k_mc_beta, gc, dim3(64), 0, st, part.ptr + (size_t)nb * C, nb, C, tol,
                       s.ptr, done.ptr);
    hipLaunchKernelGGL(k_mc_pupdate, g1((int64_t)nc), dim3(256), 0, st, p.ptr, r.ptr, n, C,
                       s.ptr, done.ptr);
    MGP_HIP_CHECK(hipGetLastError());
    if ((it & 3) == 3 || it == max_iter - 1) {
      hipLaunchKernelGGL(k_mc_alldone, dim3(1), dim3(64), 0, st, C, done.ptr);
      int dh = 0;
      MGP_HIP_CHECK(hipMemcpyAsync(&dh, done.ptr + C, sizeof(int), hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
      if (dh) {
        ++it;
        break;
      }
    }
  }
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return it;
}

namespace {

// Lanczos on K + noise I from the deterministic +-1 start vector
// (compute_lanczos_inv_root_jit, jit_prediction.mojo:974-1177), one iteration
// per step() after the caller has formed w = A v_j (w may live in a caller's
// product buffer); finish() forms the inverse root.
struct LanczosSolve {
  Provider& pv;
  int64_t n;
  hipStream_t st;
  int r, nb;
  DevBuf<float> Q, wbuf;
  DevBuf<double> part, coef;
  float* w;
  std::vector<double> alpha, beta, inner;
  float beta_prev = 0.0f;
  int j = 0;
  bool finished = false;

  LanczosSolve(Provider& pv_, int r_, float* w_ext = nullptr)
      : pv(pv_), n(pv_.n), st(pv_.st), r(r_), nb(reduction_chunks(pv_.n)) {
    MGP_REQUIRE(r >= 1 && r <= 1000, "Lanczos rank must be in [1, 1000]");
    Q.ensure((size_t)r * n);
    w = w_ext ? w_ext : wbuf.ensure(n);
    part.ensure((size_t)(r + 1) * nb + 8);
    coef.ensure((size_t)r + 1);
    fill(Q.ptr, (int64_t)r * n, 0.0f, st);
    // Deterministic +-1 start vector (jit_prediction.mojo:999-1015).
    std::vector<float> z(n);
    float zsq = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      uint64_t s = 0xC0FFEE1234567890ull ^ ((uint64_t)i * 0x9E3779B97F4A7C15ull) ^
                   ((uint64_t)r * 0xBF58476D1CE4E5B9ull);
      s ^= s >> 12;
      s ^= s << 25;
      s ^= s >> 27;
      s *= 0x2545F4914F6CDD1Dull;
      z[i] = (s & 0x20000ull) ? 1.0f : -1.0f;
      zsq += z[i] * z[i];
    }
    const float zn = std::sqrt(zsq);
    for (int64_t i = 0; i < n; ++i) z[i] /= zn;
    MGP_HIP_CHECK(hipMemcpyAsync(Q.ptr, z.data(), n * sizeof(float), hipMemcpyHostToDevice, st));
    // The start vector's host buffer must outlive the copy.
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    alpha.assign(r, 0.0);
    beta.assign(std::max(r - 1, 0), 0.0);
    inner.assign(r + 1, 0.0);
  }
  const float* vec() const { return Q.ptr + (size_t)j * n; }
  void step() {
    const float* v = vec();
    const float aj = dot_f(v, w, n, part, st);
    alpha[j] = aj;
    hipLaunchKernelGGL(k_three_term, g1(n), dim3(256), 0, st, w, v,
                       j > 0 ? Q.ptr + (size_t)(j - 1) * n : nullptr, aj, beta_prev, n);
    // Full re-orthogonalisation against Q_0..Q_j, at most two passes; the
    // second pass runs only if the first saw an inner product >= 1e-5.
    for (int pass = 0; pass < 2; ++pass) {
      multi_dot(Q.ptr, j + 1, w, n, part.ptr, nb, coef.ptr, st);
      MGP_HIP_CHECK(hipMemcpyAsync(inner.data(), coef.ptr, (j + 1) * sizeof(double),
                                   hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
      double mx = 0.0;
      for (int k = 0; k <= j; ++k) mx = std::max(mx, std::fabs(inner[k]));
      multi_axpy(Q.ptr, j + 1, coef.ptr, w, n, st);
      if (mx < 1e-5) break;
    }
    const float bj = std::sqrt(dot_f(w, w, n, part, st));
    if (j < r - 1) beta[j] = bj;
    if (bj < 1e-10f) {  // remaining Q columns stay zero
      finished = true;
      return;
    }
    if (j + 1 < r)
      hipLaunchKernelGGL(k_scale_into, g1(n), dim3(256), 0, st, Q.ptr + (size_t)(j + 1) * n, w,
                         bj, n);
    beta_prev = bj;
    if (++j >= r) finished = true;
  }
  void finish(PredictState& ps) {
    std::vector<double> ev, V;
    if (!tridiag_eigh(alpha, beta, ev, &V))
      throw Error(ST_NUMERIC, "Lanczos tridiagonal eigendecomposition did not converge");
    double max_eig = 1e-10;
    for (double e : ev) max_eig = std::max(max_eig, e);
    const double clamp = max_eig * 1e-6;
    std::vector<float> Tinv((size_t)r * r);
    for (int i = 0; i < r; ++i)
      for (int c = 0; c < r; ++c) {
        double s = 0.0;
        for (int k = 0; k < r; ++k)
          s += V[(size_t)i * r + k] * V[(size_t)c * r + k] / std::sqrt(std::max(ev[k], clamp));
        Tinv[(size_t)i * r + c] = (float)s;
      }
    DevBuf<float> Td;
    Td.ensure(Tinv.size());
    MGP_HIP_CHECK(hipMemcpyAsync(Td.ptr, Tinv.data(), Tinv.size() * sizeof(float),
                                 hipMemcpyHostToDevice, st));
    ps.root.ensure((size_t)r * n);
    gemm_nr_rr(Q.ptr, Td.ptr, n, r, ps.root.ptr, st);
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    ps.rank = r;
  }
};

}  // namespace

void lanczos_inv_root(Provider& pv, int r, PredictState& ps) {
  LanczosSolve l(pv, r);
  while (!l.finished) {
    pv.forward(l.vec(), 1, l.w);
    l.step();
  }
  l.finish(ps);
}

int solve_alpha_and_root(Provider& pv, const float* y_host, float mean, int max_iter, float tol,
                         int rank, PredictState& ps, double* alpha_s, double* root_s) {
  const auto t0 = Clock::now();
  if (!pv.column_independent_products()) {
    const int its = solve_alpha(pv, y_host, mean, max_iter, tol, ps);
    *alpha_s = secs_since(t0);
    const auto t1 = Clock::now();
    lanczos_inv_root(pv, rank, ps);
    *root_s = secs_since(t1);
    return its;
  }
  const int64_t n = pv.n;
  DevBuf<float> V2, O2;  // [p | v_j] and [A p | A v_j]
  V2.ensure((size_t)2 * n);
  O2.ensure((size_t)2 * n);
  AlphaSolve a(pv, y_host, mean, max_iter, tol, ps, V2.ptr, O2.ptr);
  LanczosSolve l(pv, rank, O2.ptr + n);
  *alpha_s = 0.0;
  while (!a.finished || !l.finished) {
    if (!a.finished && !l.finished) {
      copy(V2.ptr + n, l.vec(), n, pv.st);
      pv.forward(V2.ptr, 2, O2.ptr);
      a.step();
      if (a.finished) *alpha_s = secs_since(t0);
      l.step();
    } else if (!a.finished) {
      pv.forward(a.p, 1, a.Ap);
      a.step();
      if (a.finished) *alpha_s = secs_since(t0);
    } else {
      pv.forward(l.vec(), 1, l.w);
      l.step();
    }
  }
  MGP_HIP_CHECK(hipStreamSynchronize(pv.st));
  if (*alpha_s == 0.0) *alpha_s = secs_since(t0);
  ps.has_alpha = true;
  l.finish(ps);
  *root_s = std::max(0.0, secs_since(t0) - *alpha_s);
  return a.it;
}

namespace {
__global__ void k_exact_var(const double* __restrict__ dots, int C, float diag,
                            const float* __restrict__ dvec, float* __restrict__ var) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < C) var[c] = fmaxf((dvec ? dvec[c] : diag) - (float)dots[c], 1e-10f);
}
}  // namespace

// Reference: predict_variance_exact_jit / run_exact_variance_blocks_jit /
// solve_exact_cross_block_jit (jit_prediction.mojo:1357-1789).
void exact_variance(Provider& pv, int64_t m, const ExactVarianceOptions& o, float* var_dev,
                    ExactVarianceStats& stats) {
  hipStream_t st = pv.st;
  const int64_t n = pv.n;
  MGP_REQUIRE(pv.test.n == m, "test set is not packed");
  // choose_exact_prediction_block_cols (:1357-1386)
  int64_t block = 0;
  if (o.block_cols > 0) block = std::min<int64_t>(o.block_cols, m);
  else if (pv.materialized) block = m;
  else block = std::min<int64_t>(m, 512);
  stats = ExactVarianceStats{};
  stats.block_cols = (int)block;
  // Nystrom preconditioner (build_pivoted_cholesky_precond_unified defaults:
  // method 2, error_tol 1e-3, adaptive_tol 0.01, seed 42).
  Precond P;
  PivotOptions po;
  po.method = 2;
  po.error_tol = 1e-3f;
  build_precond(pv, o.precond_rank, po, P);
  stats.precond_rank = P.rank;
  const int nb = reduction_chunks(n);
  DevBuf<float> Kc, norms, rhsb;
  DevBuf<double> part, dots;
  CGWork w;
  const float os = pv.kdiag();
  DevBuf<float> dself;  // per-test-point k(x*, x*) of non-stationary trees
  if (pv.nonstationary()) pv.diag_values(pv.test, m, dself.ensure((size_t)m));
  for (int64_t s0 = 0; s0 < m; s0 += block) {
    const int C = (int)std::min<int64_t>(block, m - s0);
    const size_t nc = (size_t)n * C;
    float* kc = Kc.ensure(nc);
    pv.fill_block(pv.test, s0, C, kc);
    // RHS = normalised cross columns; solve; rescale (solve_exact_cross_block_jit)
    float* rhs = rhsb.ensure(nc);
    copy(rhs, kc, (int64_t)nc, st);
    float* rn = norms.ensure(C);
    double* pt = part.ensure((size_t)C * nb);
    normalize_columns(rhs, n, C, rn, pt, st);
    w.x.ensure(nc);
    const CGResult r = batched_cg(pv, P.rank > 0 ? &P : nullptr, rhs, C, o.max_cg_iter, 0,
                                  o.cg_tol, w, false);
    scale_columns(w.x.ptr, rn, n, C, false, st);
    stats.block_count += 1;
    stats.cg_total_iterations += r.iterations;
    stats.cg_max_iterations = std::max(stats.cg_max_iterations, r.iterations);
    // var = k** - <K_cross, solve>, clamped at 1e-10 (kernel_exact_variance, :235-257)
    double* dd = dots.ensure(C);
    coldot_partial(kc, w.x.ptr, n, C, nb, pt, st);
    coldot_finalize(pt, nb, C, dd, st);
    hipLaunchKernelGGL(k_exact_var, dim3((unsigned)ceil_div(C, 256)), dim3(256), 0, st, dd, C,
                       os, pv.nonstationary() ? dself.ptr + s0 : nullptr, var_dev + s0);
    MGP_HIP_CHECK(hipGetLastError());
  }
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

void predict_from_state(Provider& pv, const PredictState& ps, const float* Xs_host, int64_t m,
                        float mean, int variance_method, float* mean_out, float* var_out,
                        PredictTimes& t, const ExactVarianceOptions* exact,
                        ExactVarianceStats* exact_stats) {
  hipStream_t st = pv.st;
  MGP_REQUIRE(ps.has_alpha, "prediction state has no alpha");
  float* dx = pv.Xs.ensure((size_t)m * pv.d);
  MGP_HIP_CHECK(hipMemcpyAsync(dx, Xs_host, (size_t)m * pv.d * sizeof(float),
                               hipMemcpyHostToDevice, st));
  pv.pack(dx, m, pv.test);
  auto t0 = Clock::now();
  float* dm = pv.io_c.ensure((size_t)m);
  pv.cross(pv.test, ps.alpha.ptr, 1, dm);
  hipLaunchKernelGGL(k_add_scalar, g1(m), dim3(256), 0, st, dm, mean, m);
  MGP_HIP_CHECK(hipMemcpyAsync(mean_out, dm, m * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  t.mean_s = secs_since(t0);
  if (variance_method == 1) {
    MGP_REQUIRE(ps.rank > 0, "LOVE variance needs an inverse root");
    auto t1 = Clock::now();
    DevBuf<float> Vs, var;
    Vs.ensure((size_t)ps.rank * m);
    var.ensure(m);
    pv.cross(pv.test, ps.root.ptr, ps.rank, Vs.ptr);
    DevBuf<float> dv;
    if (pv.nonstationary()) pv.diag_values(pv.test, m, dv.ensure((size_t)m));
    love_variance(Vs.ptr, m, ps.rank, pv.kdiag(), var.ptr, st,
                  pv.nonstationary() ? dv.ptr : nullptr);
    MGP_HIP_CHECK(hipMemcpyAsync(var_out, var.ptr, m * sizeof(float), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    t.variance_s = secs_since(t1);
  } else if (variance_method == 2) {
    auto t1 = Clock::now();
    ExactVarianceOptions eo = exact ? *exact : ExactVarianceOptions{};
    ExactVarianceStats es;
    DevBuf<float> var;
    var.ensure(m);
    exact_variance(pv, m, eo, var.ptr, es);
    MGP_HIP_CHECK(hipMemcpyAsync(var_out, var.ptr, m * sizeof(float), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    if (exact_stats) *exact_stats = es;
    t.variance_s = secs_since(t1);
  }
}

}  // namespace mgp
