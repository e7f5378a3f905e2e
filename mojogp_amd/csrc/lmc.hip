// LMC operator, preconditioner, BBMM evaluation, training loop and mean
// prediction (reference files listed in lmc.h).
#include "lmc.h"

#include <algorithm>
#include <chrono>
#include <cmath>

#include "host_numerics.h"
#include "mixed.h"
#include "tree.h"

namespace mgp {

namespace {

using Clock = std::chrono::steady_clock;
constexpr float kPi = 3.14159265358979f;

dim3 g1(int64_t n) { return dim3((unsigned)ceil_div(std::max<int64_t>(n, 1), 256)); }

// out[c][t][i] (= | +=) sum_j M[t][j] in[c][j][i]   (kernel_lmc_accumulate_batched)
__global__ void k_lmc_mix(float* __restrict__ out, const float* __restrict__ in,
                          const float* __restrict__ M, int64_t n, int T, int C, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nT = n * T;
  if (idx >= nT * C) return;
  const int64_t c = idx / nT, rem = idx - c * nT;
  const int t = (int)(rem / n);
  const int64_t i = rem - (int64_t)t * n;
  const float* col = in + c * nT + i;
  float s = 0.0f;
  for (int j = 0; j < T; ++j) s = fmaf(M[t * T + j], col[(int64_t)j * n], s);
  out[idx] = accumulate ? out[idx] + s : s;
}

// out[c][t][i] = a * out + scale[t] * in   (noise add: a = 1; task scaling: a = 0)
__global__ void k_task_scale(float* __restrict__ out, const float* __restrict__ in,
                             const float* __restrict__ scale, int64_t n, int T, int C, float a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nT = n * T;
  if (idx >= nT * C) return;
  const int t = (int)((idx % nT) / n);
  const float v = scale[t] * in[idx];
  out[idx] = a == 0.0f ? v : fmaf(a, out[idx], v);
}

// rhs[(b*T + t)][t'][j] = sum_s A_s[t'][t] Kc[s][b][j]: the joint cross
// covariance column of test point b, output task t (Kc [R][nb][n]).
__global__ void k_lmc_cross_rhs(const float* __restrict__ Kc, const float* __restrict__ A, int R,
                                int T, int64_t n, int nb, float* __restrict__ rhs) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nT = n * T;
  if (idx >= nT * nb * T) return;
  const int64_t col = idx / nT, rem = idx - col * nT;
  const int b = (int)(col / T), t = (int)(col - (int64_t)b * T);
  const int tp = (int)(rem / n);
  const int64_t j = rem - (int64_t)tp * n;
  float v = 0.0f;
  for (int s = 0; s < R; ++s)
    v = fmaf(A[((int64_t)s * T + tp) * T + t], Kc[((int64_t)s * nb + b) * n + j], v);
  rhs[idx] = v;
}

// out[c][x] += fixed[x] * in[c][x]   (fixed observation noise, x < nT)
__global__ void k_add_fixed(float* __restrict__ out, const float* __restrict__ in,
                            const float* __restrict__ fixed, int64_t nT, int C) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nT * C) return;
  out[idx] = fmaf(fixed[idx % nT], in[idx], out[idx]);
}

// y[c][off + j*r + k] = sum_t Cs[t][j] Y[(c*T + t)*r + k]   (U^T w mixing, fp64
// as the reference's host mixing, lmc_preconditioner.mojo:470-480)
__global__ void k_ut_mix(const float* __restrict__ Y, const float* __restrict__ Cs, int T,
                         int r, int C, int K, int off, double* __restrict__ y) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)C * T * r) return;
  const int c = (int)(idx / ((int64_t)T * r));
  const int rem = (int)(idx - (int64_t)c * T * r);
  const int j = rem / r, k = rem - j * r;
  double s = 0.0;
  for (int t = 0; t < T; ++t) s += (double)Cs[t * T + j] * (double)Y[((int64_t)c * T + t) * r + k];
  y[(int64_t)c * K + off + j * r + k] = s;
}

// z[c][a] = sum_b Minv[a][b] y[c][b] in fp64 (M can be conditioned like
// n / noise, so its inverse is neither stored nor applied in fp32), rounded
// to fp32 for the U z products.  Grid (column, group of 4 outputs): one wave
// per output a, its lanes over b, a fixed-order shuffle sum.  (One thread per
// output walking its row alone took 14 us per call at K = 120.)
__global__ __launch_bounds__(256) void k_small_gemv(const double* __restrict__ Minv,
                                                   const double* __restrict__ y, int K,
                                                   float* __restrict__ z) {
  const int c = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int a = (int)blockIdx.y * 4 + (int)(threadIdx.x >> 6);
  if (a >= K) return;
  const double* yc = y + (int64_t)c * K;
  const double* row = Minv + (int64_t)a * K;
  double s = 0.0;
  for (int b = lane; b < K; b += 64) s = fma(row[b], yc[b], s);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) z[(int64_t)c * K + a] = (float)s;
}

// w[c][t*r + k] = raw[(t*C + c)*r + k]: the Kronecker preconditioner's rank
// draws in its probe-major-per-task order, regrouped per probe
__global__ void k_kron_zrank(const float* __restrict__ raw, int T, int r, int C,
                             float* __restrict__ w) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t K = (int64_t)T * r;
  if (idx >= K * C) return;
  const int64_t c = idx / K, rem = idx - c * K;
  const int64_t t = rem / r, k = rem - t * r;
  w[idx] = raw[(t * C + c) * r + k];
}

// out = w - dinv[t] * res   (Woodbury final step)
__global__ void k_woodbury_lmc(float* __restrict__ out, const float* __restrict__ w,
                               const float* __restrict__ res, const float* __restrict__ dinv,
                               int64_t n, int T, int C) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nT = n * T;
  if (idx >= nT * C) return;
  const int t = (int)((idx % nT) / n);
  out[idx] = w[idx] - dinv[t] * res[idx];
}

// part[b][i*T + j] = sum over chunk b, columns c of a[c][i][x] * b[c][j][x]
__global__ void k_task_pair_dots(const float* __restrict__ a, const float* __restrict__ b,
                                 int64_t n, int T, int C, int nb, double* __restrict__ part) {
  const int pair = blockIdx.y;
  const int i = pair / T, j = pair - i * T;
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t x0 = (int64_t)blockIdx.x * chunk, x1 = min(n, x0 + chunk);
  const int64_t nT = n * T;
  double acc = 0.0;
  for (int c = 0; c < C; ++c) {
    const float* ac = a + c * nT + (int64_t)i * n;
    const float* bc = b + c * nT + (int64_t)j * n;
    float f = 0.0f;
    for (int64_t x = x0 + threadIdx.x; x < x1; x += blockDim.x) f = fmaf(ac[x], bc[x], f);
    acc += (double)f;
  }
  __shared__ double sh[256];
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) sh[threadIdx.x] += sh[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[(int64_t)blockIdx.x * T * T + pair] = sh[0];
}

// mean_out[i][t] = sum over latents accumulated in acc[t][i] + mean[t] (host side)

void check(bool ok, const char* msg) {
  if (!ok) throw Error(ST_INVALID, msg);
}

// T x T helpers (row-major, fp32 as the reference's host loops).
void a_from_l(const float* L, const float* vdiag, int T, float* A) {
  for (int i = 0; i < T; ++i)
    for (int j = 0; j < T; ++j) {
      float v = 0.0f;
      const int mk = std::min(i, j);
      for (int k = 0; k <= mk; ++k) v += L[i * T + k] * L[j * T + k];
      if (i == j && vdiag) v += vdiag[i];
      A[i * T + j] = v;
    }
}

bool chol_t(const float* A, int T, float* C) {
  std::vector<double> c(A, A + (size_t)T * T);
  if (!cholesky(c, T)) return false;
  for (int i = 0; i < T; ++i)
    for (int j = 0; j < T; ++j) C[i * T + j] = j <= i ? (float)c[(size_t)i * T + j] : 0.0f;
  return true;
}

float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

}  // namespace

// ------------------------------------------------------------------ operator
std::vector<float> LMCModel::precond_noise() const {
  std::vector<float> out(noise);
  if (has_fixed())
    for (int t = 0; t < T; ++t) {
      float acc = 0.0f;
      for (int64_t i = 0; i < n; ++i) acc += fixed[(size_t)t * n + i];
      out[t] += acc / (float)n;
    }
  return out;
}

void LMCModel::upload() {
  check((int)A.size() == R * T * T && (int)noise.size() == T, "LMC A / noise sizes");
  check(!has_fixed() || (int64_t)fixed.size() == n * T, "fixed noise must have T*n entries");
  A_dev.ensure(A.size());
  noise_dev.ensure(noise.size());
  MGP_HIP_CHECK(hipMemcpyAsync(A_dev.ptr, A.data(), A.size() * sizeof(float),
                               hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipMemcpyAsync(noise_dev.ptr, noise.data(), noise.size() * sizeof(float),
                               hipMemcpyHostToDevice, st));
  if (has_fixed()) {
    fixed_dev.ensure(fixed.size());
    MGP_HIP_CHECK(hipMemcpyAsync(fixed_dev.ptr, fixed.data(), fixed.size() * sizeof(float),
                                 hipMemcpyHostToDevice, st));
  }
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

void LMCModel::latent_forward(int s, const float* V, int cols, float* out) {
  Provider& pv = *prov[s];
  const float saved = pv.noise;
  pv.noise = 0.0f;
  pv.forward(V, cols, out);
  pv.noise = saved;
}

void LMCModel::forward(const float* V, int C, float* out) {
  const int64_t total = n * T * (int64_t)C;
  // The latents share X and V: the first fused product packs V and the
  // others reuse its packing (all latent providers run on one stream).
  PackedRhs packed;
  for (int s = 0; s < R; ++s) {
    Provider& pv = *prov[s];
    if (pv.fused_route() && T <= 16) {
      // A_s mixing folded into the latent product's split-K reduction
      const float saved = pv.noise;
      pv.noise = 0.0f;
      pv.forward_mixed(V, T * C, A_dev.ptr + s * T * T, T, s > 0, out, &packed);
      pv.noise = saved;
      continue;
    }
    float* t = tmp.ensure((size_t)total);
    latent_forward(s, V, T * C, t);
    hipLaunchKernelGGL(k_lmc_mix, g1(total), dim3(256), 0, st, out, t, A_dev.ptr + s * T * T,
                       n, T, C, s > 0 ? 1 : 0);
  }
  hipLaunchKernelGGL(k_task_scale, g1(total), dim3(256), 0, st, out, V, noise_dev.ptr, n, T, C,
                     1.0f);
  if (has_fixed())
    hipLaunchKernelGGL(k_add_fixed, g1(total), dim3(256), 0, st, out, V, fixed_dev.ptr, n * T, C);
  MGP_HIP_CHECK(hipGetLastError());
}

LMCStreamGuard::LMCStreamGuard(LMCModel& model) : m(model) {
  for (Provider* p : m.prov) {
    saved.push_back(p->st);
    MGP_HIP_CHECK(hipStreamSynchronize(p->st));
    p->set_stream(m.st);
  }
}

LMCStreamGuard::~LMCStreamGuard() {
  (void)hipStreamSynchronize(m.st);
  for (size_t s = 0; s < m.prov.size(); ++s) {
    try {
      m.prov[s]->set_stream(saved[s]);
    } catch (...) {
    }
  }
}

// ------------------------------------------------------------------ preconditioner
void LMCPrecond::build(LMCModel& m, int precond_rank, const PivotOptions& po) {
  R = m.R;
  T = m.T;
  n = m.n;
  K = 0;
  if (precond_rank <= 0) return;
  hipStream_t st = m.st;
  rank.assign(R, 0);
  off.assign(R, 0);
  L.clear();
  for (int s = 0; s < R; ++s) L.push_back(std::make_unique<DevBuf<float>>());
  for (int s = 0; s < R; ++s) {
    Provider& pv = *m.prov[s];
    const float saved = pv.noise;
    pv.noise = 0.0f;  // the reference builds each factor with the noise set to 0
    L[s]->ensure((size_t)precond_rank * n);
    rank[s] = pivoted_cholesky(pv, precond_rank, po, L[s]->ptr, st);
    pv.noise = saved;
    off[s] = K;
    K += rank[s] * T;
  }
  // C_s = chol(A_s) (+1e-4 jitter retry, jit_lmc.mojo:780-788)
  Cs.assign((size_t)R * T * T, 0.0f);
  for (int s = 0; s < R; ++s) {
    std::vector<float> As(m.A.begin() + (size_t)s * T * T, m.A.begin() + (size_t)(s + 1) * T * T);
    if (!chol_t(As.data(), T, &Cs[(size_t)s * T * T])) {
      for (int i = 0; i < T; ++i) As[(size_t)i * T + i] += 1e-4f;
      if (!chol_t(As.data(), T, &Cs[(size_t)s * T * T]))
        throw Error(ST_NUMERIC, "LMC coregionalisation matrix is not positive definite");
    }
  }
  noise = m.precond_noise();
  // LtL blocks and M = I + sum G_{s1 s2} (x) LtL_{s1 s2}  (lmc_preconditioner.mojo:240-330)
  std::vector<double> M((size_t)K * K, 0.0);
  for (int a = 0; a < K; ++a) M[(size_t)a * K + a] = 1.0;
  DevBuf<double> ltl_dev;
  for (int s1 = 0; s1 < R; ++s1)
    for (int s2 = 0; s2 < R; ++s2) {
      const int r1 = rank[s1], r2 = rank[s2];
      if (r1 == 0 || r2 == 0) continue;
      ltl_dev.ensure((size_t)r1 * r2);
      cross_ltl(L[s1]->ptr, r1, L[s2]->ptr, r2, n, ltl_dev.ptr, st);
      std::vector<double> ltl((size_t)r1 * r2);
      MGP_HIP_CHECK(hipMemcpy(ltl.data(), ltl_dev.ptr, ltl.size() * sizeof(double),
                              hipMemcpyDeviceToHost));
      for (int j1 = 0; j1 < T; ++j1)
        for (int j2 = 0; j2 < T; ++j2) {
          double g = 0.0;
          for (int t = 0; t < T; ++t)
            g += (double)Cs[(size_t)s1 * T * T + t * T + j1] *
                 (double)Cs[(size_t)s2 * T * T + t * T + j2] / (double)noise[t];
          for (int k1 = 0; k1 < r1; ++k1)
            for (int k2 = 0; k2 < r2; ++k2) {
              const size_t row = (size_t)off[s1] + (size_t)j1 * r1 + k1;
              const size_t col = (size_t)off[s2] + (size_t)j2 * r2 + k2;
              M[row * K + col] += g * ltl[(size_t)k1 * r2 + k2];
            }
        }
    }
  // Cholesky (jitter 1e-6 retry, identity fallback as the reference), inverse, log|P|.
  std::vector<double> c = M;
  bool ok = cholesky(c, K);
  if (!ok) {
    c = M;
    for (int a = 0; a < K; ++a) c[(size_t)a * K + a] += 1e-6;
    ok = cholesky(c, K);
  }
  std::vector<double> inv((size_t)K * K, 0.0);
  double logdet_m = 0.0;
  if (ok) {
    for (int a = 0; a < K; ++a) logdet_m += 2.0 * std::log(c[(size_t)a * K + a]);
    // inverse from the Cholesky factor: solve L L^T X = I column by column
    std::vector<double> e(K);
    for (int col = 0; col < K; ++col) {
      std::fill(e.begin(), e.end(), 0.0);
      e[col] = 1.0;
      for (int i = 0; i < K; ++i) {
        double v = e[i];
        for (int k = 0; k < i; ++k) v -= c[(size_t)i * K + k] * e[k];
        e[i] = v / c[(size_t)i * K + i];
      }
      for (int i = K - 1; i >= 0; --i) {
        double v = e[i];
        for (int k = i + 1; k < K; ++k) v -= c[(size_t)k * K + i] * e[k];
        e[i] = v / c[(size_t)i * K + i];
      }
      for (int i = 0; i < K; ++i) inv[(size_t)i * K + col] = e[i];
    }
  } else {
    for (int a = 0; a < K; ++a) inv[(size_t)a * K + a] = 1.0;
  }
  double ld = logdet_m;
  for (int t = 0; t < T; ++t) ld += (double)n * std::log((double)noise[t]);
  logdet = (float)ld;
  Minv.ensure(inv.size());
  MGP_HIP_CHECK(hipMemcpy(Minv.ptr, inv.data(), inv.size() * sizeof(double), hipMemcpyHostToDevice));
  std::vector<float> di(T), ds(T);
  for (int t = 0; t < T; ++t) {
    di[t] = 1.0f / noise[t];
    ds[t] = std::sqrt(noise[t]);
  }
  dinv.ensure(T);
  dsqrt.ensure(T);
  Cs_dev.ensure(Cs.size());
  MGP_HIP_CHECK(hipMemcpy(dinv.ptr, di.data(), T * sizeof(float), hipMemcpyHostToDevice));
  MGP_HIP_CHECK(hipMemcpy(dsqrt.ptr, ds.data(), T * sizeof(float), hipMemcpyHostToDevice));
  MGP_HIP_CHECK(hipMemcpy(Cs_dev.ptr, Cs.data(), Cs.size() * sizeof(float), hipMemcpyHostToDevice));
}

// res = U z for C columns:  res[c][t] = sum_s sum_j C_s[t][j] L_s z[c][(s, j, .)]
// (cs: another T x T factor per latent in place of C_s)
static void lmc_u_times(LMCPrecond& P, const float* z, int C, float* res, hipStream_t st,
                        const float* cs = nullptr) {
  const int64_t total = P.n * P.T * (int64_t)C;
  bool first = true;
  for (int s = 0; s < P.R; ++s) {
    const int r = P.rank[s];
    if (r == 0) continue;
    float* ol = P.out_l.ensure((size_t)total);
    // Z[(c T + j) r + k] = z[c K + off + j r + k], read in place
    l_matmul_gather(P.L[s]->ptr, P.n, r, z, P.T, P.K, P.off[s], C * P.T, ol, st);
    hipLaunchKernelGGL(k_lmc_mix, g1(total), dim3(256), 0, st, res, ol,
                       (cs ? cs : P.Cs_dev.ptr) + (size_t)s * P.T * P.T, P.n, P.T, C,
                       first ? 0 : 1);
    first = false;
  }
  if (first) fill(res, total, 0.0f, st);
  MGP_HIP_CHECK(hipGetLastError());
}

void LMCPrecond::apply(const float* r, int C, float* z, double* rz_part, int nb,
                       hipStream_t st) {
  const int64_t nT = n * T, total = nT * C;
  // 1. w = D^-1 r
  float* wv = w.ensure((size_t)total);
  hipLaunchKernelGGL(k_task_scale, g1(total), dim3(256), 0, st, wv, r, dinv.ptr, n, T, C, 0.0f);
  // 2. y = U^T w
  double* yk_ = yk.ensure((size_t)C * K);
  for (int s = 0; s < R; ++s) {
    const int rs = rank[s];
    if (rs == 0) continue;
    float* Ys = Y.ensure((size_t)C * T * rs);
    lt_matmul(L[s]->ptr, n, rs, wv, C * T, Ys, lt_work, st);
    hipLaunchKernelGGL(k_ut_mix, g1((int64_t)C * T * rs), dim3(256), 0, st, Ys,
                       Cs_dev.ptr + (size_t)s * T * T, T, rs, C, K, off[s], yk_);
  }
  // 3. z' = M^-1 y
  float* zk_ = zk.ensure((size_t)C * K);
  hipLaunchKernelGGL(k_small_gemv, dim3(C, (unsigned)ceil_div(K, 4)), dim3(256), 0, st,
                     Minv.ptr, yk_, K, zk_);
  // 4. res = U z'
  float* rs_ = res.ensure((size_t)total);
  lmc_u_times(*this, zk_, C, rs_, st);
  // 5. z = w - D^-1 res
  hipLaunchKernelGGL(k_woodbury_lmc, g1(total), dim3(256), 0, st, z, wv, rs_, dinv.ptr, n, T, C);
  MGP_HIP_CHECK(hipGetLastError());
  if (rz_part) coldot_partial(r, z, nT, C, nb, rz_part, st);
}

void LMCPrecond::sample(float* out, int C, uint64_t seed, hipStream_t st) {
  const int64_t nT = n * T, total = nT * C;
  float* eps = w.ensure((size_t)total);
  gaussian(eps, total, seed + 1000000ull, st);
  float* wr = zk.ensure((size_t)C * K);
  gaussian(wr, (int64_t)C * K, seed, st);
  float* rs_ = res.ensure((size_t)total);
  lmc_u_times(*this, wr, C, rs_, st);
  // out = D^{1/2} eps + U w
  copy(out, rs_, total, st);
  hipLaunchKernelGGL(k_task_scale, g1(total), dim3(256), 0, st, out, eps, dsqrt.ptr, n, T, C,
                     1.0f);
  MGP_HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------ Kronecker preconditioner
void KronPrecond::build_kron(LMCModel& m, int precond_rank, const PivotOptions& po, float os,
                             const std::vector<float>& B, const std::vector<float>& noise_t) {
  R = 1;
  T = m.T;
  n = m.n;
  K = 0;
  check((int)B.size() == T * T && (int)noise_t.size() == T, "Kronecker preconditioner sizes");
  if (precond_rank <= 0) return;
  hipStream_t st = m.st;
  rank.assign(1, 0);
  off.assign(1, 0);
  L.clear();
  L.push_back(std::make_unique<DevBuf<float>>());
  Provider& pv = *m.prov[0];
  const float saved = pv.noise;
  pv.noise = 0.0f;  // factor of the base kernel at noise 0 (jit_multi_output.mojo:287-297)
  L[0]->ensure((size_t)precond_rank * n);
  const int r = pivoted_cholesky(pv, precond_rank, po, L[0]->ptr, st);
  pv.noise = saved;
  rank[0] = r;
  if (r == 0) return;
  K = r * T;
  // L^T L (fp32 as the reference's GPU matmul) and its eigenpairs
  DevBuf<double> ltl_dev;
  ltl_dev.ensure((size_t)r * r);
  cross_ltl(L[0]->ptr, r, L[0]->ptr, r, n, ltl_dev.ptr, st);
  std::vector<double> ltl((size_t)r * r);
  MGP_HIP_CHECK(hipMemcpy(ltl.data(), ltl_dev.ptr, ltl.size() * sizeof(double),
                          hipMemcpyDeviceToHost));
  std::vector<float> ltlf(ltl.begin(), ltl.end()), V((size_t)r * r), Qt((size_t)T * T);
  sigma.assign(r, 0.0f);
  lambda.assign(T, 0.0f);
  jacobi_eigen(ltlf.data(), r, V.data(), sigma.data());
  // B~ = D^-1/2 B D^-1/2 + 1e-6 I and its eigenpairs
  std::vector<float> dis(T), ds(T), Bt((size_t)T * T);
  for (int t = 0; t < T; ++t) {
    check(noise_t[t] > 0.0f, "Kronecker preconditioner needs positive task noise");
    dis[t] = 1.0f / std::sqrt(noise_t[t]);
    ds[t] = std::sqrt(noise_t[t]);
  }
  for (int a = 0; a < T; ++a)
    for (int b = 0; b < T; ++b)
      Bt[(size_t)a * T + b] = dis[a] * B[(size_t)a * T + b] * dis[b] + (a == b ? 1e-6f : 0.0f);
  jacobi_eigen(Bt.data(), T, Qt.data(), lambda.data());
  // C^-1 and log|P| with the reference's clamps (fp32)
  const float clampv = 1e-8f;
  std::vector<float> cinv((size_t)T * r);
  float ld = 0.0f;
  for (int t = 0; t < T; ++t) ld += (float)n * std::log(noise_t[t]);
  for (int j = 0; j < T; ++j) {
    const float lj = std::max(lambda[j], clampv);
    for (int i = 0; i < r; ++i) {
      const float si = std::max(sigma[i], clampv);
      cinv[(size_t)j * r + i] = 1.0f / (1.0f / (os * lj) + si);
      float arg = 1.0f + os * lj * si;
      if (arg <= 0.0f) arg = 1e-10f;
      ld += std::log(arg);
    }
  }
  logdet = ld;
  // Inner matrix (Q~ (x) V) diag(C^-1) (Q~ (x) V)^T, index t*r + k, in fp64:
  // H_j = V diag(C^-1[j][.]) V^T, then sum_j Q~[t][j] Q~[t'][j] H_j.
  std::vector<double> inner((size_t)K * K, 0.0), H((size_t)r * r);
  for (int j = 0; j < T; ++j) {
    for (int k1 = 0; k1 < r; ++k1)
      for (int k2 = 0; k2 < r; ++k2) {
        double h = 0.0;
        for (int i = 0; i < r; ++i)
          h += (double)V[(size_t)k1 * r + i] * (double)V[(size_t)k2 * r + i] *
               (double)cinv[(size_t)j * r + i];
        H[(size_t)k1 * r + k2] = h;
      }
    for (int t1 = 0; t1 < T; ++t1)
      for (int t2 = 0; t2 < T; ++t2) {
        const double q = (double)Qt[(size_t)t1 * T + j] * (double)Qt[(size_t)t2 * T + j];
        if (q == 0.0) continue;
        for (int k1 = 0; k1 < r; ++k1) {
          double* row = inner.data() + ((size_t)t1 * r + k1) * K + (size_t)t2 * r;
          const double* hr = H.data() + (size_t)k1 * r;
          for (int k2 = 0; k2 < r; ++k2) row[k2] += q * hr[k2];
        }
      }
  }
  Minv.ensure(inner.size());
  MGP_HIP_CHECK(hipMemcpy(Minv.ptr, inner.data(), inner.size() * sizeof(double),
                          hipMemcpyHostToDevice));
  // U = D^1/2 (x) L for the shared Woodbury apply; C_B for the probes
  noise = noise_t;
  Cs.assign((size_t)T * T, 0.0f);
  for (int t = 0; t < T; ++t) Cs[(size_t)t * T + t] = ds[t];
  Cb.assign((size_t)T * T, 0.0f);
  const float sos = std::sqrt(os);
  for (int a = 0; a < T; ++a)
    for (int j = 0; j < T; ++j)
      Cb[(size_t)a * T + j] =
          sos * ds[a] * Qt[(size_t)a * T + j] * std::sqrt(std::max(lambda[j], clampv));
  std::vector<float> di(T);
  for (int t = 0; t < T; ++t) di[t] = 1.0f / noise_t[t];
  dinv.ensure(T);
  dsqrt.ensure(T);
  Cs_dev.ensure(Cs.size());
  Cb_dev.ensure(Cb.size());
  MGP_HIP_CHECK(hipMemcpy(dinv.ptr, di.data(), T * sizeof(float), hipMemcpyHostToDevice));
  MGP_HIP_CHECK(hipMemcpy(dsqrt.ptr, ds.data(), T * sizeof(float), hipMemcpyHostToDevice));
  MGP_HIP_CHECK(hipMemcpy(Cs_dev.ptr, Cs.data(), Cs.size() * sizeof(float), hipMemcpyHostToDevice));
  MGP_HIP_CHECK(hipMemcpy(Cb_dev.ptr, Cb.data(), Cb.size() * sizeof(float), hipMemcpyHostToDevice));
}

void KronPrecond::sample(float* out, int C, uint64_t seed, hipStream_t st) {
  const int64_t nT = n * T, total = nT * C;
  float* eps = w.ensure((size_t)total);
  gaussian(eps, total, seed + 12345ull, st);
  float* raw = zraw.ensure((size_t)C * K);
  gaussian(raw, (int64_t)C * K, seed, st);
  float* wr = zk.ensure((size_t)C * K);
  hipLaunchKernelGGL(k_kron_zrank, g1((int64_t)C * K), dim3(256), 0, st, raw, T, rank[0], C, wr);
  float* rs_ = res.ensure((size_t)total);
  lmc_u_times(*this, wr, C, rs_, st, Cb_dev.ptr);
  copy(out, rs_, total, st);
  hipLaunchKernelGGL(k_task_scale, g1(total), dim3(256), 0, st, out, eps, dsqrt.ptr, n, T, C,
                     1.0f);
  MGP_HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------ BBMM
LMCEval lmc_bbmm(LMCModel& m, LMCPrecond* P, const float* y_c, int num_probes, int max_cg,
                 int max_tridiag, float tol, int iteration, bool recycle, LMCWork& w) {
  hipStream_t st = m.st;
  const int64_t N = m.size();
  const int Pn = num_probes;
  const int C = 1 + Pn;
  const size_t nP = (size_t)N * Pn, nC = (size_t)N * C;
  const bool pre = P && P->active();
  const uint64_t seed = (uint64_t)((int64_t)iteration * 104729 + 42);
  const int nb = reduction_chunks(N);

  float* probes = w.probes.ensure(std::max<size_t>(nP, 1));
  float* pn = w.probe_norms.ensure(std::max(Pn, 1));
  float* rn = w.rhs_norms.ensure(C);
  double* part = w.part.ensure((size_t)std::max(C, m.T * m.T) * std::max(nb, 64) + 64);
  if (Pn > 0) {
    if (pre) P->sample(probes, Pn, seed, st);
    else gaussian(probes, (int64_t)nP, seed, st);
    normalize_columns(probes, N, Pn, pn, part, st);
  }
  float* rhs = w.rhs.ensure(nC);
  copy(rhs, y_c, N, st);
  if (Pn > 0) copy(rhs + N, probes, nP, st);
  normalize_columns(rhs, N, C, rn, part, st);

  CGOperator op;
  op.n = N;
  op.st = st;
  op.matvec = [&m](const float* V, int ncols, float* out) { m.forward(V, ncols, out); };
  if (pre)
    op.precond = [P, st](const float* r, int ncols, float* z, double* rzp, int nb) {
      P->apply(r, ncols, z, rzp, nb, st);
    };
  const bool warm = recycle && iteration > 0 && w.has_x && w.cg.x.count >= nC;
  if (!warm) w.cg.x.ensure(nC);
  if (warm && C > 1) fill(w.cg.x.ptr + N, (int64_t)N * (C - 1), 0.0f, st);
  CGResult cg = batched_cg(op, rhs, C, max_cg, max_tridiag, tol, w.cg, warm);
  w.has_x = true;

  float* sol = w.sol.ensure(nC);
  copy(sol, w.cg.x.ptr, nC, st);
  scale_columns(sol, rn, N, C, false, st);

  LMCEval out;
  out.cg_iterations = cg.iterations;
  out.converged = cg.converged;
  out.cg_loop_ms = cg.loop_ms;
  {
    coldot_partial(y_c, sol, N, 1, nb, part, st);
    coldot_finalize(part, nb, 1, part + nb, st);
    double iq = 0.0;
    MGP_HIP_CHECK(hipMemcpyAsync(&iq, part + nb, sizeof(double), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    out.inv_quad = (float)iq;
  }
  float logdet = 0.0f;
  if (cg.tridiag_size > 0 && Pn > 0) {
    std::vector<std::vector<float>> pd(cg.diag.begin() + 1, cg.diag.end());
    std::vector<std::vector<float>> po(cg.offdiag.begin() + 1, cg.offdiag.end());
    logdet = slq_logdet(pd, po, N);
    if (pre) logdet += P->logdet;
  }
  out.logdet = logdet;
  const float constant = 0.5f * (float)N * std::log(2.0f * kPi);
  out.nll = (0.5f * out.inv_quad + 0.5f * logdet + constant) / (float)N;

  // Factors Lf = [-alpha/2 | (0.5/P) u], Rf = [alpha | P^-1 (Z_norm * norms)].
  std::vector<float> norms(std::max(Pn, 1), 1.0f);
  if (Pn > 0)
    MGP_HIP_CHECK(hipMemcpyAsync(norms.data(), pn, Pn * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  std::vector<float> lfac(C), rfac(C);
  lfac[0] = -0.5f;
  rfac[0] = 1.0f;
  for (int j = 0; j < Pn; ++j) {
    lfac[1 + j] = (0.5f / (float)Pn) * norms[j];
    rfac[1 + j] = norms[j];
  }
  float* facs = w.facs.ensure(2 * (size_t)C);
  std::vector<float> hfac(lfac);
  hfac.insert(hfac.end(), rfac.begin(), rfac.end());
  MGP_HIP_CHECK(hipMemcpyAsync(facs, hfac.data(), 2 * C * sizeof(float), hipMemcpyHostToDevice, st));
  float* lf = w.lf.ensure(nC);
  float* rf = w.rf.ensure(nC);
  copy(lf, sol, nC, st);
  scale_columns(lf, facs, N, C, false, st);
  copy(rf, sol, N, st);
  if (Pn > 0) {
    copy(rf + N, probes, nP, st);
    scale_columns(rf + N, facs + C + 1, N, Pn, false, st);
    if (pre) P->apply(rf + N, Pn, rf + N, nullptr, 0, st);
  }
  // Kernel-parameter gradients per latent: tr((A_s (x) dK_s) Rf Lf^T) =
  // sum over (column, task) of Lf_{c,t}^T dK_s (A_s Rf_c)_t.
  const int T = m.T;
  const int64_t n = m.n;
  float* rfm = w.rfm.ensure(nC);
  float* krf = w.krf.ensure(nC);
  out.G_A.assign((size_t)m.R * T * T, 0.0f);
  for (int s = 0; s < m.R; ++s) {
    Provider& pv = *m.prov[s];
    hipLaunchKernelGGL(k_lmc_mix, g1((int64_t)nC), dim3(256), 0, st, rfm, rf,
                       m.A_dev.ptr + (size_t)s * T * T, n, T, C, 0);
    std::vector<double> g(pv.nparams, 0.0);
    gradient_traces(pv, lf, rfm, C * T, g.data(), st);
    for (int q = 0; q < pv.nparams; ++q) {
      float gq = (float)(g[q] / (double)N);
      if (!std::isfinite(gq)) gq = 0.0f;
      out.kernel_grads.push_back(gq);
    }
    // A_s gradients: G_A[s][i][j] = (1/N) sum_c Lf_{c,i} . (K_s Rf_c)_j  (jit_lmc.mojo:582-660)
    m.latent_forward(s, rf, C * T, krf);
    const int nbp = std::min<int>(reduction_chunks(n), 64);
    hipLaunchKernelGGL(k_task_pair_dots, dim3(nbp, T * T), dim3(256), 0, st, lf, krf, n, T, C,
                       nbp, part);
    std::vector<double> hp((size_t)nbp * T * T);
    MGP_HIP_CHECK(hipMemcpyAsync(hp.data(), part, hp.size() * sizeof(double),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    for (int pr = 0; pr < T * T; ++pr) {
      double acc = 0.0;
      for (int b = 0; b < nbp; ++b) acc += hp[(size_t)b * T * T + pr];
      float v = (float)(acc / (double)N);
      out.G_A[(size_t)s * T * T + pr] = std::isfinite(v) ? v : 0.0f;
    }
  }
  // Per-task noise gradients: (1/N) sum_c Lf_{c,t} . Rf_{c,t}  (jit_lmc.mojo:662-690)
  {
    const int nbp = std::min<int>(reduction_chunks(n), 64);
    hipLaunchKernelGGL(k_task_pair_dots, dim3(nbp, T * T), dim3(256), 0, st, lf, rf, n, T, C,
                       nbp, part);
    std::vector<double> hp((size_t)nbp * T * T);
    MGP_HIP_CHECK(hipMemcpyAsync(hp.data(), part, hp.size() * sizeof(double),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    out.noise_grads.assign(T, 0.0f);
    for (int t = 0; t < T; ++t) {
      double acc = 0.0;
      for (int b = 0; b < nbp; ++b) acc += hp[(size_t)b * T * T + t * T + t];
      float v = (float)(acc / (double)N);
      out.noise_grads[t] = std::isfinite(v) ? v : 0.0f;
    }
  }
  out.alpha.resize((size_t)N);
  MGP_HIP_CHECK(hipMemcpyAsync(out.alpha.data(), sol, N * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return out;
}

// ------------------------------------------------------------------ training
LMCTrainResult lmc_train(LMCModel& m, const float* y_blocked_host,
                         const std::vector<std::vector<float>>& init_params,
                         const std::vector<std::vector<char>>& trainable,
                         const std::vector<float>& init_noise,
                         const std::vector<float>& init_mean, const LMCTrainOptions& o) {
  const int R = m.R, T = m.T, TT = T * T;
  const int64_t n = m.n, nT = n * T;
  check((int)init_params.size() == R && (int)trainable.size() == R, "per-latent params mismatch");
  check((int)init_noise.size() == T && (int)init_mean.size() == T, "per-task arrays mismatch");
  check(o.max_iterations >= 1, "max_iterations must be >= 1");
  hipStream_t st = m.st;
  LMCStreamGuard guard(m);

  std::vector<int> np(R);
  int total_kp = 0;
  std::vector<std::vector<float>> raw(R);
  for (int s = 0; s < R; ++s) {
    np[s] = (int)init_params[s].size();
    check(np[s] == m.prov[s]->nparams, "initial params length does not match the provider");
    check((int)trainable[s].size() == np[s], "trainable mask length does not match the provider");
    total_kp += np[s];
    for (float v : init_params[s]) raw[s].push_back(inv_softplus(v));
  }
  std::vector<float> raw_noise(T), raw_mean(init_mean);
  for (int t = 0; t < T; ++t) raw_noise[t] = inv_softplus(init_noise[t]);

  // L_s: diag sqrt(1/R) (softplus-parameterised), strictly lower 0.01 (s+1)/R.
  const float init_diag = std::sqrt(1.0f / (float)R);
  std::vector<float> Lall((size_t)R * TT, 0.0f), raw_Ld((size_t)R * T), raw_vd((size_t)R * T);
  for (int s = 0; s < R; ++s)
    for (int i = 0; i < T; ++i) {
      for (int j = 0; j < T; ++j) {
        float v = 0.0f;
        if (i == j) v = init_diag;
        else if (j < i) v = 0.01f * (float)(s + 1) / (float)R;
        Lall[(size_t)s * TT + i * T + j] = v;
      }
      raw_Ld[(size_t)s * T + i] = inv_softplus(init_diag);
    }
  std::fill(raw_vd.begin(), raw_vd.end(), inv_softplus(0.1f));

  const int total_adam = total_kp + T + R * TT + R * T + T;
  std::vector<float> madam(total_adam, 0.0f), vadam(total_adam, 0.0f);
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f, clipv = 10.0f;
  int t_step = 0;

  // Host copies
  std::vector<float> y_orig(y_blocked_host, y_blocked_host + nT), yh((size_t)nT);
  DevBuf<float> ydev;
  ydev.ensure(nT);

  LMCTrainResult res;
  LMCWork work;
  LMCPrecond Pc;
  const bool use_pre = o.precond_rank > 0;
  const PivotOptions po = training_pivot_options(o.precond_method);

  std::vector<float> last_rb((size_t)total_kp), last_rb_noise(init_noise);
  {
    int q = 0;
    for (int s = 0; s < R; ++s)
      for (int p = 0; p < np[s]; ++p) last_rb[q++] = init_params[s][p];
  }
  // last-good / best snapshots
  auto good_raw = raw;
  auto good_noise = raw_noise, good_mean = raw_mean;
  auto good_L = Lall, good_Ld = raw_Ld, good_vd = raw_vd;
  int nan_count = 0;
  float last_good_nll = 1e10f, best_nll = 1e30f;
  auto best_raw = raw;
  auto best_noise = raw_noise, best_mean = raw_mean;
  auto best_L = Lall, best_Ld = raw_Ld, best_vd = raw_vd;
  std::vector<float> best_alpha((size_t)nT, 0.0f);
  float nll_smoothed = 1e10f;
  int patience = 0;

  auto adam = [&](int idx, float g) {
    const float mm = b1 * madam[idx] + (1.0f - b1) * g;
    const float vv = b2 * vadam[idx] + (1.0f - b2) * g * g;
    madam[idx] = mm;
    vadam[idx] = vv;
    const float mh = mm / (1.0f - pow_float32(b1, t_step));
    const float vh = vv / (1.0f - pow_float32(b2, t_step));
    return -o.learning_rate * mh / (std::sqrt(vh) + eps);
  };
  auto clip = [&](float g) { return g > clipv ? clipv : (g < -clipv ? -clipv : g); };

  for (int it = 0; it < o.max_iterations; ++it) {
    res.iterations = it + 1;
    ++t_step;
    const auto t0 = Clock::now();
    // Constrained values into the providers.
    for (int s = 0; s < R; ++s) {
      Provider& pv = *m.prov[s];
      for (int p = 0; p < np[s]; ++p) pv.params[p] = softplus(raw[s][p]);
      pv.noise = 0.0f;
      pv.refresh_coords();
    }
    std::vector<float> cur_noise(T);
    for (int t = 0; t < T; ++t) cur_noise[t] = softplus(raw_noise[t]);
    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < n; ++i) yh[(size_t)t * n + i] = y_orig[(size_t)t * n + i] - raw_mean[t];
    MGP_HIP_CHECK(hipMemcpyAsync(ydev.ptr, yh.data(), nT * sizeof(float), hipMemcpyHostToDevice, st));
    // A_s = L_s L_s^T + diag(softplus(raw_vd))
    m.A.assign((size_t)R * TT, 0.0f);
    for (int s = 0; s < R; ++s) {
      std::vector<float> vd(T);
      for (int i = 0; i < T; ++i) {
        vd[i] = softplus(raw_vd[(size_t)s * T + i]);
        Lall[(size_t)s * TT + i * T + i] = softplus(raw_Ld[(size_t)s * T + i]);
      }
      a_from_l(&Lall[(size_t)s * TT], vd.data(), T, &m.A[(size_t)s * TT]);
      // A_s keeps a 1e-4 diagonal jitter when its Cholesky fails (jit_lmc.mojo:1032-1036).
      std::vector<float> cs((size_t)TT);
      if (!chol_t(&m.A[(size_t)s * TT], T, cs.data()))
        for (int i = 0; i < T; ++i) m.A[(size_t)s * TT + i * T + i] += 1e-4f;
    }
    m.noise = cur_noise;
    m.upload();

    bool rebuild = it == 0;
    if (!rebuild) {
      float max_rel = 0.0f;
      int q = 0;
      for (int s = 0; s < R; ++s)
        for (int p = 0; p < np[s]; ++p, ++q) {
          const float cv = softplus(raw[s][p]);
          max_rel = std::max(max_rel, std::fabs(cv - last_rb[q]) / (std::fabs(last_rb[q]) + 1e-8f));
        }
      for (int t = 0; t < T; ++t)
        max_rel = std::max(max_rel, std::fabs(cur_noise[t] - last_rb_noise[t]) /
                                        (std::fabs(last_rb_noise[t]) + 1e-8f));
      rebuild = max_rel > o.precond_rebuild_threshold;
    }
    if (rebuild) {
      if (it > 0) ++res.precond_rebuild_count;
      if (use_pre) Pc.build(m, o.precond_rank, po);
      int q = 0;
      for (int s = 0; s < R; ++s)
        for (int p = 0; p < np[s]; ++p) last_rb[q++] = softplus(raw[s][p]);
      last_rb_noise = cur_noise;
    } else if (use_pre) {
      // The reference keeps the factors and refreshes C_s / noise with the
      // current A_s only at rebuilds; the operator itself always uses the
      // current A_s and noise.
    }

    LMCEval ev = lmc_bbmm(m, use_pre ? &Pc : nullptr, ydev.ptr, o.num_probes, o.max_cg_iter,
                          o.max_tridiag_iter, o.cg_tol, it, it > 0 && !rebuild, work);
    const float nll = ev.nll;
    res.nll_history.push_back(nll);

    if (std::isnan(nll)) {
      ++nan_count;
      work.has_x = false;
      std::fill(last_rb.begin(), last_rb.end(), 0.0f);  // force a rebuild
      raw = good_raw;
      raw_noise = good_noise;
      raw_mean = good_mean;
      Lall = good_L;
      raw_Ld = good_Ld;
      const float bump = 0.7f * (float)nan_count;
      for (size_t q = 0; q < raw_vd.size(); ++q) {
        raw_vd[q] = good_vd[q] + bump;
        good_vd[q] = raw_vd[q];
      }
      res.iter_times_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
      continue;
    }
    if (nll < best_nll) {
      best_nll = nll;
      best_raw = raw;
      best_noise = raw_noise;
      best_mean = raw_mean;
      best_L = Lall;
      best_Ld = raw_Ld;
      best_vd = raw_vd;
      best_alpha = ev.alpha;
    }
    // Adam updates (jit_lmc.mojo:1233-1300).
    int ai = 0;
    {
      int off = 0;
      for (int s = 0; s < R; ++s) {
        for (int p = 0; p < np[s]; ++p) {
          if (trainable[s][p]) {
            const float g = clip(ev.kernel_grads[off + p]) * sigmoid(raw[s][p]);
            raw[s][p] += adam(ai, g);
          }
          ++ai;
        }
        off += np[s];
      }
    }
    for (int t = 0; t < T; ++t) {
      const float g = clip(ev.noise_grads[t]) * sigmoid(raw_noise[t]);
      raw_noise[t] += adam(ai, g);
      ++ai;
    }
    for (int s = 0; s < R; ++s)
      for (int i = 0; i < T; ++i) {
        for (int j = 0; j <= i; ++j) {
          float g = 0.0f;
          for (int b = 0; b < T; ++b)
            g += ev.G_A[(size_t)s * TT + i * T + b] * Lall[(size_t)s * TT + b * T + j];
          g = clip(2.0f * g);
          if (i == j) {
            raw_Ld[(size_t)s * T + i] += adam(ai, g * sigmoid(raw_Ld[(size_t)s * T + i]));
          } else {
            Lall[(size_t)s * TT + i * T + j] += adam(ai, g);
          }
          ++ai;
        }
        ai += T - 1 - i;  // upper triangle: no gradient
      }
    for (int s = 0; s < R; ++s)
      for (int i = 0; i < T; ++i) {
        const float g = clip(ev.G_A[(size_t)s * TT + i * T + i]) * sigmoid(raw_vd[(size_t)s * T + i]);
        raw_vd[(size_t)s * T + i] += adam(ai, g);
        ++ai;
      }
    for (int t = 0; t < T; ++t) {
      float g = 0.0f;
      for (int64_t i = 0; i < n; ++i) g -= ev.alpha[(size_t)t * n + i];
      g = clip(g / (float)nT);
      raw_mean[t] += adam(ai, g);
      ++ai;
    }
    // Last-good snapshot.
    const float drop = last_good_nll - nll;
    if (drop < 2.0f || it < 3) {
      nan_count = 0;
      last_good_nll = nll;
      good_raw = raw;
      good_noise = raw_noise;
      good_mean = raw_mean;
      good_L = Lall;
      good_Ld = raw_Ld;
      good_vd = raw_vd;
    }
    // Early stopping on the smoothed NLL.
    const float prev = nll_smoothed;
    nll_smoothed = it == 0 ? nll : 0.9f * nll_smoothed + 0.1f * nll;
    res.iter_times_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
    if (it > 20 && o.early_stop_tol > 0.0f) {
      const float rel = (prev - nll_smoothed) / (std::fabs(nll_smoothed) + 1e-8f);
      if (rel < o.early_stop_tol && rel > -0.1f) {
        if (++patience >= o.early_stop_patience) {
          res.converged = true;
          break;
        }
      } else {
        patience = 0;
      }
    }
  }

  // Package the best state (jit_lmc.mojo:1405-1470).
  res.params.resize(R);
  for (int s = 0; s < R; ++s)
    for (int p = 0; p < np[s]; ++p) res.params[s].push_back(softplus(best_raw[s][p]));
  res.noise.resize(T);
  for (int t = 0; t < T; ++t) res.noise[t] = softplus(best_noise[t]);
  res.mean = best_mean;
  res.L = best_L;
  res.var_diag.resize((size_t)R * T);
  res.A.assign((size_t)R * TT, 0.0f);
  for (int s = 0; s < R; ++s) {
    for (int i = 0; i < T; ++i) {
      res.L[(size_t)s * TT + i * T + i] = softplus(best_Ld[(size_t)s * T + i]);
      res.var_diag[(size_t)s * T + i] = softplus(best_vd[(size_t)s * T + i]);
    }
    a_from_l(&res.L[(size_t)s * TT], &res.var_diag[(size_t)s * T], T, &res.A[(size_t)s * TT]);
  }
  res.alpha = best_alpha;
  res.final_nll = best_nll < 1e29f ? best_nll : 0.0f;
  // Providers keep the best parameters (noise 0), as the reference leaves them.
  for (int s = 0; s < R; ++s) {
    Provider& pv = *m.prov[s];
    pv.params = res.params[s];
    pv.noise = 0.0f;
    pv.refresh_coords();
  }
  m.A = res.A;
  m.noise = res.noise;
  m.upload();
  return res;
}

// ------------------------------------------------------------------ mixed training
LMCMixedResult lmc_train_mixed(LMCModel& m, const float* y_blocked_host,
                               const std::vector<std::vector<float>>& init_params,
                               const std::vector<std::vector<int>>& cat_kinds,
                               const std::vector<std::vector<float>>& init_cat_raw,
                               const std::vector<float>& init_noise,
                               const std::vector<float>& init_mean, const LMCTrainOptions& o) {
  const int R = m.R, T = m.T, TT = T * T;
  const int64_t n = m.n, nT = n * T;
  check((int)init_params.size() == R && (int)cat_kinds.size() == R &&
            (int)init_cat_raw.size() == R,
        "per-latent arrays mismatch");
  check((int)init_noise.size() == T && (int)init_mean.size() == T, "per-task arrays mismatch");
  check(o.max_iterations >= 1, "max_iterations must be >= 1");
  check(o.num_probes >= 0, "num_probes must be >= 0");
  hipStream_t st = m.st;
  LMCStreamGuard guard(m);

  std::vector<int> np(R);
  int total_kp = 0;
  std::vector<std::vector<float>> raw(R), rcat(init_cat_raw);
  std::vector<std::vector<CatLeafRef>> cl(R);
  for (int s = 0; s < R; ++s) {
    Provider& pv = *m.prov[s];
    np[s] = (int)init_params[s].size();
    check(np[s] == pv.nparams, "initial params length does not match the provider");
    total_kp += np[s];
    for (float v : init_params[s]) raw[s].push_back(inv_softplus(v));
    if (cat_kinds[s].empty()) {
      check(rcat[s].empty(), "categorical parameters given for a latent without categorical kinds");
      check(!pv.is_tree || pv.tree.ncat == 0,
            "a latent with categorical leaves needs one categorical kind per leaf");
      continue;
    }
    check(pv.is_tree, "categorical parameters need a kernel-tree latent");
    cl[s] = cat_leaves(pv, cat_kinds[s]);
    size_t K = 0;
    for (const auto& c : cl[s]) K += (size_t)c.nparam;
    check(rcat[s].size() == K, "categorical parameter count does not match the leaves");
    for (float v : rcat[s]) check(std::isfinite(v), "categorical parameters must be finite");
  }
  std::vector<float> raw_noise(T), raw_mean(init_mean);
  for (int t = 0; t < T; ++t) raw_noise[t] = inv_softplus(init_noise[t]);

  // L_s, var_diag and A_s as lmc_train (jit_lmc_mixed.mojo:850-900).
  const float init_diag = std::sqrt(1.0f / (float)R);
  std::vector<float> Lall((size_t)R * TT, 0.0f), raw_Ld((size_t)R * T), raw_vd((size_t)R * T);
  for (int s = 0; s < R; ++s)
    for (int i = 0; i < T; ++i) {
      for (int j = 0; j < T; ++j)
        Lall[(size_t)s * TT + i * T + j] =
            i == j ? init_diag : (j < i ? 0.01f * (float)(s + 1) / (float)R : 0.0f);
      raw_Ld[(size_t)s * T + i] = inv_softplus(init_diag);
    }
  std::fill(raw_vd.begin(), raw_vd.end(), inv_softplus(0.1f));
  auto set_A = [&]() {
    m.A.assign((size_t)R * TT, 0.0f);
    std::vector<float> vd(T), cs((size_t)TT);
    for (int s = 0; s < R; ++s) {
      for (int i = 0; i < T; ++i) {
        vd[i] = softplus(raw_vd[(size_t)s * T + i]);
        Lall[(size_t)s * TT + i * T + i] = softplus(raw_Ld[(size_t)s * T + i]);
      }
      a_from_l(&Lall[(size_t)s * TT], vd.data(), T, &m.A[(size_t)s * TT]);
      if (!chol_t(&m.A[(size_t)s * TT], T, cs.data()))
        for (int i = 0; i < T; ++i) m.A[(size_t)s * TT + i * T + i] += 1e-4f;
    }
  };
  auto constrained_cat = [&](int s) {
    std::vector<float> out;
    std::vector<double> th;
    for (const auto& c : cl[s]) {
      th.resize((size_t)c.nparam);
      cat_constrain(c.kind, c.L, rcat[s].data() + c.param_off, c.nparam, th.data(), nullptr);
      for (double v : th) out.push_back((float)v);
    }
    return out;
  };

  // Adam: one moment array for the continuous parameters in the reference's
  // order, one per latent for the categorical ones, a shared step count.
  const int total_adam = total_kp + T + R * TT + R * T + T;
  std::vector<float> madam(total_adam, 0.0f), vadam(total_adam, 0.0f);
  std::vector<std::vector<float>> mcat(R), vcat(R);
  for (int s = 0; s < R; ++s) {
    mcat[s].assign(rcat[s].size(), 0.0f);
    vcat[s].assign(rcat[s].size(), 0.0f);
  }
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f, clipv = 10.0f;
  int t_step = 0;
  auto adam = [&](float* mm, float* vv, int idx, float g) {
    const float a = b1 * mm[idx] + (1.0f - b1) * g;
    const float b = b2 * vv[idx] + (1.0f - b2) * g * g;
    mm[idx] = a;
    vv[idx] = b;
    const float mh = a / (1.0f - pow_float32(b1, t_step));
    const float vh = b / (1.0f - pow_float32(b2, t_step));
    return -o.learning_rate * mh / (std::sqrt(vh) + eps);
  };
  auto clip = [&](float g) { return g > clipv ? clipv : (g < -clipv ? -clipv : g); };

  std::vector<float> y_orig(y_blocked_host, y_blocked_host + nT), yh((size_t)nT);
  DevBuf<float> ydev, rfc, rfcm;
  ydev.ensure(nT);

  LMCMixedResult res;
  LMCWork work;
  LMCPrecond Pc;
  const bool use_pre = o.precond_rank > 0;
  const PivotOptions po = training_pivot_options(o.precond_method);

  // State of the last preconditioner build (jit_lmc_mixed.mojo:950-972).
  std::vector<float> last_kp, last_noise(init_noise), last_A;
  for (int s = 0; s < R; ++s) last_kp.insert(last_kp.end(), init_params[s].begin(), init_params[s].end());
  std::vector<std::vector<float>> last_cat(R);
  for (int s = 0; s < R; ++s) last_cat[s] = constrained_cat(s);
  set_A();
  last_A = m.A;

  float best_nll = 1e30f;
  auto best_raw = raw, best_cat = rcat;
  auto best_noise = raw_noise, best_mean = raw_mean;
  auto best_L = Lall, best_Ld = raw_Ld, best_vd = raw_vd;
  std::vector<float> best_alpha((size_t)nT, 0.0f);
  int patience = 0;

  for (int it = 0; it < o.max_iterations; ++it) {
    res.iterations = it + 1;
    ++t_step;
    const auto t0 = Clock::now();
    for (int s = 0; s < R; ++s) {
      Provider& pv = *m.prov[s];
      for (int p = 0; p < np[s]; ++p) pv.params[p] = softplus(raw[s][p]);
      pv.noise = 0.0f;
      if (cl[s].empty()) pv.refresh_coords();
      else set_categorical_raw(pv, cat_kinds[s], rcat[s].data(), (int)rcat[s].size());
    }
    std::vector<float> cur_noise(T);
    for (int t = 0; t < T; ++t) cur_noise[t] = softplus(raw_noise[t]);
    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < n; ++i) yh[(size_t)t * n + i] = y_orig[(size_t)t * n + i] - raw_mean[t];
    MGP_HIP_CHECK(hipMemcpyAsync(ydev.ptr, yh.data(), nT * sizeof(float), hipMemcpyHostToDevice, st));
    set_A();
    m.noise = cur_noise;
    m.upload();

    // Rebuild when anything the preconditioner holds moved by more than the
    // threshold, relative to its last build (jit_lmc_mixed.mojo:1060-1108).
    float max_rel = 0.0f;
    auto watch = [&](float cur, float prev) {
      max_rel = std::max(max_rel, std::fabs(cur - prev) / (std::fabs(prev) + 1e-8f));
    };
    {
      int q = 0;
      for (int s = 0; s < R; ++s)
        for (int p = 0; p < np[s]; ++p) watch(softplus(raw[s][p]), last_kp[q++]);
    }
    std::vector<std::vector<float>> cur_cat(R);
    for (int s = 0; s < R; ++s) {
      cur_cat[s] = constrained_cat(s);
      for (size_t k = 0; k < cur_cat[s].size(); ++k) watch(cur_cat[s][k], last_cat[s][k]);
    }
    for (size_t i = 0; i < m.A.size(); ++i) watch(m.A[i], last_A[i]);
    for (int t = 0; t < T; ++t) watch(cur_noise[t], last_noise[t]);
    const bool moved = max_rel > o.precond_rebuild_threshold;
    if (it == 0 || moved) {
      // iteration 0 builds from the initial state, as the reference does
      // before its loop
      if (moved) ++res.precond_rebuild_count;
      if (use_pre) Pc.build(m, o.precond_rank, po);
      int q = 0;
      for (int s = 0; s < R; ++s)
        for (int p = 0; p < np[s]; ++p) last_kp[q++] = softplus(raw[s][p]);
      last_cat = cur_cat;
      last_A = m.A;
      last_noise = cur_noise;
    }

    LMCEval ev = lmc_bbmm(m, use_pre ? &Pc : nullptr, ydev.ptr, o.num_probes, o.max_cg_iter,
                          o.max_tridiag_iter, o.cg_tol, it, it > 0 && !moved, work);
    const float nll = ev.nll;
    res.nll_history.push_back(nll);
    if (std::isnan(nll)) {  // jit_lmc_mixed.mojo:1191-1215: the run ends
      res.iter_times_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
      break;
    }
    if (nll < best_nll) {
      best_nll = nll;
      patience = 0;
      best_raw = raw;
      best_cat = rcat;
      best_noise = raw_noise;
      best_mean = raw_mean;
      best_L = Lall;
      best_Ld = raw_Ld;
      best_vd = raw_vd;
      best_alpha = ev.alpha;
    }

    // Categorical gradients (jit_lmc_mixed.mojo:1259-1327): for dK = A_s (x)
    // dK_s/dtheta_k, (-0.5 alpha^T dK alpha + (0.5/P) sum_j u_j^T dK zn_j) / N
    // with u_j the probe solutions at the raw probe scale and zn_j the
    // unit-norm probes.  The evaluation's left factors are
    // Lf = [-alpha/2 | (0.5/P) u_j]; with Rf = [alpha | zn_j] mixed by A_s
    // one tree pass over the C*T columns gives the per-entry sums G.
    const int C = 1 + o.num_probes;
    bool have_rf = false;
    for (int s = 0; s < R; ++s) {
      if (cl[s].empty()) continue;
      Provider& pv = *m.prov[s];
      if (!have_rf) {
        float* rf = rfc.ensure((size_t)nT * C);
        copy(rf, work.sol.ptr, nT, st);
        if (o.num_probes > 0) copy(rf + nT, work.probes.ptr, nT * o.num_probes, st);
        have_rf = true;
      }
      float* rfm = rfcm.ensure((size_t)nT * C);
      hipLaunchKernelGGL(k_lmc_mix, g1(nT * C), dim3(256), 0, st, rfm, rfc.ptr,
                         m.A_dev.ptr + (size_t)s * TT, n, T, C, 0);
      MGP_HIP_CHECK(hipGetLastError());
      std::vector<double> G((size_t)pv.tree.table_size, 0.0);
      tree_cat_grad_tables(pv.tree, pv.tparams.ptr, pv.train.z.ptr, n, work.lf.ptr, rfm, C * T,
                           G.data(), pv.tree_gws, st);
      std::vector<float> g(rcat[s].size());
      cat_raw_gradients(cl[s], rcat[s].data(), G, 1.0 / (double)nT, clipv, g.data());
      for (size_t k = 0; k < g.size(); ++k)
        rcat[s][k] += adam(mcat[s].data(), vcat[s].data(), (int)k, g[k]);
    }

    // Continuous parameters (jit_lmc_mixed.mojo:1329-1372).
    int ai = 0;
    {
      int off = 0;
      for (int s = 0; s < R; ++s) {
        for (int p = 0; p < np[s]; ++p, ++ai)
          raw[s][p] += adam(madam.data(), vadam.data(), ai,
                            clip(ev.kernel_grads[off + p]) * sigmoid(raw[s][p]));
        off += np[s];
      }
    }
    for (int t = 0; t < T; ++t, ++ai)
      raw_noise[t] += adam(madam.data(), vadam.data(), ai,
                           clip(ev.noise_grads[t]) * sigmoid(raw_noise[t]));
    for (int s = 0; s < R; ++s)
      for (int i = 0; i < T; ++i) {
        for (int j = 0; j <= i; ++j, ++ai) {
          float g = 0.0f;
          for (int b = 0; b < T; ++b)
            g += ev.G_A[(size_t)s * TT + i * T + b] * Lall[(size_t)s * TT + b * T + j];
          g = clip(2.0f * g);
          if (i == j)
            raw_Ld[(size_t)s * T + i] +=
                adam(madam.data(), vadam.data(), ai, g * sigmoid(raw_Ld[(size_t)s * T + i]));
          else
            Lall[(size_t)s * TT + i * T + j] += adam(madam.data(), vadam.data(), ai, g);
        }
        ai += T - 1 - i;
      }
    for (int s = 0; s < R; ++s)
      for (int i = 0; i < T; ++i, ++ai)
        raw_vd[(size_t)s * T + i] +=
            adam(madam.data(), vadam.data(), ai,
                 clip(ev.G_A[(size_t)s * TT + i * T + i]) * sigmoid(raw_vd[(size_t)s * T + i]));
    for (int t = 0; t < T; ++t, ++ai) {
      float g = 0.0f;
      for (int64_t i = 0; i < n; ++i) g -= ev.alpha[(size_t)t * n + i];
      raw_mean[t] += adam(madam.data(), vadam.data(), ai, clip(g / (float)nT));
    }
    res.iter_times_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
    // Patience (jit_lmc_mixed.mojo:1375-1380): after iteration 20 every
    // evaluation not below the best counts, the one that just set it included.
    if (nll >= best_nll && it > 20 && o.early_stop_tol > 0.0f && ++patience >= o.early_stop_patience) {
      res.converged = true;
      break;
    }
  }

  // Best state, constrained (jit_lmc_mixed.mojo:1440-1500); the providers keep
  // it (noise 0) with their tables at the best categorical parameters.
  res.params.resize(R);
  for (int s = 0; s < R; ++s)
    for (int p = 0; p < np[s]; ++p) res.params[s].push_back(softplus(best_raw[s][p]));
  res.cat_raw = best_cat;
  res.noise.resize(T);
  for (int t = 0; t < T; ++t) res.noise[t] = softplus(best_noise[t]);
  res.mean = best_mean;
  res.L = best_L;
  res.var_diag.resize((size_t)R * T);
  res.A.assign((size_t)R * TT, 0.0f);
  for (int s = 0; s < R; ++s) {
    for (int i = 0; i < T; ++i) {
      res.L[(size_t)s * TT + i * T + i] = softplus(best_Ld[(size_t)s * T + i]);
      res.var_diag[(size_t)s * T + i] = softplus(best_vd[(size_t)s * T + i]);
    }
    a_from_l(&res.L[(size_t)s * TT], &res.var_diag[(size_t)s * T], T, &res.A[(size_t)s * TT]);
  }
  res.alpha = best_alpha;
  res.final_nll = best_nll < 1e29f ? best_nll : 0.0f;
  for (int s = 0; s < R; ++s) {
    Provider& pv = *m.prov[s];
    pv.params = res.params[s];
    pv.noise = 0.0f;
    if (cl[s].empty()) pv.refresh_coords();
    else set_categorical_raw(pv, cat_kinds[s], best_cat[s].data(), (int)best_cat[s].size());
  }
  m.A = res.A;
  m.noise = res.noise;
  m.upload();
  return res;
}

// ------------------------------------------------------------------ prediction
void lmc_cross_mix(LMCModel& m, const float* alpha_dev, int C, int64_t mtest, float* out_dev) {
  hipStream_t st = m.st;
  const int T = m.T;
  const int64_t total = mtest * T * (int64_t)C;
  float* cross = m.tmp.ensure((size_t)std::max<int64_t>(total, m.n * T * (int64_t)C));
  for (int s = 0; s < m.R; ++s) {
    Provider& pv = *m.prov[s];
    pv.cross(pv.test, alpha_dev, T * C, cross);  // [C][T][m]
    hipLaunchKernelGGL(k_lmc_mix, g1(total), dim3(256), 0, st, out_dev, cross,
                       m.A_dev.ptr + (size_t)s * T * T, mtest, T, C, s > 0 ? 1 : 0);
  }
  MGP_HIP_CHECK(hipGetLastError());
}

void lmc_predict_mean(LMCModel& m, const float* alpha_dev, int64_t mtest,
                      const std::vector<float>& mean, float* out_host) {
  LMCStreamGuard guard(m);
  hipStream_t st = m.st;
  const int T = m.T;
  DevBuf<float> acc;
  acc.ensure((size_t)mtest * T);
  lmc_cross_mix(m, alpha_dev, 1, mtest, acc.ptr);
  std::vector<float> h((size_t)mtest * T);
  MGP_HIP_CHECK(hipMemcpyAsync(h.data(), acc.ptr, h.size() * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  for (int t = 0; t < T; ++t)
    for (int64_t i = 0; i < mtest; ++i)
      out_host[(size_t)i * T + t] = h[(size_t)t * mtest + i] + mean[t];
}

int lmc_exact_variance(LMCModel& m, int64_t mtest, int max_cg, float tol, int block,
                       float* var_host) {
  check(mtest >= 1 && max_cg >= 1, "exact variance needs >= 1 test point and CG iteration");
  LMCStreamGuard guard(m);
  hipStream_t st = m.st;
  const int R = m.R, T = m.T;
  const int64_t n = m.n, N = m.size();
  int nb = block > 0 ? block : 512;
  nb = (int)std::min<int64_t>(nb, mtest);
  // prior diagonal: sum_s A_s[t][t] k_s(x*, x*) = sum_s A_s[t][t] os_s
  std::vector<double> prior(T, 0.0);
  for (int s = 0; s < R; ++s)
    for (int t = 0; t < T; ++t)
      prior[t] += (double)m.A[((size_t)s * T + t) * T + t] * (double)m.prov[s]->kdiag();
  CGOperator op;
  op.n = N;
  op.st = st;
  op.matvec = [&m](const float* V, int ncols, float* out) { m.forward(V, ncols, out); };
  DevBuf<float> Kc, rhs, beta;
  DevBuf<double> part, dots;
  int total_its = 0;
  for (int64_t b0 = 0; b0 < mtest; b0 += nb) {
    const int bn = (int)std::min<int64_t>(nb, mtest - b0);
    const int C = bn * T;
    Kc.ensure((size_t)R * bn * n);
    for (int s = 0; s < R; ++s) {
      Provider& pv = *m.prov[s];
      pv.fill_block(pv.test, b0, bn, Kc.ptr + (size_t)s * bn * n);
    }
    rhs.ensure((size_t)C * N);
    beta.ensure((size_t)C * N);
    hipLaunchKernelGGL(k_lmc_cross_rhs, g1((int64_t)C * N), dim3(256), 0, st, Kc.ptr, m.A_dev.ptr,
                       R, T, n, bn, rhs.ptr);
    MGP_HIP_CHECK(hipGetLastError());
    total_its += solve_columns(op, rhs.ptr, C, max_cg, tol, beta.ptr);
    const int nbc = reduction_chunks(N);
    part.ensure((size_t)C * nbc);
    dots.ensure((size_t)C);
    coldot_partial(rhs.ptr, beta.ptr, N, C, nbc, part.ptr, st);
    coldot_finalize(part.ptr, nbc, C, dots.ptr, st);
    std::vector<double> hd((size_t)C);
    MGP_HIP_CHECK(hipMemcpyAsync(hd.data(), dots.ptr, C * sizeof(double), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    for (int i = 0; i < bn; ++i)
      for (int t = 0; t < T; ++t) {
        const double v = prior[t] - hd[(size_t)i * T + t] + (double)m.noise[t];
        var_host[(size_t)(b0 + i) * T + t] = (float)std::max(v, 1e-10);
      }
  }
  return total_its;
}

int lmc_pathwise_correction(LMCModel& m, const float* resid_dev, int S, int64_t mtest,
                            int max_cg, float tol, float* corr_host) {
  check(S >= 1 && mtest >= 1, "pathwise correction needs >= 1 sample and test point");
  LMCStreamGuard guard(m);
  hipStream_t st = m.st;
  const int T = m.T;
  const int64_t N = m.size();
  CGOperator op;
  op.n = N;
  op.st = st;
  op.matvec = [&m](const float* V, int ncols, float* out) { m.forward(V, ncols, out); };
  DevBuf<float> beta, acc;
  beta.ensure((size_t)N * S);
  const int its = solve_columns(op, resid_dev, S, max_cg, tol, beta.ptr);
  acc.ensure((size_t)mtest * T * S);
  lmc_cross_mix(m, beta.ptr, S, mtest, acc.ptr);
  std::vector<float> h((size_t)mtest * T * S);
  MGP_HIP_CHECK(hipMemcpyAsync(h.data(), acc.ptr, h.size() * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  for (int c = 0; c < S; ++c)
    for (int t = 0; t < T; ++t)
      for (int64_t i = 0; i < mtest; ++i)
        corr_host[((size_t)c * mtest + i) * T + t] = h[((size_t)c * T + t) * mtest + i];
  return its;
}

}  // namespace mgp
