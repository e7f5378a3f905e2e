// Solver device kernels (see solver.h).  Reference behaviour is cited per
// kernel; reductions use a fixed chunk partition and fp64 partial sums so every
// result is bit-reproducible run to run.
#include "solver.h"

#include <functional>

#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <cmath>
#include <vector>

namespace mgp {

namespace {

constexpr int kBlock = 256;
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double block_sum_d(double v, double* sm) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sm[w] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0)
    for (int k = 0; k < (int)(blockDim.x >> 6); ++k) t += sm[k];
  return t;  // valid in thread 0
}

__device__ __forceinline__ bool is_nan(float x) { return x != x; }

inline dim3 grid1(int64_t count) {
  return dim3((unsigned)std::max<int64_t>(1, ceil_div(count, kBlock)));
}

// ------------------------------------------------------------- reductions
__global__ void k_coldot_final(const double* __restrict__ part, int nb, int ncols,
                               double* __restrict__ out) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncols) return;
  double s = 0.0;
  for (int b = 0; b < nb; ++b) s += part[(int64_t)c * nb + b];
  out[c] = s;
}

__device__ __forceinline__ float part_sum_f(const double* part, int c, int nb) {
  double s = 0.0;
  for (int b = 0; b < nb; ++b) s += part[(int64_t)c * nb + b];
  return (float)s;
}

// Fixed-order fp64 sum of part[c*nb + b] over b by one wave: lane l sums
// b = l, l + 64, ... in order, then a butterfly of shuffles (every lane adds
// the same two operands at each level, so all lanes hold the same total).
__device__ __forceinline__ double wave_part_sum(const double* part, int c, int nb) {
  const int lane = threadIdx.x & 63;
  const double* pc = part + (int64_t)c * nb;
  double s = 0.0;
  int b = lane;
  // eight independent loads in flight, added in the same order as one by one
  for (; b + 7 * 64 < nb; b += 8 * 64) {
    double t[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) t[q] = pc[b + 64 * q];
#pragma unroll
    for (int q = 0; q < 8; ++q) s += t[q];
  }
  for (; b < nb; b += 64) s += pc[b];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  return s;
}

// ------------------------------------------------------------- CG scalars
// One wave per (chunk b = blockIdx.x, column c = blockIdx.y); 4 consecutive
// elements per lane per step when vec4 (n and the chunk length multiples of
// 4, so quads never straddle a chunk or column boundary).
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// part[c*nb + b] = sum_{i in chunk b} a[c][i] b[c][i] (fp64)
__global__ __launch_bounds__(64) void k_coldot_w(const float* __restrict__ a,
                                                 const float* __restrict__ bv, int64_t n, int nb,
                                                 int vec4, double* __restrict__ part) {
  const int c = blockIdx.y, lane = threadIdx.x;
  const int64_t chunk = cg_chunk_rows(n, nb);
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const float* ac = a + (int64_t)c * n;
  const float* bc = bv + (int64_t)c * n;
  double acc = 0.0;
  if (vec4) {
    for (int64_t i = i0 + 4 * lane; i < i1; i += 256) {
      const f4v x = *reinterpret_cast<const f4v*>(ac + i), y = *reinterpret_cast<const f4v*>(bc + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc += (double)x[e] * (double)y[e];
    }
  } else {
    for (int64_t i = i0 + lane; i < i1; i += 64) acc += (double)ac[i] * (double)bc[i];
  }
  acc = wave_sum_d(acc);
  if (lane == 0) part[(int64_t)c * nb + blockIdx.x] = acc;
}

// alpha_c = safe(rz_old_c / sum of the pAp partials) (cg_solver.mojo:181-209),
// then x += alpha p, r -= alpha Ap with the reference skip rules
// (cg_solver.mojo:138-179) and rr partials of the updated r.  One wave per
// (group of G consecutive chunks, column c): each wave forms alpha itself
// with the fixed-order wave sum of the partials (every wave obtains the same
// value), the first wave of the column stores it; chunk partials are summed
// per chunk exactly as one wave per chunk would.
__global__ __launch_bounds__(64) void k_cg_update_w(float* __restrict__ x, float* __restrict__ r,
                                                    const float* __restrict__ p,
                                                    const float* __restrict__ Ap, int64_t n,
                                                    int nb, int G, int vec4,
                                                    const double* __restrict__ pap_part,
                                                    CGScalars s, double* __restrict__ rr_part) {
  const int c = blockIdx.y, lane = threadIdx.x;
  const float pap = (float)wave_part_sum(pap_part, c, nb);
  const float rz = s.rz_old[c];
  const float a = (is_nan(rz) || is_nan(pap) || pap < 1e-10f) ? 0.0f : rz / pap;
  if (blockIdx.x == 0 && lane == 0) s.alpha[c] = a;
  const bool active = !(a == 0.0f || is_nan(a));
  const int64_t chunk = cg_chunk_rows(n, nb);
  const int64_t off = (int64_t)c * n;
  const int b0 = blockIdx.x * G, b1 = min(nb, b0 + G);
  for (int bb = b0; bb < b1; ++bb) {
    const int64_t i0 = (int64_t)bb * chunk, i1 = min(n, i0 + chunk);
    double acc = 0.0;
    auto one = [&](float& xi, float& ri, float pi, float api) __attribute__((always_inline)) {
      if (active && !is_nan(pi) && !is_nan(api)) {
        xi += a * pi;
        ri -= a * api;
      }
      acc += (double)ri * (double)ri;
    };
    if (vec4) {
      for (int64_t i = i0 + 4 * lane; i < i1; i += 256) {
        f4v xv = *reinterpret_cast<const f4v*>(x + off + i);
        f4v rv = *reinterpret_cast<const f4v*>(r + off + i);
        const f4v pv = *reinterpret_cast<const f4v*>(p + off + i);
        const f4v av = *reinterpret_cast<const f4v*>(Ap + off + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float xi = xv[e], ri = rv[e];
          one(xi, ri, pv[e], av[e]);
          xv[e] = xi;
          rv[e] = ri;
        }
        if (active) {
          *reinterpret_cast<f4v*>(x + off + i) = xv;
          *reinterpret_cast<f4v*>(r + off + i) = rv;
        }
      }
    } else {
      for (int64_t i = i0 + lane; i < i1; i += 64) {
        float xi = x[off + i], ri = r[off + i];
        one(xi, ri, p[off + i], Ap[off + i]);
        if (active) {
          x[off + i] = xi;
          r[off + i] = ri;
        }
      }
    }
    acc = wave_sum_d(acc);
    if (lane == 0) rr_part[(int64_t)c * nb + bb] = acc;
  }
}

// beta_c = safe(rz_new_c / rz_old_c) from the rz partials, rz_next_c = rz_new_c
// (cg_solver.mojo:211-255; rz_old and rz_next are distinct arrays, swapped
// by the caller between iterations, so no wave reads a value another wave
// of this launch writes), the alpha / beta history slot `iter` when
// iter < max_tridiag, then p = z + beta p (cg_solver.mojo:108-136).  One wave
// per (group of G consecutive chunks, column c), beta formed by every wave
// with the same fixed-order sum and stored by the column's first wave.
__global__ __launch_bounds__(64) void k_cg_pupdate_w(float* __restrict__ p,
                                                     const float* __restrict__ z, int64_t n,
                                                     int nb, int G, int vec4,
                                                     const double* __restrict__ rz_part,
                                                     int ncols, CGScalars s, int iter,
                                                     int max_tridiag) {
  const int c = blockIdx.y, lane = threadIdx.x;
  const float rz_new = (float)wave_part_sum(rz_part, c, nb);
  const float rz_old = s.rz_old[c];
  float b = 0.0f;
  if (!is_nan(rz_old) && !is_nan(rz_new) && rz_old >= 1e-20f) {
    b = rz_new / (rz_old + 1e-20f);
    if (b < 0.0f || is_nan(b)) b = 0.0f;
  }
  if (blockIdx.x == 0 && lane == 0) {
    s.beta[c] = b;
    s.rz_next[c] = is_nan(rz_new) ? 0.0f : rz_new;
    if (iter < max_tridiag) {
      s.hist_alpha[(int64_t)iter * ncols + c] = s.alpha[c];
      s.hist_beta[(int64_t)iter * ncols + c] = b;
    }
  }
  const bool plain = (b == 0.0f || is_nan(b));
  const int64_t chunk = cg_chunk_rows(n, nb);
  const int64_t off = (int64_t)c * n;
  auto one = [&](float po, float zi) __attribute__((always_inline)) -> float {
    return (plain || is_nan(po)) ? zi : zi + b * po;
  };
  const int64_t i0 = (int64_t)blockIdx.x * G * chunk, i1 = min(n, i0 + G * chunk);
  if (vec4) {
    for (int64_t i = i0 + 4 * lane; i < i1; i += 256) {
      f4v pv = *reinterpret_cast<const f4v*>(p + off + i);
      const f4v zv = *reinterpret_cast<const f4v*>(z + off + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) pv[e] = one(pv[e], zv[e]);
      *reinterpret_cast<f4v*>(p + off + i) = pv;
    }
  } else {
    for (int64_t i = i0 + lane; i < i1; i += 64) p[off + i] = one(p[off + i], z[off + i]);
  }
}

// One wave (grid = 1, 64 threads): mean over columns of sqrt(sum of partials).
__global__ void k_mean_resnorm(const double* __restrict__ rr_part, int nb, int ncols,
                               float* __restrict__ out) {
  float sum = 0.0f;
  for (int c = 0; c < ncols; ++c) sum += sqrtf((float)wave_part_sum(rr_part, c, nb));
  if (threadIdx.x == 0) out[0] = ncols > 0 ? sum / (float)ncols : 0.0f;
}

// ------------------------------------------------------------- vectors
__global__ void k_fill(float* x, int64_t count, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) x[i] = v;
}
__global__ void k_copy(float* __restrict__ d, const float* __restrict__ s, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) d[i] = s[i];
}
__global__ void k_sub(float* y, const float* a, const float* b, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) y[i] = a[i] - b[i];
}
__global__ void k_sub_scalar(float* y, const float* x, float s, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) y[i] = x[i] - s;
}
__global__ void k_scale_columns(float* x, const float* __restrict__ scale, int64_t n,
                                int ncols, int divide) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * ncols) return;
  const float s = scale[idx / n];
  x[idx] = divide ? x[idx] / s : x[idx] * s;
}
__global__ void k_norms_final(const double* __restrict__ part, int nb, int ncols,
                              float* __restrict__ norms) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < ncols) norms[c] = sqrtf(part_sum_f(part, c, nb));
}

// ------------------------------------------------------------- RNG
__global__ void k_gaussian(float* __restrict__ out, int64_t len, uint64_t seed) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= len) return;
  const uint64_t k = (uint64_t)idx + 1ull;
  uint64_t s1 = k * 6364136223846793005ull + seed;
  s1 ^= s1 >> 33;
  s1 *= 0xff51afd7ed558ccdull;
  s1 ^= s1 >> 33;
  uint64_t s2 = k * 1442695040888963407ull + seed + 0xBEEFull;
  s2 ^= s2 >> 33;
  s2 *= 0xc4ceb9fe1a85ec53ull;
  s2 ^= s2 >> 33;
  const float u1 = ((float)(int64_t)(s1 & 0x7FFFFFull) + 1.0f) / 8388608.0f;
  const float u2 = (float)(int64_t)(s2 & 0xFFFFFFull) / 16777216.0f;
  out[idx] = sqrtf(-2.0f * logf(u1)) * cosf(2.0f * 3.14159265f * u2);
}

// ------------------------------------------------------------- pivoted Cholesky
// Argmax of the residual diagonal over unmasked rows with the reference's
// lowest-index tie rule (pivoted_cholesky.mojo:500-610), plus sum |diag|.
struct ArgmaxAcc {
  float val;
  int64_t idx;
};
__device__ __forceinline__ ArgmaxAcc amax_merge(ArgmaxAcc a, ArgmaxAcc b) {
  if (b.val > a.val || (b.val == a.val && b.idx >= 0 && (a.idx < 0 || b.idx < a.idx)))
    return b;
  return a;
}

__device__ void block_argmax_write(ArgmaxAcc loc, double abss, float* pv, int64_t* pi,
                                   double* pa, int slot) {
  __shared__ float sv[kBlock];
  __shared__ int64_t si[kBlock];
  __shared__ double sm[4];
  const double tabs = block_sum_d(abss, sm);
  sv[threadIdx.x] = loc.val;
  si[threadIdx.x] = loc.idx;
  __syncthreads();
  for (int st = kBlock / 2; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      ArgmaxAcc a{sv[threadIdx.x], si[threadIdx.x]};
      ArgmaxAcc b{sv[threadIdx.x + st], si[threadIdx.x + st]};
      ArgmaxAcc m = amax_merge(a, b);
      sv[threadIdx.x] = m.val;
      si[threadIdx.x] = m.idx;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[slot] = sv[0];
    pi[slot] = si[0];
    pa[slot] = tabs;
  }
}

__global__ void k_pc_init(float* __restrict__ diag, float* __restrict__ mask, int64_t n,
                          float os) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    diag[i] = os;
    mask[i] = 1.0f;
  }
}

__global__ void k_pc_argmax_part(const float* __restrict__ diag,
                                 const float* __restrict__ mask, int64_t n, int nb,
                                 float* pv, int64_t* pi, double* pa) {
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  ArgmaxAcc loc{-1e30f, -1};
  double abss = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    if (mask[i] > 0.5f) {
      const float d = diag[i];
      loc = amax_merge(loc, ArgmaxAcc{d, i});
      abss += (double)fabsf(d);
    }
  }
  block_argmax_write(loc, abss, pv, pi, pa, blockIdx.x);
}

struct PivotDev {
  int stopped;
  int rank;
  int64_t pivot;
  float maxval;
  float sumabs;
};

__global__ void k_pc_select(const float* __restrict__ pv, const int64_t* __restrict__ pi,
                            const double* __restrict__ pa, int nb, int m,
                            PivotDev* __restrict__ state, float* __restrict__ mask,
                            const float* __restrict__ L, int64_t n,
                            float* __restrict__ coef) {
  __shared__ int64_t piv_s;
  __shared__ int stop_s;
  if (threadIdx.x == 0) {
    stop_s = state->stopped;
    if (!stop_s) {
      ArgmaxAcc best{pv[0], pi[0]};
      double tot = pa[0];
      for (int b = 1; b < nb; ++b) {
        best = amax_merge(best, ArgmaxAcc{pv[b], pi[b]});
        tot += pa[b];
      }
      if (best.val < 1e-10f || best.idx < 0) {
        state->stopped = 1;
        state->rank = m > 0 ? m : 1;
        stop_s = 1;
      } else {
        state->pivot = best.idx;
        state->maxval = best.val;
        state->sumabs = (float)tot;
        mask[best.idx] = 0.0f;
        piv_s = best.idx;
      }
    }
  }
  __syncthreads();
  if (stop_s) return;
  const int64_t p = piv_s;
  for (int j = threadIdx.x; j < m; j += blockDim.x) coef[j] = L[(int64_t)j * n + p];
}

// Host-driven selection: merge the argmax/abs-sum partials into `state`.
__global__ void k_pc_reduce(const float* __restrict__ pv, const int64_t* __restrict__ pi,
                            const double* __restrict__ pa, int nb,
                            PivotDev* __restrict__ state) {
  if (threadIdx.x != 0) return;
  ArgmaxAcc best{pv[0], pi[0]};
  double tot = pa[0];
  for (int b = 1; b < nb; ++b) {
    best = amax_merge(best, ArgmaxAcc{pv[b], pi[b]});
    tot += pa[b];
  }
  state->stopped = 0;
  state->pivot = best.idx;
  state->maxval = best.val;
  state->sumabs = (float)tot;
}

// Host-driven selection: install the chosen pivot, mask it and gather the
// coefficients L[j][p] of the previous columns.
__global__ void k_pc_setpivot(PivotDev* __restrict__ state, float* __restrict__ mask,
                              const float* __restrict__ L, int64_t n, int m,
                              float* __restrict__ coef, int64_t p, float maxval) {
  if (threadIdx.x == 0) {
    state->stopped = 0;
    state->pivot = p;
    state->maxval = maxval;
    mask[p] = 0.0f;
  }
  for (int j = threadIdx.x; j < m; j += blockDim.x) coef[j] = L[(int64_t)j * n + p];
}

// Pivot-column kernel values: radial kinds read scaled coordinates (z rows);
// kernel trees read raw coordinates.
// lim = the exponent limit exp2_limit(kind, ard) (used by Matern-1/2; the
// RBF exponent is never clamped, the Matern-3/2 and 5/2 ones always).
template <int KIND>
struct RadialColumn {
  float os;
  int d;
  float lim;
  __device__ float operator()(const float* __restrict__ zi, const float* zp) const {
    float r2 = 0.0f;
    for (int k = 0; k < d; ++k) {
      const float df = zi[k] - zp[k];
      r2 = fmaf(df, df, r2);
    }
    if constexpr (KIND == KIND_RBF) {
      return os * __builtin_amdgcn_exp2f(-fmaxf(r2, 0.0f));
    } else if constexpr (KIND == KIND_MATERN12) {
      const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
      return os * __builtin_amdgcn_exp2f(-fminf(u, lim));
    } else if constexpr (KIND == KIND_MATERN32) {
      const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
      return os * fmaf(u, kLn2, 1.0f) * __builtin_amdgcn_exp2f(-fminf(u, kExp2Clamp));
    } else {
      const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
      const float e = __builtin_amdgcn_exp2f(-fminf(u, kExp2Clamp));
      return os * fmaf(u, fmaf(u, kLn2 * kLn2 / 3.0f, kLn2), 1.0f) * e;
    }
  }
};

struct TreeColumn {
  KernelTree t;
  const float* p;
  __device__ float operator()(const float* __restrict__ xi_g, const float* xp) const {
    float xi[kTreeMaxInputDim];
    for (int k = 0; k < t.d; ++k) xi[k] = xi_g[k];
    return tree_value(t, p, xi, xp);
  }
};

template <class Eval>
__global__ __launch_bounds__(256) void k_pc_column(
    Eval ev, const float* __restrict__ Z, int d, int64_t n, int m,
    float* __restrict__ L, float* __restrict__ diag, const float* __restrict__ mask,
    const float* __restrict__ coef, const PivotDev* __restrict__ state, int nb,
    float* pv, int64_t* pi, double* pa) {
  extern __shared__ float sh[];  // coef[m] then zp[d]
  if (state->stopped) return;    // uniform across the grid
  const int64_t p = state->pivot;
  const float scale = 1.0f / sqrtf(fmaxf(state->maxval, 1e-10f));
  float* scoef = sh;
  float* zp = sh + m;
  for (int j = threadIdx.x; j < m; j += blockDim.x) scoef[j] = coef[j];
  for (int k = threadIdx.x; k < d; k += blockDim.x) zp[k] = Z[p * d + k];
  __syncthreads();
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  ArgmaxAcc loc{-1e30f, -1};
  double abss = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float kv = ev(Z + i * d, zp);
    float sum = 0.0f;
    for (int j = 0; j < m; ++j) sum += scoef[j] * L[(int64_t)j * n + i];
    const float v = (kv - sum) * scale;
    L[(int64_t)m * n + i] = v;
    if (mask[i] > 0.5f) {
      const float dn = diag[i] - v * v;
      diag[i] = dn;
      loc = amax_merge(loc, ArgmaxAcc{dn, i});
      abss += (double)fabsf(dn);
    }
  }
  block_argmax_write(loc, abss, pv, pi, pa, blockIdx.x);
}

// M[a][b] partial over a row split; grid (tiles, tiles, splits), 16x16 threads.
// wt (optional): per-row weight applied to the a side, M = L^T diag(wt) L.
__global__ void k_syrk_part(const float* __restrict__ L, int64_t n, int k, int splits,
                            double* __restrict__ part, const float* __restrict__ wt) {
  __shared__ float ta[16][65];
  __shared__ float tb[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int a0 = blockIdx.x * 16, b0 = blockIdx.y * 16;
  const int64_t chunk = (n + splits - 1) / splits;
  const int64_t i0 = (int64_t)blockIdx.z * chunk, i1 = min(n, i0 + chunk);
  double acc = 0.0;
  for (int64_t s = i0; s < i1; s += 64) {
    for (int t = threadIdx.x; t < 16 * 64; t += 256) {
      const int col = t / 64, row = t % 64;
      const int64_t i = s + row;
      const bool ok = i < i1;
      const float la = (ok && a0 + col < k) ? L[(int64_t)(a0 + col) * n + i] : 0.0f;
      ta[col][row] = (wt && ok) ? la * wt[i] : la;
      tb[col][row] = (ok && b0 + col < k) ? L[(int64_t)(b0 + col) * n + i] : 0.0f;
    }
    __syncthreads();
    float f = 0.0f;
#pragma unroll 8
    for (int row = 0; row < 64; ++row) f = fmaf(ta[ty][row], tb[tx][row], f);
    acc += (double)f;
    __syncthreads();
  }
  const int a = a0 + ty, b = b0 + tx;
  if (a < k && b < k) part[((int64_t)blockIdx.z * k + a) * k + b] = acc;
}

__global__ void k_syrk_final(const double* __restrict__ part, int k, int splits,
                             double* __restrict__ M) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)k * k) return;
  double s = 0.0;
  for (int z = 0; z < splits; ++z) s += part[(int64_t)z * k * k + idx];
  M[idx] = s;
}

// part[z][a][b] = sum_{i in split z} La[a][i] Lb[b][i]; grid (ka tiles, kb tiles, splits).
__global__ void k_cross_part(const float* __restrict__ La, int ka, const float* __restrict__ Lb,
                             int kb, int64_t n, int splits, double* __restrict__ part) {
  __shared__ float ta[16][65];
  __shared__ float tb[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int a0 = blockIdx.x * 16, b0 = blockIdx.y * 16;
  const int64_t chunk = (n + splits - 1) / splits;
  const int64_t i0 = (int64_t)blockIdx.z * chunk, i1 = min(n, i0 + chunk);
  double acc = 0.0;
  for (int64_t s = i0; s < i1; s += 64) {
    for (int t = threadIdx.x; t < 16 * 64; t += 256) {
      const int col = t / 64, row = t % 64;
      const int64_t i = s + row;
      const bool ok = i < i1;
      ta[col][row] = (ok && a0 + col < ka) ? La[(int64_t)(a0 + col) * n + i] : 0.0f;
      tb[col][row] = (ok && b0 + col < kb) ? Lb[(int64_t)(b0 + col) * n + i] : 0.0f;
    }
    __syncthreads();
    float f = 0.0f;
#pragma unroll 8
    for (int row = 0; row < 64; ++row) f = fmaf(ta[ty][row], tb[tx][row], f);
    acc += (double)f;
    __syncthreads();
  }
  const int a = a0 + ty, b = b0 + tx;
  if (a < ka && b < kb) part[((int64_t)blockIdx.z * ka + a) * kb + b] = acc;
}

__global__ void k_cross_final(const double* __restrict__ part, int64_t count, int splits,
                              double* __restrict__ M) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  double s = 0.0;
  for (int z = 0; z < splits; ++z) s += part[(int64_t)z * count + idx];
  M[idx] = s;
}

// w-part[(b*ncols + c)*k + kk] = sum_{i in chunk b} L[kk][i] v[c][i]; block =
// 16 kk x 16 c, grid = (chunks, kk tiles, column tiles).
// rs (optional): per-row scale of v (diag(rs) v).
__global__ void k_lt_part(const float* __restrict__ L, int64_t n, int k,
                          const float* __restrict__ v, int ncols, int nb,
                          float* __restrict__ wpart, const float* __restrict__ rs) {
  __shared__ float tl[16][65];
  __shared__ float tv[16][65];
  const int tc = threadIdx.x & 15, tk = threadIdx.x >> 4;
  const int kk0 = blockIdx.y * 16, c0 = blockIdx.z * 16;
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  float acc = 0.0f;
  for (int64_t s = i0; s < i1; s += 64) {
    for (int t = threadIdx.x; t < 16 * 64; t += 256) {
      const int q = t / 64, row = t % 64;
      const int64_t i = s + row;
      const bool ok = i < i1;
      tl[q][row] = (ok && kk0 + q < k) ? L[(int64_t)(kk0 + q) * n + i] : 0.0f;
      const float vv = (ok && c0 + q < ncols) ? v[(int64_t)(c0 + q) * n + i] : 0.0f;
      tv[q][row] = (rs && ok) ? vv * rs[i] : vv;
    }
    __syncthreads();
#pragma unroll 8
    for (int row = 0; row < 64; ++row) acc = fmaf(tl[tk][row], tv[tc][row], acc);
    __syncthreads();
  }
  const int kk = kk0 + tk, c = c0 + tc;
  if (kk < k && c < ncols) wpart[((int64_t)blockIdx.x * ncols + c) * k + kk] = acc;
}

// wpart[(b*ncols + c)*k + kk] = sum_{i in chunk b} L[kk][i] v[c][i] (rs[i] v
// when rs is given) on the fp32 matrix cores, v_mfma_f32_16x16x4_f32 with
// A = L tile [16 kk x 4 rows], B = v tile [4 rows x 16 c], D[kk][c].  Lane l
// supplies rows 4 (l/16) .. + 3 of a 16-row group, element e to MFMA e (the
// same rows on both sides).  Wave w takes kk tiles w, w + 4, .. (<= 4 tiles,
// k <= 256); each pass loads U groups of 16 rows (all tiles, all columns)
// before their MFMAs so the loads overlap, double-buffered across passes.
// Every load is unconditional, with no branch between a load and its use, so
// the compiler's memory wait counts stay exact and both stages stay in flight:
// a row past the chunk, an L row past k or a column past ncols is clamped to a
// valid address and its value replaced by zero.  VEC4: n and the chunk are
// multiples of 4, so a quad of rows is all in or all out of the chunk.  RS:
// rs is given.
template <int NCT, int U, bool VEC4, bool RS>
__global__ __launch_bounds__(256) void k_ltv_mfma(const float* __restrict__ L, int64_t n, int k,
                                                  const float* __restrict__ v, int ncols,
                                                  int64_t chunk, float* __restrict__ wpart,
                                                  const float* __restrict__ rs) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lm = lane & 15, lq = lane >> 4;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const int ktiles = (k + 15) / 16;
  int nt = 0;
  while (nt < 4 && wave + 4 * nt < ktiles) ++nt;
  const int64_t safe_row = VEC4 ? n - 4 : n - 1;
  const f4v zero = f4v{0.f, 0.f, 0.f, 0.f};
  // rows r0 .. r0 + 3 of one matrix row, zero outside the chunk
  auto quad = [&](const float* base, int64_t r0) __attribute__((always_inline)) -> f4v {
    if constexpr (VEC4) {
      const bool ok = r0 < i1;
      const f4v x = *reinterpret_cast<const f4v*>(base + (ok ? r0 : safe_row));
      return ok ? x : zero;
    } else {
      f4v x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = r0 + e < i1;
        const float y = base[ok ? r0 + e : safe_row];
        x[e] = ok ? y : 0.0f;
      }
      return x;
    }
  };
  f4v acc[4][NCT];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[t][ct] = f4v{0.f, 0.f, 0.f, 0.f};
  // U groups of 16 rows starting at row i (zeros past the chunk end)
  auto load = [&](int64_t i, f4v (&a)[U][4], f4v (&b)[U][NCT]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r0 = i + 16 * u + 4 * lq;
      f4v sv = zero;
      if constexpr (RS) sv = quad(rs, r0);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const int c = ct * 16 + lm;
        f4v x = quad(v + (int64_t)(c < ncols ? c : ncols - 1) * n, r0);
        if constexpr (RS) x *= sv;
        b[u][ct] = c < ncols ? x : zero;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int kk = (wave + 4 * t) * 16 + lm;
        const f4v x = quad(L + (int64_t)(kk < k ? kk : k - 1) * n, r0);
        a[u][t] = kk < k ? x : zero;
      }
    }
  };
  auto mma = [&](const f4v (&a)[U][4], const f4v (&b)[U][NCT]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t >= nt) break;  // uniform per wave
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[t][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][t][e], b[u][ct][e], acc[t][ct],
                                                             0, 0, 0);
      }
  };
  // Two register stages: the loads of one stage are in flight while the other
  // stage's MFMAs run.
  f4v a0[U][4], b0[U][NCT], a1[U][4], b1[U][NCT];
  load(i0, a0, b0);
  for (int64_t i = i0; i < i1; i += 32 * U) {
    load(i + 16 * U, a1, b1);
    mma(a0, b0);
    load(i + 32 * U, a0, b0);
    mma(a1, b1);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t >= nt) break;
    const int kt = wave + 4 * t;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kk = kt * 16 + 4 * lq + q, c = ct * 16 + lm;
        if (kk < k && c < ncols) wpart[((int64_t)blockIdx.x * ncols + c) * k + kk] = acc[t][ct][q];
      }
  }
}

// k_ltv_mfma for ncols <= 16 and k <= 256 with the chunk's rows and kk tiles
// split over RG x TS waves: wave w takes the 64-row groups g0 = i0 +
// 64 (w % RG), + 64 RG, .. and the kk tiles t = w / RG + TS j, streaming the
// tiles over each group (16 L rows x 64 rows per stage, double buffered; the
// waves of a block read 64 RG-row runs of each L row) with the group's v
// values in registers.  MFMA roles as in k_ltv_mfma (A = L, B = v, D[kk][c]).
// The RG row groups of a tile set are added through LDS in group order, and
// the waves of group 0 write the chunk's partial.  v rows past the chunk are
// zero; other out-of-range loads use clamped addresses and only feed D
// entries that are not written.  RG = TS = 2 (4 waves) when there are enough
// chunks to fill the GPU, RG = TS = 4 (16 waves) for small n.
template <bool VEC4, bool RS, int RG, int TS>
__global__ __launch_bounds__(64 * RG * TS) void k_ltv_c16(
    const float* __restrict__ L, int64_t n, int k, const float* __restrict__ v, int ncols,
    int64_t chunk, float* __restrict__ wpart, const float* __restrict__ rs) {
  constexpr int NJ = 16 / TS;  // tiles per wave (k <= 256)
  __shared__ f4v red[RG - 1][TS][NJ][64];  // groups 1..RG-1: [group - 1][tile set][j][lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rh = wave % RG, th = wave / RG;
  const int lm = lane & 15, lq = lane >> 4;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const int ktiles = (k + 15) / 16;
  const int64_t safe = VEC4 ? n - 4 : n - 1;
  const f4v zero = f4v{0.f, 0.f, 0.f, 0.f};
  auto quad = [&](const float* base, int64_t r0) __attribute__((always_inline)) -> f4v {
    if constexpr (VEC4) {
      return *reinterpret_cast<const f4v*>(base + (r0 < n ? r0 : safe));
    } else {
      f4v x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = base[r0 + e < n ? r0 + e : safe];
      return x;
    }
  };
  f4v acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero;
  const float* vc = v + (int64_t)(lm < ncols ? lm : ncols - 1) * n;
  for (int64_t g0 = i0 + 64 * rh; g0 < i1; g0 += 64 * RG) {
    f4v b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t r0 = g0 + 16 * u + 4 * lq;
      f4v x = quad(vc, r0);
      if constexpr (RS) x *= quad(rs, r0);
      if constexpr (VEC4) {
        b[u] = r0 < i1 ? x : zero;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) b[u][e] = r0 + e < i1 ? x[e] : 0.0f;
      }
    }
    // tile t = th + TS j
    auto load = [&](int j, f4v (&a)[4]) __attribute__((always_inline)) {
      const float* lr = L + (int64_t)min(16 * (th + TS * j) + lm, k - 1) * n;
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = quad(lr, g0 + 16 * u + 4 * lq);
    };
    auto mma = [&](f4v& d, const f4v (&a)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          d = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][e], b[u][e], d, 0, 0, 0);
    };
    f4v a0[4], a1[4];
    load(0, a0);
#pragma unroll
    for (int j = 0; j < NJ; j += 2) {
      if (th + TS * j >= ktiles) break;  // uniform
      load(j + 1, a1);
      mma(acc[j], a0);
      if (th + TS * (j + 1) >= ktiles) break;
      load(j + 2, a0);
      mma(acc[j + 1], a1);
    }
  }
  if (rh > 0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (th + TS * j < ktiles) red[rh - 1][th][j][lane] = acc[j];
  }
  __syncthreads();
  if (rh > 0 || lm >= ncols) return;
  float* wp = wpart + ((int64_t)blockIdx.x * ncols + lm) * k;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int t = th + TS * j;
    if (t >= ktiles) break;
    f4v tot = acc[j];
#pragma unroll
    for (int g = 0; g < RG - 1; ++g) tot += red[g][th][j][lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kk = 16 * t + 4 * lq + q;
      if (kk < k) wp[kk] = tot[q];
    }
  }
}

// out[o] = sum_b wpart[b*total + o] (fp64, fixed order) for o < total: block =
// 16 consecutive outputs x 16 stripes of chunks (b = s, s + 16, ..); each
// thread keeps 8 loads in flight and adds them in order, then the stripes are
// added in order.
__global__ __launch_bounds__(256) void k_part_reduce(const float* __restrict__ wpart, int nb,
                                                     int64_t total, float* __restrict__ out) {
  __shared__ double sm[16][16];
  const int j = threadIdx.x & 15, sidx = threadIdx.x >> 4;
  const int64_t o = (int64_t)blockIdx.x * 16 + j;
  double acc = 0.0;
  if (o < total) {
    int b = sidx;
    for (; b + 7 * 16 < nb; b += 8 * 16) {
      float t[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) t[q] = wpart[(int64_t)(b + 16 * q) * total + o];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc += (double)t[q];
    }
    for (; b < nb; b += 16) acc += (double)wpart[(int64_t)b * total + o];
  }
  sm[sidx][j] = acc;
  __syncthreads();
  if (sidx == 0 && o < total) {
    double t = sm[0][j];
#pragma unroll
    for (int q = 1; q < 16; ++q) t += sm[q][j];
    out[o] = (float)t;
  }
}

// u = Minv w per column, written transposed by 16-column tiles:
// ut[((c/16)*k + kk)*16 + c%16] = sum_q Minv[kk*k + q] w[c*k + q] (zero for
// padding columns).  One wave per output, lanes stride q (coalesced row of
// Minv), fixed-order shuffle sum.
__global__ __launch_bounds__(256) void k_small_solve_t(const float* __restrict__ w, int k,
                                                       int ncols, const float* __restrict__ Minv,
                                                       float* __restrict__ ut) {
  const int64_t o = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int cpad = ((ncols + 15) / 16) * 16;
  if (o >= (int64_t)k * cpad) return;  // uniform per wave
  const int c = (int)(o / k), kk = (int)(o - (int64_t)c * k);
  float s = 0.0f;
  if (c < ncols)
    for (int q = lane; q < k; q += 64) s = fmaf(Minv[(int64_t)kk * k + q], w[(int64_t)c * k + q], s);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) ut[((int64_t)(c / 16) * k + kk) * 16 + (c & 15)] = s;
}

// k_part_reduce followed by k_small_solve_t in one launch, for the Woodbury
// apply.  Block (c, g) of (cpad, ceil(k / 16)): first column c's chunk
// partials w[c][kk] = sum_b wpart[(b ncols + c) k + kk] for every kk, added in
// the order of k_part_reduce (16 stripes of chunks b = s, s + 16, .., each in
// order, then the stripes in order, rounded to fp32) into LDS; then wave w
// forms ut[((c/16) k + kk) 16 + c%16] = sum_q Minv[kk k + q] w[c][q] for
// kk = 16 g + w as k_small_solve_t does (lanes stride q, fixed shuffle tree);
// zero for padding columns.
constexpr int kPartSolveMaxK = 256;
__global__ __launch_bounds__(1024) void k_part_solve_t(const float* __restrict__ wpart, int nb,
                                                       int k, int ncols,
                                                       const float* __restrict__ Minv,
                                                       float* __restrict__ ut) {
  __shared__ double sm[16][kPartSolveMaxK];
  __shared__ float wc[kPartSolveMaxK];
  const int c = blockIdx.x;
  const int kl = threadIdx.x & 63, sidx = threadIdx.x >> 6;
  const int64_t total = (int64_t)k * ncols;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  if (c < ncols) {
    const float* wc0 = wpart + (int64_t)c * k + kl;
    int b = sidx;
    for (; b + 7 * 16 < nb; b += 8 * 16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (kl + 64 * u >= k) break;
        float t[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) t[q] = wc0[(int64_t)(b + 16 * q) * total + 64 * u];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[u] += (double)t[q];
      }
    }
    for (; b < nb; b += 16)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (kl + 64 * u < k) acc[u] += (double)wc0[(int64_t)b * total + 64 * u];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (kl + 64 * u < k) sm[sidx][kl + 64 * u] = acc[u];
  __syncthreads();
  if (sidx < 4) {
    const int kk = kl + 64 * sidx;
    if (kk < k) {
      double t = sm[0][kk];
#pragma unroll
      for (int q = 1; q < 16; ++q) t += sm[q][kk];
      wc[kk] = (float)t;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kk = 16 * blockIdx.y + wave;
  if (kk >= k) return;
  float s = 0.0f;
  if (c < ncols)
    for (int q = lane; q < k; q += 64) s = fmaf(Minv[(int64_t)kk * k + q], wc[q], s);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) ut[((int64_t)(c / 16) * k + kk) * 16 + (c & 15)] = s;
}

// out[c][i] = (v[c][i] - sum_kk L[kk][i] u[c][kk]) * (DINV ? dinv[i] : inv_noise)
// for the 16 columns of tile blockIdx.y, one thread per row of chunk
// blockIdx.x (rows i0 + tid, i0 + tid + 256, ..): L read once, coalesced; u is
// the same for every row, read from ut (k_small_solve_t layout) with scalar
// loads.  DOT: dpart[c*nb + b] = sum over the chunk of dotv[c][i] out[c][i]
// (fp64, fixed order: each thread's rows in order, then the wave's shuffle
// tree, then the four waves).  v, dotv and out may alias: each element is read
// and written by one thread.  All loads are unconditional (indices clamped
// into range), so the compiler's memory wait counts stay exact: the row's v
// and dotv values and the next 16 rows of L are in flight during the FMAs.
template <bool DINV, bool DOT>
__global__ __launch_bounds__(256) void k_woodbury_rows(
    const float* __restrict__ L, int64_t n, int k, const float* __restrict__ ut, int ncols,
    float inv_noise, const float* v, float* out, const float* __restrict__ dinv,
    const float* dotv, int nb, double* __restrict__ dpart) {
  __shared__ double wsum[4][16];
  const int c0 = blockIdx.y * 16;
  const int cn = min(16, ncols - c0);
  const float* __restrict__ ub = ut + (int64_t)blockIdx.y * k * 16;
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  double dacc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) dacc[c] = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    float vin[16], din[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int64_t off = (int64_t)(c0 + (c < cn ? c : cn - 1)) * n + i;
      vin[c] = v[off];
      if constexpr (DOT) din[c] = dotv[off];
    }
    const float sc = DINV ? dinv[i] : inv_noise;
    float z[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) z[c] = 0.0f;
    // groups of 16 L rows; the next group's loads (rows clamped to k - 1) are
    // issued before this group's FMAs
    const int kmain = k & ~15;
    float lc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) lc[q] = L[(int64_t)min(q, k - 1) * n + i];
    for (int kg = 0; kg < kmain; kg += 16) {
      float ln[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) ln[q] = L[(int64_t)min(kg + 16 + q, k - 1) * n + i];
#pragma unroll
      for (int q = 0; q < 16; ++q)
#pragma unroll
        for (int c = 0; c < 16; ++c) z[c] = fmaf(lc[q], ub[(kg + q) * 16 + c], z[c]);
#pragma unroll
      for (int q = 0; q < 16; ++q) lc[q] = ln[q];
    }
    // rows kmain .. k - 1 are in lc
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (kmain + q >= k) break;  // uniform
#pragma unroll
      for (int c = 0; c < 16; ++c) z[c] = fmaf(lc[q], ub[(kmain + q) * 16 + c], z[c]);
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      if (c < cn) {
        const float zz = sc * (vin[c] - z[c]);
        out[(int64_t)(c0 + c) * n + i] = zz;
        if constexpr (DOT) dacc[c] += (double)din[c] * (double)zz;
      }
    }
  }
  if constexpr (!DOT) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    double t = dacc[c];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
    if (lane == 0) wsum[wave][c] = t;
  }
  __syncthreads();
  if (threadIdx.x < cn)
    dpart[(int64_t)(c0 + threadIdx.x) * nb + blockIdx.x] =
        ((wsum[0][threadIdx.x] + wsum[1][threadIdx.x]) + wsum[2][threadIdx.x]) +
        wsum[3][threadIdx.x];
}

// k_woodbury_rows on the fp32 matrix cores (k <= kWoodMfmaMaxK).  Block =
// chunk blockIdx.x x the 16 columns of tile blockIdx.y, 4 KS waves: wave w
// takes the 64-row groups g0 = i0 + 64 (w & 3), + 256, .. and the part w >> 2
// of KS parts of the L rows (kq rows each, a multiple of 32); KS = 4 for
// small n, where the chunks do not fill the GPU (four times as many loads in
// flight), KS = 1 (no split, no exchange) otherwise.  Per group,
// v_mfma_f32_16x16x4_f32 tile t (0..3) maps MFMA row m to row g0 + 4 m + t
// and the MFMA k index to L row kk: lane l supplies A = L[kk0 + l/16][g0 +
// 4 (l%16) + t] (one 16-byte load per L row per lane covers the four tiles,
// 256 contiguous bytes per L row) and B = u[c0 + l%16][kk0 + l/16] from the u
// tile staged in LDS (zero past k).  The parts' tiles are added through
// LDS in part order by the waves of part 0, which finish the group: D
// row 4 (l/16) + q of tile t is row g0 + 16 (l/16) + 4 q + t of column
// c0 + l%16, so each lane writes four runs of four rows.  dpart: each lane's
// rows in order, the four lanes of a column by a shuffle butterfly, then the
// row groups in order.  Loads are unconditional (addresses clamped into
// range; the D rows they feed are not stored), so wait counts stay exact.
constexpr int kWoodMfmaMaxK = 256;
template <bool VEC4, bool DINV, bool DOT, int KS>
__global__ __launch_bounds__(256 * KS) void k_woodbury_mfma(
    const float* __restrict__ L, int64_t n, int k, const float* __restrict__ ut, int ncols,
    float inv_noise, const float* v, float* out, const float* __restrict__ dinv,
    const float* dotv, int nb, double* __restrict__ dpart) {
  __shared__ float sB[kWoodMfmaMaxK * 16];
  __shared__ f4v red[KS > 1 ? KS - 1 : 1][4][4][64];  // parts 1..KS-1: [part - 1][group][tile][lane]
  __shared__ double wsum[4][16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave & 3, kh = wave >> 2;
  const int lm = lane & 15, lq = lane >> 4;
  const int c0 = blockIdx.y * 16, cn = min(16, ncols - c0);
  const int kpad = (k + 31) & ~31;
  const int kq = (((kpad + KS - 1) / KS) + 31) & ~31;
  const int kb0 = min(kpad, kh * kq), kb1 = min(kpad, kb0 + kq);
  {
    const float* __restrict__ ub = ut + (int64_t)blockIdx.y * k * 16;
    for (int j = threadIdx.x; j < kpad * 16; j += 256 * KS) sB[j] = j < k * 16 ? ub[j] : 0.0f;
  }
  __syncthreads();
  const int64_t chunk = cg_chunk_rows(n, nb);
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const int64_t safe = VEC4 ? n - 4 : n - 1;
  const f4v zero = f4v{0.f, 0.f, 0.f, 0.f};
  // rows r .. r + 3 of a matrix row (values past n come from a clamped address)
  auto quad = [&](const float* base, int64_t r) __attribute__((always_inline)) -> f4v {
    if constexpr (VEC4) {
      return *reinterpret_cast<const f4v*>(base + (r < n ? r : safe));
    } else {
      f4v x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = base[r + e < n ? r + e : safe];
      return x;
    }
  };
  const int cc = c0 + (lm < cn ? lm : cn - 1);
  double dacc = 0.0;
  // every wave makes the same number of passes (the barriers below); rows
  // past the chunk only feed D rows that are not stored
  const int64_t passes = i1 > i0 ? (i1 - i0 + 255) / 256 : 0;
  for (int64_t pass = 0; pass < passes; ++pass) {
    const int64_t g0 = i0 + 256 * pass + 64 * rg;
    const int64_t ra = g0 + 4 * lm;
    f4v acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = zero;
    // a batch = 16 L rows kb .. kb + 15: lane rows kb + 4 j + lq, j = 0..3
    auto load = [&](int kb, f4v (&a)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = quad(L + (int64_t)min(kb + 4 * j + lq, k - 1) * n, ra);
    };
    auto mma = [&](int kb, const f4v (&a)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = sB[(kb + 4 * j + lq) * 16 + lm];
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][t], b, acc[t], 0, 0, 0);
      }
    };
    if (kb0 < kb1) {
      f4v a0[4], a1[4];
      load(kb0, a0);
      for (int kb = kb0; kb < kb1; kb += 32) {
        load(kb + 16, a1);
        mma(kb, a0);
        load(kb + 32, a0);
        mma(kb + 16, a1);
      }
    }
    if constexpr (KS > 1) {
      if (kh > 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) red[kh - 1][rg][t][lane] = acc[t];
      }
      __syncthreads();
      if (kh == 0) {
#pragma unroll
        for (int g = 0; g < KS - 1; ++g)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[t] += red[g][rg][t][lane];
      }
    }
    if (kh == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r = g0 + 16 * lq + 4 * q;
        const f4v vq = quad(v + (int64_t)cc * n, r);
        f4v dq = zero, sq = f4v{inv_noise, inv_noise, inv_noise, inv_noise};
        if constexpr (DOT) dq = quad(dotv + (int64_t)cc * n, r);
        if constexpr (DINV) sq = quad(dinv, r);
        f4v zz;
#pragma unroll
        for (int t = 0; t < 4; ++t) zz[t] = sq[t] * (vq[t] - acc[t][q]);
        if (lm < cn) {
          float* o = out + (int64_t)cc * n;
          if (VEC4 && r + 3 < i1) {
            *reinterpret_cast<f4v*>(o + r) = zz;
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (r + t < i1) o[r + t] = zz[t];
          }
        }
        if constexpr (DOT) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (r + t < i1) dacc += (double)dq[t] * (double)zz[t];
        }
      }
    }
    if constexpr (KS > 1) __syncthreads();  // red is rewritten by the next pass
  }
  if constexpr (!DOT) return;
  if (kh == 0) {
    dacc += __shfl_xor(dacc, 16);
    dacc += __shfl_xor(dacc, 32);
    if (lq == 0) wsum[rg][lm] = dacc;
  }
  __syncthreads();
  if (threadIdx.x < cn)
    dpart[(int64_t)(c0 + threadIdx.x) * nb + blockIdx.x] =
        ((wsum[0][threadIdx.x] + wsum[1][threadIdx.x]) + wsum[2][threadIdx.x]) +
        wsum[3][threadIdx.x];
}

// grid = (row blocks, column tiles of 16)
// ds (optional): per-row scale of zn in place of s.
__global__ __launch_bounds__(256) void k_low_rank_sample(
    const float* __restrict__ L, int64_t n, int k, const float* __restrict__ zr,
    const float* __restrict__ zn, float s, int ncols, float* __restrict__ out,
    const float* __restrict__ ds, int gT, int gK, int goff) {
  extern __shared__ float zs[];  // [16][k]
  const int c0 = blockIdx.y * 16;
  const int cn = min(16, ncols - c0);
  for (int t = threadIdx.x; t < 16 * k; t += blockDim.x) {
    const int c = t / k, kk = t - c * k;
    const int cc = c0 + c;
    // column cc of zr, or read in place from a blocked vector (gT > 0)
    const int64_t src = gT > 0 ? (int64_t)(cc / gT) * gK + goff + (int64_t)(cc % gT) * k + kk
                               : (int64_t)cc * k + kk;
    zs[t] = c < cn ? zr[src] : 0.0f;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float z[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) z[c] = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    const float l = L[(int64_t)kk * n + i];
#pragma unroll
    for (int c = 0; c < 16; ++c) z[c] = fmaf(l, zs[c * k + kk], z[c]);
  }
  const float si = ds ? ds[i] : s;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    if (c < cn) {
      const int64_t off = (int64_t)(c0 + c) * n + i;
      out[off] = zn ? z[c] + si * zn[off] : z[c];
    }
  }
}

// ------------------------------------------------------------- gradients
// Block: 256 rows a; LDS tiles of 64 column points b.  Per pair the reference
// derivatives (see oracle/kernels.py for the closed forms) are weighted by
// g_ab = sum_c Lf[c][a] Rf[c][b] and accumulated; fp32 within a tile, fp64
// across tiles.  part[block][p] (p: per-dim lengthscale terms, then os term).
constexpr int kGradTile = 64;

template <int KIND, int DM, bool ARD>
__global__ __launch_bounds__(256) void k_grad_trace(
    const float* __restrict__ Z, int d, int64_t n, const float* __restrict__ Lf,
    const float* __restrict__ Rf, int ncols, int c0, double* __restrict__ part,
    int nterms) {
  __shared__ float zb[kGradTile][DM + 1];
  __shared__ float rb[kGradTile][17];
  __shared__ double sm[4];
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = a < n;
  const int cn = min(16, ncols - c0);
  // column range of this split (whole tiles)
  const int64_t tiles = (n + kGradTile - 1) / kGradTile;
  const int64_t tps = (tiles + gridDim.y - 1) / gridDim.y;
  const int64_t jb = min(n, (int64_t)blockIdx.y * tps * kGradTile);
  const int64_t je = min(n, jb + tps * kGradTile);
  float za[DM];
#pragma unroll
  for (int k = 0; k < DM; ++k) za[k] = (live && k < d) ? Z[a * d + k] : 0.0f;
  float la[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) la[c] = (live && c < cn) ? Lf[(int64_t)(c0 + c) * n + a] : 0.0f;
  constexpr int NT = ARD ? DM : 1;
  double accd[NT + 1];
#pragma unroll
  for (int t = 0; t <= NT; ++t) accd[t] = 0.0;
  for (int64_t b0 = jb; b0 < je; b0 += kGradTile) {
    __syncthreads();
    for (int t = threadIdx.x; t < kGradTile * DM; t += blockDim.x) {
      const int bb = t / DM, k = t - bb * DM;
      const int64_t b = b0 + bb;
      zb[bb][k] = (b < je && k < d) ? Z[b * d + k] : 0.0f;
    }
    for (int t = threadIdx.x; t < kGradTile * 16; t += blockDim.x) {
      const int bb = t / 16, c = t - bb * 16;
      const int64_t b = b0 + bb;
      rb[bb][c] = (b < je && c < cn) ? Rf[(int64_t)(c0 + c) * n + b] : 0.0f;
    }
    __syncthreads();
    float acc[NT + 1];
#pragma unroll
    for (int t = 0; t <= NT; ++t) acc[t] = 0.0f;
    const int cnt = (int)min((int64_t)kGradTile, je - b0);
    for (int bb = 0; bb < cnt; ++bb) {
      float dz2[DM];
      float r2 = 0.0f;
#pragma unroll
      for (int k = 0; k < DM; ++k) {
        const float df = za[k] - zb[bb][k];
        dz2[k] = df * df;
        r2 += dz2[k];
      }
      float kv, h;
      if constexpr (KIND == KIND_RBF) {
        kv = __builtin_amdgcn_exp2f(-fmaxf(r2, 0.0f));  // not clamped
        h = kv;
      } else if constexpr (KIND == KIND_MATERN12) {
        // h = log2(e) k / r with the reference's floored r = sqrt(r^2 + 1e-20);
        // the exponent is clamped for ARD only (exp2_limit)
        const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
        kv = __builtin_amdgcn_exp2f(ARD ? -fminf(u, kExp2Clamp) : -u);
        h = kLog2e * kv / __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f) + kM12RFloor);
      } else if constexpr (KIND == KIND_MATERN32) {
        const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
        const float e = __builtin_amdgcn_exp2f(-fminf(u, kExp2Clamp));
        kv = fmaf(u, kLn2, 1.0f) * e;
        h = 3.0f * e;
      } else {
        const float u = __builtin_amdgcn_sqrtf(fmaxf(r2, 0.0f));
        const float e = __builtin_amdgcn_exp2f(-fminf(u, kExp2Clamp));
        kv = fmaf(u, fmaf(u, kLn2 * kLn2 / 3.0f, kLn2), 1.0f) * e;
        h = (5.0f / 3.0f) * fmaf(u, kLn2, 1.0f) * e;
      }
      float g = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) g = fmaf(la[c], rb[bb][c], g);
      const float hg = h * g;
      acc[NT] = fmaf(kv, g, acc[NT]);
      if constexpr (ARD) {
#pragma unroll
        for (int k = 0; k < DM; ++k) acc[k] = fmaf(hg, dz2[k], acc[k]);
      } else {
        acc[0] = fmaf(hg, r2, acc[0]);
      }
    }
#pragma unroll
    for (int t = 0; t <= NT; ++t) accd[t] += (double)acc[t];
  }
  // Block reduction of each term.
  for (int t = 0; t < nterms; ++t) {
    const int src = (t == nterms - 1) ? NT : t;
    double v = 0.0;
#pragma unroll
    for (int q = 0; q <= NT; ++q)
      if (q == src) v = accd[q];
    const double tot = block_sum_d(live ? v : 0.0, sm);
    if (threadIdx.x == 0)
      part[((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * nterms + t] = tot;
  }
}

// Column splits of the gradient pair loop: enough blocks to fill the chip
// (>= 2048 with the row blocks) while every split keeps >= 1024 columns.
static int grad_splits(int64_t n) {
  const int64_t rows = ceil_div(n, 256);
  return (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(2048, rows), ceil_div(n, 1024)));
}

template <int KIND, bool ARD>
void launch_grad(int dm, const float* Z, int d, int64_t n, const float* Lf,
                 const float* Rf, int ncols, int c0, double* part, int nterms,
                 hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(n, 256), (unsigned)grad_splits(n));
  switch (dm) {
#define MGP_GRAD_CASE(DMV)                                                           \
  case DMV:                                                                         \
    hipLaunchKernelGGL((k_grad_trace<KIND, DMV, ARD>), grid, dim3(256), 0, st, Z, d, \
                       n, Lf, Rf, ncols, c0, part, nterms);                         \
    break;
    MGP_GRAD_CASE(1)
    MGP_GRAD_CASE(2)
    MGP_GRAD_CASE(4)
    MGP_GRAD_CASE(8)
    MGP_GRAD_CASE(16)
    MGP_GRAD_CASE(32)
#undef MGP_GRAD_CASE
    default:
      throw Error(ST_INVALID, "unsupported gradient dimension bucket");
  }
}

// ------------------------------------------------------------- Lanczos
__global__ void k_multi_dot_part(const float* __restrict__ Q, const float* __restrict__ w,
                                 int64_t n, int nb, double* __restrict__ part) {
  __shared__ double sm[4];
  const int j = blockIdx.y;
  const int64_t chunk = (n + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(n, i0 + chunk);
  const float* q = Q + (int64_t)j * n;
  double acc = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x)
    acc += (double)q[i] * (double)w[i];
  const double t = block_sum_d(acc, sm);
  if (threadIdx.x == 0) part[(int64_t)j * nb + blockIdx.x] = t;
}

__global__ void k_multi_axpy(const float* __restrict__ Q, int nvec,
                             const double* __restrict__ coef, float* __restrict__ w,
                             int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  double s = 0.0;
  for (int j = 0; j < nvec; ++j) s += coef[j] * (double)Q[(int64_t)j * n + i];
  w[i] = (float)((double)w[i] - s);
}

__global__ void k_gemm_nr_rr(const float* __restrict__ Q, const float* __restrict__ T,
                             int64_t n, int r, int c0, float* __restrict__ S) {
  extern __shared__ float ts[];  // [r][16]
  const int cn = min(16, r - c0);
  for (int t = threadIdx.x; t < r * 16; t += blockDim.x) {
    const int k = t / 16, c = t - k * 16;
    ts[t] = c < cn ? T[(int64_t)k * r + c0 + c] : 0.0f;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = 0.0f;
  for (int k = 0; k < r; ++k) {
    const float q = Q[(int64_t)k * n + i];
#pragma unroll
    for (int c = 0; c < 16; ++c) acc[c] = fmaf(q, ts[k * 16 + c], acc[c]);
  }
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c < cn) S[(int64_t)(c0 + c) * n + i] = acc[c];
}

__global__ void k_love_variance(const float* __restrict__ V, int64_t m, int r, float diag0,
                                const float* __restrict__ dvec, float* __restrict__ var) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= m) return;
  float s = 0.0f;
  for (int k = 0; k < r; ++k) {
    const float v = V[(int64_t)k * m + j];
    s = fmaf(v, v, s);
  }
  const float diag = dvec ? dvec[j] : diag0;
  var[j] = fmaxf(diag - s, 1e-10f);
}

}  // namespace

// ===================================================================== host

int reduction_chunks(int64_t n) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(256, ceil_div(n, 2048)));
}

int cg_chunks(int64_t n) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(2048, ceil_div(n, 256)));
}

// Below this many chunks (two per CU) the L-streaming kernels of the Woodbury
// apply run 16 waves per chunk instead of 4 (measured: n = 40k-50k faster,
// n = 250k slower with 16).
constexpr int kFewChunks = 512;
// The merged chunk-sum and small solve re-adds a column's chunks x k partials
// in every block; above this much work two launches are cheaper.
constexpr int64_t kPartSolveMaxWork = 32768;

// 16-byte vector access is safe when the arrays are 16-byte aligned and every
// column and chunk (cg_chunk_rows) starts on a multiple of 4 elements.
static int vec4_ok(int64_t n, int nb, std::initializer_list<const void*> ptrs) {
  if (n % 4 != 0 || cg_chunk_rows(n, nb) % 4 != 0) return 0;
  for (const void* q : ptrs)
    if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return 0;
  return 1;
}

void coldot_partial(const float* a, const float* b, int64_t n, int ncols, int nb,
                    double* part, hipStream_t st) {
  hipLaunchKernelGGL(k_coldot_w, dim3(nb, ncols), dim3(64), 0, st, a, b, n, nb,
                     vec4_ok(n, nb, {a, b}), part);
  MGP_HIP_CHECK(hipGetLastError());
}

void coldot_finalize(const double* part, int nb, int ncols, double* out, hipStream_t st) {
  hipLaunchKernelGGL(k_coldot_final, grid1(ncols), dim3(kBlock), 0, st, part, nb, ncols, out);
  MGP_HIP_CHECK(hipGetLastError());
}

// Chunks per wave of the CG vector kernels: about 2048 waves in all, so the
// per-wave reduction of a column's scalar partials stays small next to the
// vector traffic.
static int cg_group(int nb, int ncols) {
  return std::max(1, (nb * ncols) / 2048);
}

void cg_update(float* x, float* r, const float* p, const float* Ap, int64_t n, int ncols,
               int nb, const double* pap_part, CGScalars s, double* rr_part, hipStream_t st) {
  const int G = cg_group(nb, ncols);
  hipLaunchKernelGGL(k_cg_update_w, dim3((unsigned)ceil_div(nb, G), ncols), dim3(64), 0, st, x, r,
                     p, Ap, n, nb, G, vec4_ok(n, nb, {x, r, p, Ap}), pap_part, s, rr_part);
  MGP_HIP_CHECK(hipGetLastError());
}

void cg_pupdate(float* p, const float* z, int64_t n, int ncols, int nb, const double* rz_part,
                CGScalars s, int iter, int max_tridiag, hipStream_t st) {
  const int G = cg_group(nb, ncols);
  hipLaunchKernelGGL(k_cg_pupdate_w, dim3((unsigned)ceil_div(nb, G), ncols), dim3(64), 0, st, p,
                     z, n, nb, G, vec4_ok(n, nb, {p, z}), rz_part, ncols, s, iter, max_tridiag);
  MGP_HIP_CHECK(hipGetLastError());
}

void cg_mean_resnorm(const double* rr_part, int nb, int ncols, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_mean_resnorm, dim3(1), dim3(64), 0, st, rr_part, nb, ncols, out);
  MGP_HIP_CHECK(hipGetLastError());
}

void fill(float* x, int64_t count, float v, hipStream_t st) {
  if (count <= 0) return;
  hipLaunchKernelGGL(k_fill, grid1(count), dim3(kBlock), 0, st, x, count, v);
  MGP_HIP_CHECK(hipGetLastError());
}

void copy(float* dst, const float* src, int64_t count, hipStream_t st) {
  if (count <= 0) return;
  hipLaunchKernelGGL(k_copy, grid1(count), dim3(kBlock), 0, st, dst, src, count);
  MGP_HIP_CHECK(hipGetLastError());
}

void sub(float* y, const float* a, const float* b, int64_t count, hipStream_t st) {
  hipLaunchKernelGGL(k_sub, grid1(count), dim3(kBlock), 0, st, y, a, b, count);
  MGP_HIP_CHECK(hipGetLastError());
}

void sub_scalar(float* y, const float* x, float s, int64_t count, hipStream_t st) {
  hipLaunchKernelGGL(k_sub_scalar, grid1(count), dim3(kBlock), 0, st, y, x, s, count);
  MGP_HIP_CHECK(hipGetLastError());
}

void scale_columns(float* x, const float* scale, int64_t n, int ncols, bool divide,
                   hipStream_t st) {
  hipLaunchKernelGGL(k_scale_columns, grid1(n * ncols), dim3(kBlock), 0, st, x, scale, n,
                     ncols, divide ? 1 : 0);
  MGP_HIP_CHECK(hipGetLastError());
}

void normalize_columns(float* x, int64_t n, int ncols, float* norms, double* part,
                       hipStream_t st) {
  const int nb = reduction_chunks(n);
  coldot_partial(x, x, n, ncols, nb, part, st);
  hipLaunchKernelGGL(k_norms_final, grid1(ncols), dim3(kBlock), 0, st, part, nb, ncols, norms);
  MGP_HIP_CHECK(hipGetLastError());
  scale_columns(x, norms, n, ncols, true, st);
}

void gaussian(float* out, int64_t len, uint64_t seed, hipStream_t st) {
  if (len <= 0) return;
  hipLaunchKernelGGL(k_gaussian, grid1(len), dim3(kBlock), 0, st, out, len, seed);
  MGP_HIP_CHECK(hipGetLastError());
}

namespace {
// Device state of one pivoted-Cholesky build over n residual entries.
struct PivotBufs {
  int64_t n = 0;
  int nb = 0;
  DevBuf<float> diag, mask, coef, pvv;
  DevBuf<int64_t> piv;
  DevBuf<double> pa;
  DevBuf<PivotDev> state;
  PivotBufs(int64_t n_, int rank, float* L, hipStream_t st) : n(n_), nb(reduction_chunks(n_)) {
    diag.ensure(n);
    mask.ensure(n);
    coef.ensure(std::max(rank, 1));
    pvv.ensure(nb);
    piv.ensure(nb);
    pa.ensure(nb);
    state.ensure(1);
    PivotDev init{0, rank, 0, 0.f, 0.f};
    MGP_HIP_CHECK(hipMemcpyAsync(state.ptr, &init, sizeof(init), hipMemcpyHostToDevice, st));
    fill(L, (int64_t)rank * n, 0.0f, st);
  }
};

// Pivot selection and stopping (pivoted_cholesky.mojo:2195-2334) over a
// residual diagonal already in b.diag / b.mask; launch_column(m) writes
// column m of L and updates the residual and the argmax partials.
// diag_value: the provider's diagonal value (stop rule normaliser); noise:
// the provider noise (Nystrom stop rule).
int pivot_loop(PivotBufs& b, int rank, const PivotOptions& o, float* L, float diag_value,
               float noise, hipStream_t st, const std::function<void(int)>& launch_column) {
  const int64_t n = b.n;
  const int nb = b.nb;
  hipLaunchKernelGGL(k_pc_argmax_part, dim3(nb), dim3(kBlock), 0, st, b.diag.ptr, b.mask.ptr,
                     n, nb, b.pvv.ptr, b.piv.ptr, b.pa.ptr);
  MGP_HIP_CHECK(hipGetLastError());
  if (o.method == 0 && !(o.error_tol > 0.f)) {
    // Greedy without a trace stop: selection stays on the device.
    for (int m = 0; m < rank; ++m) {
      hipLaunchKernelGGL(k_pc_select, dim3(1), dim3(kBlock), 0, st, b.pvv.ptr, b.piv.ptr,
                         b.pa.ptr, nb, m, b.state.ptr, b.mask.ptr, L, n, b.coef.ptr);
      launch_column(m);
    }
    PivotDev fin;
    MGP_HIP_CHECK(hipMemcpyAsync(&fin, b.state.ptr, sizeof(fin), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    return fin.stopped ? fin.rank : rank;
  }
  // Host-driven selection.
  std::vector<char> used((size_t)n, 0);
  std::vector<float> dh;
  uint64_t rng = o.seed;
  for (int m = 0; m < rank; ++m) {
    hipLaunchKernelGGL(k_pc_reduce, dim3(1), dim3(64), 0, st, b.pvv.ptr, b.piv.ptr, b.pa.ptr,
                       nb, b.state.ptr);
    PivotDev cur;
    MGP_HIP_CHECK(hipMemcpyAsync(&cur, b.state.ptr, sizeof(cur), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    int64_t pivot = cur.pivot;
    float maxval = cur.maxval;
    if (maxval < 1e-10f || pivot < 0) return std::max(m, 1);
    if (o.method == 2) {
      const float threshold = o.adaptive_tol * (float)n * noise;
      if (cur.sumabs < threshold && m > 0) return m;
    } else if (cur.sumabs / diag_value < o.error_tol) {
      return std::max(m, 1);
    }
    if (o.method != 0) {
      dh.resize((size_t)n);
      MGP_HIP_CHECK(hipMemcpyAsync(dh.data(), b.diag.ptr, (size_t)n * sizeof(float),
                                   hipMemcpyDeviceToHost, st));
      MGP_HIP_CHECK(hipStreamSynchronize(st));
      float total = 0.0f;
      for (int64_t i = 0; i < n; ++i)
        if (!used[(size_t)i] && dh[(size_t)i] > 0.0f) total += dh[(size_t)i];
      if (total < 1e-10f) return std::max(m, 1);
      rng ^= rng >> 12;
      rng ^= rng << 25;
      rng ^= rng >> 27;
      rng *= 0x2545F4914F6CDD1DULL;
      float u = (float)(int64_t)(rng & 0x7FFFFFFFULL) / 2147483648.0f;
      u = u * total;
      float cumsum = 0.0f;
      for (int64_t i = 0; i < n; ++i) {
        if (used[(size_t)i]) continue;
        const float d = dh[(size_t)i];
        if (d > 0.0f) cumsum += d;
        if (cumsum >= u) {
          pivot = i;
          maxval = d;
          break;
        }
      }
    }
    used[(size_t)pivot] = 1;
    hipLaunchKernelGGL(k_pc_setpivot, dim3(1), dim3(kBlock), 0, st, b.state.ptr, b.mask.ptr, L,
                       n, m, b.coef.ptr, pivot, maxval);
    launch_column(m);
  }
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  return rank;
}

// Column m of the pivoted Cholesky of os_B (x) K + diag(extra) over the
// task-blocked index i = s n + j (s < T, j < n), extra = task_noise[t_p] -
// noise_min at the pivot p = t_p n + j_p only: the forward product of a unit
// vector minus the provider noise at the pivot.
template <class Eval>
__global__ __launch_bounds__(256) void k_pc_column_kron(
    Eval ev, const float* __restrict__ Z, int d, int64_t n, int T,
    const float* __restrict__ osB, const float* __restrict__ task_noise, float noise_min,
    int m, float* __restrict__ L, float* __restrict__ diag, const float* __restrict__ mask,
    const float* __restrict__ coef, const PivotDev* __restrict__ state, int nb, float* pv,
    int64_t* pi, double* pa) {
  extern __shared__ float sh[];  // coef[m], zp[d], bcol[T]
  if (state->stopped) return;    // uniform across the grid
  const int64_t N = n * T;
  const int64_t p = state->pivot;
  const int tp = (int)(p / n);
  const int64_t jp = p - (int64_t)tp * n;
  const float scale = 1.0f / sqrtf(fmaxf(state->maxval, 1e-10f));
  float* scoef = sh;
  float* zp = sh + m;
  float* bcol = zp + d;
  for (int j = threadIdx.x; j < m; j += blockDim.x) scoef[j] = coef[j];
  for (int k = threadIdx.x; k < d; k += blockDim.x) zp[k] = Z[jp * d + k];
  for (int s = threadIdx.x; s < T; s += blockDim.x) bcol[s] = osB[s * T + tp];
  __syncthreads();
  const float extra = task_noise[tp] - noise_min;
  const int64_t chunk = (N + nb - 1) / nb;
  const int64_t i0 = (int64_t)blockIdx.x * chunk, i1 = min(N, i0 + chunk);
  ArgmaxAcc loc{-1e30f, -1};
  double abss = 0.0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const int s = (int)(i / n);
    const int64_t j = i - (int64_t)s * n;
    float kv = bcol[s] * ev(Z + j * d, zp);
    if (i == p) kv += extra;
    float sum = 0.0f;
    for (int q = 0; q < m; ++q) sum += scoef[q] * L[(int64_t)q * N + i];
    const float v = (kv - sum) * scale;
    L[(int64_t)m * N + i] = v;
    if (mask[i] > 0.5f) {
      const float dn = diag[i] - v * v;
      diag[i] = dn;
      loc = amax_merge(loc, ArgmaxAcc{dn, i});
      abss += (double)fabsf(dn);
    }
  }
  block_argmax_write(loc, abss, pv, pi, pa, blockIdx.x);
}

// diag[s n + j] = os_B[s][s] (a base-kernel diagonal of 1), mask 1.
__global__ void k_pc_init_kron(float* __restrict__ diag, float* __restrict__ mask, int64_t n,
                               int T, const float* __restrict__ osB) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n * T) {
    const int s = (int)(i / n);
    diag[i] = osB[s * T + s];
    mask[i] = 1.0f;
  }
}

template <class F>
void dispatch_column(Provider& pv, F&& launch) {
  const int d = pv.d;
  const float osk = pv.outputscale();
  if (pv.is_tree) launch(TreeColumn{pv.tree, pv.tparams.ptr});
  else if (pv.kind == KIND_RBF) launch(RadialColumn<KIND_RBF>{osk, d, pv.train.exp2_limit});
  else if (pv.kind == KIND_MATERN12) launch(RadialColumn<KIND_MATERN12>{osk, d, pv.train.exp2_limit});
  else if (pv.kind == KIND_MATERN32) launch(RadialColumn<KIND_MATERN32>{osk, d, pv.train.exp2_limit});
  else launch(RadialColumn<KIND_MATERN52>{osk, d, pv.train.exp2_limit});
}
}  // namespace

int pivoted_cholesky(Provider& pv, int rank, const PivotOptions& o, float* L,
                     hipStream_t st) {
  MGP_REQUIRE(o.method >= 0 && o.method <= 2, "precond_method must be 0, 1 or 2");
  const int64_t n = pv.n;
  PivotBufs b(n, rank, L, st);
  const float os = pv.kdiag();
  hipLaunchKernelGGL(k_pc_init, grid1(n), dim3(kBlock), 0, st, b.diag.ptr, b.mask.ptr, n, os);
  if (pv.nonstationary()) pv.diag_values(pv.train, n, b.diag.ptr);  // extract_diagonal
  auto launch_column = [&](int m) {
    const size_t shm = (size_t)(m + pv.d) * sizeof(float);
    const float* Z = pv.train.z.ptr;
    dispatch_column(pv, [&](auto ev) {
      hipLaunchKernelGGL(k_pc_column<decltype(ev)>, dim3(b.nb), dim3(kBlock), shm, st, ev, Z,
                         pv.d, n, m, L, b.diag.ptr, b.mask.ptr, b.coef.ptr, b.state.ptr, b.nb,
                         b.pvv.ptr, b.piv.ptr, b.pa.ptr);
    });
    MGP_HIP_CHECK(hipGetLastError());
  };
  // diagonal value k(x, x); vector-noise providers report the 1e-6 floor as
  // their noise (impl_get_noise, fn_ptr_module.py:673-679)
  return pivot_loop(b, rank, o, L, os, pv.has_noise_vec ? 1e-6f : pv.noise, st, launch_column);
}

int pivoted_cholesky_kron(Provider& base, int T, const float* osB_dev,
                          const std::vector<float>& osB, const float* task_noise_dev,
                          float noise_min, int rank, const PivotOptions& o, float* L,
                          hipStream_t st) {
  MGP_REQUIRE(o.method >= 0 && o.method <= 2, "precond_method must be 0, 1 or 2");
  MGP_REQUIRE(T >= 1 && (int)osB.size() == T * T, "os B must be T x T");
  const int64_t n = base.n, N = n * T;
  PivotBufs b(N, rank, L, st);
  hipLaunchKernelGGL(k_pc_init_kron, grid1(N), dim3(kBlock), 0, st, b.diag.ptr, b.mask.ptr, n,
                     T, osB_dev);
  float diag_value = 0.0f;  // max_s os B_ss (get_diagonal_value)
  for (int s = 0; s < T; ++s) diag_value = std::max(diag_value, osB[(size_t)s * T + s]);
  auto launch_column = [&](int m) {
    const size_t shm = (size_t)(m + base.d + T) * sizeof(float);
    const float* Z = base.train.z.ptr;
    dispatch_column(base, [&](auto ev) {
      hipLaunchKernelGGL(k_pc_column_kron<decltype(ev)>, dim3(b.nb), dim3(kBlock), shm, st, ev,
                         Z, base.d, n, T, osB_dev, task_noise_dev, noise_min, m, L, b.diag.ptr,
                         b.mask.ptr, b.coef.ptr, b.state.ptr, b.nb, b.pvv.ptr, b.piv.ptr,
                         b.pa.ptr);
    });
    MGP_HIP_CHECK(hipGetLastError());
  };
  return pivot_loop(b, rank, o, L, diag_value, noise_min, st, launch_column);
}

void syrk_ltl(const float* L, int64_t n, int k, double* M_dev, hipStream_t st,
              const float* wt) {
  const int tiles = (int)ceil_div(k, 16);
  const int splits = (int)std::max<int64_t>(1, std::min<int64_t>(64, ceil_div(n, 4096)));
  DevBuf<double> part;
  part.ensure((size_t)splits * k * k);
  hipLaunchKernelGGL(k_syrk_part, dim3(tiles, tiles, splits), dim3(256), 0, st, L, n, k,
                     splits, part.ptr, wt);
  hipLaunchKernelGGL(k_syrk_final, grid1((int64_t)k * k), dim3(kBlock), 0, st, part.ptr, k,
                     splits, M_dev);
  MGP_HIP_CHECK(hipGetLastError());
  MGP_HIP_CHECK(hipStreamSynchronize(st));  // `part` is released on return
}

// Row chunks of the L^T V partial products: >= 256 rows each, at most 256.
static int lt_chunks(int64_t n) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(256, ceil_div(n, 256)));
}

static void launch_lt_part(const float* L, int64_t n, int k, const float* v, int ncols, int nbw,
                           float* wpart, hipStream_t st, const float* rs = nullptr) {
  const dim3 grid((unsigned)nbw, (unsigned)ceil_div(k, 16), (unsigned)ceil_div(ncols, 16));
  hipLaunchKernelGGL(k_lt_part, grid, dim3(256), 0, st, L, n, k, v, ncols, nbw, wpart, rs);
}

// fp32-MFMA L^T v partials over row chunks of a multiple of 16 rows (ncols <= 64,
// k <= 256); returns the chunk count, 0 when the shape is not served.
static int launch_ltv_mfma(const float* L, int64_t n, int k, const float* v, int ncols,
                           WoodburyWork& w, float** wpart_out, hipStream_t st, const float* rs) {
  const int nct = (ncols + 15) / 16;
  if (nct > 4 || k > 256) return 0;
  int64_t chunk = round_up(ceil_div(n, cg_chunks(n)), 16);
  // k_ltv_mfma gives wave w the L tiles w, w + 4, ...: with k <= 16 only wave
  // 0 of a block has work, so quarter the chunks and run four times as many
  // blocks (LMC latents, 64 columns at N = 20000: 12.5 us per call before).
  if (nct >= 2 && k <= 16) chunk = round_up(ceil_div(chunk, 4), 16);
  const int nbw = (int)ceil_div(n, chunk);
  float* wpart = w.wpart.ensure((size_t)nbw * k * ncols);
  const bool vec4 = n % 4 == 0 && chunk % 4 == 0 && reinterpret_cast<uintptr_t>(L) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                    (rs == nullptr || reinterpret_cast<uintptr_t>(rs) % 16 == 0);
  const dim3 grid((unsigned)nbw), block(256);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, st, L, n, k, v, ncols, chunk, wpart, rs);
  };
  auto go16 = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64 * 16), 0, st, L, n, k, v, ncols, chunk, wpart, rs);
  };
  // 16 waves per chunk while the chunks do not fill the GPU, 4 otherwise
  const bool wide = nbw < kFewChunks;
#define MGP_LTV(NCT, U)                                                          \
  (vec4 ? (rs ? go(k_ltv_mfma<NCT, U, true, true>) : go(k_ltv_mfma<NCT, U, true, false>)) \
        : (rs ? go(k_ltv_mfma<NCT, U, false, true>) : go(k_ltv_mfma<NCT, U, false, false>)))
  switch (nct) {
    case 1:
      if (wide) {
        if (vec4)
          rs ? go16(k_ltv_c16<true, true, 4, 4>) : go16(k_ltv_c16<true, false, 4, 4>);
        else
          rs ? go16(k_ltv_c16<false, true, 4, 4>) : go16(k_ltv_c16<false, false, 4, 4>);
      } else {
        if (vec4)
          rs ? go(k_ltv_c16<true, true, 2, 2>) : go(k_ltv_c16<true, false, 2, 2>);
        else
          rs ? go(k_ltv_c16<false, true, 2, 2>) : go(k_ltv_c16<false, false, 2, 2>);
      }
      break;
    case 2: MGP_LTV(2, 1); break;
    case 3: MGP_LTV(3, 1); break;
    default: MGP_LTV(4, 1); break;
  }
#undef MGP_LTV
  MGP_HIP_CHECK(hipGetLastError());
  *wpart_out = wpart;
  return nbw;
}

// L^T v for ncols columns into wsum [ncols][k] (fp32 result of fp64 partial sums).
static void ltv(const float* L, int64_t n, int k, const float* v, int ncols, float* wsum,
                WoodburyWork& w, hipStream_t st, const float* rs) {
  float* wpart = nullptr;
  int nbw = launch_ltv_mfma(L, n, k, v, ncols, w, &wpart, st, rs);
  if (nbw == 0) {
    nbw = lt_chunks(n);
    wpart = w.wpart.ensure((size_t)nbw * k * ncols);
    launch_lt_part(L, n, k, v, ncols, nbw, wpart, st, rs);
  }
  const int64_t total = (int64_t)k * ncols;
  hipLaunchKernelGGL(k_part_reduce, dim3((unsigned)ceil_div(total, 16)), dim3(256), 0, st, wpart,
                     nbw, total, wsum);
  MGP_HIP_CHECK(hipGetLastError());
}

void woodbury_apply(const float* L, int64_t n, int k, const float* Minv, float noise,
                    const float* v, int ncols, float* out, WoodburyWork& w,
                    const float* dotv, int nb, double* dot_part, hipStream_t st,
                    const float* dinv) {
  const int cpad = (int)round_up(ncols, 16);
  float* ut = w.u.ensure((size_t)cpad * k);
  if (k <= kPartSolveMaxK && (int64_t)cg_chunks(n) * k <= kPartSolveMaxWork) {
    // chunk partials of L^T v, then their sum and the small solve in one launch
    float* wpart = nullptr;
    int nbw = launch_ltv_mfma(L, n, k, v, ncols, w, &wpart, st, dinv);
    if (nbw == 0) {
      nbw = lt_chunks(n);
      wpart = w.wpart.ensure((size_t)nbw * k * ncols);
      launch_lt_part(L, n, k, v, ncols, nbw, wpart, st, dinv);
    }
    hipLaunchKernelGGL(k_part_solve_t, dim3((unsigned)cpad, (unsigned)ceil_div(k, 16)),
                       dim3(1024), 0, st, wpart, nbw, k, ncols, Minv, ut);
  } else {
    float* wsum = w.wsum.ensure((size_t)ncols * k);
    ltv(L, n, k, v, ncols, wsum, w, st, dinv);
    hipLaunchKernelGGL(k_small_solve_t, dim3((unsigned)ceil_div((int64_t)k * cpad * 64, 256)),
                       dim3(256), 0, st, wsum, k, ncols, Minv, ut);
  }
  const int nbf = nb > 0 ? nb : cg_chunks(n);
  const dim3 grid((unsigned)nbf, (unsigned)ceil_div(ncols, 16));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, L, n, k, ut, ncols, 1.0f / noise, v, out,
                       dinv, dotv, nbf, dot_part);
  };
  const bool wide = nbf < kFewChunks;  // 16 waves per chunk for small n
  auto go_mfma = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(wide ? 1024 : 256), 0, st, L, n, k, ut, ncols,
                       1.0f / noise, v, out, dinv, dotv, nbf, dot_part);
  };
  if (k <= kWoodMfmaMaxK) {
    const bool vec4 = vec4_ok(n, nbf, {L, v, out, dinv, dotv});
#define MGP_WOOD_KS(V4, KS)                                                           \
  (dinv ? (dot_part ? go_mfma(k_woodbury_mfma<V4, true, true, KS>)                      \
                    : go_mfma(k_woodbury_mfma<V4, true, false, KS>))                    \
        : (dot_part ? go_mfma(k_woodbury_mfma<V4, false, true, KS>)                     \
                    : go_mfma(k_woodbury_mfma<V4, false, false, KS>)))
#define MGP_WOOD(V4) (wide ? MGP_WOOD_KS(V4, 4) : MGP_WOOD_KS(V4, 1))
    if (vec4)
      MGP_WOOD(true);
    else
      MGP_WOOD(false);
#undef MGP_WOOD
#undef MGP_WOOD_KS
  } else if (dinv) {
    dot_part ? go(k_woodbury_rows<true, true>) : go(k_woodbury_rows<true, false>);
  } else {
    dot_part ? go(k_woodbury_rows<false, true>) : go(k_woodbury_rows<false, false>);
  }
  MGP_HIP_CHECK(hipGetLastError());
}

void low_rank_sample(const float* L, int64_t n, int k, const float* zr, const float* zn,
                     float s, int ncols, float* out, hipStream_t st, const float* ds) {
  const dim3 grid((unsigned)ceil_div(std::max<int64_t>(n, 1), 256), (unsigned)ceil_div(ncols, 16));
  hipLaunchKernelGGL(k_low_rank_sample, grid, dim3(256), (size_t)16 * k * sizeof(float), st, L,
                     n, k, zr, zn, s, ncols, out, ds, 0, 0, 0);
  MGP_HIP_CHECK(hipGetLastError());
}

void gradient_traces(const Provider& pv, const float* Lf, const float* Rf, int ncols,
                     double* g_host, hipStream_t st) {
  if (pv.is_tree) {
    tree_grad_traces(pv.tree, pv.tparams.ptr, pv.train.z.ptr, pv.n, Lf, Rf, ncols, g_host,
                     pv.tree_gws, st);
    return;
  }
  const int d = pv.d;
  MGP_REQUIRE(d <= 32, "gradient kernel supports d <= 32");
  const double s = (double)kernel_scale(pv.kind);
  const double os = (double)pv.outputscale();
  const int nls = pv.ard ? d : 1;
  if (grad_trace_mfma_route(pv.kind, pv.train, d)) {
    // Matrix-core trace: per-dimension sums, then the pair-loop's layout.
    std::vector<double> acc(d + 1, 0.0);
    grad_trace_mfma(pv.kind, pv.train, d, Lf, Rf, ncols, acc.data(), pv.gtws, st);
    double iso = 0.0;
    for (int q = 0; q < d; ++q) iso += acc[q];
    for (int q = 0; q < nls; ++q)
      g_host[q] = os * (pv.ard ? acc[q] : iso) / (s * s * (double)pv.lengthscale(q));
    g_host[nls] = acc[d];
    return;
  }
  const int dm = d <= 1 ? 1 : d <= 2 ? 2 : d <= 4 ? 4 : d <= 8 ? 8 : d <= 16 ? 16 : 32;
  const int nterms = pv.ard ? d + 1 : 2;
  const int64_t nblk = ceil_div(pv.n, 256) * grad_splits(pv.n);
  DevBuf<double> part;
  part.ensure((size_t)nblk * nterms);
  std::vector<double> acc(nterms, 0.0), hpart((size_t)nblk * nterms);
  for (int c0 = 0; c0 < ncols; c0 += 16) {
    if (pv.kind == KIND_RBF) {
      if (pv.ard) launch_grad<KIND_RBF, true>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
      else launch_grad<KIND_RBF, false>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
    } else if (pv.kind == KIND_MATERN12) {
      if (pv.ard) launch_grad<KIND_MATERN12, true>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
      else launch_grad<KIND_MATERN12, false>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
    } else if (pv.kind == KIND_MATERN32) {
      if (pv.ard) launch_grad<KIND_MATERN32, true>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
      else launch_grad<KIND_MATERN32, false>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
    } else {
      if (pv.ard) launch_grad<KIND_MATERN52, true>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
      else launch_grad<KIND_MATERN52, false>(dm, pv.train.z.ptr, d, pv.n, Lf, Rf, ncols, c0, part.ptr, nterms, st);
    }
    MGP_HIP_CHECK(hipGetLastError());
    MGP_HIP_CHECK(hipMemcpyAsync(hpart.data(), part.ptr, hpart.size() * sizeof(double),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    for (int64_t b = 0; b < nblk; ++b)
      for (int t = 0; t < nterms; ++t) acc[t] += hpart[(size_t)b * nterms + t];
  }
  // Convert pair sums (scaled coordinates z = (x - c) * kernel_scale / ls) to
  // parameter derivatives: dk/dl_d = os h (dx_d)^2 / l_d^3 = os h dz_d^2 / (s^2 l_d).
  for (int q = 0; q < nls; ++q)
    g_host[q] = os * acc[q] / (s * s * (double)pv.lengthscale(q));
  g_host[nls] = acc[nterms - 1];
}

void multi_dot(const float* Q, int nvec, const float* w, int64_t n, double* part, int nb,
               double* out, hipStream_t st) {
  if (nvec <= 0) return;
  hipLaunchKernelGGL(k_multi_dot_part, dim3(nb, nvec), dim3(kBlock), 0, st, Q, w, n, nb, part);
  coldot_finalize(part, nb, nvec, out, st);
}

void multi_axpy(const float* Q, int nvec, const double* coef, float* w, int64_t n,
                hipStream_t st) {
  if (nvec <= 0) return;
  hipLaunchKernelGGL(k_multi_axpy, grid1(n), dim3(kBlock), 0, st, Q, nvec, coef, w, n);
  MGP_HIP_CHECK(hipGetLastError());
}

void gemm_nr_rr(const float* Q, const float* T, int64_t n, int r, float* S, hipStream_t st) {
  for (int c0 = 0; c0 < r; c0 += 16) {
    hipLaunchKernelGGL(k_gemm_nr_rr, grid1(n), dim3(kBlock), (size_t)r * 16 * sizeof(float),
                       st, Q, T, n, r, c0, S);
  }
  MGP_HIP_CHECK(hipGetLastError());
}

void love_variance(const float* V, int64_t m, int r, float diag, float* var, hipStream_t st,
                   const float* diag_vec) {
  hipLaunchKernelGGL(k_love_variance, grid1(m), dim3(kBlock), 0, st, V, m, r, diag, diag_vec,
                     var);
  MGP_HIP_CHECK(hipGetLastError());
}

void cross_ltl(const float* La, int ka, const float* Lb, int kb, int64_t n, double* M_dev,
               hipStream_t st) {
  if (ka <= 0 || kb <= 0) return;
  const int splits = (int)std::max<int64_t>(1, std::min<int64_t>(64, ceil_div(n, 4096)));
  DevBuf<double> part;
  part.ensure((size_t)splits * ka * kb);
  hipLaunchKernelGGL(k_cross_part, dim3((unsigned)ceil_div(ka, 16), (unsigned)ceil_div(kb, 16), splits),
                     dim3(256), 0, st, La, ka, Lb, kb, n, splits, part.ptr);
  hipLaunchKernelGGL(k_cross_final, grid1((int64_t)ka * kb), dim3(kBlock), 0, st, part.ptr,
                     (int64_t)ka * kb, splits, M_dev);
  MGP_HIP_CHECK(hipGetLastError());
  MGP_HIP_CHECK(hipStreamSynchronize(st));  // `part` is released on return
}

void lt_matmul(const float* L, int64_t n, int k, const float* V, int ncols, float* out,
               WoodburyWork& w, hipStream_t st) {
  if (k <= 0 || ncols <= 0) return;
  ltv(L, n, k, V, ncols, out, w, st, nullptr);
}

void l_matmul(const float* L, int64_t n, int k, const float* Z, int ncols, float* out,
              hipStream_t st) {
  if (ncols <= 0) return;
  if (k <= 0) {
    fill(out, n * (int64_t)ncols, 0.0f, st);
    return;
  }
  low_rank_sample(L, n, k, Z, nullptr, 0.0f, ncols, out, st);
}

void l_matmul_gather(const float* L, int64_t n, int k, const float* z, int gT, int gK, int goff,
                     int ncols, float* out, hipStream_t st) {
  if (ncols <= 0) return;
  if (k <= 0) {
    fill(out, n * (int64_t)ncols, 0.0f, st);
    return;
  }
  MGP_REQUIRE(gT > 0 && ncols % gT == 0, "gathered columns come in blocks of gT");
  const dim3 grid((unsigned)ceil_div(std::max<int64_t>(n, 1), 256), (unsigned)ceil_div(ncols, 16));
  hipLaunchKernelGGL(k_low_rank_sample, grid, dim3(256), (size_t)16 * k * sizeof(float), st, L,
                     n, k, z, nullptr, 0.0f, ncols, out, nullptr, gT, gK, goff);
  MGP_HIP_CHECK(hipGetLastError());
}

}  // namespace mgp
