// Host-side numerics (see host_numerics.h).
#include "host_numerics.h"

#include <algorithm>
#include <cmath>

namespace mgp {

bool tridiag_eigh(const std::vector<double>& diag, const std::vector<double>& off,
                  std::vector<double>& evals, std::vector<double>* evecs) {
  const int m = (int)diag.size();
  std::vector<double> d(diag), e(m, 0.0);
  for (int i = 0; i + 1 < m; ++i) e[i] = i < (int)off.size() ? off[i] : 0.0;
  if (evecs) {
    evecs->assign((size_t)m * m, 0.0);
    for (int i = 0; i < m; ++i) (*evecs)[(size_t)i * m + i] = 1.0;
  }
  const int max_sweeps = 1000 * std::max(m, 1);
  for (int l = 0; l < m; ++l) {
    int sweeps = 0;
    for (;;) {
      int mm = l;
      for (; mm < m - 1; ++mm) {
        const double dd = std::fabs(d[mm]) + std::fabs(d[mm + 1]);
        if (std::fabs(e[mm]) <= 1e-14 * dd) break;
      }
      if (mm == l) break;
      if (sweeps++ == max_sweeps) return false;
      // Wilkinson shift from the leading 2x2 block.
      double g = (d[l + 1] - d[l]) / (2.0 * e[l]);
      double r = std::hypot(g, 1.0);
      g = d[mm] - d[l] + e[l] / (g + std::copysign(r, g));
      double s = 1.0, c = 1.0, p = 0.0;
      int i = mm - 1;
      bool deflated = false;
      for (; i >= l; --i) {
        const double f = s * e[i], b = c * e[i];
        r = std::hypot(f, g);
        e[i + 1] = r;
        if (r == 0.0) {
          d[i + 1] -= p;
          e[mm] = 0.0;
          deflated = true;
          break;
        }
        s = f / r;
        c = g / r;
        g = d[i + 1] - p;
        r = (d[i] - g) * s + 2.0 * c * b;
        p = s * r;
        d[i + 1] = g + p;
        g = c * r - b;
        if (evecs) {
          double* V = evecs->data();
          for (int k = 0; k < m; ++k) {
            const double fv = V[(size_t)k * m + i + 1];
            V[(size_t)k * m + i + 1] = s * V[(size_t)k * m + i] + c * fv;
            V[(size_t)k * m + i] = c * V[(size_t)k * m + i] - s * fv;
          }
        }
      }
      if (deflated) continue;
      d[l] -= p;
      e[l] = g;
      e[mm] = 0.0;
    }
  }
  // Ascending order (selection sort keeps the eigenvector columns paired).
  for (int i = 0; i + 1 < m; ++i) {
    int k = i;
    for (int j = i + 1; j < m; ++j)
      if (d[j] < d[k]) k = j;
    if (k != i) {
      std::swap(d[i], d[k]);
      if (evecs) {
        double* V = evecs->data();
        for (int r = 0; r < m; ++r) std::swap(V[(size_t)r * m + i], V[(size_t)r * m + k]);
      }
    }
  }
  evals = d;
  return true;
}

static bool bad_entry(float v) { return v != v || v == 1e20f || v == -1e20f; }

float slq_logdet(const std::vector<std::vector<float>>& diags,
                 const std::vector<std::vector<float>>& offdiags, int64_t n) {
  float total = 0.0f;
  int valid = 0;
  for (size_t p = 0; p < diags.size(); ++p) {
    const auto& dg = diags[p];
    const int m = (int)dg.size();
    if (m == 0) continue;
    bool bad = false;
    std::vector<double> d(m), e(std::max(m - 1, 0));
    for (int i = 0; i < m && !bad; ++i) {
      if (bad_entry(dg[i])) bad = true;
      d[i] = dg[i];
    }
    for (int i = 0; i + 1 < m && !bad; ++i) {
      const float v = i < (int)offdiags[p].size() ? offdiags[p][i] : 0.0f;
      if (bad_entry(v)) bad = true;
      e[i] = v;
    }
    if (bad) continue;
    std::vector<double> ev, V;
    if (!tridiag_eigh(d, e, ev, &V)) continue;
    float max_eig = 1e-10f;
    for (int i = 0; i < m; ++i) max_eig = std::max(max_eig, (float)ev[i]);
    const float clamp = max_eig * 1e-6f;
    float term = 0.0f;
    for (int i = 0; i < m; ++i) {
      const float lam = (float)ev[i];
      const float v0 = (float)V[i];  // first component of eigenvector i
      if (lam < 0.0f || lam < clamp) continue;
      term += v0 * v0 * std::log(lam);
    }
    total += term;
    ++valid;
  }
  if (valid == 0) return 0.0f;
  return (float)n * (total / (float)valid);
}

bool cholesky(std::vector<double>& c, int k) {
  for (int i = 0; i < k; ++i) {
    for (int j = 0; j <= i; ++j) {
      double s = c[(size_t)i * k + j];
      for (int q = 0; q < j; ++q) s -= c[(size_t)i * k + q] * c[(size_t)j * k + q];
      if (i == j) {
        if (!(s > 0.0)) return false;
        c[(size_t)i * k + i] = std::sqrt(s);
      } else {
        c[(size_t)i * k + j] = s / c[(size_t)j * k + j];
      }
    }
    for (int j = i + 1; j < k; ++j) c[(size_t)i * k + j] = 0.0;
  }
  return true;
}

// Partial-pivot LU in place; returns false if singular.  perm receives row
// order, sign the permutation parity.
static bool lu(std::vector<double>& a, int k, std::vector<int>& perm, int& sign) {
  perm.resize(k);
  for (int i = 0; i < k; ++i) perm[i] = i;
  sign = 1;
  for (int c = 0; c < k; ++c) {
    int piv = c;
    for (int r = c + 1; r < k; ++r)
      if (std::fabs(a[(size_t)r * k + c]) > std::fabs(a[(size_t)piv * k + c])) piv = r;
    if (a[(size_t)piv * k + c] == 0.0) return false;
    if (piv != c) {
      for (int q = 0; q < k; ++q) std::swap(a[(size_t)piv * k + q], a[(size_t)c * k + q]);
      std::swap(perm[piv], perm[c]);
      sign = -sign;
    }
    for (int r = c + 1; r < k; ++r) {
      const double f = a[(size_t)r * k + c] / a[(size_t)c * k + c];
      a[(size_t)r * k + c] = f;
      for (int q = c + 1; q < k; ++q) a[(size_t)r * k + q] -= f * a[(size_t)c * k + q];
    }
  }
  return true;
}

bool spd_inverse(const std::vector<double>& A, int k, std::vector<double>& inv) {
  inv.assign((size_t)k * k, 0.0);
  std::vector<double> c(A);
  if (cholesky(c, k)) {
    // inv = C^{-T} C^{-1}
    std::vector<double> ci((size_t)k * k, 0.0);
    for (int i = 0; i < k; ++i) {
      ci[(size_t)i * k + i] = 1.0 / c[(size_t)i * k + i];
      for (int j = 0; j < i; ++j) {
        double s = 0.0;
        for (int q = j; q < i; ++q) s += c[(size_t)i * k + q] * ci[(size_t)q * k + j];
        ci[(size_t)i * k + j] = -s / c[(size_t)i * k + i];
      }
    }
    for (int i = 0; i < k; ++i)
      for (int j = 0; j < k; ++j) {
        double s = 0.0;
        for (int q = std::max(i, j); q < k; ++q) s += ci[(size_t)q * k + i] * ci[(size_t)q * k + j];
        inv[(size_t)i * k + j] = s;
      }
    return true;
  }
  std::vector<double> a(A);
  std::vector<int> perm;
  int sign;
  if (!lu(a, k, perm, sign)) return false;
  for (int col = 0; col < k; ++col) {
    std::vector<double> x(k, 0.0);
    for (int i = 0; i < k; ++i) {
      double s = perm[i] == col ? 1.0 : 0.0;
      for (int q = 0; q < i; ++q) s -= a[(size_t)i * k + q] * x[q];
      x[i] = s;
    }
    for (int i = k - 1; i >= 0; --i) {
      double s = x[i];
      for (int q = i + 1; q < k; ++q) s -= a[(size_t)i * k + q] * x[q];
      x[i] = s / a[(size_t)i * k + i];
    }
    for (int i = 0; i < k; ++i) inv[(size_t)i * k + col] = x[i];
  }
  return true;
}

double logdet_spd(const std::vector<double>& A, int k) {
  std::vector<double> c(A);
  if (cholesky(c, k)) {
    double s = 0.0;
    for (int i = 0; i < k; ++i) s += std::log(c[(size_t)i * k + i]);
    return 2.0 * s;
  }
  std::vector<double> a(A);
  std::vector<int> perm;
  int sign;
  if (!lu(a, k, perm, sign)) return -INFINITY;
  double s = 0.0;
  for (int i = 0; i < k; ++i) s += std::log(std::fabs(a[(size_t)i * k + i]));
  return s;
}

float softplus(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return std::exp(x);
  return std::log(1.0f + std::exp(x));
}

float inv_softplus(float y) {
  if (y > 20.0f) return y;
  if (y < 1e-6f) return std::log(y);
  return std::log(std::exp(y) - 1.0f);
}

float softplus_derivative(float x) {
  if (x > 20.0f) return 1.0f;
  if (x < -20.0f) return std::exp(x);
  return 1.0f / (1.0f + std::exp(-x));
}

float pow_float32(float base, int e) {
  if (e == 0) return 1.0f;
  if (e == 1) return base;
  float result = 1.0f, b = base;
  while (e > 0) {
    if (e & 1) result *= b;
    b *= b;
    e >>= 1;
  }
  return result;
}

float clip_gradient(float g, float max_grad) {
  if (g != g) return 0.0f;
  if (g > 1e30f || g < -1e30f) return 0.0f;
  if (g > max_grad) return max_grad;
  if (g < -max_grad) return -max_grad;
  return g;
}

float cosine_lr(float lr_max, int iteration, int total) {
  const float lr_min = lr_max / 20.0f;
  const float pi = 3.14159265358979f;
  const float t = (float)iteration / (float)std::max(total, 1);
  return lr_min + 0.5f * (lr_max - lr_min) * (1.0f + std::cos(pi * t));
}

void jacobi_eigen(const float* A, int k, float* V, float* evals) {
  std::vector<double> a(A, A + (size_t)k * k), v((size_t)k * k, 0.0);
  for (int i = 0; i < k; ++i) v[(size_t)i * k + i] = 1.0;
  const long max_rot = 100L * k * k;
  for (long it = 0; it < max_rot && k > 1; ++it) {
    double big = 0.0;
    int p = 0, q = 1;
    for (int i = 0; i < k; ++i)
      for (int j = i + 1; j < k; ++j)
        if (std::fabs(a[(size_t)i * k + j]) > big) {
          big = std::fabs(a[(size_t)i * k + j]);
          p = i;
          q = j;
        }
    if (big < 1e-12) break;
    const double app = a[(size_t)p * k + p], aqq = a[(size_t)q * k + q];
    const double apq = a[(size_t)p * k + q];
    // tan of the rotation angle: the smaller root of t^2 + 2 tau t - 1 = 0
    const double tau = (aqq - app) / (2.0 * apq);
    const double t = tau >= 0.0 ? 1.0 / (tau + std::sqrt(1.0 + tau * tau))
                                : -1.0 / (-tau + std::sqrt(1.0 + tau * tau));
    const double c = 1.0 / std::sqrt(1.0 + t * t), s = t * c;
    for (int i = 0; i < k; ++i) {  // columns p, q
      const double ip = a[(size_t)i * k + p], iq = a[(size_t)i * k + q];
      a[(size_t)i * k + p] = c * ip - s * iq;
      a[(size_t)i * k + q] = s * ip + c * iq;
    }
    for (int j = 0; j < k; ++j) {  // rows p, q
      const double pj = a[(size_t)p * k + j], qj = a[(size_t)q * k + j];
      a[(size_t)p * k + j] = c * pj - s * qj;
      a[(size_t)q * k + j] = s * pj + c * qj;
    }
    a[(size_t)p * k + p] = app - t * apq;
    a[(size_t)q * k + q] = aqq + t * apq;
    a[(size_t)p * k + q] = 0.0;
    a[(size_t)q * k + p] = 0.0;
    for (int i = 0; i < k; ++i) {
      const double ip = v[(size_t)i * k + p], iq = v[(size_t)i * k + q];
      v[(size_t)i * k + p] = c * ip - s * iq;
      v[(size_t)i * k + q] = s * ip + c * iq;
    }
  }
  std::vector<double> e(k);
  for (int i = 0; i < k; ++i) e[i] = a[(size_t)i * k + i];
  for (int i = 0; i < k; ++i) {  // selection sort, ascending
    int mi = i;
    for (int j = i + 1; j < k; ++j)
      if (e[j] < e[mi]) mi = j;
    if (mi != i) {
      std::swap(e[i], e[mi]);
      for (int r = 0; r < k; ++r) std::swap(v[(size_t)r * k + i], v[(size_t)r * k + mi]);
    }
  }
  for (int i = 0; i < k; ++i) evals[i] = (float)e[i];
  for (size_t i = 0; i < (size_t)k * k; ++i) V[i] = (float)v[i];
}

}  // namespace mgp
