// Provider state management and the matvec entry points it serves.
#include "provider.h"

#include <algorithm>
#include <cmath>

namespace mgp {

void Provider::refresh_coords() {
  std::vector<float> coef(2 * (size_t)d);
  const float base = kernel_scale(kind);
  for (int k = 0; k < d; ++k) {
    const float ls = lengthscale(k);
    MGP_REQUIRE(std::isfinite(ls) && ls > 0.f, "lengthscales must be finite and > 0");
    coef[k] = (float)center[k];
    coef[d + k] = base / ls;
  }
  co.d = d;
  co.coef.ensure(coef.size());
  MGP_HIP_CHECK(hipMemcpyAsync(co.coef.ptr, coef.data(), coef.size() * sizeof(float),
                               hipMemcpyHostToDevice, st));
  pack_points(X.ptr, n, co, train, st);
}

void Provider::pack(const float* X_dev, int64_t m, PackedPoints& pp) {
  pack_points(X_dev, m, co, pp, st);
}

void Provider::forward(const float* V, int ncols, float* out) {
  MatvecArgs a;
  a.kind = kind;
  a.outputscale = outputscale();
  a.noise = noise;
  a.square = true;
  a.m = n;
  a.n = n;
  a.ncols = ncols;
  if (!gram_form_ok(kind, train, train)) {
    direct_matvec(a, train, train, d, V, out, st);
    return;
  }
  fused_matvec(a, train, train, V, out, ws, st);
}

void Provider::cross(const PackedPoints& rows, const float* V, int ncols,
                     float* out) {
  MatvecArgs a;
  a.kind = kind;
  a.outputscale = outputscale();
  a.noise = 0.f;
  a.square = false;
  a.m = rows.n;
  a.n = n;
  a.ncols = ncols;
  if (!gram_form_ok(kind, rows, train)) {
    direct_matvec(a, rows, train, d, V, out, st);
    return;
  }
  fused_matvec(a, rows, train, V, out, ws, st);
}

}  // namespace mgp
