// Provider state management and the matvec entry points it serves.
#include "provider.h"


#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <set>
#include <cmath>

namespace mgp {

void Provider::refresh_coords() {
  if (is_tree) {
    for (int q = 0; q < nparams; ++q)
      MGP_REQUIRE(std::isfinite(params[q]) && params[q] > 0.f,
                  "kernel tree parameters must be finite and > 0");
    tparams.ensure((size_t)nparams + (size_t)tree.table_size);
    MGP_HIP_CHECK(hipMemcpyAsync(tparams.ptr, params.data(), (size_t)nparams * sizeof(float),
                                 hipMemcpyHostToDevice, st));
    if (tree.table_size > 0)
      MGP_HIP_CHECK(hipMemcpyAsync(tparams.ptr + nparams, cat_tables.data(),
                                   (size_t)tree.table_size * sizeof(float),
                                   hipMemcpyHostToDevice, st));
    pack(X.ptr, n, train);
    if (materialized) fill_dense();
    MGP_HIP_CHECK(hipStreamSynchronize(st));  // params may change after return
    return;
  }
  std::vector<float> coef(2 * (size_t)d);
  const float base = kernel_scale(kind);
  for (int k = 0; k < d; ++k) {
    const float ls = lengthscale(k);
    MGP_REQUIRE(std::isfinite(ls) && ls > 0.f, "lengthscales must be finite and > 0");
    coef[k] = (float)center[k];
    coef[d + k] = base / ls;
  }
  co.d = d;
  co.exp2_limit = exp2_limit(kind, ard);
  co.coef.ensure(coef.size());
  MGP_HIP_CHECK(hipMemcpyAsync(co.coef.ptr, coef.data(), coef.size() * sizeof(float),
                               hipMemcpyHostToDevice, st));
  pack_points(X.ptr, n, co, train, st);
  if (materialized) fill_dense();
  // Gradient scales: dk/dl_q = os h dz_q^2 / (s^2 l_q); dk/dos = k/os.
  std::vector<float> gs((size_t)nparams);
  const double s2 = (double)base * (double)base;
  for (int q = 0; q < nparams - 1; ++q)
    gs[q] = (float)((double)outputscale() / (s2 * (double)params[q]));
  gs[nparams - 1] = 1.0f;
  gscale.ensure(gs.size());
  MGP_HIP_CHECK(hipMemcpyAsync(gscale.ptr, gs.data(), gs.size() * sizeof(float),
                               hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));  // gs is released on return
}

void Provider::gradient(const float* V, int ncols, float* out) {
  MGP_REQUIRE(!is_tree, "per-parameter gradient products are not available for kernel trees");
  gradient_matvec(kind, ard, train, d, outputscale(), gscale.ptr, V, ncols, out, st);
}

namespace {
// out[c][i] += dvec[i] * V[c][i]
__global__ void k_add_diag_vec(float* __restrict__ out, const float* __restrict__ V,
                               const float* __restrict__ dvec, int64_t n, int ncols) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * ncols) return;
  out[idx] = fmaf(dvec[idx % n], V[idx], out[idx]);
}
}  // namespace

void Provider::set_noise_vector(const float* host) {
  if (!host) {
    has_noise_vec = false;
    learned_noise_mode = 0;
    return;
  }
  for (int64_t i = 0; i < n; ++i)
    MGP_REQUIRE(std::isfinite(host[i]) && host[i] > 0.f, "noise vector entries must be finite and > 0");
  noise_vec.ensure((size_t)n);
  MGP_HIP_CHECK(hipMemcpyAsync(noise_vec.ptr, host, (size_t)n * sizeof(float),
                               hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  has_noise_vec = true;
}

void Provider::load_noise_vector(const float* host) {
  noise_vec.ensure((size_t)n);
  MGP_HIP_CHECK(hipMemcpyAsync(noise_vec.ptr, host, (size_t)n * sizeof(float),
                               hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  has_noise_vec = true;
}

float Provider::kdiag_max() {
  if (!is_tree) return outputscale();
  float* d = io_c.ensure((size_t)n);
  diag_values(train, n, d);
  std::vector<float> h((size_t)n);
  MGP_HIP_CHECK(hipMemcpyAsync(h.data(), d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  float mx = 0.f;
  for (float v : h) mx = std::max(mx, std::fabs(v));
  return mx;
}

void Provider::fill_dense() {
  // The symmetric half (products with <= 16 right-hand sides) after every
  // parameter update; the full matrix on the first wider product after it.
  float kmax = kdiag_max();
  MGP_REQUIRE(std::isfinite(kmax), "kernel diagonal is not finite");
  if (!(kmax > 0.f)) kmax = 1.f;  // K = 0: any scale
  dense_alloc_half(dense, n, kmax);
  const int64_t nb = dense.blocks();
  if (!is_tree) {
    // only the stored blocks, evaluated straight into the split storage
    fill_dense_half(kind, outputscale(), train, d, dense.shift, nb, dense.half.ptr, st);
  } else {
    float* tmp = io_c.ensure((size_t)256 * n);
    for (int64_t b = 0; b < nb; ++b) {
      const int64_t r0 = b * 256, nr = std::min<int64_t>(256, n - r0);
      if (nr > 0) fill_block(train, r0, nr, tmp);
      dense_pack_half(tmp, b, std::max<int64_t>(nr, 0), dense, st);
    }
  }
  dense.half_valid = true;
  dense.full_valid = false;
}

void Provider::fill_dense_full() {
  if (dense.full_valid) return;
  const double npad = (double)round_up(n, 256);
  MGP_REQUIRE(npad * npad * 6.0 <= 250e9,
              "the full dense K beside its symmetric half does not fit the device");
  float kmax = kdiag_max();
  MGP_REQUIRE(std::isfinite(kmax), "kernel diagonal is not finite");
  if (!(kmax > 0.f)) kmax = 1.f;
  dense_alloc(dense, n, kmax, st);
  // fp32 rows in blocks of <= 32M entries, each packed into the split storage
  const int64_t rows = std::max<int64_t>(1, std::min<int64_t>(n, ((int64_t)1 << 25) / n));
  float* tmp = io_c.ensure((size_t)rows * n);
  for (int64_t r0 = 0; r0 < n; r0 += rows) {
    const int64_t nr = std::min(rows, n - r0);
    fill_block(train, r0, nr, tmp);
    dense_pack_rows(tmp, r0, nr, dense, st);
  }
  dense.full_valid = true;
}

void Provider::diag_values(const PackedPoints& pts, int64_t m, float* out) {
  if (is_tree) {
    tree_self_values(tree, tparams.ptr, pts.z.ptr, m, out, st);
    return;
  }
  std::vector<float> h((size_t)std::max<int64_t>(m, 1), kdiag());
  MGP_HIP_CHECK(hipMemcpyAsync(out, h.data(), (size_t)m * sizeof(float), hipMemcpyHostToDevice, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

void Provider::fill_block(const PackedPoints& rows, int64_t r0, int64_t nrows, float* out) {
  if (is_tree) {
    tree_fill(tree, tparams.ptr, rows.z.ptr, r0, nrows, train.z.ptr, n, out, st);
    return;
  }
  fill_cross(kind, outputscale(), rows, r0, nrows, train, d, out, st);
}

void Provider::materialize() {
  if (!materialized) {
    const double bytes = (double)round_up(n, 256) * (double)round_up(n, 256) * sizeof(float);
    MGP_REQUIRE(bytes <= 200e9, "dense K of this size does not fit the device");
    materialized = true;
  }
  fill_dense();
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

void Provider::pack(const float* X_dev, int64_t m, PackedPoints& pp) {
  if (is_tree) {  // raw coordinates only (tree products read them directly)
    pp.n = m;
    pp.ntiles = 0;
    pp.kb = 0;
    pp.max_norm = 0.f;
    pp.z.ensure((size_t)std::max<int64_t>(m, 1) * d);
    if (m > 0)
      MGP_HIP_CHECK(hipMemcpyAsync(pp.z.ptr, X_dev, (size_t)m * d * sizeof(float),
                                   hipMemcpyDeviceToDevice, st));
    return;
  }
  pack_points(X_dev, m, co, pp, st);
}

void Provider::forward(const float* V, int ncols, float* out, MatvecWorkspace* wsp) {
  forward_scalar(V, ncols, out, wsp);
  if (has_noise_vec) {
    const int64_t total = n * (int64_t)ncols;
    hipLaunchKernelGGL(k_add_diag_vec, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       out, V, noise_vec.ptr, n, ncols);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

void Provider::forward_scalar(const float* V, int ncols, float* out, MatvecWorkspace* wsp) {
  const float noise = scalar_noise();
  MatvecArgs a;
  a.kind = kind;
  a.outputscale = outputscale();
  a.noise = noise;
  a.square = true;
  a.m = n;
  a.n = n;
  a.ncols = ncols;
  if (materialized) {
    const char* env = std::getenv("MGP_SYM_MATVEC");
    const bool sym_off = env != nullptr && env[0] == '0';
    if (ncols <= 16 && dense.half_valid && !sym_off) {
      dense_sym_forward(dense, V, ncols, noise, out, dense_ws, st);
    } else {
      fill_dense_full();
      dense_forward(dense, V, ncols, noise, out, dense_ws, st);
    }
    return;
  }
  if (is_tree) {
    tree_matvec(tree, tparams.ptr, train.z.ptr, n, train.z.ptr, n, V, ncols, noise, true, out,
                tree_ws, st);
    return;
  }
  if (!gram_form_ok(kind, train, train)) {
    direct_matvec(a, train, train, d, V, out, st);
    return;
  }
  fused_matvec(a, train, train, V, out, wsp ? *wsp : ws, st);
}

bool Provider::column_independent_products() const {
  return fused_route() && symmetric_route_taken(train, 1) && symmetric_route_taken(train, 2);
}

bool Provider::fused_route() const {
  return !is_tree && !materialized && gram_form_ok(kind, train, train);
}

void Provider::forward_mixed(const float* V, int ncols, const float* mix, int T, bool accumulate,
                             float* out, PackedRhs* reuse) {
  MGP_REQUIRE(fused_route(), "forward_mixed needs the fused tile route");
  MatvecArgs a;
  a.kind = kind;
  a.outputscale = outputscale();
  a.noise = noise;
  a.square = true;
  a.m = n;
  a.n = n;
  a.ncols = ncols;
  a.mix = mix;
  a.mix_T = T;
  a.mix_accumulate = accumulate;
  a.reuse = reuse;
  fused_matvec(a, train, train, V, out, ws, st);
}

void Provider::cross(const PackedPoints& rows, const float* V, int ncols,
                     float* out) {
  if (is_tree) {
    tree_matvec(tree, tparams.ptr, rows.z.ptr, rows.n, train.z.ptr, n, V, ncols, 0.f, false,
                out, tree_ws, st);
    return;
  }
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

namespace {
std::mutex g_provider_mu;
std::set<Provider*> g_providers;
}  // namespace

Provider* checked_provider(void* h) {
  auto* p = static_cast<Provider*>(h);
  std::lock_guard<std::mutex> lk(g_provider_mu);
  MGP_REQUIRE(h != nullptr, "null provider handle");
  MGP_REQUIRE(g_providers.count(p) != 0, "unknown or destroyed provider handle");
  return p;
}

void register_provider(Provider* p) {
  std::lock_guard<std::mutex> lk(g_provider_mu);
  g_providers.insert(p);
}

void unregister_provider(Provider* p) {
  std::lock_guard<std::mutex> lk(g_provider_mu);
  g_providers.erase(p);
}

}  // namespace mgp
