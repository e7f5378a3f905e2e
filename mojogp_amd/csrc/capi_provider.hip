// C ABI: provider lifecycle and kernel products.  Declarations and the
// reference interface each entry point replaces are in include/mojogp_amd.h.
#include <chrono>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

#include "mojogp_amd.h"
#include "provider.h"
#include "solver.h"

namespace mgp {

thread_local std::string g_last_error;
void set_last_error(const std::string& msg) { g_last_error = msg; }

static Provider* as_provider(void* h) { return checked_provider(h); }

// Plain streaming copy used to calibrate HBM byte counters.
__global__ void k_calibration_copy(const float4* __restrict__ a,
                                   float4* __restrict__ b, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
    b[i] = a[i];
}

// Work buffers of the allocation-free forward matvec
// (mgp_forward_matvec_device_noalloc): one fixed array per GPU, held until the
// process ends.  Host code never passes `scratch` itself to a kernel (on the
// host the name is only a stand-in); it uses the device address that
// hipGetSymbolAddress returns for the current device, kept per device below.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
  uint8_t* ptr = nullptr;
  hipError_t err = hipSuccess;
  bool tried = false;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxScratchDevices];
// One lock per device, held by an allocation-free call from its first use of
// the device's array until its stream has drained: calls that would share
// the array run one after another instead of racing.
std::mutex g_noalloc_mu[kMaxScratchDevices];

// Resolves this device's scratch address once, with `dev` current (called at
// provider set-up).  A failure is recorded, not raised: it only disables the
// allocation-free entry point, which reports it.
static void setup_scratch(int dev) {
  if (dev < 0 || dev >= kMaxScratchDevices) return;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  ScratchSlot& s = g_scratch[dev];
  if (s.tried) return;
  s.tried = true;
  void* p = nullptr;
  s.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (s.err == hipSuccess && p != nullptr) {
    s.ptr = static_cast<uint8_t*>(p);
  } else {
    if (s.err == hipSuccess) s.err = hipErrorInvalidSymbol;
    (void)hipGetLastError();
  }
}

static uint8_t* scratch_of(int dev) {
  MGP_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const ScratchSlot& s = g_scratch[dev];
  MGP_REQUIRE(s.tried, "scratch of this device was never set up");
  if (s.ptr == nullptr)
    throw Error(ST_HIP, std::string("scratch unavailable on this device: hipGetSymbolAddress: ") +
                            hipGetErrorString(s.err));
  return s.ptr;
}

}  // namespace mgp

using namespace mgp;

extern "C" {

int mgp_last_error(char* buf, size_t len) {
  const std::string& m = g_last_error;
  if (buf && len > 0) {
    const size_t k = std::min(len - 1, m.size());
    std::memcpy(buf, m.data(), k);
    buf[k] = '\0';
  }
  return (int)m.size();
}

const char* mgp_version(void) { return "mojogp_amd 0.1.0 gfx950"; }

int mgp_device_count(int* out) {
  return guarded([&] {
    int c = 0;
    MGP_HIP_CHECK(hipGetDeviceCount(&c));
    *out = c;
  });
}

namespace {
// Shared tail of provider creation: parameters, stream, device inputs and the
// first packing.  Owns pv (deleted on failure).
Provider* finish_provider(Provider* pv, int d, int64_t n, const float* X, const float* params,
                          int nparams, float noise) {
  try {
    pv->d = d;
    pv->n = n;
    pv->nparams = nparams;
    pv->params.assign(params, params + nparams);
    pv->noise = noise;
    pv->center.assign(d, 0.0);
    for (int64_t i = 0; i < n; ++i)
      for (int k = 0; k < d; ++k) pv->center[k] += (double)X[i * d + k];
    for (int k = 0; k < d; ++k) pv->center[k] /= (double)n;
    MGP_HIP_CHECK(hipGetDevice(&pv->device));
    setup_scratch(pv->device);
    MGP_HIP_CHECK(hipStreamCreateWithFlags(&pv->st, hipStreamNonBlocking));
    pv->X.ensure((size_t)n * d);
    MGP_HIP_CHECK(hipMemcpyAsync(pv->X.ptr, X, (size_t)n * d * sizeof(float),
                                 hipMemcpyHostToDevice, pv->st));
    pv->refresh_coords();
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  } catch (...) {
    if (pv->st) (void)hipStreamDestroy(pv->st);
    delete pv;
    throw;
  }
  register_provider(pv);
  return pv;
}
}  // namespace

int mgp_init_provider(int kind, int ard, int d, int64_t n, const float* X,
                      const float* params, int nparams, float noise,
                      void** out_handle) {
  return guarded([&] {
    MGP_REQUIRE(out_handle != nullptr, "out_handle is null");
    *out_handle = nullptr;
    MGP_REQUIRE(valid_kind(kind),
                "kernel kind must be 0 (RBF), 1 (Matern52), 2 (Matern12) or 3 (Matern32)");
    MGP_REQUIRE(d >= 1 && d <= 32, "input dimension must be in [1, 32]");
    MGP_REQUIRE(n >= 1, "n must be >= 1");
    MGP_REQUIRE(X != nullptr && params != nullptr, "null input array");
    const int expect = ard ? d + 1 : 2;
    MGP_REQUIRE(nparams == expect,
                "params has " + std::to_string(nparams) + " values, expected " +
                    std::to_string(expect));
    MGP_REQUIRE(std::isfinite(noise) && noise >= 0.f, "noise must be finite and >= 0");
    for (int p = 0; p < nparams; ++p)
      MGP_REQUIRE(std::isfinite(params[p]) && params[p] > 0.f,
                  "kernel parameters must be finite and > 0");
    auto* pv = new Provider();
    pv->kind = kind;
    pv->ard = ard != 0;
    *out_handle = finish_provider(pv, d, n, X, params, nparams, noise);
  });
}

int mgp_init_provider_tree(const int* spec, int spec_len, int d, int64_t n, const float* X,
                           const float* params, int nparams, float noise, void** out_handle) {
  return guarded([&] {
    MGP_REQUIRE(out_handle != nullptr, "out_handle is null");
    *out_handle = nullptr;
    const KernelTree t = parse_kernel_tree(spec, spec_len);
    MGP_REQUIRE(t.d == d, "kernel tree spec was built for another input dimension");
    MGP_REQUIRE(t.nparams == nparams,
                "params has " + std::to_string(nparams) + " values, the kernel tree expects " +
                    std::to_string(t.nparams));
    MGP_REQUIRE(n >= 1, "n must be >= 1");
    MGP_REQUIRE(X != nullptr && params != nullptr, "null input array");
    MGP_REQUIRE(std::isfinite(noise) && noise >= 0.f, "noise must be finite and >= 0");
    for (int p = 0; p < nparams; ++p)
      MGP_REQUIRE(std::isfinite(params[p]) && params[p] > 0.f,
                  "kernel parameters must be finite and > 0");
    auto* pv = new Provider();
    pv->kind = KIND_TREE;
    pv->ard = false;
    pv->is_tree = true;
    pv->tree = t;
    pv->cat_tables.assign((size_t)t.table_size, 0.0f);  // identity tables until set
    for (int l = 0; l < t.nleaves; ++l)
      if (t.leaf[l].kind == KIND_CAT)
        for (int a = 0; a < t.leaf[l].ard; ++a)
          pv->cat_tables[(size_t)t.leaf[l].p0 + (size_t)a * t.leaf[l].ard + a] = 1.0f;
    *out_handle = finish_provider(pv, d, n, X, params, nparams, noise);
  });
}

int mgp_destroy_provider(void* h) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    unregister_provider(pv);
    if (pv->st) (void)hipStreamSynchronize(pv->st);
    if (pv->ws.ev0) (void)hipEventDestroy(pv->ws.ev0);
    if (pv->ws.ev1) (void)hipEventDestroy(pv->ws.ev1);
    hipStream_t st = pv->st;
    delete pv;  // frees device buffers
    if (st) (void)hipStreamDestroy(st);
  });
}

int mgp_materialize(void* h) {
  return guarded([&] { as_provider(h)->materialize(); });
}

int mgp_update_params(void* h, const float* params, int nparams) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(nparams == pv->nparams, "wrong number of kernel parameters");
    for (int p = 0; p < nparams; ++p)
      MGP_REQUIRE(std::isfinite(params[p]) && params[p] > 0.f,
                  "kernel parameters must be finite and > 0");
    pv->params.assign(params, params + nparams);
    pv->refresh_coords();
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_update_noise(void* h, float noise) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(std::isfinite(noise) && noise >= 0.f, "noise must be finite and >= 0");
    pv->noise = noise;
  });
}

// Under a noise vector the reference reports a 1e-6 floor (impl_get_noise,
// fn_ptr_module.py:673-679).
int mgp_get_noise(void* h, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    *out = pv->has_noise_vec ? 1e-6f : pv->noise;
  });
}

int mgp_get_diagonal_value(void* h, float* out) {
  return guarded([&] { *out = as_provider(h)->kdiag(); });
}

// Fn-pointer exports: the reference's non-raising provider signatures
// (erased_provider.mojo:43-50), whose addresses go into the provider dict.
// They cannot return a status: a failure is recorded for mgp_last_error and
// the call returns NaN / -1 / null (update_noise leaves the noise unchanged).
void mgp_fn_update_noise(intptr_t h, float noise) {
  (void)mgp_update_noise(reinterpret_cast<void*>(h), noise);
}

float mgp_fn_get_noise(intptr_t h) {
  float v = std::nanf("");
  (void)mgp_get_noise(reinterpret_cast<void*>(h), &v);
  return v;
}

intptr_t mgp_fn_get_noise_mode(intptr_t h) {
  intptr_t mode = -1;
  (void)guarded([&] {
    const Provider* pv = as_provider(reinterpret_cast<void*>(h));
    mode = pv->learned_noise_mode > 0 ? pv->learned_noise_mode : (pv->has_noise_vec ? 1 : 0);
  });
  return mode;
}

float* mgp_fn_get_noise_vector_ptr(intptr_t h) {
  float* p = nullptr;
  (void)guarded([&] {
    Provider* pv = as_provider(reinterpret_cast<void*>(h));
    p = pv->has_noise_vec ? pv->noise_vec.ptr : nullptr;
  });
  return p;
}

float mgp_fn_get_diagonal_value(intptr_t h) {
  float v = std::nanf("");
  (void)mgp_get_diagonal_value(reinterpret_cast<void*>(h), &v);
  return v;
}

int mgp_provider_info(void* h, int64_t* n, int* d, int* nparams, int* kind,
                      int* ard) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    if (n) *n = pv->n;
    if (d) *d = pv->d;
    if (nparams) *nparams = pv->nparams;
    if (kind) *kind = pv->kind;
    if (ard) *ard = pv->ard ? 1 : 0;
  });
}

int mgp_forward_matvec(void* h, const float* V, int ncols, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
    MGP_REQUIRE(V && out, "null array");
    const size_t tot = (size_t)pv->n * ncols;
    float* dv = pv->io_a.ensure(tot);
    float* dout = pv->io_b.ensure(tot);
    MGP_HIP_CHECK(hipMemcpyAsync(dv, V, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    pv->forward(dv, ncols, dout);
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout, tot * sizeof(float), hipMemcpyDeviceToHost, pv->st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_forward_matvec_device(void* h, const float* V_dev, int ncols,
                              float* out_dev) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
    MGP_REQUIRE(V_dev && out_dev, "null device array");
    pv->forward(V_dev, ncols, out_dev);
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_forward_matvec_device_noalloc(void* h, const float* V_dev, int ncols, float* out_dev) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
    MGP_REQUIRE(V_dev && out_dev, "null device array");
    MGP_REQUIRE(!pv->is_tree, "the allocation-free matvec does not serve kernel trees");
    MGP_REQUIRE(!pv->materialized, "the allocation-free matvec does not serve the materialized "
                                   "route");
    uint8_t* arena = scratch_of(pv->device);
    std::lock_guard<std::mutex> lk(g_noalloc_mu[pv->device]);
    MatvecWorkspace w;  // fixed-arena mode: its own buffers stay unallocated
    w.arena = arena;
    w.arena_bytes = kNoAllocScratchBytes;
    if (pv->fused_route()) {
      const size_t need = fused_matvec_min_arena(pv->train, ncols);
      MGP_REQUIRE(need <= kNoAllocScratchBytes,
                  "n = " + std::to_string(pv->n) + " with " + std::to_string(ncols) +
                      " columns needs " + std::to_string(need) +
                      " bytes of scratch; the allocation-free matvec holds at most " +
                      std::to_string(kNoAllocScratchBytes) + " (64 MiB)");
    }
    pv->forward(V_dev, ncols, out_dev, &w);
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_direct_matvec(void* h, const float* V, int ncols, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
    const size_t tot = (size_t)pv->n * ncols;
    float* dv = pv->io_a.ensure(tot);
    float* dout = pv->io_b.ensure(tot);
    MGP_HIP_CHECK(hipMemcpyAsync(dv, V, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    MGP_REQUIRE(!pv->is_tree, "the direct radial matvec does not serve kernel trees");
    MatvecArgs a;
    a.kind = pv->kind;
    a.outputscale = pv->outputscale();
    a.noise = pv->noise;
    a.square = true;
    a.m = a.n = pv->n;
    a.ncols = ncols;
    direct_matvec(a, pv->train, pv->train, pv->d, dv, dout, pv->st);
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout, tot * sizeof(float), hipMemcpyDeviceToHost, pv->st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_cross_matvec(void* h, const float* Xs, int64_t m, const float* V,
                     int ncols, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(m >= 1 && ncols >= 1, "m and ncols must be >= 1");
    MGP_REQUIRE(Xs && V && out, "null array");
    float* dx = pv->Xs.ensure((size_t)m * pv->d);
    MGP_HIP_CHECK(hipMemcpyAsync(dx, Xs, (size_t)m * pv->d * sizeof(float),
                                 hipMemcpyHostToDevice, pv->st));
    pv->pack(dx, m, pv->test);
    const size_t tv = (size_t)pv->n * ncols, to = (size_t)m * ncols;
    float* dv = pv->io_a.ensure(tv);
    float* dout = pv->io_b.ensure(to);
    MGP_HIP_CHECK(hipMemcpyAsync(dv, V, tv * sizeof(float), hipMemcpyHostToDevice, pv->st));
    pv->cross(pv->test, dv, ncols, dout);
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout, to * sizeof(float), hipMemcpyDeviceToHost, pv->st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_set_categorical_tables(void* h, const float* tables, int size) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(pv->is_tree, "categorical tables belong to kernel-tree providers");
    MGP_REQUIRE(size == pv->tree.table_size,
                "expected " + std::to_string(pv->tree.table_size) + " table entries");
    MGP_REQUIRE(tables != nullptr || size == 0, "null tables");
    for (int e = 0; e < size; ++e)
      MGP_REQUIRE(std::isfinite(tables[e]), "categorical tables must be finite");
    pv->cat_tables.assign(tables, tables + size);
    pv->refresh_coords();
  });
}

int mgp_set_learned_noise(void* h, int mode, const int* group_ids, int num_groups) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(mode == 0 || (mode >= 2 && mode <= 4), "learned noise mode must be 0, 2, 3 or 4");
    if (mode == 0) {
      pv->learned_noise_mode = 0;
      return;
    }
    MGP_REQUIRE(pv->has_noise_vec, "set the initial noise vector before a learned noise mode");
    if (mode == 3) {
      MGP_REQUIRE(group_ids != nullptr && num_groups >= 1, "grouped noise needs group ids");
      for (int64_t i = 0; i < pv->n; ++i)
        MGP_REQUIRE(group_ids[i] >= 0 && group_ids[i] < num_groups,
                    "noise group id outside [0, num_groups)");
      pv->noise_groups.assign(group_ids, group_ids + pv->n);
      pv->num_noise_groups = num_groups;
    }
    pv->learned_noise_mode = mode;
  });
}

int mgp_set_noise_vector(void* h, const float* noise_vec) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    pv->set_noise_vector(noise_vec);
  });
}

// k(x, x) of a stationary kernel is the outputscale (r = 1e-10 for Matern
// rounds to exactly os in fp32).
int mgp_extract_diagonal(void* h, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    if (pv->nonstationary()) {
      DevBuf<float> d;
      pv->diag_values(pv->train, pv->n, d.ensure((size_t)pv->n));
      MGP_HIP_CHECK(hipMemcpyAsync(out, d.ptr, (size_t)pv->n * sizeof(float),
                                   hipMemcpyDeviceToHost, pv->st));
      MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
      return;
    }
    const float os = pv->kdiag();
    for (int64_t i = 0; i < pv->n; ++i) out[i] = os;
  });
}

int mgp_extract_diagonal_test(void* h, const float* Xs, int64_t m, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    if (pv->nonstationary()) {
      MGP_REQUIRE(Xs != nullptr && m >= 1, "non-stationary diagonals need test points");
      float* dx = pv->Xs.ensure((size_t)m * pv->d);
      MGP_HIP_CHECK(hipMemcpyAsync(dx, Xs, (size_t)m * pv->d * sizeof(float),
                                   hipMemcpyHostToDevice, pv->st));
      pv->pack(dx, m, pv->test);
      DevBuf<float> d;
      pv->diag_values(pv->test, m, d.ensure((size_t)m));
      MGP_HIP_CHECK(hipMemcpyAsync(out, d.ptr, (size_t)m * sizeof(float), hipMemcpyDeviceToHost,
                                   pv->st));
      MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
      return;
    }
    const float os = pv->kdiag();
    for (int64_t i = 0; i < m; ++i) out[i] = os;
  });
}

// op 0: forward matvec (the north-star unit).  times_ms[r] is the host wall
// time of repeat r (launch + device + sync); tile_ms_avg receives the mean
// HIP-event duration of the fused tile kernel over the repeats.
int mgp_gradient_matvec(void* h, const float* V, int ncols, float* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(V && out && ncols >= 1, "bad arguments");
    const size_t tot = (size_t)pv->n * ncols;
    const size_t outn = tot * (size_t)pv->nparams;
    float* dv = pv->io_a.ensure(tot);
    float* dout = pv->io_b.ensure(outn);
    MGP_HIP_CHECK(hipMemcpyAsync(dv, V, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    pv->gradient(dv, ncols, dout);
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout, outn * sizeof(float), hipMemcpyDeviceToHost, pv->st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_gradient_trace(void* h, const float* Lf, const float* Rf, int ncols, double* out) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(Lf && Rf && out && ncols >= 1, "bad arguments");
    const size_t tot = (size_t)pv->n * ncols;
    float* dl = pv->io_a.ensure(tot);
    float* dr = pv->io_b.ensure(tot);
    MGP_HIP_CHECK(hipMemcpyAsync(dl, Lf, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    MGP_HIP_CHECK(hipMemcpyAsync(dr, Rf, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    gradient_traces(*pv, dl, dr, ncols, out, pv->st);
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
  });
}

int mgp_benchmark_provider_ops(void* h, const float* rhs, int ncols, int op,
                               int repeats, int warmup, double* times_ms,
                               double* tile_ms_avg, float* out_or_null) {
  return guarded([&] {
    Provider* pv = as_provider(h);
    MGP_REQUIRE(ncols >= 1, "num_cols must be positive");
    MGP_REQUIRE(repeats >= 1, "repeats must be positive");
    MGP_REQUIRE(warmup >= 0, "warmup must be non-negative");
    MGP_REQUIRE(op >= 0 && op <= 3, "op_code must be one of 0, 1, 2, 3");
    const size_t tot = (size_t)pv->n * ncols;
    float* dv = pv->io_a.ensure(tot);
    float* dout = pv->io_b.ensure(op == 0 ? tot : tot * (size_t)pv->nparams);
    MGP_HIP_CHECK(hipMemcpyAsync(dv, rhs, tot * sizeof(float), hipMemcpyHostToDevice, pv->st));
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
    if (op != 0) {
      // ops 1-3 (jit_engine_bindings.mojo:494-540): fused gradient products,
      // + the quadratic forms dots[p][c] = <rhs_c, out_pc>, or the dots alone
      // after one gradient pass.
      const int P = pv->nparams;
      const int nb = reduction_chunks(pv->n);
      DevBuf<double> part, dots;
      part.ensure((size_t)ncols * nb);
      dots.ensure((size_t)P * ncols);
      auto dots_pass = [&]() {
        for (int p = 0; p < P; ++p) {
          coldot_partial(dv, dout + (size_t)p * tot, pv->n, ncols, nb, part.ptr, pv->st);
          coldot_finalize(part.ptr, nb, ncols, dots.ptr + (size_t)p * ncols, pv->st);
        }
      };
      auto run = [&]() {
        if (op != 3) pv->gradient(dv, ncols, dout);
        if (op != 1) dots_pass();
        MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
      };
      if (op == 3) pv->gradient(dv, ncols, dout);
      for (int w = 0; w < warmup; ++w) run();
      for (int r = 0; r < repeats; ++r) {
        auto t0 = std::chrono::steady_clock::now();
        run();
        auto t1 = std::chrono::steady_clock::now();
        if (times_ms) times_ms[r] = std::chrono::duration<double, std::milli>(t1 - t0).count();
      }
      if (tile_ms_avg) *tile_ms_avg = 0.0;
      if (out_or_null)
        MGP_HIP_CHECK(hipMemcpy(out_or_null, dout, tot * (size_t)P * sizeof(float),
                                hipMemcpyDeviceToHost));
      return;
    }
    for (int w = 0; w < warmup; ++w) pv->forward(dv, ncols, dout);
    MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
    if (!pv->ws.ev0) MGP_HIP_CHECK(hipEventCreate(&pv->ws.ev0));
    if (!pv->ws.ev1) MGP_HIP_CHECK(hipEventCreate(&pv->ws.ev1));
    pv->ws.time_tile = true;
    pv->ws.tile_ms = 0.0;
    pv->ws.tile_calls = 0;
    try {
      for (int r = 0; r < repeats; ++r) {
        auto t0 = std::chrono::steady_clock::now();
        pv->forward(dv, ncols, dout);
        MGP_HIP_CHECK(hipStreamSynchronize(pv->st));
        auto t1 = std::chrono::steady_clock::now();
        if (times_ms)
          times_ms[r] = std::chrono::duration<double, std::milli>(t1 - t0).count();
      }
    } catch (...) {
      pv->ws.time_tile = false;
      throw;
    }
    pv->ws.time_tile = false;
    if (tile_ms_avg)
      *tile_ms_avg = pv->ws.tile_calls ? pv->ws.tile_ms / (double)pv->ws.tile_calls : 0.0;
    if (out_or_null)
      MGP_HIP_CHECK(hipMemcpy(out_or_null, dout, tot * sizeof(float), hipMemcpyDeviceToHost));
  });
}

// Copies `bytes` (rounded down to 16) between two fresh device buffers
// `repeats` times; ms_avg receives the mean HIP-event duration of one copy.
int mgp_calibration_copy(int64_t bytes, int repeats, double* ms_avg) {
  return guarded([&] {
    MGP_REQUIRE(bytes >= 16 && repeats >= 1, "bytes >= 16 and repeats >= 1 required");
    const int64_t n4 = bytes / 16;
    DevBuf<float4> a, b;
    a.ensure((size_t)n4);
    b.ensure((size_t)n4);
    MGP_HIP_CHECK(hipMemset(a.ptr, 0, (size_t)n4 * 16));
    hipEvent_t e0, e1;
    MGP_HIP_CHECK(hipEventCreate(&e0));
    MGP_HIP_CHECK(hipEventCreate(&e1));
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(n4, 256), 8192);
    MGP_HIP_CHECK(hipEventRecord(e0, nullptr));
    for (int r = 0; r < repeats; ++r)
      hipLaunchKernelGGL(k_calibration_copy, dim3(blocks), dim3(256), 0, nullptr,
                         a.ptr, b.ptr, n4);
    MGP_HIP_CHECK(hipGetLastError());
    MGP_HIP_CHECK(hipEventRecord(e1, nullptr));
    MGP_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    MGP_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (ms_avg) *ms_avg = ms / repeats;
  });
}

}  // extern "C"
