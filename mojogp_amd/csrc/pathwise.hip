// Random-Fourier-feature prior draws for pathwise posterior sampling, in fp64
// as the reference's NumPy evaluation (pathwise_prior.py:37-47 and the
// stationary feature map of pathwise_prior.py:130-160):
//
//   phi_f(x)   = sqrt(2/F) cos(sum_q (x_q / l_q) W[f][q] + phase[f])
//   out[k][i]  = scale * sum_f weights[k][f] phi_f(x_i)      (scale = sqrt(os))
//
// The features of a row chunk are written feature-major ([F][rows], fp64) by a
// hand-written kernel and contracted against the K weight rows with one
// rocBLAS dgemm; rows are processed in chunks so the feature block stays
// bounded (F * 32768 * 8 bytes).
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "mgp_common.h"
#include "mojogp_amd.h"

using namespace mgp;

namespace {

#define PW_BLAS_CHECK(expr)                                                         \
  do {                                                                              \
    const rocblas_status s_ = (expr);                                               \
    if (s_ != rocblas_status_success)                                               \
      throw Error(ST_HIP, std::string("rocBLAS error in " #expr ": ") +             \
                              rocblas_status_to_string(s_));                        \
  } while (0)

constexpr int64_t kRowChunk = 32768;

// phi[f*rows + i] = amp * cos(sum_q (x[(r0+i)*d + q] / ls[q]) * W[f*d + q] + phase[f])
__global__ void k_rff_features(const float* __restrict__ X, int64_t r0, int64_t rows, int d,
                               const double* __restrict__ ls, const double* __restrict__ W,
                               const double* __restrict__ phase, int F, double amp,
                               double* __restrict__ phi) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int f = blockIdx.y;
  if (i >= rows || f >= F) return;
  const float* xr = X + (r0 + i) * d;
  const double* wf = W + (int64_t)f * d;
  double arg = 0.0;
  for (int q = 0; q < d; ++q) arg = fma((double)xr[q] / ls[q], wf[q], arg);
  phi[(int64_t)f * rows + i] = amp * cos(arg + phase[f]);
}

// out[k*n + r0 + i] = (float)(scale * acc[k*rows + i])
__global__ void k_store_prior(const double* __restrict__ acc, int64_t rows, int K, double scale,
                              int64_t n, int64_t r0, float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * K) return;
  const int64_t k = idx / rows, i = idx - k * rows;
  out[k * n + r0 + i] = (float)(scale * acc[idx]);
}

template <class T>
struct HipArray {
  T* ptr = nullptr;
  explicit HipArray(size_t count) {
    MGP_HIP_CHECK(hipMalloc(&ptr, std::max<size_t>(count, 1) * sizeof(T)));
  }
  ~HipArray() {
    if (ptr) (void)hipFree(ptr);
  }
  HipArray(const HipArray&) = delete;
  HipArray& operator=(const HipArray&) = delete;
};

struct BlasHandle {
  rocblas_handle h = nullptr;
  explicit BlasHandle(hipStream_t st) {
    PW_BLAS_CHECK(rocblas_create_handle(&h));
    PW_BLAS_CHECK(rocblas_set_stream(h, st));
  }
  ~BlasHandle() {
    if (h) (void)rocblas_destroy_handle(h);
  }
};

}  // namespace

extern "C" {

int mgp_rff_prior_values(const float* X, int64_t n, int d, const double* lengthscales,
                         const double* W, const double* phase, int F, double outputscale,
                         const double* weights, int K, float* out) {
  return guarded([&] {
    MGP_REQUIRE(X && lengthscales && W && phase && weights && out, "null argument");
    MGP_REQUIRE(n >= 1 && d >= 1 && F >= 1 && K >= 1, "sizes must be >= 1");
    MGP_REQUIRE(F <= 65535, "at most 65535 features");
    MGP_REQUIRE(std::isfinite(outputscale) && outputscale >= 0.0, "outputscale must be >= 0");
    hipStream_t st = nullptr;
    MGP_HIP_CHECK(hipStreamCreate(&st));
    struct StreamGuard {
      hipStream_t s;
      ~StreamGuard() { (void)hipStreamDestroy(s); }
    } sg{st};
    const int64_t chunk = std::min<int64_t>(n, kRowChunk);
    HipArray<float> dX((size_t)n * d), dout((size_t)n * K);
    HipArray<double> dls(d), dW((size_t)F * d), dph(F), dwt((size_t)K * F);
    HipArray<double> phi((size_t)F * chunk), acc((size_t)K * chunk);
    MGP_HIP_CHECK(hipMemcpyAsync(dX.ptr, X, (size_t)n * d * sizeof(float), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dls.ptr, lengthscales, d * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dW.ptr, W, (size_t)F * d * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dph.ptr, phase, F * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dwt.ptr, weights, (size_t)K * F * sizeof(double), hipMemcpyHostToDevice, st));
    BlasHandle blas(st);
    const double amp = std::sqrt(2.0 / (double)F);
    const double scale = std::sqrt(outputscale);
    const double one = 1.0, zero = 0.0;
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
      const int64_t rows = std::min(chunk, n - r0);
      hipLaunchKernelGGL(k_rff_features, dim3((unsigned)ceil_div(rows, 256), (unsigned)F),
                         dim3(256), 0, st, dX.ptr, r0, rows, d, dls.ptr, dW.ptr, dph.ptr, F, amp,
                         phi.ptr);
      MGP_HIP_CHECK(hipGetLastError());
      // acc (rows x K, col-major) = phi (rows x F, col-major) * weights^T (F x K)
      PW_BLAS_CHECK(rocblas_dgemm(blas.h, rocblas_operation_none, rocblas_operation_none,
                                  (rocblas_int)rows, K, F, &one, phi.ptr, (rocblas_int)rows,
                                  dwt.ptr, F, &zero, acc.ptr, (rocblas_int)rows));
      hipLaunchKernelGGL(k_store_prior, dim3((unsigned)ceil_div(rows * K, 256)), dim3(256), 0, st,
                         acc.ptr, rows, K, scale, n, r0, dout.ptr);
      MGP_HIP_CHECK(hipGetLastError());
    }
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout.ptr, (size_t)n * K * sizeof(float), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
  });
}

}  // extern "C"
