// Random-Fourier-feature prior draws for pathwise posterior sampling, in fp64
// as the reference's NumPy evaluation (pathwise_prior.py:37-47 and the
// stationary feature map of pathwise_prior.py:130-160):
//
//   phi_f(x)   = sqrt(2/F) cos(sum_q (x_q / l_q) W[f][q] + phase[f])
//   out[k][i]  = scale * sum_f weights[k][f] phi_f(x_i)      (scale = sqrt(os))
//
// The features of a row chunk are written feature-major ([F][rows], fp64) by
// one kernel and contracted against the K weight rows by a second (one thread
// per row and 8 weight rows, the weights staged through LDS, the feature sum
// taken in order f = 0..F-1); rows are processed in chunks so the feature
// block stays bounded (F * 32768 * 8 bytes).
#include <algorithm>
#include <cmath>
#include <string>

#include "mgp_common.h"
#include "mojogp_amd.h"

using namespace mgp;

namespace {

constexpr int64_t kRowChunk = 32768;
constexpr int kContractCols = 8;     // weight rows per thread
constexpr int kContractTile = 256;   // features per LDS stage

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

// out[k*n + r0 + i] = (float)(scale * sum_f wt[k*F + f] phi[f*rows + i]) for
// the kContractCols weight rows k0 = blockIdx.y * kContractCols ... of this
// block; blockDim.x = kContractTile.  Every thread takes part in the LDS
// staging (no early return before the barriers).
__global__ __launch_bounds__(kContractTile) void k_rff_contract(
    const double* __restrict__ phi, int64_t rows, const double* __restrict__ wt, int K, int F,
    double scale, int64_t n, int64_t r0, float* __restrict__ out) {
  __shared__ double wl[kContractCols][kContractTile];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int k0 = blockIdx.y * kContractCols;
  const bool live = i < rows;
  double acc[kContractCols];
#pragma unroll
  for (int c = 0; c < kContractCols; ++c) acc[c] = 0.0;
  for (int f0 = 0; f0 < F; f0 += kContractTile) {
    const int cnt = min(kContractTile, F - f0);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kContractCols; ++c) {
      const int k = k0 + c;
      wl[c][threadIdx.x] =
          (k < K && (int)threadIdx.x < cnt) ? wt[(int64_t)k * F + f0 + threadIdx.x] : 0.0;
    }
    __syncthreads();
    if (live) {
      for (int f = 0; f < cnt; ++f) {
        const double p = phi[(int64_t)(f0 + f) * rows + i];
#pragma unroll
        for (int c = 0; c < kContractCols; ++c) acc[c] = fma(p, wl[c][f], acc[c]);
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int c = 0; c < kContractCols; ++c) {
    const int k = k0 + c;
    if (k < K) out[(int64_t)k * n + r0 + i] = (float)(scale * acc[c]);
  }
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

}  // namespace

extern "C" {

int mgp_rff_prior_values(const float* X, int64_t n, int d, const double* lengthscales,
                         const double* W, const double* phase, int F, double outputscale,
                         const double* weights, int K, float* out) {
  return guarded([&] {
    MGP_REQUIRE(X && lengthscales && W && phase && weights && out, "null argument");
    MGP_REQUIRE(n >= 1 && d >= 1 && F >= 1 && K >= 1, "sizes must be >= 1");
    MGP_REQUIRE(F <= 65535, "at most 65535 features");
    MGP_REQUIRE(K <= 65535 * kContractCols, "too many weight rows");
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
    HipArray<double> phi((size_t)F * chunk);
    MGP_HIP_CHECK(hipMemcpyAsync(dX.ptr, X, (size_t)n * d * sizeof(float), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dls.ptr, lengthscales, d * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dW.ptr, W, (size_t)F * d * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dph.ptr, phase, F * sizeof(double), hipMemcpyHostToDevice, st));
    MGP_HIP_CHECK(hipMemcpyAsync(dwt.ptr, weights, (size_t)K * F * sizeof(double), hipMemcpyHostToDevice, st));
    const double amp = std::sqrt(2.0 / (double)F);
    const double scale = std::sqrt(outputscale);
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
      const int64_t rows = std::min(chunk, n - r0);
      hipLaunchKernelGGL(k_rff_features, dim3((unsigned)ceil_div(rows, 256), (unsigned)F),
                         dim3(256), 0, st, dX.ptr, r0, rows, d, dls.ptr, dW.ptr, dph.ptr, F, amp,
                         phi.ptr);
      MGP_HIP_CHECK(hipGetLastError());
      const dim3 grid((unsigned)ceil_div(rows, kContractTile),
                      (unsigned)ceil_div(K, kContractCols));
      hipLaunchKernelGGL(k_rff_contract, grid, dim3(kContractTile), 0, st, phi.ptr, rows,
                         dwt.ptr, K, F, scale, n, r0, dout.ptr);
      MGP_HIP_CHECK(hipGetLastError());
    }
    MGP_HIP_CHECK(hipMemcpyAsync(out, dout.ptr, (size_t)n * K * sizeof(float), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
  });
}

}  // extern "C"
