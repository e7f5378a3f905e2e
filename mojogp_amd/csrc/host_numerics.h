// Small dense/tridiagonal linear algebra on the host (fp64) and the fp32
// scalar helpers of the training loop.
//
// Reference counterparts (caspbian/mojogp):
//   tridiagonal eigensolver    kernels/native_numerics.mojo:271-400, 724-850
//   SLQ log-det                kernels/native_numerics.mojo:403-536
//   Cholesky / inverse / LU    kernels/native_numerics.mojo:24-256,
//                              kernels/pivoted_cholesky.mojo:1083-1208, 1411-1518
//   softplus / Adam / LR       kernels/utils.mojo:14-90, kernels/training_utils.mojo:23-320
#pragma once

#include <cstdint>
#include <vector>

namespace mgp {

// Eigen-decomposition of a symmetric tridiagonal matrix (diag d[m], off e[m-1])
// by implicit QL with Wilkinson shifts.  Eigenvalues ascending in `evals`;
// `evecs` (row-major m x m, columns are eigenvectors) if non-null.  Returns
// false if an eigenvalue failed to converge within 1000*m sweeps.
bool tridiag_eigh(const std::vector<double>& d, const std::vector<double>& e,
                  std::vector<double>& evals, std::vector<double>* evecs);

// SLQ estimate of log|A| from per-probe tridiagonals (GPyTorch conventions of
// the reference: skip probes with NaN/+-1e20 entries, skip negative
// eigenvalues and those below 1e-6 * max eigenvalue, average over valid
// probes, scale by n).
float slq_logdet(const std::vector<std::vector<float>>& diags,
                 const std::vector<std::vector<float>>& offdiags, int64_t n);

// Lower Cholesky of a symmetric positive definite matrix (row-major, in
// place in `c`); false if a non-positive pivot is met.
bool cholesky(std::vector<double>& c, int k);
// Inverse via Cholesky, falling back to partial-pivot LU.
bool spd_inverse(const std::vector<double>& A, int k, std::vector<double>& inv);
// log|det A| via Cholesky, falling back to partial-pivot LU.
double logdet_spd(const std::vector<double>& A, int k);

// Symmetric eigen-decomposition of a small row-major matrix by the classical
// (largest off-diagonal pivot) Jacobi method in fp64: rotations until the
// largest |off-diagonal| < 1e-12 or 100 k^2 rotations, eigenvalues sorted
// ascending with their eigenvector columns (V row-major, A = V diag(e) V^T).
// The same convergence rule, rotation and ordering as the reference's
// _symmetric_eigen_cpu (kernels/kronecker_preconditioner.mojo:736-822), so the
// eigenvector signs agree with it.
void jacobi_eigen(const float* A, int k, float* V, float* evals);

// fp32 helpers with the reference's thresholds.
float softplus(float x);
float inv_softplus(float y);
float softplus_derivative(float x);
float pow_float32(float base, int e);
float clip_gradient(float g, float max_grad = 100.0f);
float cosine_lr(float lr_max, int iteration, int total);

}  // namespace mgp
