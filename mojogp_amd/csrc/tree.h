// Host entry points of the composite-kernel-tree products (kernel_tree.h).
#pragma once

#include "kernel_tree.h"

namespace mgp {

// out[c][i] = sum_j K(Xr_i, Xc_j) V[c][j] (+ noise V[c][i] when square) for
// device row-major points Xr [m][d], Xc [n][d] and column-major V [ncols][n].
void tree_matvec(const KernelTree& t, const float* p_dev, const float* Xr, int64_t m,
                 const float* Xc, int64_t n, const float* V, int ncols, float noise,
                 bool square, float* out, DevBuf<float>& work, hipStream_t st);
// out[i] = K(X_i, X_i) for device points X [m][d].
void tree_self_values(const KernelTree& t, const float* p_dev, const float* X, int64_t m,
                      float* out, hipStream_t st);
// out[c*n + i] = K(Xr[r0 + c], Xc[i]) for c < rows.
void tree_fill(const KernelTree& t, const float* p_dev, const float* Xr, int64_t r0,
               int64_t rows, const float* Xc, int64_t n, float* out, hipStream_t st);
// G[e] = sum_{a,b} dK_ab/dR_l[level_a][level_b] sum_c Lf[c][a] Rf[c][b] for every
// categorical table entry e (fp64, host, G[table_size]).
// work: device partials (grown on demand, owned by the caller).
void tree_cat_grad_tables(const KernelTree& t, const float* p_dev, const float* X, int64_t n,
                          const float* Lf, const float* Rf, int ncols, double* G_host,
                          DevBuf<double>& work, hipStream_t st);
// g[q] = sum_{a,b} dK_ab/dtheta_q sum_c Lf[c][a] Rf[c][b] (fp64, host).
void tree_grad_traces(const KernelTree& t, const float* p_dev, const float* X, int64_t n,
                      const float* Lf, const float* Rf, int ncols, double* g_host,
                      DevBuf<double>& work, hipStream_t st);

}  // namespace mgp
