// Composite kernel trees on gfx950: products, dense blocks, pivot columns and
// gradient traces evaluated per pair from raw coordinate differences (VALU;
// the Gram-form tile path serves single radial leaves).  Tree semantics and
// reference citations are in kernel_tree.h.
#include "tree.h"
#include "tree_jit.h"

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

namespace mgp {

namespace {

constexpr int kTile = 128;      // column points per LDS tile
constexpr int kMaxCols = 16;    // right-hand sides per pass
constexpr int kGradCols = 16;   // gradient-trace factor columns per pass
static_assert(kTreeChunk % 4 == 0 && kTile % kTreeChunk == 0, "float4 chunk reads");

void require(bool ok, const std::string& msg) {
  if (!ok) throw Error(ST_INVALID, msg);
}

// out[c][i] = sum_y part[y][c][i] (+ noise V[c][i]), splits summed in order.
__global__ void k_tree_reduce(const float* __restrict__ part, int splits, int64_t m, int ncols,
                              const float* __restrict__ V, float noise, int add_noise,
                              float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= m * ncols) return;
  double s = 0.0;
  for (int y = 0; y < splits; ++y) s += (double)part[(int64_t)y * ncols * m + idx];
  float o = (float)s;
  if (add_noise) o = fmaf(noise, V[idx], o);
  out[idx] = o;
}

// out[i] = K(x_i, x_i)
__global__ void k_tree_self(const float* __restrict__ X, int64_t m, KernelTree t,
                            const float* __restrict__ p, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  float x[kTreeMaxInputDim];
  for (int k = 0; k < t.d; ++k) x[k] = X[i * t.d + k];
  out[i] = tree_value(t, p, x, x);
}

// out[c*n + i] = K(rows[r0 + c], cols[i])
__global__ void k_tree_fill(const float* __restrict__ Xr, int64_t r0, int64_t rows,
                            const float* __restrict__ Xc, int64_t n, KernelTree t,
                            const float* __restrict__ p, float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * n) return;
  const int64_t c = idx / n, i = idx - c * n;
  const int d = t.d;
  float xr[kTreeMaxInputDim], xc[kTreeMaxInputDim];
  for (int k = 0; k < d; ++k) {
    xr[k] = Xr[(r0 + c) * d + k];
    xc[k] = Xc[i * d + k];
  }
  out[idx] = tree_value(t, p, xr, xc);
}

// part[(y*gx + x)*P + q] = sum over the block's pairs (a, b) of
// dK_ab/dtheta_q sum_c Lf[c][a] Rf[c][b]; grid = (row blocks, column splits).
__global__ __launch_bounds__(256) void k_tree_grad_trace(
    const float* __restrict__ X, int64_t n, KernelTree t, const float* __restrict__ p,
    const float* __restrict__ Lf, const float* __restrict__ Rf, int ncols, int c0,
    double* __restrict__ part) {
  __shared__ float xb[64][kTreeMaxInputDim];
  __shared__ float rb[64][kGradCols];
  __shared__ double red[256];
  const int d = t.d, P = t.nparams;
  const int cn = min(kGradCols, ncols - c0);
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = a < n;
  float xa[kTreeMaxInputDim], la[kGradCols];
  for (int k = 0; k < d; ++k) xa[k] = live ? X[a * d + k] : 0.0f;
  for (int c = 0; c < kGradCols; ++c) la[c] = (live && c < cn) ? Lf[(int64_t)(c0 + c) * n + a] : 0.0f;
  const int64_t tiles = (n + 63) / 64;
  const int64_t tps = (tiles + gridDim.y - 1) / gridDim.y;
  const int64_t jb = min(n, (int64_t)blockIdx.y * tps * 64);
  const int64_t je = min(n, jb + tps * 64);
  double accd[kTreeMaxParams];
  for (int q = 0; q < kTreeMaxParams; ++q) accd[q] = 0.0;
  for (int64_t b0 = jb; b0 < je; b0 += 64) {
    __syncthreads();
    for (int q = threadIdx.x; q < 64 * kTreeMaxInputDim; q += blockDim.x) {
      const int bb = q / kTreeMaxInputDim, k = q - bb * kTreeMaxInputDim;
      const int64_t b = b0 + bb;
      xb[bb][k] = (b < je && k < d) ? X[b * d + k] : 0.0f;
    }
    for (int q = threadIdx.x; q < 64 * kGradCols; q += blockDim.x) {
      const int bb = q / kGradCols, c = q - bb * kGradCols;
      const int64_t b = b0 + bb;
      rb[bb][c] = (b < je && c < cn) ? Rf[(int64_t)(c0 + c) * n + b] : 0.0f;
    }
    __syncthreads();
    float g[kTreeMaxParams];
    for (int q = 0; q < kTreeMaxParams; ++q) g[q] = 0.0f;
    const int cnt = (int)min((int64_t)64, je - b0);
    if (live) {
      for (int bb = 0; bb < cnt; ++bb) {
        float w = 0.0f;
        for (int c = 0; c < kGradCols; ++c) w = fmaf(la[c], rb[bb][c], w);
        tree_grad_accumulate(t, p, xa, xb[bb], w, g);
      }
    }
    for (int q = 0; q < P; ++q) accd[q] += (double)g[q];
  }
  for (int q = 0; q < P; ++q) {
    red[threadIdx.x] = live ? accd[q] : 0.0;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
      __syncthreads();
    }
    if (threadIdx.x == 0) part[((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * P + q] = red[0];
    __syncthreads();
  }
}

// part[(y*gx + x)*table_size + e] = sum over the block's pairs (a, b) of
// w_ab dK_ab/dv_l at table entry e = p0_l + level_a * L + level_b of every
// categorical leaf l, with w_ab = sum_c Lf[c][a] Rf[c][b].
__global__ __launch_bounds__(256) void k_tree_cat_grad(
    const float* __restrict__ X, int64_t n, KernelTree t, const float* __restrict__ p,
    const float* __restrict__ Lf, const float* __restrict__ Rf, int ncols, int c0,
    double* __restrict__ part) {
  __shared__ float xb[64][kTreeMaxInputDim];
  __shared__ float rb[64][kGradCols];
  __shared__ float tab[kTreeMaxTable];
  const int d = t.d;
  const int cn = min(kGradCols, ncols - c0);
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = a < n;
  for (int e = threadIdx.x; e < t.table_size; e += blockDim.x) tab[e] = 0.0f;
  float xa[kTreeMaxInputDim], la[kGradCols];
  for (int k = 0; k < d; ++k) xa[k] = live ? X[a * d + k] : 0.0f;
  for (int c = 0; c < kGradCols; ++c) la[c] = (live && c < cn) ? Lf[(int64_t)(c0 + c) * n + a] : 0.0f;
  float acc[kTreeMaxCatRow];
  for (int q = 0; q < kTreeMaxCatRow; ++q) acc[q] = 0.0f;
  const int64_t tiles = (n + 63) / 64;
  const int64_t tps = (tiles + gridDim.y - 1) / gridDim.y;
  const int64_t jb = min(n, (int64_t)blockIdx.y * tps * 64);
  const int64_t je = min(n, jb + tps * 64);
  for (int64_t b0 = jb; b0 < je; b0 += 64) {
    __syncthreads();
    for (int q = threadIdx.x; q < 64 * kTreeMaxInputDim; q += blockDim.x) {
      const int bb = q / kTreeMaxInputDim, k = q - bb * kTreeMaxInputDim;
      const int64_t b = b0 + bb;
      xb[bb][k] = (b < je && k < d) ? X[b * d + k] : 0.0f;
    }
    for (int q = threadIdx.x; q < 64 * kGradCols; q += blockDim.x) {
      const int bb = q / kGradCols, c = q - bb * kGradCols;
      const int64_t b = b0 + bb;
      rb[bb][c] = (b < je && c < cn) ? Rf[(int64_t)(c0 + c) * n + b] : 0.0f;
    }
    __syncthreads();
    const int cnt = (int)min((int64_t)64, je - b0);
    if (live) {
      for (int bb = 0; bb < cnt; ++bb) {
        float w = 0.0f;
        for (int c = 0; c < kGradCols; ++c) w = fmaf(la[c], rb[bb][c], w);
        float ladj[kTreeMaxLeaves];
        tree_leaf_adjoints(t, p, xa, xb[bb], w, ladj);
        int off = 0;
        for (int l = 0; l < t.nleaves; ++l) {
          const TreeLeaf& lf = t.leaf[l];
          if (lf.kind != KIND_CAT) continue;
          acc[off + tree_level(xb[bb][t.dims[lf.dim_off]], lf.ard)] += ladj[l];
          off += lf.ard;
        }
      }
    }
  }
  __syncthreads();
  if (live) {
    int off = 0;
    for (int l = 0; l < t.nleaves; ++l) {
      const TreeLeaf& lf = t.leaf[l];
      if (lf.kind != KIND_CAT) continue;
      const int L = lf.ard;
      const int row = lf.p0 + tree_level(xa[t.dims[lf.dim_off]], L) * L;
      for (int lb = 0; lb < L; ++lb) atomicAdd(&tab[row + lb], acc[off + lb]);
      off += L;
    }
  }
  __syncthreads();
  double* dst = part + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * t.table_size;
  for (int e = threadIdx.x; e < t.table_size; e += blockDim.x) dst[e] = (double)tab[e];
}

}  // namespace

KernelTree parse_kernel_tree(const int* spec, int len) {
  require(spec != nullptr && len >= 4, "kernel tree spec is too short");
  KernelTree t;
  int pos = 0;
  auto next = [&]() {
    require(pos < len, "kernel tree spec is truncated");
    return spec[pos++];
  };
  t.d = next();
  t.nparams = next();
  t.nleaves = next();
  t.nnodes = next();
  require(t.d >= 1 && t.d <= kTreeMaxInputDim, "kernel tree input dimension must be in [1, 32]");
  require(t.nparams >= 1 && t.nparams <= kTreeMaxParams, "kernel tree has too many parameters");
  require(t.nleaves >= 1 && t.nleaves <= kTreeMaxLeaves, "kernel tree needs 1..8 leaves");
  require(t.nnodes >= 1 && t.nnodes <= kTreeMaxNodes, "kernel tree needs 1..16 nodes");
  int doff = 0, cat_levels = 0;
  for (int l = 0; l < t.nleaves; ++l) {
    TreeLeaf& lf = t.leaf[l];
    lf.kind = next();
    lf.ard = next();
    lf.ndim = next();
    lf.p0 = next();
    lf.dim_off = doff;
    lf.deg = 0;
    if (lf.kind == KIND_POLY) {
      lf.deg = next();
      require(lf.deg >= 1 && lf.deg <= 16, "polynomial degree must be an integer in [1, 16]");
    }
    require(lf.kind >= KIND_RBF && lf.kind <= KIND_POLY, "unknown kernel tree leaf kind");
    require(lf.ndim >= 1 && doff + lf.ndim <= kTreeMaxDims, "kernel tree leaf dimensions");
    for (int q = 0; q < lf.ndim; ++q) {
      const int dq = next();
      require(dq >= 0 && dq < t.d, "kernel tree leaf dimension out of range");
      t.dims[doff++] = dq;
    }
    if (lf.kind == KIND_CAT) {
      require(lf.ndim == 1, "a categorical leaf reads one input column");
      require(lf.ard >= 2 && lf.ard <= kTreeMaxLevels, "categorical leaves need 2..32 levels");
      require(lf.p0 >= 0 && lf.p0 + lf.ard * lf.ard <= kTreeMaxTable,
              "categorical tables exceed 1024 entries");
      t.table_size = std::max(t.table_size, lf.p0 + lf.ard * lf.ard);
      t.ncat += 1;
      cat_levels += lf.ard;
      continue;
    }
    const int nls = lf.ard ? lf.ndim : 1;
    const int extra = (lf.kind == KIND_RQ || lf.kind == KIND_PERIODIC) ? 1
                      : lf.kind == KIND_POLY                           ? 2
                                                                       : 0;
    require(lf.p0 >= 0 && lf.p0 + nls + extra + 1 <= t.nparams,
            "kernel tree leaf parameters out of range");
    if (lf.kind == KIND_LINEAR || lf.kind == KIND_POLY) t.nonstationary = 1;
  }
  require(cat_levels <= kTreeMaxCatRow, "categorical leaves exceed 64 levels in total");
  int leaf_uses[kTreeMaxLeaves] = {0};
  for (int i = 0; i < t.nnodes; ++i) {
    TreeNode& nd = t.node[i];
    nd.code = next();
    nd.a = next();
    nd.b = next();
    switch (nd.code) {
      case TN_LEAF:
        require(nd.a >= 0 && nd.a < t.nleaves, "kernel tree leaf node index");
        require(++leaf_uses[nd.a] == 1, "a kernel tree leaf appears in more than one node");
        break;
      case TN_ADD:
      case TN_MUL:
        require(nd.a >= 0 && nd.a < i && nd.b >= 0 && nd.b < i, "kernel tree child order");
        break;
      case TN_SCALE:
        require(nd.a >= 0 && nd.a < i, "kernel tree child order");
        require(nd.b >= 0 && nd.b < t.nparams, "kernel tree scale parameter index");
        break;
      default:
        require(false, "unknown kernel tree node code");
    }
  }
  require(pos == len, "kernel tree spec has trailing entries");
  for (int l = 0; l < t.nleaves; ++l)
    require(leaf_uses[l] == 1, "every kernel tree leaf needs one leaf node");
  return t;
}

double tree_diag(const KernelTree& t, const float* params) {
  std::vector<double> v((size_t)t.nnodes);
  for (int i = 0; i < t.nnodes; ++i) {
    const TreeNode& nd = t.node[i];
    if (nd.code == TN_LEAF && t.leaf[nd.a].kind == KIND_CAT) {
      v[i] = 1.0;  // every correlation table has a unit diagonal
    } else if (nd.code == TN_LEAF) {
      const TreeLeaf& lf = t.leaf[nd.a];
      const int nls = lf.ard ? lf.ndim : 1;
      const int extra = (lf.kind == KIND_RQ || lf.kind == KIND_PERIODIC) ? 1
                        : lf.kind == KIND_POLY                           ? 2
                                                                         : 0;
      // os of a stationary leaf at zero distance (linear / polynomial trees
      // take per-point diagonals, tree_self_values)
      v[i] = (double)params[lf.p0 + nls + extra];
    } else if (nd.code == TN_ADD) {
      v[i] = v[(size_t)nd.a] + v[(size_t)nd.b];
    } else if (nd.code == TN_MUL) {
      v[i] = v[(size_t)nd.a] * v[(size_t)nd.b];
    } else {
      v[i] = (double)params[nd.b] * v[(size_t)nd.a];
    }
  }
  return v[(size_t)t.nnodes - 1];
}

void tree_matvec(const KernelTree& t, const float* p_dev, const float* Xr, int64_t m,
                 const float* Xc, int64_t n, const float* V, int ncols, float noise,
                 bool square, float* out, DevBuf<float>& work, hipStream_t st) {
  if (m <= 0) return;
  // Column splits so that the launch covers the chip (>= ~2048 blocks of
  // 256 rows), at least one 128-column tile per split.
  const int64_t rows = ceil_div(m, 256);
  const int64_t tiles = ceil_div(std::max<int64_t>(n, 1), kTile);
  const int splits = (int)std::max<int64_t>(
      1, std::min<int64_t>(ceil_div(2048, rows), tiles));
  for (int c0 = 0; c0 < ncols; c0 += kMaxCols) {
    const int nc = std::min(kMaxCols, ncols - c0);
    float* part = work.ensure((size_t)splits * nc * m);
    // the tree's straight-line kernel (tree_jit.hip)
    const TreeJitKernel jk = tree_jit_kernel(t, nc);
    const int64_t rblocks = ceil_div(m, jk.rows_per_block);
    {
      const float* vc = V + (int64_t)c0 * n;
      long long mm = m, nn = n;
      int ncc = nc;
      void* args[] = {(void*)&Xr, &mm, (void*)&Xc, &nn, (void*)&p_dev, (void*)&vc, &ncc,
                      (void*)&part};
      MGP_HIP_CHECK(hipModuleLaunchKernel(jk.fn, (unsigned)rblocks, (unsigned)splits, 1, 256, 1, 1,
                                          (unsigned)jk.lds_bytes, st, args, nullptr));
    }
    hipLaunchKernelGGL(k_tree_reduce, dim3((unsigned)ceil_div(m * nc, 256)), dim3(256), 0, st,
                       part, splits, m, nc, V + (int64_t)c0 * n, noise, square ? 1 : 0,
                       out + (int64_t)c0 * m);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

void tree_self_values(const KernelTree& t, const float* p_dev, const float* X, int64_t m,
                      float* out, hipStream_t st) {
  if (m <= 0) return;
  hipLaunchKernelGGL(k_tree_self, dim3((unsigned)ceil_div(m, 256)), dim3(256), 0, st, X, m, t,
                     p_dev, out);
  MGP_HIP_CHECK(hipGetLastError());
}

void tree_fill(const KernelTree& t, const float* p_dev, const float* Xr, int64_t r0,
               int64_t rows, const float* Xc, int64_t n, float* out, hipStream_t st) {
  const int64_t total = rows * n;
  if (total == 0) return;
  hipLaunchKernelGGL(k_tree_fill, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st, Xr,
                     r0, rows, Xc, n, t, p_dev, out);
  MGP_HIP_CHECK(hipGetLastError());
}

namespace {
// acc[q] (+)= sum_b part[b * Q + q] for q < Q: one wave per q, lane l sums
// b = l, l + 64, .. in order, then a butterfly of shuffles (fixed order).
__global__ void k_tree_part_sum(const double* __restrict__ part, int64_t nblk, int Q,
                                int accumulate, double* __restrict__ acc) {
  const int q = blockIdx.x, lane = threadIdx.x;
  double s = 0.0;
  for (int64_t b = lane; b < nblk; b += 64) s += part[b * Q + q];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) acc[q] = accumulate ? acc[q] + s : s;
}

int64_t grad_splits(int64_t n) {
  const int64_t rows = ceil_div(n, 256);
  return std::max<int64_t>(1, std::min<int64_t>(ceil_div(2048, rows), ceil_div(n, 1024)));
}
}  // namespace

void tree_cat_grad_tables(const KernelTree& t, const float* p_dev, const float* X, int64_t n,
                          const float* Lf, const float* Rf, int ncols, double* G_host,
                          DevBuf<double>& work, hipStream_t st) {
  const int S = t.table_size;
  for (int e = 0; e < S; ++e) G_host[e] = 0.0;
  if (S == 0) return;
  const int64_t rows = ceil_div(n, 256), splits = grad_splits(n), nblk = rows * splits;
  double* part = work.ensure((size_t)nblk * S + S);
  double* acc = part + (size_t)nblk * S;
  for (int c0 = 0; c0 < ncols; c0 += kGradCols) {
    hipLaunchKernelGGL(k_tree_cat_grad, dim3((unsigned)rows, (unsigned)splits), dim3(256), 0, st,
                       X, n, t, p_dev, Lf, Rf, ncols, c0, part);
    hipLaunchKernelGGL(k_tree_part_sum, dim3((unsigned)S), dim3(64), 0, st, part, nblk, S,
                       c0 > 0 ? 1 : 0, acc);
    MGP_HIP_CHECK(hipGetLastError());
  }
  MGP_HIP_CHECK(hipMemcpyAsync(G_host, acc, (size_t)S * sizeof(double), hipMemcpyDeviceToHost,
                               st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

void tree_grad_traces(const KernelTree& t, const float* p_dev, const float* X, int64_t n,
                      const float* Lf, const float* Rf, int ncols, double* g_host,
                      DevBuf<double>& work, hipStream_t st) {
  const int P = t.nparams;
  const int64_t rows = ceil_div(n, 256), splits = grad_splits(n), nblk = rows * splits;
  double* part = work.ensure((size_t)nblk * P + P);
  double* acc = part + (size_t)nblk * P;
  for (int c0 = 0; c0 < ncols; c0 += kGradCols) {
    hipLaunchKernelGGL(k_tree_grad_trace, dim3((unsigned)rows, (unsigned)splits), dim3(256), 0,
                       st, X, n, t, p_dev, Lf, Rf, ncols, c0, part);
    hipLaunchKernelGGL(k_tree_part_sum, dim3((unsigned)P), dim3(64), 0, st, part, nblk, P,
                       c0 > 0 ? 1 : 0, acc);
    MGP_HIP_CHECK(hipGetLastError());
  }
  MGP_HIP_CHECK(hipMemcpyAsync(g_host, acc, (size_t)P * sizeof(double), hipMemcpyDeviceToHost,
                               st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
}

}  // namespace mgp
