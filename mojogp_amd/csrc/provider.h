// Device-resident kernel provider: training inputs, hyperparameters, packed
// tile operands and the stream every call of a handle runs on.
//
// Reference counterpart: the generated JITProvider struct and its impl_* entry
// points (mojogp/codegen_engine/emit/fn_ptr_module.py:159-211, 651-703).
#pragma once

#include <vector>

#include "dense.h"
#include "matvec.h"
#include "tree.h"

namespace mgp {

struct Provider {
  int kind = KIND_RBF;
  bool ard = false;
  int d = 0;
  int64_t n = 0;
  int nparams = 0;             // engine layout: [ls | ls_0..ls_{d-1}], os
  std::vector<float> params;   // constrained values
  float noise = 0.f;
  // Fixed per-point noise variances (the reference's noise mode 1): when set,
  // forward() adds diag(noise_vec) and ignores the scalar noise, and the
  // preconditioner is built for L L^T + diag(noise_vec).
  DevBuf<float> noise_vec;
  bool has_noise_vec = false;
  // Learned per-point noise (the reference's noise modes 2-4): 2 one variance
  // per point, 3 one per group (noise_groups[i] in [0, num_noise_groups)),
  // 4 softplus of a linear function of the raw inputs.  Training recomputes
  // noise_vec from the learned state every iteration; 0 = not learned.
  int learned_noise_mode = 0;
  std::vector<int> noise_groups;
  int num_noise_groups = 0;
  std::vector<double> center;  // column means of the training inputs
  // Composite kernel tree (sums / products / scales of stationary leaves on
  // dimension subsets): products are evaluated per pair from raw inputs; the
  // packed point sets then hold raw coordinates in z and params live on the
  // device in tparams (tree parameter layout, nparams entries).
  bool is_tree = false;
  KernelTree tree;
  DevBuf<float> tparams;
  // Categorical correlation tables of the tree's categorical leaves
  // (tree.table_size entries, placed after the parameters in tparams).
  std::vector<float> cat_tables;
  DevBuf<float> tree_ws;  // column-split partial products of the tree matvec
  // block partials of the tree gradient / table traces (scratch, so usable
  // through a const provider)
  mutable DevBuf<double> tree_gws;
  // work buffers of the matrix-core gradient trace (scratch, as above)
  mutable GradTraceWorkspace gtws;

  hipStream_t st = nullptr;
  int device = 0;              // HIP device current when the provider was created
  DevBuf<float> X;             // raw training inputs [n][d]
  Coords co;
  PackedPoints train;
  MatvecWorkspace ws;

  // Scratch for the host-pointer entry points.
  DevBuf<float> io_a, io_b, io_c;
  PackedPoints test;
  DevBuf<float> Xs;

  // Dense K (materialized route) as a scaled two-term fp16 split (dense.h):
  // its symmetric half refilled on every parameter update (products with up
  // to 16 right-hand sides), the full matrix filled on demand (wider products).
  bool materialized = false;
  DenseK dense;
  DenseWorkspace dense_ws;

  float outputscale() const { return params[nparams - 1]; }
  // k(x, x) (every supported kernel is stationary): the outputscale for a
  // single leaf, the tree evaluated at zero distance for composite kernels.
  float kdiag() const {
    if (!is_tree) return outputscale();
    // non-stationary trees: the last parameter, as the reference's
    // get_diagonal_value hint (fn_ptr_module.py:948-961); per-point
    // diagonals come from diag_values
    return tree.nonstationary ? params.back() : (float)tree_diag(tree, params.data());
  }
  bool nonstationary() const { return is_tree && tree.nonstationary; }
  // out[i] = k(x_i, x_i) for m device points of a packed set (device out).
  void diag_values(const PackedPoints& pts, int64_t m, float* out);
  float lengthscale(int k) const { return ard ? params[k] : params[0]; }

  // Recompute the coordinate map from params and repack the training points.
  void refresh_coords();
  // Pack an arbitrary point set with the current coordinate map.
  void pack(const float* X_dev, int64_t m, PackedPoints& pp);

  // Allocate and fill the dense K (materialized route, _do_materialize).
  void materialize();
  void fill_dense();       // symmetric half of K (dense.h), after every update
  void fill_dense_full();  // full K, when a product needs it and it is stale
  // max_i k(x_i, x_i): bounds every |K_ij| of a positive semi-definite kernel.
  float kdiag_max();
  // Rebind the provider to another stream.
  void set_stream(hipStream_t s) { st = s; }

  // Host [n] noise variances (all finite and > 0), or nullptr to clear.
  void set_noise_vector(const float* host);
  // Upload n host variances into the active noise vector without validation
  // (training's learned-noise updates; values are softplus + floor).
  void load_noise_vector(const float* host);
  // The scalar noise the operator uses: 0 under a noise vector.
  float scalar_noise() const { return has_noise_vec ? 0.f : noise; }

  // (K + noise I) V (or (K + diag(noise_vec)) V) for device arrays V, out
  // ([ncols][n] column-major).
  // wsp: work buffers of the fused tile route (default: the provider's own,
  // grown on demand; a fixed-arena workspace keeps the call allocation-free).
  void forward(const float* V, int ncols, float* out, MatvecWorkspace* wsp = nullptr);
  void forward_scalar(const float* V, int ncols, float* out,  // without the noise vector
                      MatvecWorkspace* wsp = nullptr);
  // True when forward() runs the fused tile kernel (not materialized, Gram form
  // accurate for the packed training set).
  bool fused_route() const;
  // True when forward() gives every column the same bits whether it runs
  // alone or beside other columns (one and two columns on the symmetric
  // kernel), so independent solvers may share products.
  bool column_independent_products() const;
  // Fused route only: out[cc][t] (+)= sum_t' mix[t][t'] ((K + noise I) V)[cc][t'] for
  // task blocks of T columns (mix: device [T][T]), mixing folded into the
  // split-K reduction.
  void forward_mixed(const float* V, int ncols, const float* mix, int T, bool accumulate,
                     float* out, PackedRhs* reuse = nullptr);
  // out[p][c][i] = sum_j dk_p(x_i, x_j) V[c][j] for all P parameters (device
  // arrays; out is [P][ncols][n]).
  DevBuf<float> gscale;  // per-parameter scale of the gradient sums
  void gradient(const float* V, int ncols, float* out);

  // K(Xs, X) V for a packed test set.
  void cross(const PackedPoints& rows, const float* V, int ncols, float* out);
  // out[c*n + i] = k(rows[r0 + c], x_i) for c < nrows (dense cross block).
  void fill_block(const PackedPoints& rows, int64_t r0, int64_t nrows, float* out);
};

// Live provider handles.  Every C entry point turns a handle into a Provider
// through checked_provider(), which rejects null, unknown and destroyed handles
// without dereferencing them; creation registers a provider, destruction
// unregisters it first.
Provider* checked_provider(void* h);
void register_provider(Provider* p);
void unregister_provider(Provider* p);

}  // namespace mgp
