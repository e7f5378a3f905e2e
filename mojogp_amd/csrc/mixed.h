// Mixed continuous x categorical kernels: categorical correlation tables and
// the split-Adam training loop of the reference's mixed GP
// (kernels/jit/jit_mixed.mojo:428-909).
#pragma once

#include <functional>
#include <vector>

#include "engine.h"

namespace mgp {

enum CatKind : int { CAT_GD = 0, CAT_CR = 1, CAT_EHH = 2, CAT_HH = 3, CAT_FE = 4 };

int cat_num_params(int kind, int L);
// Raw -> constrained parameters (softplus; pi * sigmoid for angles) and,
// optionally, d(constrained)/d(raw).
void cat_constrain(int kind, int L, const float* raw, int K, double* theta, double* chain);
// R[L][L] from constrained parameters; with dR, also dR/dtheta_k [K][L][L].
void cat_correlation(int kind, int L, const double* theta, double* R, std::vector<double>* dR);
// Tables of every categorical leaf (tree order) from raw parameters; refreshes
// the provider.
void set_categorical_raw(Provider& pv, const std::vector<int>& kinds, const float* raw,
                         int nraw);

// A categorical leaf of a tree provider: kind, levels, table offset (after the
// tree parameters), offset and count of its raw parameters.
struct CatLeafRef {
  int kind, L, table_off, param_off, nparam;
};
std::vector<CatLeafRef> cat_leaves(const Provider& pv, const std::vector<int>& kinds);
// Raw-parameter gradients from per-entry table sums G[table_size]:
// out[k] = clip(scale sum_e dR_k[e] G[e]) * d(theta_k)/d(raw_k), clip at +-clipv.
void cat_raw_gradients(const std::vector<CatLeafRef>& cl, const float* rcat,
                       const std::vector<double>& G, double scale, float clipv, float* out);

struct MixedTrainResult {
  TrainResult base;            // continuous params, noise, mean, histories
  std::vector<float> cat_raw;  // best raw categorical parameters
};

MixedTrainResult train_mixed(Provider& pv, const float* y_host,
                             const std::vector<float>& init_params, float init_noise,
                             const std::vector<int>& cat_kinds,
                             const std::vector<float>& init_cat_raw, const TrainOptions& o,
                             const std::function<void(const ProgressEvent&)>& progress);

}  // namespace mgp
