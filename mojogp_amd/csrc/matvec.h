// Fused kernel-matrix products on gfx950: declarations shared by the C ABI.
#pragma once

#include "mgp_common.h"

namespace mgp {

// Per-dimension affine map applied to raw inputs before any kernel tile is
// formed: z_d = (x_d - center_d) * scale_d.  scale_d folds the lengthscale and
// the kernel's base-2 exponent constant (see kernel_scale()).
struct Coords {
  int d = 0;
  DevBuf<float> coef;  // [2*d]: center[d] then scale[d]
};

// Points laid out as 16x16x4 fp32 MFMA operands.
//   A-side (columns j): aug = [z_0..z_{d-1}, |z|^2, 1, 0 ...]
//   B-side (rows i):    aug = [-2 z_0..-2 z_{d-1}, 1, |z|^2, 0 ...]
//   pack[tile][kk][lane] = aug[16*tile + lane%16][4*kk + lane/16]
// so one MFMA over kk-slices of A(j) and B(i) accumulates |z_i - z_j|^2.
struct PackedPoints {
  int64_t n = 0;       // real points
  int64_t ntiles = 0;  // 16-point tiles (zero padded)
  int kk = 0;          // number of K=4 slices (augmented dim / 4)
  DevBuf<float> A, B;
  DevBuf<float> z;     // scaled coordinates, row-major [n][d] (direct path)
};

// Multiplier applied to (x - center)/lengthscale so that the squared distance
// of the scaled points feeds exp2 directly:
//   RBF:       s = 0.5*log2(e)*r^2,  k = os*2^-min(s, 20 log2 e)
//   Matern52:  s = 5*log2(e)^2*r^2,   u = sqrt(s) = sqrt(5) r log2(e)
inline float kernel_scale(int kind) {
  return kind == KIND_RBF ? 0.84932180028801904272f   // sqrt(0.5*log2 e)
                          : 3.22596433305849393025f;  // sqrt(5)*log2 e
}

// Builds packed operands (and scaled coordinates) for n points X[n][d].
void pack_points(const float* X_dev, int64_t n, const Coords& co,
                 PackedPoints& pp, hipStream_t st);

struct MatvecArgs {
  int kind = KIND_RBF;
  float outputscale = 1.f;
  float noise = 0.f;     // added as noise*V on the diagonal (square only)
  bool square = false;   // rows and columns are the same point set
  int64_t m = 0;         // rows (output length per column)
  int64_t n = 0;         // columns (input length per column)
  int ncols = 0;         // right-hand sides
};

// out[c*m + i] = os * sum_j k(r_i, c_j) V[c*n + j]  (+ noise*V[c*m+i] if square)
// V and out are column-major device arrays.  Work buffers are grown in `ws`.
struct MatvecWorkspace {
  DevBuf<float> vpack;    // packed right-hand sides
  DevBuf<float> partial;  // split-K partial sums
  // Optional HIP-event timing of the tile kernel alone (bench hook).
  bool time_tile = false;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double tile_ms = 0.0;
  int64_t tile_calls = 0;
};

void fused_matvec(const MatvecArgs& a, const PackedPoints& rows,
                  const PackedPoints& cols, const float* V_dev, float* out_dev,
                  MatvecWorkspace& ws, hipStream_t st, int force_splits = 0);

// Reference-form product evaluated per pair from per-dimension differences of
// the scaled coordinates (no Gram form, no MFMA).  Used as an independent
// device cross-check and for dimensions beyond the MFMA tile path.
void direct_matvec(const MatvecArgs& a, const PackedPoints& rows,
                   const PackedPoints& cols, int d, const float* V_dev,
                   float* out_dev, hipStream_t st);

// Maximum input dimension served by the MFMA tile path (augmented K <= 32).
constexpr int kMaxMfmaDim = 30;

}  // namespace mgp
