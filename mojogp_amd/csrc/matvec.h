// Fused kernel-matrix products on gfx950: declarations shared by the C ABI.
#pragma once

#include <vector>

#include "mgp_common.h"

namespace mgp {

// Per-dimension affine map applied to raw inputs before any kernel tile is
// formed: z_d = (x_d - center_d) * scale_d.  scale_d folds the lengthscale and
// the kernel's base-2 exponent constant (see kernel_scale()).
struct Coords {
  int d = 0;
  DevBuf<float> coef;  // [2*d]: center[d] then scale[d]
  // Limit on the base-2 exponent of the kernel value, exp2_limit(kind, ard)
  // (mgp_common.h): where the reference's generated code clamps exp at -20.
  float exp2_limit = kExp2Clamp;
};

// Points laid out as v_mfma_f32_16x16x32_f16 operands.
//   A-side (columns j): aug = [z_0..z_{d-1}, |z|^2, 1]
//   B-side (rows i):    aug = [-2 z_0..-2 z_{d-1}, 1, |z|^2]
// Every fp32 aug value x is split into two fp16 parts, hi = RNE16(x) and
// lo = RNE16(x - hi) (x - hi is exact in fp32).  The dot product of the two
// augmented vectors is then the sum of three part-products per dimension,
//   hi.hi + hi.lo + lo.hi,
// with the dropped lo.lo term and the rounding of lo below 3 * 2^-24 |a b| per
// slot (subnormal lo parts of values under 2^-3 add at most 2^-25 absolute),
// which yields |z_i - z_j|^2 at fp32 accuracy on the fp16 matrix cores.  The
// aug values stay inside fp16's range wherever the Gram form is used (|z|^2 up
// to the norm bounds below, all under 65504).
// Slot k (0 <= k < 32*kb) of a point holds product p = k / D, dimension
// t = k % D (D = d + 2), zero for k >= 3 D; lane (li + 16 g) of MFMA m carries
// slots 32 m + 8 g + e, e = 0..7:
//   pack[tile][m][lane][e] (fp16), lane = point%16 + 16 g
struct PackedPoints {
  int64_t n = 0;       // real points
  int64_t ntiles = 0;  // 16-point tiles (zero padded)
  int64_t ntiles_alloc = 0;  // tiles packed (>= ntiles, a multiple of kPackTileAlign)
  int kb = 0;          // K=32 fp16 MFMAs per 16x16 distance tile
  DevBuf<uint32_t> A, B;  // two fp16 per dword
  DevBuf<float> z;     // scaled coordinates, row-major [n][d] (direct path)
  float max_norm = 0.f;      // max_i |z_i|^2 (Gram-form error scale)
  float exp2_limit = kExp2Clamp;  // the Coords' exponent limit
  DevBuf<uint32_t> max_norm_dev;
};

// Upper bound on max|z_i|^2 + max|z_j|^2 for the Gram-form tile path.  Its
// distance error is ~2^-23 (|z_i|^2 + |z_j|^2) from the fp32 accumulation of
// the norm terms, so the product error grows with the norms of the pairs that
// carry weight.  The worst case is data whose every point sits near the
// largest norm (an annulus of radius many lengthscales, near-coincident pairs
// everywhere): measured there on gfx950, the normwise relative product error
// is 5.3e-6 (RBF) at a sum of 128, 4.3e-6 (Matern-3/2) at 512 and 7.6e-6
// (Matern-5/2) at 2048, and crosses 1e-5 at the next power of two (the error
// steps with the binade of the norms).  Beyond these bounds the products are
// evaluated from per-dimension differences (direct_matvec) instead.  RBF is the
// most sensitive: dk/ds = -ln2 k against at most -0.08 os for Matern-5/2.
// Matern-1/2 is never evaluated in Gram form: k = 2^-sqrt(s) has an unbounded
// slope in s at s = 0, so the absolute distance error e of near-coincident
// pairs becomes a kernel error of ~ln2 sqrt(e) instead of ~e.
constexpr float kGramMaxNormSumRBF = 128.0f;
constexpr float kGramMaxNormSumM52 = 2048.0f;
constexpr float kGramMaxNormSumM32 = 512.0f;
inline bool gram_form_ok(int kind, const PackedPoints& rows, const PackedPoints& cols) {
  if (kind == KIND_MATERN12) return false;
  const float bound = kind == KIND_RBF       ? kGramMaxNormSumRBF
                      : kind == KIND_MATERN32 ? kGramMaxNormSumM32
                                              : kGramMaxNormSumM52;
  return rows.kb > 0 && rows.max_norm + cols.max_norm <= bound;
}

// Number of K=32 MFMAs for input dimension d: ceil(3 (d + 2) / 32).
inline int split_mfma_count(int d) { return (3 * (d + 2) + 31) / 32; }

// Multiplier applied to (x - center)/lengthscale so that the squared distance
// of the scaled points feeds exp2 directly:
//   RBF:       s = 0.5*log2(e)*r^2,  k = os*2^-s  (not clamped)
//   Matern52:  s = 5*log2(e)^2*r^2,   u = sqrt(s) = sqrt(5) r log2(e)
//   Matern12:  u = sqrt(s) = r log2(e),  k = os*2^-min(u, lim)  (lim: 20 log2 e
//              for ARD kernels, none for isotropic ones; exp2_limit)
//   Matern32:  u = sqrt(3) r log2(e),   k = os*(1 + u ln2)*2^-min(u, 20 log2 e)
inline float kernel_scale(int kind) {
  switch (kind) {
    case KIND_RBF: return 0.84932180028801904272f;       // sqrt(0.5*log2 e)
    case KIND_MATERN12: return 1.44269504088896340736f;  // log2 e
    case KIND_MATERN32: return 2.49882111064734320000f;  // sqrt(3)*log2 e
    default: return 3.22596433305849393025f;             // sqrt(5)*log2 e
  }
}

// Packed tile counts are padded to a multiple of this (1536 points) so the
// symmetric product's blocks (256, 512 or 768 points) never read past the packing.
constexpr int64_t kPackTileAlign = 96;

// Builds packed operands (and scaled coordinates) for n points X[n][d].
void pack_points(const float* X_dev, int64_t n, const Coords& co,
                 PackedPoints& pp, hipStream_t st);

// Right-hand sides packed for the tile kernels by one product, for reuse by
// the next product of the same columns V over the same column points (the
// latents of an LMC product share V and X).
struct PackedRhs {
  const float* src = nullptr;  // V the packing was made from
  int64_t col_tiles = -1;      // column tiles of the points it was packed for
  int ncols = 0;
  const void* vp = nullptr;    // packed fp16 parts
  const uint32_t* colmax = nullptr;
};

struct MatvecArgs {
  int kind = KIND_RBF;
  float outputscale = 1.f;
  float noise = 0.f;     // added as noise*V on the diagonal (square only)
  bool square = false;   // rows and columns are the same point set
  int64_t m = 0;         // rows (output length per column)
  int64_t n = 0;         // columns (input length per column)
  int ncols = 0;         // right-hand sides
  // Optional task mixing in the epilogue (LMC): the columns form blocks of
  // mix_T (column c = cc*mix_T + t'), and the result is
  // out[cc][t][i] (+)= sum_t' mix[t*mix_T + t'] ((K + noise I) V)[cc][t'][i]
  // with mix a device [mix_T][mix_T] array; ncols must be a multiple of mix_T.
  const float* mix = nullptr;
  int mix_T = 0;
  bool mix_accumulate = false;
  // Optional packing reuse for a one-chunk product (ncols <= 64) on the
  // one-sided tile kernel without a fixed arena: when *reuse describes V at
  // these column points its packing is used, otherwise this product packs V
  // and records its buffers in *reuse.  The recorded buffers live in this
  // product's workspace and stay valid until that workspace's next product on
  // the same stream.
  PackedRhs* reuse = nullptr;
};

// out[c*m + i] = os * sum_j k(r_i, c_j) V[c*n + j]  (+ noise*V[c*m+i] if square)
// V and out are column-major device arrays.  Work buffers are grown in `ws`.
struct MatvecWorkspace {
  DevBuf<float> vpack;    // packed right-hand sides
  DevBuf<uint32_t> colmax;       // per-column max |V| (fp16 scaling of the product)
  DevBuf<uint32_t> colmax_part;  // [64][chunks] row-chunk maxima
  DevBuf<float> partial;  // split-K partial sums
  DevBuf<float> sym_tp;   // transposed partial sums of the symmetric product
  // Fixed-arena mode (allocation-free callers): when arena is set, every work
  // buffer above is carved from [arena, arena + arena_bytes) instead of being
  // grown with hipMalloc; the split count is capped so the partial sums fit,
  // and a request that cannot fit even unsplit raises ST_INVALID.
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  // Optional HIP-event timing of the tile kernel alone (bench hook).
  bool time_tile = false;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double tile_ms = 0.0;
  int64_t tile_calls = 0;
};

// A square product (rows and cols the same packed points) with 1..16
// right-hand sides runs on the symmetric kernel, which forms each
// off-diagonal kernel value once for both of its entries, when the points fill
// at least kSymMinBlocks 512-point blocks (n >= 47 * 512 + 1 = 24065) and its
// transposed partial sums (n^2/16 bytes) stay within kSymMaxBytes.  The environment variable
// MGP_SYM_MATVEC=0 turns that route off, =1 takes it for every square product
// the kernel can serve (any n), for tests and measurements.
void fused_matvec(const MatvecArgs& a, const PackedPoints& rows,
                  const PackedPoints& cols, const float* V_dev, float* out_dev,
                  MatvecWorkspace& ws, hipStream_t st, int force_splits = 0);
constexpr int64_t kSymMinBlocks = 48;
// True when a square product of the packed points with ncols right-hand
// sides (own work buffers) runs on the symmetric kernel, whose result for
// each column does not depend on the other columns.
bool symmetric_route_taken(const PackedPoints& pts, int ncols);
constexpr double kSymMaxBytes = 16e9;

// Bytes of work buffers one fused_matvec call with ncols right-hand sides
// over cols needs at the least (no split partials): the arena size below which
// the fixed-arena mode rejects the call.
size_t fused_matvec_min_arena(const PackedPoints& cols, int ncols);

// Reference-form product evaluated per pair from per-dimension differences of
// the scaled coordinates (no Gram form, no MFMA).  Used as an independent
// device cross-check and for dimensions beyond the MFMA tile path.
void direct_matvec(const MatvecArgs& a, const PackedPoints& rows,
                   const PackedPoints& cols, int d, const float* V_dev,
                   float* out_dev, hipStream_t st);

// Dense block of K(rows, cols): out[c*cols.n + i] = os k(row r0 + c, col i),
// c < nrows, from per-dimension differences of the scaled coordinates
// (fused_fill_cross_covariance, gpu_kernel.py:762-835).
void fill_cross(int kind, float outputscale, const PackedPoints& rows, int64_t r0,
                int64_t nrows, const PackedPoints& cols, int d, float* out, hipStream_t st);

// The symmetric half of the dense K (dense.h layout: nb blocks of 256 points,
// block index dense_half_index) filled directly from the packed points with
// the arithmetic of fill_cross, each value scaled by 2^shift and split.
void fill_dense_half(int kind, float outputscale, const PackedPoints& pts, int d, int shift,
                     int64_t nb, uint32_t* half, hipStream_t st);

// out[p][c][i] = sum_j dk(x_i, x_j)/dtheta_p V[c][j] for the P engine
// parameters ([l | l_0..l_{d-1}, os]); pscale_dev[p] converts the per-pair sums
// (h |dz|^2 terms, k/os terms) into derivatives: 1/(s^2 l_p) for lengthscales
// (times os), 1 for the outputscale (see the kernel's comment).
void gradient_matvec(int kind, bool ard, const PackedPoints& pts, int d, float outputscale,
                     const float* pscale_dev, const float* V_dev, int ncols, float* out_dev,
                     hipStream_t st);

// Maximum input dimension served by the MFMA tile path (three K=32 MFMAs).
constexpr int kMaxMfmaDim = 30;

// Work buffers of the matrix-core gradient trace (grown on demand, kept by
// the provider).
struct GradTraceWorkspace {
  DevBuf<float> wa, wb;          // packed [Rf'|Lf'] / [Lf';Rf'] operands (fp16 pairs)
  DevBuf<float> zz;              // packed [z | z^2] column operands (fp16 pairs)
  DevBuf<uint32_t> colmax, colmax_part;  // |Lf|, |Rf| column maxima (32) and row-chunk parts
  DevBuf<int> shifts;            // per-column exponents of Lf', Rf' and the common scale T
  DevBuf<double> part;           // workgroup partials
  std::vector<double> hpart;
};

// Gradient traces on the matrix cores, for the Gram-form kernels (RBF,
// Matern-3/2, Matern-5/2; not Matern-1/2) in up to 16 dimensions over a packed
// point set whose norms keep the Gram form accurate:
//   acc[q] += sum_ab W_ab h_ab (z_aq - z_bq)^2   (q < d),
//   acc[d] += sum_ab W_ab k_ab / os,
// with W = Lf^T Rf over ncols columns ([ncols][n] device arrays), z the
// scaled coordinates and h the kernel's lengthscale factor (RBF k/os,
// Matern-3/2 3 e^{-u}, Matern-5/2 (5/3)(1 + u) e^{-u}), the same sums as the
// pair-loop trace.  Only the symmetric part of W meets the symmetric h dz^2,
// so each unordered block pair is formed once with (W + W^T).  The
// environment variable MGP_GRAD_MFMA=0 keeps the pair-loop trace, =1 takes
// this one for any n the route allows.
bool grad_trace_mfma_route(int kind, const PackedPoints& pts, int d);
void grad_trace_mfma(int kind, const PackedPoints& pts, int d, const float* Lf,
                     const float* Rf, int ncols, double* acc, GradTraceWorkspace& ws,
                     hipStream_t st);
constexpr int64_t kGradMfmaMinPoints = 4096;

}  // namespace mgp
