// Dense kernel matrix of the materialized route and its products on the fp16
// matrix cores.
//
// Reference counterpart: the dense K of the reference's materialized mode and
// its matmul (_do_materialize / impl_forward_matvec with a stored K,
// mojogp/codegen_engine/emit/fn_ptr_module.py:363-420) and the exact-variance
// block products (kernels/jit/jit_prediction.mojo:438-587).
//
// Storage: K is held as a scaled two-term fp16 split.  Every entry is scaled
// by 2^shift (max |K| in [2^14, 2^15), so the e^-20 floor of the clamped
// kernels stays a normal fp16 number; unclamped RBF tails below that fall into
// fp16's subnormal range with absolute error <= 2^-25 of the scaled value) and
// split into hi = RNE16(x), lo = RNE16(x - hi), 4 bytes per entry like fp32.
// Both layouts store 8 consecutive columns of one row and one part as a
// 16-byte unit, lane-ordered so that 64 consecutive units are one 1 KB
// v_mfma_f32_16x16x32_f16 operand (16 rows x 32 columns) and one load per
// lane fetches it.  Rows and columns are padded with zeros to
// npad = round_up(n, 256).
#pragma once

#include "mgp_common.h"

namespace mgp {

struct DenseK {
  int64_t n = 0, npad = 0;
  int shift = 0;              // stored value = K * 2^shift (split)
  DevBuf<uint32_t> data;      // full K, fragment order (frag_index in dense.hip)
  bool full_valid = false;    // data holds K for the current parameters
  int64_t groups_per_row() const { return npad / 8; }
  // Symmetric half: for nb = npad / 256 blocks of 256 points, the blocks
  // (b, (b + delta) mod nb), delta = 0 .. sym_span(b, nb) (the diagonal block
  // and the cyclic half of the others, each unordered pair once), each 256 KB
  // of the split format above in fragment order (half_frag_index), at block
  // index dense_half_index(b, delta, nb): n^2/2 + 128 n entries instead of n^2.
  DevBuf<uint32_t> half;
  bool half_valid = false;
  int64_t blocks() const { return npad / 256; }
};

// Storage position of block (b, (b + delta) mod nb) of the symmetric half.
__host__ __device__ inline int64_t dense_half_index(int64_t b, int64_t delta, int64_t nb) {
  if (nb & 1) return b * ((nb - 1) / 2 + 1) + delta;
  const int64_t h = nb / 2;
  return (b < h ? b * (h + 1) : h * (h + 1) + (b - h) * h) + delta;
}
inline int64_t dense_half_blocks(int64_t nb) { return nb * (nb + 1) / 2; }

// Fragment order of a stored block: the 8-fp16 unit (h8 index) holding part p
// (0 hi, 1 lo) of row r (0..255), columns 8 g .. 8 g + 7 (g = 0..31) of
// stored block hb.  Per 32-column step s = g / 4 and 32-row slice w = r / 32,
// the two 16-row tiles' hi and lo parts are four consecutive 1 KB
// v_mfma_f32_16x16x32_f16 A operands (lane = r % 16 + 16 (g % 4)), so a
// wave's loads of one step are 4 KB contiguous and a workgroup of 8 such
// waves streams each step's 32 KB in one run.
__host__ __device__ inline int64_t half_frag_index(int64_t hb, int r, int g, int p) {
  const int lane = (r & 15) + 16 * (g & 3);
  return ((((hb * 8 + (g >> 2)) * 8 + (r >> 5)) * 2 + ((r >> 4) & 1)) * 2 + p) * 64 + lane;
}

// Work buffers of dense_forward, grown on demand.
struct DenseWorkspace {
  DevBuf<uint32_t> vpack;           // packed right-hand sides [cpad][npad / 8] groups
  DevBuf<uint32_t> vpair;           // right-hand sides in row-tile-pair order (symmetric route)
  DevBuf<uint32_t> colmax, colmax_part;
  DevBuf<uint32_t> shifts;          // output exponents of the symmetric route [16]
  DevBuf<uint32_t> colmax_sym;      // column maxima of the symmetric route, zero between products
  DevBuf<float> part;               // [splits][cpad][npad]
  DevBuf<float> tpart;              // transposed partial sums of the symmetric route
};

// Allocate K for n points (npad^2 entries, padding zeroed) with the scale of
// entries of magnitude up to kmax (> 0).
void dense_alloc(DenseK& K, int64_t n, float kmax, hipStream_t st);
// Pack rows [r0, r0 + nrows) of K given in fp32 with row stride n.
void dense_pack_rows(const float* rows, int64_t r0, int64_t nrows, DenseK& K, hipStream_t st);
// Allocate the symmetric half for n points with the scale of kmax (> 0).
void dense_alloc_half(DenseK& K, int64_t n, float kmax);
// Pack the symmetric half's blocks of row block b from its rows of K in fp32
// ([nrows][n], row stride n, nrows <= 256; rows past nrows are zero).
void dense_pack_half(const float* rows, int64_t b, int64_t nrows, DenseK& K, hipStream_t st);
// out = K V + noise V for 1..16 columns from the symmetric half: every
// off-diagonal block is read once and used for both of its products (the
// transposed one through gfx950's transposing LDS read), half the bytes of
// dense_forward.
void dense_sym_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                       DenseWorkspace& w, hipStream_t st);
// out = K V + noise V for V, out device [ncols][n]: products on the fp16 matrix
// cores (Kh Vh + Kh Vl + Kl Vh, each right-hand side split after scaling its
// column to max |V| in [2^14, 2^15)), fp32 accumulation over split ranges of
// columns of K, the split partials added in fixed order in fp64.
void dense_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                   DenseWorkspace& w, hipStream_t st);

}  // namespace mgp
