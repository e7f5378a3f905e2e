// Dense kernel matrix (materialized route) on the fp16 matrix cores: storage
// as a scaled two-term fp16 split and out = K V + noise V (see dense.h).
//
// Reference behaviour: the stored-K forward product of the materialized mode
// (mojogp/codegen_engine/emit/fn_ptr_module.py:363-420) and the exact-variance
// block products (kernels/jit/jit_prediction.mojo:438-587), both fp32 there.
// Here each product term is Kh Vh + Kh Vl + Kl Vh of the two-term splits: the
// dropped Kl Vl term and the rounding of the lo parts stay below ~3 2^-22 of
// |K V| per entry, and the accumulation is fp32 per column split, as in an
// fp32 GEMM; split partials are added in fp64.
#include "dense.h"
#include "sym_common.h"

#include <algorithm>
#include <cmath>

namespace mgp {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16 __attribute__((ext_vector_type(16)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void g_void;

namespace {

constexpr int kScaleLog2 = 15;  // scaled magnitudes in [2^14, 2^15)

// Power-of-two exponent that brings max |x| = mx into [2^14, 2^15); 0 for a
// zero or non-finite maximum.
__host__ __device__ inline int scale_shift(float mx) {
  if (!(mx > 0.0f) || mx > 3.0e38f) return 0;
  int e;
  (void)frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
  return kScaleLog2 - e;
}

__device__ __forceinline__ h16 split16(const float (&x)[8]) {
  h16 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const _Float16 hi = (_Float16)x[e];
    o[e] = hi;
    o[8 + e] = (_Float16)(x[e] - (float)hi);
  }
  return o;
}

__device__ __forceinline__ h8 first8(const h16& v) {
  return __builtin_shufflevector(v, v, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ h8 last8(const h16& v) {
  return __builtin_shufflevector(v, v, 8, 9, 10, 11, 12, 13, 14, 15);
}

// Fragment layout of the full K and of the packed right-hand sides (dense.h):
// the h8 index of row (or right-hand side) i, columns 8 g .. 8 g + 7, part p.
__host__ __device__ inline int64_t frag_index(int64_t i, int64_t g, int64_t nks, int p) {
  const int64_t lane = (i & 15) + 16 * (g & 3);
  return (((i >> 4) * nks + (g >> 2)) * 2 + p) * 64 + lane;
}

// Rows [r0, r0 + nrows) of 2^shift src (row stride n, zero past column n) into
// the fragment layout; one thread per (row, 8-column group).  vec4: n a
// multiple of 4 (16-byte rows).
__global__ void k_dense_pack(const float* __restrict__ src, int64_t r0, int64_t nrows, int64_t n,
                             int64_t gpr, int shift, int vec4, h8* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nrows * gpr) return;
  const int64_t r = idx / gpr, g = idx - r * gpr;
  const float* s = src + r * n;
  const int64_t j0 = 8 * g;
  float x[8];
  if (vec4 && j0 + 8 <= n) {
    const f4 a = *reinterpret_cast<const f4*>(s + j0);
    const f4 b = *reinterpret_cast<const f4*>(s + j0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = j0 + e < n ? s[j0 + e] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = ldexpf(x[e], shift);
  const h16 v = split16(x);
  const int64_t nks = gpr / 4;
  dst[frag_index(r0 + r, g, nks, 0)] = first8(v);
  dst[frag_index(r0 + r, g, nks, 1)] = last8(v);
}

// Zero rows [r0, r1) of the fragment layout (padding rows).
__global__ void k_dense_zero_rows(int64_t r0, int64_t r1, int64_t gpr, h8* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (r1 - r0) * gpr) return;
  const int64_t r = r0 + idx / gpr, g = idx % gpr;
  h8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (_Float16)0.0f;
  dst[frag_index(r, g, gpr / 4, 0)] = z;
  dst[frag_index(r, g, gpr / 4, 1)] = z;
}

// part[c * chunks + b] = max |V[c][i]| over row chunk b (float bits; grid =
// (chunks, ncols), 256 threads).
__global__ __launch_bounds__(256) void k_dense_absmax_part(const float* __restrict__ V, int64_t n,
                                                          uint32_t* __restrict__ part) {
  __shared__ uint32_t wm[4];
  const int c = blockIdx.y, chunks = gridDim.x;
  const int64_t len = (n + chunks - 1) / chunks;
  const int64_t i0 = (int64_t)blockIdx.x * len, i1 = min(n, i0 + len);
  const float* col = V + (int64_t)c * n;
  uint32_t mx = 0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x)
    mx = max(mx, __float_as_uint(fabsf(col[i])));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0)
    part[(int64_t)c * chunks + blockIdx.x] = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
}

// colmax[c] = max over the chunks (chunks <= 64); one wave per column.
__global__ void k_dense_absmax_final(const uint32_t* __restrict__ part, int chunks,
                                     uint32_t* __restrict__ colmax) {
  const int c = blockIdx.x, lane = threadIdx.x;
  uint32_t mx = lane < chunks ? part[(int64_t)c * chunks + lane] : 0u;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
  if (lane == 0) colmax[c] = mx;
}

// Right-hand sides in the fragment layout: column c, group g holds the split
// of 2^s_c V[c][8 g + e] (zero for c >= ncols or past n), s_c from the column
// maximum.
__global__ void k_dense_pack_rhs(const float* __restrict__ V, int64_t n, int ncols, int cpad,
                                 int64_t gpr, const uint32_t* __restrict__ colmax, int vec4,
                                 h8* __restrict__ Vp) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)cpad * gpr) return;
  const int c = (int)(idx / gpr);
  const int64_t g = idx - (int64_t)c * gpr, j0 = 8 * g;
  float x[8];
  if (c >= ncols) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
  } else {
    const float* s = V + (int64_t)c * n;
    if (vec4 && j0 + 8 <= n) {
      const f4 a = *reinterpret_cast<const f4*>(s + j0);
      const f4 b = *reinterpret_cast<const f4*>(s + j0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = a[e];
        x[4 + e] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = j0 + e < n ? s[j0 + e] : 0.0f;
    }
    const int sh = scale_shift(__uint_as_float(colmax[c]));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = ldexpf(x[e], sh);
  }
  const h16 v = split16(x);
  Vp[frag_index(c, g, gpr / 4, 0)] = first8(v);
  Vp[frag_index(c, g, gpr / 4, 1)] = last8(v);
}

// D = K V over the 32-column steps [s0, s1) of split blockIdx.z (narrow
// products).  Wave (wr, wc) of the block computes R row tiles x NCT column
// tiles of 16: rows i0 + 16 r + m, right-hand sides c0 + 16 ct + n.
// v_mfma_f32_16x16x32_f16 operands come straight from global memory: the
// fragment layout stores each 16 x 32 operand lane-ordered (hi 1 KB, lo 1 KB),
// so lane l loads 16 contiguous bytes per part.  Each tile accumulates
// Kh.Vh + Kh.Vl + Kl.Vh.  The loads of the next step are issued before this
// step's MFMAs (two register stages; the address of the prefetch is clamped
// into the split so no load is conditional).  DIRECT (one split):
// out[c][i] = 2^-(kshift + s_c) D + noise V[c][i] for i < n, c < ncols;
// otherwise part[(z cpad + c) npad + i] = D.
template <int R, int NCT, int WR, bool DIRECT>
__global__ __launch_bounds__(256) void k_dense_mm(
    const h8* __restrict__ Kp, int64_t nks, const h8* __restrict__ Vp, int64_t ssplit,
    int64_t npad, int cpad, float* __restrict__ part, int64_t n, int ncols, int kshift,
    const uint32_t* __restrict__ colmax, float noise, const float* __restrict__ V,
    float* __restrict__ out) {
  constexpr int WC = 4 / WR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave % WR, wc = wave / WR;
  const int lm = lane & 15, lq = lane >> 4;
  const int64_t i0 = ((int64_t)blockIdx.x * WR + wr) * (R * 16);
  const int c0 = (blockIdx.y * WC + wc) * (NCT * 16);
  const int64_t s0 = (int64_t)blockIdx.z * ssplit, s1 = min(nks, s0 + ssplit);
  // fragment (tile t, step s, part p) at ((t nks + s) 2 + p) 64 + lane
  const h8* ka[R];
#pragma unroll
  for (int r = 0; r < R; ++r) ka[r] = Kp + ((i0 / 16 + r) * nks) * 128 + lane;
  const h8* vb[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) vb[ct] = Vp + ((int64_t)(c0 / 16 + ct) * nks) * 128 + lane;
  f4 acc[R][NCT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[r][ct] = f4{0.f, 0.f, 0.f, 0.f};
  auto load = [&](int64_t s, h8 (&ah)[R], h8 (&al)[R], h8 (&bh)[NCT], h8 (&bl)[NCT])
      __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ah[r] = ka[r][s * 128];
      al[r] = ka[r][s * 128 + 64];
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      bh[ct] = vb[ct][s * 128];
      bl[ct] = vb[ct][s * 128 + 64];
    }
  };
  auto mma = [&](const h8 (&ah)[R], const h8 (&al)[R], const h8 (&bh)[NCT],
                 const h8 (&bl)[NCT]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[r], bh[ct], acc[r][ct], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[r], bl[ct], acc[r][ct], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[r], bh[ct], acc[r][ct], 0, 0, 0);
  };
  if (s0 < s1) {
    const int64_t slast = s1 - 1;
    h8 a0h[R], a0l[R], b0h[NCT], b0l[NCT], a1h[R], a1l[R], b1h[NCT], b1l[NCT];
    load(s0, a0h, a0l, b0h, b0l);
    for (int64_t s = s0; s < s1; s += 2) {
      load(min(s + 1, slast), a1h, a1l, b1h, b1l);
      mma(a0h, a0l, b0h, b0l);
      if (s + 1 >= s1) break;
      load(min(s + 2, slast), a0h, a0l, b0h, b0l);
      mma(a1h, a1l, b1h, b1l);
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int c = c0 + 16 * ct + lm;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = i0 + 16 * r + 4 * lq;
      if constexpr (DIRECT) {
        if (c < ncols) {
          const double sc = ldexp(1.0, -(kshift + scale_shift(__uint_as_float(colmax[c]))));
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (i + q < n) {
              const int64_t o = (int64_t)c * n + i + q;
              out[o] = fmaf(noise, V[o], (float)(sc * (double)acc[r][ct][q]));
            }
        }
      } else {
        *reinterpret_cast<f4*>(part + ((int64_t)blockIdx.z * cpad + c) * npad + i) = acc[r][ct];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide products (ncols > 128, the exact-variance blocks): D = K V for a
// 128-row x 256-column workgroup tile of 8 waves (2 x 4; each wave 4 x 4
// tiles of 16 x 16).  Per 32-column step the workgroup's 8 K fragments and 16
// V fragments (2 KB each, lane-ordered in global memory) are brought into LDS
// by the global-to-LDS DMA, 6 blocks of 1 KB per wave, into one of three
// stage buffers (48 KB each), two steps ahead of the MFMAs, so every operand
// byte crosses L2 once per workgroup instead of once per wave.  Workgroups are
// ordered for the XCDs: XCD x takes the row blocks x, x + 8, ... and walks
// them in groups of 8 row blocks x 4 column blocks, so the 32 workgroups an
// XCD runs at a time share their K rows and V columns in its L2.  The
// epilogue is the narrow kernel's DIRECT one (one split).
// ---------------------------------------------------------------------------
constexpr int kWideWaves = 8;
constexpr int kWideRowTiles = 8;    // 128 rows per workgroup
constexpr int kWideColTiles = 16;   // 256 right-hand sides per workgroup
constexpr int kWideStages = 3;
constexpr int kWideBlocks = 2 * (kWideRowTiles + kWideColTiles);  // 1-KB blocks per stage
constexpr int kWideGroupRows = 8, kWideGroupCols = 4;

__global__ __launch_bounds__(64 * kWideWaves) void k_dense_mm_wide(
    const h8* __restrict__ Kp, int64_t nks, const h8* __restrict__ Vp, int64_t rblocks,
    int64_t cblocks, int gcols, int64_t n, int ncols, int kshift,
    const uint32_t* __restrict__ colmax, float noise, const float* __restrict__ V,
    float* __restrict__ out) {
  __shared__ h8 lds[kWideStages][kWideBlocks][64];
  // workgroup -> (row block, column block), XCD-grouped (see above)
  const int64_t L = blockIdx.x;
  const int64_t x = L % kXcds, j = L / kXcds;
  const int64_t rbx = (rblocks - x + kXcds - 1) / kXcds;   // row blocks of XCD x
  if (j >= rbx * cblocks) return;                          // whole workgroup: no barrier yet
  const int64_t per_group = (int64_t)kWideGroupRows * cblocks;
  const int64_t g_r = j / per_group, rem = j - g_r * per_group;
  const int64_t ga = min((int64_t)kWideGroupRows, rbx - g_r * kWideGroupRows);
  const int64_t g_c = rem / (ga * gcols), inner = rem - g_c * (ga * gcols);
  const int64_t rr = g_r * kWideGroupRows + inner / gcols;
  const int64_t rb = x + kXcds * rr;
  const int64_t cb = g_c * gcols + inner % gcols;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave & 1, wc = wave >> 1;        // 2 row x 4 column waves
  const int64_t rt0 = rb * kWideRowTiles, ct0 = cb * kWideColTiles;
  // LDS block b of a stage: b < 16: K fragment (row tile b / 2, part b % 2);
  // b >= 16: V fragment (column tile (b - 16) / 2, part b % 2).
  auto fill = [&](int st, int64_t s) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kWideBlocks / kWideWaves; ++k) {
      const int b = wave + kWideWaves * k;
      const h8* src = b < 2 * kWideRowTiles
                          ? Kp + (((rt0 + (b >> 1)) * nks + s) * 2 + (b & 1)) * 64
                          : Vp + (((ct0 + ((b - 2 * kWideRowTiles) >> 1)) * nks + s) * 2 +
                                  (b & 1)) * 64;
      __builtin_amdgcn_global_load_lds((const g_void*)(src + lane), (lds_void*)&lds[st][b][0],
                                       16, 0, 0);
    }
  };
  f4 acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = f4{0.f, 0.f, 0.f, 0.f};
  fill(0, 0);
  if (nks > 1) fill(1, 1);
  for (int64_t s = 0; s < nks; ++s) {
    const int st = (int)(s % kWideStages);
    // this wave's blocks of step s have landed (those of s + 1 may be in
    // flight); the barrier makes every wave's blocks of step s visible and
    // frees the buffer of step s - 1 for step s + 2
    if (s + 1 < nks)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (kWideBlocks / kWideWaves));  // vmcnt <= 6
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);                              // vmcnt = 0
    __syncthreads();
    if (s + 2 < nks) fill((int)((s + 2) % kWideStages), s + 2);
    h8 ah[4], al[4], bh[4], bl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ah[r] = lds[st][2 * (4 * wr + r)][lane];
      al[r] = lds[st][2 * (4 * wr + r) + 1][lane];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bh[c] = lds[st][2 * kWideRowTiles + 2 * (4 * wc + c)][lane];
      bl[c] = lds[st][2 * kWideRowTiles + 2 * (4 * wc + c) + 1][lane];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[r], bh[c], acc[r][c], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[r], bl[c], acc[r][c], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[r], bh[c], acc[r][c], 0, 0, 0);
  }
  const int lm = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t col = (ct0 + 4 * wc + c) * 16 + lm;
    if (col >= ncols) continue;
    const double sc = ldexp(1.0, -(kshift + scale_shift(__uint_as_float(colmax[col]))));
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = (rt0 + 4 * wr + r) * 16 + 4 * lq;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (i + q < n) {
          const int64_t o = col * n + i + q;
          out[o] = fmaf(noise, V[o], (float)(sc * (double)acc[r][c][q]));
        }
    }
  }
}

// out[c][i] = 2^-(kshift + s_c) sum_z part[(z cpad + c) npad + i] (fp64, split
// order) + noise V[c][i].
__global__ void k_dense_reduce(const float* __restrict__ part, int splits, int cpad,
                               int64_t npad, int64_t n, int ncols, int kshift,
                               const uint32_t* __restrict__ colmax, float noise,
                               const float* __restrict__ V, float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)ncols * n) return;
  const int c = (int)(idx / n);
  const int64_t i = idx - (int64_t)c * n;
  const float* p = part + (int64_t)c * npad + i;
  const int64_t stride = (int64_t)cpad * npad;
  double s = 0.0;
  int z = 0;
  for (; z + 4 <= splits; z += 4) {
    float t[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) t[q] = p[(z + q) * stride];
#pragma unroll
    for (int q = 0; q < 4; ++q) s += (double)t[q];
  }
  for (; z < splits; ++z) s += (double)p[z * stride];
  const double sc = ldexp(1.0, -(kshift + scale_shift(__uint_as_float(colmax[c]))));
  out[idx] = fmaf(noise, V[idx], (float)(sc * s));
}

// ---------------------------------------------------------------------------
// Symmetric half of K and its products.
//
// K is symmetric, so the half keeps the diagonal blocks and the cyclic half
// of the off-diagonal blocks of 256 points (sym_span), each unordered pair
// once, in fragment order.  A product with <= 16 right-hand sides reads every
// stored block once, each wave one 32-column slice of it:
//   * forward, out_b += K_bJ V_J: the block's fragments straight from global
//     memory as the A operand, V_J's fragment as the B operand;
//   * transposed (J != b), out_J += K_bJ^T V_b: the wave stores each row
//     pair's 8-byte chunks (row, 4 columns) of both parts to a wave-private
//     LDS scratch and reads them back with ds_read_b64_tr_b16, which yields
//     the slice transposed into the B operand of O_J^T += V_b^T K_bJ,
//     contracted over the pair's rows in the row-tile-pair order of the
//     pair-packed V_b (A operand, loaded once per wave) and accumulated over
//     the block's 8 row pairs, so the slice's 256-row partial tp[b][delta - 1]
//     is complete in the wave;
//   * k_dense_sym_reduce adds, per point, the forward split partials and the
//     partials of the row blocks that formed its column block (fp64, fixed
//     order).
// ---------------------------------------------------------------------------
constexpr int kDsRows = 256;                    // points per block
constexpr int kDsGroups = kDsRows / 8;          // 8-column groups per block row
constexpr int kDsWaves = 8;                     // waves per workgroup, one column step each
constexpr int kDsSteps = kDsRows / 32;          // 32-column steps per block
constexpr int kDsRing = 4;                      // register sets of sub-step operands
constexpr int kDsDepth = 3;                     // sub-steps loaded ahead

// One thread per (delta, row, group) of row block b's stored blocks, in
// fragment order (consecutive threads write consecutive 16-byte units).
__global__ void k_dense_pack_half(const float* __restrict__ rows, int64_t nrows, int64_t n,
                                  int64_t b, int64_t nb, int64_t span, int shift, int vec4,
                                  h8* __restrict__ half) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (span + 1) * kDsRows * kDsGroups) return;
  const int64_t delta = idx / (kDsRows * kDsGroups);
  const int u = (int)(idx - delta * (kDsRows * kDsGroups));
  const int lane = u & 63;
  const int r = 32 * ((u >> 7) & 7) + 16 * ((u >> 6) & 1) + (lane & 15);
  const int g = 4 * (u >> 10) + (lane >> 4);
  int64_t J = b + delta;
  if (J >= nb) J -= nb;
  const int64_t j0 = J * kDsRows + 8 * g;
  float x[8];
  const float* s = rows + r * n;
  if (r < nrows && vec4 && j0 + 8 <= n) {
    const f4 a = *reinterpret_cast<const f4*>(s + j0);
    const f4 c = *reinterpret_cast<const f4*>(s + j0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = c[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (r < nrows && j0 + e < n) ? s[j0 + e] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = ldexpf(x[e], shift);
  const h16 v = split16(x);
  const int64_t hb = dense_half_index(b, delta, nb);
  half[half_frag_index(hb, r, g, 0)] = first8(v);
  half[half_frag_index(hb, r, g, 1)] = last8(v);
}

// Column maxima of |V| for the symmetric route in one launch: block
// (chunk, c) folds the max of its rows' |V| bits into cm[c] with an unsigned
// atomicMax, which is order independent, so cm[c] equals the two-launch
// k_dense_absmax_part / _final result bit for bit.  cm holds zeros on entry:
// k_dense_sym_reduce clears it for the next product.
__global__ __launch_bounds__(256) void k_dense_colmax_atomic(const float* __restrict__ V,
                                                            int64_t n, uint32_t* __restrict__ cm) {
  __shared__ uint32_t wm[4];
  const int c = blockIdx.y, chunks = gridDim.x;
  const int64_t len = (n + chunks - 1) / chunks;
  const int64_t i0 = (int64_t)blockIdx.x * len, i1 = min(n, i0 + len);
  const float* col = V + (int64_t)c * n;
  uint32_t mx = 0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x)
    mx = max(mx, __float_as_uint(fabsf(col[i])));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(cm + c, max(max(wm[0], wm[1]), max(wm[2], wm[3])));
}

// Both right-hand-side layouts of the symmetric route in one launch, one
// thread per (column c < 16, 32-point unit u): the fragment layout of
// k_dense_pack_rhs (Vf, 16 columns) and the row-tile-pair layout (Vpp[(2 u +
// part) 64 + c + 16 lg] holds points 32 u + 16 (e/4) + 4 lg + e%4), with the
// scaling and split of k_dense_pack_rhs, plus the output exponents
// shifts[c] = kshift + s_c.  Zero for c >= ncols or past n.
__global__ __launch_bounds__(256) void k_dense_pack_sym(
    const float* __restrict__ V, int64_t n, int ncols, int64_t units,
    const uint32_t* __restrict__ cm, int kshift, int vec4, int* __restrict__ shifts,
    h8* __restrict__ Vf, h8* __restrict__ Vpp) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= units * 16) return;
  const int c = (int)(idx & 15);
  const int64_t u = idx >> 4;
  const int sh = c < ncols ? scale_shift(__uint_as_float(cm[c])) : 0;
  if (u == 0) shifts[c] = kshift + sh;
  float x[32];
  const int64_t j0 = 32 * u;
  const float* src = V + (int64_t)(c < ncols ? c : 0) * n + j0;
  if (c < ncols && vec4 && j0 + 32 <= n) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const f4 a = *reinterpret_cast<const f4*>(src + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * q + e] = a[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) x[e] = (c < ncols && j0 + e < n) ? src[e] : 0.0f;
  }
  _Float16 hi[32], lo[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float v = ldexpf(x[e], sh);
    hi[e] = (_Float16)v;
    lo[e] = (_Float16)(v - (float)hi[e]);
  }
  // fragment layout: group g = 4 u + k holds points 8 g .. 8 g + 7
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    h8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = hi[8 * k + e];
      b[e] = lo[8 * k + e];
    }
    Vf[(u * 2) * 64 + c + 16 * k] = a;
    Vf[(u * 2 + 1) * 64 + c + 16 * k] = b;
  }
  // pair layout: lane c + 16 lg holds points 32 u + 16 (e / 4) + 4 lg + e % 4
#pragma unroll
  for (int lg = 0; lg < 4; ++lg) {
    h8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int p = 16 * (e >> 2) + 4 * lg + (e & 3);
      a[e] = hi[p];
      b[e] = lo[p];
    }
    Vpp[(u * 2) * 64 + c + 16 * lg] = a;
    Vpp[(u * 2 + 1) * 64 + c + 16 * lg] = b;
  }
}

__global__ void k_dense_clear16(uint32_t* __restrict__ p) {
  if (threadIdx.x < 16) p[threadIdx.x] = 0u;
}

// Work item L = (row block b, delta split) of the symmetric half product.
// Kf: the half in fragment order (half_frag_index); Vf: the right-hand sides
// in the fragment layout of k_dense_pack_rhs (16 columns, one tile), so the
// B operand of 32-column step S of the points is Vf[(2 S + p) 64 + lane];
// Vpp: the right-hand sides in row-tile-pair order (element e of lane
// c + 16 lg of unit u is point 32 u + 16 (e/4) + 4 lg + e%4) and shifts the
// output exponents (both from k_dense_pack_sym).
// Wave w owns the 32-column step w of every block of the item and streams
// its column slice (8 row pairs of 4 KB, one contiguous 32 KB run) forming
//   forward     acc[tile] += K[tile rows, step w] V_J[step w]  (16 row tiles)
//   transposed  tacc[tt]  += V_b[pair rows]^T K[pair rows, step w]
// so the transposed sums of the block's 32 columns complete inside the wave
// over all 256 rows and go straight to tp, and only the forward sums, which
// accumulate over the item's blocks, are added across the 8 waves, once.
// fwd[(split*16 + c)*mpad + i]: forward sums of the split's blocks, unscaled;
// tp[((b*hmax + delta - 1)*256 + column)*16 + c]: transposed block sums.
__global__ __launch_bounds__(64 * kDsWaves) void k_dense_sym(
    const h8* __restrict__ Kf, const h8* __restrict__ Vf, const h8* __restrict__ Vpp,
    int64_t nb, int64_t splits, int64_t dps, int64_t hmax, const int* __restrict__ shifts,
    float* __restrict__ fwd, float* __restrict__ tp, int64_t mpad) {
  constexpr int W = kDsWaves;
  static_assert(W == kDsSteps, "one wave per 32-column step of a block");
  // Wave-private transposition scratch: [column tile][hi, lo][row tile][chunk].
  __shared__ uint64_t tsc[W][2][2][2][64];
  // Forward sums of 8 row tiles per wave, for the cross-wave addition.
  __shared__ f4 red[W][8][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Items in launch order (the XCDs are dealt workgroups in turn): the short
  // last split's items are spread over all XCDs instead of loading one.
  const int64_t L = blockIdx.x;
  if (L >= nb * splits) return;  // whole workgroup, before any barrier
  const int64_t b = L % nb;
  const int64_t split = L / nb;
  const int li = lane & 15, lg = lane >> 4;
  const int chunk_r = sym_read_chunk(lane);
  const int tw = lg >> 1, q0 = 2 * (lg & 1);  // column tile and first quad of this lane's group

  const int64_t span = sym_span(b, nb);
  const int64_t d0 = split * dps;
  const int64_t nblk = max(min(d0 + dps, span + 1) - d0, (int64_t)0);
  const int64_t nsub = nblk * kDsSteps;  // (block, row pair) sub-steps of the item
  // Sub-step t: the wave's step of row pair t % 8 of block d0 + t / 8, both
  // row tiles, hi and lo (lane: row 16 r + li, group 4 w + lg).  The half is
  // read once per product, so its loads are non-temporal: they do not
  // displace the partial sums and operands held in the caches.
  auto load = [&](int64_t t, h8 (&kh)[2], h8 (&kl)[2]) __attribute__((always_inline)) {
    const int64_t delta = d0 + t / kDsSteps;
    const int rp = (int)(t % kDsSteps);
    const h8* kp =
        Kf + half_frag_index(dense_half_index(b, delta, nb), 32 * rp, 4 * wave, 0) + lane;
    kh[0] = __builtin_nontemporal_load(kp);
    kl[0] = __builtin_nontemporal_load(kp + 64);
    kh[1] = __builtin_nontemporal_load(kp + 128);
    kl[1] = __builtin_nontemporal_load(kp + 192);
  };

  // V_J of block bi (column step w), loaded one block ahead: a load issued at
  // the block start and consumed at once would also wait for the previous
  // block's tp stores, which the memory counter orders before it.
  auto load_v = [&](int64_t bi, h8& vh, h8& vl) __attribute__((always_inline)) {
    int64_t J = b + d0 + bi;
    if (J >= nb) J -= nb;
    const h8* vp = Vf + (J * kDsSteps + wave) * 128 + lane;
    vh = vp[0];
    vl = vp[64];
  };
  // Loads run kDsDepth sub-steps ahead in a ring of kDsRing register sets;
  // a block's 8 sub-steps are unrolled, so every set is addressed statically
  // (no register copies, which would wait for loads still in flight).  The
  // item's first loads go out oldest-first in the order they are consumed,
  // so no wait inside the loop covers more than the operand it needs.
  constexpr int R = kDsRing, D = kDsDepth;
  static_assert(kDsSteps % R == 0 && D < R, "the ring must tile a block's sub-steps");
  h8 bkh[R][2], bkl[R][2];
  h8 vh, vl, nvh, nvl;
  if (nblk > 0) load_v(0, vh, vl);
#pragma unroll
  for (int k = 0; k < D; ++k)
    if (nsub > 0) load(min((int64_t)k, nsub - 1), bkh[k], bkl[k]);
  // V_b in row-tile-pair order: the A operand of the transposed products.
  h8 vbh[kDsSteps], vbl[kDsSteps];
#pragma unroll
  for (int rp = 0; rp < kDsSteps; ++rp) {
    const int64_t u = b * kDsSteps + rp;
    vbh[rp] = Vpp[(u * 2) * 64 + lane];
    vbl[rp] = Vpp[(u * 2 + 1) * 64 + lane];
  }
  // Output exponents: the lane's transposed right-hand sides 4 lg + q and its
  // forward right-hand side li.
  const int4 tsh = *reinterpret_cast<const int4*>(shifts + 4 * lg);
  const int fsh = shifts[li];

  f4 acc[2 * kDsSteps];
#pragma unroll
  for (int u = 0; u < 2 * kDsSteps; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};
  for (int64_t bi = 0; bi < nblk; ++bi) {
    const int64_t delta = d0 + bi;
    const bool sym = delta > 0;
    f4 tacc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int k = 0; k < kDsSteps; ++k) {
      const int64_t t = bi * kDsSteps + k;
      const int cur = k % R, nxt = (k + D) % R;
      load(min(t + D, nsub - 1), bkh[nxt], bkl[nxt]);  // clamped: always a valid block
      if (k == 0) load_v(min(bi + 1, nblk - 1), nvh, nvl);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        f4 a = acc[2 * k + r];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(bkh[cur][r], vh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(bkh[cur][r], vl, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(bkl[cur][r], vh, a, 0, 0, 0);
        acc[2 * k + r] = a;
      }
      if (sym) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const u64x2 h = __builtin_bit_cast(u64x2, bkh[cur][r]);
          const u64x2 l = __builtin_bit_cast(u64x2, bkl[cur][r]);
          tsc[wave][tw][0][r][sym_chunk(li, q0)] = h[0];
          tsc[wave][tw][0][r][sym_chunk(li, q0 + 1)] = h[1];
          tsc[wave][tw][1][r][sym_chunk(li, q0)] = l[0];
          tsc[wave][tw][1][r][sym_chunk(li, q0 + 1)] = l[1];
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          h8 tp2[2];
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const u64x2 v = {tr_read(&tsc[wave][tt][p][0][chunk_r]),
                             tr_read(&tsc[wave][tt][p][1][chunk_r])};
            tp2[p] = __builtin_bit_cast(h8, v);
          }
          f4 a = tacc[tt];
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbh[k], tp2[0], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbl[k], tp2[0], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbh[k], tp2[1], a, 0, 0, 0);
          tacc[tt] = a;
        }
        asm volatile("" ::: "memory");
      }
    }
    if (sym) {
      // lane: right-hand sides 4 lg + q of column 32 w + 16 tt + li of block J
      const int64_t blk = b * hmax + delta - 1;
      const f4 tscale = {ldexpf(1.0f, -tsh.x), ldexpf(1.0f, -tsh.y), ldexpf(1.0f, -tsh.z),
                         ldexpf(1.0f, -tsh.w)};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        *reinterpret_cast<f4*>(tp + (blk * kDsRows + 32 * wave + 16 * tt + li) * 16 + 4 * lg) =
            tacc[tt] * tscale;
    }
    vh = nvh;
    vl = nvl;
  }
  // Forward sums: the 8 waves' fp32 sums of each row tile added in wave order
  // in fp64, 8 row tiles per round (thread: tile wave, lane = column li, rows
  // 4 lg + q of the tile).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; ++u) red[wave][u][lane] = acc[8 * h + u];
    __syncthreads();
    double sum[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const f4 v = red[w][wave][lane];
#pragma unroll
      for (int q = 0; q < 4; ++q) sum[q] += (double)v[q];
    }
    f4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = (float)ldexp(sum[q], -fsh);
    const int tile = 8 * h + wave;
    *reinterpret_cast<f4*>(fwd + (split * 16 + li) * mpad + b * kDsRows + 16 * tile + 4 * lg) = o;
  }
}

// out[c*n + j] = sum_s fwd[s][c][j] + the transposed partials of the row
// blocks that formed j's column block (delta order) + noise V; four threads
// per point, four right-hand sides each, fp64 sums.
__global__ __launch_bounds__(256) void k_dense_sym_reduce(
    const float* __restrict__ fwd, int splits, const float* __restrict__ tp, int64_t nb,
    int64_t hmax, int64_t mpad, int64_t n, int ncols, float noise,
    const float* __restrict__ V, float* __restrict__ out, uint32_t* __restrict__ cm) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < 16) cm[t] = 0u;  // the column maxima of the next product start from zero
  const int64_t j = t >> 2;
  const int c4 = (int)(t & 3);
  if (j >= n) return;
  double tot[4] = {0.0, 0.0, 0.0, 0.0};
  for (int s = 0; s < splits; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 4 * c4 + e;
      if (c < ncols) tot[e] += fwd[((int64_t)s * 16 + c) * mpad + j];
    }
  const int64_t J = j / kDsRows, jl = j - J * kDsRows;
  const float* col = tp + jl * 16 + 4 * c4;
  // Four partials in flight at a time (every slot is allocated; the formed
  // ones are kept by a select), in delta order.
  auto slot = [&](int64_t dl, bool& formed) {
    int64_t bb = J - dl;
    if (bb < 0) bb += nb;
    formed = dl <= sym_span(bb, nb);
    return *reinterpret_cast<const f4*>(col + (bb * hmax + dl - 1) * (int64_t)kDsRows * 16);
  };
  int64_t dl = 1;
  for (; dl + 3 <= hmax; dl += 4) {
    f4 v[4];
    bool ok[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = slot(dl + q, ok[q]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) tot[e] += ok[q] ? (double)v[q][e] : 0.0;
  }
  for (; dl <= hmax; ++dl) {
    bool ok;
    const f4 v = slot(dl, ok);
#pragma unroll
    for (int e = 0; e < 4; ++e) tot[e] += ok ? (double)v[e] : 0.0;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int c = 4 * c4 + e;
    if (c < ncols) {
      const int64_t idx = (int64_t)c * n + j;
      out[idx] = fmaf(noise, V[idx], (float)tot[e]);
    }
  }
}

}  // namespace

void dense_alloc(DenseK& K, int64_t n, float kmax, hipStream_t st) {
  MGP_REQUIRE(n >= 1, "dense K needs at least one point");
  MGP_REQUIRE(std::isfinite(kmax) && kmax > 0.f, "dense K scale needs a finite maximum > 0");
  K.n = n;
  K.npad = round_up(n, 256);
  K.shift = scale_shift(kmax);
  const int64_t gpr = K.groups_per_row();
  K.data.ensure((size_t)K.npad * (size_t)gpr * 8);
  // padding rows [n, npad); padding columns are written by the row packing
  const int64_t pad = (K.npad - n) * gpr;
  if (pad > 0) {
    hipLaunchKernelGGL(k_dense_zero_rows, dim3((unsigned)ceil_div(pad, 256)), dim3(256), 0, st,
                       n, K.npad, gpr, reinterpret_cast<h8*>(K.data.ptr));
    MGP_HIP_CHECK(hipGetLastError());
  }
}

void dense_pack_rows(const float* rows, int64_t r0, int64_t nrows, DenseK& K, hipStream_t st) {
  MGP_REQUIRE(r0 >= 0 && nrows >= 0 && r0 + nrows <= K.n, "dense K rows out of range");
  if (nrows == 0) return;
  const int64_t gpr = K.groups_per_row();
  const int64_t total = nrows * gpr;
  const int vec4 = (K.n % 4 == 0 && reinterpret_cast<uintptr_t>(rows) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st, rows,
                     r0, nrows, K.n, gpr, K.shift, vec4, reinterpret_cast<h8*>(K.data.ptr));
  MGP_HIP_CHECK(hipGetLastError());
}

void dense_alloc_half(DenseK& K, int64_t n, float kmax) {
  MGP_REQUIRE(n >= 1, "dense K needs at least one point");
  MGP_REQUIRE(std::isfinite(kmax) && kmax > 0.f, "dense K scale needs a finite maximum > 0");
  K.n = n;
  K.npad = round_up(n, kDsRows);
  K.shift = scale_shift(kmax);
  K.half.ensure((size_t)dense_half_blocks(K.blocks()) * kDsRows * kDsGroups * 8);
}

void dense_pack_half(const float* rows, int64_t b, int64_t nrows, DenseK& K, hipStream_t st) {
  const int64_t nb = K.blocks();
  MGP_REQUIRE(b >= 0 && b < nb && nrows >= 0 && nrows <= kDsRows, "dense K block out of range");
  const int64_t span = sym_span(b, nb);
  const int64_t total = (span + 1) * kDsRows * kDsGroups;
  const int vec4 = (K.n % 4 == 0 && reinterpret_cast<uintptr_t>(rows) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack_half, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                     rows, nrows, K.n, b, nb, span, K.shift, vec4,
                     reinterpret_cast<h8*>(K.half.ptr));
  MGP_HIP_CHECK(hipGetLastError());
}

void dense_sym_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                       DenseWorkspace& w, hipStream_t st) {
  MGP_REQUIRE(ncols >= 1 && ncols <= 16, "the symmetric dense product takes 1..16 columns");
  MGP_REQUIRE(K.half_valid, "the symmetric half of K is not filled");
  const int64_t n = K.n, npad = K.npad, gpr = K.groups_per_row(), nb = K.blocks();
  const int64_t hmax = nb / 2;
  int64_t splits = std::min<int64_t>(std::max<int64_t>(ceil_div(2048, nb), 1), hmax + 1);
  const int64_t dps = ceil_div(hmax + 1, splits);
  splits = ceil_div(hmax + 1, dps);
  // every buffer first: nothing may fail between the column maxima (which
  // accumulate into cm) and the reduction that clears cm again
  const bool fresh = w.colmax_sym.count < 16;
  uint32_t* cm = w.colmax_sym.ensure(16);
  const int64_t vtot = 16 * gpr;
  h8* vf = reinterpret_cast<h8*>(w.vpack.ensure((size_t)vtot * 8));
  const int64_t units = npad / 32;
  h8* vp = reinterpret_cast<h8*>(w.vpair.ensure((size_t)units * 2 * 64 * 4));
  int* shifts = reinterpret_cast<int*>(w.shifts.ensure(16));
  float* fwd = w.part.ensure((size_t)splits * 16 * npad);
  float* tp = w.tpart.ensure((size_t)std::max<int64_t>(nb * hmax, 1) * kDsRows * 16);
  if (fresh) hipLaunchKernelGGL(k_dense_clear16, dim3(1), dim3(64), 0, st, cm);
  const int chunks = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(n, 4096)));
  hipLaunchKernelGGL(k_dense_colmax_atomic, dim3((unsigned)chunks, (unsigned)ncols), dim3(256), 0,
                     st, V, n, cm);
  const int vec4 = (n % 4 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack_sym, dim3((unsigned)ceil_div(units * 16, 256)), dim3(256), 0,
                     st, V, n, ncols, units, cm, K.shift, vec4, shifts, vf, vp);
  MGP_HIP_CHECK(hipGetLastError());
  const int64_t items = nb * splits;
  hipLaunchKernelGGL(k_dense_sym, dim3((unsigned)items), dim3(64 * kDsWaves), 0, st,
                     reinterpret_cast<const h8*>(K.half.ptr), vf, vp, nb, splits, dps, hmax,
                     shifts, fwd, tp, npad);
  MGP_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_dense_sym_reduce, dim3((unsigned)ceil_div(4 * n, 256)), dim3(256), 0, st,
                     fwd, (int)splits, tp, nb, hmax, npad, n, ncols, noise, V, out, cm);
  MGP_HIP_CHECK(hipGetLastError());
}

void dense_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                   DenseWorkspace& w, hipStream_t st) {
  MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
  const int64_t n = K.n, npad = K.npad, gpr = K.groups_per_row(), nks = gpr / 4;
  const bool wide = ncols > 128;
  // block shape: rows x right-hand sides per workgroup
  int R = 4, NCT, WR;
  if (ncols <= 16) { NCT = 1; WR = 4; }
  else if (ncols <= 32) { NCT = 2; WR = 4; }
  else if (ncols <= 64) { NCT = 4; WR = 4; }
  else { NCT = 4; WR = 2; }
  const int WC = 4 / WR;
  const int64_t brows = (int64_t)WR * R * 16;
  const int64_t bcols = wide ? 16 * kWideColTiles : (int64_t)WC * NCT * 16;
  const int cpad = (int)round_up(ncols, bcols);
  const int64_t rblocks = wide ? npad / (16 * kWideRowTiles) : npad / brows;
  const int64_t cblocks = cpad / bcols;

  // column maxima and packed right-hand sides
  const int chunks = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(n, 4096)));
  uint32_t* cpart = w.colmax_part.ensure((size_t)chunks * ncols);
  uint32_t* colmax = w.colmax.ensure((size_t)ncols);
  hipLaunchKernelGGL(k_dense_absmax_part, dim3((unsigned)chunks, (unsigned)ncols), dim3(256), 0,
                     st, V, n, cpart);
  hipLaunchKernelGGL(k_dense_absmax_final, dim3((unsigned)ncols), dim3(64), 0, st, cpart, chunks,
                     colmax);
  const int64_t vtot = (int64_t)cpad * gpr;
  h8* vp = reinterpret_cast<h8*>(w.vpack.ensure((size_t)vtot * 8));
  const int vec4 = (n % 4 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack_rhs, dim3((unsigned)ceil_div(vtot, 256)), dim3(256), 0, st, V,
                     n, ncols, cpad, gpr, colmax, vec4, vp);
  MGP_HIP_CHECK(hipGetLastError());
  const h8* kp = reinterpret_cast<const h8*>(K.data.ptr);

  if (wide) {
    const int gcols = cblocks % kWideGroupCols == 0 ? kWideGroupCols : (cblocks % 2 == 0 ? 2 : 1);
    const int64_t per_xcd = ceil_div(rblocks, kXcds) * cblocks;
    hipLaunchKernelGGL(k_dense_mm_wide, dim3((unsigned)(per_xcd * kXcds)),
                       dim3(64 * kWideWaves), 0, st, kp, nks, vp, rblocks, cblocks, gcols, n,
                       ncols, K.shift, colmax, noise, V, out);
    MGP_HIP_CHECK(hipGetLastError());
    return;
  }

  // splits of the K columns: >= 2048 workgroups while every split keeps >= 8
  // steps (256 columns of K)
  int64_t splits = 1;
  while (rblocks * cblocks * splits < 2048 && nks / (splits * 2) >= 8 && splits < 64) splits *= 2;
  const int64_t ssplit = ceil_div(nks, splits);
  splits = ceil_div(nks, ssplit);
  float* part = nullptr;
  if (splits > 1) part = w.part.ensure((size_t)splits * cpad * npad);
  const dim3 grid((unsigned)rblocks, (unsigned)cblocks, (unsigned)splits);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, kp, nks, vp, ssplit, npad, cpad, part, n,
                       ncols, K.shift, colmax, noise, V, out);
  };
#define MGP_DENSE(NCT_, WR_)                                                          \
  (splits == 1 ? go(k_dense_mm<4, NCT_, WR_, true>) : go(k_dense_mm<4, NCT_, WR_, false>))
  if (NCT == 1) MGP_DENSE(1, 4);
  else if (NCT == 2) MGP_DENSE(2, 4);
  else if (WR == 4) MGP_DENSE(4, 4);
  else MGP_DENSE(4, 2);
#undef MGP_DENSE
  MGP_HIP_CHECK(hipGetLastError());
  if (splits > 1) {
    const int64_t tot = (int64_t)ncols * n;
    hipLaunchKernelGGL(k_dense_reduce, dim3((unsigned)ceil_div(tot, 256)), dim3(256), 0, st, part,
                       (int)splits, cpad, npad, n, ncols, K.shift, colmax, noise, V, out);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace mgp
