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

// Right-hand sides in group order for the symmetric route: Vn[c * gpr + g] =
// split of 2^s_c V[c][8 g + e] (zero for c >= ncols or past n).
__global__ void k_dense_pack_rhs_groups(const float* __restrict__ V, int64_t n, int ncols,
                                        int cpad, int64_t gpr,
                                        const uint32_t* __restrict__ colmax, int vec4,
                                        h16* __restrict__ Vn) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)cpad * gpr) return;
  const int c = (int)(idx / gpr);
  const int64_t g = idx - (int64_t)c * gpr, j0 = 8 * g;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = 0.0f;
  if (c < ncols) {
    const float* src = V + (int64_t)c * n;
    if (vec4 && j0 + 8 <= n) {
      const f4 a = *reinterpret_cast<const f4*>(src + j0);
      const f4 b = *reinterpret_cast<const f4*>(src + j0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = a[e];
        x[4 + e] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = j0 + e < n ? src[j0 + e] : 0.0f;
    }
    const int sh = scale_shift(__uint_as_float(colmax[c]));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = ldexpf(x[e], sh);
  }
  Vn[idx] = split16(x);
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
// once.  A product with <= 16 right-hand sides reads every stored block once:
//   * forward, out_b += K_bJ V_J: the block rows straight from global memory
//     as the A operand (the layout of dense_forward), V_J in the same group
//     order as the B operand;
//   * transposed (J != b), out_J += K_bJ^T V_b: each wave stores its two row
//     tiles' 8-byte chunks (row, 4 columns) of both parts to a wave-private
//     LDS scratch and reads them back with ds_read_b64_tr_b16, which yields
//     the block transposed into the B operand of O_J^T += V_b^T K_bJ,
//     contracted over the wave's two row tiles in the row-tile-pair order of
//     the pair-packed V_b (A operand, loaded once per wave);
//   * the waves' transposed sums (32 rows each) are added in wave order after
//     the next barrier and written as the 256-row partial tp[b][delta - 1];
//     k_dense_sym_reduce adds, per point, the forward split partials and the
//     partials of the row blocks that formed its column block (fp64, fixed
//     order).
// ---------------------------------------------------------------------------
constexpr int kDsRows = 256;                    // points per block
constexpr int kDsGroups = kDsRows / 8;          // 8-column groups per block row
constexpr int kDsWaves = 8;                     // waves per workgroup, 32 rows each
constexpr int kDsSteps = kDsRows / 32;          // 32-column steps per block
constexpr int kDsStage = 2;                     // steps per transposed hand-off
constexpr int kDsStages = kDsSteps / kDsStage;  // hand-offs per block

// One thread per (delta, row, group) of row block b's stored blocks.
__global__ void k_dense_pack_half(const float* __restrict__ rows, int64_t nrows, int64_t n,
                                  int64_t b, int64_t nb, int64_t span, int shift, int vec4,
                                  h16* __restrict__ half) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (span + 1) * kDsRows * kDsGroups) return;
  const int64_t delta = idx / (kDsRows * kDsGroups);
  const int64_t rem = idx - delta * (kDsRows * kDsGroups);
  const int64_t r = rem / kDsGroups, g = rem - r * kDsGroups;
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
  half[(dense_half_index(b, delta, nb) * kDsRows + r) * kDsGroups + g] = split16(x);
}

// Right-hand sides in row-tile-pair order: Vp[(u*2 + part)*64 + lane] (8
// fp16), element e = 2^s_c V[c = lane%16][32 u + 16 (e/4) + 4 (lane/16) + e%4],
// part 0 = hi, 1 = lo; zero for c >= ncols or past n.
__global__ void k_dense_pack_pair(const float* __restrict__ V, int64_t n, int ncols,
                                  int64_t pairs, const uint32_t* __restrict__ colmax,
                                  h8* __restrict__ Vp) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs * 64) return;
  const int lane = (int)(idx & 63);
  const int64_t u = idx >> 6;
  const int c = lane & 15;
  const int sh = c < ncols ? scale_shift(__uint_as_float(colmax[c])) : 0;
  h8 hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t j = 32 * u + 16 * (e >> 2) + 4 * (lane >> 4) + (e & 3);
    const float v = (c < ncols && j < n) ? ldexpf(V[(int64_t)c * n + j], sh) : 0.0f;
    hi[e] = (_Float16)v;
    lo[e] = (_Float16)(v - (float)hi[e]);
  }
  Vp[(u * 2) * 64 + lane] = hi;
  Vp[(u * 2 + 1) * 64 + lane] = lo;
}

// Work item L = (row block b, delta split) of the symmetric half product.
// fwd[(split*16 + c)*mpad + i]: forward sums of the split's blocks, unscaled;
// tp[((b*hmax + delta - 1)*256 + column)*16 + c]: transposed block sums.
__global__ __launch_bounds__(64 * kDsWaves) void k_dense_sym(
    const h16* __restrict__ Kh, const h16* __restrict__ Vn, const h8* __restrict__ Vpp,
    int64_t nb, int64_t splits, int64_t dps, int64_t hmax, int64_t gpr, int ncols, int kshift,
    const uint32_t* __restrict__ colmax, float* __restrict__ fwd, float* __restrict__ tp,
    int64_t mpad) {
  constexpr int W = kDsWaves;
  // Wave-private transposition scratch: [column tile][hi, lo][row tile][chunk].
  __shared__ uint64_t tsc[W][2][2][2][64];
  // Transposed sums per hand-off: [buffer][step][wave][column tile][lane].
  __shared__ f4 tbuf[2][kDsStage][W][2][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t per = (int64_t)gridDim.x / kXcds;
  const int64_t L = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (L >= nb * splits) return;  // whole workgroup, before any barrier
  const int64_t b = L % nb;
  const int64_t split = L / nb;
  const int li = lane & 15, lg = lane >> 4;
  const int row0 = 32 * wave;  // this wave's rows within the block
  const int64_t upr = (b * kDsRows + row0) / 32;
  const h8 vih = Vpp[(upr * 2) * 64 + lane], vil = Vpp[(upr * 2 + 1) * 64 + lane];
  const int chunk_r = sym_read_chunk(lane);
  const int tw = lg >> 1, q0 = 2 * (lg & 1);  // column tile and first quad of this lane's group

  f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
  double accd[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) accd[r][q] = 0.0;

  const int64_t span = sym_span(b, nb);
  const int64_t d0 = split * dps;
  const int64_t d1 = min(d0 + dps, span + 1);
  const int64_t nsteps = d1 > d0 ? (d1 - d0) * kDsSteps : 0;
  const int64_t nst = nsteps / kDsStage;
  auto step_delta = [&](int64_t t) { return d0 + t / kDsSteps; };
  // Loads of step t: the wave's two row tiles of the block (lane: row
  // 16 r + li, group 4 s + lg) and V_J (lane: column li, same group).
  auto load = [&](int64_t t, h16 (&ka)[2], h16& va) __attribute__((always_inline)) {
    const int64_t delta = step_delta(t);
    const int s = (int)(t % kDsSteps);
    int64_t J = b + delta;
    if (J >= nb) J -= nb;
    const h16* kp = Kh + (dense_half_index(b, delta, nb) * kDsRows + row0) * kDsGroups + 4 * s + lg;
    ka[0] = kp[(int64_t)li * kDsGroups];
    ka[1] = kp[(int64_t)(16 + li) * kDsGroups];
    va = Vn[(int64_t)li * gpr + J * kDsGroups + 4 * s + lg];
  };
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int q = 0; q < 4; ++q) accd[r][q] += (double)acc[r][q];
      acc[r] = f4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // Stage reduction (all 512 threads): unit u < kDsStage*256 is two
  // right-hand sides (2h, 2h + 1 of the lane's four) of one lane of one
  // column tile; a thread's units share the lane half, so its scales are fixed.
  constexpr int kRedUnits = kDsStage * 256;
  const int ru = threadIdx.x;
  const int r_ln = (ru >> 1) & 63, r_h = ru & 1;
  const int r_c = 4 * (r_ln >> 4) + 2 * r_h;
  f2 r_scale;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int cc = r_c + e;
    const int sh = cc < ncols ? scale_shift(__uint_as_float(colmax[cc])) : 0;
    r_scale[e] = ldexpf(1.0f, -(kshift + sh));
  }
  auto reduce_stage = [&](int64_t c) __attribute__((always_inline)) {
    const int slot = (int)(c & 1);
    const int64_t blk = b * hmax + step_delta(c * kDsStage) - 1;
    constexpr int wstride = (int)(sizeof(tbuf[0][0][0]) / sizeof(float));
#pragma unroll
    for (int uu = 0; uu < kRedUnits; uu += 64 * W) {
      const int u = uu + ru;
      if (u >= kRedUnits) break;
      const int kk = u >> 8, t = (u >> 7) & 1;
      const float* src = reinterpret_cast<const float*>(&tbuf[slot][kk][0][t][r_ln]) + 2 * r_h;
      f2 sum = *reinterpret_cast<const f2*>(src);
#pragma unroll
      for (int w = 1; w < W; ++w) sum += *reinterpret_cast<const f2*>(src + w * wstride);
      const int64_t s = (c * kDsStage) % kDsSteps + kk;
      const int64_t jl = 32 * s + 16 * t + (r_ln & 15);
      *reinterpret_cast<f2*>(tp + (blk * kDsRows + jl) * 16 + r_c) = sum * r_scale;
    }
  };

  h16 ka[2], va, kn[2], vn;
  if (nsteps > 0) load(0, ka, va);
  for (int64_t c = 0; c < nst; ++c) {
    __syncthreads();
    if (c > 0 && step_delta((c - 1) * kDsStage) > 0) reduce_stage(c - 1);
    const bool sym = step_delta(c * kDsStage) > 0;
#pragma unroll
    for (int k = 0; k < kDsStage; ++k) {
      const int64_t t = c * kDsStage + k;
      load(min(t + 1, nsteps - 1), kn, vn);  // next step (clamped: always a valid block)
      const h8 vh = first8(va), vl = last8(va);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const h8 kh = first8(ka[r]), kl = last8(ka[r]);
        f4 a = acc[r];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, vh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, vl, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, vh, a, 0, 0, 0);
        acc[r] = a;
      }
      if (sym) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const u64x2 h = __builtin_bit_cast(u64x2, first8(ka[r]));
          const u64x2 l = __builtin_bit_cast(u64x2, last8(ka[r]));
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
          f4 a = f4{0.f, 0.f, 0.f, 0.f};
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vih, tp2[0], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vil, tp2[0], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vih, tp2[1], a, 0, 0, 0);
          tbuf[c & 1][k][wave][tt][lane] = a;
        }
        asm volatile("" ::: "memory");
      }
      ka[0] = kn[0];
      ka[1] = kn[1];
      va = vn;
    }
    if ((c + 1) % kDsStages == 0) flush();  // end of a block
  }
  if (nst > 0 && step_delta((nst - 1) * kDsStage) > 0) {
    __syncthreads();
    reduce_stage(nst - 1);
  }
  flush();
  // Forward partials (lane: column li, rows 16 r + 4 lg + q of the wave).
  const int sh = li < ncols ? scale_shift(__uint_as_float(colmax[li])) : 0;
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t i = b * kDsRows + row0 + 16 * r + 4 * lg + q;
      fwd[(split * 16 + li) * mpad + i] = (float)ldexp(accd[r][q], -(kshift + sh));
    }
}

// out[c*n + j] = sum_s fwd[s][c][j] + the transposed partials of the row
// blocks that formed j's column block (delta order) + noise V; four threads
// per point, four right-hand sides each, fp64 sums.
__global__ __launch_bounds__(256) void k_dense_sym_reduce(
    const float* __restrict__ fwd, int splits, const float* __restrict__ tp, int64_t nb,
    int64_t hmax, int64_t mpad, int64_t n, int ncols, float noise,
    const float* __restrict__ V, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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
                     reinterpret_cast<h16*>(K.half.ptr));
  MGP_HIP_CHECK(hipGetLastError());
}

void dense_sym_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                       DenseWorkspace& w, hipStream_t st) {
  MGP_REQUIRE(ncols >= 1 && ncols <= 16, "the symmetric dense product takes 1..16 columns");
  MGP_REQUIRE(K.half_valid, "the symmetric half of K is not filled");
  const int64_t n = K.n, npad = K.npad, gpr = K.groups_per_row(), nb = K.blocks();
  const int64_t hmax = nb / 2;
  const int chunks = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(n, 4096)));
  uint32_t* cpart = w.colmax_part.ensure((size_t)chunks * ncols);
  uint32_t* colmax = w.colmax.ensure((size_t)ncols);
  hipLaunchKernelGGL(k_dense_absmax_part, dim3((unsigned)chunks, (unsigned)ncols), dim3(256), 0,
                     st, V, n, cpart);
  hipLaunchKernelGGL(k_dense_absmax_final, dim3((unsigned)ncols), dim3(64), 0, st, cpart, chunks,
                     colmax);
  const int64_t vtot = 16 * gpr;
  h16* vn = reinterpret_cast<h16*>(w.vpack.ensure((size_t)vtot * 8));
  const int vec4 = (n % 4 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack_rhs_groups, dim3((unsigned)ceil_div(vtot, 256)), dim3(256), 0,
                     st, V, n, ncols, 16, gpr, colmax, vec4, vn);
  const int64_t pairs = npad / 32;
  h8* vp = reinterpret_cast<h8*>(w.vpair.ensure((size_t)pairs * 2 * 64 * 4));
  hipLaunchKernelGGL(k_dense_pack_pair, dim3((unsigned)ceil_div(pairs * 64, 256)), dim3(256), 0,
                     st, V, n, ncols, pairs, colmax, vp);
  MGP_HIP_CHECK(hipGetLastError());

  int64_t splits = std::min<int64_t>(std::max<int64_t>(ceil_div(2048, nb), 1), hmax + 1);
  const int64_t dps = ceil_div(hmax + 1, splits);
  splits = ceil_div(hmax + 1, dps);
  float* fwd = w.part.ensure((size_t)splits * 16 * npad);
  float* tp = w.tpart.ensure((size_t)std::max<int64_t>(nb * hmax, 1) * kDsRows * 16);
  const int64_t items = round_up(nb * splits, kXcds);
  hipLaunchKernelGGL(k_dense_sym, dim3((unsigned)items), dim3(64 * kDsWaves), 0, st,
                     reinterpret_cast<const h16*>(K.half.ptr), vn, vp, nb, splits, dps, hmax, gpr,
                     ncols, K.shift, colmax, fwd, tp, npad);
  MGP_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_dense_sym_reduce, dim3((unsigned)ceil_div(4 * n, 256)), dim3(256), 0, st,
                     fwd, (int)splits, tp, nb, hmax, npad, n, ncols, noise, V, out);
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
