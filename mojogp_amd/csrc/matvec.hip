// Fused kernel-matrix x right-hand-side products for gfx950.
//
// Reference behaviour (caspbian/mojogp):
//   fused_forward_matvec_ncols  mojogp/codegen_engine/emit/gpu_kernel.py:151-260
//   fused_cross_matvec_ncols    mojogp/codegen_engine/emit/gpu_kernel.py:487-565
//   kernel arithmetic + guards  mojogp/codegen_engine/expressions.py:77-240,
//                               mojogp/codegen_engine/passes/numerical_stability.py:1-112
//
// Design (not a translation): the product out = K V is evaluated like an
// attention block.  Per 16x16 tile of (row i, column j) pairs:
//   1. S^T = A_j . B_i   (v_mfma_f32_16x16x32_f16 over the two-term fp16
//      split of the augmented coordinates, see PackedPoints) yields the scaled
//      squared distance |z_i - z_j|^2 at fp32 accuracy (Gram form, norms in two
//      extra dimensions); 2 MFMAs at d = 16;
//   2. the kernel value is formed in registers (RBF: med3 + exp2;
//      Matern-5/2: sqrt, min, exp2, two FMAs, one multiply);
//   3. O^T += V^T . P^T  (four more 16x16x4 MFMAs per 16 right-hand sides).
// K never touches HBM.  Accumulators are flushed into fp64 every 256 columns
// (512 in the symmetric kernel) so the long N-term sums keep ~1e-7 relative
// accuracy.
#include "dense.h"
#include "matvec.h"
#include "sym_common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

namespace mgp {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void g_void;

namespace {

constexpr int kWaves = 4;           // waves per workgroup
constexpr int kStageSteps = 2;      // column-tile pairs per LDS stage of the tile kernel
constexpr int kFlushTiles = 16;     // j tiles between fp64 flushes
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left free (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int kWaitVmcnt0 = 0x0F70;
constexpr float kM52A = 0.69314718055994530942f;                     // ln 2
constexpr float kM52B = 0.69314718055994530942f * 0.69314718055994530942f / 3.0f;

// kExp2Clamp held in a VGPR (hoisted out of the hot loop by the caller).
__device__ __forceinline__ float clamp_reg() {
  float c = kExp2Clamp;
  asm volatile("" : "+v"(c));
  return c;
}

// Kernel value from the scaled squared distance s (see kernel_scale()).
// clampv = the exponent limit exp2_limit(kind, ard) (kExp2Clamp, from
// clamp_reg() in hot loops, for the Matern-3/2 and 5/2 kernels; the point
// set's exp2_limit for Matern-1/2; RBF has none).
template <int KIND>
__device__ __forceinline__ float kval(float s, float clampv = kExp2Clamp) {
  if constexpr (KIND == KIND_RBF) {
    // os * exp(-0.5 r^2) = os * 2^-max(s, 0) (the max only absorbs Gram-form
    // rounding below zero; the reference does not clamp the RBF exponent)
    return __builtin_amdgcn_exp2f(-fmaxf(s, 0.0f));
  } else if constexpr (KIND == KIND_MATERN12) {
    // os * exp(-r) (isotropic) or os * exp(max(-r, -20)) (ARD),  u = r log2 e
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    return __builtin_amdgcn_exp2f(-fminf(u, clampv));
  } else if constexpr (KIND == KIND_MATERN32) {
    // os * (1 + sqrt3 r) * exp(max(-sqrt3 r, -20)),  u = sqrt3 r log2 e
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    return fmaf(u, kLn2, 1.0f) * __builtin_amdgcn_exp2f(-fminf(u, clampv));
  } else {
    // os * (1 + sqrt5 r + 5/3 r^2) * exp(max(-sqrt5 r, -20)),  u = sqrt5 r log2 e
    // sqrt(|s|): s < 0 only from Gram-form rounding of a near-zero distance,
    // where |s| and max(s, 0) agree to the rounding error (dk/du = 0 at u = 0);
    // the abs is a free source modifier of v_sqrt_f32.
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    // min(u, C) kept opaque so that the negation is not rewritten into
    // max(-u, -C) + v_xor but lands on v_exp_f32 as a source modifier.
    float m = fminf(u, clampv);
    asm("" : "+v"(m));
    const float e = __builtin_amdgcn_exp2f(-m);
    const float p = fmaf(u, fmaf(u, kM52B, kM52A), 1.0f);
    return p * e;
  }
}

// ---------------------------------------------------------------------------
// Packing
// ---------------------------------------------------------------------------
__global__ void k_fill_u32(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Two-term fp16 split of an fp32 value: hi = RNE16(x), lo = RNE16(x - hi).
// Returns the requested part's bits.
__device__ __forceinline__ uint16_t f16_part(float x, int part) {
  const _Float16 hi = (_Float16)x;
  const _Float16 v = part == 0 ? hi : (_Float16)(x - (float)hi);
  return __builtin_bit_cast(uint16_t, v);
}

// Part-product table: slot product p multiplies A part kPartA[p] with B part
// kPartB[p] (hi = 0, lo = 1).
__constant__ int kPartA[3] = {0, 0, 1};
__constant__ int kPartB[3] = {0, 1, 0};

// One thread per (padded) point: scaled coordinates, norm, and the 32*kb fp16
// slots of both operand sides.
__global__ void k_pack_points(const float* __restrict__ X, int64_t n, int d,
                              const float* __restrict__ coef, int kb,
                              int64_t ntiles, uint16_t* __restrict__ A,
                              uint16_t* __restrict__ B, float* __restrict__ Z,
                              uint32_t* __restrict__ max_norm) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = i < ntiles * 16;  // no early return: the wave reduces below
  const int li = (int)(i & 15);
  const int64_t tile = i >> 4;
  const bool real = i < n;
  auto zval = [&](int k) -> float {
    return real ? (X[i * d + k] - coef[k]) * coef[d + k] : 0.0f;
  };
  float nrm = 0.0f;
  for (int k = 0; k < d; ++k) {
    const float z = zval(k);
    if (real) Z[i * d + k] = z;
    nrm = fmaf(z, z, nrm);
  }
  // Wave max of the norms (non-negative floats order as unsigned integers).
  uint32_t mx = __float_as_uint(nrm);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if ((threadIdx.x & 63) == 0) atomicMax(max_norm, mx);
  if (!active) return;
  const int D = d + 2;
  for (int k = 0; k < 32 * kb; ++k) {
    uint16_t a = 0, b = 0;
    if (k < 3 * D) {
      const int p = k / D, t = k - p * D;
      float av, bv;
      if (t < d) {
        const float z = zval(t);
        av = z;
        bv = -2.0f * z;
      } else if (t == d) {
        av = nrm;
        bv = 1.0f;
      } else {
        av = 1.0f;
        bv = nrm;
      }
      a = f16_part(av, kPartA[p]);
      b = f16_part(bv, kPartB[p]);
    }
    const int m = k >> 5, g = (k >> 3) & 3, e = k & 7;
    const int64_t off = ((tile * kb + m) * 64 + li + 16 * g) * 8 + e;
    A[off] = a;
    B[off] = b;
  }
}

// ---------------------------------------------------------------------------
// Right-hand sides for the fp16 product O^T += V^T P^T
//
// P is formed as P' = 2^kPScaleLog2 * k / os <= 2^15.  Where the kernel's
// exponent is clamped (Matern-3/2 and 5/2: k/os >= e^-20) P' >= 2^-13.9 is a
// normal fp16 number and its two-term split P' = Ph + Pl (both
// round-to-nearest fp16) carries 22+ significant bits.  The RBF exponent is
// not clamped: values with P' below 2^-14 (k/os < 2^-29) lose relative
// precision in the subnormal range, but their absolute error stays below
// 2^-25 in P', i.e. 2^-40 os per pair.
// Each column of V is scaled by 2^shift_c so max|V'_c| lies in [2^14, 2^15) and
// split the same way.  Ph.Vh + Ph.Vl + Pl.Vh then reproduces P.V to ~2^-23
// relative; the dropped Pl.Vl term is below 2^-24.  The result is unscaled
// exactly by 2^-(shift_c + kPScaleLog2).
// ---------------------------------------------------------------------------
constexpr int kPScaleLog2 = 15;

__device__ __forceinline__ int col_shift(uint32_t maxbits) {
  const float mx = __uint_as_float(maxbits);
  if (!(mx > 0.0f) || mx > 3.0e38f) return 0;  // zero or non-finite column
  int e;
  (void)frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
  return 15 - e;
}

// part[c*chunks + b] = max |V[c*n + j]| over the contiguous row chunk b, as
// float bits (non-negative floats order as unsigned integers).  grid =
// (chunks, ncols); no atomics, so no same-address serialisation.  Chunks are
// a multiple of 4 rows; vec4 (n a multiple of 4) reads 16 bytes per lane.
__global__ __launch_bounds__(256) void k_col_absmax_part(const float* __restrict__ V, int64_t n,
                                                         int vec4, uint32_t* __restrict__ part) {
  __shared__ uint32_t wm[4];
  const int c = blockIdx.y;
  const int chunks = gridDim.x;
  const int64_t len = (((n + chunks - 1) / chunks) + 3) & ~(int64_t)3;
  const int64_t j0 = min(n, (int64_t)blockIdx.x * len), j1 = min(n, j0 + len);
  const float* col = V + (int64_t)c * n;
  uint32_t mx = 0;
  if (vec4) {
#pragma unroll 4
    for (int64_t j = j0 + 4 * threadIdx.x; j < j1; j += 4 * blockDim.x) {
      const f4 x = *reinterpret_cast<const f4*>(col + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) mx = max(mx, __float_as_uint(fabsf(x[e])));
    }
  } else {
    for (int64_t j = j0 + threadIdx.x; j < j1; j += blockDim.x)
      mx = max(mx, __float_as_uint(fabsf(col[j])));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0)
    part[(int64_t)c * chunks + blockIdx.x] = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
}

// colmax[c] = max_b part[c*chunks + b] (chunks <= 64): one wave per column.
__global__ void k_col_absmax_final(const uint32_t* __restrict__ part, int chunks,
                                   uint32_t* __restrict__ colmax) {
  const int c = blockIdx.x, lane = threadIdx.x;
  uint32_t mx = lane < chunks ? part[(int64_t)c * chunks + lane] : 0u;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if (lane == 0) colmax[c] = mx;
}

// Vp[((g*upairs + u)*2 + part)*64 + lane] (8 fp16): element e holds
// V'[c = 16g + lane%16][j = 16 (2u + e/4) + 4 (lane/16) + e%4], part 0 = hi,
// part 1 = lo.  One thread per (g, u, lane).
__global__ void k_pack_rhs16(const float* __restrict__ V, int64_t n, int ncols,
                             int ncg, int64_t upairs, const uint32_t* __restrict__ colmax,
                             int vec4, h8* __restrict__ P) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)ncg * upairs * 64) return;
  const int lane = (int)(idx & 63);
  const int64_t u = (idx >> 6) % upairs;
  const int g = (int)((idx >> 6) / upairs);
  const int c = 16 * g + (lane & 15);
  h8 hi, lo;
  const int shift = c < ncols ? col_shift(colmax[c]) : 0;
  // rows j0 .. j0 + 3 (e < 4) and j0 + 16 .. j0 + 19 (e >= 4)
  const int64_t j0 = 32 * u + 4 * (lane >> 4);
  float x[8];
  if (vec4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t j = j0 + 16 * h;
      const f4 q = (c < ncols && j < n) ? *reinterpret_cast<const f4*>(V + (int64_t)c * n + j)
                                        : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * h + e] = q[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t j = j0 + 16 * (e >> 2) + (e & 3);
      x[e] = (c < ncols && j < n) ? V[(int64_t)c * n + j] : 0.0f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = ldexpf(x[e], shift);
    hi[e] = (_Float16)v;
    lo[e] = (_Float16)(v - (float)hi[e]);
  }
  const int64_t base = ((int64_t)g * upairs + u) * 2;
  P[base * 64 + lane] = hi;
  P[(base + 1) * 64 + lane] = lo;
}

// Single right-hand side: zero padded copy.
__global__ void k_pad_vec(const float* __restrict__ V, int64_t n, int64_t npad,
                          float* __restrict__ P) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < npad) P[j] = j < n ? V[j] : 0.0f;
}

// 2^kPScaleLog2 * k / os from the scaled squared distance s, returned as a
// product f * g (Matern-5/2: polynomial times exponential; RBF: g = 1) so the
// fp16 split can round the exact product (see split_pair).
template <int KIND>
__device__ __forceinline__ void kval_scaled(float s, float clampv, float one, float& f,
                                            float& g) {
  constexpr float P = (float)(1 << kPScaleLog2);
  if constexpr (KIND == KIND_RBF) {
    (void)clampv;  // the RBF exponent is not clamped
    // max(s, 0) as v_med3_f32, which takes the MFMA result as it is; fmaxf
    // would first canonicalize it (IEEE mode), one more VALU instruction per
    // value.  Same value for every finite s.
    const float t = __builtin_amdgcn_fmed3f(s, 0.0f, 3.0e38f);
    f = __builtin_amdgcn_exp2f((float)kPScaleLog2 - t);
    g = one;
  } else if constexpr (KIND == KIND_MATERN32) {
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    float mn = fminf(u, clampv);
    asm("" : "+v"(mn));
    g = __builtin_amdgcn_exp2f(-mn);
    f = fmaf(u, kLn2 * P, P);
  } else {
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    float mn = fminf(u, clampv);
    asm("" : "+v"(mn));
    g = __builtin_amdgcn_exp2f(-mn);
    f = fmaf(u, fmaf(u, kM52B * P, kM52A * P), P);
  }
}

// Two-term fp16 split of x0 = f0 g0 and x1 = f1 g1 into packed pairs:
// hi = RNE16(fl(f g)) (v_cvt_pk_f16_f32), lo = RNE16(f g - hi) from the exact
// fma inside v_fma_mix{lo,hi}_f16 reading hi's halves via op_sel.  Plain C so
// the compiler schedules these and tracks their VALU->MFMA hazards.  For the
// RBF path g is an opaque register 1.0 (keeps the residual an fma).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
template <bool UNIT_G>
__device__ __forceinline__ void split_pair(float f0, float g0, float f1, float g1,
                                           h2& hi, h2& lo) {
  if constexpr (UNIT_G)
    hi = __builtin_convertvector((f2){f0, f1}, h2);
  else
    hi = __builtin_convertvector((f2){f0 * g0, f1 * g1}, h2);
  lo[0] = (_Float16)__builtin_fmaf(f0, g0, -(float)hi[0]);
  lo[1] = (_Float16)__builtin_fmaf(f1, g1, -(float)hi[1]);
}

// ---------------------------------------------------------------------------
// MFMA tile kernel
//   NCG > 0 : NCG groups of 16 right-hand sides, fp16 split products on MFMA
//   NCG == 0: one right-hand side accumulated on VALU (fp32)
//   R       : 16-row tiles per wave (even)
// The j loop walks pairs of column tiles (2u, 2u+1): one K=32 fp16 MFMA covers
// the 32 columns of a pair.  grid = (row blocks, splits); block y covers pairs
// [y*pairs_per_split, ...).  If `partial` is set, unscaled-by-os sums are
// written to partial[(split*cpad + c)*mpad + i]; otherwise the epilogue applies
// os and the noise diagonal and writes out[c*m + i].
// ---------------------------------------------------------------------------
template <int KIND, int KB, int NCG, int R>
__global__ __launch_bounds__(256) void k_fused_tile(
    const h8* __restrict__ Bi, int64_t row_tiles, const h8* __restrict__ Aj,
    const void* __restrict__ Vp, int64_t col_pairs, int64_t pairs_per_split,
    int64_t diag_shift, int64_t m, int ncols, float os, float noise,
    const uint32_t* __restrict__ colmax, const float* __restrict__ Vin,
    float* __restrict__ out, float* __restrict__ partial, int64_t mpad, int cpad) {
  static_assert(R % 2 == 0, "row tiles per wave must be even (pair alignment)");
  static_assert(KIND != KIND_MATERN12, "Matern-1/2 is evaluated from coordinate differences");
  // LDS stages: kStageSteps column-tile pairs each, as 1-KB blocks (64 lanes x
  // 16 B, the MFMA operand layout): per step 2 KB blocks of A (tiles 2u, 2u+1),
  // then per right-hand-side group 2 blocks of V (hi, lo) after all A blocks.
  constexpr int kA = 2 * KB;
  constexpr int kV = NCG > 0 ? 2 * NCG : 0;
  constexpr int kBlocks = kStageSteps * (kA + kV);
  __shared__ h8 lds[2][kBlocks][64];

  const int lane = threadIdx.x & 63;
  // Wave index made wave-uniform (SGPR) so loop bounds and LDS bases stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t tile0 = ((int64_t)blockIdx.x * kWaves + wave) * R;
  // Waves without rows still fill LDS stages and meet every barrier.
  const bool active = tile0 < row_tiles;

  h8 bi[R][KB];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t it = tile0 + r;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (it < row_tiles) {
        bi[r][kb] = Bi[(it * KB + kb) * 64 + lane];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) bi[r][kb][e] = (_Float16)0.0f;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // row operands before the loop (see k_sym_tile)

  constexpr int G = NCG > 0 ? NCG : 1;
  f4 acc[R][G];
  double accd[R][G][4];
  float acc1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc1[r] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      acc[r][g] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) accd[r][g][q] = 0.0;
    }
  }

  const float clampv = clamp_reg();
  float one = 1.0f;
  asm volatile("" : "+v"(one));

  // Lane holds S^T[j = 4(lane/16)+q][i = lane%16] of a 16x16 tile.
  const int li = lane & 15;
  const int lj = 4 * (lane >> 4);
  const h8* V16 = reinterpret_cast<const h8*>(Vp);
  const float* V32 = reinterpret_cast<const float*>(Vp);

  // Stage fill: steps [u0, u0 + ns) of A and V into lds[st] by LDS DMA, the
  // blocks dealt round-robin to the four waves.  Both ranges are contiguous in
  // global memory (A blocks 2 u0 KB .., V blocks (g col_pairs + u0) 2 ..).
  auto fill = [&](int st, int64_t u0, int ns) __attribute__((always_inline)) {
    const int na = ns * kA;
    for (int b = wave; b < na; b += kWaves)
      __builtin_amdgcn_global_load_lds(
          (const g_void*)(Aj + (2 * u0 * KB + b) * 64 + lane), (lds_void*)&lds[st][b][0], 16, 0,
          0);
    if constexpr (NCG > 0) {
      const int nv = 2 * ns;
      for (int b = wave; b < NCG * nv; b += kWaves) {
        const int g = b / nv, k = b - g * nv;
        __builtin_amdgcn_global_load_lds(
            (const g_void*)(V16 + (((int64_t)g * col_pairs + u0) * 2 + k) * 64 + lane),
            (lds_void*)&lds[st][kStageSteps * kA + g * 2 * kStageSteps + k][0], 16, 0, 0);
      }
    }
  };

  // One pair of j tiles (step k of stage st) against the wave's R row tiles.
  // MASK restores the exact zero self-distance on diagonal tiles (Gram-form
  // cancellation guard).
  auto step = [&](int st, int k, int64_t u, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int64_t jt0 = 2 * u;
    h8 a0[KB], a1[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      a0[kb] = lds[st][k * kA + kb][lane];
      a1[kb] = lds[st][k * kA + KB + kb][lane];
    }
    h8 vh[G], vl[G];
    f4 v0, v1;
    if constexpr (NCG > 0) {
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        vh[g] = lds[st][kStageSteps * kA + g * 2 * kStageSteps + 2 * k][lane];
        vl[g] = lds[st][kStageSteps * kA + g * 2 * kStageSteps + 2 * k + 1][lane];
      }
    } else {
      v0 = *reinterpret_cast<const f4*>(V32 + 16 * jt0 + lj);
      v1 = *reinterpret_cast<const f4*>(V32 + 16 * jt0 + 16 + lj);
    }
    // Software pipeline over the wave's row tiles: stage r issues the
    // distance MFMAs of row r + 1 and the product MFMAs of row r - 1 while
    // the VALU forms row r's kernel values, so the matrix cores and the VALU
    // work side by side within the wave.
    auto dist = [&](int r, f4& s0, f4& s1) __attribute__((always_inline)) {
      s0 = f4{0.f, 0.f, 0.f, 0.f};
      s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[kb], bi[r][kb], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[kb], bi[r][kb], s1, 0, 0, 0);
      }
    };
    auto product = [&](int r, const h8& ph, const h8& pl) __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        f4 a = acc[r][g];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[g], ph, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl[g], ph, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[g], pl, a, 0, 0, 0);
        acc[r][g] = a;
      }
    };
    f4 S0[2], S1[2];
    h8 PH[2], PL[2];
    dist(0, S0[0], S1[0]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f4 s0 = S0[r & 1], s1 = S1[r & 1];
      if (r + 1 < R) dist(r + 1, S0[(r + 1) & 1], S1[(r + 1) & 1]);
      if constexpr (NCG > 0) {
        if (r > 0) product(r - 1, PH[(r - 1) & 1], PL[(r - 1) & 1]);
      }
      if constexpr (MASK) {
        const int64_t dt = tile0 + r + diag_shift;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (jt0 == dt && li == lj + q) s0[q] = 0.0f;
          if (jt0 + 1 == dt && li == lj + q) s1[q] = 0.0f;
        }
      }
      float f0[4], g0[4], f1[4], g1[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        kval_scaled<KIND>(s0[q], clampv, one, f0[q], g0[q]);
        kval_scaled<KIND>(s1[q], clampv, one, f1[q], g1[q]);
      }
      if constexpr (NCG > 0) {
        // B operand halves e = 0..3 from tile jt0, 4..7 from jt0 + 1.
        h2 hA, hB, hC, hD, lA, lB, lC, lD;
        split_pair<KIND != KIND_MATERN52 && KIND != KIND_MATERN32>(f0[0], g0[0], f0[1], g0[1], hA, lA);
        split_pair<KIND != KIND_MATERN52 && KIND != KIND_MATERN32>(f0[2], g0[2], f0[3], g0[3], hB, lB);
        split_pair<KIND != KIND_MATERN52 && KIND != KIND_MATERN32>(f1[0], g1[0], f1[1], g1[1], hC, lC);
        split_pair<KIND != KIND_MATERN52 && KIND != KIND_MATERN32>(f1[2], g1[2], f1[3], g1[3], hD, lD);
        PH[r & 1] = h8{hA[0], hA[1], hB[0], hB[1], hC[0], hC[1], hD[0], hD[1]};
        PL[r & 1] = h8{lA[0], lA[1], lB[0], lB[1], lC[0], lC[1], lD[0], lD[1]};
      } else {
        float a = acc1[r];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a = fmaf(f0[q] * g0[q], v0[q], a);
          a = fmaf(f1[q] * g1[q], v1[q], a);
        }
        acc1[r] = a;
      }
    }
    if constexpr (NCG > 0) product(R - 1, PH[(R - 1) & 1], PL[(R - 1) & 1]);
#ifdef MGP_TILE_SCHED
    // Interleave: one MFMA, then VALU, through the step.
#pragma unroll
    for (int i = 0; i < R * (2 * KB + 3 * NCG); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, MGP_TILE_SCHED, 0);
    }
#endif
  };
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (NCG > 0) {
#pragma unroll
        for (int g = 0; g < NCG; ++g) {
#pragma unroll
          for (int q = 0; q < 4; ++q) accd[r][g][q] += (double)acc[r][g][q];
          acc[r][g] = f4{0.f, 0.f, 0.f, 0.f};
        }
      } else {
        accd[r][0][0] += (double)acc1[r];
        acc1[r] = 0.0f;
      }
    }
  };

  // Walk the split's pairs stage by stage: while stage c is consumed, stage
  // c + 1 streams into the other buffer.  The barrier at the top of each
  // stage makes stage c visible to all waves and frees the buffer of c - 1.
  const int64_t u_begin = (int64_t)blockIdx.y * pairs_per_split;
  const int64_t u_end = min(col_pairs, u_begin + pairs_per_split);
  const int64_t dlo = (tile0 + diag_shift) / 2, dhi = dlo + R / 2;
  const int64_t npairs = max((int64_t)0, u_end - u_begin);
  const int64_t nfull = npairs / kStageSteps;  // full stages; a last partial one follows
  const int64_t nstages = (npairs + kStageSteps - 1) / kStageSteps;
  fill(0, u_begin, (int)min((int64_t)kStageSteps, npairs));
  auto stage_top = [&](int64_t c) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (c + 1 < nstages) {
      const int64_t u1 = u_begin + (c + 1) * kStageSteps;
      fill((int)((c + 1) & 1), u1, (int)min((int64_t)kStageSteps, u_end - u1));
    }
  };
  if (!active) {
    for (int64_t c = 0; c < nstages; ++c) stage_top(c);
    return;
  }
  // The stage loops below hold no branch that merges accumulator values: the
  // full stages without a diagonal pair of this wave run as straight code,
  // the fp64 flush (every kFlushStages full stages, 256 columns) closes a
  // group of them, and the stages holding a diagonal pair and the last
  // partial stage are peeled off.  As one loop with those branches inside,
  // every stage copied the accumulators (48 v_mov_b64 with 64 right-hand
  // sides).  Flush points and summation order are those of a per-stage
  // column count.
  constexpr int kFlushStages = kFlushTiles / (2 * kStageSteps);
  auto plain_stage = [&](int64_t c) __attribute__((always_inline)) {
    const int st = (int)(c & 1);
    const int64_t u0 = u_begin + c * kStageSteps;
#pragma unroll
    for (int k = 0; k < kStageSteps; ++k) step(st, k, u0 + k, std::false_type{});
  };
  auto checked_stage = [&](int64_t c, int ns) __attribute__((always_inline)) {
    const int st = (int)(c & 1);
    const int64_t u0 = u_begin + c * kStageSteps;
    auto one = [&](int k) __attribute__((always_inline)) {
      const int64_t u = u0 + k;
      if (u >= dlo && u < dhi)
        step(st, k, u, std::true_type{});
      else
        step(st, k, u, std::false_type{});
    };
    if (ns == kStageSteps) {
#pragma unroll
      for (int k = 0; k < kStageSteps; ++k) one(k);
    } else {
      for (int k = 0; k < ns; ++k) one(k);
    }
  };
  auto run_plain = [&](int64_t c0, int64_t c1) __attribute__((always_inline)) {
    for (int64_t g = c0; g < c1;) {
      const int64_t ge = min(c1, (g / kFlushStages + 1) * kFlushStages);
      for (int64_t c = g; c < ge; ++c) {
        stage_top(c);
        plain_stage(c);
      }
      if (ge % kFlushStages == 0) flush();
      g = ge;
    }
  };
  // Full stages [cd0, cd1) hold the wave's diagonal pairs [dlo, dhi).
  int64_t cd0 = 0, cd1 = 0;
  if (dlo < u_end && dhi > u_begin) {
    cd0 = min(nfull, (max(dlo, u_begin) - u_begin) / kStageSteps);
    cd1 = min(nfull, (min(dhi, u_end) - 1 - u_begin) / kStageSteps + 1);
  }
  run_plain(0, cd0);
  for (int64_t c = cd0; c < cd1; ++c) {
    stage_top(c);
    checked_stage(c, kStageSteps);
    if (c % kFlushStages == kFlushStages - 1) flush();
  }
  run_plain(cd1, nfull);
  if (nstages > nfull) {
    stage_top(nfull);
    checked_stage(nfull, (int)(npairs - nfull * kStageSteps));
  }
  flush();

  // Epilogue: undo the fp16 scaling exactly (powers of two).
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t it = tile0 + r;
    if (it >= row_tiles) continue;
    if constexpr (NCG > 0) {
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = 16 * g + lj + q;
          const int64_t i = 16 * it + li;
          const int shift = c < ncols ? col_shift(colmax[c]) : 0;
          const double tot = ldexp(accd[r][g][q] + (double)acc[r][g][q], -(shift + kPScaleLog2));
          if (partial) {
            partial[((int64_t)blockIdx.y * cpad + c) * mpad + i] = (float)tot;
          } else if (c < ncols && i < m) {
            float o = os * (float)tot;
            if (diag_shift == 0) o = fmaf(noise, Vin[(int64_t)c * m + i], o);
            out[(int64_t)c * m + i] = o;
          }
        }
      }
    } else {
      double tot = accd[r][0][0] + (double)acc1[r];
      // rows are shared by the four lane groups (lane/16): fold them
      tot += __shfl_xor(tot, 16);
      tot += __shfl_xor(tot, 32);
      tot = ldexp(tot, -kPScaleLog2);
      const int64_t i = 16 * it + li;
      if (lane < 16) {
        if (partial) {
          partial[(int64_t)blockIdx.y * mpad + i] = (float)tot;
        } else if (i < m) {
          float o = os * (float)tot;
          if (diag_shift == 0) o = fmaf(noise, Vin[i], o);
          out[i] = o;
        }
      }
    }
  }
}

// out[c*m+i] = os * sum_s partial[(s*cpad + c)*mpad + i] (+ noise V)
__global__ void k_reduce_splits(const float* __restrict__ partial, int splits,
                                int cpad, int64_t mpad, int64_t m, int ncols,
                                float os, float noise, int add_noise,
                                const float* __restrict__ Vin,
                                float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)ncols * m) return;
  const int c = (int)(idx / m);
  const int64_t i = idx - (int64_t)c * m;
  double tot = 0.0;
  for (int s = 0; s < splits; ++s) tot += partial[((int64_t)s * cpad + c) * mpad + i];
  float o = os * (float)tot;
  if (add_noise) o = fmaf(noise, Vin[idx], o);
  out[idx] = o;
}

// k_reduce_splits for four consecutive rows per thread (m and mpad multiples
// of 4): idx4 indexes quads of out; the splits are loaded four at a time and
// added in split order, as above.
__global__ void k_reduce_splits4(const float* __restrict__ partial, int splits, int cpad,
                                 int64_t mpad, int64_t m, int ncols, float os, float noise,
                                 int add_noise, const float* __restrict__ Vin,
                                 float* __restrict__ out) {
  const int64_t q4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q4 >= (int64_t)ncols * (m / 4)) return;
  const int64_t idx = 4 * q4;
  const int c = (int)(idx / m);
  const int64_t i = idx - (int64_t)c * m;
  const float* pc = partial + (int64_t)c * mpad + i;
  const int64_t sstride = (int64_t)cpad * mpad;
  double tot[4] = {0.0, 0.0, 0.0, 0.0};
  int s = 0;
  for (; s + 4 <= splits; s += 4) {
    f4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const f4*>(pc + (s + q) * sstride);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) tot[e] += v[q][e];
  }
  for (; s < splits; ++s) {
    const f4 v = *reinterpret_cast<const f4*>(pc + s * sstride);
#pragma unroll
    for (int e = 0; e < 4; ++e) tot[e] += v[e];
  }
  f4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = os * (float)tot[e];
  if (add_noise) {
    const f4 vin = *reinterpret_cast<const f4*>(Vin + idx);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf(noise, vin[e], o[e]);
  }
  *reinterpret_cast<f4*>(out + idx) = o;
}

// ---------------------------------------------------------------------------
// Symmetric product K(X, X) V (rows and columns the same points, 1..16
// right-hand sides): every off-diagonal kernel value is formed once and used
// twice, out[i] += k_ij V[j] and out[j] += k_ij V[i], which halves the
// transcendental and VALU work that bounds the tile kernel.
//
// The points form nb blocks of kSymRows; row block b owns the diagonal block
// and the off-diagonal column blocks J = (b + delta) mod nb for
// delta = 1 .. sym_span(b, nb), so every unordered pair of blocks is formed
// exactly once and each row block carries the same work.  Workgroup (b, s)
// takes deltas [s dps, (s + 1) dps); its kSymWaves waves own 64 rows each.
// Per column-tile pair a wave forms its 4 row tiles exactly as k_fused_tile
// (distances, values, forward product into out[i]), and also:
//   * stores each row tile's fp16 values (hi and lo, both column tiles) to a
//     wave-private LDS scratch as 8-byte chunks (row i, columns 4s .. 4s + 3)
//     at chunk index 16 s + (i ^ 4 s), a swizzle under which both the
//     stores and the transposed reads below touch every bank once per 16
//     lanes;
//   * reads them back with ds_read_b64_tr_b16 (lane 16g + 4e + s fetches the
//     chunk of row 4g + e, columns 4s ..; the instruction then hands lane
//     16g + k the elements P[4g + e][k], e = 0..3): the values transposed into the B
//     operand of O_J^T += V_I^T P, contracted over the rows of a row-tile
//     pair with the same K permutation as the packed right-hand sides (so
//     V_I is the packed V of the row pair, copied once per wave into LDS);
//   * hands its transposed sums (32 columns x 16 right-hand sides over its 64
//     rows) to the workgroup through LDS; after the next barrier the
//     waves' sums are added in wave order and written to
//     tp[b][delta - 1][column][c].
// The diagonal block is formed once without the transposed half (both of its
// triangles), with the exact zero self-distance restored on diagonal tiles.
// k_sym_reduce sums, per point, the forward split partials and the transposed
// partials of every row block that formed its column block, in a fixed order.
// ---------------------------------------------------------------------------
constexpr int kSymR = 4;                            // row tiles per wave
constexpr int kSymWaves = 8;                        // waves per workgroup
constexpr int kSymRows = 16 * kSymR * kSymWaves;    // rows (and columns) per block
constexpr int kSymPairs = kSymRows / 32;            // column-tile pairs per block
constexpr int kSymSteps = 2;                        // column-tile pairs per LDS stage
constexpr int kSymStages = kSymPairs / kSymSteps;   // LDS stages per block
constexpr int kSymSchedValu = 8;                    // VALU instructions per MFMA slot
static_assert((16 * kPackTileAlign) % kSymRows == 0, "blocks must tile the packed points");

template <int KIND, int KB>
__global__ __launch_bounds__(64 * kSymWaves) void k_sym_tile(
    const h8* __restrict__ Bi, const h8* __restrict__ Aj, const h8* __restrict__ Vp,
    int64_t nb, int64_t splits, int64_t dps, int64_t hmax, int ncols,
    const uint32_t* __restrict__ colmax, float* __restrict__ fwd, float* __restrict__ tp,
    int64_t mpad) {
  constexpr int R = kSymR, W = kSymWaves;
  static_assert(R == 4, "the pipeline below is written for two row-tile pairs");
  static_assert(W % 2 == 0, "the stage reduction strides by a multiple of 128 threads");
  constexpr bool UNIT_G = KIND != KIND_MATERN52 && KIND != KIND_MATERN32;
  constexpr int kA = 2 * KB;
  constexpr int kBlocks = kSymSteps * (kA + 2);
  __shared__ h8 lds[2][kBlocks][64];
  // Wave-private value scratch: [column tile][hi, lo][row tile of the pair][chunk].
  __shared__ uint64_t tsc[W][2][2][2][64];
  // Transposed sums per stage: [buffer][step][wave][column tile][lane].
  __shared__ f4 tbuf[2][kSymSteps][W][2][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // XCD-aware order: the hardware deals consecutive workgroups to the eight
  // XCDs in turn; logical work item L = xcd * per + k (b fastest) gives each
  // XCD a run of consecutive row blocks, which read the same column blocks a
  // step apart from its L2.  Items past nb * splits leave before any barrier.
  const int64_t per = (int64_t)gridDim.x / kXcds;
  const int64_t L = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (L >= nb * splits) return;
  const int64_t b = L % nb;
  const int64_t split = L / nb;
  const int64_t tile0 = (b * W + wave) * R;

  h8 bi[R][KB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) bi[r][kb] = Bi[((tile0 + r) * KB + kb) * 64 + lane];
  // Packed right-hand sides of the wave's two row-tile pairs (A operand of the
  // transposed product), kept in LDS and read where they are used.
  __shared__ h8 vrow[W][R / 2][2][64];
#pragma unroll
  for (int w = 0; w < R / 2; ++w) {
    const int64_t upr = tile0 / 2 + w;
    vrow[wave][w][0][lane] = Vp[(upr * 2) * 64 + lane];
    vrow[wave][w][1][lane] = Vp[(upr * 2 + 1) * 64 + lane];
  }
  // Row operands in registers before the loop: otherwise the wait for them,
  // merged at the loop head with the path that skips the loop, drains the
  // next stage's operand loads at the first MFMA of every stage.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

  f4 acc[R];
  double accd[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) accd[r][q] = 0.0;
  }
  const float clampv = clamp_reg();
  float one = 1.0f;
  asm volatile("" : "+v"(one));
  const int li = lane & 15;
  const int lj = 4 * (lane >> 4);
  // Chunk this lane stores (row li, quad lane/16) and the chunk it fetches
  // for the transposed operand (row 4 (lane/16) + (lane/4)%4, quad lane%4).
  const int chunk_w = sym_chunk(li, lane >> 4);
  const int chunk_r = sym_read_chunk(lane);

  const int64_t span = sym_span(b, nb);
  const int64_t d0 = split * dps;
  const int64_t d1 = min(d0 + dps, span + 1);
  const int64_t nst = d1 > d0 ? (d1 - d0) * kSymStages : 0;
  auto stage_delta = [&](int64_t c) { return d0 + c / kSymStages; };
  auto stage_u0 = [&](int64_t c) {
    int64_t J = b + stage_delta(c);
    if (J >= nb) J -= nb;
    return J * kSymPairs + (c % kSymStages) * kSymSteps;
  };

  // Stage operands go through registers: the loads of stage c + 1 are issued
  // at the top of stage c and written to the other LDS buffer at its end, so
  // the wait for them falls after stage c's arithmetic.  (An LDS DMA fill
  // makes the compiler wait for it before the first LDS read of stage c,
  // since it cannot tell the two buffers apart.)
  // The older wave of each SIMD (waves 0 .. W/2 - 1) stages all blocks: it
  // reaches the barrier first, so its extra loads and LDS writes fill that
  // wait (15.62 -> 15.50 ms at config 3).  The younger waves issue none.
  constexpr int kFillPerWave = (kBlocks + W / 2 - 1) / (W / 2);
  h8 pre[kFillPerWave];
  // Branch-free (one load per slot, blocks past the stage clamped onto its
  // last block) so the loads stay in one basic block and no wait separates them.
  auto fetch = [&](int64_t u0) __attribute__((always_inline)) {
    if (wave >= W / 2) return;
#pragma unroll
    for (int q = 0; q < kFillPerWave; ++q) {
      const int bb = min(wave + q * (W / 2), kBlocks - 1);
      const h8* src = bb < kSymSteps * kA ? Aj + (2 * u0 * KB + bb) * 64
                                          : Vp + (u0 * 2 + (bb - kSymSteps * kA)) * 64;
      pre[q] = src[lane];
    }
  };
  auto commit = [&](int st) __attribute__((always_inline)) {
    if (wave >= W / 2) return;
#pragma unroll
    for (int q = 0; q < kFillPerWave; ++q) {
      const int bb = wave + q * (W / 2);
      if (bb < kBlocks) lds[st][bb][lane] = pre[q];
    }
  };

  // One pair of column tiles against the wave's R row tiles.  SYM adds the
  // transposed product into tbuf[slot][k][wave]; MASK restores the exact zero
  // self-distance on diagonal tiles.
  auto step = [&](int st, int k, int64_t u, int slot, auto mask_tag, auto sym_tag)
                  __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr bool SYM = decltype(sym_tag)::value;
    const int64_t jt0 = 2 * u;
    h8 a0[KB], a1[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      a0[kb] = lds[st][k * kA + kb][lane];
      a1[kb] = lds[st][k * kA + KB + kb][lane];
    }
    const h8 vh = lds[st][kSymSteps * kA + 2 * k][lane];
    const h8 vl = lds[st][kSymSteps * kA + 2 * k + 1][lane];
    auto dist = [&](int r, f4& s0, f4& s1) __attribute__((always_inline)) {
      s0 = f4{0.f, 0.f, 0.f, 0.f};
      s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[kb], bi[r][kb], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[kb], bi[r][kb], s1, 0, 0, 0);
      }
    };
    auto product = [&](int r, const h8& ph, const h8& pl) __attribute__((always_inline)) {
      f4 a = acc[r];
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, a, 0, 0, 0);
      acc[r] = a;
    };
    f4 tacc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
    // Transposed operands of one row-tile pair: [column tile][hi, lo].
    h8 TP[2][2];
    auto tr_issue = [&]() __attribute__((always_inline)) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const u64x2 v = {tr_read(&tsc[wave][t][p][0][chunk_r]),
                           tr_read(&tsc[wave][t][p][1][chunk_r])};
          TP[t][p] = __builtin_bit_cast(h8, v);
        }
      asm volatile("" ::: "memory");
    };
    auto tr_product = [&](int w) __attribute__((always_inline)) {
      const h8 vih = vrow[wave][w][0][lane], vil = vrow[wave][w][1][lane];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f4 a = tacc[t];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vih, TP[t][0], a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vil, TP[t][0], a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vih, TP[t][1], a, 0, 0, 0);
        tacc[t] = a;
      }
    };
    f4 S0[2], S1[2];
    h8 PH[2], PL[2];
    dist(0, S0[0], S1[0]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f4 s0 = S0[r & 1], s1 = S1[r & 1];
      if (r + 1 < R) dist(r + 1, S0[(r + 1) & 1], S1[(r + 1) & 1]);
      if (r > 0) product(r - 1, PH[(r - 1) & 1], PL[(r - 1) & 1]);
      if constexpr (MASK) {
        const int64_t dt = tile0 + r;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (jt0 == dt && li == lj + q) s0[q] = 0.0f;
          if (jt0 + 1 == dt && li == lj + q) s1[q] = 0.0f;
        }
      }
      float f0[4], g0[4], f1[4], g1[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        kval_scaled<KIND>(s0[q], clampv, one, f0[q], g0[q]);
        kval_scaled<KIND>(s1[q], clampv, one, f1[q], g1[q]);
      }
      h2 hA, hB, hC, hD, lA, lB, lC, lD;
      split_pair<UNIT_G>(f0[0], g0[0], f0[1], g0[1], hA, lA);
      split_pair<UNIT_G>(f0[2], g0[2], f0[3], g0[3], hB, lB);
      split_pair<UNIT_G>(f1[0], g1[0], f1[1], g1[1], hC, lC);
      split_pair<UNIT_G>(f1[2], g1[2], f1[3], g1[3], hD, lD);
      PH[r & 1] = h8{hA[0], hA[1], hB[0], hB[1], hC[0], hC[1], hD[0], hD[1]};
      PL[r & 1] = h8{lA[0], lA[1], lB[0], lB[1], lC[0], lC[1], lD[0], lD[1]};
      if constexpr (SYM) {
        const u64x2 ph = __builtin_bit_cast(u64x2, PH[r & 1]);
        const u64x2 pl = __builtin_bit_cast(u64x2, PL[r & 1]);
        tsc[wave][0][0][r & 1][chunk_w] = ph[0];
        tsc[wave][1][0][r & 1][chunk_w] = ph[1];
        tsc[wave][0][1][r & 1][chunk_w] = pl[0];
        tsc[wave][1][1][r & 1][chunk_w] = pl[1];
        // Row-tile pair w = r/2 complete: fetch its transposed operands now,
        // multiply them one row tile later (after the next tile's VALU work).
        if (r & 1) tr_issue();
        if (r == 2) tr_product(0);
      }
    }
    product(R - 1, PH[(R - 1) & 1], PL[(R - 1) & 1]);
    if constexpr (SYM) {
      // Issue order: one MFMA, then kSymSchedValu VALU instructions, through
      // the step (measured at config 3: 16.8 -> 16.1 ms against the
      // compiler's default order, which bunches the kernel-value VALU; with
      // the unrolled stage loop 8 beats 7, 6 and 10 by 1-4%).
#pragma unroll
      for (int i = 0; i < R * (2 * KB + 3) + 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kSymSchedValu, 0);
      }
    }
    if constexpr (SYM) {
      tr_product(R / 2 - 1);
      tbuf[slot][k][wave][0][lane] = tacc[0];
      tbuf[slot][k][wave][1][lane] = tacc[1];
    }
  };
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int q = 0; q < 4; ++q) accd[r][q] += (double)acc[r][q];
      acc[r] = f4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // Adds the waves' transposed sums of stage c (buffer c & 1) in wave order
  // and writes them, unscaled, to tp.  Unit u < kSymSteps * 256 is two
  // right-hand sides (2h, 2h + 1 of the lane's four) of one lane of one
  // column tile; a thread's units share the lane half, so its column scales
  // are fixed for the kernel.  Only the first W / 2 waves reduce: they are
  // the older wave of each SIMD, which the issue arbiter favours, and they
  // reach the stage barrier ~1000 cycles before their SIMD partner, so the
  // reduction fills that wait while the younger waves go straight on to the
  // next stage's arithmetic.
  constexpr int kRedUnits = kSymSteps * 256;
  constexpr int kRedThreads = 64 * (W / 2);
  const int ru = threadIdx.x;
  const int r_ln = (ru >> 1) & 63, r_h = ru & 1;
  const int r_c = 4 * (r_ln >> 4) + 2 * r_h;
  f2 r_scale = {0.f, 0.f};
  {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int cc = r_c + e;
      const int shift = cc < ncols ? col_shift(colmax[cc]) : 0;
      r_scale[e] = ldexpf(1.0f, -(shift + kPScaleLog2));
    }
  }
  auto reduce_stage = [&](int64_t c) __attribute__((always_inline)) {
    const int slot = (int)(c & 1);
    const int64_t blk = b * hmax + stage_delta(c) - 1;
    constexpr int wstride = (int)(sizeof(tbuf[0][0][0]) / sizeof(float));
    if (wave >= W / 2) return;
    // Units ru, ru + kRedThreads, ...: the same lane half (kRedThreads is a
    // multiple of 128).
#pragma unroll
    for (int uu = 0; uu < kRedUnits; uu += kRedThreads) {
      const int u = uu + ru;
      if (u >= kRedUnits) break;
      const int kk = u >> 8, t = (u >> 7) & 1;
      const float* src = reinterpret_cast<const float*>(&tbuf[slot][kk][0][t][r_ln]) + 2 * r_h;
      f2 sum = *reinterpret_cast<const f2*>(src);
#pragma unroll
      for (int w = 1; w < W; ++w) sum += *reinterpret_cast<const f2*>(src + w * wstride);
      const int64_t jl = 32 * ((c % kSymStages) * kSymSteps + kk) + 16 * t + (r_ln & 15);
      // read once, by k_sym_reduce after this kernel: non-temporal, so the
      // partials do not displace the column operands the XCDs share in L2
      __builtin_nontemporal_store(sum * r_scale,
                                  reinterpret_cast<f2*>(tp + (blk * kSymRows + jl) * 16 + r_c));
    }
  };

  const int64_t dlo = tile0 / 2, dhi = dlo + R / 2;
  if (nst > 0) {
    fetch(stage_u0(0));
    commit(0);
  }
  int since_flush = 0;
  for (int64_t c = 0; c < nst; ++c) {
    const int st = (int)(c & 1);
    __syncthreads();
    if (c + 1 < nst) fetch(stage_u0(c + 1));
    if (c > 0 && stage_delta(c - 1) > 0) reduce_stage(c - 1);
    const int64_t u0 = stage_u0(c);
    // Wave priority per step: the younger wave of each SIMD leads the first
    // step, the older one the second.  Under the arbiter's default (oldest
    // first) the older wave finished its stage ~3000 cycles before its
    // partner, which then ran alone at single-wave speed until the barrier.
    auto lead = [&](int k) __attribute__((always_inline)) {
      if ((wave < W / 2) == (k == 0))
        __builtin_amdgcn_s_setprio(0);
      else
        __builtin_amdgcn_s_setprio(1);
    };
    if (stage_delta(c) == 0) {
      for (int k = 0; k < kSymSteps; ++k) {
        lead(k);
        const int64_t u = u0 + k;
        if (u >= dlo && u < dhi)
          step(st, k, u, st, std::true_type{}, std::false_type{});
        else
          step(st, k, u, st, std::false_type{}, std::false_type{});
      }
    } else {
      // Unrolled: no accumulator copies at a step back-edge (15.88 -> 15.72
      // ms at config 3, measured once the loop head no longer waited for the
      // next stage's operand loads; before that it measured slower).
#pragma unroll
      for (int k = 0; k < kSymSteps; ++k) {
        lead(k);
        step(st, k, u0 + k, st, std::false_type{}, std::true_type{});
      }
    }
    since_flush += kSymSteps;
    // fp64 flush every 16 column-tile pairs (512 columns; 256 in the
    // one-sided kernel): 48 fp32 MFMA accumulations per flush.  The config-3
    // product stays well inside 1e-5 of fp64, and the tile kernel gained
    // 0.6% against a 256-column flush, alternated.
    if (since_flush >= kFlushTiles) {
      flush();
      since_flush = 0;
    }
    if (c + 1 < nst) commit(st ^ 1);
  }
  if (nst > 0 && stage_delta(nst - 1) > 0) {
    __syncthreads();
    reduce_stage(nst - 1);
  }
  flush();

  // Forward partials of this split, unscaled by the fp16 factors.
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = lj + q;
      const int64_t i = 16 * (tile0 + r) + li;
      const int shift = c < ncols ? col_shift(colmax[c]) : 0;
      fwd[(split * 16 + c) * mpad + i] =
          (float)ldexp(accd[r][q] + (double)acc[r][q], -(shift + kPScaleLog2));
    }
  }
}

// ---------------------------------------------------------------------------
// Gradient traces on the matrix cores (Gram-form kernels).
//
// The pair-loop trace (solver.hip k_grad_trace) spends ~90 VALU instructions
// per pair on per-dimension differences, the 16-column dot g_ab = sum_c
// Lf_ca Rf_cb and the per-dimension accumulation.  Here, per 16x16 tile:
//   * the scaled squared distance comes from the Gram-form distance MFMAs of
//     the product kernels (KB per tile);
//   * D = W + W^T comes from one K=32 contraction of [Rf'_b | Lf'_b] with
//     [Lf'_a ; Rf'_a] (3 MFMAs for the two-term fp16 split).  Lf and Rf are
//     scaled per column by powers of two (Lf' = 2^sL_c Lf_c with max |Lf'_c|
//     in [2^13, 2^14), Rf' = 2^(T - sL_c) Rf_c) so every product carries the
//     common factor 2^T and the largest column products sit at 2^28;
//   * M = D h (the kernel's lengthscale factor, scaled by 2^-kGtMExp into
//     fp16 range) is contracted with [z_b | z_b^2] on the matrix cores (3 per
//     tile per 16 dimensions), and its row sums R_a on VALU;
//   * every kGtFold column-tile pairs the point's terms
//       sum_b M_ab (z_aq - z_bq)^2 = z_aq^2 R_a - 2 z_aq (M z)_aq + (M z^2)_aq
//     are formed in fp64 (the expansion cancels; each fp32 input carries 24
//     bits over at most 256 columns) and accumulated.
// Since h (z_aq - z_bq)^2 and k are symmetric, only the symmetric part of W
// contributes: row block b forms its diagonal block with weight 1/2 on D and
// the off-diagonal blocks of the cyclic half (sym_span) with weight 1, so
// every ordered pair is counted once.  The os term sum_ab W_ab k_ab/os is
// accumulated from D k on VALU alongside.
// ---------------------------------------------------------------------------
constexpr int kGtR = 2;                              // row tiles per wave
constexpr int kGtWaves = 8;                          // waves per workgroup
constexpr int kGtRows = 16 * kGtR * kGtWaves;        // rows (and columns) per block
constexpr int kGtPairs = kGtRows / 32;               // column-tile pairs per block
constexpr int kGtSteps = 2;                          // column-tile pairs per LDS stage
constexpr int kGtStages = kGtPairs / kGtSteps;       // LDS stages per block
constexpr int kGtFold = 8;                           // column-tile pairs between fp64 folds
constexpr int kGtMExp = 20;                          // M = D h 2^-kGtMExp before its split
static_assert((16 * kPackTileAlign) % kGtRows == 0, "blocks must tile the packed points");

// Column exponents of a 16-column chunk: colmax[0..15] = max |Lf_c|,
// colmax[16..31] = max |Rf_c| (float bits).  shifts[c] = sL_c,
// shifts[16 + c] = T - sL_c, shifts[32] = T.  One thread.
__global__ void k_grad_shifts(const uint32_t* __restrict__ colmax, int nc,
                              int* __restrict__ shifts) {
  if (threadIdx.x != 0) return;
  int eL[16], eR[16];
  bool live[16];
  int smax = -100000;
  for (int c = 0; c < 16; ++c) {
    const float ml = c < nc ? __uint_as_float(colmax[c]) : 0.0f;
    const float mr = c < nc ? __uint_as_float(colmax[16 + c]) : 0.0f;
    live[c] = ml > 0.0f && mr > 0.0f && ml < 3.0e38f && mr < 3.0e38f;
    (void)frexpf(live[c] ? ml : 1.0f, &eL[c]);
    (void)frexpf(live[c] ? mr : 1.0f, &eR[c]);
    if (live[c]) smax = max(smax, eL[c] + eR[c]);
  }
  const int T = smax == -100000 ? 0 : 28 - smax;
  for (int c = 0; c < 16; ++c) {
    shifts[c] = live[c] ? 14 - eL[c] : 0;
    shifts[16 + c] = live[c] ? T - (14 - eL[c]) : 0;
  }
  shifts[32] = T;
}

// One thread per (tile, lane) of ntiles tiles: WA (column side, A operand,
// row m = point, K = [Rf' c0..15 | Lf' c0..15]) and WB (row side, B operand,
// column n = point, K = [Lf' | Rf']), lane l holding K = 8 (l/16) .. + 7 of
// point 16 tile + l%16; parts hi, lo at [(tile*2 + part)*64 + lane].
__global__ void k_pack_grad_w(const float* __restrict__ Lf, const float* __restrict__ Rf,
                              int64_t n, int nc, int64_t ntiles, const int* __restrict__ shifts,
                              h8* __restrict__ WA, h8* __restrict__ WB) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= ntiles * 64) return;
  const int lane = (int)(idx & 63);
  const int64_t tile = idx >> 6;
  const int64_t p = 16 * tile + (lane & 15);
  const int k0 = 8 * (lane >> 4);
  h8 ah, al, bh, bl;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = k0 + e;
    const int c = k & 15;
    const bool live = p < n && c < nc;
    const float lf = live ? ldexpf(Lf[(int64_t)c * n + p], shifts[c]) : 0.0f;
    const float rf = live ? ldexpf(Rf[(int64_t)c * n + p], shifts[16 + c]) : 0.0f;
    const float va = k < 16 ? rf : lf;  // column side [Rf' | Lf']
    const float vb = k < 16 ? lf : rf;  // row side [Lf' ; Rf']
    ah[e] = (_Float16)va;
    al[e] = (_Float16)(va - (float)ah[e]);
    bh[e] = (_Float16)vb;
    bl[e] = (_Float16)(vb - (float)bh[e]);
  }
  WA[(tile * 2) * 64 + lane] = ah;
  WA[(tile * 2 + 1) * 64 + lane] = al;
  WB[(tile * 2) * 64 + lane] = bh;
  WB[(tile * 2 + 1) * 64 + lane] = bl;
}

// One thread per (pair u, group gr < 2 QG, lane): the A operand of U = [z|z^2] M
// (row m = dimension q = 16 (gr % QG) + lane%16, squares for gr >= QG; K = the
// pair's 32 columns in the packed right-hand-side order: element e holds point
// 16 (2u + e/4) + 4 (lane/16) + e%4); parts hi, lo at
// [((u*2QG + gr)*2 + part)*64 + lane].
__global__ void k_pack_grad_zz(const float* __restrict__ Z, int64_t n, int d, int qg,
                               int64_t pairs, h8* __restrict__ ZZ) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs * 2 * qg * 64) return;
  const int lane = (int)(idx & 63);
  const int gr = (int)((idx >> 6) % (2 * qg));
  const int64_t u = (idx >> 6) / (2 * qg);
  const int q = 16 * (gr % qg) + (lane & 15);
  const bool sq = gr >= qg;
  h8 hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t b = 32 * u + 16 * (e >> 2) + 4 * (lane >> 4) + (e & 3);
    float v = (b < n && q < d) ? Z[b * d + q] : 0.0f;
    if (sq) v = v * v;
    hi[e] = (_Float16)v;
    lo[e] = (_Float16)(v - (float)hi[e]);
  }
  ZZ[((u * 2 * qg + gr) * 2) * 64 + lane] = hi;
  ZZ[((u * 2 * qg + gr) * 2 + 1) * 64 + lane] = lo;
}

// kv = k/os and h (the derivative factor of the pair-loop trace) from the
// scaled squared distance s.
template <int KIND>
__device__ __forceinline__ void grad_factors(float s, float clampv, float& kv, float& h) {
  if constexpr (KIND == KIND_RBF) {
    (void)clampv;  // the RBF exponent is not clamped
    // med3 rather than fmaxf on the MFMA result (see kval_scaled)
    kv = __builtin_amdgcn_exp2f(-__builtin_amdgcn_fmed3f(s, 0.0f, 3.0e38f));
    h = kv;
  } else if constexpr (KIND == KIND_MATERN32) {
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    float mn = fminf(u, clampv);
    asm("" : "+v"(mn));
    const float e = __builtin_amdgcn_exp2f(-mn);
    kv = fmaf(u, kLn2, 1.0f) * e;
    h = 3.0f * e;
  } else {
    const float u = __builtin_amdgcn_sqrtf(fabsf(s));
    float mn = fminf(u, clampv);
    asm("" : "+v"(mn));
    const float e = __builtin_amdgcn_exp2f(-mn);
    kv = fmaf(u, fmaf(u, kLn2 * kLn2 / 3.0f, kLn2), 1.0f) * e;
    h = fmaf(u, (5.0f / 3.0f) * kLn2, 5.0f / 3.0f) * e;
  }
}

// part[L][q] (q < 16 QG: sum_ab M (z_aq - z_bq)^2 at scale 2^(T - kGtMExp)),
// part[L][16 QG] (sum_ab D k/os at scale 2^T) for work item L = (row block b,
// delta split).
template <int KIND, int KB, int QG>
__global__ __launch_bounds__(64 * kGtWaves) void k_grad_sym(
    const h8* __restrict__ Bi, const h8* __restrict__ Aj, const h8* __restrict__ WA,
    const h8* __restrict__ WB, const h8* __restrict__ ZZ, const float* __restrict__ Z, int d,
    int64_t n, int64_t nb, int64_t splits, int64_t dps, double* __restrict__ part) {
  constexpr int R = kGtR, W = kGtWaves;
  constexpr int kA = 2 * KB;   // distance operand blocks per pair
  constexpr int kW = 4;        // W operand blocks per pair (2 tiles x hi, lo)
  constexpr int kZ = 4 * QG;   // [z|z^2] blocks per pair (2 QG groups x hi, lo)
  constexpr int kBlocks = kGtSteps * (kA + kW + kZ);
  constexpr int NQ = 16 * QG;
  __shared__ h8 lds[2][kBlocks][64];
  __shared__ double red[W][NQ + 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t per = (int64_t)gridDim.x / kXcds;
  const int64_t L = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (L >= nb * splits) return;  // whole workgroup, before any barrier
  const int64_t b = L % nb;
  const int64_t split = L / nb;
  const int64_t tile0 = (b * W + wave) * R;
  const int li = lane & 15, lg = lane >> 4, lj = 4 * lg;

  h8 bi[R][KB], wb[R][2];
  float zr[R][QG][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) bi[r][kb] = Bi[((tile0 + r) * KB + kb) * 64 + lane];
    wb[r][0] = WB[((tile0 + r) * 2) * 64 + lane];
    wb[r][1] = WB[((tile0 + r) * 2 + 1) * 64 + lane];
    const int64_t a = 16 * (tile0 + r) + li;
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = 16 * g + lj + e;
        zr[r][g][e] = (a < n && q < d) ? Z[a * d + q] : 0.0f;
      }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // row operands before the loop (see k_sym_tile)
  f4 U[R][2 * QG];
  float rs[R];
  double T[QG][4];
  float osf = 0.0f;
  double osd = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rs[r] = 0.0f;
#pragma unroll
    for (int g = 0; g < 2 * QG; ++g) U[r][g] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int g = 0; g < QG; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) T[g][e] = 0.0;
  const float clampv = clamp_reg();

  const int64_t span = sym_span(b, nb);
  const int64_t d0 = split * dps;
  const int64_t d1 = min(d0 + dps, span + 1);
  const int64_t nst = d1 > d0 ? (d1 - d0) * kGtStages : 0;
  auto stage_delta = [&](int64_t c) { return d0 + c / kGtStages; };
  auto stage_u0 = [&](int64_t c) {
    int64_t J = b + stage_delta(c);
    if (J >= nb) J -= nb;
    return J * kGtPairs + (c % kGtStages) * kGtSteps;
  };

  // Stage operands through registers (see k_sym_tile): blocks [distance |
  // W | z], each range contiguous in global memory.
  constexpr int kFillPerWave = (kBlocks + W - 1) / W;
  h8 pre[kFillPerWave];
  auto fetch = [&](int64_t u0) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kFillPerWave; ++q) {
      const int bb = min(wave + q * W, kBlocks - 1);
      const h8* src = bb < kGtSteps * kA ? Aj + (2 * u0 * KB + bb) * 64
                      : bb < kGtSteps * (kA + kW)
                          ? WA + (4 * u0 + (bb - kGtSteps * kA)) * 64
                          : ZZ + (u0 * kZ + (bb - kGtSteps * (kA + kW))) * 64;
      pre[q] = src[lane];
    }
  };
  auto commit = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kFillPerWave; ++q) {
      const int bb = wave + q * W;
      if (bb < kBlocks) lds[st][bb][lane] = pre[q];
    }
  };

  // One column-tile pair against the wave's R row tiles.  DIAG: a tile of the
  // diagonal block (weight 1/2 on D); MASK: restore the exact zero
  // self-distance on diagonal tiles.
  auto step = [&](int st, int k, int64_t u, auto mask_tag, auto diag_tag)
                  __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr bool DIAG = decltype(diag_tag)::value;
    constexpr float wd = DIAG ? 0.5f : 1.0f;
    constexpr float mscale = wd * (1.0f / (float)(1 << kGtMExp));
    const int64_t jt0 = 2 * u;
    h8 a0[KB], a1[KB], wa[2][2], zz[2 * QG][2];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      a0[kb] = lds[st][k * kA + kb][lane];
      a1[kb] = lds[st][k * kA + KB + kb][lane];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int p = 0; p < 2; ++p) wa[t][p] = lds[st][kGtSteps * kA + k * kW + 2 * t + p][lane];
#pragma unroll
    for (int g = 0; g < 2 * QG; ++g)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        zz[g][p] = lds[st][kGtSteps * (kA + kW) + k * kZ + 2 * g + p][lane];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f4 s0 = f4{0.f, 0.f, 0.f, 0.f}, s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[kb], bi[r][kb], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[kb], bi[r][kb], s1, 0, 0, 0);
      }
      f4 D0 = f4{0.f, 0.f, 0.f, 0.f}, D1 = f4{0.f, 0.f, 0.f, 0.f};
      D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[0][0], wb[r][0], D0, 0, 0, 0);
      D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[1][0], wb[r][0], D1, 0, 0, 0);
      D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[0][1], wb[r][0], D0, 0, 0, 0);
      D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[1][1], wb[r][0], D1, 0, 0, 0);
      D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[0][0], wb[r][1], D0, 0, 0, 0);
      D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[1][0], wb[r][1], D1, 0, 0, 0);
      if constexpr (MASK) {
        const int64_t dt = tile0 + r;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (jt0 == dt && li == lj + q) s0[q] = 0.0f;
          if (jt0 + 1 == dt && li == lj + q) s1[q] = 0.0f;
        }
      }
      float m0[4], m1[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float kv, h;
        grad_factors<KIND>(s0[q], clampv, kv, h);
        m0[q] = D0[q] * (h * mscale);
        osf = fmaf(D0[q] * wd, kv, osf);
        grad_factors<KIND>(s1[q], clampv, kv, h);
        m1[q] = D1[q] * (h * mscale);
        osf = fmaf(D1[q] * wd, kv, osf);
        rs[r] += m0[q] + m1[q];
      }
      h2 hA, hB, hC, hD, lA, lB, lC, lD;
      split_pair<true>(m0[0], 1.0f, m0[1], 1.0f, hA, lA);
      split_pair<true>(m0[2], 1.0f, m0[3], 1.0f, hB, lB);
      split_pair<true>(m1[0], 1.0f, m1[1], 1.0f, hC, lC);
      split_pair<true>(m1[2], 1.0f, m1[3], 1.0f, hD, lD);
      const h8 mh = h8{hA[0], hA[1], hB[0], hB[1], hC[0], hC[1], hD[0], hD[1]};
      const h8 ml = h8{lA[0], lA[1], lB[0], lB[1], lC[0], lC[1], lD[0], lD[1]};
#pragma unroll
      for (int g = 0; g < 2 * QG; ++g) {
        f4 a = U[r][g];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(zz[g][0], mh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(zz[g][1], mh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(zz[g][0], ml, a, 0, 0, 0);
        U[r][g] = a;
      }
    }
  };
  // Per point: z^2 R - 2 z (M z) + (M z^2) in fp64, accumulated per lane.
  auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float rsum = rs[r];
      rsum += __shfl_xor(rsum, 16);
      rsum += __shfl_xor(rsum, 32);
      const double Rd = (double)rsum;
#pragma unroll
      for (int g = 0; g < QG; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double z = (double)zr[r][g][e];
          T[g][e] += z * z * Rd - 2.0 * z * (double)U[r][g][e] + (double)U[r][QG + g][e];
        }
      rs[r] = 0.0f;
#pragma unroll
      for (int g = 0; g < 2 * QG; ++g) U[r][g] = f4{0.f, 0.f, 0.f, 0.f};
    }
    osd += (double)osf;
    osf = 0.0f;
  };

  const int64_t dlo = tile0 / 2, dhi = dlo + R / 2;
  if (nst > 0) {
    fetch(stage_u0(0));
    commit(0);
  }
  int since_fold = 0;
  for (int64_t c = 0; c < nst; ++c) {
    const int st = (int)(c & 1);
    __syncthreads();
    if (c + 1 < nst) fetch(stage_u0(c + 1));
    const int64_t u0 = stage_u0(c);
    if (stage_delta(c) == 0) {
      for (int k = 0; k < kGtSteps; ++k) {
        const int64_t u = u0 + k;
        if (u >= dlo && u < dhi)
          step(st, k, u, std::true_type{}, std::true_type{});
        else
          step(st, k, u, std::false_type{}, std::true_type{});
      }
    } else {
      for (int k = 0; k < kGtSteps; ++k) {
        // Wave priority per step as in k_sym_tile (24.7 -> 24.0 ms at config 3).
        if ((wave < W / 2) == (k == 0))
          __builtin_amdgcn_s_setprio(0);
        else
          __builtin_amdgcn_s_setprio(1);
        step(st, k, u0 + k, std::false_type{}, std::false_type{});
      }
    }
    since_fold += kGtSteps;
    if (since_fold >= kGtFold) {
      fold();
      since_fold = 0;
    }
    if (c + 1 < nst) commit(st ^ 1);
  }
  fold();

  // Sum over the 16 rows of each lane group, then over the waves in order.
#pragma unroll
  for (int g = 0; g < QG; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      double v = T[g][e];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off);
      if (li == 0) red[wave][16 * g + lj + e] = v;
    }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) osd += __shfl_xor(osd, off);
  if (lane == 0) red[wave][NQ] = osd;
  __syncthreads();
  if (threadIdx.x <= NQ) {
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < W; ++w) tot += red[w][threadIdx.x];
    part[L * (NQ + 1) + threadIdx.x] = tot;
  }
}

// out[c*m + j] = os * (sum_s fwd[s][c][j] + sum of the transposed partials of
// the row blocks that formed j's column block, in delta order) + noise V.
// Four threads per point, each owning four right-hand sides (16 contiguous
// bytes of every partial row); fp64 sums in a fixed order.  The delta loop
// loads four partials at a time unconditionally (every (block, delta) slot
// is allocated) and keeps the formed ones by a select.
__global__ __launch_bounds__(256) void k_sym_reduce(const float* __restrict__ fwd, int splits,
                                                    const float* __restrict__ tp, int64_t nb,
                                                    int64_t hmax, int64_t mpad, int64_t m,
                                                    int ncols, float os, float noise,
                                                    const float* __restrict__ Vin,
                                                    float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t j = t >> 2;
  const int c4 = (int)(t & 3);
  if (j >= m) return;
  double tot[4] = {0.0, 0.0, 0.0, 0.0};
  for (int s = 0; s < splits; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 4 * c4 + e;
      if (c < ncols) tot[e] += fwd[((int64_t)s * 16 + c) * mpad + j];
    }
  const int64_t J = j / kSymRows, jl = j - J * kSymRows;
  const float* col = tp + jl * 16 + 4 * c4;
  // The partials are read once: non-temporal loads, eight in flight.
  auto slot = [&](int64_t dl, bool& formed) {
    int64_t bb = J - dl;
    if (bb < 0) bb += nb;
    formed = dl <= sym_span(bb, nb);
    return __builtin_nontemporal_load(
        reinterpret_cast<const f4*>(col + (bb * hmax + dl - 1) * (int64_t)kSymRows * 16));
  };
  int64_t dl = 1;
  for (; dl + 7 <= hmax; dl += 8) {
    f4 v[8];
    bool ok[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = slot(dl + q, ok[q]);
#pragma unroll
    for (int q = 0; q < 8; ++q)
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
      const int64_t idx = (int64_t)c * m + j;
      out[idx] = fmaf(noise, Vin[idx], os * (float)tot[e]);
    }
  }
}

// Task-mixing reduction: one thread per (column block cc, row i) sums the split
// partials of the block's T columns once, then writes the T mixed outputs
// out[(cc*T + t)*m + i] (+)= sum_t' mix[t*T + t'] (os sum_s partial + noise V).
constexpr int kMaxMixT = 16;
__global__ void k_reduce_mix(const float* __restrict__ partial, int splits, int cpad,
                             int64_t mpad, int64_t m, int nblocks, int T, float os, float noise,
                             int add_noise, const float* __restrict__ Vin,
                             const float* __restrict__ mix, int accumulate,
                             float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)nblocks * m) return;
  const int cc = (int)(idx / m);
  const int64_t i = idx - (int64_t)cc * m;
  float v[kMaxMixT];
#pragma unroll
  for (int tp = 0; tp < kMaxMixT; ++tp) {
    if (tp < T) {
      const int c = cc * T + tp;
      double tot = 0.0;
      for (int sp = 0; sp < splits; ++sp) tot += partial[((int64_t)sp * cpad + c) * mpad + i];
      float o = os * (float)tot;
      if (add_noise) o = fmaf(noise, Vin[(int64_t)c * m + i], o);
      v[tp] = o;
    }
  }
  for (int t = 0; t < T; ++t) {
    float o = 0.0f;
#pragma unroll
    for (int tp = 0; tp < kMaxMixT; ++tp)
      if (tp < T) o = fmaf(mix[t * T + tp], v[tp], o);
    const int64_t off = (int64_t)(cc * T + t) * m + i;
    out[off] = accumulate ? out[off] + o : o;
  }
}

// k_reduce_mix over four consecutive rows per thread with 16-byte loads and
// stores (m and mpad multiples of 4, 16-byte aligned arrays); the same sums
// in the same order per row.
__global__ void k_reduce_mix4(const float* __restrict__ partial, int splits, int cpad,
                              int64_t mpad, int64_t m, int nblocks, int T, float os, float noise,
                              int add_noise, const float* __restrict__ Vin,
                              const float* __restrict__ mix, int accumulate,
                              float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t m4 = m / 4;
  if (idx >= (int64_t)nblocks * m4) return;
  const int cc = (int)(idx / m4);
  const int64_t i = 4 * (idx - (int64_t)cc * m4);
  f4 v[kMaxMixT];
#pragma unroll
  for (int tp = 0; tp < kMaxMixT; ++tp) {
    if (tp < T) {
      const int c = cc * T + tp;
      double tot[4] = {0.0, 0.0, 0.0, 0.0};
      // Four split partials in flight per step (same summation order).
      int sp = 0;
      for (; sp + 4 <= splits; sp += 4) {
        f4 q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          q[k] = *reinterpret_cast<const f4*>(partial + ((int64_t)(sp + k) * cpad + c) * mpad + i);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) tot[e] += (double)q[k][e];
      }
      for (; sp < splits; ++sp) {
        const f4 q = *reinterpret_cast<const f4*>(partial + ((int64_t)sp * cpad + c) * mpad + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) tot[e] += (double)q[e];
      }
      f4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = os * (float)tot[e];
      if (add_noise) {
        const f4 x = *reinterpret_cast<const f4*>(Vin + (int64_t)c * m + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = fmaf(noise, x[e], o[e]);
      }
      v[tp] = o;
    }
  }
  for (int t = 0; t < T; ++t) {
    f4 o = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tp = 0; tp < kMaxMixT; ++tp)
      if (tp < T) {
        const float w = mix[t * T + tp];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = fmaf(w, v[tp][e], o[e]);
      }
    f4* dst = reinterpret_cast<f4*>(out + (int64_t)(cc * T + t) * m + i);
    if (accumulate) {
      const f4 prev = *dst;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] += prev[e];
    }
    *dst = o;
  }
}

// ---------------------------------------------------------------------------
// Direct (per-dimension difference) product: one thread per row, LDS tiles of
// column points.  Arithmetic follows the reference order: r^2 = sum_d diff^2.
// ---------------------------------------------------------------------------
constexpr int kDirectTile = 128;
constexpr int kDirectMaxCols = 16;

template <int KIND>
__global__ __launch_bounds__(256) void k_direct(
    const float* __restrict__ Zr, int64_t m, const float* __restrict__ Zc,
    int64_t n, int d, const float* __restrict__ V, int ncols, float os,
    float noise, int add_noise, float lim, float* __restrict__ out) {
  extern __shared__ float sm[];  // [kDirectTile][d + ncols]
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int w = d + ncols;
  float xi[32];
  for (int k = 0; k < d; ++k) xi[k] = (i < m) ? Zr[i * d + k] : 0.0f;
  double acc[kDirectMaxCols];
  for (int c = 0; c < kDirectMaxCols; ++c) acc[c] = 0.0;
  for (int64_t j0 = 0; j0 < n; j0 += kDirectTile) {
    __syncthreads();
    for (int t = threadIdx.x; t < kDirectTile * w; t += blockDim.x) {
      const int jj = t / w, k = t - jj * w;
      const int64_t j = j0 + jj;
      float val = 0.0f;
      if (j < n) val = (k < d) ? Zc[j * d + k] : V[(int64_t)(k - d) * n + j];
      sm[t] = val;
    }
    __syncthreads();
    const int cnt = (int)min((int64_t)kDirectTile, n - j0);
    for (int jj = 0; jj < cnt; ++jj) {
      const float* row = sm + jj * w;
      float r2 = 0.0f;
      for (int k = 0; k < d; ++k) {
        const float df = xi[k] - row[k];
        r2 = fmaf(df, df, r2);
      }
      const float kv = kval<KIND>(r2, lim);
      for (int c = 0; c < ncols; ++c) acc[c] += (double)(kv * row[d + c]);
    }
  }
  if (i < m) {
    for (int c = 0; c < ncols; ++c) {
      float o = os * (float)acc[c];
      if (add_noise) o = fmaf(noise, V[(int64_t)c * m + i], o);
      out[(int64_t)c * m + i] = o;
    }
  }
}

// Dense cross-covariance block: out[c*n + i] = os * k(zr[r0 + c], zc[i]) for
// c < rows, i < n, from per-dimension differences (reference arithmetic).
template <int KIND>
__global__ __launch_bounds__(256) void k_fill_cross(const float* __restrict__ Zr, int64_t r0,
                                                    int64_t rows, const float* __restrict__ Zc,
                                                    int64_t n, int d, float os, float lim,
                                                    float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * n) return;
  const int64_t c = idx / n, i = idx - c * n;
  const float* zr = Zr + (r0 + c) * d;
  const float* zc = Zc + i * d;
  float r2 = 0.0f;
  for (int k = 0; k < d; ++k) {
    const float df = zr[k] - zc[k];
    r2 = fmaf(df, df, r2);
  }
  out[idx] = os * kval<KIND>(r2, lim);
}

// Symmetric half of the dense K (dense.h layout), one workgroup per stored
// block: the block's 256 row points and 256 column points are staged in LDS
// dimension-major ([k][256], zero past n); thread t forms the units t,
// t + 256, .. of the block in fragment order: os * k(z_row, z_col) for one
// row and eight columns from per-dimension differences (the arithmetic of
// k_fill_cross), scaled by 2^shift and stored as the two-term fp16 split, hi
// and lo as two 16-byte units (consecutive threads write consecutive units);
// rows and columns past n are zero.  d <= kFillLdsMaxD (the provider's
// dimension limit).
constexpr int kHalfRows = 256;
constexpr int kFillLdsMaxD = 32;
template <int KIND>
__global__ __launch_bounds__(256) void k_fill_half_lds(const float* __restrict__ Z, int64_t n,
                                                       int d, float os, float lim, int shift,
                                                       int64_t nb, uint32_t* __restrict__ half) {
  extern __shared__ float zs[];  // [2][d][256]: rows, then columns
  constexpr int kGroups = kHalfRows / 8;
  const int64_t blk = blockIdx.x;
  // block index -> (b, delta), the inverse of dense_half_index (uniform)
  int64_t b, delta;
  if (nb & 1) {
    const int64_t w = (nb - 1) / 2 + 1;
    b = blk / w;
    delta = blk - b * w;
  } else {
    const int64_t h = nb / 2;
    if (blk < h * (h + 1)) {
      b = blk / (h + 1);
      delta = blk - b * (h + 1);
    } else {
      const int64_t q = blk - h * (h + 1);
      b = h + q / h;
      delta = q - (q / h) * h;
    }
  }
  int64_t J = b + delta;
  if (J >= nb) J -= nb;
  for (int t = threadIdx.x; t < 2 * kHalfRows * d; t += 256) {
    const int side = t / (kHalfRows * d);
    const int rem = t - side * (kHalfRows * d);
    const int p = rem / d, k = rem - p * d;
    const int64_t pt = (side ? J : b) * kHalfRows + p;
    zs[(side * d + k) * kHalfRows + p] = pt < n ? Z[pt * d + k] : 0.0f;
  }
  __syncthreads();
  const float* zr_s = zs;
  const float* zc_s = zs + d * kHalfRows;
  const int64_t row0 = b * kHalfRows, col0 = J * kHalfRows;
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  for (int u = threadIdx.x; u < kHalfRows * kGroups; u += 256) {
    const int lane = u & 63;
    const int r = 32 * ((u >> 7) & 7) + 16 * ((u >> 6) & 1) + (lane & 15);
    const int g = 4 * (u >> 10) + (lane >> 4);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    if (row0 + r < n) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 8 * g + e;
        if (col0 + c < n) {
          float r2 = 0.0f;
          for (int k = 0; k < d; ++k) {
            const float df = zr_s[k * kHalfRows + r] - zc_s[k * kHalfRows + c];
            r2 = fmaf(df, df, r2);
          }
          x[e] = ldexpf(os * kval<KIND>(r2, lim), shift);
        }
      }
    }
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hi[e] = (_Float16)x[e];
      lo[e] = (_Float16)(x[e] - (float)hi[e]);
    }
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[e] = (uint32_t)__builtin_bit_cast(uint16_t, hi[2 * e]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, hi[2 * e + 1]) << 16);
      w[4 + e] = (uint32_t)__builtin_bit_cast(uint16_t, lo[2 * e]) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, lo[2 * e + 1]) << 16);
    }
    *reinterpret_cast<u4*>(half + half_frag_index(blk, r, g, 0) * 4) = u4{w[0], w[1], w[2], w[3]};
    *reinterpret_cast<u4*>(half + half_frag_index(blk, r, g, 1) * 4) = u4{w[4], w[5], w[6], w[7]};
  }
}

// ---------------------------------------------------------------------------
// Gradient products: out[p][c][i] = sum_j dk(x_i, x_j)/dtheta_p V[c][j] for the
// engine parameters theta = [l | l_0..l_{d-1}, os] (fused_all_gradients_matvec,
// gpu_kernel.py:382-484).  Per pair, from per-dimension differences dz of the
// scaled coordinates (dz = diff * s / l):
//   RBF       h = k (clamped);  Matern-5/2  h = (5/3) os (1 + sqrt5 r) e^{max(-sqrt5 r, -20)}
//   dk/dl_q = h dz_q^2 / (s^2 l_q)   (iso: h |dz|^2 / (s^2 l))
//   dk/dos  = k / os
// One thread per row, LDS tiles of column points, kGradCols right-hand sides
// per pass, fp32 sums flushed into fp64 every tile.
// ---------------------------------------------------------------------------
constexpr int kGradTile = 64;
constexpr int kGradCols = 2;
constexpr int kGradMaxDim = 32;

template <int KIND, bool ARD>
__global__ __launch_bounds__(256) void k_grad_matvec(
    const float* __restrict__ Z, int64_t n, int d, const float* __restrict__ V, int ncols,
    int c0, float os, float lim, const float* __restrict__ pscale, float* __restrict__ out) {
  extern __shared__ float sm[];  // [kGradTile][d + kGradCols]
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int w = d + kGradCols;
  const int np = ARD ? d + 1 : 2;
  float zi[kGradMaxDim];
  for (int k = 0; k < d; ++k) zi[k] = (i < n) ? Z[i * d + k] : 0.0f;
  double accd[(kGradMaxDim + 1) * kGradCols];
  float acc[(kGradMaxDim + 1) * kGradCols];
  for (int q = 0; q < np * kGradCols; ++q) {
    accd[q] = 0.0;
    acc[q] = 0.0f;
  }
  for (int64_t j0 = 0; j0 < n; j0 += kGradTile) {
    __syncthreads();
    for (int t = threadIdx.x; t < kGradTile * w; t += blockDim.x) {
      const int jj = t / w, k = t - jj * w;
      const int64_t j = j0 + jj;
      float val = 0.0f;
      if (j < n) {
        if (k < d) {
          val = Z[j * d + k];
        } else {
          const int c = c0 + (k - d);
          val = c < ncols ? V[(int64_t)c * n + j] : 0.0f;
        }
      }
      sm[t] = val;
    }
    __syncthreads();
    const int cnt = (int)min((int64_t)kGradTile, n - j0);
    for (int jj = 0; jj < cnt; ++jj) {
      const float* row = sm + jj * w;
      float dz2[kGradMaxDim];
      float S = 0.0f;
      for (int k = 0; k < d; ++k) {
        const float df = zi[k] - row[k];
        dz2[k] = df * df;
        S += dz2[k];
      }
      const float kv = kval<KIND>(S, lim);  // k / os
      float h;
      if constexpr (KIND == KIND_RBF) {
        h = kv;
      } else if constexpr (KIND == KIND_MATERN12) {
        // log2(e) e^{max(-r,-20)} / r with the reference's r = sqrt(r^2 + 1e-20)
        h = kLog2e * kv / sqrtf(S + kM12RFloor);
      } else if constexpr (KIND == KIND_MATERN32) {
        // 3 e^{max(-sqrt3 r,-20)}
        h = 3.0f * __builtin_amdgcn_exp2f(-fminf(sqrtf(S), kExp2Clamp));
      } else {
        // (5/3)(1 + sqrt5 r) e^{max(-sqrt5 r,-20)} with sqrt5 r = u ln2, u = sqrt(S)
        const float u = sqrtf(S);
        const float e = __builtin_amdgcn_exp2f(-fminf(u, kExp2Clamp));
        h = (5.0f / 3.0f) * fmaf(u, kLn2, 1.0f) * e;
      }
      for (int c = 0; c < kGradCols; ++c) {
        const float v = row[d + c];
        const float hv = h * v;
        if constexpr (ARD) {
          for (int q = 0; q < d; ++q) acc[q * kGradCols + c] = fmaf(hv, dz2[q], acc[q * kGradCols + c]);
        } else {
          acc[c] = fmaf(hv, S, acc[c]);
        }
        acc[(np - 1) * kGradCols + c] = fmaf(kv, v, acc[(np - 1) * kGradCols + c]);
      }
    }
    for (int q = 0; q < np * kGradCols; ++q) {
      accd[q] += (double)acc[q];
      acc[q] = 0.0f;
    }
  }
  if (i >= n) return;
  for (int p = 0; p < np; ++p) {
    for (int c = 0; c < kGradCols; ++c) {
      const int cc = c0 + c;
      if (cc >= ncols) continue;
      out[((int64_t)p * ncols + cc) * n + i] = (float)(accd[p * kGradCols + c] * pscale[p]);
    }
  }
}

// ---------------------------------------------------------------------------
// Dispatch tables
// ---------------------------------------------------------------------------
using TileFn = void (*)(const h8*, int64_t, const h8*, const void*, int64_t,
                        int64_t, int64_t, int64_t, int, float, float,
                        const uint32_t*, const float*, float*, float*, int64_t, int);

// Row tiles per wave: 4, or 2 where the register budget needs it (more than 16
// right-hand sides).
constexpr int rows_per_wave_tiles(int, int ncg) { return ncg >= 2 ? 2 : 4; }

template <int KIND, int NCG>
TileFn pick_kb(int kb) {
  switch (kb) {
    case 1: return k_fused_tile<KIND, 1, NCG, rows_per_wave_tiles(1, NCG)>;
    case 2: return k_fused_tile<KIND, 2, NCG, rows_per_wave_tiles(2, NCG)>;
    case 3: return k_fused_tile<KIND, 3, NCG, rows_per_wave_tiles(3, NCG)>;
  }
  return nullptr;
}

template <int KIND>
TileFn pick_tile(int kb, int ncg) {
  switch (ncg) {
    case 0: return pick_kb<KIND, 0>(kb);
    case 1: return pick_kb<KIND, 1>(kb);
    case 2: return pick_kb<KIND, 2>(kb);
    case 4: return pick_kb<KIND, 4>(kb);
  }
  return nullptr;
}

}  // namespace

void pack_points(const float* X_dev, int64_t n, const Coords& co,
                 PackedPoints& pp, hipStream_t st) {
  const int d = co.d;
  MGP_REQUIRE(d >= 1, "dimension must be >= 1");
  pp.n = n;
  pp.exp2_limit = co.exp2_limit;
  // Even tile count: the tile kernel walks column tiles in pairs.
  pp.ntiles = 2 * ceil_div(std::max<int64_t>(n, 1), 32);
  pp.ntiles_alloc = round_up(pp.ntiles, kPackTileAlign);
  // Beyond kMaxMfmaDim only the scaled coordinates are built (direct path).
  pp.kb = d <= kMaxMfmaDim ? split_mfma_count(d) : 0;
  const size_t sz = (size_t)pp.ntiles_alloc * std::max(pp.kb, 1) * 64 * 4;  // dwords
  pp.A.ensure(sz);
  pp.B.ensure(sz);
  pp.z.ensure((size_t)std::max<int64_t>(n, 1) * d);
  const int64_t threads = pp.ntiles_alloc * 16;
  uint32_t* mx = pp.max_norm_dev.ensure(1);
  hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(64), 0, st, mx, (int64_t)1, 0u);
  hipLaunchKernelGGL(k_pack_points, dim3((unsigned)ceil_div(threads, 256)),
                     dim3(256), 0, st, X_dev, n, d, co.coef.ptr, pp.kb,
                     pp.ntiles_alloc, reinterpret_cast<uint16_t*>(pp.A.ptr),
                     reinterpret_cast<uint16_t*>(pp.B.ptr), pp.z.ptr, mx);
  MGP_HIP_CHECK(hipGetLastError());
  uint32_t bits = 0;
  MGP_HIP_CHECK(hipMemcpyAsync(&bits, mx, sizeof(bits), hipMemcpyDeviceToHost, st));
  MGP_HIP_CHECK(hipStreamSynchronize(st));
  std::memcpy(&pp.max_norm, &bits, sizeof(bits));
}

namespace {

// Work-buffer source of one fused_matvec column chunk: the workspace's growable
// buffers, or 256-byte aligned slices of its fixed arena (reset per chunk; the
// chunks run in stream order, so a later chunk may reuse an earlier one's bytes).
struct ChunkBuffers {
  MatvecWorkspace& ws;
  size_t off = 0;
  explicit ChunkBuffers(MatvecWorkspace& w) : ws(w) {}
  size_t left() const { return ws.arena_bytes - off; }
  template <class T>
  T* take(DevBuf<T>& buf, size_t count) {
    if (ws.arena == nullptr) return buf.ensure(count);
    const size_t bytes = round_up((int64_t)std::max<size_t>(count, 1) * sizeof(T), 256);
    MGP_REQUIRE(bytes <= left(), "fused matvec work buffers exceed the fixed scratch arena");
    T* p = reinterpret_cast<T*>(ws.arena + off);
    off += bytes;
    return p;
  }
};

size_t rhs_pack_bytes(int64_t col_tiles, int ncg) {
  if (ncg == 0) return (size_t)round_up(col_tiles * 16 * 4, 256);
  return (size_t)round_up((int64_t)ncg * (col_tiles / 2) * 64 * 32, 256);
}

}  // namespace

size_t fused_matvec_min_arena(const PackedPoints& cols, int ncols) {
  const int nc = std::min(ncols, 64);
  const int ncg = nc == 1 ? 0 : (nc <= 16 ? 1 : (nc <= 32 ? 2 : 4));
  size_t b = rhs_pack_bytes(cols.ntiles, ncg);
  if (ncg > 0) b += 256 + (size_t)round_up(64 * 64 * 4, 256);
  return b;
}

namespace {

// Symmetric-route choice for one column chunk of nc right-hand sides.
bool sym_route(const MatvecArgs& a, const PackedPoints& rows, const PackedPoints& cols, int nc,
               const MatvecWorkspace& ws) {
  if (!a.square || a.mix != nullptr || ws.arena != nullptr || &rows != &cols) return false;
  if (nc < 1 || nc > 16 || a.m != a.n || a.n != rows.n) return false;
  const char* env = std::getenv("MGP_SYM_MATVEC");
  const int mode = env == nullptr ? -1 : (env[0] == '0' ? 0 : 1);
  if (mode == 0) return false;
  const int64_t nb = ceil_div(std::max<int64_t>(a.n, 1), kSymRows);
  if (nb * kSymRows > rows.ntiles_alloc * 16) return false;
  if (mode < 0 && nb < kSymMinBlocks) return false;
  const double tp_bytes = (double)nb * (double)(nb / 2) * kSymRows * 16 * 4;
  return tp_bytes <= kSymMaxBytes;
}

}  // namespace

bool symmetric_route_taken(const PackedPoints& pts, int ncols) {
  MatvecArgs a;
  a.square = true;
  a.m = a.n = pts.n;
  a.ncols = ncols;
  MatvecWorkspace ws;  // no fixed arena
  return pts.kb >= 1 && sym_route(a, pts, pts, ncols, ws);
}

namespace {

using SymFn = void (*)(const h8*, const h8*, const h8*, int64_t, int64_t, int64_t, int64_t,
                       int, const uint32_t*, float*, float*, int64_t);

template <int KIND>
SymFn pick_sym(int kb) {
  switch (kb) {
    case 1: return k_sym_tile<KIND, 1>;
    case 2: return k_sym_tile<KIND, 2>;
    case 3: return k_sym_tile<KIND, 3>;
  }
  return nullptr;
}

// Delta splits of the symmetric kernels (k_sym_tile, k_grad_sym).  They run
// one workgroup per CU; item L of the grid goes to XCD L / per (launch order
// deals workgroups to the XCDs in turn), and each XCD's CUs take its items in
// order as they free up.  A partly filled last round of items leaves CUs idle
// for up to one item, so the split count is chosen by simulating that
// dispatch: an item costs `stages` per delta plus about one stage of set-up
// (fitted to measured k_sym_tile launches at nb = 489: 5, 9, 12 and 35
// splits gave 3.81 to 3.87 us per simulated stage), and each split's partial
// sums (`split_bytes`) cost their extra read in the reduction (priced at 2 us
// per stage, a short stage, so the choice leans towards fewer splits).
// Cached per kernel, block count and device.
int64_t delta_splits(int64_t nb, int stages, const void* fn, int threads, double split_bytes) {
  static std::mutex mu;
  static std::unordered_map<std::string, int64_t> cache;
  int dev = 0;
  MGP_HIP_CHECK(hipGetDevice(&dev));
  const std::string key = std::to_string(reinterpret_cast<uintptr_t>(fn)) + ":" +
                          std::to_string(nb) + ":" + std::to_string(dev);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  MGP_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  MGP_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0));
  const int slots = std::max(1, cus * std::max(per_cu, 1) / kXcds);
  const int64_t hmax = nb / 2;
  constexpr double kStageUs = 2.0, kReduceBytesPerUs = 6.0e6;
  int64_t best_s = 1, last_dps = -1;
  double best = 0.0;
  for (int64_t s0 = 1; s0 <= std::min<int64_t>(hmax + 1, 64); ++s0) {
    const int64_t dps = ceil_div(hmax + 1, s0);
    if (dps == last_dps) continue;
    last_dps = dps;
    const int64_t splits = ceil_div(hmax + 1, dps);
    const int64_t items = nb * splits;
    const int64_t per = round_up(items, (int64_t)kXcds) / kXcds;
    double make = 0.0;
    for (int x = 0; x < kXcds; ++x) {
      std::priority_queue<double, std::vector<double>, std::greater<double>> cu;
      for (int i = 0; i < slots; ++i) cu.push(0.0);
      for (int64_t k = 0; k < per; ++k) {
        const int64_t L = x * per + k;
        if (L >= items) break;
        const int64_t b = L % nb, d0 = (L / nb) * dps;
        const int64_t d1 = std::min(d0 + dps, sym_span(b, nb) + 1);
        const double cost = (double)std::max<int64_t>(d1 - d0, 0) * stages + 1.0;
        const double t = cu.top();
        cu.pop();
        cu.push(t + cost);
      }
      while (cu.size() > 1) cu.pop();
      make = std::max(make, cu.top());
    }
    const double total = make + (double)splits * split_bytes / kReduceBytesPerUs / kStageUs;
    if (s0 == 1 || total < best - 1e-9) {
      best = total;
      best_s = splits;
    }
  }
  cache.emplace(key, best_s);
  return best_s;
}

// out = (K + noise I) V for nc <= 16 columns of V on the symmetric kernel.
void sym_matvec(const MatvecArgs& a, const PackedPoints& pts, const float* Vc, int nc,
                float* outc, MatvecWorkspace& ws, hipStream_t st) {
  const int64_t n = a.n;
  const int64_t nb = ceil_div(std::max<int64_t>(n, 1), kSymRows);
  const int64_t hmax = nb / 2;
  const int64_t pairs = nb * kSymPairs;
  const int64_t mpad = nb * kSymRows;

  uint32_t* colmax = ws.colmax.ensure(64);
  const int chunks = (int)std::min<int64_t>(ceil_div(std::max<int64_t>(n, 1), 4096), 64);
  uint32_t* cpart = ws.colmax_part.ensure((size_t)64 * chunks);
  const int vec4 = (n % 4 == 0 && reinterpret_cast<uintptr_t>(Vc) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_col_absmax_part, dim3((unsigned)chunks, (unsigned)nc), dim3(256), 0, st,
                     Vc, n, vec4, cpart);
  hipLaunchKernelGGL(k_col_absmax_final, dim3((unsigned)nc), dim3(64), 0, st, cpart, chunks,
                     colmax);
  const int64_t total = pairs * 64;  // 8-half vectors per part, one column group
  float* vp = ws.vpack.ensure((size_t)total * 2 * 4);
  hipLaunchKernelGGL(k_pack_rhs16, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st, Vc,
                     n, nc, 1, pairs, colmax, vec4, reinterpret_cast<h8*>(vp));
  MGP_HIP_CHECK(hipGetLastError());

  SymFn fn = a.kind == KIND_RBF        ? pick_sym<KIND_RBF>(pts.kb)
             : a.kind == KIND_MATERN32 ? pick_sym<KIND_MATERN32>(pts.kb)
                                       : pick_sym<KIND_MATERN52>(pts.kb);
  MGP_REQUIRE(fn != nullptr, "no symmetric tile kernel for this shape");
  int64_t splits = delta_splits(nb, kSymStages, reinterpret_cast<const void*>(fn),
                                64 * kSymWaves, (double)nb * kSymRows * 16 * 4);
  const int64_t dps = ceil_div(hmax + 1, splits);
  splits = ceil_div(hmax + 1, dps);
  float* fwd = ws.partial.ensure((size_t)splits * 16 * mpad);
  float* tp = ws.sym_tp.ensure((size_t)std::max<int64_t>(nb * hmax, 1) * kSymRows * 16);

  if (ws.time_tile) MGP_HIP_CHECK(hipEventRecord(ws.ev0, st));
  const int64_t items = round_up(nb * splits, kXcds);
  hipLaunchKernelGGL(fn, dim3((unsigned)items), dim3(64 * kSymWaves), 0, st,
                     reinterpret_cast<const h8*>(pts.B.ptr), reinterpret_cast<const h8*>(pts.A.ptr),
                     reinterpret_cast<const h8*>(vp), nb, splits, dps, hmax, nc, colmax, fwd, tp,
                     mpad);
  MGP_HIP_CHECK(hipGetLastError());
  if (ws.time_tile) {
    MGP_HIP_CHECK(hipEventRecord(ws.ev1, st));
    MGP_HIP_CHECK(hipEventSynchronize(ws.ev1));
    float ms = 0.f;
    MGP_HIP_CHECK(hipEventElapsedTime(&ms, ws.ev0, ws.ev1));
    ws.tile_ms += ms;
    ws.tile_calls += 1;
  }
  hipLaunchKernelGGL(k_sym_reduce, dim3((unsigned)ceil_div(4 * n, 256)), dim3(256), 0, st, fwd,
                     (int)splits, tp, nb, hmax, mpad, n, nc, a.outputscale, a.noise, Vc, outc);
  MGP_HIP_CHECK(hipGetLastError());
}

}  // namespace

// ---------------------------------------------------------------------------
// Matrix-core gradient trace: host side.
// ---------------------------------------------------------------------------
bool grad_trace_mfma_route(int kind, const PackedPoints& pts, int d) {
  const char* env = std::getenv("MGP_GRAD_MFMA");
  const int mode = env == nullptr ? -1 : (env[0] == '0' ? 0 : 1);
  if (mode == 0) return false;
  // d <= 16: one 16-dimension group of [z | z^2] (two groups spill registers).
  if (kind == KIND_MATERN12 || d < 1 || d > 16 || pts.kb < 1 || pts.kb > 3) return false;
  if (!gram_form_ok(kind, pts, pts)) return false;
  const int64_t nb = ceil_div(std::max<int64_t>(pts.n, 1), kGtRows);
  if (nb * kGtRows > pts.ntiles_alloc * 16) return false;
  return mode > 0 || pts.n >= kGradMfmaMinPoints;
}

namespace {

using GradFn = void (*)(const h8*, const h8*, const h8*, const h8*, const h8*, const float*, int,
                        int64_t, int64_t, int64_t, int64_t, double*);

template <int KIND, int QG>
GradFn pick_grad_kb(int kb) {
  switch (kb) {
    case 1: return k_grad_sym<KIND, 1, QG>;
    case 2: return k_grad_sym<KIND, 2, QG>;
    case 3: return k_grad_sym<KIND, 3, QG>;
  }
  return nullptr;
}

template <int KIND>
GradFn pick_grad(int kb, int qg) {
  return qg == 1 ? pick_grad_kb<KIND, 1>(kb) : nullptr;
}

}  // namespace

void grad_trace_mfma(int kind, const PackedPoints& pts, int d, const float* Lf,
                     const float* Rf, int ncols, double* acc, GradTraceWorkspace& ws,
                     hipStream_t st) {
  MGP_REQUIRE(grad_trace_mfma_route(kind, pts, d),
              "matrix-core gradient trace does not serve this point set");
  const int64_t n = pts.n;
  const int64_t nb = ceil_div(std::max<int64_t>(n, 1), kGtRows);
  const int64_t ntiles = nb * 16;
  const int64_t pairs = nb * kGtPairs;
  const int qg = d <= 16 ? 1 : 2;
  const int nq = 16 * qg;
  const int64_t hmax = nb / 2;
  GradFn fn = kind == KIND_RBF        ? pick_grad<KIND_RBF>(pts.kb, qg)
              : kind == KIND_MATERN32 ? pick_grad<KIND_MATERN32>(pts.kb, qg)
                                      : pick_grad<KIND_MATERN52>(pts.kb, qg);
  MGP_REQUIRE(fn != nullptr, "no gradient trace kernel for this shape");
  // Each split's per-item partials travel to the host over PCIe (~25 GB/s,
  // 240x slower than the HBM read the split model prices).
  int64_t splits = delta_splits(nb, kGtStages, reinterpret_cast<const void*>(fn), 64 * kGtWaves,
                                240.0 * (double)nb * (nq + 1) * sizeof(double));
  const int64_t dps = ceil_div(hmax + 1, splits);
  splits = ceil_div(hmax + 1, dps);
  const int64_t items = round_up(nb * splits, kXcds);

  h8* ZZ = reinterpret_cast<h8*>(ws.zz.ensure((size_t)pairs * 2 * qg * 2 * 64 * 4));
  h8* WA = reinterpret_cast<h8*>(ws.wa.ensure((size_t)ntiles * 2 * 64 * 4));
  h8* WB = reinterpret_cast<h8*>(ws.wb.ensure((size_t)ntiles * 2 * 64 * 4));
  uint32_t* colmax = ws.colmax.ensure(32);
  const int chunks = (int)std::min<int64_t>(ceil_div(std::max<int64_t>(n, 1), 4096), 64);
  uint32_t* cpart = ws.colmax_part.ensure((size_t)64 * chunks);
  int* shifts = ws.shifts.ensure(33);
  double* part = ws.part.ensure((size_t)nb * splits * (nq + 1));
  ws.hpart.resize((size_t)nb * splits * (nq + 1));

  const int64_t zthreads = pairs * 2 * qg * 64;
  hipLaunchKernelGGL(k_pack_grad_zz, dim3((unsigned)ceil_div(zthreads, 256)), dim3(256), 0, st,
                     pts.z.ptr, n, d, qg, pairs, ZZ);
  MGP_HIP_CHECK(hipGetLastError());

  for (int c0 = 0; c0 < ncols; c0 += 16) {
    const int nc = std::min(16, ncols - c0);
    const float* L = Lf + (int64_t)c0 * n;
    const float* Rr = Rf + (int64_t)c0 * n;
    const int vecL = (n % 4 == 0 && reinterpret_cast<uintptr_t>(L) % 16 == 0) ? 1 : 0;
    const int vecR = (n % 4 == 0 && reinterpret_cast<uintptr_t>(Rr) % 16 == 0) ? 1 : 0;
    hipLaunchKernelGGL(k_col_absmax_part, dim3((unsigned)chunks, (unsigned)nc), dim3(256), 0, st,
                       L, n, vecL, cpart);
    hipLaunchKernelGGL(k_col_absmax_final, dim3((unsigned)nc), dim3(64), 0, st, cpart, chunks,
                       colmax);
    hipLaunchKernelGGL(k_col_absmax_part, dim3((unsigned)chunks, (unsigned)nc), dim3(256), 0, st,
                       Rr, n, vecR, cpart);
    hipLaunchKernelGGL(k_col_absmax_final, dim3((unsigned)nc), dim3(64), 0, st, cpart, chunks,
                       colmax + 16);
    hipLaunchKernelGGL(k_grad_shifts, dim3(1), dim3(64), 0, st, colmax, nc, shifts);
    hipLaunchKernelGGL(k_pack_grad_w, dim3((unsigned)ceil_div(ntiles * 64, 256)), dim3(256), 0,
                       st, L, Rr, n, nc, ntiles, shifts, WA, WB);
    MGP_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(fn, dim3((unsigned)items), dim3(64 * kGtWaves), 0, st,
                       reinterpret_cast<const h8*>(pts.B.ptr), reinterpret_cast<const h8*>(pts.A.ptr),
                       WA, WB, ZZ, pts.z.ptr, d, n, nb, splits, dps, part);
    MGP_HIP_CHECK(hipGetLastError());
    int T = 0;
    MGP_HIP_CHECK(hipMemcpyAsync(&T, shifts + 32, sizeof(int), hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipMemcpyAsync(ws.hpart.data(), part, ws.hpart.size() * sizeof(double),
                                 hipMemcpyDeviceToHost, st));
    MGP_HIP_CHECK(hipStreamSynchronize(st));
    std::vector<double> sum(nq + 1, 0.0);
    for (int64_t it = 0; it < nb * splits; ++it)
      for (int q = 0; q <= nq; ++q) sum[q] += ws.hpart[(size_t)it * (nq + 1) + q];
    const double sm = std::ldexp(1.0, kGtMExp - T), so = std::ldexp(1.0, -T);
    for (int q = 0; q < d; ++q) acc[q] += sum[q] * sm;
    acc[d] += sum[nq] * so;
  }
}

void fused_matvec(const MatvecArgs& a, const PackedPoints& rows,
                  const PackedPoints& cols, const float* V_dev, float* out_dev,
                  MatvecWorkspace& ws, hipStream_t st, int force_splits) {
  MGP_REQUIRE(a.ncols >= 1, "ncols must be >= 1");
  MGP_REQUIRE(rows.kb == cols.kb && rows.kb >= 1 && rows.kb <= 3,
              "MFMA tile path supports input dimension <= 30");
  const int kb = rows.kb;
  const int64_t row_tiles = rows.ntiles, col_tiles = cols.ntiles;
  const int64_t mpad = row_tiles * 16;

  const bool mixing = a.mix != nullptr;
  if (mixing)
    MGP_REQUIRE(a.mix_T >= 1 && a.mix_T <= kMaxMixT && a.ncols % a.mix_T == 0,
                "task mixing needs ncols a multiple of T <= 16");
  // Column chunks of at most 64 right-hand sides per launch (whole task blocks
  // when mixing).
  const int chunk = mixing ? (64 / a.mix_T) * a.mix_T : 64;
  for (int c0 = 0; c0 < a.ncols; c0 += chunk) {
    const int nc = std::min(chunk, a.ncols - c0);
    const int ncg = nc == 1 ? 0 : (nc <= 16 ? 1 : (nc <= 32 ? 2 : 4));
    const int R = rows_per_wave_tiles(kb, ncg);
    const int cpad = ncg == 0 ? 1 : 16 * ncg;
    const float* Vc = V_dev + (int64_t)c0 * a.n;
    float* outc = out_dev + (int64_t)c0 * a.m;
    const float* Vin = a.square ? V_dev + (int64_t)c0 * a.m : nullptr;
    if (force_splits <= 0 && sym_route(a, rows, cols, nc, ws)) {
      sym_matvec(a, rows, Vc, nc, outc, ws, st);
      continue;
    }

    // Pack right-hand sides (or take the packing a previous product of the
    // same V made over the same column points).
    const int64_t col_pairs = col_tiles / 2;
    ChunkBuffers buf(ws);
    const void* vp;
    const uint32_t* colmax = nullptr;
    PackedRhs* share = (a.reuse != nullptr && a.ncols <= chunk && ncg > 0 && ws.arena == nullptr)
                           ? a.reuse : nullptr;
    if (share != nullptr && share->vp != nullptr && share->src == Vc &&
        share->col_tiles == col_tiles && share->ncols == nc) {
      vp = share->vp;
      colmax = share->colmax;
    } else if (ncg == 0) {
      const int64_t npad = col_tiles * 16;
      float* padded = buf.take(ws.vpack, (size_t)npad);
      hipLaunchKernelGGL(k_pad_vec, dim3((unsigned)ceil_div(npad, 256)), dim3(256),
                         0, st, Vc, a.n, npad, padded);
      vp = padded;
    } else {
      uint32_t* cm = buf.take(ws.colmax, 64);
      const int chunks = (int)std::min<int64_t>(ceil_div(std::max<int64_t>(a.n, 1), 4096), 64);
      uint32_t* cpart = buf.take(ws.colmax_part, (size_t)64 * chunks);
      const int vec4 = (a.n % 4 == 0 && reinterpret_cast<uintptr_t>(Vc) % 16 == 0) ? 1 : 0;
      hipLaunchKernelGGL(k_col_absmax_part, dim3((unsigned)chunks, (unsigned)nc), dim3(256), 0,
                         st, Vc, a.n, vec4, cpart);
      hipLaunchKernelGGL(k_col_absmax_final, dim3((unsigned)nc), dim3(64), 0, st, cpart, chunks,
                         cm);
      const int64_t total = (int64_t)ncg * col_pairs * 64;  // 8-half vectors per part
      float* packed = buf.take(ws.vpack, (size_t)total * 2 * 4);
      hipLaunchKernelGGL(k_pack_rhs16, dim3((unsigned)ceil_div(total, 256)), dim3(256),
                         0, st, Vc, a.n, nc, ncg, col_pairs, cm, vec4,
                         reinterpret_cast<h8*>(packed));
      vp = packed;
      colmax = cm;
      if (share != nullptr) {
        share->src = Vc;
        share->col_tiles = col_tiles;
        share->ncols = nc;
        share->vp = packed;
        share->colmax = cm;
      }
    }
    MGP_HIP_CHECK(hipGetLastError());

    // Grid: row blocks x j splits.  Aim for >= 2048 workgroups (1024 with 64
    // right-hand sides, whose waves carry 4x the work and whose split partials
    // cost 4x the traffic) so 256 CUs see several waves each, while every split
    // keeps >= 32 j tiles of work.
    const int64_t row_blocks = ceil_div(row_tiles, (int64_t)kWaves * R);
    const int64_t target_blocks = ncg >= 4 ? 1024 : 2048;
    int64_t splits = force_splits > 0 ? force_splits : 1;
    if (force_splits <= 0) {
      while (row_blocks * splits < target_blocks && col_pairs / (splits * 2) >= 16 &&
             splits < 64)
        splits *= 2;
    }
    if (ws.arena != nullptr && splits > 1) {
      // Fixed arena: as many splits as the remaining bytes hold partials for.
      const size_t per_split = (size_t)round_up((int64_t)cpad * mpad * 4, 256);
      const int64_t fit = (int64_t)(buf.left() / per_split);
      while (splits > 1 && splits > fit) splits /= 2;
    }
    const int64_t pairs_per_split = ceil_div(col_pairs, splits);
    splits = ceil_div(col_pairs, pairs_per_split);

    float* partial = nullptr;
    if (splits > 1 || mixing)
      partial = buf.take(ws.partial, (size_t)splits * cpad * mpad);

    MGP_REQUIRE(a.kind != KIND_MATERN12, "Matern-1/2 has no Gram-form tile path");
    TileFn fn = a.kind == KIND_RBF        ? pick_tile<KIND_RBF>(kb, ncg)
                : a.kind == KIND_MATERN32 ? pick_tile<KIND_MATERN32>(kb, ncg)
                                          : pick_tile<KIND_MATERN52>(kb, ncg);
    MGP_REQUIRE(fn != nullptr, "no tile kernel for this shape");
    const int64_t diag_shift = a.square ? 0 : (int64_t)1 << 40;
    if (ws.time_tile) MGP_HIP_CHECK(hipEventRecord(ws.ev0, st));
    hipLaunchKernelGGL(fn, dim3((unsigned)row_blocks, (unsigned)splits), dim3(256), 0,
                       st, reinterpret_cast<const h8*>(rows.B.ptr), row_tiles,
                       reinterpret_cast<const h8*>(cols.A.ptr), (const void*)vp, col_pairs,
                       pairs_per_split, diag_shift, a.m, nc, a.outputscale, a.noise,
                       colmax, Vin, outc, partial, mpad, cpad);
    MGP_HIP_CHECK(hipGetLastError());
    if (ws.time_tile) {
      MGP_HIP_CHECK(hipEventRecord(ws.ev1, st));
      MGP_HIP_CHECK(hipEventSynchronize(ws.ev1));
      float ms = 0.f;
      MGP_HIP_CHECK(hipEventElapsedTime(&ms, ws.ev0, ws.ev1));
      ws.tile_ms += ms;
      ws.tile_calls += 1;
    }
    if (mixing) {
      const int nblk = nc / a.mix_T;
      const int64_t tot = (int64_t)nblk * a.m;
      const bool q4 = a.m % 4 == 0 && mpad % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(outc) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(partial) % 16 == 0 &&
                      (Vin == nullptr || reinterpret_cast<uintptr_t>(Vin) % 16 == 0);
      if (q4)
        hipLaunchKernelGGL(k_reduce_mix4, dim3((unsigned)ceil_div(tot / 4, 256)), dim3(256), 0,
                           st, partial, (int)splits, cpad, mpad, a.m, nblk, a.mix_T,
                           a.outputscale, a.noise, a.square ? 1 : 0, Vin, a.mix,
                           a.mix_accumulate ? 1 : 0, outc);
      else
        hipLaunchKernelGGL(k_reduce_mix, dim3((unsigned)ceil_div(tot, 256)), dim3(256), 0, st,
                           partial, (int)splits, cpad, mpad, a.m, nblk, a.mix_T, a.outputscale,
                           a.noise, a.square ? 1 : 0, Vin, a.mix, a.mix_accumulate ? 1 : 0, outc);
      MGP_HIP_CHECK(hipGetLastError());
    } else if (splits > 1) {
      const int64_t tot = (int64_t)nc * a.m;
      const bool q4 = a.m % 4 == 0 && mpad % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(outc) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(partial) % 16 == 0 &&
                      (Vin == nullptr || reinterpret_cast<uintptr_t>(Vin) % 16 == 0);
      if (q4)
        hipLaunchKernelGGL(k_reduce_splits4, dim3((unsigned)ceil_div(tot / 4, 256)), dim3(256),
                           0, st, partial, (int)splits, cpad, mpad, a.m, nc, a.outputscale,
                           a.noise, a.square ? 1 : 0, Vin, outc);
      else
        hipLaunchKernelGGL(k_reduce_splits, dim3((unsigned)ceil_div(tot, 256)), dim3(256),
                           0, st, partial, (int)splits, cpad, mpad, a.m, nc,
                           a.outputscale, a.noise, a.square ? 1 : 0, Vin, outc);
      MGP_HIP_CHECK(hipGetLastError());
    }
  }
}

void direct_matvec(const MatvecArgs& a, const PackedPoints& rows,
                   const PackedPoints& cols, int d, const float* V_dev,
                   float* out_dev, hipStream_t st) {
  MGP_REQUIRE(d >= 1 && d <= 32, "direct path supports input dimension <= 32");
  for (int c0 = 0; c0 < a.ncols; c0 += kDirectMaxCols) {
    const int nc = std::min(kDirectMaxCols, a.ncols - c0);
    const size_t shm = (size_t)kDirectTile * (d + nc) * sizeof(float);
    const dim3 grid((unsigned)ceil_div(std::max<int64_t>(a.m, 1), 256));
    auto fn = a.kind == KIND_RBF        ? k_direct<KIND_RBF>
              : a.kind == KIND_MATERN12 ? k_direct<KIND_MATERN12>
              : a.kind == KIND_MATERN32 ? k_direct<KIND_MATERN32>
                                        : k_direct<KIND_MATERN52>;
    hipLaunchKernelGGL(fn, grid, dim3(256), shm, st, rows.z.ptr, a.m, cols.z.ptr,
                       a.n, d, V_dev + (int64_t)c0 * a.n, nc, a.outputscale,
                       a.noise, a.square ? 1 : 0, cols.exp2_limit, out_dev + (int64_t)c0 * a.m);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

void fill_cross(int kind, float outputscale, const PackedPoints& rows, int64_t r0,
                int64_t nrows, const PackedPoints& cols, int d, float* out, hipStream_t st) {
  MGP_REQUIRE(r0 >= 0 && nrows >= 0 && r0 + nrows <= rows.n, "cross block out of range");
  const int64_t total = nrows * cols.n;
  if (total == 0) return;
  auto fn = kind == KIND_RBF        ? k_fill_cross<KIND_RBF>
            : kind == KIND_MATERN12 ? k_fill_cross<KIND_MATERN12>
            : kind == KIND_MATERN32 ? k_fill_cross<KIND_MATERN32>
                                    : k_fill_cross<KIND_MATERN52>;
  hipLaunchKernelGGL(fn, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st, rows.z.ptr,
                     r0, nrows, cols.z.ptr, cols.n, d, outputscale, cols.exp2_limit, out);
  MGP_HIP_CHECK(hipGetLastError());
}

void fill_dense_half(int kind, float outputscale, const PackedPoints& pts, int d, int shift,
                     int64_t nb, uint32_t* half, hipStream_t st) {
  MGP_REQUIRE(d >= 1 && pts.n >= 1, "dense fill needs points");
  MGP_REQUIRE(d <= kFillLdsMaxD, "dense fill supports input dimension <= 32");
  const int64_t nblocks = nb * (nb + 1) / 2;
  auto fn = kind == KIND_RBF        ? k_fill_half_lds<KIND_RBF>
            : kind == KIND_MATERN12 ? k_fill_half_lds<KIND_MATERN12>
            : kind == KIND_MATERN32 ? k_fill_half_lds<KIND_MATERN32>
                                    : k_fill_half_lds<KIND_MATERN52>;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3(256),
                     (size_t)2 * d * kHalfRows * sizeof(float), st, pts.z.ptr, pts.n, d,
                     outputscale, pts.exp2_limit, shift, nb, half);
  MGP_HIP_CHECK(hipGetLastError());
}

void gradient_matvec(int kind, bool ard, const PackedPoints& pts, int d, float outputscale,
                     const float* pscale_dev, const float* V_dev, int ncols, float* out_dev,
                     hipStream_t st) {
  MGP_REQUIRE(d >= 1 && d <= kGradMaxDim, "gradient products support input dimension <= 32");
  MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
  const int64_t n = pts.n;
  const size_t shm = (size_t)kGradTile * (d + kGradCols) * sizeof(float);
  const dim3 grid((unsigned)ceil_div(std::max<int64_t>(n, 1), 256));
  using Fn = void (*)(const float*, int64_t, int, const float*, int, int, float, float,
                      const float*, float*);
  Fn fn;
  if (kind == KIND_RBF) fn = ard ? k_grad_matvec<KIND_RBF, true> : k_grad_matvec<KIND_RBF, false>;
  else if (kind == KIND_MATERN12)
    fn = ard ? k_grad_matvec<KIND_MATERN12, true> : k_grad_matvec<KIND_MATERN12, false>;
  else if (kind == KIND_MATERN32)
    fn = ard ? k_grad_matvec<KIND_MATERN32, true> : k_grad_matvec<KIND_MATERN32, false>;
  else fn = ard ? k_grad_matvec<KIND_MATERN52, true> : k_grad_matvec<KIND_MATERN52, false>;
  for (int c0 = 0; c0 < ncols; c0 += kGradCols) {
    hipLaunchKernelGGL(fn, grid, dim3(256), shm, st, pts.z.ptr, n, d, V_dev, ncols, c0,
                       outputscale, pts.exp2_limit, pscale_dev, out_dev);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace mgp
