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
//   1. S^T = A_j . B_i   (v_mfma_f32_16x16x4f32 over the augmented coordinates)
//      yields the scaled squared distance |z_i - z_j|^2 directly (Gram form with
//      the norms folded into two extra K slots);
//   2. the kernel value is formed in registers (RBF: med3 + exp2;
//      Matern-5/2: sqrt, min, exp2, two FMAs, one multiply);
//   3. O^T += V^T . P^T  (four more 16x16x4 MFMAs per 16 right-hand sides).
// K never touches HBM.  Accumulators are flushed into fp64 every 256 columns so
// the long N-term sums keep ~1e-7 relative accuracy.
#include "matvec.h"

#include <algorithm>
#include <vector>

namespace mgp {

typedef float f4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWaves = 4;           // waves per workgroup
constexpr int kFlushTiles = 16;     // j tiles between fp64 flushes
constexpr float kM52A = 0.69314718055994530942f;                     // ln 2
constexpr float kM52B = 0.69314718055994530942f * 0.69314718055994530942f / 3.0f;

// kExp2Clamp held in a VGPR (hoisted out of the hot loop by the caller).
__device__ __forceinline__ float clamp_reg() {
  float c = kExp2Clamp;
  asm volatile("" : "+v"(c));
  return c;
}

// Kernel value from the scaled squared distance s (see kernel_scale()).
// clampv = kExp2Clamp (from clamp_reg() in hot loops).
template <int KIND>
__device__ __forceinline__ float kval(float s, float clampv = kExp2Clamp) {
  if constexpr (KIND == KIND_RBF) {
    // os * exp(max(-0.5 r^2, -20)) = os * 2^-clamp(s, 0, 20 log2 e)
    const float t = __builtin_amdgcn_fmed3f(s, 0.0f, kExp2Clamp);
    return __builtin_amdgcn_exp2f(-t);
  } else {
    // os * (1 + sqrt5 r + 5/3 r^2) * exp(max(-sqrt5 r, -20)),  u = sqrt5 r log2 e
    // max(s, 0) as a signed-integer max of the bit pattern: one VALU op and no
    // NaN canonicalization of the MFMA result.
    const float sc = __builtin_bit_cast(float, max(__builtin_bit_cast(int, s), 0));
    const float u = __builtin_amdgcn_sqrtf(sc);
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
__global__ void k_pack_points(const float* __restrict__ X, int64_t n, int d,
                              const float* __restrict__ coef, int kk,
                              int64_t ntiles, float* __restrict__ A,
                              float* __restrict__ B, float* __restrict__ Z) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntiles * 16) return;
  const int li = (int)(i & 15);
  const int64_t tile = i >> 4;
  const int ka = kk * 4;
  float nrm = 0.0f;
  const bool real = i < n;
  for (int k = 0; k < ka; ++k) {
    float a = 0.0f, b = 0.0f;
    if (k < d) {
      float z = 0.0f;
      if (real) {
        z = (X[i * d + k] - coef[k]) * coef[d + k];
        Z[i * d + k] = z;
      }
      nrm = fmaf(z, z, nrm);
      a = z;
      b = -2.0f * z;
    } else if (k == d) {
      a = nrm;
      b = 1.0f;
    } else if (k == d + 1) {
      a = 1.0f;
      b = nrm;
    }
    const int64_t off = ((tile * kk + (k >> 2)) * 64) + li + 16 * (k & 3);
    A[off] = a;
    B[off] = b;
  }
}

// packV[g][jt][lane][q] = V[c = 16g + lane%16][j = 16 jt + 4 (lane/16) + q]
__global__ void k_pack_rhs(const float* __restrict__ V, int64_t n, int ncols,
                           int ncg, int64_t ntiles, float* __restrict__ P) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
  const int64_t total = (int64_t)ncg * ntiles * 64;
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  const int64_t jt = (idx >> 6) % ntiles;
  const int g = (int)((idx >> 6) / ntiles);
  const int c = 16 * g + (lane & 15);
  const int64_t j0 = 16 * jt + 4 * (lane >> 4);
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (c < ncols) {
    const float* col = V + (int64_t)c * n;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = (j0 + q < n) ? col[j0 + q] : 0.0f;
  }
  reinterpret_cast<f4*>(P)[idx] = v;
}

// Single right-hand side: zero padded copy.
__global__ void k_pad_vec(const float* __restrict__ V, int64_t n, int64_t npad,
                          float* __restrict__ P) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < npad) P[j] = j < n ? V[j] : 0.0f;
}

// ---------------------------------------------------------------------------
// MFMA tile kernel
//   NCG > 0 : NCG groups of 16 right-hand sides accumulated on MFMA
//   NCG == 0: one right-hand side accumulated on VALU
//   R       : 16-row tiles per wave
// grid = (row blocks, splits); each block covers kWaves*R row tiles and the
// j-tile range [blockIdx.y*jt_per_split, ...).  If `partial` is set, raw sums
// are written to partial[(split*cpad + c)*mpad + i]; otherwise the epilogue
// applies os and the noise diagonal and writes out[c*m + i].
// ---------------------------------------------------------------------------
template <int KIND, int KK, int NCG, int R>
__global__ __launch_bounds__(256) void k_fused_tile(
    const float* __restrict__ Bi, int64_t row_tiles, const float* __restrict__ Aj,
    const float* __restrict__ Vp, int64_t col_tiles, int64_t jt_per_split,
    int64_t diag_shift, int64_t m, int ncols, float os, float noise,
    const float* __restrict__ Vin, float* __restrict__ out,
    float* __restrict__ partial, int64_t mpad, int cpad) {
  const int lane = threadIdx.x & 63;
  // Wave index made wave-uniform (SGPR) so the j-loop bounds stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t tile0 = ((int64_t)blockIdx.x * kWaves + wave) * R;
  if (tile0 >= row_tiles) return;  // whole wave idle (no barriers used)

  float bi[R][KK];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t it = tile0 + r;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      bi[r][kk] = (it < row_tiles) ? Bi[(it * KK + kk) * 64 + lane] : 0.0f;
  }

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

  // Lane holds S^T[j = 4(lane/16)+q][i = lane%16] of a 16x16 tile.
  const int li = lane & 15;
  const int lj = 4 * (lane >> 4);

  // One j tile against the wave's R row tiles.  MASK restores the exact zero
  // self-distance on diagonal tiles (Gram-form cancellation guard).
  auto step = [&](int64_t jt, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    float aj[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) aj[kk] = Aj[(jt * KK + kk) * 64 + lane];
    f4 vj[G];
    if constexpr (NCG > 0) {
#pragma unroll
      for (int g = 0; g < NCG; ++g)
        vj[g] = reinterpret_cast<const f4*>(Vp)[(g * col_tiles + jt) * 64 + lane];
    } else {
      vj[0] = *reinterpret_cast<const f4*>(Vp + 16 * jt + lj);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        s = __builtin_amdgcn_mfma_f32_16x16x4f32(aj[kk], bi[r][kk], s, 0, 0, 0);
      if constexpr (MASK) {
        if (jt == tile0 + r + diag_shift) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (li == lj + q) s[q] = 0.0f;
        }
      }
      float p[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) p[q] = kval<KIND>(s[q], clampv);
      if constexpr (NCG > 0) {
#pragma unroll
        for (int g = 0; g < NCG; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x4f32(vj[g][q], p[q],
                                                             acc[r][g], 0, 0, 0);
      } else {
        float a = acc1[r];
#pragma unroll
        for (int q = 0; q < 4; ++q) a = fmaf(p[q], vj[0][q], a);
        acc1[r] = a;
      }
    }
  };
  auto flush = [&]() {
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
  // Plain tiles in chunks of kFlushTiles (no branch in the hot loop), then the
  // diagonal tiles with the mask.
  auto run = [&](int64_t a, int64_t b) {
    for (int64_t c0 = a; c0 < b; c0 += kFlushTiles) {
      const int64_t e = min(b, c0 + kFlushTiles);
      for (int64_t jt = c0; jt < e; ++jt) step(jt, std::false_type{});
      flush();
    }
  };

  const int64_t jt_begin = (int64_t)blockIdx.y * jt_per_split;
  const int64_t jt_end = min(col_tiles, jt_begin + jt_per_split);
  const int64_t dlo = tile0 + diag_shift, dhi = dlo + R;
  run(jt_begin, min(jt_end, dlo));
  run(max(jt_begin, dhi), jt_end);
  for (int64_t jt = max(jt_begin, dlo); jt < min(jt_end, dhi); ++jt) step(jt, std::true_type{});
  flush();

  // Epilogue.
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t it = tile0 + r;
    if (it >= row_tiles) continue;
    if constexpr (NCG > 0) {
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const double tot = accd[r][g][q] + (double)acc[r][g][q];
          const int c = 16 * g + lj + q;
          const int64_t i = 16 * it + li;
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
    float noise, int add_noise, float* __restrict__ out) {
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
      const float kv = kval<KIND>(r2);
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

// ---------------------------------------------------------------------------
// Dispatch tables
// ---------------------------------------------------------------------------
using TileFn = void (*)(const float*, int64_t, const float*, const float*,
                        int64_t, int64_t, int64_t, int64_t, int, float, float,
                        const float*, float*, float*, int64_t, int);

template <int KIND, int NCG, int R>
TileFn pick_kk(int kk) {
  switch (kk) {
    case 1: return k_fused_tile<KIND, 1, NCG, R>;
    case 2: return k_fused_tile<KIND, 2, NCG, R>;
    case 3: return k_fused_tile<KIND, 3, NCG, R>;
    case 4: return k_fused_tile<KIND, 4, NCG, R>;
    case 5: return k_fused_tile<KIND, 5, NCG, R>;
    case 6: return k_fused_tile<KIND, 6, NCG, R>;
    case 7: return k_fused_tile<KIND, 7, NCG, R>;
    case 8: return k_fused_tile<KIND, 8, NCG, R>;
  }
  return nullptr;
}

template <int KIND>
TileFn pick_tile(int kk, int ncg) {
  switch (ncg) {
    case 0: return pick_kk<KIND, 0, 4>(kk);
    case 1: return pick_kk<KIND, 1, 4>(kk);
    case 2: return pick_kk<KIND, 2, 4>(kk);
    case 4: return pick_kk<KIND, 4, 2>(kk);
  }
  return nullptr;
}

int rows_per_wave_tiles(int ncg) { return ncg == 4 ? 2 : 4; }

}  // namespace

void pack_points(const float* X_dev, int64_t n, const Coords& co,
                 PackedPoints& pp, hipStream_t st) {
  const int d = co.d;
  MGP_REQUIRE(d >= 1, "dimension must be >= 1");
  pp.n = n;
  pp.ntiles = ceil_div(std::max<int64_t>(n, 1), 16);
  pp.kk = (int)ceil_div(d + 2, 4);
  const size_t sz = (size_t)pp.ntiles * pp.kk * 64;
  pp.A.ensure(sz);
  pp.B.ensure(sz);
  pp.z.ensure((size_t)std::max<int64_t>(n, 1) * d);
  const int64_t threads = pp.ntiles * 16;
  hipLaunchKernelGGL(k_pack_points, dim3((unsigned)ceil_div(threads, 256)),
                     dim3(256), 0, st, X_dev, n, d, co.coef.ptr, pp.kk,
                     pp.ntiles, pp.A.ptr, pp.B.ptr, pp.z.ptr);
  MGP_HIP_CHECK(hipGetLastError());
}

void fused_matvec(const MatvecArgs& a, const PackedPoints& rows,
                  const PackedPoints& cols, const float* V_dev, float* out_dev,
                  MatvecWorkspace& ws, hipStream_t st, int force_splits) {
  MGP_REQUIRE(a.ncols >= 1, "ncols must be >= 1");
  MGP_REQUIRE(rows.kk == cols.kk && rows.kk >= 1 && rows.kk <= 8,
              "MFMA tile path supports input dimension <= 30");
  const int kk = rows.kk;
  const int64_t row_tiles = rows.ntiles, col_tiles = cols.ntiles;
  const int64_t mpad = row_tiles * 16;

  // Column chunks of at most 64 right-hand sides per launch.
  for (int c0 = 0; c0 < a.ncols; c0 += 64) {
    const int nc = std::min(64, a.ncols - c0);
    const int ncg = nc == 1 ? 0 : (nc <= 16 ? 1 : (nc <= 32 ? 2 : 4));
    const int R = rows_per_wave_tiles(ncg);
    const int cpad = ncg == 0 ? 1 : 16 * ncg;
    const float* Vc = V_dev + (int64_t)c0 * a.n;
    float* outc = out_dev + (int64_t)c0 * a.m;
    const float* Vin = a.square ? V_dev + (int64_t)c0 * a.m : nullptr;

    // Pack right-hand sides.
    float* vp;
    if (ncg == 0) {
      const int64_t npad = col_tiles * 16;
      vp = ws.vpack.ensure((size_t)npad);
      hipLaunchKernelGGL(k_pad_vec, dim3((unsigned)ceil_div(npad, 256)), dim3(256),
                         0, st, Vc, a.n, npad, vp);
    } else {
      const int64_t total = (int64_t)ncg * col_tiles * 64;
      vp = ws.vpack.ensure((size_t)total * 4);
      hipLaunchKernelGGL(k_pack_rhs, dim3((unsigned)ceil_div(total, 256)), dim3(256),
                         0, st, Vc, a.n, nc, ncg, col_tiles, vp);
    }
    MGP_HIP_CHECK(hipGetLastError());

    // Grid: row blocks x j splits.  Aim for >= 2048 workgroups so 256 CUs see
    // several waves each, while every split keeps >= 32 j tiles of work.
    const int64_t row_blocks = ceil_div(row_tiles, (int64_t)kWaves * R);
    int64_t splits = force_splits > 0 ? force_splits : 1;
    if (force_splits <= 0) {
      while (row_blocks * splits < 2048 && col_tiles / (splits * 2) >= 32 &&
             splits < 64)
        splits *= 2;
    }
    const int64_t jt_per_split = ceil_div(col_tiles, splits);
    splits = ceil_div(col_tiles, jt_per_split);

    float* partial = nullptr;
    if (splits > 1)
      partial = ws.partial.ensure((size_t)splits * cpad * mpad);

    TileFn fn = a.kind == KIND_RBF ? pick_tile<KIND_RBF>(kk, ncg)
                                   : pick_tile<KIND_MATERN52>(kk, ncg);
    MGP_REQUIRE(fn != nullptr, "no tile kernel for this shape");
    const int64_t diag_shift = a.square ? 0 : (int64_t)1 << 40;
    if (ws.time_tile) MGP_HIP_CHECK(hipEventRecord(ws.ev0, st));
    hipLaunchKernelGGL(fn, dim3((unsigned)row_blocks, (unsigned)splits), dim3(256), 0,
                       st, rows.B.ptr, row_tiles, cols.A.ptr, vp, col_tiles,
                       jt_per_split, diag_shift, a.m, nc, a.outputscale, a.noise,
                       Vin, outc, partial, mpad, cpad);
    MGP_HIP_CHECK(hipGetLastError());
    if (ws.time_tile) {
      MGP_HIP_CHECK(hipEventRecord(ws.ev1, st));
      MGP_HIP_CHECK(hipEventSynchronize(ws.ev1));
      float ms = 0.f;
      MGP_HIP_CHECK(hipEventElapsedTime(&ms, ws.ev0, ws.ev1));
      ws.tile_ms += ms;
      ws.tile_calls += 1;
    }
    if (splits > 1) {
      const int64_t tot = (int64_t)nc * a.m;
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
    auto fn = a.kind == KIND_RBF ? k_direct<KIND_RBF> : k_direct<KIND_MATERN52>;
    hipLaunchKernelGGL(fn, grid, dim3(256), shm, st, rows.z.ptr, a.m, cols.z.ptr,
                       a.n, d, V_dev + (int64_t)c0 * a.n, nc, a.outputscale,
                       a.noise, a.square ? 1 : 0, out_dev + (int64_t)c0 * a.m);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace mgp
