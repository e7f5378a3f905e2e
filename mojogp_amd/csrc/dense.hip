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

#include <algorithm>
#include <cmath>

namespace mgp {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16 __attribute__((ext_vector_type(16)));

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

__global__ void k_zero_u32(uint32_t* __restrict__ p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0u;
}

// dst[r * gpr + g] = split of 2^shift src[r * n + 8 g + e], e = 0..7 (zero
// past n), for r < nrows, g < gpr.  vec4: n a multiple of 4 (16-byte rows).
__global__ void k_dense_pack(const float* __restrict__ src, int64_t nrows, int64_t n,
                             int64_t gpr, int shift, int vec4, h16* __restrict__ dst) {
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
  dst[idx] = split16(x);
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

// Vp[c * gpr + g] = split of 2^s_c V[c][8 g + e] (zero for c >= ncols or past
// n), s_c from the column maximum.
__global__ void k_dense_pack_rhs(const float* __restrict__ V, int64_t n, int ncols, int cpad,
                                 int64_t gpr, const uint32_t* __restrict__ colmax, int vec4,
                                 h16* __restrict__ Vp) {
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
  Vp[idx] = split16(x);
}

// D = K V over the column groups [g0, g1) of split blockIdx.z (4 groups = 32
// columns of K per step).  Wave (wr, wc) of the block computes R row tiles x
// NCT column tiles of 16: rows i0 + 16 r + m, right-hand sides c0 + 16 ct + n.
// v_mfma_f32_16x16x32_f16 operands come straight from global memory in MFMA
// layout: lane l holds K[i0 + 16 r + l%16][8 (g + l/16) .. + 7] (A, both
// parts in one 32-byte load) and V[c0 + 16 ct + l%16][same columns] (B).  Each
// tile accumulates Kh.Vh + Kh.Vl + Kl.Vh.  The loads of the next step are
// issued before this step's MFMAs (two register stages; the address of the
// prefetch is clamped into the split so no load is conditional).  DIRECT
// (one split): out[c][i] = 2^-(kshift + s_c) D + noise V[c][i] for i < n,
// c < ncols; otherwise part[(z cpad + c) npad + i] = D.
template <int R, int NCT, int WR, bool DIRECT>
__global__ __launch_bounds__(256) void k_dense_mm(
    const h16* __restrict__ Kp, int64_t gpr, const h16* __restrict__ Vp, int64_t gsplit,
    int64_t npad, int cpad, float* __restrict__ part, int64_t n, int ncols, int kshift,
    const uint32_t* __restrict__ colmax, float noise, const float* __restrict__ V,
    float* __restrict__ out) {
  constexpr int WC = 4 / WR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave % WR, wc = wave / WR;
  const int lm = lane & 15, lq = lane >> 4;
  const int64_t i0 = ((int64_t)blockIdx.x * WR + wr) * (R * 16);
  const int c0 = (blockIdx.y * WC + wc) * (NCT * 16);
  const int64_t g0 = (int64_t)blockIdx.z * gsplit, g1 = min(gpr, g0 + gsplit);
  const h16* ka[R];
#pragma unroll
  for (int r = 0; r < R; ++r) ka[r] = Kp + (i0 + 16 * r + lm) * gpr + lq;
  const h16* vb[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) vb[ct] = Vp + (int64_t)(c0 + 16 * ct + lm) * gpr + lq;
  f4 acc[R][NCT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[r][ct] = f4{0.f, 0.f, 0.f, 0.f};
  auto load = [&](int64_t g, h16 (&a)[R], h16 (&b)[NCT]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) a[r] = ka[r][g];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) b[ct] = vb[ct][g];
  };
  auto mma = [&](const h16 (&a)[R], const h16 (&b)[NCT]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const h8 ah = first8(a[r]), al = last8(a[r]);  // hi, lo parts
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const h8 bh = first8(b[ct]), bl = last8(b[ct]);
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc[r][ct], 0, 0, 0);
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc[r][ct], 0, 0, 0);
        acc[r][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc[r][ct], 0, 0, 0);
      }
    }
  };
  if (g0 < g1) {
    const int64_t glast = g1 - 4;  // (g1 - g0) is a multiple of 4
    h16 a0[R], b0[NCT], a1[R], b1[NCT];
    load(g0, a0, b0);
    for (int64_t g = g0; g < g1; g += 8) {
      load(min(g + 4, glast), a1, b1);
      mma(a0, b0);
      if (g + 4 >= g1) break;
      load(min(g + 8, glast), a0, b0);
      mma(a1, b1);
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
  const int64_t pad = (K.npad - n) * gpr * 8;
  if (pad > 0) {
    hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)ceil_div(pad, 256)), dim3(256), 0, st,
                       K.data.ptr + (size_t)n * gpr * 8, pad);
    MGP_HIP_CHECK(hipGetLastError());
  }
}

void dense_pack_rows(const float* rows, int64_t r0, int64_t nrows, DenseK& K, hipStream_t st) {
  MGP_REQUIRE(r0 >= 0 && nrows >= 0 && r0 + nrows <= K.n, "dense K rows out of range");
  if (nrows == 0) return;
  const int64_t gpr = K.groups_per_row();
  const int64_t total = nrows * gpr;
  const int vec4 = (K.n % 4 == 0 && reinterpret_cast<uintptr_t>(rows) % 16 == 0) ? 1 : 0;
  h16* dst = reinterpret_cast<h16*>(K.data.ptr) + r0 * gpr;
  hipLaunchKernelGGL(k_dense_pack, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st, rows,
                     nrows, K.n, gpr, K.shift, vec4, dst);
  MGP_HIP_CHECK(hipGetLastError());
}

void dense_forward(const DenseK& K, const float* V, int ncols, float noise, float* out,
                   DenseWorkspace& w, hipStream_t st) {
  MGP_REQUIRE(ncols >= 1, "ncols must be >= 1");
  const int64_t n = K.n, npad = K.npad, gpr = K.groups_per_row();
  // block shape: rows x right-hand sides per workgroup
  int R = 4, NCT, WR;
  if (ncols <= 16) { NCT = 1; WR = 4; }
  else if (ncols <= 32) { NCT = 2; WR = 4; }
  else if (ncols <= 64) { NCT = 4; WR = 4; }
  else { NCT = 4; WR = 2; }
  const int WC = 4 / WR;
  const int64_t brows = (int64_t)WR * R * 16, bcols = (int64_t)WC * NCT * 16;
  const int cpad = (int)round_up(ncols, bcols);
  const int64_t rblocks = npad / brows, cblocks = cpad / bcols;

  // column maxima and packed right-hand sides
  const int chunks = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(n, 4096)));
  uint32_t* cpart = w.colmax_part.ensure((size_t)chunks * ncols);
  uint32_t* colmax = w.colmax.ensure((size_t)ncols);
  hipLaunchKernelGGL(k_dense_absmax_part, dim3((unsigned)chunks, (unsigned)ncols), dim3(256), 0,
                     st, V, n, cpart);
  hipLaunchKernelGGL(k_dense_absmax_final, dim3((unsigned)ncols), dim3(64), 0, st, cpart, chunks,
                     colmax);
  const int64_t vtot = (int64_t)cpad * gpr;
  h16* vp = reinterpret_cast<h16*>(w.vpack.ensure((size_t)vtot * 8));
  const int vec4 = (n % 4 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(k_dense_pack_rhs, dim3((unsigned)ceil_div(vtot, 256)), dim3(256), 0, st, V,
                     n, ncols, cpad, gpr, colmax, vec4, vp);
  MGP_HIP_CHECK(hipGetLastError());

  // splits of the K columns: >= 2048 workgroups while every split keeps >= 32
  // groups (256 columns of K)
  int64_t splits = 1;
  while (rblocks * cblocks * splits < 2048 && gpr / (splits * 2) >= 32 && splits < 64) splits *= 2;
  const int64_t gsplit = round_up(ceil_div(gpr, splits), 4);
  splits = ceil_div(gpr, gsplit);
  float* part = nullptr;
  if (splits > 1) part = w.part.ensure((size_t)splits * cpad * npad);
  const h16* kp = reinterpret_cast<const h16*>(K.data.ptr);
  const dim3 grid((unsigned)rblocks, (unsigned)cblocks, (unsigned)splits);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, kp, gpr, vp, gsplit, npad, cpad, part, n,
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
