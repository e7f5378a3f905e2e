// Composite kernel trees (sums, products and scales of stationary leaves,
// each leaf on its own subset of the input dimensions) evaluated per pair
// from raw coordinate differences.
//
// Reference semantics (caspbian/mojogp):
//   leaf expressions      codegen_engine/expressions.py:77-380 (RBF, Matern
//                         1/2, 3/2, 5/2, periodic, RQ)
//   guards                codegen_engine/passes/numerical_stability.py:29-85
//                         (sqrt(max(x, 1e-20)); exp(max(x, -20)) where the
//                         emitted exponent matches its syntactic test: the
//                         Matern-3/2 and 5/2 leaves and ARD Matern-1/2 leaves,
//                         not RBF, isotropic Matern-1/2 or periodic leaves;
//                         exp2_limit in mgp_common.h)
//   engine param layout   mojogp/kernel.py:462-640 (leaves in tree order,
//                         a scale's factor after its subtree)
//
// A leaf's parameters start at p0:
//   RBF / Matern     [ls | ls_0..ls_{q-1}], os
//   RQ               [ls | ls_0..ls_{q-1}], alpha, os
//   periodic         [ls | ls_0..ls_{q-1}], period, os
//   linear           [variance | var_0..var_{q-1}], os:
//                    os * var * x.x'  |  os * sum_q var_q x_q x'_q
//   polynomial       [variance | var_0..var_{q-1}], degree, offset, os:
//                    os * (var * x.x' + offset)^D (ARD: sum_q var_q x_q x'_q),
//                    D the leaf's fixed integer degree (deg field); the
//                    degree parameter slot is carried but not read
//                    (expressions.py:57-71, 327-421)
//   categorical      no parameters: the leaf value is R[l_i][l_j] of an L x L
//                    correlation table (L in the leaf's ard field) stored at
//                    table offset p0 after the nparams parameters; the leaf's
//                    one dimension holds the level index as a float
//                    (the reference's mixed kernels,
//                    codegen_engine/expressions.py:493-516, cat_k symbols).
// Nodes are listed children first; the last node is the root.
#pragma once

#include "mgp_common.h"

namespace mgp {

constexpr int kTreeMaxLeaves = 8;
constexpr int kTreeMaxNodes = 16;
constexpr int kTreeMaxDims = 64;    // sum over leaves of their dimension counts
constexpr int kTreeMaxParams = 48;
constexpr int kTreeMaxInputDim = 32;
constexpr int kTreeMaxLevels = 32;     // categorical levels per leaf
constexpr int kTreeMaxTable = 1024;    // correlation-table entries over all leaves
constexpr int kTreeMaxCatRow = 64;     // sum over categorical leaves of their levels

// Leaf families beyond the radial kinds of mgp_common.h.
constexpr int KIND_RQ = 4;
constexpr int KIND_PERIODIC = 5;
constexpr int KIND_CAT = 6;
constexpr int KIND_LINEAR = 7;
constexpr int KIND_POLY = 8;
// Provider kind reported for composite kernel trees.
constexpr int KIND_TREE = -1;

enum TreeCode : int { TN_LEAF = 0, TN_ADD = 1, TN_MUL = 2, TN_SCALE = 3 };

struct TreeLeaf {
  int kind, ard, ndim, dim_off, p0;
  int deg;  // polynomial degree (KIND_POLY)
};
// LEAF: a = leaf index; ADD / MUL: a, b = child nodes; SCALE: a = child node,
// b = index of the scale factor in the parameter vector.
struct TreeNode {
  int code, a, b;
};

struct KernelTree {
  int d = 0, nparams = 0, nleaves = 0, nnodes = 0;
  int table_size = 0;  // categorical table entries after the parameters
  int ncat = 0;        // categorical leaves
  int nonstationary = 0;  // linear / polynomial leaves: k(x, x) varies with x
  TreeLeaf leaf[kTreeMaxLeaves];
  TreeNode node[kTreeMaxNodes];
  int dims[kTreeMaxDims];
};

// Flat spec (the C ABI's form): [d, nparams, nleaves, nnodes,
//   per leaf: kind, ard, ndim, p0, dims[ndim] ...,
//   per node: code, a, b ...].  Throws on malformed specs.
KernelTree parse_kernel_tree(const int* spec, int len);
// k(x, x) at the given parameters (all leaves are stationary).
double tree_diag(const KernelTree& t, const float* params);

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)
constexpr float kTreePi = 3.14159265358979323846f;
// Every evaluator of a tree (the run-time compiled products of tree_jit.hip,
// the chunk and pair evaluators below for fills, pivots and gradients) uses
// the same arithmetic: exp as __expf, RQ's B^-alpha as exp2(-alpha log2 B),
// the periodic sine as __sinf (v_sin_f32; absolute error ~2^-21 for arguments
// within 256 revolutions), so the operator, the dense K and the gradients
// agree to rounding.

// Leaf value and the pair quantities its gradient needs.
struct LeafEval {
  float k;   // leaf value (os included)
  float r2;  // scaled squared distance (radial / RQ) or the periodic sum
  float h;   // radial / RQ: dk/dl_q = h dx_q^2 / l_q^3; periodic: k (see below)
};

// Level index of a categorical coordinate, clamped into [0, L).
__device__ __forceinline__ int tree_level(float x, int L) {
  const int v = (int)x;
  return v < 0 ? 0 : (v >= L ? L - 1 : v);
}

__device__ __forceinline__ LeafEval tree_leaf_eval(const KernelTree& t, int l,
                                                   const float* __restrict__ p,
                                                   const float* xi, const float* xj) {
  const TreeLeaf& lf = t.leaf[l];
  LeafEval e;
  if (lf.kind == KIND_CAT) {
    const int dq = t.dims[lf.dim_off];
    const int L = lf.ard;
    e.k = p[t.nparams + lf.p0 + tree_level(xi[dq], L) * L + tree_level(xj[dq], L)];
    e.r2 = 0.0f;
    e.h = 0.0f;
    return e;
  }
  if (lf.kind == KIND_LINEAR || lf.kind == KIND_POLY) {
    // r2 holds the (weighted) dot product, h the derivative factor
    float dot = 0.0f;
    for (int q = 0; q < lf.ndim; ++q) {
      const int dq = t.dims[lf.dim_off + q];
      const float xx = xi[dq] * xj[dq];
      dot = lf.ard ? fmaf(p[lf.p0 + q], xx, dot) : dot + xx;
    }
    const int nls = lf.ard ? lf.ndim : 1;
    if (!lf.ard) dot *= p[lf.p0];
    e.r2 = dot;
    if (lf.kind == KIND_LINEAR) {
      const float os = p[lf.p0 + nls];
      e.k = os * dot;
      e.h = os;
      return e;
    }
    const float offset = p[lf.p0 + nls + 1];
    const float os = p[lf.p0 + nls + 2];
    const float B = dot + offset;
    float bp = 1.0f;  // B^(D-1)
    for (int k = 1; k < lf.deg; ++k) bp *= B;
    e.k = os * bp * B;
    e.h = os * (float)lf.deg * bp;  // dk/dB
    return e;
  }
  if (lf.kind == KIND_PERIODIC) {
    const float period = p[lf.p0 + (lf.ard ? lf.ndim : 1)];
    const float os = p[lf.p0 + (lf.ard ? lf.ndim : 1) + 1];
    float s = 0.0f;
    for (int q = 0; q < lf.ndim; ++q) {
      const int dq = t.dims[lf.dim_off + q];
      const float sn = __sinf(kTreePi * (xi[dq] - xj[dq]) / period);
      s += lf.ard ? sn * sn / p[lf.p0 + q] : sn * sn;
    }
    if (!lf.ard) s /= p[lf.p0];
    e.r2 = s;
    e.k = os * __expf(-2.0f * s);  // not clamped by the reference
    e.h = e.k;
    return e;
  }
  const int nls = lf.ard ? lf.ndim : 1;
  float r2 = 0.0f;
  for (int q = 0; q < lf.ndim; ++q) {
    const int dq = t.dims[lf.dim_off + q];
    const float u = (xi[dq] - xj[dq]) / p[lf.p0 + (lf.ard ? q : 0)];
    r2 = fmaf(u, u, r2);
  }
  e.r2 = r2;
  if (lf.kind == KIND_RQ) {
    const float alpha = p[lf.p0 + nls];
    const float os = p[lf.p0 + nls + 1];
    const float B = 1.0f + r2 / (2.0f * alpha);
    const float Bm = exp2f(-alpha * __log2f(B));
    e.k = os * Bm;
    e.h = os * Bm / B;
    return e;
  }
  const float os = p[lf.p0 + nls];
  if (lf.kind == KIND_RBF) {
    e.k = os * __expf(-0.5f * r2);  // not clamped by the reference
    e.h = e.k;
    return e;
  }
  const float r = sqrtf(fmaxf(r2 + 1e-20f, 1e-20f));
  if (lf.kind == KIND_MATERN12) {
    // clamped for ARD leaves only (exp2_limit in mgp_common.h)
    const float ex = __expf(lf.ard ? fmaxf(-r, -20.0f) : -r);
    e.k = os * ex;
    e.h = os * ex / r;
  } else if (lf.kind == KIND_MATERN32) {
    const float s3 = 1.7320508075688772f * r;
    const float ex = __expf(fmaxf(-s3, -20.0f));
    e.k = os * (1.0f + s3) * ex;
    e.h = 3.0f * os * ex;
  } else {  // Matern-5/2
    const float s5 = 2.2360679774997897f * r;
    const float ex = __expf(fmaxf(-s5, -20.0f));
    e.k = os * (1.0f + s5 + (5.0f / 3.0f) * r * r) * ex;
    e.h = (5.0f / 3.0f) * os * (1.0f + s5) * ex;
  }
  return e;
}

// Leaf values of one row against kTreeChunk columns (rows of xc with stride
// w): the leaf's fields and parameters are read once for the whole chunk.
constexpr int kTreeChunk = 8;

__device__ __forceinline__ void tree_leaf_chunk(const KernelTree& t, int l,
                                                const float* __restrict__ p, const float* xi,
                                                const float* xc, int w, float* out) {
  const TreeLeaf lf = t.leaf[l];
  if (lf.kind == KIND_CAT || lf.kind == KIND_LINEAR || lf.kind == KIND_POLY) {
    for (int c = 0; c < kTreeChunk; ++c) out[c] = tree_leaf_eval(t, l, p, xi, xc + c * w).k;
    return;
  }
  const int nls = lf.ard ? lf.ndim : 1;
  if (lf.kind == KIND_PERIODIC) {
    const float ip = kTreePi / p[lf.p0 + nls];
    const float os = p[lf.p0 + nls + 1];
    float s[kTreeChunk];
    for (int c = 0; c < kTreeChunk; ++c) s[c] = 0.0f;
    for (int q = 0; q < lf.ndim; ++q) {
      const int dq = t.dims[lf.dim_off + q];
      const float il = 1.0f / p[lf.p0 + (lf.ard ? q : 0)];
      const float a = xi[dq];
      for (int c = 0; c < kTreeChunk; ++c) {
        const float sn = __sinf((a - xc[c * w + dq]) * ip);
        s[c] = fmaf(sn * sn, il, s[c]);
      }
    }
    for (int c = 0; c < kTreeChunk; ++c) out[c] = os * __expf(-2.0f * s[c]);
    return;
  }
  float r2[kTreeChunk];
  for (int c = 0; c < kTreeChunk; ++c) r2[c] = 0.0f;
  for (int q = 0; q < lf.ndim; ++q) {
    const int dq = t.dims[lf.dim_off + q];
    const float inv = 1.0f / p[lf.p0 + (lf.ard ? q : 0)];
    const float a = xi[dq];
    for (int c = 0; c < kTreeChunk; ++c) {
      const float u = (a - xc[c * w + dq]) * inv;
      r2[c] = fmaf(u, u, r2[c]);
    }
  }
  if (lf.kind == KIND_RQ) {
    const float alpha = p[lf.p0 + nls], os = p[lf.p0 + nls + 1];
    const float ia = 0.5f / alpha;
    // B^-alpha = 2^(-alpha log2 B), B >= 1
    for (int c = 0; c < kTreeChunk; ++c)
      out[c] = os * exp2f(-alpha * __log2f(fmaf(r2[c], ia, 1.0f)));
    return;
  }
  const float os = p[lf.p0 + nls];
  if (lf.kind == KIND_RBF) {
    for (int c = 0; c < kTreeChunk; ++c) out[c] = os * __expf(-0.5f * r2[c]);
    return;
  }
  for (int c = 0; c < kTreeChunk; ++c) {
    const float r = sqrtf(fmaxf(r2[c] + 1e-20f, 1e-20f));
    if (lf.kind == KIND_MATERN12) {
      out[c] = os * __expf(lf.ard ? fmaxf(-r, -20.0f) : -r);
    } else if (lf.kind == KIND_MATERN32) {
      const float s3 = 1.7320508075688772f * r;
      out[c] = os * (1.0f + s3) * __expf(fmaxf(-s3, -20.0f));
    } else {
      const float s5 = 2.2360679774997897f * r;
      out[c] = os * (1.0f + s5 + (5.0f / 3.0f) * r2[c]) * __expf(fmaxf(-s5, -20.0f));
    }
  }
}

// Tree values of one row against kTreeChunk columns.
__device__ __forceinline__ void tree_value_chunk(const KernelTree& t, const float* __restrict__ p,
                                                 const float* xi, const float* xc, int w,
                                                 float* out) {
  float v[kTreeMaxNodes][kTreeChunk];
  for (int i = 0; i < t.nnodes; ++i) {
    const TreeNode nd = t.node[i];
    float x[kTreeChunk];
    if (nd.code == TN_LEAF) {
      tree_leaf_chunk(t, nd.a, p, xi, xc, w, x);
    } else if (nd.code == TN_ADD) {
      for (int c = 0; c < kTreeChunk; ++c) x[c] = v[nd.a][c] + v[nd.b][c];
    } else if (nd.code == TN_MUL) {
      for (int c = 0; c < kTreeChunk; ++c) x[c] = v[nd.a][c] * v[nd.b][c];
    } else {
      const float s = p[nd.b];
      for (int c = 0; c < kTreeChunk; ++c) x[c] = s * v[nd.a][c];
    }
    for (int c = 0; c < kTreeChunk; ++c) v[i][c] = x[c];
  }
  for (int c = 0; c < kTreeChunk; ++c) out[c] = v[t.nnodes - 1][c];
}

// Tree value for one pair; node values (and leaf evaluations) optionally kept.
__device__ __forceinline__ float tree_value(const KernelTree& t, const float* __restrict__ p,
                                            const float* xi, const float* xj,
                                            LeafEval* leaves = nullptr,
                                            float* vals = nullptr) {
  float v[kTreeMaxNodes];
  for (int i = 0; i < t.nnodes; ++i) {
    const TreeNode& nd = t.node[i];
    float x;
    if (nd.code == TN_LEAF) {
      const LeafEval le = tree_leaf_eval(t, nd.a, p, xi, xj);
      if (leaves) leaves[nd.a] = le;
      x = le.k;
    } else if (nd.code == TN_ADD) {
      x = v[nd.a] + v[nd.b];
    } else if (nd.code == TN_MUL) {
      x = v[nd.a] * v[nd.b];
    } else {
      x = p[nd.b] * v[nd.a];
    }
    v[i] = x;
    if (vals) vals[i] = x;
  }
  return v[t.nnodes - 1];
}

// dK/dtheta_p for every parameter at one pair, accumulated as g[p] += w dK/dp.
__device__ __forceinline__ void tree_grad_accumulate(const KernelTree& t,
                                                     const float* __restrict__ p,
                                                     const float* xi, const float* xj, float w,
                                                     float* g) {
  LeafEval le[kTreeMaxLeaves];
  float val[kTreeMaxNodes], adj[kTreeMaxNodes];
  tree_value(t, p, xi, xj, le, val);
  for (int i = 0; i < t.nnodes; ++i) adj[i] = 0.0f;
  adj[t.nnodes - 1] = w;
  for (int i = t.nnodes - 1; i >= 0; --i) {
    const TreeNode& nd = t.node[i];
    const float a = adj[i];
    if (nd.code == TN_ADD) {
      adj[nd.a] += a;
      adj[nd.b] += a;
    } else if (nd.code == TN_MUL) {
      adj[nd.a] += a * val[nd.b];
      adj[nd.b] += a * val[nd.a];
    } else if (nd.code == TN_SCALE) {
      adj[nd.a] += a * p[nd.b];
      g[nd.b] += a * val[nd.a];
    } else {
      const int l = nd.a;
      const TreeLeaf& lf = t.leaf[l];
      const LeafEval& e = le[l];
      if (lf.kind == KIND_CAT) continue;  // tables are learned outside this pass
      const int nls = lf.ard ? lf.ndim : 1;
      if (lf.kind == KIND_LINEAR || lf.kind == KIND_POLY) {
        // dk/dvar: h x.x' (iso) or h x_q x'_q (ARD); h = os (linear) or
        // os D B^(D-1) (polynomial); dk/doffset = h; dk/dos = k / os
        if (lf.ard) {
          for (int q = 0; q < lf.ndim; ++q) {
            const int dq = t.dims[lf.dim_off + q];
            g[lf.p0 + q] += a * e.h * xi[dq] * xj[dq];
          }
        } else {
          g[lf.p0] += a * e.h * e.r2 / p[lf.p0];
        }
        const int ios = lf.p0 + nls + (lf.kind == KIND_POLY ? 2 : 0);
        if (lf.kind == KIND_POLY) g[lf.p0 + nls + 1] += a * e.h;
        g[ios] += a * e.k / p[ios];
        continue;
      }
      if (lf.kind == KIND_PERIODIC) {
        const float period = p[lf.p0 + nls];
        const int ios = lf.p0 + nls + 1;
        // k = os exp(-2 S), S = sum_q sin^2(pi dx_q / period) / l_q
        float dperiod = 0.0f;
        for (int q = 0; q < lf.ndim; ++q) {
          const int dq = t.dims[lf.dim_off + q];
          const float dx = xi[dq] - xj[dq];
          const float ang = kTreePi * dx / period;
          const float sn = __sinf(ang), cs = __cosf(ang);
          const float lq = p[lf.p0 + (lf.ard ? q : 0)];
          if (lf.ard) g[lf.p0 + q] += a * e.k * 2.0f * sn * sn / (lq * lq);
          dperiod += sn * cs * dx / lq;
        }
        if (!lf.ard) g[lf.p0] += a * e.k * 2.0f * e.r2 / p[lf.p0];
        g[lf.p0 + nls] += a * e.k * 4.0f * kTreePi * dperiod / (period * period);
        g[ios] += a * e.k / p[ios];
        continue;
      }
      // radial / RQ lengthscales: dk/dl_q = h dx_q^2 / l_q^3
      float iso = 0.0f;
      for (int q = 0; q < lf.ndim; ++q) {
        const int dq = t.dims[lf.dim_off + q];
        const float dx = xi[dq] - xj[dq];
        const float lq = p[lf.p0 + (lf.ard ? q : 0)];
        const float term = dx * dx / (lq * lq * lq);
        if (lf.ard) g[lf.p0 + q] += a * e.h * term;
        else iso += term;
      }
      if (!lf.ard) g[lf.p0] += a * e.h * iso;
      int ios = lf.p0 + nls;
      if (lf.kind == KIND_RQ) {
        const float alpha = p[lf.p0 + nls];
        const float B = 1.0f + e.r2 / (2.0f * alpha);
        g[lf.p0 + nls] += a * e.k * (-logf(B) + e.r2 / (2.0f * alpha * B));
        ios += 1;
      }
      g[ios] += a * e.k / p[ios];
    }
  }
}

// Adjoint w dK/dv_l of every leaf value v_l at one pair (leaf_adj[nleaves]).
__device__ __forceinline__ void tree_leaf_adjoints(const KernelTree& t,
                                                   const float* __restrict__ p,
                                                   const float* xi, const float* xj, float w,
                                                   float* leaf_adj) {
  float val[kTreeMaxNodes], adj[kTreeMaxNodes];
  tree_value(t, p, xi, xj, nullptr, val);
  for (int i = 0; i < t.nnodes; ++i) adj[i] = 0.0f;
  adj[t.nnodes - 1] = w;
  for (int i = t.nnodes - 1; i >= 0; --i) {
    const TreeNode& nd = t.node[i];
    const float a = adj[i];
    if (nd.code == TN_ADD) {
      adj[nd.a] += a;
      adj[nd.b] += a;
    } else if (nd.code == TN_MUL) {
      adj[nd.a] += a * val[nd.b];
      adj[nd.b] += a * val[nd.a];
    } else if (nd.code == TN_SCALE) {
      adj[nd.a] += a * p[nd.b];
    } else {
      leaf_adj[nd.a] = a;
    }
  }
}
#endif

}  // namespace mgp
