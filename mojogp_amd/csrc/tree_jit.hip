// Straight-line product kernels of composite kernel trees, compiled at run time
// with hiprtc: the gfx950 counterpart of the reference's per-kernel code
// generation (codegen_engine/emit/gpu_kernel.py:151-260 emits one Mojo kernel
// per kernel expression; expressions.py:77-421 holds the leaf formulas).
//
// The interpreted tree kernels (tree.hip) walk the node list per pair with the
// node values in private memory.  Here the tree's value is emitted as one
// expression per leaf and node, with the leaf constants (inverse
// lengthscales, outputscales, ...) computed once per thread from the
// parameter vector, so a pair costs only its arithmetic: coordinates come
// from broadcast LDS reads, the products accumulate in registers.  The leaf
// arithmetic is the interpreted chunk evaluator's (kernel_tree.h,
// tree_leaf_chunk), term for term.  One compile per (tree, device), cached
// for the process.
#include "tree_jit.h"

#include <hip/hiprtc.h>

#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

namespace mgp {

namespace {

constexpr int kJitTile = 128;  // column points per LDS tile
const int kJitCols[] = {1, 2, 4, 8, 16};
constexpr int kJitMfmaMinCols = 8;   // column counts from here use the MFMA product
constexpr int kJitMfmaRowTiles = 2;  // 16-row tiles per wave in the MFMA kernel

std::string f(float v) {
  std::ostringstream o;
  o.precision(9);
  o << std::scientific << v << "f";
  return o.str();
}

// Prologue (per-thread constants from p) and pair code (k from xi, xj) of the
// tree; leaf l's value is v<node>, the tree value the last node's.
void emit_tree(const KernelTree& t, std::string& pro, std::string& pair) {
  std::ostringstream P, Q;
  for (int l = 0; l < t.nleaves; ++l) {
    const TreeLeaf& lf = t.leaf[l];
    const int nls = lf.ard ? lf.ndim : 1;
    const std::string L = "l" + std::to_string(l);
    auto dim = [&](int q) { return t.dims[lf.dim_off + q]; };
    if (lf.kind == KIND_CAT) {
      const int L_ = lf.ard;
      Q << "  float " << L << ";\n  {\n"
        << "    int a = (int)xi[" << dim(0) << "], b = (int)xj[" << dim(0) << "];\n"
        << "    a = a < 0 ? 0 : (a >= " << L_ << " ? " << L_ - 1 << " : a);\n"
        << "    b = b < 0 ? 0 : (b >= " << L_ << " ? " << L_ - 1 << " : b);\n"
        << "    " << L << " = p[" << t.nparams + lf.p0 << " + a * " << L_ << " + b];\n  }\n";
      continue;
    }
    if (lf.kind == KIND_LINEAR || lf.kind == KIND_POLY) {
      for (int q = 0; q < nls; ++q)
        P << "  const float " << L << "w" << q << " = p[" << lf.p0 + q << "];\n";
      P << "  const float " << L << "os = p[" << lf.p0 + nls + (lf.kind == KIND_POLY ? 2 : 0)
        << "];\n";
      if (lf.kind == KIND_POLY)
        P << "  const float " << L << "off = p[" << lf.p0 + nls + 1 << "];\n";
      Q << "  float " << L << "d = 0.0f;\n";
      for (int q = 0; q < lf.ndim; ++q) {
        const std::string xx = "xi[" + std::to_string(dim(q)) + "] * xj[" +
                               std::to_string(dim(q)) + "]";
        if (lf.ard)
          Q << "  " << L << "d = fmaf(" << L << "w" << q << ", " << xx << ", " << L << "d);\n";
        else
          Q << "  " << L << "d = " << L << "d + " << xx << ";\n";
      }
      if (!lf.ard) Q << "  " << L << "d *= " << L << "w0;\n";
      if (lf.kind == KIND_LINEAR) {
        Q << "  const float " << L << " = " << L << "os * " << L << "d;\n";
      } else {
        Q << "  const float " << L << "B = " << L << "d + " << L << "off;\n"
          << "  float " << L << "bp = 1.0f;\n";
        for (int k = 1; k < lf.deg; ++k) Q << "  " << L << "bp *= " << L << "B;\n";
        Q << "  const float " << L << " = " << L << "os * " << L << "bp * " << L << "B;\n";
      }
      continue;
    }
    // radial, RQ and periodic leaves: inverse lengthscales
    for (int q = 0; q < nls; ++q)
      P << "  const float " << L << "il" << q << " = 1.0f / p[" << lf.p0 + q << "];\n";
    if (lf.kind == KIND_PERIODIC) {
      P << "  const float " << L << "ip = " << f(kTreePi) << " / p[" << lf.p0 + nls << "];\n"
        << "  const float " << L << "os = p[" << lf.p0 + nls + 1 << "];\n";
      Q << "  float " << L << "s = 0.0f;\n";
      for (int q = 0; q < lf.ndim; ++q)
        Q << "  { const float sn = __sinf((xi[" << dim(q) << "] - xj[" << dim(q) << "]) * " << L
          << "ip); " << L << "s = fmaf(sn * sn, " << L << "il" << (lf.ard ? q : 0) << ", " << L
          << "s); }\n";
      Q << "  const float " << L << " = " << L << "os * __expf(-2.0f * " << L << "s);\n";
      continue;
    }
    Q << "  float " << L << "r2 = 0.0f;\n";
    for (int q = 0; q < lf.ndim; ++q)
      Q << "  { const float u = (xi[" << dim(q) << "] - xj[" << dim(q) << "]) * " << L << "il"
        << (lf.ard ? q : 0) << "; " << L << "r2 = fmaf(u, u, " << L << "r2); }\n";
    if (lf.kind == KIND_RQ) {
      P << "  const float " << L << "al = p[" << lf.p0 + nls << "];\n"
        << "  const float " << L << "ia = 0.5f / " << L << "al;\n"
        << "  const float " << L << "os = p[" << lf.p0 + nls + 1 << "];\n";
      Q << "  const float " << L << " = " << L << "os * exp2f(-" << L << "al * __log2f(fmaf("
        << L << "r2, " << L << "ia, 1.0f)));\n";
      continue;
    }
    P << "  const float " << L << "os = p[" << lf.p0 + nls << "];\n";
    if (lf.kind == KIND_RBF) {
      Q << "  const float " << L << " = " << L << "os * __expf(-0.5f * " << L << "r2);\n";
      continue;
    }
    Q << "  const float " << L << "r = sqrtf(fmaxf(" << L << "r2 + 1e-20f, 1e-20f));\n";
    if (lf.kind == KIND_MATERN12) {
      // the -20 clamp applies to ARD Matern-1/2 leaves only (exp2_limit)
      if (lf.ard)
        Q << "  const float " << L << " = " << L << "os * __expf(fmaxf(-" << L
          << "r, -20.0f));\n";
      else
        Q << "  const float " << L << " = " << L << "os * __expf(-" << L << "r);\n";
    } else if (lf.kind == KIND_MATERN32) {
      Q << "  const float " << L << "s3 = 1.7320508075688772f * " << L << "r;\n"
        << "  const float " << L << " = " << L << "os * (1.0f + " << L << "s3) * __expf(fmaxf(-"
        << L << "s3, -20.0f));\n";
    } else {
      Q << "  const float " << L << "s5 = 2.2360679774997897f * " << L << "r;\n"
        << "  const float " << L << " = " << L << "os * (1.0f + " << L << "s5 + (5.0f / 3.0f) * "
        << L << "r2) * __expf(fmaxf(-" << L << "s5, -20.0f));\n";
    }
  }
  for (int i = 0; i < t.nnodes; ++i) {
    const TreeNode& nd = t.node[i];
    const std::string N = "n" + std::to_string(i);
    if (nd.code == TN_LEAF)
      Q << "  const float " << N << " = l" << nd.a << ";\n";
    else if (nd.code == TN_ADD)
      Q << "  const float " << N << " = n" << nd.a << " + n" << nd.b << ";\n";
    else if (nd.code == TN_MUL)
      Q << "  const float " << N << " = n" << nd.a << " * n" << nd.b << ";\n";
    else {
      P << "  const float s" << i << " = p[" << nd.b << "];\n";
      Q << "  const float " << N << " = s" << i << " * n" << nd.a << ";\n";
    }
  }
  Q << "  return n" << t.nnodes - 1 << ";\n";
  pro = P.str();
  pair = Q.str();
}

// The kernel source: out partials part[y][c][i] = sum over split y of
// K(Xr_i, Xc_j) V[c][j] for c < nc (the interpreted kernel's layout), one row
// per thread, NC >= nc accumulators.
std::string tree_source(const KernelTree& t) {
  std::string pro, pair;
  emit_tree(t, pro, pair);
  const int D = t.d, DP = (D + 3) / 4 * 4;
  std::ostringstream s;
  s << "#define D " << D << "\n#define DP " << DP << "\n#define TILE " << kJitTile << "\n"
    << "template <int NC>\n"
    << "__device__ __forceinline__ void body(const float* __restrict__ Xr, long long m,\n"
    << "    const float* __restrict__ Xc, long long n, const float* __restrict__ p,\n"
    << "    const float* __restrict__ V, int nc, float* __restrict__ part) {\n"
    << "  extern __shared__ float sm[];\n"
    << "  float* sx = sm;\n"
    << "  float* sv = sm + TILE * DP;\n"
    << pro
    << "  auto kval = [&](const float* __restrict__ xi, const float* __restrict__ xj)\n"
    << "      __attribute__((always_inline)) -> float {\n"
    << pair
    << "  };\n"
    << "  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n"
    << "  float xi[DP];\n"
    << "#pragma unroll\n"
    << "  for (int k = 0; k < DP; ++k) xi[k] = (i < m && k < D) ? Xr[i * D + k] : 0.0f;\n"
    << "  double acc[NC];\n"
    << "#pragma unroll\n"
    << "  for (int c = 0; c < NC; ++c) acc[c] = 0.0;\n"
    << "  const long long tiles = (n + TILE - 1) / TILE;\n"
    << "  const long long tps = (tiles + gridDim.y - 1) / gridDim.y;\n"
    << "  const long long jbeg = (long long)blockIdx.y * tps * TILE;\n"
    << "  const long long jend = n < jbeg + tps * TILE ? n : jbeg + tps * TILE;\n"
    << "  for (long long j0 = jbeg; j0 < jend; j0 += TILE) {\n"
    << "    __syncthreads();\n"
    << "    for (int q = threadIdx.x; q < TILE * DP; q += blockDim.x) {\n"
    << "      const int jj = q / DP, k = q - jj * DP;\n"
    << "      const long long j = j0 + jj;\n"
    << "      sx[q] = (j < n && k < D) ? Xc[j * D + k] : 0.0f;\n"
    << "    }\n"
    << "    for (int q = threadIdx.x; q < TILE * NC; q += blockDim.x) {\n"
    << "      const int c = q / TILE, jj = q - c * TILE;\n"
    << "      const long long j = j0 + jj;\n"
    << "      sv[q] = (c < nc && j < n) ? V[(long long)c * n + j] : 0.0f;\n"
    << "    }\n"
    << "    __syncthreads();\n"
    << "    float pa[NC];\n"
    << "#pragma unroll\n"
    << "    for (int c = 0; c < NC; ++c) pa[c] = 0.0f;\n"
    << "    const int cnt = (int)(jend - j0 < TILE ? jend - j0 : TILE);\n"
    << "#pragma unroll 2\n"
    << "    for (int jj = 0; jj < cnt; ++jj) {\n"
    << "      const float k = kval(xi, sx + jj * DP);\n"
    << "#pragma unroll\n"
    << "      for (int c = 0; c < NC; ++c) pa[c] = fmaf(k, sv[c * TILE + jj], pa[c]);\n"
    << "    }\n"
    << "#pragma unroll\n"
    << "    for (int c = 0; c < NC; ++c) acc[c] += (double)pa[c];\n"
    << "  }\n"
    << "  if (i < m) {\n"
    << "    float* dst = part + (long long)blockIdx.y * nc * m;\n"
    << "#pragma unroll\n"
    << "    for (int c = 0; c < NC; ++c)\n"
    << "      if (c < nc) dst[(long long)c * m + i] = (float)acc[c];\n"
    << "  }\n"
    << "}\n";
  // 8..16 right-hand sides: the product on the fp32 matrix cores.  Wave w
  // owns row tiles i0 + 16 r (r < R); per step of 4 columns j = j0 + 4 s +
  // l/16 each lane evaluates the pair (row i0 + 16 r + l%16, column j) as the
  // A operand of v_mfma_f32_16x16x4_f32 and supplies B = V[l%16][j]; D holds
  // rows i0 + 16 r + 4 (l/16) + q of right-hand side l%16.  Per column tile
  // the fp32 D is added into fp64.
  s << "typedef float f4m __attribute__((ext_vector_type(4)));\n"
    << "#define R " << kJitMfmaRowTiles << "\n"
    << "__device__ __forceinline__ void body_mfma(const float* __restrict__ Xr, long long m,\n"
    << "    const float* __restrict__ Xc, long long n, const float* __restrict__ p,\n"
    << "    const float* __restrict__ V, int nc, float* __restrict__ part) {\n"
    << "  extern __shared__ float sm[];\n"
    << "  float* sx = sm;\n"
    << "  float* sv = sm + TILE * DP;\n"
    << pro
    << "  auto kval = [&](const float* __restrict__ xi, const float* __restrict__ xj)\n"
    << "      __attribute__((always_inline)) -> float {\n"
    << pair
    << "  };\n"
    << "  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n"
    << "  const int lm = lane & 15, lq = lane >> 4;\n"
    << "  const long long i0 = ((long long)blockIdx.x * 4 + wave) * (16 * R);\n"
    << "  float xi[R][DP];\n"
    << "#pragma unroll\n"
    << "  for (int r = 0; r < R; ++r) {\n"
    << "    const long long i = i0 + 16 * r + lm;\n"
    << "#pragma unroll\n"
    << "    for (int k = 0; k < DP; ++k) xi[r][k] = (i < m && k < D) ? Xr[i * D + k] : 0.0f;\n"
    << "  }\n"
    << "  double acc[R][4];\n"
    << "#pragma unroll\n"
    << "  for (int r = 0; r < R; ++r)\n"
    << "#pragma unroll\n"
    << "    for (int q = 0; q < 4; ++q) acc[r][q] = 0.0;\n"
    << "  const long long tiles = (n + TILE - 1) / TILE;\n"
    << "  const long long tps = (tiles + gridDim.y - 1) / gridDim.y;\n"
    << "  const long long jbeg = (long long)blockIdx.y * tps * TILE;\n"
    << "  const long long jend = n < jbeg + tps * TILE ? n : jbeg + tps * TILE;\n"
    << "  for (long long j0 = jbeg; j0 < jend; j0 += TILE) {\n"
    << "    __syncthreads();\n"
    << "    for (int q = threadIdx.x; q < TILE * DP; q += blockDim.x) {\n"
    << "      const int jj = q / DP, k = q - jj * DP;\n"
    << "      const long long j = j0 + jj;\n"
    << "      sx[q] = (j < n && k < D) ? Xc[j * D + k] : 0.0f;\n"
    << "    }\n"
    << "    for (int q = threadIdx.x; q < TILE * 16; q += blockDim.x) {\n"
    << "      const int c = q / TILE, jj = q - c * TILE;\n"
    << "      const long long j = j0 + jj;\n"
    << "      sv[q] = (c < nc && j < jend) ? V[(long long)c * n + j] : 0.0f;\n"
    << "    }\n"
    << "    __syncthreads();\n"
    << "    f4m d[R];\n"
    << "#pragma unroll\n"
    << "    for (int r = 0; r < R; ++r) d[r] = f4m{0.0f, 0.0f, 0.0f, 0.0f};\n"
    << "    const int steps = (int)((jend - j0 < TILE ? jend - j0 : TILE) + 3) / 4;\n"
    << "#pragma unroll 2\n"
    << "    for (int st = 0; st < steps; ++st) {\n"
    << "      const int jj = 4 * st + lq;\n"
    << "      const float* xj = sx + jj * DP;\n"
    << "      const float b = sv[lm * TILE + jj];\n"
    << "#pragma unroll\n"
    << "      for (int r = 0; r < R; ++r)\n"
    << "        d[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(kval(xi[r], xj), b, d[r], 0, 0, 0);\n"
    << "    }\n"
    << "#pragma unroll\n"
    << "    for (int r = 0; r < R; ++r)\n"
    << "#pragma unroll\n"
    << "      for (int q = 0; q < 4; ++q) acc[r][q] += (double)d[r][q];\n"
    << "  }\n"
    << "  if (lm < nc) {\n"
    << "    float* dst = part + ((long long)blockIdx.y * nc + lm) * m;\n"
    << "#pragma unroll\n"
    << "    for (int r = 0; r < R; ++r)\n"
    << "#pragma unroll\n"
    << "      for (int q = 0; q < 4; ++q) {\n"
    << "        const long long i = i0 + 16 * r + 4 * lq + q;\n"
    << "        if (i < m) dst[i] = (float)acc[r][q];\n"
    << "      }\n"
    << "  }\n"
    << "}\n";
  for (int nc : kJitCols) {
    s << "extern \"C\" __global__ __launch_bounds__(256) void k_tree_jit_" << nc
      << "(const float* Xr, long long m, const float* Xc, long long n, const float* p,\n"
      << "    const float* V, int nc, float* part) { ";
    if (nc >= kJitMfmaMinCols)
      s << "body_mfma(Xr, m, Xc, n, p, V, nc, part); }\n";
    else
      s << "body<" << nc << ">(Xr, m, Xc, n, p, V, nc, part); }\n";
  }
  return s.str();
}

std::string spec_key(const KernelTree& t) {
  std::ostringstream o;
  o << t.d << ' ' << t.nparams << ' ' << t.nleaves << ' ' << t.nnodes << ' ' << t.table_size;
  for (int l = 0; l < t.nleaves; ++l) {
    const TreeLeaf& lf = t.leaf[l];
    o << " L" << lf.kind << ',' << lf.ard << ',' << lf.ndim << ',' << lf.dim_off << ','
      << lf.p0 << ',' << lf.deg;
  }
  for (int i = 0; i < t.nnodes; ++i) o << " N" << t.node[i].code << ',' << t.node[i].a << ','
                                       << t.node[i].b;
  int nd = 0;
  for (int l = 0; l < t.nleaves; ++l) nd += t.leaf[l].ndim;
  for (int q = 0; q < nd; ++q) o << " d" << t.dims[q];
  return o.str();
}

struct Compiled {
  hipModule_t mod = nullptr;
  hipFunction_t fn[5] = {};
};

std::mutex g_jit_mu;
std::map<std::pair<std::string, int>, Compiled> g_jit;

#define MGP_RTC_CHECK(expr, prog)                                                         \
  do {                                                                                    \
    const hiprtcResult r_ = (expr);                                                       \
    if (r_ != HIPRTC_SUCCESS) {                                                           \
      std::string log_;                                                                   \
      size_t n_ = 0;                                                                      \
      if (prog && hiprtcGetProgramLogSize(prog, &n_) == HIPRTC_SUCCESS && n_ > 1) {        \
        log_.resize(n_);                                                                  \
        (void)hiprtcGetProgramLog(prog, &log_[0]);                                        \
      }                                                                                   \
      throw Error(ST_INTERNAL, std::string("hiprtc: ") + hiprtcGetErrorString(r_) + " in " \
                                   #expr + (log_.empty() ? "" : "\n" + log_));            \
    }                                                                                     \
  } while (0)

Compiled compile_tree(const KernelTree& t) {
  const std::string src = tree_source(t);
  hiprtcProgram prog = nullptr;
  MGP_RTC_CHECK(hiprtcCreateProgram(&prog, src.c_str(), "kernel_tree_jit.hip", 0, nullptr,
                                    nullptr),
                prog);
  // packed-FP32 VALU forms are disabled here as for every device file
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
  std::vector<char> code;
  try {
    MGP_RTC_CHECK(rc, prog);
    size_t size = 0;
    MGP_RTC_CHECK(hiprtcGetCodeSize(prog, &size), prog);
    code.resize(size);
    MGP_RTC_CHECK(hiprtcGetCode(prog, code.data()), prog);
  } catch (...) {
    (void)hiprtcDestroyProgram(&prog);
    throw;
  }
  (void)hiprtcDestroyProgram(&prog);
  Compiled c;
  MGP_HIP_CHECK(hipModuleLoadData(&c.mod, code.data()));
  for (int k = 0; k < 5; ++k) {
    const std::string name = "k_tree_jit_" + std::to_string(kJitCols[k]);
    MGP_HIP_CHECK(hipModuleGetFunction(&c.fn[k], c.mod, name.c_str()));
  }
  return c;
}

}  // namespace

std::string tree_jit_source(const KernelTree& t) { return tree_source(t); }

TreeJitKernel tree_jit_kernel(const KernelTree& t, int nc) {
  MGP_REQUIRE(nc >= 1 && nc <= 16, "tree product pass takes 1..16 right-hand sides");
  int dev = 0;
  MGP_HIP_CHECK(hipGetDevice(&dev));
  const auto key = std::make_pair(spec_key(t), dev);
  std::lock_guard<std::mutex> lk(g_jit_mu);
  auto it = g_jit.find(key);
  if (it == g_jit.end()) it = g_jit.emplace(key, compile_tree(t)).first;
  int k = 0;
  while (kJitCols[k] < nc) ++k;
  TreeJitKernel out;
  out.fn = it->second.fn[k];
  out.ncols = kJitCols[k];
  const int DP = (t.d + 3) / 4 * 4;
  const bool mfma = out.ncols >= kJitMfmaMinCols;
  out.rows_per_block = mfma ? 4 * 16 * kJitMfmaRowTiles : 256;
  out.lds_bytes = (size_t)kJitTile * (DP + (mfma ? 16 : out.ncols)) * sizeof(float);
  return out;
}

}  // namespace mgp
