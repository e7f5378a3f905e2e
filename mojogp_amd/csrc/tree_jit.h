// Run-time compiled (hiprtc) product kernels of composite kernel trees.
#pragma once

#include <string>

#include "kernel_tree.h"

namespace mgp {

struct TreeJitKernel {
  hipFunction_t fn = nullptr;  // extern "C" k_tree_jit_<ncols>
  int ncols = 0;               // right-hand sides the kernel accumulates (>= requested)
  size_t lds_bytes = 0;        // dynamic LDS per 256-thread block
  int rows_per_block = 256;    // rows of Xr per block (grid x = ceil(m / rows_per_block))
};

// The straight-line product kernel of tree t for nc <= 16 right-hand sides:
// arguments (const float* Xr, long long m, const float* Xc, long long n,
// const float* p, const float* V, int nc, float* part), grid
// (ceil(m / rows_per_block), column splits), 256 threads; part[y][c][i] = split y's sum over its columns
// j of K(Xr_i, Xc_j) V[c][j].  Compiled on first use per (tree, device).
TreeJitKernel tree_jit_kernel(const KernelTree& t, int nc);
// The generated source (tests and inspection).
std::string tree_jit_source(const KernelTree& t);

}  // namespace mgp
