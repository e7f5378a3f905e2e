// Pieces shared by the symmetric products (matvec.hip k_sym_tile, dense.hip
// k_dense_sym): the cyclic half of block pairs, the wave-private LDS scratch
// swizzle and gfx950's transposing LDS read.
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace mgp {

constexpr int kXcds = 8;  // XCDs of the MI355X (workgroups are dealt to them in turn)

// Off-diagonal column blocks formed by row block b of nb: row block b forms
// blocks (b, (b + delta) mod nb) for delta = 1 .. sym_span(b, nb), so every
// unordered pair of distinct blocks is formed exactly once and every row
// block carries the same work (nb even: delta = nb/2 belongs to b < nb/2).
__host__ __device__ inline int64_t sym_span(int64_t b, int64_t nb) {
  if (nb & 1) return (nb - 1) / 2;
  return b < nb / 2 ? nb / 2 : nb / 2 - 1;
}

typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
typedef __fp16 tr4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) tr4 lds_tr4;

// Scratch chunk index of (row i, column quad s) of a 16x16 fp16 tile held as
// 64 8-byte chunks (4 columns of one row each): a swizzle under which both
// the stores (lane i + 16 s stores chunk (i, s)) and the transposing reads
// below touch every bank once per 16 lanes.
__device__ __forceinline__ int sym_chunk(int i, int s) { return 16 * s + (i ^ (4 * s)); }

// ds_read_b64_tr_b16 of the chunk at p.  When lane 16g + 4e + s fetches the
// chunk (row 4g + e, quad s) of a tile X, the instruction hands lane 16g + k
// the elements X[4g + e][k], e = 0..3 (gfx950 lane semantics, pinned by an
// in-bounds probe): the tile transposed into a v_mfma_f32_16x16x32_f16
// operand contracted over its rows.
__device__ __forceinline__ uint64_t tr_read(const uint64_t* p) {
  const tr4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      (lds_tr4*)((__attribute__((address_space(3))) char*)(p)));
  return __builtin_bit_cast(uint64_t, v);
}

// The chunk lane `lane` fetches for the transposed operand of a 16x16 tile.
__device__ __forceinline__ int sym_read_chunk(int lane) {
  return sym_chunk(4 * (lane >> 4) + ((lane >> 2) & 3), lane & 3);
}

}  // namespace mgp
