// head_dim 64 flash attention kernels for gfx950 built on swizzled row-major
// LDS tiles and ds_read_b64_tr_b16.
//
// Every tile row is 64 bf16 = 128 B = 8 chunks of 16 B; chunk c of row r is
// stored at position c ^ g(r >> 1), g(t) = ((t & 1) << 2) | ((t >> 1) & 3).
// With 64 four-byte banks that layout serves both access patterns without
// bank conflicts:
//   * row reads (MFMA operand with k along the row): 16 consecutive rows at
//     one chunk hit 16 distinct 4-bank groups;
//   * transposed reads (ds_read_b64_tr_b16, k along the column): 4 rows of
//     4 consecutive chunks per half-wave hit 16 distinct 4-bank groups.
// Transposed reads hand lane i of each 16-lane group rows rho(0..3) of column
// m0 + i, where lane 4j + q supplies the address of row rho(j), columns
// m0 + 4q .. +3.  Choosing rho lets the k-slots match whatever row order the
// other MFMA operand has in registers (see trfrag).
#pragma once

#include "gemm_core.h"

namespace at64 {

using gemm::lds_t;
using gemm::lds_x8;
using gemm::read_tr;

__device__ __forceinline__ int swz(int row, int chunk) {
  const int t = (row >> 1) & 7;
  const int g = ((t & 1) << 2) | (t >> 1);
  return row * 64 + 8 * (chunk ^ g);
}

// Row-read MFMA operand: 8 values at (row, chunk).
__device__ __forceinline__ bf16x8 rowfrag(const lds_t* tile, int row, int chunk) {
  return *(const lds_x8*)(tile + swz(row, chunk));
}

// Transposed MFMA operand for rows m0 + lane%32 of a logical X[k][m] stored
// as tile rows = k.  kslot(j) gives the k of slot j for this lane's half:
//   interleaved == false: k = kbase + 8*half + j            (j = 0..7)
//   interleaved == true:  k = kbase + 4*half + j (+8 for j >= 4),
// the second being the row order of a 32x32 MFMA accumulator (rows
// 8*(i/4) + 4*(lane/32) + i%4), so P and dS feed straight from registers.
template <bool kInterleaved>
__device__ __forceinline__ bf16x8 trfrag(const lds_t* tile, int m0, int kbase, int lane) {
  const int hl = lane >> 5, cq = lane & 15;
  const int m = m0 + 16 * ((lane >> 4) & 1) + 4 * (cq & 3);
  const int chunk = m >> 3, half = (m >> 2) & 1;
  const int k_lo = kInterleaved ? kbase + 4 * hl + (cq >> 2) : kbase + 8 * hl + (cq >> 2);
  const int k_hi = kInterleaved ? k_lo + 8 : k_lo + 4;
  bf16x4 lo = read_tr(tile + swz(k_lo, chunk) + 4 * half);
  bf16x4 hi = read_tr(tile + swz(k_hi, chunk) + 4 * half);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

}  // namespace at64
