// MFMA tile core shared by the GEMM and implicit-GEMM convolution kernels.
//
// LDS tiles are stored k-contiguous: tile[row][k] with 64 k-values (128 bytes) per
// row, split in eight 16-byte chunks whose index is XOR-swizzled by
// (row ^ row >> 3) & 7.  For v_mfma_f32_32x32x16 each lane supplies, for its row
// (lane % 32), the 8 k-values of chunk (2*kk + lane / 32) of a 16-wide k-slice kk;
// a and b use the same k-to-(lane half, slot) assignment, so the products pair up
// whatever order the hardware sums them in.  Accumulator register r of a lane holds
// row (r / 4) * 8 + (lane / 32) * 4 + r % 4 and column lane % 32 of the 32 x 32 block.
#pragma once

#include "nt_common.h"

namespace nt {

constexpr int TILE_K = 64;

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

__device__ __forceinline__ int lds_index(int row, int k) { return row * TILE_K + swz(row, k >> 3) * 8 + (k & 7); }

template <typename T>
struct mfma_traits;
template <>
struct mfma_traits<f16_t> {
  typedef half8 frag;
  __device__ __forceinline__ static floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct mfma_traits<bf16_t> {
  typedef bf16x8 frag;
  __device__ __forceinline__ static floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// Accumulator row (within a 32 x 32 block) of register r for this lane.
__device__ __forceinline__ int acc_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

// One 64-deep k-tile of a (WI*32) x (WJ*32) wave tile: rows from sA starting at
// a_row0, columns from sB starting at b_row0.
template <typename T, int WI, int WJ>
__device__ __forceinline__ void mma_ktile(const uint16_t* sA, const uint16_t* sB, int a_row0, int b_row0, int lane,
                                          floatx16 (&acc)[WI][WJ]) {
  typedef typename mfma_traits<T>::frag frag;
#pragma unroll
  for (int kk = 0; kk < TILE_K / 16; ++kk) {
    const int chunk = kk * 2 + (lane >> 5);
    frag fa[WI], fb[WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int row = a_row0 + i * 32 + (lane & 31);
      fa[i] = *(const frag*)(sA + row * TILE_K + swz(row, chunk) * 8);
    }
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
      const int row = b_row0 + j * 32 + (lane & 31);
      fb[j] = *(const frag*)(sB + row * TILE_K + swz(row, chunk) * 8);
    }
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < WJ; ++j) acc[i][j] = mfma_traits<T>::mma(fa[i], fb[j], acc[i][j]);
  }
}

template <int WI, int WJ>
__device__ __forceinline__ void zero_acc(floatx16 (&acc)[WI][WJ]) {
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < WJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// Write the 32-row slab `acc_i` (WJ blocks of 32 x 32) of one wave into `stage` as
// fp32 [32][WJ*32], scaled by `scale`, ordered after the wave's earlier reads of `stage`
// and before its later ones.  Every register index is a compile-time
// constant, so the accumulators stay in registers; the epilogue that follows reads
// the slab back with plain runtime loops (and coalesced global accesses).
template <int WJ>
__device__ __forceinline__ void stage_slab(float* stage, const floatx16 (&acc_i)[WJ], int lane, float scale = 1.0f) {
  wave_lds_order();  // reads of the previous slab come first
#pragma unroll
  for (int j = 0; j < WJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) stage[acc_row(r, lane) * (WJ * 32) + j * 32 + (lane & 31)] = acc_i[j][r] * scale;
  wave_lds_order();  // every lane's writes before any lane reads the slab
}

// 8x8 transpose of 16-bit values held as 8 rows of 4 dwords (row r, dword d holds
// columns 2d and 2d+1); out[j] holds column j as 8 values down the rows.
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int d = j >> 1;
    const bool hi = j & 1;
    uint32_t w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t x0 = in[2 * r][d], x1 = in[2 * r + 1][d];
      w[r] = hi ? ((x0 >> 16) | (x1 & 0xffff0000u)) : ((x0 & 0xffffu) | (x1 << 16));
    }
    out[j] = u32x4{w[0], w[1], w[2], w[3]};
  }
}

}  // namespace nt
