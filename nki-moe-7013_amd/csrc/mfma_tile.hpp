// 128x128 bf16 MFMA tile engine for gfx950 (CDNA4).
//
// One workgroup of 256 threads (4 wave64s in a 2x2 grid) computes a
// 128 x 128 fp32 tile  C = A . B^T  where A rows and B rows are both
// K-contiguous bf16 ("NT" layout: every operand is read along K).
//
//  - K is consumed in slabs of 64; each slab of A and B (2 x 16 KB) is staged
//    through LDS with a 16-byte row pad (row stride 144 B), which keeps the
//    16-lane groups of ds_read_b128 on distinct banks.
//  - Two LDS buffers: slab k+1 is fetched from global memory into registers
//    while slab k feeds the MFMAs, then stored to the other buffer; one
//    barrier per slab.
//  - Each wave owns a 64 x 64 sub-tile = 2 x 2 blocks of
//    v_mfma_f32_32x32x16_bf16.
//  - A rows are addressed through a per-thread pointer table so the grouped
//    expert GEMM can gather token rows on load (no permuted copy of X).
//
// Accumulator layout of one 32x32 block (wave64): lane l holds column l%32,
// and acc[i] is row (i/4)*8 + (l/32)*4 + i%4.
#pragma once

#include "common.hpp"

namespace qmoe {
namespace tile {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded row length in bf16 elements (144 B)
constexpr int THREADS = 256;
constexpr int SMEM_BYTES = 2 * (BM + BN) * LDK * 2;  // 73728 B

struct Acc {
  f32x16 c[2][2];
};

// Row/column of accumulator element (mi, ni, i) inside the 128x128 tile.
__device__ __forceinline__ int acc_row(int wave, int lane, int mi, int i) {
  return (wave >> 1) * 64 + mi * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
}
__device__ __forceinline__ int acc_col(int wave, int lane, int ni) {
  return (wave & 1) * 64 + ni * 32 + (lane & 31);
}

// Thread t stages chunks c = t + 256*j (j < 4) of each slab: row c/8
// (= t/8 + 32j), 16-byte column chunk c%8 (= t%8).
__device__ __forceinline__ int stage_row(int t, int j) { return (t >> 3) + 32 * j; }

// Compute the tile.  a_ptr[j] / b_ptr[j] are this thread's row pointers for
// stage rows stage_row(t, j) (already offset to k = 0 and to this thread's
// 16-byte chunk); a null A pointer stands for a zero row.  K % 64 == 0.
__device__ __forceinline__ void mma_128x128(const uint16_t* const a_ptr[4],
                                            const uint16_t* const b_ptr[4], int K,
                                            uint16_t* smem, Acc& acc) {
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  uint16_t* As[2] = {smem, smem + BM * LDK};
  uint16_t* Bs[2] = {smem + 2 * BM * LDK, smem + 2 * BM * LDK + BN * LDK};

#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc.c[mi][ni][i] = 0.0f;

  u32x4 ra[4], rb[4];
  const int kc = (t & 7) * 8;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ra[j] = a_ptr[j] ? ld16(a_ptr[j] + k0) : u32x4{0u, 0u, 0u, 0u};
      rb[j] = ld16(b_ptr[j] + k0);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = stage_row(t, j);
      *reinterpret_cast<u32x4*>(As[buf] + r * LDK + kc) = ra[j];
      *reinterpret_cast<u32x4*>(Bs[buf] + r * LDK + kc) = rb[j];
    }
  };

  const int nk = K / BK;
  fetch(0);
  stash(0);
  __syncthreads();
  const int frag_k = (lane >> 5) * 8;
  const int frag_r = lane & 31;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) fetch((kt + 1) * BK);
    const uint16_t* a_base = As[cur] + (wm * 64 + frag_r) * LDK + frag_k;
    const uint16_t* b_base = Bs[cur] + (wn * 64 + frag_r) * LDK + frag_k;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a0 = *reinterpret_cast<const bf16x8*>(a_base + kk);
      bf16x8 a1 = *reinterpret_cast<const bf16x8*>(a_base + 32 * LDK + kk);
      bf16x8 b0 = *reinterpret_cast<const bf16x8*>(b_base + kk);
      bf16x8 b1 = *reinterpret_cast<const bf16x8*>(b_base + 32 * LDK + kk);
      acc.c[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc.c[0][0], 0, 0, 0);
      acc.c[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc.c[0][1], 0, 0, 0);
      acc.c[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc.c[1][0], 0, 0, 0);
      acc.c[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc.c[1][1], 0, 0, 0);
    }
    if (kt + 1 < nk) stash(cur ^ 1);
    __syncthreads();
  }
}

}  // namespace tile
}  // namespace qmoe
