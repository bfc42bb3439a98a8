// Helpers shared by the decode-shape (GEMV) kernels.
#pragma once

#include "common.hpp"

namespace qmoe {

constexpr int DEC_MAX_T = 64;

// Keeps a register value opaque to the optimiser inside a loop, so that
// loop-invariant conversions of it are not hoisted (hoisting the bf16 -> fp32
// unpack of streamed weights doubles their registers and serialises the loads).
__device__ __forceinline__ void opaque(u32x4& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

// Copies n 16-byte chunks into LDS (dst[c] = *src(c)) with NT threads.  Up to
// MAXI chunks per thread are all loaded before the first is stored, so the
// copy costs one memory round trip (a plain strided loop would wait for each
// load before issuing the next); chunks beyond NT * MAXI take a loop.
template <int NT, int MAXI, class Src>
__device__ __forceinline__ void stage16(u32x4* dst, int n, Src src) {
  u32x4 v[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const int c = int(threadIdx.x) + NT * i;
    if (c < n) v[i] = ld16(src(c));
  }
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const int c = int(threadIdx.x) + NT * i;
    if (c < n) dst[c] = v[i];
  }
  for (int c = int(threadIdx.x) + NT * MAXI; c < n; c += NT) dst[c] = ld16(src(c));
}

// Stage n token rows (bf16 [H]) into LDS; rows given by an index map or direct.
// A plain strided loop: it keeps the caller's registers free, which matters
// more than batching these loads where several workgroups share a CU.
__device__ __forceinline__ void stage_rows_bf16(uint16_t* dst, const uint16_t* src,
                                                const int32_t* row_map, int r0, int n, int H) {
  const int hch = H / 8;
  for (int q = threadIdx.x; q < n * hch; q += blockDim.x) {
    const int j = q / hch, kc = q - j * hch;
    const int64_t row = row_map ? row_map[r0 + j] : (r0 + j);
    *reinterpret_cast<u32x4*>(dst + j * H + kc * 8) = ld16(src + row * H + kc * 8);
  }
}

}  // namespace qmoe
