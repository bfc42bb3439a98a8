// Row RMSNorm pieces shared by the kernels that normalise a row they have
// just produced (rmsnorm_residual_kernel, the combine and the split-K
// reduction with a fused norm), so every one of them rounds alike: thread t
// of NORM_THREADS holds the row's float4 chunks t, t + 256, ...; its sum of
// squares runs over them in that order, the block total is the four wave
// sums in wave order, and y = bf16(w * (h * r)) with r = rsqrt(mean(h^2) + eps).
#pragma once

#include "common.hpp"

namespace qmoe {

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAX_CHUNKS = 8;  // H <= 256 * 4 * 8 = 8192

__device__ __forceinline__ float norm_sq4(float4 a) { return a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w; }

// r = rsqrt(sum / H + eps) from each thread's partial sum; `red` holds
// NORM_THREADS / 64 floats of LDS.  Every thread of the block must call it.
__device__ __forceinline__ float norm_rsqrt(float ss, int H, float eps, float* red) {
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
  return rsqrtf(tot / float(H) + eps);
}

// Four normalised, weighted values as two bf16 pairs (chunk c of the row).
__device__ __forceinline__ uint2 norm_out4(float4 a, float r, const uint16_t* __restrict__ w, int c) {
  const uint2 wv = reinterpret_cast<const uint2*>(w)[c];
  uint2 o;
  o.x = pack_bf16x2(bf16_lo(wv.x) * (a.x * r), bf16_hi(wv.x) * (a.y * r));
  o.y = pack_bf16x2(bf16_lo(wv.y) * (a.z * r), bf16_hi(wv.y) * (a.w * r));
  return o;
}

}  // namespace qmoe
