// Measurement probe (not part of the product ABI): the bf16 MFMA rate this
// GPU sustains on realistic operands.  MI355X's published dense bf16 peak
// (2.5 PFLOP/s) assumes a clock that a fully loaded chip holds only with
// low-toggle data; with random operands the power limit lowers the clock.
// bench.py reports roofline fractions against both figures.
//
// Each wave holds 4 + 4 random bf16 operand registers (loaded from `src`,
// distinct per lane and workgroup) and runs `iters` rounds of 32
// v_mfma_f32_32x32x16_bf16 over 8 independent accumulators; nothing else.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void mfma_peak_kernel(const bf16x8* __restrict__ src, int iters,
                                                        float* __restrict__ out) {
  const int t = threadIdx.x;
  bf16x8 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = src[(blockIdx.x * 8 + i) * 256 + t];
    b[i] = src[(blockIdx.x * 8 + 4 + i) * 256 + t];
  }
  f32x16 c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        c[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(r + i) & 3], b[(r + (i >> 1)) & 3], c[i], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[i][e];
  out[blockIdx.x * 256 + t] = s;  // keeps the MFMAs live
}
}  // namespace

// src: bf16 [blocks * 8 * 256 * 8] random values; out: f32 [blocks * 256].
// Returns 0, or the HIP error code of the launch.
extern "C" int qmoe_probe_mfma(const void* src, int blocks, int iters, float* out, void* stream) {
  if (!src || !out || blocks <= 0 || iters <= 0) return 1;
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const bf16x8*>(src), iters, out);
  return int(hipGetLastError());
}

// Flops of one qmoe_probe_mfma call.
extern "C" double qmoe_probe_mfma_flops(int blocks, int iters) {
  return double(blocks) * 4.0 /* waves */ * double(iters) * 32.0 * (2.0 * 32 * 32 * 16);
}
