// Residual RMSNorm: h = x (+ delta); y = bf16(w * h * rsqrt(mean(h^2) + eps)).
// One workgroup per row; each thread keeps its float4 chunks in registers so
// the row is read once.  HBM-bound: 4H (x) [+4H delta] [+4H h] + 2H (y) + 2H (w) bytes.
#include "norm_impl.hpp"

namespace qmoe {

__global__ __launch_bounds__(NORM_THREADS) void rmsnorm_residual_kernel(
    const float* __restrict__ x, const float* __restrict__ delta, const uint16_t* __restrict__ w,
    int H, float eps, float* h_out, uint16_t* __restrict__ y) {
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const float* xr = x + int64_t(row) * H;
  const float* dr = delta ? delta + int64_t(row) * H : nullptr;
  float4 v[NORM_MAX_CHUNKS];
  float ss = 0.0f;
  const int nchunk = H / 4;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = t + j * NORM_THREADS;
    if (c < nchunk) {
      float4 a = reinterpret_cast<const float4*>(xr)[c];
      if (dr) {
        const float4 d = reinterpret_cast<const float4*>(dr)[c];
        a.x += d.x; a.y += d.y; a.z += d.z; a.w += d.w;
      }
      v[j] = a;
      ss += norm_sq4(a);
    }
  }
  __shared__ float red[NORM_THREADS / 64];
  const float r = norm_rsqrt(ss, H, eps, red);
  float* hr = h_out ? h_out + int64_t(row) * H : nullptr;
  uint16_t* yr = y + int64_t(row) * H;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = t + j * NORM_THREADS;
    if (c < nchunk) {
      if (hr) reinterpret_cast<float4*>(hr)[c] = v[j];
      reinterpret_cast<uint2*>(yr)[c] = norm_out4(v[j], r, w, c);
    }
  }
}

}  // namespace qmoe

extern "C" int qmoe_rmsnorm_residual(const float* x, const float* delta, const qmoe_bf16* w,
                                     int64_t rows, int64_t H, float eps, float* h_out,
                                     qmoe_bf16* y_out, qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(w && (rows == 0 || (x && y_out)), "qmoe_rmsnorm_residual: null pointer");
  QMOE_REQUIRE(rows >= 0 && rows < (1ll << 31), "qmoe_rmsnorm_residual: bad rows %lld", (long long)rows);
  QMOE_REQUIRE(H > 0 && H % 4 == 0 && H <= NORM_THREADS * 4 * NORM_MAX_CHUNKS,
               "qmoe_rmsnorm_residual: H must be a multiple of 4 and <= 8192 (H=%lld)", (long long)H);
  QMOE_REQUIRE(eps >= 0.0f, "qmoe_rmsnorm_residual: eps < 0");
  if (rows == 0) return QMOE_OK;
  hipLaunchKernelGGL(rmsnorm_residual_kernel, dim3(unsigned(rows)), dim3(NORM_THREADS), 0,
                     as_stream(stream), x, delta, w, int(H), eps, h_out, y_out);
  return hip_status("qmoe_rmsnorm_residual");
}
