// Weighted unpermute-combine with optional fused residual add.
//   out[t] = residual[t] + sum_{j<k} topk_w[t,j] * y_slot[token_slot[t*k+j]]
// The k terms are summed in fp32 in fixed order j = 0..k-1: deterministic, no
// atomics.  HBM-bound: k*H*|y| + 4H (residual) + 4H (out) bytes per token.
#include "common.hpp"

namespace qmoe {

template <bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ y_slot,
                                                      const int32_t* __restrict__ token_slot,
                                                      const float* __restrict__ topk_w,
                                                      const float* residual, int k, int H,
                                                      float* out) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j = 0; j < k; ++j) {
    const int64_t s = token_slot[int64_t(t) * k + j];
    const float w = topk_w[int64_t(t) * k + j];
    float4 y;
    if constexpr (BF16) {
      const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(y_slot) +
                                                      s * H + h);
      y = make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
    } else {
      y = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(y_slot) + s * H + h);
    }
    acc.x = fmaf(w, y.x, acc.x);
    acc.y = fmaf(w, y.y, acc.y);
    acc.z = fmaf(w, y.z, acc.z);
    acc.w = fmaf(w, y.w, acc.w);
  }
  const int64_t o = int64_t(t) * H + h;
  if (residual) {
    const float4 r = *reinterpret_cast<const float4*>(residual + o);
    acc.x += r.x;
    acc.y += r.y;
    acc.z += r.z;
    acc.w += r.w;
  }
  *reinterpret_cast<float4*>(out + o) = acc;
}

}  // namespace qmoe

extern "C" int qmoe_moe_combine(const void* y_slot, int y_is_bf16, const int32_t* token_slot,
                                const float* topk_w, const float* residual, int64_t T, int64_t k,
                                int64_t H, float* out, qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(y_slot && token_slot && topk_w && out, "qmoe_moe_combine: null pointer");
  QMOE_REQUIRE(T >= 0 && T < (1 << 30) && k > 0 && k <= 64, "qmoe_moe_combine: bad T/k");
  QMOE_REQUIRE(H > 0 && H % 4 == 0 && H < (1 << 24), "qmoe_moe_combine: H %% 4 != 0");
  if (T == 0) return QMOE_OK;
  dim3 grid(unsigned(T), unsigned((H / 4 + 255) / 256));
  if (y_is_bf16)
    hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, as_stream(stream), y_slot,
                       token_slot, topk_w, residual, int(k), int(H), out);
  else
    hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, as_stream(stream), y_slot,
                       token_slot, topk_w, residual, int(k), int(H), out);
  return hip_status("qmoe_moe_combine");
}
