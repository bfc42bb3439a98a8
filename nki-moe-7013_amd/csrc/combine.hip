// Weighted unpermute-combine with optional fused residual add.
//   out[t] = residual[t] + sum_{j<k} topk_w[t,j] * y_slot[token_slot[t*k+j]]
// The k terms are summed in fp32 in fixed order j = 0..k-1: deterministic, no
// atomics.  HBM-bound: k*H*|y| + 4H (residual) + 4H (out) bytes per token.
// combine_norm_kernel also writes the RMSNorm of each finished row (the next
// layer's input norm), with the bits of rmsnorm_residual_kernel on `out`.
#include "norm_impl.hpp"

namespace qmoe {

template <bool BF16>
__device__ __forceinline__ float4 load_y4(const void* __restrict__ y_slot, int64_t s, int H, int h) {
  if constexpr (BF16) {
    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(y_slot) + s * H + h);
    return make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
  } else {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(y_slot) + s * H + h);
  }
}

__device__ __forceinline__ void fma4(float w, float4 y, float4& acc) {
  acc.x = fmaf(w, y.x, acc.x);
  acc.y = fmaf(w, y.y, acc.y);
  acc.z = fmaf(w, y.z, acc.z);
  acc.w = fmaf(w, y.w, acc.w);
}

// out[t, h..h+3] (before the residual) in the fixed order j = 0..k-1.  KC > 0:
// k == KC, unrolled so that all k gathered rows are requested together (a
// runtime-bounded loop waits for each row before requesting the next).
template <bool BF16, int KC>
__device__ __forceinline__ float4 combine4(const void* __restrict__ y_slot, const int32_t* __restrict__ token_slot,
                                           const float* __restrict__ topk_w, int k, int H, int t, int h) {
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (KC > 0) {
    float4 y[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) y[j] = load_y4<BF16>(y_slot, token_slot[int64_t(t) * KC + j], H, h);
#pragma unroll
    for (int j = 0; j < KC; ++j) fma4(topk_w[int64_t(t) * KC + j], y[j], acc);
  } else {
    for (int j = 0; j < k; ++j)
      fma4(topk_w[int64_t(t) * k + j], load_y4<BF16>(y_slot, token_slot[int64_t(t) * k + j], H, h), acc);
  }
  return acc;
}

// KC > 0, CH > 0: k == KC and H == CH * 4 * NORM_THREADS; the row's slots
// and weights are read once and all CH * KC gathered chunks requested
// together (the sums are those of combine4).
template <bool BF16, int KC, int CH>
__device__ __forceinline__ void combine_row(const void* __restrict__ y_slot, const int32_t* __restrict__ token_slot,
                                            const float* __restrict__ topk_w, int H, int t, float4 (&acc)[CH]) {
  int32_t sl[KC];
  float wj[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    sl[j] = token_slot[int64_t(t) * KC + j];
    wj[j] = topk_w[int64_t(t) * KC + j];
  }
  float4 y[CH][KC];
#pragma unroll
  for (int i = 0; i < CH; ++i)
#pragma unroll
    for (int j = 0; j < KC; ++j) y[i][j] = load_y4<BF16>(y_slot, sl[j], H, 4 * (int(threadIdx.x) + i * NORM_THREADS));
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < KC; ++j) fma4(wj[j], y[i][j], acc[i]);
  }
}

template <bool BF16, int KC, int CH>
__global__ __launch_bounds__(NORM_THREADS) void combine_norm_kernel(
    const void* __restrict__ y_slot, const int32_t* __restrict__ token_slot, const float* __restrict__ topk_w,
    const float* residual, int k, int H, float* out, const uint16_t* __restrict__ rms_w, float eps,
    uint16_t* __restrict__ x_out) {
  const int t = blockIdx.x;
  float4 v[NORM_MAX_CHUNKS];
  float ss = 0.0f;
  const int nchunk = H / 4;
  float4 pre[CH > 0 ? CH : 1];
  if constexpr (CH > 0) combine_row<BF16, KC, CH>(y_slot, token_slot, topk_w, H, t, pre);
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = int(threadIdx.x) + j * NORM_THREADS;
    if (CH > 0 ? j < CH : c < nchunk) {
      float4 acc;
      if constexpr (CH > 0)
        acc = pre[j < CH ? j : 0];
      else
        acc = combine4<BF16, KC>(y_slot, token_slot, topk_w, k, H, t, 4 * c);
      const int64_t o = int64_t(t) * H + 4 * c;
      if (residual) {
        const float4 r = *reinterpret_cast<const float4*>(residual + o);
        acc.x += r.x;
        acc.y += r.y;
        acc.z += r.z;
        acc.w += r.w;
      }
      *reinterpret_cast<float4*>(out + o) = acc;
      v[j] = acc;
      ss += norm_sq4(acc);
    }
  }
  __shared__ float red[NORM_THREADS / 64];
  const float r = norm_rsqrt(ss, H, eps, red);
  uint16_t* xr = x_out + int64_t(t) * H;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = int(threadIdx.x) + j * NORM_THREADS;
    if (c < nchunk) reinterpret_cast<uint2*>(xr)[c] = norm_out4(v[j], r, rms_w, c);
  }
}

template <bool BF16, int KC>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ y_slot,
                                                      const int32_t* __restrict__ token_slot,
                                                      const float* __restrict__ topk_w,
                                                      const float* residual, int k, int H,
                                                      float* out) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  float4 acc = combine4<BF16, KC>(y_slot, token_slot, topk_w, k, H, t, h);
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
  QMOE_REQUIRE(T == 0 || (y_slot && token_slot && topk_w && out), "qmoe_moe_combine: null pointer");
  QMOE_REQUIRE(T >= 0 && T < (1 << 30) && k > 0 && k <= 64, "qmoe_moe_combine: bad T/k");
  QMOE_REQUIRE(H > 0 && H % 4 == 0 && H < (1 << 24), "qmoe_moe_combine: H %% 4 != 0");
  if (T == 0) return QMOE_OK;
  dim3 grid(unsigned(T), unsigned((H / 4 + 255) / 256));
#define QMOE_COMBINE(BF, KC)                                                                               \
  hipLaunchKernelGGL((combine_kernel<BF, KC>), grid, dim3(256), 0, as_stream(stream), y_slot, token_slot, \
                     topk_w, residual, int(k), int(H), out)
  if (y_is_bf16) {
    if (k == 8) QMOE_COMBINE(true, 8); else QMOE_COMBINE(true, 0);
  } else {
    if (k == 8) QMOE_COMBINE(false, 8); else QMOE_COMBINE(false, 0);
  }
#undef QMOE_COMBINE
  return hip_status("qmoe_moe_combine");
}

extern "C" int qmoe_moe_combine_norm(const void* y_slot, int y_is_bf16, const int32_t* token_slot,
                                     const float* topk_w, const float* residual, int64_t T, int64_t k,
                                     int64_t H, float* out, const qmoe_bf16* rms_w, float eps, qmoe_bf16* x_out,
                                     qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(rms_w && (T == 0 || (y_slot && token_slot && topk_w && out && x_out)),
               "qmoe_moe_combine_norm: null pointer");
  QMOE_REQUIRE(T >= 0 && T < (1 << 30) && k > 0 && k <= 64, "qmoe_moe_combine_norm: bad T/k");
  QMOE_REQUIRE(H > 0 && H % 4 == 0 && H <= NORM_THREADS * 4 * NORM_MAX_CHUNKS,
               "qmoe_moe_combine_norm: H must be a multiple of 4 and <= 8192 (H=%lld)", (long long)H);
  QMOE_REQUIRE(eps >= 0.0f, "qmoe_moe_combine_norm: eps < 0");
  if (T == 0) return QMOE_OK;
#define QMOE_COMBINE_NORM(BF, KC, CH)                                                                          \
  hipLaunchKernelGGL((combine_norm_kernel<BF, KC, CH>), dim3(unsigned(T)), dim3(NORM_THREADS), 0,              \
                     as_stream(stream), y_slot, token_slot, topk_w, residual, int(k), int(H), out,               \
                     reinterpret_cast<const uint16_t*>(rms_w), eps, reinterpret_cast<uint16_t*>(x_out))
  const bool two = k == 8 && H == 2 * 4 * NORM_THREADS;  // the Qwen3-30B-A3B shape: top-8, H = 2048
  if (y_is_bf16) {
    if (two) QMOE_COMBINE_NORM(true, 8, 2); else if (k == 8) QMOE_COMBINE_NORM(true, 8, 0); else QMOE_COMBINE_NORM(true, 0, 0);
  } else {
    if (two) QMOE_COMBINE_NORM(false, 8, 2); else if (k == 8) QMOE_COMBINE_NORM(false, 8, 0); else QMOE_COMBINE_NORM(false, 0, 0);
  }
#undef QMOE_COMBINE_NORM
  return hip_status("qmoe_moe_combine_norm");
}
