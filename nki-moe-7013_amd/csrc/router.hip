// Router: fp32 logits (GEMM / GEMV with fp32 accumulation), then per token
// softmax -> top-k -> renormalise, one wave64 per token.
//
// Selection runs on the logits (softmax is monotone); the k weights are
// exp(l_j - l_max) / sum over the chosen k, which equals softmax over all E
// followed by the L1 renormalisation of the chosen k.
#include "common.hpp"
#include "gemm.hpp"

namespace qmoe {

constexpr int ROUTER_MAX_E = 256;
constexpr int ROUTER_MAX_K = 16;

__global__ __launch_bounds__(256) void topk_softmax_kernel(float* __restrict__ logits,
                                                           const float* __restrict__ bias, int T,
                                                           int E, int k,
                                                           int32_t* __restrict__ topk_idx,
                                                           float* __restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  float* lr = logits + int64_t(tok) * E;
  float v[ROUTER_MAX_E / 64];
#pragma unroll
  for (int j = 0; j < ROUTER_MAX_E / 64; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      float l = lr[e];
      if (bias) {
        l += bias[e];
        lr[e] = l;
      }
      v[j] = l;
    } else {
      v[j] = -INFINITY;
    }
  }
  float top_v[ROUTER_MAX_K];
  int top_i[ROUTER_MAX_K];
#pragma unroll
  for (int r = 0; r < ROUTER_MAX_K; ++r) {
    if (r >= k) continue;
    // lane-local best (lowest index on ties: j ascending == e ascending)
    float bv = v[0];
    int bi = lane;
#pragma unroll
    for (int j = 1; j < ROUTER_MAX_E / 64; ++j) {
      if (v[j] > bv) {
        bv = v[j];
        bi = lane + 64 * j;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    top_v[r] = bv;
    top_i[r] = bi;
    if ((bi & 63) == lane) {
#pragma unroll
      for (int j = 0; j < ROUTER_MAX_E / 64; ++j)
        if (bi == lane + 64 * j) v[j] = -INFINITY;
    }
  }
  if (lane == 0) {
    const float m = top_v[0];
    float p[ROUTER_MAX_K];
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < ROUTER_MAX_K; ++r) {
      if (r < k) {
        p[r] = expf(top_v[r] - m);
        s += p[r];
      }
    }
    const float inv = 1.0f / s;
#pragma unroll
    for (int r = 0; r < ROUTER_MAX_K; ++r) {
      if (r >= k) continue;
      topk_idx[int64_t(tok) * k + r] = top_i[r];
      topk_w[int64_t(tok) * k + r] = p[r] * inv;
    }
  }
}

}  // namespace qmoe

extern "C" int qmoe_router_topk(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                                int64_t T, int64_t H, int64_t E, int64_t k, int32_t* topk_idx,
                                float* topk_w, float* logits, qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(x && w_router && topk_idx && topk_w && logits,
               "qmoe_router_topk: null pointer (logits is required)");
  QMOE_REQUIRE(T >= 0 && T < (1ll << 31), "qmoe_router_topk: bad T");
  QMOE_REQUIRE(E > 0 && E <= ROUTER_MAX_E, "qmoe_router_topk: E must be in [1, 256] (E=%lld)", (long long)E);
  QMOE_REQUIRE(k > 0 && k <= ROUTER_MAX_K && k <= E, "qmoe_router_topk: k must be in [1, min(16, E)]");
  QMOE_REQUIRE(H > 0 && H % 8 == 0, "qmoe_router_topk: H %% 8 != 0");
  if (T == 0) return QMOE_OK;
  hipStream_t s = as_stream(stream);
  if (T <= 16) {
    QMOE_REQUIRE(H % 512 == 0, "qmoe_router_topk: decode path needs H %% 512 == 0");
  } else {
    QMOE_REQUIRE(E % 128 == 0 && H % 64 == 0, "qmoe_router_topk: prefill path needs E %% 128 == 0, H %% 64 == 0");
  }
  int rc = gemm_launch(x, H, w_router, T, E, H, QMOE_GEMM_STORE_F32, logits, E, s);
  if (rc) return rc;
  hipLaunchKernelGGL(topk_softmax_kernel, dim3(unsigned((T + 3) / 4)), dim3(256), 0, s, logits,
                     bias, int(T), int(E), int(k), topk_idx, topk_w);
  return hip_status("qmoe_router_topk");
}
