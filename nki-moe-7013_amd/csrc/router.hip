// Router: fp32 logits (GEMM / GEMV with fp32 accumulation), then per token
// softmax -> top-k -> renormalise, one wave64 per token.
//
// Selection runs on the logits (softmax is monotone); the k weights are
// exp(l_j - l_max) / sum over the chosen k, which equals softmax over all E
// followed by the L1 renormalisation of the chosen k.
#include "common.hpp"
#include "gemm.hpp"
#include "topk_impl.hpp"

namespace qmoe {

// Largest token count whose router logits run split-K.
constexpr int64_t ROUTER_SPLIT_MAX_T = 1024;

// With splits > 0 the logits are first summed from the split-K partials
// part[slice][T][E] in slice order (fixed: the same bits every call) and
// written to logits; then the bias is added and the top-k taken.
__global__ __launch_bounds__(256) void topk_softmax_kernel(float* __restrict__ logits,
                                                           const float* __restrict__ bias, int T,
                                                           int E, int k,
                                                           int32_t* __restrict__ topk_idx,
                                                           float* __restrict__ topk_w,
                                                           const float* __restrict__ part, int splits) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  float* lr = logits + int64_t(tok) * E;
  if (splits > 0) {
    // every partial of the lane's logits requested before the first add
    constexpr int J = ROUTER_MAX_E / 64, MAXS = 16;
    float v[J][MAXS];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int q = 0; q < MAXS; ++q) {
        const int e = lane + 64 * j;
        v[j][q] = (e < E && q < splits) ? part[(int64_t(q) * T + tok) * E + e] : 0.0f;
      }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + 64 * j;
      float a = v[j][0];
#pragma unroll
      for (int q = 1; q < MAXS; ++q)
        if (q < splits) a += v[j][q];
      if (e < E) lr[e] = a;  // this lane reads back only its own entries
    }
  }
  if (bias) {
    for (int e = lane; e < E; e += 64) lr[e] += bias[e];
  }
  topk_softmax_wave(lr, E, k, topk_idx + int64_t(tok) * k, topk_w + int64_t(tok) * k);
}

int router_launch(const uint16_t* x, const uint16_t* w_router, const float* bias, int64_t T,
                  int64_t H, int64_t E, int64_t k, int32_t* topk_idx, float* topk_w, float* logits,
                  void* workspace, int64_t workspace_bytes, hipStream_t s) {
  QMOE_REQUIRE(w_router && (T == 0 || (x && topk_idx && topk_w && logits)),
               "qmoe_router_topk: null pointer (logits is required)");
  QMOE_REQUIRE(T >= 0 && T < (1ll << 31), "qmoe_router_topk: bad T");
  QMOE_REQUIRE(E > 0 && E <= ROUTER_MAX_E, "qmoe_router_topk: E must be in [1, 256] (E=%lld)", (long long)E);
  QMOE_REQUIRE(k > 0 && k <= ROUTER_MAX_K && k <= E, "qmoe_router_topk: k must be in [1, min(16, E)]");
  QMOE_REQUIRE(H > 0 && H % 8 == 0, "qmoe_router_topk: H %% 8 != 0");
  if (T == 0) return QMOE_OK;
  if (T <= 16) {
    QMOE_REQUIRE(H % 512 == 0, "qmoe_router_topk: decode path needs H %% 512 == 0");
  } else {
    QMOE_REQUIRE(E % 128 == 0 && H % 64 == 0, "qmoe_router_topk: prefill path needs E %% 128 == 0, H %% 64 == 0");
  }
  // 16 < T <= ROUTER_SPLIT_MAX_T: the logits GEMM has few tiles (E = 128
  // columns) over a long K, so with a workspace it runs split-K (the slices
  // summed by the top-k kernel; at most 16 slices, which that launch sums
  // from registers).  Above that the unsplit GEMM already has 128 tiles at
  // T = 4096 and the slices' extra traffic costs more than it saves
  // (18.9 us unsplit against 21.5 us split for logits + top-k there).
  int splits = 0;
  if (T > 16 && T <= ROUTER_SPLIT_MAX_T &&
      gemm_splitk_bytes(T, E, H) <= 16 * T * E * int64_t(sizeof(float))) {
    if (int rc = gemm_splitk_slices(x, H, w_router, T, E, H, static_cast<float*>(workspace), workspace_bytes,
                                    &splits, s))
      return rc;
  }
  if (splits == 0) {
    int rc = gemm_launch(x, H, w_router, T, E, H, QMOE_GEMM_STORE_F32, logits, E, s);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(topk_softmax_kernel, dim3(unsigned((T + 3) / 4)), dim3(256), 0, s, logits,
                     bias, int(T), int(E), int(k), topk_idx, topk_w, static_cast<const float*>(workspace),
                     splits);
  return hip_status("qmoe_router_topk");
}

int64_t router_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  const int64_t n = T > 16 && T <= ROUTER_SPLIT_MAX_T ? gemm_splitk_bytes(T, E, H) : 0;
  return n <= 16 * T * E * int64_t(sizeof(float)) ? n : 0;
}

}  // namespace qmoe

extern "C" int qmoe_router_topk(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                                int64_t T, int64_t H, int64_t E, int64_t k, int32_t* topk_idx,
                                float* topk_w, float* logits, qmoe_stream_t stream) {
  return qmoe::router_launch(x, w_router, bias, T, H, E, k, topk_idx, topk_w, logits, nullptr, 0,
                             qmoe::as_stream(stream));
}

extern "C" int qmoe_router_topk_ws(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                                   int64_t T, int64_t H, int64_t E, int64_t k, int32_t* topk_idx,
                                   float* topk_w, float* logits, void* workspace, int64_t workspace_bytes,
                                   qmoe_stream_t stream) {
  return qmoe::router_launch(x, w_router, bias, T, H, E, k, topk_idx, topk_w, logits, workspace,
                             workspace_bytes, qmoe::as_stream(stream));
}

extern "C" int64_t qmoe_router_workspace(int64_t T, int64_t H, int64_t E) {
  if (T < 0 || H <= 0 || E <= 0) return -1;
  return qmoe::router_workspace_bytes(T, H, E);
}

extern "C" int qmoe_moe_route(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                              int64_t T, int64_t H, int64_t E, int64_t k, int64_t tile_m,
                              int64_t max_tiles, float* logits, int32_t* topk_idx, float* topk_w,
                              int32_t* counts, int32_t* offsets, int32_t* slot_token,
                              int32_t* token_slot, int32_t* active, int32_t* tiles, int32_t* meta,
                              qmoe_stream_t stream) {
  hipStream_t s = qmoe::as_stream(stream);
  int rc = qmoe::router_launch(x, w_router, bias, T, H, E, k, topk_idx, topk_w, logits, nullptr, 0, s);
  if (rc) return rc;
  return qmoe::permute_launch(topk_idx, T, k, E, tile_m, max_tiles, counts, offsets, slot_token,
                              token_slot, active, tiles, meta, s);
}

extern "C" int qmoe_moe_route_ws(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                                 int64_t T, int64_t H, int64_t E, int64_t k, int64_t tile_m,
                                 int64_t max_tiles, float* logits, int32_t* topk_idx, float* topk_w,
                                 int32_t* counts, int32_t* offsets, int32_t* slot_token,
                                 int32_t* token_slot, int32_t* active, int32_t* tiles, int32_t* meta,
                                 void* workspace, int64_t workspace_bytes, qmoe_stream_t stream) {
  hipStream_t s = qmoe::as_stream(stream);
  int rc = qmoe::router_launch(x, w_router, bias, T, H, E, k, topk_idx, topk_w, logits, workspace,
                               workspace_bytes, s);
  if (rc) return rc;
  return qmoe::permute_launch(topk_idx, T, k, E, tile_m, max_tiles, counts, offsets, slot_token,
                              token_slot, active, tiles, meta, s);
}
