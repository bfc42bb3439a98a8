// Per-token softmax -> top-k -> renormalise, one wave64 per token.
//
// Selection runs on the logits (softmax is monotone; ties go to the lower
// expert index); the k weights are exp(l_j - l_max) / sum over the chosen k,
// which equals softmax over all E followed by L1 renormalisation of the k.
#pragma once

#include "common.hpp"

namespace qmoe {

constexpr int ROUTER_MAX_E = 256;
constexpr int ROUTER_MAX_K = 16;

// lr: the token's E logits (bias already added if any).  Lane 0 writes
// out_idx[0..k) / out_w[0..k).
__device__ __forceinline__ void topk_softmax_wave(const float* lr, int E, int k, int32_t* out_idx,
                                                  float* out_w) {
  const int lane = threadIdx.x & 63;
  float v[ROUTER_MAX_E / 64];
#pragma unroll
  for (int j = 0; j < ROUTER_MAX_E / 64; ++j) {
    const int e = lane + 64 * j;
    v[j] = (e < E) ? lr[e] : -INFINITY;
  }
  float top_v[ROUTER_MAX_K];
  int top_i[ROUTER_MAX_K];
#pragma unroll
  for (int r = 0; r < ROUTER_MAX_K; ++r) {
    if (r >= k) continue;
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
#pragma unroll
    for (int j = 0; j < ROUTER_MAX_E / 64; ++j)
      if (bi == lane + 64 * j) v[j] = -INFINITY;
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
      out_idx[r] = top_i[r];
      out_w[r] = p[r] * inv;
    }
  }
}

}  // namespace qmoe
