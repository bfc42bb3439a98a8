// Per-token softmax -> top-k -> renormalise, one wave64 per token.
//
// Selection runs on the logits (softmax is monotone; ties go to the lower
// expert index); the k weights are exp(l_j - l_max) / sum over the chosen k,
// which equals softmax over all E followed by L1 renormalisation of the k.
// Lanes write their own selected entries (no single-lane epilogue).
#pragma once

#include "common.hpp"

namespace qmoe {

constexpr int ROUTER_MAX_E = 256;
constexpr int ROUTER_MAX_K = 16;

// Selection by k rounds of wave-wide reductions over order-preserving 32-bit
// keys (the monotone bit pattern of the logit): a DPP max finds the largest
// remaining logit, a DPP min the lowest expert index holding it (ties go to
// the lower index); the owner lane records the rank and clears the key.  No
// LDS traffic.
// The weights use the exact logits: exp(l - l_max) / sum over the chosen k.
// lr: the token's E logits (bias already added if any); may point to LDS.
// Writes every slot of out_idx[0..k) / out_w[0..k) (NaN logits rank as -inf).
template <bool MAX>
__device__ __forceinline__ uint32_t dpp_reduce_u32_wave(uint32_t v) {
#define QMOE_RED(CTRL, RM)                                                                     \
  {                                                                                            \
    const uint32_t o = uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), CTRL, RM, 0xf, false)); \
    v = MAX ? max(v, o) : min(v, o);                                                           \
  }
  QMOE_RED(QMOE_DPP_ROW_SHR(1), 0xf)
  QMOE_RED(QMOE_DPP_ROW_SHR(2), 0xf)
  QMOE_RED(QMOE_DPP_ROW_SHR(4), 0xf)
  QMOE_RED(QMOE_DPP_ROW_SHR(8), 0xf)
  QMOE_RED(QMOE_DPP_ROW_BCAST15, 0xa)
  QMOE_RED(QMOE_DPP_ROW_BCAST31, 0xc)
#undef QMOE_RED
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

__device__ __forceinline__ void topk_softmax_wave(const float* lr, int E, int k, int32_t* out_idx,
                                                  float* out_w) {
  constexpr int J = ROUTER_MAX_E / 64;
  const int lane = threadIdx.x & 63;
  float v[J];
  uint32_t key[J];
  int rank[J];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    float l = (e < E) ? lr[e] : -INFINITY;
    l = (l != l) ? -INFINITY : l;
    v[j] = l;
    m = fmaxf(m, l);
    const uint32_t b = __float_as_uint(l);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    key[j] = (e < E) ? ord : 0u;  // valid keys are >= ord(-inf) = 0x007fffff
    rank[j] = -1;
  }
#pragma unroll
  for (int r = 0; r < ROUTER_MAX_K; ++r) {
    if (r < k) {
      uint32_t best = key[0];
#pragma unroll
      for (int j = 1; j < J; ++j) best = max(best, key[j]);
      best = dpp_reduce_u32_wave<true>(best);
      uint32_t cand = 0xffffffffu;
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (key[j] == best) cand = min(cand, uint32_t(lane + 64 * j));
      const uint32_t win = dpp_reduce_u32_wave<false>(cand);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if (uint32_t(lane + 64 * j) == win) {
          rank[j] = r;
          key[j] = 0u;
        }
      }
    }
  }
  m = wave_max(m);
  float p[J];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    p[j] = (rank[j] >= 0) ? expf(v[j] - m) : 0.0f;
    s += p[j];
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (rank[j] >= 0) {
      out_idx[rank[j]] = lane + 64 * j;
      out_w[rank[j]] = p[j] * inv;
    }
  }
}

}  // namespace qmoe
