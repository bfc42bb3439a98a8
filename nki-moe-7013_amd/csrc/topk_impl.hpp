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
// remaining logit, a second DPP max over complemented indices the lowest
// expert index holding it (ties go to the lower index); the owner lane
// records the rank and clears the key.  No LDS traffic.
// The weights use the exact logits: exp(l - l_max) / sum over the chosen k.
// lr: the token's E logits (bias already added if any); may point to LDS.
// Writes every slot of out_idx[0..k) / out_w[0..k) (NaN logits rank as -inf).
// Wave-wide unsigned max, lane 63's value broadcast.  Each step is one
// v_max_u32_dpp in place: row_shr with bound_ctrl reads 0 (the identity)
// past a row's start, and the masked row_bcast steps leave the other rows'
// value as it is.  DPP reads a VGPR that the previous VALU op wrote, which
// needs two wait states: the s_nop 1 between steps (and before the first).
// Every lane of the wave must be active.
__device__ __forceinline__ uint32_t dpp_max_u32_wave(uint32_t v) {
  asm volatile(
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(v));
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

// J = keys per lane (E <= 64*J); topk_softmax_wave picks the smallest J.
template <int J>
__device__ __forceinline__ void topk_softmax_wave_j(const float* lr, int E, int k, int32_t* out_idx,
                                                    float* out_w) {
  const int lane = threadIdx.x & 63;
  float v[J];
  uint32_t key[J];
  int rank[J];
  uint32_t top = 0u;  // round 0's key: the largest logit
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    float l = lr[min(e, E - 1)];  // unconditional, so the J loads issue together
    l = (e >= E || l != l) ? -INFINITY : l;
    v[j] = l;
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
      best = dpp_max_u32_wave(best);
      if (r == 0) top = best;
      // lowest index holding `best`: a max over complemented indices
      uint32_t cand = 0u;
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (key[j] == best) cand = max(cand, ~uint32_t(lane + 64 * j));
      const uint32_t win = ~dpp_max_u32_wave(cand);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if (uint32_t(lane + 64 * j) == win) {
          rank[j] = r;
          key[j] = 0u;
        }
      }
    }
  }
  const float m = __uint_as_float((top & 0x80000000u) ? (top & 0x7fffffffu) : ~top);
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

__device__ __forceinline__ void topk_softmax_wave(const float* lr, int E, int k, int32_t* out_idx,
                                                  float* out_w) {
  static_assert(ROUTER_MAX_E == 256, "dispatch below covers E <= 256");
  if (E <= 64)
    topk_softmax_wave_j<1>(lr, E, k, out_idx, out_w);
  else if (E <= 128)
    topk_softmax_wave_j<2>(lr, E, k, out_idx, out_w);
  else
    topk_softmax_wave_j<4>(lr, E, k, out_idx, out_w);
}

}  // namespace qmoe
