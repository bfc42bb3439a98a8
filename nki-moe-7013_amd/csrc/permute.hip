// Expert dispatch metadata: histogram, exclusive scan, stable permutation,
// active-expert list and the row-tile table of the grouped GEMM.
//
// One workgroup of 1024 threads.  The histogram uses LDS atomics (order does
// not matter for counts).  Placement is deterministic and stable: pairs
// s = t*k + j are processed in chunks of 1024 in order; inside a wave the rank
// of a pair among the lanes routed to the same expert comes from ballot-based
// match masks (8 ballots over the expert id bits), and wave counts are
// prefix-summed across the 16 waves of the chunk.  So slot order within an
// expert is exactly increasing s, i.e. increasing token.
#include "common.hpp"

namespace qmoe {

constexpr int PERM_THREADS = 1024;
constexpr int PERM_WAVES = PERM_THREADS / 64;
constexpr int PERM_MAX_E = 256;

// Inclusive scan of v over the first `n` (<= 256) threads of the block, using
// wave shuffles plus a 4-entry LDS carry.  Every thread must call it.
__device__ int block_scan_256(int v, int* carry) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (wave < 4 && lane == 63) carry[wave] = v;
  __syncthreads();
  int add = 0;
  for (int w = 0; w < wave && w < 4; ++w) add += carry[w];
  __syncthreads();
  return v + add;
}

__global__ __launch_bounds__(PERM_THREADS) void permute_kernel(
    const int32_t* __restrict__ topk_idx, int N, int k, int E, int tile_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ slot_token,
    int32_t* __restrict__ token_slot, int32_t* __restrict__ active, int32_t* __restrict__ tiles,
    int32_t* __restrict__ meta) {
  __shared__ int s_count[PERM_MAX_E];
  __shared__ int s_run[PERM_MAX_E];
  __shared__ int s_wave[PERM_WAVES][PERM_MAX_E];
  __shared__ int s_carry[4];
  __shared__ int s_bad;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

  if (t < PERM_MAX_E) s_count[t] = 0;
  if (t == 0) s_bad = 0;
  __syncthreads();
  for (int s = t; s < N; s += PERM_THREADS) {
    const int e = topk_idx[s];
    if (e < 0 || e >= E)
      s_bad = 1;
    else
      atomicAdd(&s_count[e], 1);
  }
  __syncthreads();
  if (s_bad) {
    // Out-of-range expert ids: report an empty dispatch instead of writing
    // out of bounds (meta[2] = 1 flags the error to the host).  The slot maps
    // are set to the identity so that later kernels stay in bounds.
    for (int s = t; s < N; s += PERM_THREADS) {
      token_slot[s] = s;
      slot_token[s] = s / k;
    }
    if (t == 0) {
      meta[0] = 0;
      meta[1] = 0;
      meta[2] = 1;
      meta[3] = 0;
    }
    return;
  }

  // exclusive scans: offsets, active-expert index, tile index
  const int c = (t < E) ? s_count[t] : 0;
  const int ntile = (c + tile_m - 1) / tile_m;
  const int inc_rows = block_scan_256(c, s_carry);
  const int inc_act = block_scan_256(c > 0 ? 1 : 0, s_carry);
  const int inc_tiles = block_scan_256(ntile, s_carry);
  if (t < E) {
    const int base = inc_rows - c;
    counts[t] = c;
    offsets[t] = base;
    if (t == E - 1) {
      offsets[E] = inc_rows;
      meta[0] = inc_tiles;
      meta[1] = inc_act;
      meta[2] = 0;
      meta[3] = 0;
    }
    if (c > 0) active[inc_act - 1] = t;
    int tile = inc_tiles - ntile;
    for (int r0 = 0; r0 < c; r0 += tile_m, ++tile) {
      int32_t* tp = tiles + 4 * int64_t(tile);
      tp[0] = t;
      tp[1] = base + r0;
      tp[2] = base + min(r0 + tile_m, c);
      tp[3] = 0;
    }
    s_run[t] = base;
  }
  __syncthreads();

  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c0 = 0; c0 < N; c0 += PERM_THREADS) {
    const int s = c0 + t;
    const bool valid = s < N;
    const int e = valid ? topk_idx[s] : 0;
    unsigned long long match = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long bal = __ballot((e >> b) & 1);
      match &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank = __popcll(match & lt_mask);
    const int cnt = __popcll(match);
    for (int i = t; i < PERM_WAVES * PERM_MAX_E; i += PERM_THREADS) (&s_wave[0][0])[i] = 0;
    __syncthreads();
    if (valid && rank == 0) s_wave[wave][e] = cnt;
    __syncthreads();
    if (t < E) {
      int run = s_run[t];
#pragma unroll
      for (int w = 0; w < PERM_WAVES; ++w) {
        const int n = s_wave[w][t];
        s_wave[w][t] = run;
        run += n;
      }
      s_run[t] = run;
    }
    __syncthreads();
    if (valid) {
      const int pos = s_wave[wave][e] + rank;
      slot_token[pos] = s / k;
      token_slot[s] = pos;
    }
    __syncthreads();
  }
}

}  // namespace qmoe

extern "C" int qmoe_moe_permute(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E,
                                int64_t tile_m, int64_t max_tiles, int32_t* counts,
                                int32_t* offsets, int32_t* slot_token, int32_t* token_slot,
                                int32_t* active, int32_t* tiles, int32_t* meta,
                                qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(topk_idx && counts && offsets && slot_token && token_slot && active && tiles && meta,
               "qmoe_moe_permute: null pointer");
  QMOE_REQUIRE(E > 0 && E <= PERM_MAX_E, "qmoe_moe_permute: E must be in [1, 256]");
  QMOE_REQUIRE(k > 0 && k <= E, "qmoe_moe_permute: k must be in [1, E]");
  QMOE_REQUIRE(T >= 0 && T * k < (1ll << 30), "qmoe_moe_permute: T*k too large");
  QMOE_REQUIRE(tile_m > 0 && tile_m <= (1 << 20), "qmoe_moe_permute: bad tile_m");
  const int64_t need = (T * k + tile_m - 1) / tile_m + E;
  QMOE_REQUIRE(max_tiles >= need, "qmoe_moe_permute: max_tiles=%lld < %lld", (long long)max_tiles,
               (long long)need);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(PERM_THREADS), 0, as_stream(stream), topk_idx,
                     int(T * k), int(k), int(E), int(tile_m), counts, offsets, slot_token,
                     token_slot, active, tiles, meta);
  return hip_status("qmoe_moe_permute");
}
