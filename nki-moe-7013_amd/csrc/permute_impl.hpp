// Dispatch-metadata construction inside one workgroup of NT threads
// (NT in {256, 1024}): histogram, exclusive scans, active-expert list, row-tile
// table and the stable permutation, for the single-workgroup permute kernel.
//
// Placement is deterministic and stable: pairs s = t*k + j are processed in
// chunks of NT in order; inside a wave the rank of a pair among the lanes
// routed to the same expert comes from ballot-based match masks (8 ballots
// over the expert-id bits), and the per-wave counts are prefix-summed across
// the waves of the chunk.  Slot order within an expert is increasing s, i.e.
// increasing token.
#pragma once

#include "common.hpp"

namespace qmoe {

constexpr int PERM_MAX_E = 256;

template <int NT>
struct PermuteSmem {
  int count[PERM_MAX_E];
  int run[PERM_MAX_E];
  int wave_cnt[NT / 64][PERM_MAX_E];
  int carry[4];
  int bad;
};

// Inclusive scan over the first 256 threads (others contribute their v too but
// only t < 256 results are used).  Every thread must call it.
__device__ __forceinline__ int block_scan_256(int v, int* carry) {
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

// Zeroes the grouped expert GEMMs' work counters (meta[4..QMOE_META_INTS)).
__device__ __forceinline__ void clear_work_counters(int32_t* meta) {
  const int t = threadIdx.x;
  if (t >= 4 && t < QMOE_META_INTS) meta[t] = 0;
}

// idx: expert id of pair s (N = T*k pairs).  Writes counts[E], offsets[E+1],
// slot_token[N], token_slot[N], active[<=E], tiles[n_tiles][4], meta[0..2]
// and zeroes meta[4..QMOE_META_INTS).
template <int NT>
__device__ void permute_block(const int32_t* idx, int N, int k, int E, int tile_m,
                              int32_t* counts, int32_t* offsets, int32_t* slot_token,
                              int32_t* token_slot, int32_t* active, int32_t* tiles,
                              int32_t* meta, PermuteSmem<NT>& sm) {
  constexpr int WAVES = NT / 64;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  clear_work_counters(meta);
  if (t < PERM_MAX_E) sm.count[t] = 0;
  if (t == 0) sm.bad = 0;
  __syncthreads();
  for (int s = t; s < N; s += NT) {
    const int e = idx[s];
    if (e < 0 || e >= E)
      sm.bad = 1;
    else
      atomicAdd(&sm.count[e], 1);
  }
  __syncthreads();
  if (sm.bad) {
    // Out-of-range expert ids: report an empty dispatch (meta[2] = 1) and set
    // the slot maps to the identity so later kernels stay in bounds.
    for (int s = t; s < N; s += NT) {
      token_slot[s] = s;
      slot_token[s] = s / k;
    }
    if (t == 0) {
      meta[0] = 0;
      meta[1] = 0;
      meta[2] = 1;
    }
    return;
  }
  const int c = (t < E) ? sm.count[t] : 0;
  const int ntile = (c + tile_m - 1) / tile_m;
  const int inc_rows = block_scan_256(c, sm.carry);
  const int inc_act = block_scan_256(c > 0 ? 1 : 0, sm.carry);
  const int inc_tiles = block_scan_256(ntile, sm.carry);
  if (t < E) {
    const int base = inc_rows - c;
    counts[t] = c;
    offsets[t] = base;
    if (t == E - 1) {
      offsets[E] = inc_rows;
      meta[0] = inc_tiles;
      meta[1] = inc_act;
      meta[2] = 0;
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
    sm.run[t] = base;
  }
  __syncthreads();

  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c0 = 0; c0 < N; c0 += NT) {
    const int s = c0 + t;
    const bool valid = s < N;
    const int e = valid ? idx[s] : 0;
    unsigned long long match = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long bal = __ballot((e >> b) & 1);
      match &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank = __popcll(match & lt_mask);
    const int cnt = __popcll(match);
    for (int i = t; i < WAVES * PERM_MAX_E; i += NT) (&sm.wave_cnt[0][0])[i] = 0;
    __syncthreads();
    if (valid && rank == 0) sm.wave_cnt[wave][e] = cnt;
    __syncthreads();
    if (t < E) {
      int run = sm.run[t];
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const int n = sm.wave_cnt[w][t];
        sm.wave_cnt[w][t] = run;
        run += n;
      }
      sm.run[t] = run;
    }
    __syncthreads();
    if (valid) {
      const int pos = sm.wave_cnt[wave][e] + rank;
      slot_token[pos] = s / k;
      token_slot[s] = pos;
    }
    __syncthreads();
  }
}

// One round of NT consecutive pairs, thread t holding pair t's expert e
// (valid = the pair exists; e in [0, E) when valid): returns run[e] on entry
// plus the number of earlier pairs of the round routed to the same expert
// (stable: increasing pair index); run[e] ends up advanced by the round's
// count of expert e.  Same wave-ballot / cross-wave prefix scheme as
// permute_block.  Every thread must call it.
template <int NT>
__device__ int rank_round(int e, bool valid, int* run, int (&wave_cnt)[NT / 64][PERM_MAX_E], int E) {
  constexpr int WAVES = NT / 64;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  if (!valid) e = 0;
  unsigned long long match = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const unsigned long long bal = __ballot((e >> b) & 1);
    match &= ((e >> b) & 1) ? bal : ~bal;
  }
  const int rank = __popcll(match & lt_mask);
  const int cnt = __popcll(match);
  for (int i = t; i < WAVES * PERM_MAX_E; i += NT) (&wave_cnt[0][0])[i] = 0;
  __syncthreads();
  if (valid && rank == 0) wave_cnt[wave][e] = cnt;
  __syncthreads();
  if (t < E) {
    int r = run[t];
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const int m = wave_cnt[w][t];
      wave_cnt[w][t] = r;
      r += m;
    }
    run[t] = r;
  }
  __syncthreads();
  const int out = valid ? wave_cnt[wave][e] + rank : 0;
  __syncthreads();
  return out;
}

}  // namespace qmoe
