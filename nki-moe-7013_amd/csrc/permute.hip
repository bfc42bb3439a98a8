// Stand-alone dispatch-metadata construction.
//
// Up to PERM_ONE_WG_MAX pairs: one workgroup of 1024 threads runs
// permute_block() (permute_impl.hpp).  Above that, two launches:
//   permute_rank_kernel    one workgroup per chunk of PERM_CHUNK pairs: each
//                          pair's stable rank among the chunk's pairs of the
//                          same expert (into token_slot, used as scratch) and
//                          the chunk's per-expert counts (into slot_token,
//                          used as scratch, followed by a bad-id flag per chunk);
//   permute_place_kernel   one workgroup: chunk bases by a scan over chunks
//                          per expert, the expert-level scans (offsets, active
//                          list, tiles, meta), then every pair's slot =
//                          offsets[e] + base[chunk][e] + rank.
// Both produce the same stable order: within an expert, increasing pair index.
#include "permute_impl.hpp"

namespace qmoe {

constexpr int PERM_THREADS = 1024;
constexpr int PERM_CHUNK = 4096;              // pairs per rank workgroup
constexpr int PERM_MAX_CHUNKS = 32;           // chunk bases held in LDS: 32 x 256 ints
constexpr int PERM_ONE_WG_MAX = 4096;         // pairs handled by the single-workgroup kernel
constexpr int PLACE_UNROLL = 8;

__global__ __launch_bounds__(PERM_THREADS) void permute_rank_kernel(
    const int32_t* __restrict__ topk_idx, int N, int E, int32_t* __restrict__ rank,
    int32_t* __restrict__ chunk_scratch) {
  __shared__ int run[PERM_MAX_E];
  __shared__ int wave_cnt[PERM_THREADS / 64][PERM_MAX_E];
  __shared__ int bad;
  const int t = threadIdx.x, c = blockIdx.x;
  const int c0 = c * PERM_CHUNK, n = min(PERM_CHUNK, N - c0);
  if (t < PERM_MAX_E) run[t] = 0;
  if (t == 0) bad = 0;
  __syncthreads();
  for (int s = c0 + t; s < c0 + n; s += PERM_THREADS) {
    const int e = topk_idx[s];
    if (e < 0 || e >= E) bad = 1;
  }
  __syncthreads();
  const int nchunks = int(gridDim.x);
  if (bad) {  // ranks are meaningless; the place kernel reports the error
    if (t == 0) chunk_scratch[nchunks * E + c] = 1;
    return;
  }
  rank_range<PERM_THREADS>(topk_idx, c0, n, rank, run, wave_cnt, E);
  if (t < E) chunk_scratch[c * E + t] = run[t];
  if (t == 0) chunk_scratch[nchunks * E + c] = 0;
}

// slot_token and token_slot are distinct buffers (restrict lets the placement
// loads run ahead of its stores).
__global__ __launch_bounds__(PERM_THREADS) void permute_place_kernel(
    const int32_t* __restrict__ topk_idx, int N, int k, int E, int tile_m, int nchunks,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ slot_token,
    int32_t* __restrict__ token_slot, int32_t* __restrict__ active, int32_t* __restrict__ tiles,
    int32_t* __restrict__ meta) {
  __shared__ int base[PERM_MAX_CHUNKS][PERM_MAX_E];
  __shared__ int carry[4];
  __shared__ int bad;
  const int t = threadIdx.x;
  if (t == 0) bad = 0;
  __syncthreads();
  // every read of the scratch (slot_token) happens before the first write
  for (int i = t; i < nchunks * E; i += PERM_THREADS) base[i / E][i % E] = slot_token[i];
  for (int c = t; c < nchunks; c += PERM_THREADS)
    if (slot_token[nchunks * E + c]) bad = 1;
  __syncthreads();
  if (bad) {
    // Out-of-range expert ids: report an empty dispatch (meta[2] = 1) and set
    // the slot maps to the identity so later kernels stay in bounds.
    for (int s = t; s < N; s += PERM_THREADS) {
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
  int cnt = 0;
  if (t < E) {
    for (int c = 0; c < nchunks; ++c) {
      const int m = base[c][t];
      base[c][t] = cnt;
      cnt += m;
    }
  }
  const int ntile = (cnt + tile_m - 1) / tile_m;
  const int inc_rows = block_scan_256(cnt, carry);
  const int inc_act = block_scan_256(cnt > 0 ? 1 : 0, carry);
  const int inc_tiles = block_scan_256(ntile, carry);
  if (t < E) {
    const int off = inc_rows - cnt;
    counts[t] = cnt;
    offsets[t] = off;
    if (t == E - 1) {
      offsets[E] = inc_rows;
      meta[0] = inc_tiles;
      meta[1] = inc_act;
      meta[2] = 0;
    }
    if (cnt > 0) active[inc_act - 1] = t;
    int tile = inc_tiles - ntile;
    for (int r0 = 0; r0 < cnt; r0 += tile_m, ++tile) {
      int32_t* tp = tiles + 4 * int64_t(tile);
      tp[0] = t;
      tp[1] = off + r0;
      tp[2] = off + min(r0 + tile_m, cnt);
      tp[3] = 0;
    }
    for (int c = 0; c < nchunks; ++c) base[c][t] += off;
  }
  __syncthreads();
  // PLACE_UNROLL pairs per thread per round: all their loads are issued
  // before the first store (the rounds are latency-bound otherwise)
  for (int s0 = t; s0 < N; s0 += PLACE_UNROLL * PERM_THREADS) {
    int e[PLACE_UNROLL], r[PLACE_UNROLL];
#pragma unroll
    for (int u = 0; u < PLACE_UNROLL; ++u) {
      const int s = s0 + u * PERM_THREADS;
      e[u] = s < N ? topk_idx[s] : 0;
      r[u] = s < N ? token_slot[s] : 0;
    }
#pragma unroll
    for (int u = 0; u < PLACE_UNROLL; ++u) {
      const int s = s0 + u * PERM_THREADS;
      if (s < N) {
        const int pos = base[s / PERM_CHUNK][e[u]] + r[u];
        slot_token[pos] = s / k;
        token_slot[s] = pos;
      }
    }
  }
}

__global__ __launch_bounds__(PERM_THREADS) void permute_kernel(
    const int32_t* __restrict__ topk_idx, int N, int k, int E, int tile_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ slot_token,
    int32_t* __restrict__ token_slot, int32_t* __restrict__ active, int32_t* __restrict__ tiles,
    int32_t* __restrict__ meta) {
  __shared__ PermuteSmem<PERM_THREADS> sm;
  permute_block<PERM_THREADS>(topk_idx, N, k, E, tile_m, counts, offsets, slot_token, token_slot,
                              active, tiles, meta, sm);
}

int permute_launch(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E, int64_t tile_m,
                   int64_t max_tiles, int32_t* counts, int32_t* offsets, int32_t* slot_token,
                   int32_t* token_slot, int32_t* active, int32_t* tiles, int32_t* meta,
                   hipStream_t s) {
  QMOE_REQUIRE(topk_idx && counts && offsets && slot_token && token_slot && active && tiles && meta,
               "qmoe_moe_permute: null pointer");
  QMOE_REQUIRE(E > 0 && E <= PERM_MAX_E, "qmoe_moe_permute: E must be in [1, 256]");
  QMOE_REQUIRE(k > 0 && k <= E, "qmoe_moe_permute: k must be in [1, E]");
  QMOE_REQUIRE(T >= 0 && T * k < (1ll << 30), "qmoe_moe_permute: T*k too large");
  QMOE_REQUIRE(tile_m > 0 && tile_m <= (1 << 20), "qmoe_moe_permute: bad tile_m");
  const int64_t need = (T * k + tile_m - 1) / tile_m + E;
  QMOE_REQUIRE(max_tiles >= need, "qmoe_moe_permute: max_tiles=%lld < %lld", (long long)max_tiles,
               (long long)need);
  const int64_t N = T * k;
  const int64_t nchunks = (N + PERM_CHUNK - 1) / PERM_CHUNK;
  if (N <= PERM_ONE_WG_MAX || nchunks > PERM_MAX_CHUNKS) {
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(PERM_THREADS), 0, s, topk_idx, int(N),
                       int(k), int(E), int(tile_m), counts, offsets, slot_token, token_slot,
                       active, tiles, meta);
    return hip_status("qmoe_moe_permute");
  }
  // scratch in slot_token: nchunks*E counts + nchunks flags (<= N here)
  hipLaunchKernelGGL(permute_rank_kernel, dim3(unsigned(nchunks)), dim3(PERM_THREADS), 0, s,
                     topk_idx, int(N), int(E), token_slot, slot_token);
  if (int rc = hip_status("qmoe_moe_permute(rank)")) return rc;
  hipLaunchKernelGGL(permute_place_kernel, dim3(1), dim3(PERM_THREADS), 0, s, topk_idx, int(N),
                     int(k), int(E), int(tile_m), int(nchunks), counts, offsets, slot_token,
                     token_slot, active, tiles, meta);
  return hip_status("qmoe_moe_permute(place)");
}

}  // namespace qmoe

extern "C" int qmoe_moe_permute(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E,
                                int64_t tile_m, int64_t max_tiles, int32_t* counts,
                                int32_t* offsets, int32_t* slot_token, int32_t* token_slot,
                                int32_t* active, int32_t* tiles, int32_t* meta,
                                qmoe_stream_t stream) {
  return qmoe::permute_launch(topk_idx, T, k, E, tile_m, max_tiles, counts, offsets, slot_token,
                              token_slot, active, tiles, meta, qmoe::as_stream(stream));
}
