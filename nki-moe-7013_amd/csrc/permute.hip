// Stand-alone dispatch-metadata construction.
//
// Up to PERM_ONE_WG_MAX pairs (or when `tiles` has no room for the scratch
// below): one workgroup of 1024 threads runs permute_block()
// (permute_impl.hpp).  Above that, two launches of one workgroup per chunk of
// PERM_CHUNK pairs:
//   permute_rank_kernel    each pair's stable rank among the chunk's pairs of
//                          the same expert (into token_slot) and the chunk's
//                          per-expert counts and bad-id flag (into the scratch
//                          rows of `tiles` past the tile table);
//   permute_place_kernel   every workgroup sums the chunk counts (all chunks
//                          for the expert totals, the earlier chunks for its
//                          own bases) and runs the expert-level scans; chunk 0
//                          writes counts, offsets, active list, tiles and
//                          meta (work counters zeroed); each workgroup places
//                          its own chunk:
//                          slot = offsets[e] + (rows of e in earlier chunks)
//                          + rank.
// Both produce the same stable order: within an expert, increasing pair index.
// The scratch rows start at row ceil(N / tile_m) + E, which bounds the tile
// table, so the tile writes of chunk 0 never touch what the others read.
#include "permute_impl.hpp"

namespace qmoe {

constexpr int PERM_THREADS = 1024;
constexpr int PERM_CHUNK = PERM_THREADS;  // pairs per workgroup: one per thread
constexpr int PERM_MAX_CHUNKS = 4096;     // chunk counts summed per expert thread
constexpr int PERM_ONE_WG_MAX = 4096;     // pairs handled by the single-workgroup kernel

// Rows of `tiles` the two-launch path needs: the tile table bound plus the
// scratch (per chunk: E counts and one flag, four ints per row); just the
// bound where that path is not taken (too few or too many chunks).
int64_t permute_tiles_rows(int64_t N, int64_t E, int64_t tile_m) {
  const int64_t nchunks = (N + PERM_CHUNK - 1) / PERM_CHUNK;
  const int64_t need = (N + tile_m - 1) / tile_m + E;
  if (N <= PERM_ONE_WG_MAX || nchunks > PERM_MAX_CHUNKS) return need;
  return need + (nchunks * (E + 1) + 3) / 4;
}

__global__ __launch_bounds__(PERM_THREADS) void permute_rank_kernel(
    const int32_t* __restrict__ topk_idx, int N, int E, int32_t* __restrict__ rank,
    int32_t* __restrict__ chunk_scratch) {
  __shared__ int run[PERM_MAX_E];
  __shared__ int wave_cnt[PERM_THREADS / 64][PERM_MAX_E];
  __shared__ int bad;
  const int t = threadIdx.x, c = blockIdx.x, nchunks = int(gridDim.x);
  const int s = c * PERM_CHUNK + t;
  const bool valid = s < N;
  const int e = valid ? topk_idx[s] : 0;
  if (t < PERM_MAX_E) run[t] = 0;
  if (t == 0) bad = 0;
  __syncthreads();
  if (valid && (e < 0 || e >= E)) bad = 1;
  __syncthreads();
  if (bad) {  // ranks are meaningless; the place kernel reports the error
    if (t == 0) chunk_scratch[nchunks * E + c] = 1;
    return;
  }
  const int r = rank_round<PERM_THREADS>(e, valid, run, wave_cnt, E);
  if (valid) rank[s] = r;
  if (t < E) chunk_scratch[c * E + t] = run[t];
  if (t == 0) chunk_scratch[nchunks * E + c] = 0;
}

// chunk_scratch lies in `tiles` past every row chunk 0 writes; slot_token and
// token_slot are distinct buffers (restrict lets the placement loads run ahead
// of its stores).
__global__ __launch_bounds__(PERM_THREADS) void permute_place_kernel(
    const int32_t* __restrict__ topk_idx, int N, int k, int E, int tile_m,
    const int32_t* __restrict__ chunk_scratch, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ slot_token,
    int32_t* __restrict__ token_slot, int32_t* __restrict__ active, int32_t* __restrict__ tiles,
    int32_t* __restrict__ meta) {
  __shared__ int base[PERM_MAX_E];
  __shared__ int carry[4];
  __shared__ int bad;
  const int t = threadIdx.x, c = blockIdx.x, nchunks = int(gridDim.x);
  const int c0 = c * PERM_CHUNK, n = min(PERM_CHUNK, N - c0);
  if (c == 0) clear_work_counters(meta);
  if (t == 0) bad = 0;
  __syncthreads();
  for (int j = t; j < nchunks; j += PERM_THREADS)
    if (chunk_scratch[nchunks * E + j]) bad = 1;
  __syncthreads();
  if (bad) {
    // Out-of-range expert ids: report an empty dispatch (meta[2] = 1) and set
    // the slot maps to the identity so later kernels stay in bounds.
    for (int s = c0 + t; s < c0 + n; s += PERM_THREADS) {
      token_slot[s] = s;
      slot_token[s] = s / k;
    }
    if (c == 0 && t == 0) {
      meta[0] = 0;
      meta[1] = 0;
      meta[2] = 1;
    }
    return;
  }
  int cnt = 0, before = 0;
  if (t < E) {
#pragma unroll 8
    for (int j = 0; j < nchunks; ++j) {
      const int m = chunk_scratch[j * E + t];
      before += j < c ? m : 0;
      cnt += m;
    }
  }
  const int ntile = (cnt + tile_m - 1) / tile_m;
  const int inc_rows = block_scan_256(cnt, carry);
  const int inc_act = block_scan_256(cnt > 0 ? 1 : 0, carry);
  const int inc_tiles = block_scan_256(ntile, carry);
  if (t < E) {
    const int off = inc_rows - cnt;
    base[t] = off + before;
    if (c == 0) {
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
    }
  }
  __syncthreads();
  const int i = c0 + t;
  if (t < n) {
    const int pos = base[topk_idx[i]] + token_slot[i];
    slot_token[pos] = i / k;
    token_slot[i] = pos;
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
  QMOE_REQUIRE(counts && offsets && active && tiles && meta && (T == 0 || (topk_idx && slot_token && token_slot)),
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
  if (N <= PERM_ONE_WG_MAX || nchunks > PERM_MAX_CHUNKS || max_tiles < permute_tiles_rows(N, E, tile_m)) {
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(PERM_THREADS), 0, s, topk_idx, int(N),
                       int(k), int(E), int(tile_m), counts, offsets, slot_token, token_slot,
                       active, tiles, meta);
    return hip_status("qmoe_moe_permute");
  }
  int32_t* scratch = tiles + 4 * need;
  hipLaunchKernelGGL(permute_rank_kernel, dim3(unsigned(nchunks)), dim3(PERM_THREADS), 0, s,
                     topk_idx, int(N), int(E), token_slot, scratch);
  if (int rc = hip_status("qmoe_moe_permute(rank)")) return rc;
  hipLaunchKernelGGL(permute_place_kernel, dim3(unsigned(nchunks)), dim3(PERM_THREADS), 0, s,
                     topk_idx, int(N), int(k), int(E), int(tile_m), scratch, counts, offsets,
                     slot_token, token_slot, active, tiles, meta);
  return hip_status("qmoe_moe_permute(place)");
}

}  // namespace qmoe

extern "C" int64_t qmoe_moe_permute_tiles(int64_t T, int64_t k, int64_t E, int64_t tile_m) {
  if (T < 0 || k <= 0 || E <= 0 || tile_m <= 0) return -1;
  return qmoe::permute_tiles_rows(T * k, E, tile_m);
}

extern "C" int qmoe_moe_permute(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E,
                                int64_t tile_m, int64_t max_tiles, int32_t* counts,
                                int32_t* offsets, int32_t* slot_token, int32_t* token_slot,
                                int32_t* active, int32_t* tiles, int32_t* meta,
                                qmoe_stream_t stream) {
  return qmoe::permute_launch(topk_idx, T, k, E, tile_m, max_tiles, counts, offsets, slot_token,
                              token_slot, active, tiles, meta, qmoe::as_stream(stream));
}
