// Stand-alone dispatch-metadata kernel (one workgroup of 1024 threads); the
// construction itself is permute_block() in permute_impl.hpp.
#include "permute_impl.hpp"

namespace qmoe {

constexpr int PERM_THREADS = 1024;

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
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(PERM_THREADS), 0, s, topk_idx, int(T * k),
                     int(k), int(E), int(tile_m), counts, offsets, slot_token, token_slot, active,
                     tiles, meta);
  return hip_status("qmoe_moe_permute");
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
