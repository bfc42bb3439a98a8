// Prefill-shape expert MLPs as two grouped GEMMs on bf16 MFMA.
//
// The row-tile table from qmoe_moe_permute (tile_m = 128) lists, for every
// expert, runs of at most 128 expert-sorted slots.  Each workgroup takes one
// (row tile, 256-column tile) pair on the direct-to-LDS pipeline
// (mfma_pipe.hpp, 128 x 256 x 32, three stages: 72 KB of LDS and at most 256
// registers, so two workgroups share a CU and one's prologue and epilogue
// overlap the other's MFMAs):
//
//   gate_up:  A rows gathered on load from x[slot_token[s]] (no permuted copy
//             of X; rows past the tile's run read as zeros), B = 256 packed
//             rows of w13[e].  The packed layout puts 32 gate rows next to
//             their 32 up rows, so each wave's column blocks pair up as
//             (gate, up) in the same lane and register: the SwiGLU epilogue
//             act = bf16(silu(g) * u) is elementwise, fp32 before the cast.
//   down:     A rows = act[s] (already contiguous in slot order),
//             B = 256 rows h of w2[e] in the blocked layout [I/8][H][8]: the
//             16-byte chunk (h, k..k+7) sits at ((k/8)*H + h)*16, so a stage
//             of BK = 32 columns is 4 chunks of every row, BK/8*H*16 bytes
//             further on per stage; the epilogue writes y_slot[s] in bf16.
//
// Grid: one workgroup per (tile, column tile) up to max_tiles; the live ones
// (tile < meta[0]) are renumbered XCD-contiguously, column tiles fastest, so
// one XCD works through consecutive tiles (mostly one expert at a time) and
// its L2 holds that expert's weight panels and the tiles' token rows.
#include "mfma_pipe.hpp"

namespace qmoe {

namespace {
using GP = pipe::Pipe<128, 256, 32, 3>;
static_assert(GP::BK % QMOE_W2_BLOCK == 0, "a stage covers whole w2 blocks");

struct TileJob {
  int e, s0, rows, n0;
};

// Returns false for a workgroup beyond the live tiles.
__device__ __forceinline__ bool tile_job(const int32_t* __restrict__ tiles,
                                         const int32_t* __restrict__ meta, int ncols, TileJob& job) {
  const int live = meta[0] * ncols;
  const int hw = int(blockIdx.x);
  if (hw >= live) return false;
  const int item = pipe::xcd_contiguous(hw, live);
  const int t = item / ncols;
  job.n0 = (item - t * ncols) * GP::BN;
  job.e = tiles[4 * t];
  job.s0 = tiles[4 * t + 1];
  job.rows = tiles[4 * t + 2] - job.s0;
  return true;
}
}  // namespace

__global__ __launch_bounds__(256, 2) void moe_gateup_grouped_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ slot_token, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ meta, int T, int H, int I, uint16_t* __restrict__ act) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  TileJob job;
  if (!tile_job(tiles, meta, 2 * I / GP::BN, job)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const pipe::i32x4 ra = pipe::make_rsrc(x, uint32_t(int64_t(T) * H * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(w13 + int64_t(job.e) * 2 * I * H, uint32_t(int64_t(2) * I * H * 2));
  uint32_t vo[GP::NDMA];
#pragma unroll
  for (int j = 0; j < GP::NDMA; ++j) {
    const int r = GP::dma_row(j, wave, lane);
    const uint32_t c = GP::dma_chunk(r, lane);
    if (j < GP::AI)
      vo[j] = r < job.rows ? uint32_t(slot_token[job.s0 + r]) * uint32_t(H * 2) + c : pipe::PAD;
    else
      vo[j] = uint32_t(job.n0 + r) * uint32_t(H * 2) + c;
  }
  GP::Acc acc;
  GP::run(ra, rb, vo, H / GP::BK, smem, acc);
  // column blocks (2p, 2p+1) = gate / up rows of units n0/2 + wn*64 + p*32 + [0, 32)
  const int unit0 = job.n0 / 2 + (wave & 1) * (GP::WN / 2) + (lane & 31);
#pragma unroll
  for (int i = 0; i < GP::FM; ++i)
#pragma unroll
    for (int p = 0; p < GP::FN / 2; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = GP::acc_row(wave, i, e, lane);
        if (row < job.rows) {
          const float g = acc[i][2 * p][e], u = acc[i][2 * p + 1][e];
          act[int64_t(job.s0 + row) * I + unit0 + p * 32] = f32_to_bf16(silu(g) * u);
        }
      }
}

__global__ __launch_bounds__(256, 2) void moe_down_grouped_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, int slots, int H, int I,
    uint16_t* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  TileJob job;
  if (!tile_job(tiles, meta, H / GP::BN, job)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const pipe::i32x4 ra = pipe::make_rsrc(act, uint32_t(int64_t(slots) * I * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(w2 + int64_t(job.e) * H * I, uint32_t(int64_t(H) * I * 2));
  uint32_t vo[GP::NDMA];
#pragma unroll
  for (int j = 0; j < GP::NDMA; ++j) {
    const int r = GP::dma_row(j, wave, lane);
    const uint32_t c = GP::dma_chunk(r, lane);
    if (j < GP::AI)
      vo[j] = r < job.rows ? uint32_t(job.s0 + r) * uint32_t(I * 2) + c : pipe::PAD;
    else  // chunk index c/16 of this stage = k block; rows h contiguous within a block
      vo[j] = ((c / 16) * uint32_t(H) + uint32_t(job.n0 + r)) * 16u;
  }
  GP::Acc acc;
  GP::run(ra, rb, vo, I / GP::BK, smem, acc, uint32_t(GP::BK / QMOE_W2_BLOCK) * uint32_t(H) * 16u);
#pragma unroll
  for (int i = 0; i < GP::FM; ++i)
#pragma unroll
    for (int j = 0; j < GP::FN; ++j) {
      const int col = job.n0 + GP::acc_col(wave, j, lane);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = GP::acc_row(wave, i, e, lane);
        if (row < job.rows) y_slot[int64_t(job.s0 + row) * H + col] = f32_to_bf16(acc[i][j][e]);
      }
    }
}

}  // namespace qmoe

extern "C" int qmoe_moe_experts_grouped(const qmoe_bf16* x, const qmoe_bf16* w13,
                                        const qmoe_bf16* w2, const int32_t* slot_token,
                                        const int32_t* tiles, const int32_t* meta,
                                        int64_t max_tiles, int64_t T, int64_t H, int64_t I,
                                        int64_t E, int64_t k, qmoe_bf16* act, qmoe_bf16* y_slot,
                                        qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(x && w13 && w2 && slot_token && tiles && meta && act && y_slot,
               "qmoe_moe_experts_grouped: null pointer");
  QMOE_REQUIRE(T >= 0 && T * k < (1ll << 30), "qmoe_moe_experts_grouped: bad T");
  QMOE_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= E, "qmoe_moe_experts_grouped: bad E/k");
  QMOE_REQUIRE(H % 256 == 0 && H > 0, "qmoe_moe_experts_grouped: H %% 256 != 0");
  QMOE_REQUIRE(I % 128 == 0 && I > 0, "qmoe_moe_experts_grouped: I %% 128 != 0");
  // every buffer the DMA reads must stay below 2 GiB (32-bit offsets, PAD above)
  QMOE_REQUIRE(T * H * 2 < (1ll << 31) && T * k * I * 2 < (1ll << 31) && 2 * I * H * 2 < (1ll << 31),
               "qmoe_moe_experts_grouped: operand larger than 2 GiB");
  QMOE_REQUIRE(max_tiles >= (T * k + 127) / 128 + E && max_tiles < (1 << 20),
               "qmoe_moe_experts_grouped: max_tiles must be in [ceil(T*k/128)+E, 2^20)");
  if (T == 0) return QMOE_OK;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_gateup_grouped_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, GP::SMEM);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_down_grouped_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, GP::SMEM);
    return true;
  }();
  (void)attr;
  hipStream_t s = as_stream(stream);
  const unsigned g1 = unsigned(max_tiles * (2 * I / GP::BN)), g2 = unsigned(max_tiles * (H / GP::BN));
  hipLaunchKernelGGL(moe_gateup_grouped_kernel, dim3(g1), dim3(256), GP::SMEM, s, x, w13, slot_token,
                     tiles, meta, int(T), int(H), int(I), act);
  int rc = hip_status("qmoe_moe_experts_grouped(gate_up)");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_down_grouped_kernel, dim3(g2), dim3(256), GP::SMEM, s, act, w2, tiles, meta,
                     int(T * k), int(H), int(I), y_slot);
  return hip_status("qmoe_moe_experts_grouped(down)");
}
