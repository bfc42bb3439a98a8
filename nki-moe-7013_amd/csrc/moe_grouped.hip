// Prefill-shape expert MLPs as two grouped GEMMs on bf16 MFMA.
//
// The row-tile table from qmoe_moe_permute (tile_m = 128) lists, for every
// expert, runs of at most 128 expert-sorted slots.  Each workgroup takes one
// (row tile, 128-column tile) pair:
//
//   gate_up:  A rows gathered on load from x[slot_token[s]] (no permuted copy
//             of X), B = 128 packed rows of w13[e].  The packed layout puts 32
//             gate rows next to their 32 up rows, so each wave's 64 columns are
//             one gate block (ni = 0) and the matching up block (ni = 1) and
//             the SwiGLU epilogue pairs registers of the same lane:
//             act = bf16(silu(g) * u), fp32 before the single cast.
//   down:     A rows = act[s] (already contiguous in slot order),
//             B = 128 rows of w2[e]; epilogue writes y_slot[s] in bf16.
//
// Grid = (column tiles, max_tiles); a workgroup beyond meta[0] tiles exits.
// Column tiles vary fastest so the workgroups sharing one A row tile are
// dispatched together and hit it in L2.
#include "mfma_tile.hpp"

namespace qmoe {

__global__ __launch_bounds__(256) void moe_gateup_grouped_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ slot_token, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ meta, int H, int I, uint16_t* __restrict__ act) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[tile::SMEM_BYTES / 2];
  const int tid = blockIdx.y;
  if (tid >= meta[0]) return;
  const int e = tiles[4 * tid], s0 = tiles[4 * tid + 1], s1 = tiles[4 * tid + 2];
  const int rows = s1 - s0;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * tile::BN;
  const int kc = (t & 7) * 8;
  const uint16_t* we = w13 + int64_t(e) * 2 * I * H;
  const uint16_t* ap[4];
  const uint16_t* bp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = tile::stage_row(t, j);
    ap[j] = (r < rows) ? x + int64_t(slot_token[s0 + r]) * H + kc : nullptr;
    bp[j] = we + int64_t(n0 + r) * H + kc;
  }
  tile::Acc acc;
  tile::mma_128x128(ap, bp, H, smem, acc);
  const int unit = (n0 / 64 + (wave & 1)) * 32 + (lane & 31);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = tile::acc_row(wave, lane, mi, i);
      if (row < rows) {
        const float g = acc.c[mi][0][i], u = acc.c[mi][1][i];
        act[int64_t(s0 + row) * I + unit] = f32_to_bf16(silu(g) * u);
      }
    }
}

__global__ __launch_bounds__(256) void moe_down_grouped_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, int H, int I,
    uint16_t* __restrict__ y_slot) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[tile::SMEM_BYTES / 2];
  const int tid = blockIdx.y;
  if (tid >= meta[0]) return;
  const int e = tiles[4 * tid], s0 = tiles[4 * tid + 1], s1 = tiles[4 * tid + 2];
  const int rows = s1 - s0;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * tile::BN;
  const int kc = (t & 7) * 8;
  const uint16_t* we = w2 + int64_t(e) * H * I;
  const uint16_t* ap[4];
  const uint16_t* bp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = tile::stage_row(t, j);
    ap[j] = (r < rows) ? act + int64_t(s0 + r) * I + kc : nullptr;
    bp[j] = we + int64_t(n0 + r) * I + kc;
  }
  tile::Acc acc;
  tile::mma_128x128(ap, bp, I, smem, acc);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int col = n0 + tile::acc_col(wave, lane, ni);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = tile::acc_row(wave, lane, mi, i);
        if (row < rows) y_slot[int64_t(s0 + row) * H + col] = f32_to_bf16(acc.c[mi][ni][i]);
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
  QMOE_REQUIRE(H % 128 == 0 && H > 0, "qmoe_moe_experts_grouped: H %% 128 != 0");
  QMOE_REQUIRE(I % 64 == 0 && I > 0, "qmoe_moe_experts_grouped: I %% 64 != 0");
  QMOE_REQUIRE(max_tiles >= (T * k + 127) / 128 + E && max_tiles < 65536,
               "qmoe_moe_experts_grouped: max_tiles must be in [ceil(T*k/128)+E, 65535]");
  if (T == 0) return QMOE_OK;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(moe_gateup_grouped_kernel, dim3(unsigned(2 * I / tile::BN), unsigned(max_tiles)),
                     dim3(256), 0, s, x, w13, slot_token, tiles, meta, int(H), int(I), act);
  int rc = hip_status("qmoe_moe_experts_grouped(gate_up)");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_down_grouped_kernel, dim3(unsigned(H / tile::BN), unsigned(max_tiles)),
                     dim3(256), 0, s, act, w2, tiles, meta, int(H), int(I), y_slot);
  return hip_status("qmoe_moe_experts_grouped(down)");
}
