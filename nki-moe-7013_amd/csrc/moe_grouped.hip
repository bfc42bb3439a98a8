// Prefill-shape expert MLPs as two grouped GEMMs on bf16 MFMA.
//
// The row-tile table from qmoe_moe_permute (tile_m <= 256) lists, for every
// expert, runs of at most 256 expert-sorted slots.  Each item of work is one
// (row tile, 256-row weight panel) pair on the direct-to-LDS pipeline of
// mfma_wide.hpp (512 threads; A = 256 weight rows, B = up to 256 tokens; one
// workgroup per CU).  Two pipelines share the kernel, chosen per tile:
//   - more than 64 live rows: 256 x 256 x 32 stages, four deep, only the
//     live 32-row token blocks computed;
//   - at most 64 live rows (cold experts, where streaming the weights is the
//     whole cost): 256 x 64 x 64 stages, four deep, so three 32 KB weight
//     slabs are in flight and one barrier covers 64 columns of K.
//
//   gate_up:  A = 256 packed rows of w13[e] (32 gate rows next to their 32 up
//             rows), B rows gathered on load from x[slot_token[s]] (no
//             permuted copy of X; rows past the run read as zeros).  A wave's
//             two A blocks are one gate block and its up block, so the SwiGLU
//             epilogue act = bf16(silu(g) * u) is elementwise in fp32.
//   down:     A = 256 rows h of w2[e] in the blocked layout [I/8][H][8]: the
//             16-byte chunk (h, k..k+7) sits at ((k/8)*H + h)*16, so a stage
//             of BK columns is BK/8 chunks of every row, BK/8*H*16 bytes
//             further on per stage; B = act[s] (contiguous in slot order).
//   Both epilogues stage the bf16 tile through LDS (rows padded by 16 bytes)
//   and write whole 16-byte chunks of contiguous output rows.
//
// Work distribution: persistent workgroups (one per CU) take (tile, panel)
// items from per-XCD queues; see the queue helpers below.  Both GEMMs run in
// one launch (moe_experts_fused_kernel) when the act rows are whole cache
// lines, else as two launches.
#include <atomic>

#include "mfma_wide.hpp"


namespace qmoe {

namespace {
// Full and partial tiles (more than 64 live rows): 256 x 256 x 32, four
// stages (three 32 KB stages in flight: a tile's weights are usually
// streamed from HBM), 8 waves (2 per SIMD) of 64 x 128.
using Hot = pipe::Wide<4, 2, 32, 4, 256>;
// Cold tiles (at most 64 live rows: weight streaming dominates): 256 x 64 x 64,
// four stages, so three 32 KB weight slabs are in flight and a barrier covers
// 64 columns of K.
using Cold = pipe::Wide<4, 2, 64, 4, 64>;
constexpr int COLD_MAX_ROWS = Cold::BN;
constexpr int PIPE_SMEM = Hot::SMEM > Cold::SMEM ? Hot::SMEM : Cold::SMEM;
constexpr int PANEL = Hot::BM;
static_assert(Hot::BM == Cold::BM && Hot::THREADS == Cold::THREADS, "one grid for both pipelines");
static_assert(Cold::BK % QMOE_W2_BLOCK == 0 && Hot::BK % QMOE_W2_BLOCK == 0, "a stage covers whole w2 blocks");
static_assert(PANEL % (2 * QMOE_W13_GROUP) == 0 && QMOE_W13_GROUP == 32,
              "a wave's 64 packed w13 rows are one gate block and its up block");

// Epilogue staging rows (bf16 elements): PANEL/2 act units or PANEL y columns + 16 B.
constexpr int ACT_LD = PANEL / 2 + 8, Y_LD = PANEL + 8;
constexpr int EPI_SMEM = Hot::BN * Y_LD * 2;
constexpr int SMEM = PIPE_SMEM > EPI_SMEM ? PIPE_SMEM : EPI_SMEM;
static_assert(SMEM <= 160 * 1024, "LDS");

struct TileJob {
  int e, s0, rows, n0;
};

// Work queues.  One persistent workgroup per CU takes (tile, weight panel)
// items, tile-major with panels fastest.  XCD v owns the v-th of 8 equal
// contiguous shares of the items and hands them out in order through its
// counter, as the hardware dispatcher would: one XCD works through
// consecutive tiles (mostly one expert at a time) and its L2 serves that
// expert's weight panels and the tiles' token rows to all of them.  A
// workgroup whose XCD has run dry takes the next item of another XCD's share,
// so the XCDs finish together whatever the tiles cost (a hot expert's full
// tiles take about twice as long as a cold expert's partial ones).
// meta[META_CTR + 8 * kind + v] = items of share v handed out so far;
// meta[META_DONE + kind] = workgroups finished.  The last workgroup to finish
// puts both back to zero, so the next launch on the same meta starts clean.
constexpr int META_CTR = 4, META_DONE = 20;
static_assert(META_DONE + 2 <= QMOE_META_INTS, "work counters fit in meta");

// The items of one launch in 8 shares: share v = [base(v), base(v) + n(v)).
struct Queue {
  int32_t* ctr;  // meta[META_CTR + 8 * kind], one counter per share
  int q, r, x;   // live = 8 q + r items; x = this workgroup's XCD
  __device__ Queue(int32_t* c, int live, int xcd) : ctr(c), q(live >> 3), r(live & 7), x(xcd) {}
  __device__ int n(int v) const { return q + (v < r ? 1 : 0); }
  __device__ int base(int v) const { return v * q + min(v, r); }
};

// Next item by scanning the shares, nearest first (own share, then XCD x+1,
// ...), or -1 when all are handed out.  Wave 0 calls it (every lane gets the
// result).  Lanes 0-7 read the 8 counters at once; lane 0 takes an item from
// the first share with items left.  A counter only grows, so a share seen
// exhausted stays so, and a failed take (another workgroup was faster)
// exhausts that share: at most 8 failed rounds, and when every share is
// empty one round of loads decides it (a take per share in turn would cost
// 8 serial atomic round trips at the end of every launch).
__device__ __forceinline__ int claim_scan(const Queue& qu) {
  const int lane = threadIdx.x & 63;
  const int v = (qu.x + lane) & 7;
  for (int round = 0; round < 9; ++round) {
    int left = 0;
    if (lane < 8) left = qu.n(v) - __hip_atomic_load(qu.ctr + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long m = __ballot(lane < 8 && left > 0);
    if (m == 0ull) return -1;
    const int vv = (qu.x + __builtin_ctzll(m)) & 7;
    int j = 0;
    if (lane == 0) j = atomicAdd(qu.ctr + vv, 1);
    j = __builtin_amdgcn_readfirstlane(j);
    if (j < qu.n(vv)) return qu.base(vv) + j;
  }
  return -1;  // not reached: each share can fail a take at most once
}

// The whole workgroup's item (through LDS word 0, which no tile is using
// between items), -1 when done.  `reserve` is thread 0's take of its own
// share's next item, issued when the previous item started so that its
// latency hid behind the tile (NO_RESERVE: none was taken).
constexpr int NO_RESERVE = -(1 << 30);
__device__ __forceinline__ int next_item(const Queue& qu, int reserve, uint8_t* smem) {
  int* slot = reinterpret_cast<int*>(smem);
  __syncthreads();  // the previous tile's epilogue has read its LDS
  if (threadIdx.x < 64) {
    const int j = __builtin_amdgcn_readfirstlane(reserve);
    const int item = (j >= 0 && j < qu.n(qu.x)) ? qu.base(qu.x) + j : claim_scan(qu);
    if (threadIdx.x == 0) slot[0] = item;
  }
  __syncthreads();
  const int item = slot[0];
  __syncthreads();  // every wave has it before the next tile's DMA lands
  return item;
}

// Thread 0's take of the next item of its own share (the result is read only
// by the next next_item), while the share has more than one more item per
// workgroup of the XCD left after `item`: a reserved item cannot move to a
// workgroup that finishes first, so the last round is claimed on demand.
// The kernels reserve only while a cold tile (weight streaming, at most 64
// rows) runs: with every item cold (T = 128) this hides the take's round
// trip (about 1 us an item, 4% of the launch); reserving during hot tiles
// measured slower under skewed routing.
__device__ __forceinline__ int reserve_own(const Queue& qu, int item) {
  const int own = item - qu.base(qu.x);
  const bool early = own >= 0 && own < qu.n(qu.x) && qu.n(qu.x) - own - 1 > int(gridDim.x >> 3);
  return (early && threadIdx.x == 0) ? atomicAdd(qu.ctr + qu.x, 1) : NO_RESERVE;
}

__device__ __forceinline__ void finish_queue(int32_t* ctr, int32_t* done) {
  if (threadIdx.x == 0 && atomicAdd(done, 1) == int(gridDim.x) - 1) {
    // every other workgroup has made its last claim
    for (int v = 0; v < 8; ++v) atomicExch(ctr + v, 0);
    atomicExch(done, 0);
  }
}

__device__ __forceinline__ TileJob job_of(int item, const int32_t* __restrict__ tiles, int npanels) {
  TileJob job;
  const int t = item / npanels;
  job.n0 = (item - t * npanels) * PANEL;
  job.e = tiles[4 * t];
  job.s0 = tiles[4 * t + 1];
  job.rows = min(tiles[4 * t + 2] - job.s0, Hot::BN);
  return job;
}

__device__ __forceinline__ uint2 pack4_bf16(float a, float b, float c, float d) {
  return make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
}

// 16-byte store written through to memory (device scope), so a workgroup on
// another XCD that reads the line after a later signal sees it.
__device__ __forceinline__ void st16_device(void* p, uint4 v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}

// DEVICE: the act rows are stored with st16_device and the wave waits for
// its stores to complete (the single-launch form signals the tile after it).
template <class P, bool DEVICE>
__device__ __forceinline__ void gateup_tile(const TileJob& job, const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w13,
                                            const int32_t* __restrict__ slot_token, int T, int H, int I,
                                            uint16_t* act, uint8_t* smem) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const pipe::i32x4 ra = pipe::make_rsrc(w13 + int64_t(job.e) * 2 * I * H, uint32_t(int64_t(2) * I * H * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(x, uint32_t(int64_t(T) * H * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int r = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(r, lane);
    if (j < P::AI)
      vo[j] = job.n0 + r < 2 * I ? uint32_t(job.n0 + r) * uint32_t(H * 2) + c : pipe::PAD;
    else
      vo[j] = r < job.rows ? uint32_t(slot_token[job.s0 + r]) * uint32_t(H * 2) + c : pipe::PAD;
  }
  // The last panel holds 2I - n0 < 256 packed rows when 2I % 256 != 0: the
  // waves whose 64 rows lie past 2I run no MFMAs (they still DMA and meet
  // the barriers), and only the live units are stored.
  const bool live_a = job.n0 + P::wave_arow(wave) < 2 * I;
  const int nbw = live_a ? P::wave_blocks(wave, (job.rows + 31) / 32) : 0;
  const int units = min(PANEL / 2, I - job.n0 / 2);
  typename P::Acc acc;
  P::run_dyn(nbw, ra, rb, vo, H / P::BK, smem, acc, uint32_t(P::BK * 2), uint32_t(P::BK * 2));
  // A block 0 = gate rows, block 1 = up rows of units n0/2 + 32 wm + [0, 32).  The
  // tile goes through LDS ([token][128 units], rows padded to 272 B) so that the
  // global stores are whole 16-byte chunks of contiguous act rows.
  __syncthreads();  // every wave is past its last fragment read
  uint16_t* tl = reinterpret_cast<uint16_t*>(smem);
  const int u_wave = P::wave_arow(wave) / 2 + (lane >> 5) * 4;  // FM/2 (gate, up) block pairs per wave
#pragma unroll
  for (int j = 0; j < P::FN; ++j) {
    if (j >= nbw) break;
    const int tok = P::acc_brow(wave, j, lane);
#pragma unroll
    for (int p = 0; p < P::FM / 2; ++p) {
      const f32x16& g = acc[2 * p][j];
      const f32x16& u = acc[2 * p + 1][j];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint2*>(tl + tok * ACT_LD + u_wave + p * 32 + q * 8) =
            pack4_bf16(silu(g[4 * q]) * u[4 * q], silu(g[4 * q + 1]) * u[4 * q + 1],
                       silu(g[4 * q + 2]) * u[4 * q + 2], silu(g[4 * q + 3]) * u[4 * q + 3]);
    }
  }
  __syncthreads();
  uint16_t* dst = act + int64_t(job.s0) * I + job.n0 / 2;
  const int chunks = units / 8;
  for (int c = threadIdx.x; c < job.rows * chunks; c += P::THREADS) {
    const int r = c / chunks, k = c % chunks;
    const uint4 v = *reinterpret_cast<const uint4*>(tl + r * ACT_LD + k * 8);
    if constexpr (DEVICE)
      st16_device(dst + int64_t(r) * I + k * 8, v);
    else
      *reinterpret_cast<uint4*>(dst + int64_t(r) * I + k * 8) = v;
  }
  if constexpr (DEVICE) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <class P>
__device__ __forceinline__ void down_tile(const TileJob& job, const uint16_t* act,
                                          const uint16_t* __restrict__ w2, int slots, int H, int I,
                                          uint16_t* __restrict__ y_slot, uint8_t* smem) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const pipe::i32x4 ra = pipe::make_rsrc(w2 + int64_t(job.e) * H * I, uint32_t(int64_t(H) * I * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(act, uint32_t(int64_t(slots) * I * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int r = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(r, lane);
    if (j < P::AI)  // chunk index c/16 of this stage = k block; rows h contiguous within a block
      vo[j] = ((c / 16) * uint32_t(H) + uint32_t(job.n0 + r)) * 16u;
    else
      vo[j] = r < job.rows ? uint32_t(job.s0 + r) * uint32_t(I * 2) + c : pipe::PAD;
  }
  const int nbw = P::wave_blocks(wave, (job.rows + 31) / 32);
  typename P::Acc acc;
  P::run_dyn(nbw, ra, rb, vo, I / P::BK, smem, acc, uint32_t(P::BK / QMOE_W2_BLOCK) * uint32_t(H) * 16u,
             uint32_t(P::BK * 2));
  // Through LDS ([token][256 h], rows padded to 528 B), then 16-byte row chunks.
  __syncthreads();
  uint16_t* tl = reinterpret_cast<uint16_t*>(smem);
  const int h_local = P::wave_arow(wave) + (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < P::FN; ++j) {
    if (j >= nbw) break;
    const int tok = P::acc_brow(wave, j, lane);
#pragma unroll
    for (int i = 0; i < P::FM; ++i) {
      const f32x16& a = acc[i][j];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint2*>(tl + tok * Y_LD + h_local + i * 32 + q * 8) =
            pack4_bf16(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    }
  }
  __syncthreads();
  uint16_t* dst = y_slot + int64_t(job.s0) * H + job.n0;
  for (int c = threadIdx.x; c < job.rows * (PANEL / 8); c += P::THREADS) {
    const int r = c / (PANEL / 8), k = c % (PANEL / 8);
    *reinterpret_cast<uint4*>(dst + int64_t(r) * H + k * 8) = *reinterpret_cast<const uint4*>(tl + r * Y_LD + k * 8);
  }
}
}  // namespace

__global__ __launch_bounds__(Hot::THREADS, 1) void moe_gateup_grouped_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ slot_token, const int32_t* __restrict__ tiles, int32_t* meta, int T,
    int H, int I, uint16_t* __restrict__ act) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int npanels = (2 * I + PANEL - 1) / PANEL, live = meta[0] * npanels, xcd = xcc_id();
  int32_t* ctr = meta + META_CTR;
  const Queue qu(ctr, live, xcd);
  for (int item = next_item(qu, NO_RESERVE, smem); item >= 0;) {
    const TileJob job = job_of(item, tiles, npanels);
    const int reserve = job.rows <= COLD_MAX_ROWS ? reserve_own(qu, item) : NO_RESERVE;
    if (job.rows <= COLD_MAX_ROWS)
      gateup_tile<Cold, false>(job, x, w13, slot_token, T, H, I, act, smem);
    else
      gateup_tile<Hot, false>(job, x, w13, slot_token, T, H, I, act, smem);
    item = next_item(qu, reserve, smem);
  }
  finish_queue(ctr, meta + META_DONE);
}

__global__ __launch_bounds__(Hot::THREADS, 1) void moe_down_grouped_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ tiles, int32_t* meta, int slots, int H, int I,
    uint16_t* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int npanels = H / PANEL, live = meta[0] * npanels, xcd = xcc_id();
  int32_t* ctr = meta + META_CTR + 8;
  const Queue qu(ctr, live, xcd);
  for (int item = next_item(qu, NO_RESERVE, smem); item >= 0;) {
    const TileJob job = job_of(item, tiles, npanels);
    const int reserve = job.rows <= COLD_MAX_ROWS ? reserve_own(qu, item) : NO_RESERVE;
    if (job.rows <= COLD_MAX_ROWS && I % Cold::BK == 0)
      down_tile<Cold>(job, act, w2, slots, H, I, y_slot, smem);
    else
      down_tile<Hot>(job, act, w2, slots, H, I, y_slot, smem);
    item = next_item(qu, reserve, smem);
  }
  finish_queue(ctr, meta + META_DONE + 1);
}

// Both GEMMs in one launch.  The workgroups first take gate_up items (queue
// 0), then down items (queue 1), so the down items of early tiles fill the
// CUs that the last gate_up items leave idle, and no launch boundary sits
// between the two.  A down item of tile t reads the act rows of all of
// tile t's gate_up panels: each gate_up item stores its act rows through to
// memory (st16_device), waits for them, and only then adds 1 to the tile's
// counter tiles[4t + 3] (0 from the permute); a down item waits until the
// counter holds every panel.  No other line of those act rows reaches the
// reading XCD's L2 before that (rows are whole cache lines: I % 64 == 0 and
// act 128-byte aligned, checked by the host), so its DMA reads the stored
// values.  Waits cannot deadlock: a workgroup takes down items only after
// every gate_up item has been taken, and gate_up items wait for nothing.  A
// wait still gives up after TILE_WAIT_SPIN polls (it then sets bit 1 of
// meta[2] and goes on).  The last workgroup to finish sets the queue
// counters and the tile counters back to zero.
constexpr int TILE_WAIT_SPIN = 1 << 20;

__device__ __forceinline__ void wait_tile(const int32_t* cnt, int need, int32_t* meta) {
  if (threadIdx.x < 64) {
    bool ok = false;
    for (int n = 0; n < TILE_WAIT_SPIN; ++n) {
      ok = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need;
      if (ok) break;
      __builtin_amdgcn_s_sleep(8);
    }
    if (!ok && threadIdx.x == 0) atomicOr(meta + 2, 2);
  }
  __syncthreads();
}

__global__ __launch_bounds__(Hot::THREADS, 1) void moe_experts_fused_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ slot_token, int32_t* tiles, int32_t* meta, int T, int H, int I, int slots,
    uint16_t* act, uint16_t* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int n_tiles = meta[0], np1 = (2 * I + PANEL - 1) / PANEL, np2 = H / PANEL, xcd = xcc_id();
  {
    const Queue qu(meta + META_CTR, n_tiles * np1, xcd);
    for (int item = next_item(qu, NO_RESERVE, smem); item >= 0;) {
      const TileJob job = job_of(item, tiles, np1);
      const int reserve = job.rows <= COLD_MAX_ROWS ? reserve_own(qu, item) : NO_RESERVE;
      if (job.rows <= COLD_MAX_ROWS)
        gateup_tile<Cold, true>(job, x, w13, slot_token, T, H, I, act, smem);
      else
        gateup_tile<Hot, true>(job, x, w13, slot_token, T, H, I, act, smem);
      __syncthreads();  // every wave's act stores are complete
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(tiles + 4 * (item / np1) + 3, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      item = next_item(qu, reserve, smem);
    }
  }
  {
    const Queue qu(meta + META_CTR + 8, n_tiles * np2, xcd);
    for (int item = next_item(qu, NO_RESERVE, smem); item >= 0;) {
      const TileJob job = job_of(item, tiles, np2);
      wait_tile(tiles + 4 * (item / np2) + 3, np1, meta);
      const int reserve = job.rows <= COLD_MAX_ROWS ? reserve_own(qu, item) : NO_RESERVE;
      if (job.rows <= COLD_MAX_ROWS && I % Cold::BK == 0)
        down_tile<Cold>(job, act, w2, slots, H, I, y_slot, smem);
      else
        down_tile<Hot>(job, act, w2, slots, H, I, y_slot, smem);
      item = next_item(qu, reserve, smem);
    }
  }
  int* last = reinterpret_cast<int*>(smem);
  if (threadIdx.x == 0) *last = atomicAdd(meta + META_DONE, 1) == int(gridDim.x) - 1;
  __syncthreads();
  if (*last) {  // every other workgroup is done with the counters
    for (int t = threadIdx.x; t < n_tiles; t += blockDim.x)
      __hip_atomic_store(tiles + 4 * t + 3, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < 16) atomicExch(meta + META_CTR + threadIdx.x, 0);
    if (threadIdx.x == 0) atomicExch(meta + META_DONE, 0);
  }
}

// Workgroups per grouped launch: one per CU (the kernels need all of a CU's
// LDS), no more than there are items.
unsigned grouped_grid(int64_t items) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return unsigned(std::max<int64_t>(1, std::min<int64_t>(n, items)));
}

}  // namespace qmoe

extern "C" int qmoe_moe_experts_grouped(const qmoe_bf16* x, const qmoe_bf16* w13,
                                        const qmoe_bf16* w2, const int32_t* slot_token,
                                        int32_t* tiles, int32_t* meta,
                                        int64_t max_tiles, int64_t T, int64_t H, int64_t I,
                                        int64_t E, int64_t k, qmoe_bf16* act, qmoe_bf16* y_slot,
                                        qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(w13 && w2 && tiles && meta && (T == 0 || (x && slot_token && act && y_slot)),
               "qmoe_moe_experts_grouped: null pointer");
  QMOE_REQUIRE(T >= 0 && T * k < (1ll << 30), "qmoe_moe_experts_grouped: bad T");
  QMOE_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= E, "qmoe_moe_experts_grouped: bad E/k");
  QMOE_REQUIRE(H % 256 == 0 && H > 0, "qmoe_moe_experts_grouped: H %% 256 != 0");
  QMOE_REQUIRE(I % QMOE_W13_GROUP == 0 && I > 0, "qmoe_moe_experts_grouped: I %% 32 != 0");
  // every buffer the DMA reads must stay below 2 GiB (32-bit offsets, PAD above)
  QMOE_REQUIRE(T * H * 2 < (1ll << 31) && T * k * I * 2 < (1ll << 31) && 2 * I * H * 2 < (1ll << 31),
               "qmoe_moe_experts_grouped: operand larger than 2 GiB");
  QMOE_REQUIRE(max_tiles >= (T * k + 255) / 256 + E && max_tiles < (1 << 20),
               "qmoe_moe_experts_grouped: max_tiles must be in [ceil(T*k/256)+E, 2^20)");
  if (T == 0) return QMOE_OK;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_gateup_grouped_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, SMEM);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_down_grouped_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, SMEM);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_experts_fused_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, SMEM);
    return true;
  }();
  (void)attr;
  hipStream_t s = as_stream(stream);
  if (I % 64 == 0 && reinterpret_cast<uintptr_t>(act) % 128 == 0) {  // act rows are whole cache lines
    const unsigned g = grouped_grid(max_tiles * std::max<int64_t>((2 * I + PANEL - 1) / PANEL, H / PANEL));
    hipLaunchKernelGGL(moe_experts_fused_kernel, dim3(g), dim3(Hot::THREADS), SMEM, s, x, w13, w2, slot_token,
                       tiles, meta, int(T), int(H), int(I), int(T * k), act, y_slot);
    return hip_status("qmoe_moe_experts_grouped");
  }
  const unsigned g1 = grouped_grid(max_tiles * ((2 * I + PANEL - 1) / PANEL)), g2 = grouped_grid(max_tiles * (H / PANEL));
  hipLaunchKernelGGL(moe_gateup_grouped_kernel, dim3(g1), dim3(Hot::THREADS), SMEM, s, x, w13, slot_token,
                     tiles, meta, int(T), int(H), int(I), act);
  int rc = hip_status("qmoe_moe_experts_grouped(gate_up)");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_down_grouped_kernel, dim3(g2), dim3(Hot::THREADS), SMEM, s, act, w2, tiles, meta,
                     int(T * k), int(H), int(I), y_slot);
  return hip_status("qmoe_moe_experts_grouped(down)");
}
