// Direct-to-LDS bf16 MFMA pipeline with a variable number of live B rows, for
// the grouped expert GEMMs (gfx950 / CDNA4).
//
// One workgroup of 2 * WA wave64s (WA along A rows x 2 along B rows) computes
// C = A . B^T for an A panel of BM = 32 * FM * WA rows (expert weight rows)
// and up to BN B rows (tokens).  Wave (wm, wn) = (wave % WA, wave / WA) owns A
// rows [32 FM wm, 32 FM (wm + 1)) and B rows [BN/2 wn, BN/2 (wn + 1)): FM x
// BN/64 blocks of v_mfma_f32_32x32x16_bf16.
//
// Live B rows.  The caller says how many 32-row B blocks hold real rows
// (nb); a wave runs the k-loop instantiated for its own count (0..BN/64
// blocks), so padding past the last live 32-row block costs neither MFMAs
// nor fragment reads.  DMA and barriers are the same in every instantiation:
// all waves load their share of both operands (dead rows use a source offset
// past the resource, which reads zeros without touching memory) and meet at
// the same barriers.
//
// Loads.  Operands go global -> LDS with `buffer_load_dwordx4 ... lds`: one
// instruction writes 64 lanes x 16 B = 1 KB of LDS at M0 + 16 * lane, each
// lane choosing its source (per-lane 32-bit byte offsets into a buffer
// resource), so the caller gathers rows freely.  Chunk c of LDS row r sits at
// slot c ^ ((r / (16/CH)) % CH), which keeps the 16-lane groups of a fragment
// read on distinct banks.
//
// Schedule (S >= 3 stages of BK columns).  The barrier that publishes stage
// kt+1 sits before the last k-step of stage kt: the fragment reads of the
// next stage's first k-step are issued right after it and overlap that
// k-step's MFMAs, so a wave never waits on LDS latency at a stage boundary.
// Stage kt+S-1 is DMA'd during stage kt, spread over its k-steps, into the
// buffer of stage kt-1 (whose last fragment reads completed before the
// barrier of stage kt-1).  A stage is waited for with an explicit vmcnt (the
// DMAs issued after it), exact in steady state and vmcnt(0) near the end.
//
// Accumulator (i, j) of a wave: lane l holds B row (token)
// BN/2 wn + 32 j + l % 32 and, in element e, A row
// 32 FM wm + 32 i + (e / 4) * 8 + (l / 32) * 4 + e % 4, so each lane owns runs
// of 4 consecutive A rows.
#pragma once

#include <type_traits>

#include "mfma_pipe.hpp"

namespace qmoe {
namespace pipe {

template <int WA_, int FM_, int BK_, int S_, int BN_>
struct Wide {
  static constexpr int WA = WA_, FM = FM_;  // waves along A; A blocks per wave
  static constexpr int BM = 32 * FM * WA, BN = BN_, BK = BK_, S = S_, WAVES = 2 * WA, THREADS = 64 * WAVES;
  static constexpr int FN = BN / 64;     // B blocks per wave (at most)
  static constexpr int CH = BK / 8;      // 16-byte chunks per LDS row
  static constexpr int RPI = 64 / CH;    // rows written by one DMA instruction
  static constexpr int ROWB = BK * 2;    // bytes per LDS row
  static constexpr int A_BYTES = BM * ROWB, STAGE = (BM + BN) * ROWB, SMEM = S * STAGE;
  static constexpr int AI = BM / RPI / WAVES, BI = BN / RPI / WAVES, NDMA = AI + BI;  // per wave per stage
  static constexpr int KS = BK / 16;     // MFMA k-steps per stage
  static_assert(WA == 2 || WA == 4, "WA");
  static_assert(FM >= 1 && FM <= 5, "FM");
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(BN == 64 || BN == 128 || BN == 256, "BN");
  static_assert(S >= 3 && S <= 5, "stages");
  static_assert(AI * RPI * WAVES == BM && BI * RPI * WAVES == BN, "shape");
  static_assert(SMEM <= 160 * 1024, "LDS");

  typedef f32x16 Acc[FM][FN];

  __device__ static int dma_row(int j, int wave, int lane) {
    return j < AI ? (wave * AI + j) * RPI + lane / CH : (wave * BI + (j - AI)) * RPI + lane / CH;
  }
  __device__ static uint32_t dma_chunk(int row, int lane) {
    return uint32_t(((lane % CH) ^ ((row / (16 / CH)) % CH)) * 16);
  }
  // First A row of this wave's accumulators; B row of block j for this lane.
  __device__ static int wave_arow(int wave) { return (wave % WA) * FM * 32; }
  __device__ static int acc_brow(int wave, int j, int lane) { return (wave / WA) * (BN / 2) + j * 32 + (lane & 31); }
  // Live 32-row B blocks of this wave, given the tile's live blocks nb (0..BN/32).
  __device__ static int wave_blocks(int wave, int nb) { return min(FN, max(0, nb - FN * (wave / WA))); }

  // acc[i][j] (j < NB) = A_panel . B_rows^T over nk stages of BK.  vo[j] =
  // source byte offset of DMA instruction j for this lane at k = 0 (PAD for a
  // zero row); the k advance goes in soffset: a_step / b_step bytes per
  // stage.  Callers that reuse smem afterwards must __syncthreads() first.
  template <int NB>
  __device__ static void run(i32x4 ra, i32x4 rb, const uint32_t (&vo)[NDMA], int nk, uint8_t* smem, Acc& acc,
                             uint32_t a_step, uint32_t b_step) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[i][j] = f32x16{};

    // DMA instructions [part*NDMA/KS, (part+1)*NDMA/KS) of stage kt
    auto dma_part = [&](int kt, int part) {
      const uint32_t sb = lds0 + uint32_t((kt % S) * STAGE);
      const uint32_t soff_a = uint32_t(kt) * a_step, soff_b = uint32_t(kt) * b_step;
#pragma unroll
      for (int j = part * NDMA / KS; j < (part + 1) * NDMA / KS; ++j) {
        if (j < AI)
          dma16(sb + uint32_t((wave * AI + j) * 1024), vo[j], ra, soff_a);
        else
          dma16(sb + uint32_t(A_BYTES + (wave * BI + (j - AI)) * 1024), vo[j], rb, soff_b);
      }
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
      if (s < nk)
#pragma unroll
        for (int p = 0; p < KS; ++p) dma_part(s, p);

    const int f = ((lane & 31) / (16 / CH)) % CH;
    const int hi = lane >> 5;
    const uint32_t a_row = uint32_t((wave_arow(wave) + (lane & 31)) * ROWB);
    const uint32_t b_row = uint32_t(A_BYTES + ((wave / WA) * (BN / 2) + (lane & 31)) * ROWB);
    constexpr int NBX = NB > 0 ? NB : 1;
    bf16x8 fa[2][FM], fb[2][NBX];
    auto load = [&](int kt, int s, int buf) {
      const uint8_t* sb = smem + (kt % S) * STAGE;
      const uint32_t co = uint32_t(((2 * s + hi) ^ f) << 4);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[buf][i] = *reinterpret_cast<const bf16x8*>(sb + a_row + i * 32 * ROWB + co);
#pragma unroll
      for (int j = 0; j < NB; ++j)
        fb[buf][j] = *reinterpret_cast<const bf16x8*>(sb + b_row + j * 32 * ROWB + co);
    };
    if (nk >= S - 1)
      wait_vm<NDMA * (S - 2)>();
    else
      wait_vm<0>();
    __syncthreads();
    if (NB > 0) load(0, 0, 0);
    // One stage.  MORE: stage kt+S-1 exists and is DMA'd during this one.
    // LAST: no stage follows (no barrier, no next-stage reads).  The three
    // variants are separate straight-line bodies (steady state, drain, last
    // stage): with one body and runtime flags the compiler's wait-count
    // analysis merges the paths and waits on the next stage's fragment reads
    // before the MFMAs of this stage's last k-step, which use fragments
    // loaded long before.
    auto stage = [&](int kt, auto more_c, auto last_c) {
      constexpr bool MORE = decltype(more_c)::value, LAST = decltype(last_c)::value;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (s + 1 < KS) {
          if (NB > 0) load(kt, s + 1, (s + 1) & 1);
        } else if (!LAST) {
          // stage kt+1 landed: the DMAs issued after it are the full stages
          // kt+2..kt+S-2 and the first KS-1 parts of stage kt+S-1
          if (MORE)
            wait_vm<NDMA * (S - 3) + (KS - 1) * NDMA / KS>();
          else
            wait_vm<0>();
          __syncthreads();
          if (NB > 0) load(kt + 1, 0, 0);
        }
        if (MORE) dma_part(kt + S - 1, s);
        // keep the next k-step's fragment reads (and the DMAs) ahead of this
        // k-step's MFMAs: left alone, the scheduler sinks the reads below the
        // MFMAs, reuses the registers and every k-step waits on LDS latency
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    int kt = 0;
    for (; kt < nk - (S - 1); ++kt) stage(kt, T_{}, F_{});
    for (; kt < nk - 1; ++kt) stage(kt, F_{}, F_{});
    if (kt < nk) stage(kt, F_{}, T_{});
  }

  // run<NB> for a runtime block count nb in [0, FN].
  __device__ static void run_dyn(int nb, i32x4 ra, i32x4 rb, const uint32_t (&vo)[NDMA], int nk, uint8_t* smem,
                                 Acc& acc, uint32_t a_step, uint32_t b_step) {
    switch (nb) {
      case 4: if constexpr (FN >= 4) run<4>(ra, rb, vo, nk, smem, acc, a_step, b_step); break;
      case 3: if constexpr (FN >= 3) run<3>(ra, rb, vo, nk, smem, acc, a_step, b_step); break;
      case 2: if constexpr (FN >= 2) run<2>(ra, rb, vo, nk, smem, acc, a_step, b_step); break;
      case 1: run<1>(ra, rb, vo, nk, smem, acc, a_step, b_step); break;
      default: run<0>(ra, rb, vo, nk, smem, acc, a_step, b_step); break;
    }
  }
};

}  // namespace pipe
}  // namespace qmoe
