// Direct-to-LDS multi-stage bf16 MFMA pipeline for gfx950 (CDNA4).
//
// One workgroup of 256 threads (4 wave64s in a 2x2 grid) computes a BM x BN
// fp32 tile  C = A . B^T  where A rows and B rows are both K-contiguous bf16
// ("NT": every operand is read along K).  Each wave owns a (BM/2) x (BN/2)
// sub-tile of v_mfma_f32_32x32x16_bf16 blocks, accumulators in AGPRs.
//
// Loads.  Operands go global -> LDS with `buffer_load_dwordx4 ... lds` (the
// LDS-DMA path): no VGPR staging, so S stages of BK columns can be in flight
// at once.  One DMA instruction writes 64 lanes x 16 B = 1 KB of LDS at
// M0 + 16*lane; each lane chooses its source, so the caller gathers rows
// freely (per-lane 32-bit byte offsets into a buffer resource).  A source
// offset past the resource's size reads as zero: padding rows cost nothing
// and need no branch.
//
// LDS layout.  A stage holds BM then BN rows of BK bf16 (BK*2 bytes, no pad).
// The 16-byte chunk c of row r sits at slot c ^ f(r), f(r) = (r / (16/CH)) % CH
// with CH = BK/8 chunks per row, so the ds_read_b128 of an MFMA fragment
// (16 consecutive rows, one chunk) touches 16 distinct 16-byte bank groups.
//
// Synchronisation.  The DMA counts in vmcnt like any vector load.  A stage is
// waited for with an explicit `s_waitcnt vmcnt(n)` (n = DMA instructions
// issued after it), then one barrier makes every wave's part visible and
// releases the buffer that the next DMA overwrites.  The compiler does not
// see the DMA (inline asm), so it adds no conservative vmcnt(0) of its own.
//
// Accumulator layout of one 32x32 block (wave64): lane l holds column l%32,
// and element e is row (e/4)*8 + (l/32)*4 + e%4.
#pragma once

#include "common.hpp"

namespace qmoe {
namespace pipe {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource over [p, p + bytes): raw (stride 0), 32-bit dword format.
__device__ __forceinline__ i32x4 make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(p);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(b)));
  r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(b >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane(int(bytes));
  r.w = 0x00020000;
  return r;
}

// Source offset that reads as zeros (past any resource of < 2 GiB).
constexpr uint32_t PAD = 0x80000000u;

// One LDS-DMA: 16 bytes per lane from rsrc + voff + soff into LDS at
// lds_addr + 16*lane.  M0 carries the wave-uniform LDS address.
__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voff, i32x4 rsrc, uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
      : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BM_, int BN_, int BK_, int S_>
struct Pipe {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, S = S_;
  static constexpr int CH = BK / 8;     // 16-byte chunks per LDS row
  static constexpr int RPI = 64 / CH;   // rows written by one DMA instruction
  static constexpr int ROWB = BK * 2;   // bytes per LDS row
  static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB, STAGE = A_BYTES + B_BYTES;
  static constexpr int SMEM = S * STAGE;
  static constexpr int AI = BM / RPI / 4, BI = BN / RPI / 4, NDMA = AI + BI;  // per wave per stage
  static constexpr int KS = BK / 16;    // MFMA k-steps per stage
  static constexpr int PER = (NDMA + KS - 1) / KS;  // DMA instructions issued per k-step (the last k-steps may issue fewer)
  static constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(S >= 2 && S <= 4, "stages");
  static_assert(AI * RPI * 4 == BM && BI * RPI * 4 == BN, "tile rows per DMA");
  static_assert(FM >= 1 && FN >= 1, "shape");
  static_assert(SMEM <= 160 * 1024, "LDS");

  typedef f32x16 Acc[FM][FN];

  // Tile row fetched by (wave, lane) with DMA instruction j (j < AI: A rows,
  // else B rows), and the byte offset of that lane's 16-byte chunk in the row.
  __device__ static int dma_row(int j, int wave, int lane) {
    return j < AI ? (wave * AI + j) * RPI + lane / CH : (wave * BI + (j - AI)) * RPI + lane / CH;
  }
  __device__ static uint32_t dma_chunk(int row, int lane) {
    return uint32_t(((lane % CH) ^ ((row / (16 / CH)) % CH)) * 16);
  }
  // Tile row / column of accumulator element (i, j, e) of this lane.
  __device__ static int acc_row(int wave, int i, int e, int lane) {
    return (wave >> 1) * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
  }
  __device__ static int acc_col(int wave, int j, int lane) {
    return (wave & 1) * WN + j * 32 + (lane & 31);
  }

  // acc = A_tile . B_tile^T over nk stages of BK.  vo[j] = source byte offset
  // of DMA instruction j for this lane at k = 0 (PAD for a zero row); the k
  // advance goes in soffset: BK*2 bytes per stage for A, b_step for B (BK*2
  // for a K-contiguous B; other values for blocked B layouts).  Ends with
  // every wave past its last LDS read only after the caller's next barrier,
  // so callers that reuse smem must __syncthreads() first.
  __device__ static void run(i32x4 ra, i32x4 rb, const uint32_t (&vo)[NDMA], int nk, uint8_t* smem,
                             Acc& acc, uint32_t b_step = uint32_t(BK * 2)) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

    auto dma_part = [&](int kt, int part) {
      const uint32_t sb = lds0 + uint32_t((kt % S) * STAGE);
      const uint32_t soff_a = uint32_t(kt * BK * 2), soff_b = uint32_t(kt) * b_step;
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int j = part * PER + q;
        if (j >= NDMA) break;
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
    const uint32_t a_row = uint32_t(((wave >> 1) * WM + (lane & 31)) * ROWB);
    const uint32_t b_row = uint32_t(A_BYTES + ((wave & 1) * WN + (lane & 31)) * ROWB);
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt has landed once at most (stages issued after it) DMA groups are pending
      const int ahead = nk - 1 - kt;
      if (S == 2 || ahead == 0)
        wait_vm<0>();
      else if (S == 3 || ahead == 1)
        wait_vm<(S >= 3 ? NDMA : 0)>();
      else
        wait_vm<(S >= 4 ? 2 * NDMA : 0)>();
      __syncthreads();
      const bool more = kt + S - 1 < nk;
      const uint8_t* sb = smem + (kt % S) * STAGE;
      bf16x8 fa[2][FM], fb[2][FN];
      auto load = [&](int s, int buf) {
        const uint32_t co = uint32_t(((2 * s + hi) ^ f) << 4);
#pragma unroll
        for (int i = 0; i < FM; ++i)
          fa[buf][i] = *reinterpret_cast<const bf16x8*>(sb + a_row + i * 32 * ROWB + co);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          fb[buf][j] = *reinterpret_cast<const bf16x8*>(sb + b_row + j * 32 * ROWB + co);
      };
      load(0, 0);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (s + 1 < KS) load(s + 1, (s + 1) & 1);
        if (more) dma_part(kt + S - 1, s);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
      }
    }
  }
};

// Workgroup -> work-item order that keeps consecutive items on one XCD.
// Workgroups are dispatched round-robin over the 8 XCDs (id % 8); this maps
// hardware ids [0, n) one-to-one onto items [0, n) so that XCD x takes the
// contiguous range of items that starts at x*floor(n/8) + min(x, n%8).  Only
// locality depends on the dispatch rule, never correctness.
__device__ __forceinline__ int xcd_contiguous(int hw, int n) {
  const int x = hw & 7, q = n >> 3, r = n & 7;
  return x * q + min(x, r) + (hw >> 3);
}

}  // namespace pipe
}  // namespace qmoe
