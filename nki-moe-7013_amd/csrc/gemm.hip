// Dense bf16 GEMM  C = A . B^T  (A [M,K], B [N,K], fp32 accumulate).
//
// Two shapes of work:
//  * M <= 16 ("GEMV", decode): HBM-bound on B.  The M activation rows are
//    staged once in LDS; each wave streams R rows of B with 16-byte
//    non-temporal loads (K/512 loads per row per lane, all in flight), and
//    reduces the per-lane partial dots with cross-lane shuffles.
//  * M > 16: the direct-to-LDS MFMA pipelines (mfma_pipe.hpp; from 224
//    tiles of 256 x 256 on, the deep-staged 8-wave one of mfma_wide.hpp).
#include "decode_util.hpp"
#include "gemm.hpp"
#include "mfma_pipe.hpp"
#include "mfma_wide.hpp"
#include "norm_impl.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace qmoe {

template <int MODE>
__device__ __forceinline__ void store_out(void* C, int64_t idx, float v) {
  if constexpr (MODE == QMOE_GEMM_STORE_BF16) {
    reinterpret_cast<uint16_t*>(C)[idx] = f32_to_bf16(v);
  } else if constexpr (MODE == QMOE_GEMM_STORE_F32) {
    reinterpret_cast<float*>(C)[idx] = v;
  } else {
    reinterpret_cast<float*>(C)[idx] += v;
  }
}

// ------------------------------------------------------------------ GEMV
template <int MT, int R, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                   const uint16_t* __restrict__ B, int M, int N,
                                                   int K, void* __restrict__ C, int64_t ldc) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // stage the M activation rows (16-byte chunks)
  const int kchunks = K / 8;
  stage16<256, 16>(reinterpret_cast<u32x4*>(xs), M * kchunks, [&](int c) {
    const int m = c / kchunks;
    return A + m * lda + (c - m * kchunks) * 8;
  });
  __syncthreads();

  const int n0 = (blockIdx.x * 4 + wave) * R;
  float acc[MT][R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  const uint16_t* brow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) brow[r] = B + int64_t(min(n0 + r, N - 1)) * K;

#pragma unroll 4
  for (int k = lane * 8; k < K; k += 512) {
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = ld_stream(brow[r] + k);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + m * K + k);
        float x8[8] = {bf16_lo(xv.x), bf16_hi(xv.x), bf16_lo(xv.y), bf16_hi(xv.y),
                       bf16_lo(xv.z), bf16_hi(xv.z), bf16_lo(xv.w), bf16_hi(xv.w)};
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] += dot8(w[r], x8);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m < M) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[m][r]);
        if (lane == 0 && n0 + r < N) store_out<MODE>(C, int64_t(m) * ldc + n0 + r, v);
      }
    }
  }
}

// GEMV for K = 512 * KC <= 4096: every weight load of a wave (R rows x KC
// 16-byte chunks per lane) is issued before the activation rows are staged,
// so the weight stream starts with the workgroup and all of it is in flight
// at once (R * KC <= 16 loads per lane).
template <int MT, int R, int KC, int MODE>
__global__ __launch_bounds__(256) void gemv_reg_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                       const uint16_t* __restrict__ B, int M, int N,
                                                       int K, void* __restrict__ C, int64_t ldc) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  u32x4 w[R][KC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint16_t* brow = B + int64_t(min(n0 + r, N - 1)) * K + lane * 8;
#pragma unroll
    for (int c = 0; c < KC; ++c) w[r][c] = ld_stream(brow + c * 512);
  }
  const int kchunks = K / 8;
  stage16<256, 16>(reinterpret_cast<u32x4*>(xs), M * kchunks, [&](int c) {
    const int m = c / kchunks;
    return A + m * lda + (c - m * kchunks) * 8;
  });
  __syncthreads();
  float acc[MT][R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + m * K + c * 512 + lane * 8);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = dot8_bf16(w[r][c], xv, acc[m][r]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m < M) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[m][r]);
        if (lane == 0 && n0 + r < N) store_out<MODE>(C, int64_t(m) * ldc + n0 + r, v);
      }
    }
  }
}

// Single-row GEMV with the input RMSNorm fused into the activation staging:
// x = bf16(w_rms * h * rsqrt(mean(h^2) + eps)) from the fp32 residual row h,
// with the same chunking, summation order and rounding as
// rmsnorm_residual_kernel (so x has the same bits), then the one-row-per-wave
// dot of gemv_reg_kernel.  Weight loads are issued first, so the norm's
// reduction overlaps the weight stream.
template <int KC, int MODE>
__global__ __launch_bounds__(256) void gemv_rms_kernel(const float* __restrict__ h,
                                                       const uint16_t* __restrict__ rms_w, float eps,
                                                       const uint16_t* __restrict__ B, int N,
                                                       void* __restrict__ C) {
  constexpr int K = KC * 512, NCH = K / 4 / 256 > 0 ? K / 4 / 256 : 1;  // float4 chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t xs[K];
  __shared__ float red[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * 4 + wave;
  u32x4 w[KC];
  {
    const uint16_t* brow = B + int64_t(min(n0, N - 1)) * K + lane * 8;
#pragma unroll
    for (int c = 0; c < KC; ++c) w[c] = ld_stream(brow + c * 512);
  }
  float4 v[NCH];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = t + j * 256;
    if (c < K / 4) {
      const float4 a = reinterpret_cast<const float4*>(h)[c];
      v[j] = a;
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) tot += red[i];
  const float r = rsqrtf(tot / float(K) + eps);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = t + j * 256;
    if (c < K / 4) {
      const float4 a = v[j];
      const uint2 wv = reinterpret_cast<const uint2*>(rms_w)[c];
      uint2 o;
      o.x = pack_bf16x2(bf16_lo(wv.x) * (a.x * r), bf16_hi(wv.x) * (a.y * r));
      o.y = pack_bf16x2(bf16_lo(wv.y) * (a.z * r), bf16_hi(wv.y) * (a.w * r));
      reinterpret_cast<uint2*>(xs)[c] = o;
    }
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < KC; ++c)
    acc = dot8_bf16(w[c], *reinterpret_cast<const u32x4*>(xs + c * 512 + lane * 8), acc);
  const float out = wave_sum(acc);
  if (lane == 0 && n0 < N) store_out<MODE>(C, n0, out);
}

// Skinny GEMM for 2 <= M <= 16 rows of A (batched decode), K = 128 * KS:
// v_mfma_f32_16x16x32_bf16 with the A rows padded to 16 (zeros past M).  A
// workgroup owns NB (8 or 16) output columns; wave w owns the K range
// [w*K/4, (w+1)*K/4): its KS B operands (16 bytes of a weight row each, lane
// l -> column l % 16, k offset (l / 16) * 8) are all loaded before A is
// staged (plain loads: a load touches half of each 128-byte line and the next
// one the other half, which the nontemporal form does not keep in L1; 3-4%
// faster), the KS MFMAs accumulate, and the four waves' 16x16 partials are
// added in wave order through LDS.  HBM-bound like the M = 1 GEMV: the
// arithmetic that makes dot-product GEMVs slow at M = 8 costs KS MFMAs here.
template <int NB, int KS, int MODE>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                        const uint16_t* __restrict__ B, int M, int N,
                                                        int K, void* __restrict__ C, int64_t ldc) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [M][K] bf16
  __shared__ float red[4][16][17];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * NB;
  const int col = lane & 15, kq = lane >> 4;
  const int kw = wave * (K / 4);
  u32x4 bw[KS];
  {
    const bool live = col < NB && n0 + col < N;
    const uint16_t* bp = B + int64_t(min(n0 + col, N - 1)) * K + kw + kq * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) bw[s] = live ? ld16(bp + s * 32) : u32x4{0u, 0u, 0u, 0u};
  }
  const int kchunks = K / 8;
  stage16<256, 16>(reinterpret_cast<u32x4*>(xs), M * kchunks, [&](int c) {
    const int m = c / kchunks;
    return A + m * lda + (c - m * kchunks) * 8;
  });
  __syncthreads();
  f32x4 acc = f32x4{};
  const uint16_t* ap = xs + min(col, M - 1) * K + kw + kq * 8;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const u32x4 a = col < M ? *reinterpret_cast<const u32x4*>(ap + s * 32) : u32x4{0u, 0u, 0u, 0u};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, bw[s]), acc, 0, 0, 0);
  }
  // lane l holds column l % 16, rows (l / 16) * 4 + 0..3
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][kq * 4 + i][col] = acc[i];
  __syncthreads();
  const int m = t >> 4, n = t & 15;
  if (m < M && n < NB && n0 + n < N) {
    const float v = ((red[0][m][n] + red[1][m][n]) + red[2][m][n]) + red[3][m][n];
    store_out<MODE>(C, int64_t(m) * ldc + n0 + n, v);
  }
}

// Skinny GEMM for 2 <= M <= 8 rows of A (batched decode) with the weights
// streamed through LDS: K = 512 * WAVES, wave w owns k in [512 w, 512 w +
// 512), a workgroup owns NB output columns (one workgroup per CU at the
// decode shapes: 20 for N = 5120, 8 for N = 2048).  Each wave copies its NB
// weight rows (1 KB each) into LDS with one non-temporal LDS-DMA per row (64
// lanes x 16 contiguous bytes: whole 128-byte lines, the access the one-row
// GEMV streams at), rows GV_ROWB = 1040 bytes apart so the 16 rows of an MFMA
// B fragment fall on distinct LDS banks.
// The A fragments come straight from global memory (the activation rows are
// L2-resident) and are loaded packed: the 16x16x32 MFMA has 16 A rows and
// only rows 0-7 are live, so lane (c, g) loads 8 k-values of row c % 8 at
// step 2p + c / 8 and a DPP rotation by 8 within each row of 16 lanes hands
// step 2p + 1 to lanes 0-7 (rows 8-15 of the product are never read).  Every
// lane's load is live: half the A load instructions of a zero-padded
// fragment, which is what an 8-row GEMV pays for (the A bytes per workgroup
// equal the weight bytes at 8 columns).  The waves' 8 x NB partials are added
// in k order through LDS.
constexpr int GV_ROWB = 1040;
template <int WAVES, int NB, int MODE>
__global__ __launch_bounds__(64 * WAVES) void gemv_pk_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                             const uint16_t* __restrict__ B, int M, int N,
                                                             int K, void* __restrict__ C, int64_t ldc) {
  constexpr int NT = (NB + 15) / 16;  // 16-column MFMA tiles
  __shared__ __attribute__((aligned(1024))) uint8_t wl[WAVES][NB * GV_ROWB];
  __shared__ float red[WAVES][8][NB + 1];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n0 = blockIdx.x * NB;
  const int kw = wave * 512;
  const int col = lane & 15, kg = lane >> 4;
  u32x4 ap[8];  // ap[p]: row col % 8, k = kw + (2p + col / 8) * 32 + 8 kg .. + 8
  {
    const uint16_t* p = A + min(col & 7, M - 1) * lda + kw + (col >> 3) * 32 + kg * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s) ap[s] = ld16(p + s * 64);
  }
  {
    const pipe::i32x4 rb = pipe::make_rsrc(B, uint32_t(int64_t(N) * K * 2));
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(&wl[wave][0]));
#pragma unroll
    for (int r = 0; r < NB; ++r) {
      const uint32_t off = n0 + r < N ? uint32_t((int64_t(n0 + r) * K + kw) * 2) + lane * 16u : pipe::PAD;
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                   :
                   : "s"(lds0 + uint32_t(r * GV_ROWB)), "v"(off), "s"(rb)
                   : "memory");
    }
  }
  pipe::wait_vm<0>();  // this wave's weight rows are in LDS (and its A fragments in registers)
  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x4{};
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    u32x4 a = ap[s >> 1];
    if (s & 1) {
#pragma unroll
      for (int d = 0; d < 4; ++d) a[d] = __builtin_amdgcn_update_dpp(0u, a[d], 0x128, 0xf, 0xf, false);  // row_ror:8
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const u32x4 b = *reinterpret_cast<const u32x4*>(&wl[wave][0] + min(j * 16 + col, NB - 1) * GV_ROWB +
                                                      kg * 16 + s * 64);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc[j], 0, 0, 0);
    }
  }
  // lane l holds column l % 16 of tile j, rows (l / 16) * 4 + 0..3; rows 8-15 are not used
  if (kg < 2) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
      if (j * 16 + col < NB)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][kg * 4 + i][j * 16 + col] = acc[j][i];
  }
  __syncthreads();
  for (int i = t; i < 8 * NB; i += 64 * WAVES) {
    const int m = i / NB, n = i % NB;
    if (m < M && n0 + n < N) {
      float v = red[0][m][n];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) v += red[w][m][n];
      store_out<MODE>(C, int64_t(m) * ldc + n0 + n, v);
    }
  }
}

// ------------------------------------------------------------------ MFMA tile
// Grid = every (row tile, column tile) pair, renumbered XCD-contiguously and
// then walked in groups of 8 row tiles per column sweep, so the workgroups
// one XCD runs together share A row panels and B column panels in its L2.
template <class P, int OCC, int MODE>
__global__ __launch_bounds__(256, OCC) void gemm_pipe_kernel(const uint16_t* __restrict__ A,
                                                             int64_t lda,
                                                             const uint16_t* __restrict__ B,
                                                             int M, int N, int K,
                                                             void* __restrict__ C, int64_t ldc) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int gx = (N + P::BN - 1) / P::BN, gy = (M + P::BM - 1) / P::BM;
  const int item = pipe::xcd_contiguous(int(blockIdx.x), gx * gy);
  constexpr int GM = 8;
  const int group = item / (GM * gx), first = group * GM, gm = min(gy - first, GM);
  const int r = item - group * GM * gx;
  const int m0 = (first + r % gm) * P::BM, n0 = (r / gm) * P::BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const pipe::i32x4 ra = pipe::make_rsrc(A, uint32_t((int64_t(M) - 1) * lda * 2 + int64_t(K) * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(B, uint32_t(int64_t(N) * K * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int rr = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(rr, lane);
    if (j < P::AI)
      vo[j] = m0 + rr < M ? uint32_t(int64_t(m0 + rr) * lda * 2) + c : pipe::PAD;
    else
      vo[j] = n0 + rr < N ? uint32_t(int64_t(n0 + rr) * K * 2) + c : pipe::PAD;
  }
  typename P::Acc acc;
  P::run(ra, rb, vo, K / P::BK, smem, acc);
#pragma unroll
  for (int i = 0; i < P::FM; ++i)
#pragma unroll
    for (int j = 0; j < P::FN; ++j) {
      const int col = n0 + P::acc_col(wave, j, lane);
      if (col < N) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + P::acc_row(wave, i, e, lane);
          if (row < M) store_out<MODE>(C, int64_t(row) * ldc + col, acc[i][j][e]);
        }
      }
    }
}

template <class P, int OCC, int MODE>
static int launch_pipe(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                       void* C, int64_t ldc, hipStream_t s) {
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_pipe_kernel<P, OCC, MODE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, P::SMEM);
    return true;
  }();
  (void)attr;
  const int64_t tiles = int64_t((M + P::BM - 1) / P::BM) * ((N + P::BN - 1) / P::BN);
  hipLaunchKernelGGL((gemm_pipe_kernel<P, OCC, MODE>), dim3(unsigned(tiles)), dim3(256), P::SMEM, s,
                     A, lda, B, M, N, K, C, ldc);
  return hip_status("qmoe_gemm(tile)");
}

// ------------------------------------------------------------------ large GEMMs
// Problems of at least 224 tiles of 256 x 256 run the grouped expert GEMMs'
// mainloop (mfma_wide.hpp: 8 waves, four 32-column stages, three in flight).
// Its A operand is B (weight rows n, 256 per tile) and its B operand is A
// (rows m), so each lane holds one output row m and, per 32 x 32 block, runs
// of 4 consecutive columns n: the epilogue stores them as one 16-byte fp32
// (8-byte bf16) piece straight from the accumulators (N % 4 == 0, ldc % 4 ==
// 0, C 16-byte aligned).  Tiles are walked as in gemm_pipe_kernel: XCD-
// contiguous, in groups of 8 row tiles per column sweep.
using WideDense = pipe::Wide<4, 2, 32, 4, 256>;

template <int MODE>
__device__ __forceinline__ void store_out4(void* C, int64_t idx, float a, float b, float c, float d) {
  if constexpr (MODE == QMOE_GEMM_STORE_BF16) {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(C) + idx) = make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
  } else if constexpr (MODE == QMOE_GEMM_STORE_F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(C) + idx) = make_float4(a, b, c, d);
  } else {
    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(C) + idx);
    const float4 v = *p;
    *p = make_float4(v.x + a, v.y + b, v.z + c, v.w + d);
  }
}

template <int MODE>
__global__ __launch_bounds__(WideDense::THREADS, 1) void gemm_wide_kernel(const uint16_t* __restrict__ A,
                                                                        int64_t lda,
                                                                        const uint16_t* __restrict__ B, int M,
                                                                        int N, int K, void* __restrict__ C,
                                                                        int64_t ldc) {
  using P = WideDense;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int gx = (N + P::BM - 1) / P::BM, gy = (M + P::BN - 1) / P::BN;
  const int item = pipe::xcd_contiguous(int(blockIdx.x), gx * gy);
  constexpr int GM = 8;
  const int group = item / (GM * gx), first = group * GM, gm = min(gy - first, GM);
  const int r = item - group * GM * gx;
  const int m0 = (first + r % gm) * P::BN, n0 = (r / gm) * P::BM;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const pipe::i32x4 ra = pipe::make_rsrc(B, uint32_t(int64_t(N) * K * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(A, uint32_t((int64_t(M) - 1) * lda * 2 + int64_t(K) * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int rr = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(rr, lane);
    if (j < P::AI)
      vo[j] = n0 + rr < N ? uint32_t(int64_t(n0 + rr) * K * 2) + c : pipe::PAD;
    else
      vo[j] = m0 + rr < M ? uint32_t(int64_t(m0 + rr) * lda * 2) + c : pipe::PAD;
  }
  // this wave's live 32-row blocks of A rows (none when its weight rows lie past N)
  const int nb = n0 + P::wave_arow(wave) < N ? P::wave_blocks(wave, (min(M - m0, P::BN) + 31) / 32) : 0;
  typename P::Acc acc;
  P::run_dyn(nb, ra, rb, vo, K / P::BK, smem, acc, uint32_t(P::BK * 2), uint32_t(P::BK * 2));
#pragma unroll
  for (int j = 0; j < P::FN; ++j) {
    if (j >= nb) break;
    const int row = m0 + P::acc_brow(wave, j, lane);
    if (row >= M) continue;
#pragma unroll
    for (int i = 0; i < P::FM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + P::wave_arow(wave) + i * 32 + q * 8 + (lane >> 5) * 4;
        if (col < N)
          store_out4<MODE>(C, int64_t(row) * ldc + col, acc[i][j][4 * q], acc[i][j][4 * q + 1],
                           acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
      }
  }
}

template <int MODE>
static int launch_wide(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K, void* C,
                       int64_t ldc, hipStream_t s) {
  using P = WideDense;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_wide_kernel<MODE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, P::SMEM);
    return true;
  }();
  (void)attr;
  const int64_t tiles = int64_t((M + P::BN - 1) / P::BN) * ((N + P::BM - 1) / P::BM);
  hipLaunchKernelGGL((gemm_wide_kernel<MODE>), dim3(unsigned(tiles)), dim3(P::THREADS), P::SMEM, s, A, lda, B,
                     M, N, K, C, ldc);
  return hip_status("qmoe_gemm(wide)");
}

// Tile shape by how many tiles the problem has: 256x256 (one workgroup per
// CU, least L2 traffic per flop) once it fills the GPU, else smaller tiles
// with two workgroups per CU; problems that would still leave most CUs idle
// (the prefill router: 4096 x 128 x 2048) take 64x64 tiles with four stages
// in flight, since each of their few workgroups walks a long K.
// Large fp32-output GEMMs (the 8-wave pipeline's sizes, K >= 2048: the
// batch-8 prompt's o_proj, 8192 x 2048 x 4096) go to hipBLASLt, a plain
// library GEMM: C (fp32, ldc) = A . B^T (+ C with ADD_F32).  It keeps the
// long-K tiles' MFMA rate and overlaps the fp32 C read-modify-write that the
// one-tile-per-CU pipeline leaves to the end (8192 x 2048 x 4096: 103 us
// against 145-155 us).  One handle per device, one plan per shape (the
// heuristic's first algorithm, no workspace); a shape the library has no
// algorithm for stays on the pipeline.
namespace {
struct BltPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};
std::mutex blt_mu;
std::map<int, hipblasLtHandle_t> blt_handles;
std::map<std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t>, BltPlan> blt_plans;

const BltPlan* blt_plan(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldc, hipblasLtHandle_t* h) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> g(blt_mu);
  auto hi = blt_handles.find(dev);
  if (hi == blt_handles.end()) {
    hipblasLtHandle_t nh = nullptr;
    if (hipblasLtCreate(&nh) != HIPBLAS_STATUS_SUCCESS) nh = nullptr;
    hi = blt_handles.emplace(dev, nh).first;
  }
  if (!hi->second) return nullptr;
  *h = hi->second;
  auto key = std::make_tuple(dev, M, N, K, lda, ldc);
  auto pi = blt_plans.find(key);
  if (pi != blt_plans.end()) return pi->second.ok ? &pi->second : nullptr;
  BltPlan p;
  // column-major view: C^T (N x M, ld ldc) = B (N x K row-major = K x N, op T) . A^T (K x M, ld lda)
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, uint64_t(K), uint64_t(N), K) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, uint64_t(K), uint64_t(M), lda) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, uint64_t(N), uint64_t(M), ldc) == HIPBLAS_STATUS_SUCCESS;
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    uint64_t wsb = 0;
    hipblasLtMatmulHeuristicResult_t res{};
    int n = 0;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                               sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulAlgoGetHeuristic(*h, p.op, p.la, p.lb, p.lc, p.lc, pref, 1, &res, &n) ==
             HIPBLAS_STATUS_SUCCESS &&
         n > 0 && res.workspaceSize == 0;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (ok) p.algo = res.algo;
  }
  p.ok = ok;
  auto& slot = blt_plans[key] = p;
  return ok ? &slot : nullptr;
}
}  // namespace

// true when the call went to hipBLASLt (rc holds its status)
static bool blt_gemm(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N, int64_t K, float* C,
                     int64_t ldc, bool add, hipStream_t s, int* rc) {
  hipblasLtHandle_t h = nullptr;
  const BltPlan* p = blt_plan(M, N, K, lda, ldc, &h);
  if (!p) return false;
  const float alpha = 1.0f, beta = add ? 1.0f : 0.0f;
  const hipblasStatus_t st = hipblasLtMatmul(h, p->op, &alpha, B, p->la, A, p->lb, &beta, C, p->lc, C, p->lc,
                                             &p->algo, nullptr, 0, s);
  *rc = st == HIPBLAS_STATUS_SUCCESS ? hip_status("qmoe_gemm(hipblaslt)")
                                     : fail(QMOE_ERR_HIP, "qmoe_gemm: hipblasLtMatmul failed (%d)", int(st));
  return true;
}

template <int MODE>
static int launch_tile(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                       void* C, int64_t ldc, hipStream_t s) {
  using Big = pipe::Pipe<256, 256, 64, 2>;
  using Mid = pipe::Pipe<128, 256, 32, 3>;
  using Small = pipe::Pipe<128, 128, 64, 2>;
  using Tiny = pipe::Pipe<64, 64, 64, 4>;
  auto count = [&](int bm, int bn) { return int64_t((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (MODE != QMOE_GEMM_STORE_BF16 && count(256, 256) >= 224 && K >= 2048) {
    int rc = QMOE_OK;
    if (blt_gemm(A, lda, B, M, N, K, static_cast<float*>(C), ldc, MODE == QMOE_GEMM_ADD_F32, s, &rc)) return rc;
  }
  if (count(256, 256) >= 224 && N % 4 == 0 && ldc % 4 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0)
    return launch_wide<MODE>(A, lda, B, M, N, K, C, ldc, s);
  if (count(256, 256) >= 224) return launch_pipe<Big, 1, MODE>(A, lda, B, M, N, K, C, ldc, s);
  if (count(128, 256) >= 224) return launch_pipe<Mid, 2, MODE>(A, lda, B, M, N, K, C, ldc, s);
  if (count(128, 128) >= 96) return launch_pipe<Small, 2, MODE>(A, lda, B, M, N, K, C, ldc, s);
  return launch_pipe<Tiny, 2, MODE>(A, lda, B, M, N, K, C, ldc, s);
}

// ------------------------------------------------------------------ split-K
// For problems with too few output tiles to occupy the GPU (prefill-size
// o_proj: 640 x 2048 with K = 4096 is 80 tiles of 128 x 128; the router
// logits: 640 x 128 with K = 2048 is 20 tiles of 64 x 64), K is split into
// `splits` slices: workgroup (tile, slice) writes its fp32 partial tile to a
// caller-owned workspace part[slice][M][N], and splitk_reduce_kernel adds the
// slices in slice order (fixed order: repeat calls are bit-identical) and
// applies the epilogue mode.
template <class P, int OCC>
__global__ __launch_bounds__(256, OCC) void gemm_splitk_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                               const uint16_t* __restrict__ B, int M, int N,
                                                               int K, int splits, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int tiles_n = (N + P::BN - 1) / P::BN;
  const int slice = int(blockIdx.x) % splits, tile = int(blockIdx.x) / splits;
  const int m0 = (tile / tiles_n) * P::BM, n0 = (tile % tiles_n) * P::BN;
  const int ks = K / splits;
  const uint32_t k0b = uint32_t(slice) * uint32_t(ks) * 2u;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const pipe::i32x4 ra = pipe::make_rsrc(A, uint32_t((int64_t(M) - 1) * lda * 2 + int64_t(K) * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(B, uint32_t(int64_t(N) * K * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int rr = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(rr, lane);
    if (j < P::AI)
      vo[j] = m0 + rr < M ? uint32_t(int64_t(m0 + rr) * lda * 2) + k0b + c : pipe::PAD;
    else
      vo[j] = n0 + rr < N ? uint32_t(int64_t(n0 + rr) * K * 2) + k0b + c : pipe::PAD;
  }
  typename P::Acc acc;
  P::run(ra, rb, vo, ks / P::BK, smem, acc);
  float* dst = part + int64_t(slice) * M * N;
#pragma unroll
  for (int i = 0; i < P::FM; ++i)
#pragma unroll
    for (int j = 0; j < P::FN; ++j) {
      const int col = n0 + P::acc_col(wave, j, lane);
      if (col < N) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + P::acc_row(wave, i, e, lane);
          if (row < M) dst[int64_t(row) * N + col] = acc[i][j][e];
        }
      }
    }
}

// C (mode) = sum over slices in order; 4 consecutive columns per thread.
template <int MODE>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits, int M,
                                                           int N, void* C, int64_t ldc) {
  const int64_t q = int64_t(blockIdx.x) * 256 + threadIdx.x;  // float4 index
  const int64_t per_row = N / 4;
  if (q >= int64_t(M) * per_row) return;
  const int64_t row = q / per_row, col = (q - row * per_row) * 4;
  const int64_t slab = int64_t(M) * N;
  float4 v = *reinterpret_cast<const float4*>(part + row * N + col);
  for (int s = 1; s < splits; ++s) {
    const float4 w = *reinterpret_cast<const float4*>(part + s * slab + row * N + col);
    v.x += w.x;
    v.y += w.y;
    v.z += w.z;
    v.w += w.w;
  }
  store_out<MODE>(C, row * ldc + col, v.x);
  store_out<MODE>(C, row * ldc + col + 1, v.y);
  store_out<MODE>(C, row * ldc + col + 2, v.z);
  store_out<MODE>(C, row * ldc + col + 3, v.w);
}

// The ADD_F32 reduction of whole rows (one workgroup per row, the chunks of
// norm_impl.hpp) followed by the row's RMSNorm: C[row] += sum of the slices
// (splitk_reduce_kernel's order), x_out[row] = bf16(rms_w * C[row] * r).
__global__ __launch_bounds__(NORM_THREADS) void splitk_reduce_norm_kernel(
    const float* __restrict__ part, int splits, int M, int N, float* C, const uint16_t* __restrict__ rms_w,
    float eps, uint16_t* __restrict__ x_out) {
  const int64_t row = blockIdx.x;
  const int64_t slab = int64_t(M) * N;
  float4 v[NORM_MAX_CHUNKS];
  float ss = 0.0f;
  const int nchunk = N / 4;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = int(threadIdx.x) + j * NORM_THREADS;
    if (c < nchunk) {
      const int64_t o = row * N + 4 * c;
      float4 a = *reinterpret_cast<const float4*>(part + o);
      for (int s = 1; s < splits; ++s) {
        const float4 w = *reinterpret_cast<const float4*>(part + s * slab + o);
        a.x += w.x;
        a.y += w.y;
        a.z += w.z;
        a.w += w.w;
      }
      float4 h = *reinterpret_cast<const float4*>(C + o);
      h.x += a.x;
      h.y += a.y;
      h.z += a.z;
      h.w += a.w;
      *reinterpret_cast<float4*>(C + o) = h;
      v[j] = h;
      ss += norm_sq4(h);
    }
  }
  __shared__ float red[NORM_THREADS / 64];
  const float r = norm_rsqrt(ss, N, eps, red);
  uint16_t* xr = x_out + row * N;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = int(threadIdx.x) + j * NORM_THREADS;
    if (c < nchunk) reinterpret_cast<uint2*>(xr)[c] = norm_out4(v[j], r, rms_w, c);
  }
}

using SplitSmall = pipe::Pipe<128, 128, 64, 2>;
using SplitMid = pipe::Pipe<64, 128, 64, 3>;
using SplitTiny = pipe::Pipe<64, 64, 64, 4>;

// Tile shape of a split-K plan.
enum SplitTile { SPLIT_TINY = 0, SPLIT_SMALL = 1, SPLIT_MID = 2 };

// Split-K plan for an M > 16 problem: 0 slices = do not split (the problem
// already has at least 256 tiles, or K is too short to split).  Tiles: 128 x
// 128 when there are at least 16 of them, but 64 x 128 when there are 40-127
// (twice the tiles at half the slices: the o_proj of a 640-token prompt,
// 640 x 2048 x 4096, runs 29.8 us as 80 tiles x 4 slices and 26.8 us as 160
// x 2; 384 x 2048 x 4096: 21.7 -> 20.5 us), else 64 x 64.  Slices double
// while the grid stays within 512 workgroups and each slice keeps >= 512
// (128-column tiles) or >= 256 (64 x 64) columns of K, a multiple of the
// 64-column stage.
static int splitk_plan(int64_t M, int64_t N, int64_t K, SplitTile* tile) {
  if (M <= 16 || N % 4 != 0 || K % 64 != 0) return 0;
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  *tile = t128 >= 40 && t128 < 128 ? SPLIT_MID : t128 >= 16 ? SPLIT_SMALL : SPLIT_TINY;
  const int64_t tiles = *tile == SPLIT_SMALL ? t128
                        : *tile == SPLIT_MID ? ((M + 63) / 64) * ((N + 127) / 128)
                                             : ((M + 63) / 64) * ((N + 63) / 64);
  const int64_t kmin = *tile == SPLIT_TINY ? 256 : 512;
  if (t128 >= 256) return 0;
  int splits = 1;
  while (tiles * splits * 2 <= 512 && K % (int64_t(splits) * 2 * 64) == 0 && K / (splits * 2) >= kmin) splits *= 2;
  return splits > 1 ? splits : 0;
}

template <class P, int MODE>
static int launch_splitk(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K, int splits,
                         float* part, void* C, int64_t ldc, hipStream_t s, const uint16_t* rms_w = nullptr,
                         float eps = 0.0f, uint16_t* x_out = nullptr) {
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_splitk_kernel<P, 2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, P::SMEM);
    return true;
  }();
  (void)attr;
  const int64_t tiles = int64_t((M + P::BM - 1) / P::BM) * ((N + P::BN - 1) / P::BN);
  hipLaunchKernelGGL((gemm_splitk_kernel<P, 2>), dim3(unsigned(tiles * splits)), dim3(256), P::SMEM, s, A, lda,
                     B, M, N, K, splits, part);
  if (int rc = hip_status("qmoe_gemm_ws(slices)")) return rc;
  if (x_out) {  // ADD_F32 into rows of N floats, then their RMSNorm
    hipLaunchKernelGGL(splitk_reduce_norm_kernel, dim3(unsigned(M)), dim3(NORM_THREADS), 0, s, part, splits, M, N,
                       static_cast<float*>(C), rms_w, eps, x_out);
    return hip_status("qmoe_gemm_ws(reduce + norm)");
  }
  const int64_t n4 = int64_t(M) * (N / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel<MODE>, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0, s, part, splits,
                     M, N, C, ldc);
  return hip_status("qmoe_gemm_ws(reduce)");
}

int64_t gemm_splitk_bytes(int64_t M, int64_t N, int64_t K) {
  SplitTile tile = SPLIT_TINY;
  const int splits = (M >= 0 && N >= 0 && K >= 0) ? splitk_plan(M, N, K, &tile) : 0;
  return splits ? int64_t(splits) * M * N * int64_t(sizeof(float)) : 0;
}

int gemm_splitk_slices(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N, int64_t K,
                       float* part, int64_t part_bytes, int* splits, hipStream_t s) {
  SplitTile tile = SPLIT_TINY;
  const int n = splitk_plan(M, N, K, &tile);
  *splits = 0;
  if (n == 0 || part == nullptr || part_bytes < int64_t(n) * M * N * int64_t(sizeof(float)) ||
      M >= (1ll << 31) || N >= (1ll << 31) || lda < K || lda % 8 != 0 ||
      (M - 1) * lda * 2 + K * 2 >= (1ll << 31) || N * K * 2 >= (1ll << 31))
    return QMOE_OK;
  QMOE_REQUIRE(A && B, "gemm_splitk_slices: null pointer");
  auto go = [&](auto tile) {
    using P = decltype(tile);
    static const bool attr = [] {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_splitk_kernel<P, 2>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, P::SMEM);
      return true;
    }();
    (void)attr;
    const int64_t tiles = ((M + P::BM - 1) / P::BM) * ((N + P::BN - 1) / P::BN);
    hipLaunchKernelGGL((gemm_splitk_kernel<P, 2>), dim3(unsigned(tiles * n)), dim3(256), P::SMEM, s, A, lda, B,
                       int(M), int(N), int(K), n, part);
  };
  if (tile == SPLIT_SMALL)
    go(SplitSmall{});
  else if (tile == SPLIT_MID)
    go(SplitMid{});
  else
    go(SplitTiny{});
  *splits = n;
  return hip_status("gemm_splitk_slices");
}

// ------------------------------------------------------------------ launcher
template <int MT, int MODE>
static int launch_gemv_reg(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                           void* C, int64_t ldc, hipStream_t s) {
  // One weight row per wave for a single activation row (the most waves, each
  // with its whole row in flight); more rows per wave amortise the staging
  // of several activation rows.
  constexpr int R = MT == 1 ? 1 : 4;
  const size_t shm = size_t(M) * K * 2;
  static const bool attr = [] {
    for (const void* f : {reinterpret_cast<const void*>(gemv_reg_kernel<MT, R, 1, MODE>),
                          reinterpret_cast<const void*>(gemv_reg_kernel<MT, R, 2, MODE>),
                          reinterpret_cast<const void*>(gemv_reg_kernel<MT, R, 4, MODE>),
                          reinterpret_cast<const void*>(gemv_reg_kernel<MT, (R > 2 ? 2 : R), 8, MODE>)})
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
    return true;
  }();
  (void)attr;
  switch (K / 512) {
#define QMOE_GR(RR, KC)                                                                            \
  case KC:                                                                                         \
    hipLaunchKernelGGL((gemv_reg_kernel<MT, RR, KC, MODE>), dim3(unsigned((N + 4 * RR - 1) / (4 * RR))), \
                       dim3(256), shm, s, A, lda, B, M, N, K, C, ldc);                             \
    return hip_status("qmoe_gemm(gemv)");
    QMOE_GR(R, 1)
    QMOE_GR(R, 2)
    QMOE_GR(R, 4)
    QMOE_GR((R > 2 ? 2 : R), 8)
#undef QMOE_GR
    default:
      return fail(QMOE_ERR_INVALID, "qmoe_gemm: gemv register path needs K in {512, 1024, 2048, 4096}");
  }
}

template <int MODE>
static int launch_gemv_mfma(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                            void* C, int64_t ldc, hipStream_t s) {
  const size_t shm = size_t(M) * K * 2;
  // 8 columns per workgroup unless that makes very many workgroups: at 8 rows
  // the QKV (N = 5120, K = 2048) and o_proj (N = 2048, K = 4096) shapes run
  // 8.7 -> 8.4 and 8.8 -> 7.9 us against 16 columns
  const bool narrow = (N + 15) / 16 < 1024;
  static const bool attr = [] {
    for (const void* f : {reinterpret_cast<const void*>(gemv_mfma_kernel<8, 4, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<16, 4, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<8, 8, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<16, 8, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<8, 16, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<16, 16, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<8, 32, MODE>),
                          reinterpret_cast<const void*>(gemv_mfma_kernel<16, 32, MODE>)})
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
    return true;
  }();
  (void)attr;
  switch (K / 128) {
#define QMOE_GM(KS)                                                                                \
  case KS:                                                                                         \
    if (narrow)                                                                                    \
      hipLaunchKernelGGL((gemv_mfma_kernel<8, KS, MODE>), dim3(unsigned((N + 7) / 8)), dim3(256), shm, \
                         s, A, lda, B, M, N, K, C, ldc);                                           \
    else                                                                                           \
      hipLaunchKernelGGL((gemv_mfma_kernel<16, KS, MODE>), dim3(unsigned((N + 15) / 16)), dim3(256),  \
                         shm, s, A, lda, B, M, N, K, C, ldc);                                      \
    return hip_status("qmoe_gemm(gemv mfma)");
    QMOE_GM(4)
    QMOE_GM(8)
    QMOE_GM(16)
    QMOE_GM(32)
#undef QMOE_GM
    default:
      return fail(QMOE_ERR_INVALID, "qmoe_gemm: skinny MFMA path needs K in {512, 1024, 2048, 4096}");
  }
}

template <int MODE>
static int launch_gemv_pk(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                          void* C, int64_t ldc, hipStream_t s) {
  // the most columns per workgroup that still leaves one workgroup per CU
  // (fewer workgroups load the A rows fewer times: at 8 rows the QKV shape N
  // = 5120, K = 2048 runs 7.3 / 6.5 / 6.0 us at 8 / 10 / 20 columns, and
  // o_proj N = 2048, K = 4096 5.7 us at 8 columns against 7.2 at 4)
  const int cus = current_device_cus();
  const int nb = N >= 20 * cus && K <= 2048 ? 20 : N >= 16 * cus ? 16 : N >= 8 * cus ? 8 : 4;
#define QMOE_PK(W, NB_)                                                                            \
  if (K == 512 * W && nb == NB_) {                                                                 \
    hipLaunchKernelGGL((gemv_pk_kernel<W, NB_, MODE>), dim3(unsigned((N + NB_ - 1) / NB_)), dim3(64 * W), 0, \
                       s, A, lda, B, M, N, K, C, ldc);                                             \
    return hip_status("qmoe_gemm(gemv pk)");                                                       \
  }
#define QMOE_PK_W(W) QMOE_PK(W, 4) QMOE_PK(W, 8) QMOE_PK(W, 16)
  QMOE_PK_W(1)
  QMOE_PK_W(2)
  QMOE_PK_W(4)
  QMOE_PK_W(8)
  QMOE_PK(1, 20)
  QMOE_PK(2, 20)
  QMOE_PK(4, 20)
#undef QMOE_PK_W
#undef QMOE_PK
  return fail(QMOE_ERR_INVALID, "qmoe_gemm: packed GEMV needs K in {512, 1024, 2048, 4096}");
}

template <int MODE>
static int launch_gemv(const uint16_t* A, int64_t lda, const uint16_t* B, int M, int N, int K,
                       void* C, int64_t ldc, hipStream_t s) {
  const size_t shm = size_t(M) * K * 2;
  const int kc = K / 512;
  if (M >= 2 && M <= 8 && (kc == 1 || kc == 2 || kc == 4 || kc == 8) && int64_t(N) * K * 2 < (1ll << 31))
    return launch_gemv_pk<MODE>(A, lda, B, M, N, K, C, ldc, s);
  if (M >= 2 && (kc == 1 || kc == 2 || kc == 4 || kc == 8))
    return launch_gemv_mfma<MODE>(A, lda, B, M, N, K, C, ldc, s);
  if (kc == 1 || kc == 2 || kc == 4 || kc == 8) {
    if (M <= 1) return launch_gemv_reg<1, MODE>(A, lda, B, M, N, K, C, ldc, s);
    if (M <= 4) return launch_gemv_reg<4, MODE>(A, lda, B, M, N, K, C, ldc, s);
    if (M <= 8) return launch_gemv_reg<8, MODE>(A, lda, B, M, N, K, C, ldc, s);
    return launch_gemv_reg<16, MODE>(A, lda, B, M, N, K, C, ldc, s);
  }
  // 16 rows per workgroup (4 per wave) for wide outputs, and whenever the
  // staged activations are large (fewer workgroups re-staging them)
  const bool wide = N >= 4096 || shm > 16384;
  const int rows_per_block = wide ? 16 : 4;
  dim3 grid((N + rows_per_block - 1) / rows_per_block);
#define QMOE_GEMV(MT)                                                                        \
  if (M <= MT) {                                                                             \
    if (wide)                                                                                \
      hipLaunchKernelGGL((gemv_kernel<MT, 4, MODE>), grid, dim3(256), shm, s, A, lda, B, M, N, \
                         K, C, ldc);                                                         \
    else                                                                                     \
      hipLaunchKernelGGL((gemv_kernel<MT, 1, MODE>), grid, dim3(256), shm, s, A, lda, B, M, N, \
                         K, C, ldc);                                                         \
    return hip_status("qmoe_gemm(gemv)");                                                    \
  }
  QMOE_GEMV(1)
  QMOE_GEMV(2)
  QMOE_GEMV(4)
  QMOE_GEMV(8)
  QMOE_GEMV(16)
#undef QMOE_GEMV
  return fail(QMOE_ERR_INVALID, "qmoe_gemm: gemv path needs M <= 16");
}

int gemm_launch(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N,
                int64_t K, int mode, void* C, int64_t ldc, hipStream_t s) {
  QMOE_REQUIRE(B && (M == 0 || (A && C)), "qmoe_gemm: null pointer");
  QMOE_REQUIRE(M >= 0 && N > 0 && K > 0, "qmoe_gemm: empty shape M=%lld N=%lld K=%lld",
               (long long)M, (long long)N, (long long)K);
  QMOE_REQUIRE(mode >= 0 && mode <= 2, "qmoe_gemm: bad mode %d", mode);
  QMOE_REQUIRE(lda >= K && ldc >= N, "qmoe_gemm: lda/ldc smaller than the row length");
  QMOE_REQUIRE(lda % 8 == 0, "qmoe_gemm: lda must be a multiple of 8");
  QMOE_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), "qmoe_gemm: dims overflow");
  if (M == 0) return QMOE_OK;
  if (M <= 16 && M * K <= 32768) {
    QMOE_REQUIRE(K % 512 == 0, "qmoe_gemm: gemv path needs K %% 512 == 0 (K=%lld)", (long long)K);
    switch (mode) {
      case QMOE_GEMM_STORE_BF16:
        return launch_gemv<QMOE_GEMM_STORE_BF16>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
      case QMOE_GEMM_STORE_F32:
        return launch_gemv<QMOE_GEMM_STORE_F32>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
      default:
        return launch_gemv<QMOE_GEMM_ADD_F32>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
    }
  }
  QMOE_REQUIRE(K % 64 == 0, "qmoe_gemm: K %% 64 != 0 (K=%lld)", (long long)K);
  // DMA offsets are 32-bit with the zero-row marker at 2^31
  QMOE_REQUIRE((M - 1) * lda * 2 + K * 2 < (1ll << 31) && N * K * 2 < (1ll << 31),
               "qmoe_gemm: A or B larger than 2 GiB");
  switch (mode) {
    case QMOE_GEMM_STORE_BF16:
      return launch_tile<QMOE_GEMM_STORE_BF16>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
    case QMOE_GEMM_STORE_F32:
      return launch_tile<QMOE_GEMM_STORE_F32>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
    default:
      return launch_tile<QMOE_GEMM_ADD_F32>(A, lda, B, int(M), int(N), int(K), C, ldc, s);
  }
}

}  // namespace qmoe

namespace qmoe {
template <int MODE>
static int launch_gemv_rms(const float* h, const uint16_t* rms_w, float eps, const uint16_t* B, int N, int K,
                           void* C, hipStream_t s) {
  const dim3 grid(unsigned((N + 3) / 4));
  switch (K / 512) {
#define QMOE_GRMS(KC)                                                                                \
  case KC:                                                                                           \
    hipLaunchKernelGGL((gemv_rms_kernel<KC, MODE>), grid, dim3(256), 0, s, h, rms_w, eps, B, N, C); \
    return hip_status("qmoe_gemv_rmsnorm");
    QMOE_GRMS(1)
    QMOE_GRMS(2)
    QMOE_GRMS(4)
    QMOE_GRMS(8)
#undef QMOE_GRMS
    default:
      return fail(QMOE_ERR_INVALID, "qmoe_gemv_rmsnorm: K must be 512, 1024, 2048 or 4096");
  }
}

int gemv_rmsnorm_launch(const float* h, const uint16_t* rms_w, float eps, const uint16_t* B, int64_t N,
                        int64_t K, int mode, void* C, hipStream_t s) {
  QMOE_REQUIRE(h && rms_w && B && C, "qmoe_gemv_rmsnorm: null pointer");
  QMOE_REQUIRE(N > 0 && N < (1ll << 31), "qmoe_gemv_rmsnorm: bad N");
  QMOE_REQUIRE(K == 512 || K == 1024 || K == 2048 || K == 4096, "qmoe_gemv_rmsnorm: K must be 512, 1024, 2048 or 4096");
  QMOE_REQUIRE(mode >= 0 && mode <= 2, "qmoe_gemv_rmsnorm: bad mode %d", mode);
  QMOE_REQUIRE(eps >= 0.0f, "qmoe_gemv_rmsnorm: eps < 0");
  switch (mode) {
    case QMOE_GEMM_STORE_BF16:
      return launch_gemv_rms<QMOE_GEMM_STORE_BF16>(h, rms_w, eps, B, int(N), int(K), C, s);
    case QMOE_GEMM_STORE_F32:
      return launch_gemv_rms<QMOE_GEMM_STORE_F32>(h, rms_w, eps, B, int(N), int(K), C, s);
    default:
      return launch_gemv_rms<QMOE_GEMM_ADD_F32>(h, rms_w, eps, B, int(N), int(K), C, s);
  }
}
}  // namespace qmoe

extern "C" int qmoe_gemv_rmsnorm(const float* h, const qmoe_bf16* rms_w, float eps, const qmoe_bf16* B,
                                 int64_t N, int64_t K, int mode, void* C, qmoe_stream_t stream) {
  return qmoe::gemv_rmsnorm_launch(h, rms_w, eps, B, N, K, mode, C, qmoe::as_stream(stream));
}

extern "C" int qmoe_gemm(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
                         int64_t K, int mode, void* C, int64_t ldc, qmoe_stream_t stream) {
  return qmoe::gemm_launch(A, lda, B, M, N, K, mode, C, ldc, qmoe::as_stream(stream));
}

extern "C" int64_t qmoe_gemm_ws_workspace(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return -1;
  qmoe::SplitTile tile = qmoe::SPLIT_TINY;
  const int splits = qmoe::splitk_plan(M, N, K, &tile);
  return splits ? int64_t(splits) * M * N * int64_t(sizeof(float)) : 0;
}

extern "C" int qmoe_gemm_ws(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
                            int64_t K, int mode, void* C, int64_t ldc, void* workspace, int64_t workspace_bytes,
                            qmoe_stream_t stream) {
  using namespace qmoe;
  SplitTile tile = SPLIT_TINY;
  const int splits = splitk_plan(M, N, K, &tile);
  const int64_t need = splits ? int64_t(splits) * M * N * int64_t(sizeof(float)) : 0;
  if (splits == 0 || workspace == nullptr || workspace_bytes < need || M >= (1ll << 31) || N >= (1ll << 31))
    return gemm_launch(A, lda, B, M, N, K, mode, C, ldc, as_stream(stream));
  QMOE_REQUIRE(A && B && C, "qmoe_gemm_ws: null pointer");
  QMOE_REQUIRE(mode >= 0 && mode <= 2, "qmoe_gemm_ws: bad mode %d", mode);
  QMOE_REQUIRE(lda >= K && ldc >= N && lda % 8 == 0, "qmoe_gemm_ws: bad lda/ldc");
  QMOE_REQUIRE((M - 1) * lda * 2 + K * 2 < (1ll << 31) && N * K * 2 < (1ll << 31),
               "qmoe_gemm_ws: A or B larger than 2 GiB");
  hipStream_t s = as_stream(stream);
  float* part = static_cast<float*>(workspace);
#define QMOE_SPLIT(MODE)                                                                                    \
  return tile == SPLIT_SMALL ? launch_splitk<SplitSmall, MODE>(A, lda, B, int(M), int(N), int(K), splits, part, C, \
                                                               ldc, s)                                            \
         : tile == SPLIT_MID ? launch_splitk<SplitMid, MODE>(A, lda, B, int(M), int(N), int(K), splits, part, C,   \
                                                             ldc, s)                                              \
                             : launch_splitk<SplitTiny, MODE>(A, lda, B, int(M), int(N), int(K), splits, part, C,  \
                                                              ldc, s);
  switch (mode) {
    case QMOE_GEMM_STORE_BF16:
      QMOE_SPLIT(QMOE_GEMM_STORE_BF16)
    case QMOE_GEMM_STORE_F32:
      QMOE_SPLIT(QMOE_GEMM_STORE_F32)
    default:
      QMOE_SPLIT(QMOE_GEMM_ADD_F32)
  }
#undef QMOE_SPLIT
}

extern "C" int qmoe_gemm_ws_add_rmsnorm(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
                                       int64_t K, float* C, const qmoe_bf16* rms_w, float eps, qmoe_bf16* x_out,
                                       void* workspace, int64_t workspace_bytes, qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(B && rms_w && (M == 0 || (A && C && x_out)), "qmoe_gemm_ws_add_rmsnorm: null pointer");
  QMOE_REQUIRE(M >= 0 && M < (1ll << 31) && N > 0 && K > 0, "qmoe_gemm_ws_add_rmsnorm: bad shape");
  QMOE_REQUIRE(N % 4 == 0 && N <= NORM_THREADS * 4 * NORM_MAX_CHUNKS,
               "qmoe_gemm_ws_add_rmsnorm: N must be a multiple of 4 and <= 8192 (N=%lld)", (long long)N);
  QMOE_REQUIRE(eps >= 0.0f, "qmoe_gemm_ws_add_rmsnorm: eps < 0");
  QMOE_REQUIRE(lda >= K && lda % 8 == 0, "qmoe_gemm_ws_add_rmsnorm: bad lda");
  if (M == 0) return QMOE_OK;
  SplitTile tile = SPLIT_TINY;
  const int splits = splitk_plan(M, N, K, &tile);
  const int64_t need = splits ? int64_t(splits) * M * N * int64_t(sizeof(float)) : 0;
  hipStream_t s = as_stream(stream);
  if (splits == 0 || workspace == nullptr || workspace_bytes < need) {
    // no split: the GEMM's own epilogue adds into C, then the norm reads it back
    if (int rc = gemm_launch(A, lda, B, M, N, K, QMOE_GEMM_ADD_F32, C, N, s)) return rc;
    return qmoe_rmsnorm_residual(C, nullptr, rms_w, M, N, eps, nullptr, x_out, stream);
  }
  QMOE_REQUIRE((M - 1) * lda * 2 + K * 2 < (1ll << 31) && N * K * 2 < (1ll << 31),
               "qmoe_gemm_ws_add_rmsnorm: A or B larger than 2 GiB");
  float* part = static_cast<float*>(workspace);
  const uint16_t* w = reinterpret_cast<const uint16_t*>(rms_w);
  uint16_t* xo = reinterpret_cast<uint16_t*>(x_out);
  return tile == SPLIT_SMALL ? launch_splitk<SplitSmall, QMOE_GEMM_ADD_F32>(A, lda, B, int(M), int(N), int(K), splits,
                                                                           part, C, N, s, w, eps, xo)
         : tile == SPLIT_MID ? launch_splitk<SplitMid, QMOE_GEMM_ADD_F32>(A, lda, B, int(M), int(N), int(K), splits,
                                                                         part, C, N, s, w, eps, xo)
                             : launch_splitk<SplitTiny, QMOE_GEMM_ADD_F32>(A, lda, B, int(M), int(N), int(K),
                                                                          splits, part, C, N, s, w, eps, xo);
}
