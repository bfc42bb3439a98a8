// GQA attention pieces for head_dim 128:
//
//  qkv_norm_rope  -- QKV projection on the MFMA tile engine with a 128-column
//                    tile = exactly one head, so the per-head RMSNorm and the
//                    RoPE pairs (i, i+64) are tile-local.  The fp32 tile goes
//                    through LDS; two threads per token row finish the head.
//                    K and V rows go straight into the contiguous cache.
//  attn_prefill   -- causal flash attention on MFMA.  Scores are computed
//                    transposed, S^T = K . Q^T, so each lane owns one query
//                    column: row max / row sum are lane-local plus one
//                    exchange with lane^32, and the probabilities already sit
//                    in the B-operand layout of O^T = V^T . P^T.  K and V
//                    tiles reach LDS by DMA, row-major; the V^T fragments
//                    come from transposing LDS reads (ds_read_b64_tr_b16) in
//                    the key order of the P^T registers.
//  attn_decode    -- split-KV flash decoding on MFMA: a wave owns 64 keys of
//                    one (batch, kv head) and all q heads of that GQA group
//                    (S^T = K.Q^T, softmax per column, O^T = V^T.P^T), so each
//                    K/V row is read from HBM once, with every load of the
//                    wave in flight together; a second kernel merges the
//                    per-wave partials that hold keys.
#include "decode_util.hpp"
#include "gemm.hpp"
#include "mfma_pipe.hpp"
#include "mfma_tile.hpp"
#include "mfma_wide.hpp"

#include <type_traits>

namespace qmoe {

constexpr int HD = 128;  // head_dim

// ====================================================================== QKV
// Per-(token, head) finish shared by the QKV kernels: PARTS threads (part =
// 0 .. PARTS-1, consecutive lanes) each load W = 64 / PARTS of the head's
// fp32 values v (LDS or global, 16-byte aligned: elements [W part, W part + W)
// and their RoPE partners + 64) into registers: q/k heads get the RMSNorm
// over head_dim and RoPE, then q goes to q_out and k / v to the cache row at
// the token's position (rejected positions write nothing).
template <int PARTS>
__device__ __forceinline__ void qkv_finish_head(
    const float* v, int part, int tok, int head, const int32_t* __restrict__ positions, int S,
    int Hq, int Hkv, int S_max, int max_pos, float eps, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ rope_cos,
    const float* __restrict__ rope_sin, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache) {
  constexpr int W = 64 / PARTS;
  static_assert(PARTS == 2 || PARTS == 4, "two or four threads per head");
  float lo[W], hi[W];
#pragma unroll
  for (int i = 0; i < W; i += 4) {
    const float4 a = *reinterpret_cast<const float4*>(v + part * W + i);
    const float4 c = *reinterpret_cast<const float4*>(v + 64 + part * W + i);
    lo[i] = a.x; lo[i + 1] = a.y; lo[i + 2] = a.z; lo[i + 3] = a.w;
    hi[i] = c.x; hi[i + 1] = c.y; hi[i + 2] = c.z; hi[i + 3] = c.w;
  }
  const int pos = positions[tok];
  if (pos < 0 || pos >= S_max || pos >= max_pos) return;  // rejected: nothing written
  const int b = tok / S;
  uint16_t* dst;
  if (head < Hq + Hkv) {
    const uint16_t* nw = head < Hq ? qn_w : kn_w;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < W; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
    ss += __shfl_xor(ss, 1, 64);
    if constexpr (PARTS == 4) ss += __shfl_xor(ss, 2, 64);
    const float r = rsqrtf(ss / float(HD) + eps);
    const float* cs = rope_cos + int64_t(pos) * (HD / 2) + part * W;
    const float* sn = rope_sin + int64_t(pos) * (HD / 2) + part * W;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const float a = bf16_to_f32(nw[part * W + i]) * (lo[i] * r);
      const float bb = bf16_to_f32(nw[64 + part * W + i]) * (hi[i] * r);
      const float c = cs[i], s = sn[i];
      lo[i] = a * c - bb * s;
      hi[i] = bb * c + a * s;
    }
    if (head < Hq)
      dst = q_out + (int64_t(tok) * Hq + head) * HD;
    else
      dst = k_cache + ((int64_t(b) * Hkv + (head - Hq)) * S_max + pos) * HD;
  } else {
    dst = v_cache + ((int64_t(b) * Hkv + (head - Hq - Hkv)) * S_max + pos) * HD;
  }
#pragma unroll
  for (int c = 0; c < W / 8; ++c) {
    u32x4 v0, v1;
    v0.x = pack_bf16x2(lo[c * 8 + 0], lo[c * 8 + 1]);
    v0.y = pack_bf16x2(lo[c * 8 + 2], lo[c * 8 + 3]);
    v0.z = pack_bf16x2(lo[c * 8 + 4], lo[c * 8 + 5]);
    v0.w = pack_bf16x2(lo[c * 8 + 6], lo[c * 8 + 7]);
    v1.x = pack_bf16x2(hi[c * 8 + 0], hi[c * 8 + 1]);
    v1.y = pack_bf16x2(hi[c * 8 + 2], hi[c * 8 + 3]);
    v1.z = pack_bf16x2(hi[c * 8 + 4], hi[c * 8 + 5]);
    v1.w = pack_bf16x2(hi[c * 8 + 6], hi[c * 8 + 7]);
    *reinterpret_cast<u32x4*>(dst + part * W + c * 8) = v0;
    *reinterpret_cast<u32x4*>(dst + 64 + part * W + c * 8) = v1;
  }
}

// Decode-size QKV (T <= QKV_DEC_MAX_T token rows): the projection runs as a
// bandwidth-bound GEMV over every CU (qmoe_gemm's register GEMV: all weight
// rows streamed once) into an fp32 workspace [T][(Hq+2Hkv)*D]; this kernel
// then finishes each (token, head) from there, one wave per (head, token):
// lane l holds element l and its RoPE partner l + 64, so the head's values,
// norm weights and position are all requested at once, the cos/sin row right
// after the position arrives, and the norm is one wave reduction.  Same
// arithmetic per element as qkv_finish_head; the sum of squares runs in the
// wave's reduction order.
constexpr int QKV_DEC_MAX_T = 16;
#ifndef QMOE_QKV_PIPE_MIN_T
#define QMOE_QKV_PIPE_MIN_T 256
#endif
constexpr int QKV_PIPE_MIN_T = QMOE_QKV_PIPE_MIN_T;  // token rows from which the 256-row pipeline is used

// One head row of the decode finish, lane l holding elements l and l + 64
// (its RoPE partner): RMSNorm over the 128 values (one wave reduction), the
// norm weight, then RoPE with this position's (c, sn).  Shared by the finish
// kernel and the fused decode attention so both give the same bits.
__device__ __forceinline__ void finish_head(float& lo, float& hi, float wl, float wh, float c, float sn,
                                            float eps) {
  const float r = rsqrtf(wave_sum(lo * lo + hi * hi) / float(HD) + eps);
  const float a = wl * (lo * r), bb = wh * (hi * r);
  lo = a * c - bb * sn;
  hi = bb * c + a * sn;
}

__global__ __launch_bounds__(64) void qkv_finish_kernel(
    const float* __restrict__ raw, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ rope_cos,
    const float* __restrict__ rope_sin, const int32_t* __restrict__ positions, int T, int S, int Hq,
    int Hkv, int S_max, int max_pos, float eps, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache) {
  const int l = threadIdx.x, head = blockIdx.x, tok = blockIdx.y;
  const float* v = raw + int64_t(tok) * (Hq + 2 * Hkv) * HD + head * HD;
  const bool normed = head < Hq + Hkv;
  const uint16_t* nw = head < Hq ? qn_w : kn_w;
  float lo = v[l], hi = v[l + 64];
  const float wl = normed ? bf16_to_f32(nw[l]) : 0.0f, wh = normed ? bf16_to_f32(nw[l + 64]) : 0.0f;
  const int pos = positions[tok];
  if (pos < 0 || pos >= S_max || pos >= max_pos) return;  // rejected: nothing written
  const int b = tok / S;
  uint16_t* dst;
  if (normed) {
    const float c = rope_cos[int64_t(pos) * (HD / 2) + l], sn = rope_sin[int64_t(pos) * (HD / 2) + l];
    finish_head(lo, hi, wl, wh, c, sn, eps);
    if (head < Hq)
      dst = q_out + (int64_t(tok) * Hq + head) * HD;
    else
      dst = k_cache + ((int64_t(b) * Hkv + (head - Hq)) * S_max + pos) * HD;
  } else {
    dst = v_cache + ((int64_t(b) * Hkv + (head - Hq - Hkv)) * S_max + pos) * HD;
  }
  dst[l] = f32_to_bf16(lo);
  dst[l + 64] = f32_to_bf16(hi);
}

__global__ __launch_bounds__(256) void qkv_norm_rope_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wqkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    const int32_t* __restrict__ positions, int T, int S, int H, int Hq, int Hkv, int S_max,
    int max_pos, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[tile::SMEM_BYTES / 2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int head = blockIdx.x;  // 0..Hq+2Hkv-1
  const int m0 = blockIdx.y * tile::BM;
  const int n0 = head * HD;
  const int kc = (t & 7) * 8;
  const uint16_t* ap[4];
  const uint16_t* bp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = tile::stage_row(t, j);
    ap[j] = (m0 + r < T) ? x + int64_t(m0 + r) * H + kc : nullptr;
    bp[j] = wqkv + int64_t(n0 + r) * H + kc;
  }
  tile::Acc acc;
  tile::mma_128x128(ap, bp, H, smem, acc);  // ends with a barrier

  constexpr int LDC = HD + 4;
  float* ct = reinterpret_cast<float*>(smem);  // [128][LDC] fp32 (66 KB)
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int col = tile::acc_col(wave, lane, ni);
#pragma unroll
      for (int i = 0; i < 16; ++i) ct[tile::acc_row(wave, lane, mi, i) * LDC + col] = acc.c[mi][ni][i];
    }
  __syncthreads();

  const int row = t >> 1, half = t & 1;
  const int tok = m0 + row;
  if (tok >= T) return;
  qkv_finish_head<2>(ct + row * LDC, half, tok, head, positions, S, Hq, Hkv, S_max, max_pos, eps, qn_w,
                  kn_w, rope_cos, rope_sin, q_out, k_cache, v_cache);
}

// Large-T QKV: the same per-head epilogue on the direct-to-LDS MFMA pipeline
// (pipe::Pipe, as qmoe_gemm uses): a workgroup computes BM token rows x one
// head (128 columns), stages the fp32 accumulators in LDS and finishes the
// rows with qkv_finish_head, 128 rows per pass.  Workgroups of one row block
// are consecutive (head fastest), so the x rows they share are read from L2.
template <class P>
struct QkvPipe {
  static constexpr int LDC = HD + 4;
  static constexpr int EPI = P::BM * LDC * 4;
  static constexpr int SMEM = P::SMEM > EPI ? P::SMEM : EPI;
  static_assert(P::BN == HD, "one head per tile");
  static_assert(SMEM <= 160 * 1024, "LDS");
};

template <class P, int OCC>
__global__ __launch_bounds__(256, OCC) void qkv_pipe_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wqkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    const int32_t* __restrict__ positions, int T, int S, int H, int Hq, int Hkv, int S_max,
    int max_pos, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  constexpr int LDC = QkvPipe<P>::LDC;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int head = blockIdx.x, m0 = blockIdx.y * P::BM, n0 = head * HD;
  const pipe::i32x4 ra = pipe::make_rsrc(x, uint32_t(int64_t(T) * H * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(wqkv + int64_t(n0) * H, uint32_t(int64_t(HD) * H * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int rr = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(rr, lane);
    if (j < P::AI)
      vo[j] = m0 + rr < T ? uint32_t(int64_t(m0 + rr) * H * 2) + c : pipe::PAD;
    else
      vo[j] = uint32_t(int64_t(rr) * H * 2) + c;
  }
  typename P::Acc acc;
  P::run(ra, rb, vo, H / P::BK, smem, acc);
  __syncthreads();  // pipeline buffers are reused for the accumulators
  float* ct = reinterpret_cast<float*>(smem);  // [BM][LDC] fp32
#pragma unroll
  for (int i = 0; i < P::FM; ++i)
#pragma unroll
    for (int j = 0; j < P::FN; ++j) {
      const int col = P::acc_col(wave, j, lane);
#pragma unroll
      for (int e = 0; e < 16; ++e) ct[P::acc_row(wave, i, e, lane) * LDC + col] = acc[i][j][e];
    }
  __syncthreads();
  for (int r0 = 0; r0 < P::BM; r0 += 128) {
    const int row = r0 + (t >> 1), tok = m0 + row;
    if (row < P::BM && tok < T)
      qkv_finish_head<2>(ct + row * LDC, t & 1, tok, head, positions, S, Hq, Hkv, S_max, max_pos, eps, qn_w,
                      kn_w, rope_cos, rope_sin, q_out, k_cache, v_cache);
  }
}

// Large-T QKV on the 8-wave wide pipeline (mfma_wide.hpp): a workgroup
// computes 128 token rows x 640 weight rows (5 heads), 8 waves of 32 x 5
// blocks over 64 tokens x 160 columns, three 48 KB stages.  At B = 8 x 1024
// tokens that is 64 x 8 = 512 tiles, two full rounds of 256 CUs (the
// one-head 256-row tiles of qkv_pipe_kernel make 1280 tiles at a lower rate
// each).  The epilogue stages the fp32 accumulators one head at a time in
// LDS ([128 tokens][128 + 4]) and finishes each (token, head) with four
// threads (qkv_finish_head<4>), so the accumulators plus one thread's 32
// finish values fit the register budget.
using QkvWide = pipe::Wide<4, 5, 32, 3, 128>;
constexpr int QW_HEADS = QkvWide::BM / HD;
constexpr int QW_LDC = HD + 4;
constexpr int QW_SMEM = QkvWide::SMEM > QkvWide::BN * QW_LDC * 4 ? QkvWide::SMEM : QkvWide::BN * QW_LDC * 4;
static_assert(QkvWide::BM % HD == 0 && QW_SMEM <= 160 * 1024, "QKV wide tile");
static_assert(QkvWide::THREADS == 4 * QkvWide::BN, "four threads per token row of a head");

__global__ __launch_bounds__(QkvWide::THREADS, 1) void qkv_wide_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wqkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    const int32_t* __restrict__ positions, int T, int S, int H, int Hq, int Hkv, int S_max,
    int max_pos, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
  using P = QkvWide;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int NH = Hq + 2 * Hkv, N = NH * HD;
  // tile order as in gemm_wide_kernel: XCD-contiguous items, groups of 8
  // token blocks walking every panel
  const int gx = (N + P::BM - 1) / P::BM, gy = (T + P::BN - 1) / P::BN;
  const int item = pipe::xcd_contiguous(int(blockIdx.x), gx * gy);
  constexpr int GM = 8;
  const int group = item / (GM * gx), first = group * GM, gm = min(gy - first, GM);
  const int r = item - group * GM * gx;
  const int m0 = (first + r % gm) * P::BN, n0 = (r / gm) * P::BM;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const pipe::i32x4 ra = pipe::make_rsrc(wqkv, uint32_t(int64_t(N) * H * 2));
  const pipe::i32x4 rb = pipe::make_rsrc(x, uint32_t(int64_t(T) * H * 2));
  uint32_t vo[P::NDMA];
#pragma unroll
  for (int j = 0; j < P::NDMA; ++j) {
    const int rr = P::dma_row(j, wave, lane);
    const uint32_t c = P::dma_chunk(rr, lane);
    if (j < P::AI)
      vo[j] = n0 + rr < N ? uint32_t(int64_t(n0 + rr) * H * 2) + c : pipe::PAD;
    else
      vo[j] = m0 + rr < T ? uint32_t(int64_t(m0 + rr) * H * 2) + c : pipe::PAD;
  }
  // this wave's live 32-token blocks (none when its weight rows lie past N)
  const int nb = n0 + P::wave_arow(wave) < N ? P::wave_blocks(wave, (min(T - m0, P::BN) + 31) / 32) : 0;
  typename P::Acc acc;
  P::run_dyn(nb, ra, rb, vo, H / P::BK, smem, acc, uint32_t(P::BK * 2), uint32_t(P::BK * 2));
  float* ct = reinterpret_cast<float*>(smem);
  const int part = threadIdx.x & 3, row = threadIdx.x >> 2;
#pragma unroll
  for (int th = 0; th < QW_HEADS; ++th) {
    const int c0 = th * HD;
    __syncthreads();  // the pipeline's (or the previous head's) LDS reads are done
#pragma unroll
    for (int j = 0; j < P::FN; ++j) {
      if (j >= nb) break;
      const int tr = P::acc_brow(wave, j, lane);
#pragma unroll
      for (int i = 0; i < P::FM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = P::wave_arow(wave) + i * 32 + q * 8 + (lane >> 5) * 4 - c0;
          if (col >= 0 && col < HD)
            *reinterpret_cast<float4*>(ct + tr * QW_LDC + col) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        }
    }
    __syncthreads();
    const int head = n0 / HD + th, tok = m0 + row;
    if (head < NH && tok < T)
      qkv_finish_head<4>(ct + row * QW_LDC, part, tok, head, positions, S, Hq, Hkv, S_max, max_pos, eps, qn_w,
                         kn_w, rope_cos, rope_sin, q_out, k_cache, v_cache);
  }
}

static int qkv_wide_launch(const uint16_t* x, const uint16_t* wqkv, const uint16_t* qn_w, const uint16_t* kn_w,
                           const float* rope_cos, const float* rope_sin, const int32_t* positions, int64_t T,
                           int64_t S, int64_t H, int64_t Hq, int64_t Hkv, int64_t S_max, int max_p, float eps,
                           uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, hipStream_t s) {
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(qkv_wide_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, QW_SMEM);
    return true;
  }();
  (void)attr;
  const int64_t N = (Hq + 2 * Hkv) * HD;
  const int64_t tiles = (T + QkvWide::BN - 1) / QkvWide::BN * ((N + QkvWide::BM - 1) / QkvWide::BM);
  hipLaunchKernelGGL(qkv_wide_kernel, dim3(unsigned(tiles)), dim3(QkvWide::THREADS), QW_SMEM, s, x, wqkv, qn_w, kn_w,
                     rope_cos, rope_sin, positions, int(T), int(S), int(H), int(Hq), int(Hkv), int(S_max), max_p, eps,
                     q_out, k_cache, v_cache);
  return hip_status("qmoe_qkv_norm_rope(wide)");
}

template <class P, int OCC>
static int qkv_pipe_launch(const uint16_t* x, const uint16_t* wqkv, const uint16_t* qn_w, const uint16_t* kn_w,
                           const float* rope_cos, const float* rope_sin, const int32_t* positions, int64_t T,
                           int64_t S, int64_t H, int64_t Hq, int64_t Hkv, int64_t S_max, int max_p, float eps,
                           uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, hipStream_t s) {
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(qkv_pipe_kernel<P, OCC>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, QkvPipe<P>::SMEM);
    return true;
  }();
  (void)attr;
  dim3 grid(unsigned(Hq + 2 * Hkv), unsigned((T + P::BM - 1) / P::BM));
  hipLaunchKernelGGL((qkv_pipe_kernel<P, OCC>), grid, dim3(256), QkvPipe<P>::SMEM, s, x, wqkv, qn_w, kn_w, rope_cos,
                     rope_sin, positions, int(T), int(S), int(H), int(Hq), int(Hkv), int(S_max), max_p, eps,
                     q_out, k_cache, v_cache);
  return hip_status("qmoe_qkv_norm_rope");
}

// ====================================================================== prefill
constexpr int AP_QT = 128;               // query rows per workgroup (4 waves x 32)
constexpr int AP_KT = 64;                // keys per step
constexpr int AP_ROWB = HD * 2;          // bytes per K / V row in LDS (no pad: chunks are swizzled)
constexpr int AP_TILE = AP_KT * AP_ROWB;  // 16 KB per K or V tile
constexpr float AP_TAU = 8.0f;           // lazy-max slack (log2 units): p < 2^8 between rescales
// The tile DMAs address a (batch, kv head) cache slice with 32-bit byte
// offsets: (S_max + AP_KT) * AP_ROWB must stay below 2^31.
constexpr int AP_MAX_SMAX = 1 << 22;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// LDS slot of the 16-byte chunk c of K row r.  A fragment read (ds_read_b128)
// takes one chunk of 16 consecutive rows; r % 16 puts them on 16 distinct
// bank groups.
__device__ __forceinline__ int ap_kslot(int r, int c) { return c ^ (r & 15); }
// LDS slot of chunk c of V row r.  A transposing read (ds_read_b64_tr_b16)
// covers, per half-wave, 4 consecutive rows (4-aligned) x 4 consecutive
// chunks (4-aligned), and per 16-lane group 4 rows x 2 chunks; this XOR keeps
// both on distinct bank groups.
__device__ __forceinline__ int ap_vslot(int r, int c) { return c ^ (4 * (r & 3) + 2 * ((r >> 1) & 1)); }

// ds_read_b64_tr_b16: each group of 16 lanes reads a block of 16 x 4 bf16
// (lane j supplies the address of row j: 4 consecutive elements) and lane i
// receives column i % 4 of rows i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12.
__device__ __forceinline__ s16x4 lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// start_dev, when not null, holds the chunk start in device memory (read here,
// clamped into [0, S_max - S]) so a captured graph can replay the same
// launch at a new position; otherwise `start` is used.
//
// K and V tiles go global -> LDS by DMA (`buffer_load_dwordx4 ... lds`, no
// VGPR staging), both row-major with swizzled chunks, double-buffered.  S^T =
// K . Q^T reads K fragments with ds_read_b128; O^T = V^T . P^T reads its V^T
// fragments straight out of the row-major V tile with the transposing LDS
// read, in the key order of the P^T registers (no transposed copy of V).
// Per 64-key step kt: the S^T MFMAs of step kt+1 are issued before the
// softmax and the O^T MFMAs of step kt, so the softmax's VALU work runs while
// the matrix pipe is busy; then one barrier, after which K(kt+3) and V(kt+2)
// are DMA'd into the buffers that K(kt+1) and V(kt) just left.  The DMA
// sources are range-checked buffer loads ending at kv_end, so rows past the
// visible range read as zeros.
// Key-split form (kt_split > 0, host-known start): a query tile whose keys
// span n_kt > kt_split 64-key tiles is split into ceil(n_kt / kt_split) <=
// AP_MAX_SPLITS workgroups over consecutive key ranges, so a small grid (a
// batch-1 prompt) fills the GPU and its longest chain of key steps shortens.
// Each split stores its unnormalised partial (m, l, O) through to memory
// (ap_st16), waits for the stores and adds 1 to the tile's counter; the
// split that counts in last merges the partials in split order (its own
// from registers), writes the output and sets the counter back to zero.
// Partial records sit at the workgroup's grid index.  (Counting arrivals
// first, so the last split skips its own store, was slower: the stores of
// the others then start a round trip later.)
struct ApSplit {
  int kt_split;   // 0: every query tile in one workgroup
  float* part;    // [gridDim.x][AP_PREC]
  int32_t* cnt;   // [B * Hq * n_qt], zero between calls
};
constexpr int AP_PREC = 2 * AP_QT + AP_QT * HD;  // m[128], l[128], O (fp32, register order)
constexpr int AP_MAX_SPLITS = 2;  // key splits per query tile

__device__ __forceinline__ void ap_st16(float* p, float a, float b, float c, float d) {
  const f32x4 w = {a, b, c, d};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}

__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int B, int S, int Hq, int Hkv, int S_max, int start,
    const int32_t* __restrict__ start_dev, float scale_log2, uint16_t* __restrict__ out, ApSplit sp) {
  if (start_dev) start = min(max(start_dev[0], 0), S_max - S);
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * AP_TILE];  // K0, K1, V0, V1
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  // One-dimensional grid in bands of one query tile each, the heaviest (latest)
  // tile first, so the long workgroups start first and the short ones fill
  // the end.  Inside a band, item r = hin * (B * Hkv) + (b * Hkv + kvh): the q
  // heads sharing a kv head sit B * Hkv items apart, i.e. on one XCD when
  // B * Hkv is a multiple of 8 (workgroup i runs on XCD i % 8), whose L2
  // then serves their K/V tiles.
  const int n_qt = (S + AP_QT - 1) / AP_QT, G = Hq / Hkv, n_grp = B * Hkv;
  // query tile, key split (bands of ns(qt) * B * Hq workgroups, latest tile first)
  auto n_kt_of = [&](int t) { return (start + min((t + 1) * AP_QT, S) + AP_KT - 1) / AP_KT; };
  auto ns_of = [&](int t) { return sp.kt_split > 0 ? (n_kt_of(t) + sp.kt_split - 1) / sp.kt_split : 1; };
  int qt = n_qt - 1 - int(blockIdx.x) / (n_grp * G), rem = int(blockIdx.x) % (n_grp * G), band0 = 0;
  if (sp.kt_split > 0) {  // a few bands (the host splits small grids only)
    qt = n_qt - 1;
    rem = int(blockIdx.x);
    for (; qt > 0 && rem >= ns_of(qt) * n_grp * G; --qt) {
      rem -= ns_of(qt) * n_grp * G;
      band0 += ns_of(qt) * n_grp * G;
    }
  }
  const int ns = ns_of(qt), split = rem / (n_grp * G);
  const int r_band = rem % (n_grp * G), grp = r_band % n_grp;
  const int kvh = grp % Hkv, b = grp / Hkv, h = kvh * G + r_band / n_grp;
  const int q0 = qt * AP_QT;
  const int qrow = q0 + wave * 32 + (lane & 31);  // this lane's query (column of S^T)
  const int hl = lane >> 5;
  const int64_t kv_base = (int64_t(b) * Hkv + kvh) * S_max * HD;

  // Q fragments (B operand of S^T = K Q^T): d = ks*16 + hl*8 + [0,8)
  bf16x8 qf[HD / 16];
  {
    const bool ok = qrow < S;
    const uint16_t* qp = q + ((int64_t(b) * S + (ok ? qrow : 0)) * Hq + h) * HD + hl * 8;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      u32x4 v = ok ? ld16(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
      qf[ks] = *reinterpret_cast<bf16x8*>(&v);
    }
  }
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  // Running max m_run (log2 units, shared by lanes l and l ^ 32, which hold
  // the same query) and this lane's share of the row sum l_run.  The max is
  // updated lazily: O and l are rescaled only when a query's tile max exceeds
  // m_run by more than AP_TAU, so p = 2^(s - m_run) stays below 2^AP_TAU
  // and most steps skip the rescale (O / l does not depend on which
  // reference max was used).
  float m_run = -INFINITY, l_run = 0.0f;
  const int q_idx = start + qrow;               // cache index of this query
  const int kv_end = start + min(q0 + AP_QT, S);  // keys [0, kv_end) can be visible
  // this workgroup's key tiles: [kt0, kt0 + n_kt) of the query tile's
  const int kt0 = ns > 1 ? split * sp.kt_split : 0;
  const int n_kt = ns > 1 ? min(sp.kt_split, (kv_end + AP_KT - 1) / AP_KT - kt0) : (kv_end + AP_KT - 1) / AP_KT;
  const int kv_hi = ns > 1 ? min(kv_end, (kt0 + n_kt) * AP_KT) : kv_end;  // keys the DMA may read
  // keys this wave can see: [0, wave_last]; a tile that ends at or below
  // wave_first is visible to every query of the wave (no mask)
  const int wave_first = start + q0 + wave * 32;
  const int wave_last = min(wave_first + 31, kv_end - 1);
  const int lim = min(q_idx, kv_end - 1);  // keys visible to this lane's query: [0, lim]

  // DMA: wave w writes rows [16w, 16w + 16) of each K / V tile with four
  // instructions of 4 rows (1 KB of LDS each); lane j fills slot j % 16 of row
  // 16w + 4i + j / 16, so it fetches the chunk whose swizzled slot that is
  // (both swizzles are XOR involutions).
  const int64_t kv_lo = kv_base + int64_t(kt0) * AP_KT * HD;
  const pipe::i32x4 rk = pipe::make_rsrc(k_cache + kv_lo, uint32_t(kv_hi - kt0 * AP_KT) * AP_ROWB);
  const pipe::i32x4 rv = pipe::make_rsrc(v_cache + kv_lo, uint32_t(kv_hi - kt0 * AP_KT) * AP_ROWB);
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + (lane >> 4), s = lane & 15;
    koff[i] = uint32_t(r * AP_ROWB + ap_kslot(r, s) * 16);
    voff[i] = uint32_t(r * AP_ROWB + ap_vslot(r, s) * 16);
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  auto dma_k = [&](int kt, int buf) {
    const uint32_t dst = lds0 + uint32_t(buf * AP_TILE + wave * 4096), adv = uint32_t(kt) * AP_TILE;
#pragma unroll
    for (int i = 0; i < 4; ++i) pipe::dma16(dst + i * 1024, koff[i] + adv, rk, 0);
  };
  auto dma_v = [&](int kt, int buf) {
    const uint32_t dst = lds0 + uint32_t((2 + buf) * AP_TILE + wave * 4096), adv = uint32_t(kt) * AP_TILE;
#pragma unroll
    for (int i = 0; i < 4; ++i) pipe::dma16(dst + i * 1024, voff[i] + adv, rv, 0);
  };

  // S^T blocks of the tile in K buffer buf: keys [0,32) and [32,64) x this
  // wave's 32 queries, the two MFMA chains interleaved, both always computed
  // (keys past the wave's last query are masked in the softmax; a partial
  // 32-key half would make the score registers a merge of two paths, which
  // the compiler resolves with a copy of all 32 of them on every step).  Row
  // lane % 32 (+ 32) of the tile, chunk 2 ks + hl.
  auto qk = [&](int buf, f32x16 (&st)[2]) {
    const uint8_t* kp = smem + buf * AP_TILE + (lane & 31) * AP_ROWB;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      const int so = ap_kslot(lane, 2 * ks + hl) * 16;
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(kp + so);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(kp + 32 * AP_ROWB + so);
      st[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[ks], ks ? st[0] : f32x16{}, 0, 0, 0);
      st[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[ks], ks ? st[1] : f32x16{}, 0, 0, 0);
    }
  };

  // V^T fragments.  MFMA s of O^T += V^T P^T takes keys 16s..16s+15 in the
  // order of the P^T registers: element jj of lane l (hl = l / 32) is key
  // 16s + 8 (jj / 4) + 4 hl + jj % 4, and the A operand of lane l is dim
  // 32 db + l % 32 at those keys.  Two transposing reads give it: read rd
  // (keys 16s + 8 rd + 4 hl + [0, 4)) has lane l of 16-lane group g point at
  // row 16s + 8 rd + 4 (g / 2) + e (e = (l / 4) % 4), dims
  // 32 db + 16 (g % 2) + 4 (l % 4) + [0, 4): chunk 4 db + 2 (g % 2) + (l % 4) / 2,
  // byte 8 ((l % 4) % 2) in it.  With r % 4 == e the slot is
  // 4 (db ^ e) + ((2 (g % 2) + (l % 4) / 2) ^ 2 (e / 2)).
  const int vg = lane >> 4, ve = (lane >> 2) & 3, vq = lane & 3;
  const uint32_t vlane = uint32_t((4 * (vg >> 1) + ve) * AP_ROWB +
                                  (((2 * (vg & 1) + (vq >> 1)) ^ (2 * (ve >> 1))) * 16) + 8 * (vq & 1));
  uint32_t vdb[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) vdb[db] = vlane + uint32_t(64 * (db ^ ve));

  // softmax of the tile at kv0 and O^T += V^T P^T (V of this tile in buffer buf)
  auto softmax_pv = [&](int buf, int kv0, f32x16 (&st)[2]) {
    const bool live1 = kv0 + 32 <= wave_last;
    // causal / range mask only where a tile reaches past the wave's first
    // query (this covers every tile with keys 32..63 past the wave's last
    // query: live1 false)
    if (kv0 + AP_KT - 1 > wave_first || kv0 + AP_KT > kv_end) {
      asm volatile("");  // keeps this a branch: the mask is not worth computing on every step
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kv0 + kb * 32 + (i >> 2) * 8 + hl * 4 + (i & 3);
          if (key > lim) st[kb][i] = -INFINITY;
        }
    }
    // max as a tree of 3-input maxima (v_max3_f32): 17 instructions, 4 deep
    float mx[11];
#pragma unroll
    for (int g = 0; g < 11; ++g) {
      const int a = 3 * g, b = 3 * g + 1, c = 3 * g + 2;
      const float va = st[a >> 4][a & 15], vb = st[b >> 4][b & 15];
      mx[g] = c < 32 ? fmaxf(fmaxf(va, vb), st[c >> 4][c & 15]) : fmaxf(va, vb);
    }
    const float m0 = fmaxf(fmaxf(mx[0], mx[1]), mx[2]), m1 = fmaxf(fmaxf(mx[3], mx[4]), mx[5]);
    const float m2 = fmaxf(fmaxf(mx[6], mx[7]), mx[8]), m3 = fmaxf(mx[9], mx[10]);
    float mloc = fmaxf(fmaxf(fmaxf(m0, m1), m2), m3);
    {  // max with lane l ^ 32 (the other half of the same query's keys)
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
      mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
    }
    const bool grow = mloc > m_run + AP_TAU;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mloc : m_run;
      // 1 where the max stays; 0 on a query's first visible tile (O, l are 0)
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
      m_run = m_new;
    }
    // p = 2^(s * scale - m) in one FMA + v_exp (masked s = -inf gives 0); a
    // lane with no visible key yet keeps m_run = -inf and every s = -inf.
    // The row sum adds the fp32 p; P goes to bf16 pairs (the MFMA's B operand).
    const float mb = m_run == -INFINITY ? 0.0f : m_run;
    uint32_t pk[2][8];
    float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four partial row sums (short chains)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(st[kb][2 * i], scale_log2, -mb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(st[kb][2 * i + 1], scale_log2, -mb));
        const bf16x2_t pp = {static_cast<__bf16>(p0), static_cast<__bf16>(p1)};
        pk[kb][i] = __builtin_bit_cast(uint32_t, pp);
        ls[2 * (i & 1)] += p0;
        ls[2 * (i & 1) + 1] += p1;
      }
    l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    // O^T += V^T P^T over 4 steps of 16 keys (the last two only for live keys 32..63)
    const uint8_t* vb = smem + (2 + buf) * AP_TILE;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s >= 2 && !live1) break;
      const u32x4 pw = {pk[s >> 1][(s & 1) * 4], pk[s >> 1][(s & 1) * 4 + 1], pk[s >> 1][(s & 1) * 4 + 2],
                        pk[s >> 1][(s & 1) * 4 + 3]};
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const s16x4 v0 = lds_read_tr16(vb + vdb[db] + (16 * s) * AP_ROWB);
        const s16x4 v1 = lds_read_tr16(vb + vdb[db] + (16 * s + 8) * AP_ROWB);
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, o[db], 0, 0, 0);
      }
    }
  };

  // Prologue: K(0), V(0), K(1), V(1) in flight; wait for the first three.
  dma_k(0, 0);
  dma_v(0, 0);
  if (n_kt > 1) {
    dma_k(1, 1);
    dma_v(1, 1);
    pipe::wait_vm<4>();
  } else {
    pipe::wait_vm<0>();
  }
  __syncthreads();  // K(0), V(0), K(1) visible
  f32x16 sc[2], sn[2];
  qk(0, sc);
  if (n_kt > 2) {
    __syncthreads();  // every wave is done with K(0)'s buffer
    dma_k(2, 0);
  }
  // Steps in pairs, the score registers swapping roles (no copy of the next
  // tile's scores).  Step kt: the next tile's S^T into nxt (whenever there
  // is a next tile, also past this wave's last query: the scores are then
  // never read, and an unconditional nxt keeps its old value dead), this
  // tile's softmax and O^T; then K(kt+2) and V(kt+1), issued after the
  // previous barrier, have landed, and the barrier makes them visible and
  // frees K(kt+1)'s and V(kt)'s buffers.
  auto one = [&](int kt, f32x16 (&cur)[2], f32x16 (&nxt)[2], auto has_next) {
    const int kv0 = (kt0 + kt) * AP_KT, buf = kt & 1;
    if constexpr (decltype(has_next)::value) qk(buf ^ 1, nxt);
    if (kv0 <= wave_last) softmax_pv(buf, kv0, cur);  // past this wave's queries: nothing (wave-uniform)
    pipe::wait_vm<0>();
    __syncthreads();
    if (kt + 3 < n_kt) dma_k(kt + 3, buf ^ 1);
    if (kt + 2 < n_kt) dma_v(kt + 2, buf);
  };
  int kt = 0;
  for (; kt + 2 < n_kt; kt += 2) {
    one(kt, sc, sn, std::true_type{});
    one(kt + 1, sn, sc, std::true_type{});
  }
  if (kt + 1 < n_kt) {
    one(kt, sc, sn, std::true_type{});
    one(kt + 1, sn, sc, std::false_type{});
  } else {
    one(kt, sc, sn, std::false_type{});
  }
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (ns > 1) {
    // partial of this split -> memory; the split that counts in last merges
    const int qloc = wave * 32 + (lane & 31);
    float* rec = sp.part + int64_t(blockIdx.x) * AP_PREC;
    if (hl == 0) {
      __hip_atomic_store(rec + qloc, m_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(rec + AP_QT + qloc, l_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // O in register order: chunk (wave, db, g) of 64 lanes x 16 bytes, so each
    // store (and the merging workgroup's load) covers 1 KB of contiguous memory
    float* ob = rec + 2 * AP_QT + (wave * 16 * 64 + lane) * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        ap_st16(ob + (db * 4 + g) * 256, o[db][g * 4], o[db][g * 4 + 1], o[db][g * 4 + 2], o[db][g * 4 + 3]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // every wave's partial is in memory (and the K/V tiles are free)
    int* s_last = reinterpret_cast<int*>(smem);
    int32_t* cnt = sp.cnt + (int64_t(b) * Hq + h) * n_qt + qt;
    if (t == 0) *s_last = atomicAdd(cnt, 1) == ns - 1;
    __syncthreads();
    if (!*s_last) return;
    if (t == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    auto rec_of = [&](int j) { return sp.part + int64_t(band0 + j * n_grp * G + r_band) * AP_PREC; };
    // every other split's (m, l, O) requested at once (ns <= AP_MAX_SPLITS),
    // then combined in split order
    float mj[AP_MAX_SPLITS], lj[AP_MAX_SPLITS];
    float4 oj[AP_MAX_SPLITS][16];
#pragma unroll
    for (int j = 0; j < AP_MAX_SPLITS; ++j) {
      if (j < ns && j != split) {
        const float* rj = rec_of(j);
        mj[j] = rj[qloc];
        lj[j] = rj[AP_QT + qloc];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            oj[j][db * 4 + g] = *reinterpret_cast<const float4*>(rj + 2 * AP_QT + (wave * 16 * 64 + lane) * 4 +
                                                                 (db * 4 + g) * 256);
      } else {
        mj[j] = j == split ? m_run : -INFINITY;
        lj[j] = j == split ? l_run : 0.0f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            oj[j][db * 4 + g] = j == split ? make_float4(o[db][g * 4], o[db][g * 4 + 1], o[db][g * 4 + 2],
                                                         o[db][g * 4 + 3])
                                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < AP_MAX_SPLITS; ++j) M = fmaxf(M, mj[j]);
    float L = 0.0f;
    f32x16 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[db][i] = 0.0f;
#pragma unroll
    for (int j = 0; j < AP_MAX_SPLITS; ++j) {  // split order, whichever split counted in last
      const float w = mj[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mj[j] - M);
      L += w * lj[j];
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 v = oj[j][db * 4 + g];
          acc[db][g * 4] += w * v.x;
          acc[db][g * 4 + 1] += w * v.y;
          acc[db][g * 4 + 2] += w * v.z;
          acc[db][g * 4 + 3] += w * v.w;
        }
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = acc[db];
    l_run = L;
  }
  if (qrow >= S) return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  uint16_t* op = out + ((int64_t(b) * S + qrow) * Hq + h) * HD;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = db * 32 + g * 8 + hl * 4;
      u32x2 v;
      v.x = pack_bf16x2(o[db][g * 4 + 0] * inv, o[db][g * 4 + 1] * inv);
      v.y = pack_bf16x2(o[db][g * 4 + 2] * inv, o[db][g * 4 + 3] * inv);
      *reinterpret_cast<u32x2*>(op + d) = v;
    }
}

// ====================================================================== decode
constexpr int AD_WKEYS = 64;            // keys per wave
constexpr int AD_MAX_SUBS = 4;          // waves per workgroup (one merged partial per workgroup)
constexpr int AD_MAX_G = 16;            // q heads per kv head
constexpr int AD_VCH = AD_WKEYS * HD / 8 / 64;  // 16-byte V chunks per lane (16)
constexpr int AD_PSTR = HD + 4;         // partial record: m, l, 2 pad, o[HD] (16-byte aligned o)
constexpr int AD_MERGE_PF = 16;         // o values the merge requests before the max is known

// Completes this wave's LDS writes before its own lanes read them (a wave's
// DS instructions run in order; this also keeps the compiler from moving
// reads above the writes).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Query rows: blockIdx.z.  With chunk_start == nullptr each query row is a
// batch row (cache row = query row) with ctx_len[row] keys; otherwise qpb
// consecutive query rows share cache row row / qpb and query s = row % qpb
// sits at position start + s (start = *chunk_start clamped into
// [0, S_max - qpb]) and sees keys [0, start + s].
__device__ __forceinline__ int ad_ctx(const int32_t* ctx_len, const int32_t* chunk_start, int row, int qpb,
                                      int S_max, int max_ctx) {
  if (chunk_start) return min(max(chunk_start[0], 0), S_max - qpb) + row % qpb + 1;
  return min(ctx_len[row], max_ctx);
}

// Fused decode (one query per batch row at positions[row]): the row sees the
// cache entries [0, position] once its own K/V row is in, at most max_ctx of
// them; a position outside [0, min(S_max, max_pos)) sees none (output 0).
__device__ __forceinline__ int ad_ctx_pos(const int32_t* positions, int row, int S_max, int max_pos,
                                          int max_ctx) {
  const int p = positions[row];
  return (p >= 0 && p < S_max && p < max_pos) ? min(p + 1, max_ctx) : 0;
}

// What the fused decode attention reads in place of q: the fp32 QKV
// projection rows and the finish parameters (as qkv_finish_kernel takes
// them), and the caches it writes each row's new K/V into.
struct AdFinish {
  const float* raw;  // [B][(Hq + 2 Hkv) * HD]
  const uint16_t* qn_w;
  const uint16_t* kn_w;
  const float* cos;  // [max_pos][HD / 2]
  const float* sin;
  const int32_t* positions;  // [B]
  int max_pos;
  float eps;
  uint16_t* k_out;  // the caches
  uint16_t* v_out;
};

// Workgroup = (split of SUBS x 64 keys, kv head, query row); wave w owns the
// split's keys [64 w, 64 w + 64) and all G q heads of the group.  Per wave,
// on v_mfma_f32_32x32x16_bf16:
//   S^T [64 keys x 32] = K [64 x 128] . Q^T [128 x 32]   (q heads in columns
//       0..G-1; K rows loaded from the cache straight into A-operand registers)
//   softmax over keys per column: lane l holds column l % 32, 32 keys; one
//       exchange with lane l ^ 32
//   O^T [128 x 32] = V^T [128 x 64] . P^T [64 x 32]   (P^T straight from the
//       S^T registers, which already hold it in the B-operand layout; V goes
//       into this wave's LDS row-major and the V^T fragments come from
//       transposing reads in the key order of those registers)
// Every global load of the wave is issued first (K, V, q), so a wave costs
// one HBM round trip.  With SUBS == 1 (small batch x context: the K/V
// stream of a batch-1 step spreads over ctx/64 x Hkv CUs) each wave writes
// its partial (m, l, o); with SUBS > 1 the waves merge theirs through LDS
// and the workgroup writes one, so the merge kernel reads SUBS times fewer.
//
// FUSED: the QKV finish of the step runs here instead of in its own launch.
// The workgroup's waves normalise and rotate the group's G q heads from the
// fp32 projection (heads w, w + SUBS, ... per wave; finish_head, so the same
// bits as qkv_finish_kernel) into LDS, and the one wave whose keys hold the
// row's position p computes that row's K and V, stores them to the caches
// for later steps and uses them in place of the cache row p it loaded (no
// other workgroup reads row p: it lies in exactly one wave's key range).
// The K/V stream and the score/PV MFMAs are then those of the unfused path.
template <int SUBS, bool FUSED>
__global__ __launch_bounds__(SUBS * 64) void attn_decode_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, const int32_t* __restrict__ ctx_len,
    const int32_t* __restrict__ chunk_start, int qpb, int Hq, int Hkv, int S_max, int max_ctx, int nsplit,
    float scale, float* __restrict__ partial, AdFinish fin) {
  __shared__ __attribute__((aligned(1024))) uint8_t vs[SUBS][AP_TILE];  // V tile per wave (16 KB)
  __shared__ __attribute__((aligned(16))) uint16_t qs[FUSED ? AD_MAX_G * HD : 8];  // finished q heads
  __shared__ __attribute__((aligned(16))) uint16_t ns[FUSED ? 2 * HD : 8];         // the new K and V rows
  const int lane = threadIdx.x & 63;
  const int wave = SUBS > 1 ? __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)) : 0;
  const int kvh = blockIdx.y, b = blockIdx.z, bc = chunk_start ? b / qpb : b;  // query row, cache row
  const int G = Hq / Hkv;
  const int pos = FUSED ? fin.positions[b] : -1;
  const int ctx = FUSED ? ad_ctx_pos(fin.positions, b, S_max, fin.max_pos, max_ctx)
                        : ad_ctx(ctx_len, chunk_start, b, qpb, S_max, max_ctx);
  const int kw0 = (int(blockIdx.x) * SUBS + wave) * AD_WKEYS;
  const int nk = min(AD_WKEYS, ctx - kw0);
  const int col = lane & 31, hi = lane >> 5;
  // partial record per (b, q head, split): [m, l, -, -, o[0..127]]
  float* pbase = partial + ((int64_t(b) * Hq + kvh * G) * nsplit + blockIdx.x) * AD_PSTR;
  const int64_t pstride = int64_t(nsplit) * AD_PSTR;  // next q head
  if (int(blockIdx.x) * SUBS * AD_WKEYS >= ctx) {  // no key of the split is visible (workgroup-uniform)
    if (threadIdx.x < unsigned(G)) {
      pbase[threadIdx.x * pstride] = -INFINITY;
      pbase[threadIdx.x * pstride + 1] = 0.0f;
    }
    return;
  }
  // FUSED: the projection values this wave finishes are requested before
  // the K/V stream, so the finish waits for them alone
  constexpr int HPW = FUSED ? (AD_MAX_G + SUBS - 1) / SUBS : 1;  // q heads per wave, at most
  const bool owner = FUSED && pos < ctx && pos >= kw0 && pos < kw0 + AD_WKEYS;  // wave-uniform
  // a position at or past max_ctx lies in no visible key range: split 0's
  // wave 0 still stores its K/V row (as qmoe_qkv_finish would)
  const bool writer = owner || (FUSED && pos >= ctx && blockIdx.x == 0 && wave == 0);
  // (the first 8 heads branch-free, heads past G loading head G - 1 again;
  // heads 8-15 behind one test; a scheduling barrier keeps all of it ahead
  // of the K/V requests, so the finish waits for these loads alone)
  constexpr int HLO = (8 + SUBS - 1) / SUBS;  // per-wave share of the first 8 heads
  float rlo[HPW], rhi[HPW], nlo[2], nhi[2], c = 0.0f, sn = 0.0f;
  uint16_t wq[2] = {0, 0}, wk[2] = {0, 0};  // norm weights, converted where used
  if constexpr (FUSED) {
    const float* rq = fin.raw + (int64_t(b) * (Hq + 2 * Hkv) + kvh * G) * HD;
#pragma unroll
    for (int i = 0; i < HLO; ++i) {
      const int h = min(wave + i * SUBS, G - 1);
      rlo[i] = rq[h * HD + lane];
      rhi[i] = rq[h * HD + lane + 64];
    }
    if (G > 8) {
#pragma unroll
      for (int i = HLO; i < HPW; ++i) {
        const int h = min(wave + i * SUBS, G - 1);
        rlo[i] = rq[h * HD + lane];
        rhi[i] = rq[h * HD + lane + 64];
      }
    }
    c = fin.cos[int64_t(pos) * (HD / 2) + lane];
    sn = fin.sin[int64_t(pos) * (HD / 2) + lane];
    wq[0] = fin.qn_w[lane];
    wq[1] = fin.qn_w[lane + 64];
    wk[0] = fin.kn_w[lane];
    wk[1] = fin.kn_w[lane + 64];
    const float* rk = fin.raw + (int64_t(b) * (Hq + 2 * Hkv) + Hq + kvh) * HD;
    const float* rv = rk + int64_t(Hkv) * HD;
    nlo[0] = rk[lane];
    nhi[0] = rk[lane + 64];
    nlo[1] = rv[lane];
    nhi[1] = rv[lane + 64];
    __builtin_amdgcn_sched_barrier(0);
  }
  float m = -INFINITY, l = 0.0f;
  f32x16 oacc[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db) oacc[db] = f32x16{};
  const int64_t kv_base = (int64_t(bc) * Hkv + kvh) * S_max * HD;
  // K rows as A operands: block mb, k-step ks: key kw0 + mb*32 + col, dims ks*16 + hi*8
  u32x4 ka[2][HD / 16];
  // V: chunk c = lane + 64 i is row c / 16 (key), dim chunk c % 16; rows
  // past nk repeat the last visible key (their p is 0)
  u32x4 vr[AD_VCH];
  // FUSED: waves past the context load row ctx - 1 and use none of it, so the
  // loads need no branch (one would make the finish wait for every load)
  if (FUSED || nk > 0) {  // wave-uniform
    const int r0 = nk > 0 ? kw0 : ctx - 1, rl = max(nk, 1) - 1;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint16_t* kp = k_cache + kv_base + int64_t(r0 + min(mb * 32 + col, rl)) * HD + hi * 8;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) ka[mb][ks] = ld16(kp + ks * 16);
    }
#pragma unroll
    for (int i = 0; i < AD_VCH; ++i) {
      const int c = lane + 64 * i;
      vr[i] = ld16(v_cache + kv_base + int64_t(r0 + min(c >> 4, rl)) * HD + (c & 15) * 8);
    }
  }
  // Q^T as B operands: column col = q head, dims ks*16 + hi*8 (zero past G)
  u32x4 qb[HD / 16];
  if constexpr (FUSED) {  // every wave, keys or not: the q heads are shared out over all of them
    const float wl = bf16_to_f32(wq[0]), wh = bf16_to_f32(wq[1]);
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int h = wave + i * SUBS;
      if (h < G) {  // wave-uniform
        finish_head(rlo[i], rhi[i], wl, wh, c, sn, fin.eps);
        qs[h * HD + lane] = f32_to_bf16(rlo[i]);
        qs[h * HD + lane + 64] = f32_to_bf16(rhi[i]);
      }
    }
    if (writer) {
      finish_head(nlo[0], nhi[0], bf16_to_f32(wk[0]), bf16_to_f32(wk[1]), c, sn, fin.eps);
      const int64_t row = kv_base + int64_t(pos) * HD;
      const uint16_t k0 = f32_to_bf16(nlo[0]), k1 = f32_to_bf16(nhi[0]);
      const uint16_t v0 = f32_to_bf16(nlo[1]), v1 = f32_to_bf16(nhi[1]);
      fin.k_out[row + lane] = k0;
      fin.k_out[row + lane + 64] = k1;
      fin.v_out[row + lane] = v0;
      fin.v_out[row + lane + 64] = v1;
      ns[lane] = k0;
      ns[lane + 64] = k1;
      ns[HD + lane] = v0;
      ns[HD + lane + 64] = v1;
    }
    if constexpr (SUBS > 1)
      __syncthreads();
    else
      wave_lds_sync();
    const uint16_t* qp = qs + min(col, G - 1) * HD + hi * 8;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks)
      qb[ks] = col < G ? *reinterpret_cast<const u32x4*>(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
    if (owner) {  // row p of the cache is not written yet: take the new row
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        if (kw0 + min(mb * 32 + col, nk - 1) == pos) {
#pragma unroll
          for (int ks = 0; ks < HD / 16; ++ks) ka[mb][ks] = *reinterpret_cast<const u32x4*>(ns + ks * 16 + hi * 8);
        }
#pragma unroll
      for (int i = 0; i < AD_VCH; ++i) {
        const int cc = lane + 64 * i;
        if (kw0 + min(cc >> 4, nk - 1) == pos) vr[i] = *reinterpret_cast<const u32x4*>(ns + HD + (cc & 15) * 8);
      }
    }
  } else if (nk > 0) {
    const uint16_t* qp = q + (int64_t(b) * Hq + kvh * G + min(col, G - 1)) * HD + hi * 8;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qb[ks] = col < G ? ld16(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
  }
  if (nk > 0) {  // wave-uniform
    // V into this wave's LDS, row-major with the prefill's chunk swizzle
    uint8_t* vb = vs[wave];
#pragma unroll
    for (int i = 0; i < AD_VCH; ++i) {
      const int c = lane + 64 * i, r = c >> 4;
      *reinterpret_cast<u32x4*>(vb + r * AP_ROWB + ap_vslot(r, c & 15) * 16) = vr[i];
    }

    f32x16 sacc[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      sacc[mb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks)
        sacc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ka[mb][ks]),
                                                           __builtin_bit_cast(bf16x8, qb[ks]), sacc[mb], 0,
                                                           0, 0);
    }
    // element e of block mb: key mb*32 + (e/4)*8 + hi*4 + e%4, column col
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = mb * 32 + (e >> 2) * 8 + hi * 4 + (e & 3);
        const float sv = key < nk ? sacc[mb][e] * scale : -INFINITY;
        sacc[mb][e] = sv;
        m = fmaxf(m, sv);
      }
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    uint32_t pk[2][8];  // P^T as bf16 pairs: the B operand, keys in accumulator order
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p0 = __expf(sacc[mb][2 * i] - m), p1 = __expf(sacc[mb][2 * i + 1] - m);
        l += p0 + p1;
        const bf16x2_t pp = {static_cast<__bf16>(p0), static_cast<__bf16>(p1)};
        pk[mb][i] = __builtin_bit_cast(uint32_t, pp);
      }
    l += __shfl_xor(l, 32, 64);
    wave_lds_sync();

    // O^T += V^T P^T, 16 keys per MFMA: element jj of the P^T operand of
    // lane l is key 16s + 8 (jj / 4) + 4 (l / 32) + jj % 4, and two
    // transposing reads give the matching V^T rows (same addressing as the
    // prefill kernel's V^T fragments)
    const int vg = lane >> 4, ve = (lane >> 2) & 3, vq = lane & 3;
    const uint32_t vlane = uint32_t((4 * (vg >> 1) + ve) * AP_ROWB +
                                    (((2 * (vg & 1) + (vq >> 1)) ^ (2 * (ve >> 1))) * 16) + 8 * (vq & 1));
#pragma unroll
    for (int s = 0; s < AD_WKEYS / 16; ++s) {
      const u32x4 pw = {pk[s >> 1][(s & 1) * 4], pk[s >> 1][(s & 1) * 4 + 1], pk[s >> 1][(s & 1) * 4 + 2],
                        pk[s >> 1][(s & 1) * 4 + 3]};
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) {
        const uint32_t va = vlane + uint32_t(64 * (db ^ ve));
        const s16x4 v0 = lds_read_tr16(vb + va + (16 * s) * AP_ROWB);
        const s16x4 v1 = lds_read_tr16(vb + va + (16 * s + 8) * AP_ROWB);
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, oacc[db], 0, 0, 0);
      }
    }
  }
  // element e of block db: d = db*32 + (e/4)*8 + hi*4 + e%4, column col = q head
  if constexpr (SUBS == 1) {
    if (col < G) {
      float* pg = pbase + col * pstride;
      if (hi == 0) {
        pg[0] = m;
        pg[1] = l;
      }
#pragma unroll
      for (int db = 0; db < HD / 32; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
          *reinterpret_cast<float4*>(pg + 4 + db * 32 + e4 * 8 + hi * 4) =
              make_float4(oacc[db][e4 * 4], oacc[db][e4 * 4 + 1], oacc[db][e4 * 4 + 2], oacc[db][e4 * 4 + 3]);
    }
  } else {
    // Merge the waves' (m, l, o) in LDS: wave w's record of column c at
    // float offset (w * AD_MAX_G + c) * AD_PSTR of the V area (free once
    // every wave's O^T MFMAs have read it).
    float* rec = reinterpret_cast<float*>(&vs[0][0]);
    static_assert(SUBS * AD_MAX_G * AD_PSTR * 4 <= SUBS * AP_TILE, "merge records fit the V tiles");
    __syncthreads();
    if (col < G) {
      float* pg = rec + (wave * AD_MAX_G + col) * AD_PSTR;
      if (hi == 0) {
        pg[0] = m;
        pg[1] = l;
      }
#pragma unroll
      for (int db = 0; db < HD / 32; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
          *reinterpret_cast<float4*>(pg + 4 + db * 32 + e4 * 8 + hi * 4) =
              make_float4(oacc[db][e4 * 4], oacc[db][e4 * 4 + 1], oacc[db][e4 * 4 + 2], oacc[db][e4 * 4 + 3]);
    }
    __syncthreads();
    // thread t: column t / (SUBS * 64 / G) ... every (column, dim) once;
    // waves without visible keys carry m = -inf, l = 0, o = 0 (weight 0)
    for (int i = int(threadIdx.x); i < G * HD; i += SUBS * 64) {
      const int c = i / HD, d = i % HD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < SUBS; ++w) M = fmaxf(M, rec[(w * AD_MAX_G + c) * AD_PSTR]);
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < SUBS; ++w) {
        const float* r = rec + (w * AD_MAX_G + c) * AD_PSTR;
        const float wt = r[0] == -INFINITY ? 0.0f : __expf(r[0] - M);
        L = fmaf(wt, r[1], L);
        O = fmaf(wt, r[4 + d], O);
      }
      float* pg = pbase + c * pstride;
      if (d == 0) {
        pg[0] = M;
        pg[1] = L;
      }
      pg[4 + d] = O;
    }
  }
}

// Merge of the partials that hold keys (ceil(ctx / keys_per_split) of them),
// in chunks of HD partials: thread i reads partial i's (m, l) and its weight
// exp(m - M) goes to LDS; then every thread (one output dim d) adds its o[d]
// of the chunk, eight loads in flight at a time.
// max_pos > 0: the fused decode's merge (ctx_len holds the positions).  A
// row without visible keys gets zeros.
__global__ __launch_bounds__(HD) void attn_decode_merge_kernel(const float* __restrict__ partial,
                                                               const int32_t* __restrict__ ctx_len,
                                                               const int32_t* __restrict__ chunk_start,
                                                               int qpb, int S_max, int Hq, int max_ctx, int nsplit,
                                                               int split_keys, int max_pos,
                                                               uint16_t* __restrict__ out) {
  __shared__ float sw[HD];
  __shared__ float sred[2];
  const int bh = blockIdx.x;  // b * Hq + h
  const int d = threadIdx.x, lane = d & 63, wave = d >> 6;
  const float* p = partial + int64_t(bh) * nsplit * AD_PSTR;
  // Loads that wait for nothing go out first, together with the context
  // length: this thread's (m, l) of partial min(d, nsplit - 1) and the first
  // AD_MERGE_PF o values of its dim.  Every index stays below nsplit (the
  // row's records); values of partials past the visible ones are dropped by
  // the selects below and never enter arithmetic.
  const int dr = min(d, nsplit - 1);
  const float m_raw = p[int64_t(dr) * AD_PSTR];
  const float l_raw = p[int64_t(dr) * AD_PSTR + 1];
  float ov[AD_MERGE_PF];
#pragma unroll
  for (int u = 0; u < AD_MERGE_PF; ++u) ov[u] = p[int64_t(min(u, nsplit - 1)) * AD_PSTR + 4 + d];
  const int ctx = max_pos > 0 ? ad_ctx_pos(ctx_len, bh / Hq, S_max, max_pos, max_ctx)
                              : ad_ctx(ctx_len, chunk_start, bh / Hq, qpb, S_max, max_ctx);
  const int live = min(nsplit, (ctx + split_keys - 1) / split_keys);
  const float mv = d < live ? m_raw : -INFINITY;
  const float lv = d < live ? l_raw : 0.0f;
#pragma unroll
  for (int u = 0; u < AD_MERGE_PF; ++u) ov[u] = u < live ? ov[u] : 0.0f;
  float mloc = mv;
  for (int s = d + HD; s < live; s += HD) mloc = fmaxf(mloc, p[int64_t(s) * AD_PSTR]);
  mloc = wave_max(mloc);
  if (lane == 0) sred[wave] = mloc;
  __syncthreads();
  const float M = fmaxf(sred[0], sred[1]);
  float L = 0.0f, O = 0.0f;
  for (int c0 = 0; c0 < live; c0 += HD) {
    const int n = min(HD, live - c0);
    __syncthreads();
    if (d < n) {
      const float m = c0 == 0 ? mv : p[int64_t(c0 + d) * AD_PSTR];
      const float lsum = c0 == 0 ? lv : p[int64_t(c0 + d) * AD_PSTR + 1];
      sw[d] = m == -INFINITY ? 0.0f : __expf(m - M);
      L += sw[d] * lsum;  // summed over threads below
    }
    __syncthreads();
    int first = 0;
    if (c0 == 0) {
#pragma unroll
      for (int u = 0; u < AD_MERGE_PF; ++u)
        if (u < n) O = fmaf(sw[u], ov[u], O);
      first = AD_MERGE_PF;
    }
    for (int s0 = first; s0 < n; s0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = s0 + u < n ? p[int64_t(c0 + s0 + u) * AD_PSTR + 4 + d] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < n) O = fmaf(sw[s0 + u], v[u], O);
    }
  }
  L = wave_sum(L);
  __syncthreads();
  if (lane == 0) sred[wave] = L;
  __syncthreads();
  const float Lt = sred[0] + sred[1];
  out[int64_t(bh) * HD + d] = f32_to_bf16(Lt > 0.0f ? O / Lt : 0.0f);
}

}  // namespace qmoe

using namespace qmoe;

// The GEMV + finish path: decode-size token counts whose activations fit the
// register GEMV (K = H in {512, 1024, 2048, 4096}, T * H <= 32768).
static bool qkv_decode_path(int64_t T, int64_t H) {
  return T <= QKV_DEC_MAX_T && (H == 512 || H == 1024 || H == 2048 || H == 4096) && T * H <= 32768;
}

extern "C" int64_t qmoe_qkv_norm_rope_workspace(int64_t T, int64_t H, int64_t Hq, int64_t Hkv,
                                                int64_t D) {
  if (T < 0 || H < 0 || Hq < 0 || Hkv < 0 || D < 0) return -1;
  return qkv_decode_path(T, H) ? T * (Hq + 2 * Hkv) * D * int64_t(sizeof(float)) : 0;
}

extern "C" int qmoe_qkv_norm_rope(const qmoe_bf16* x, const qmoe_bf16* wqkv,
                                  const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                                  const float* rope_cos, const float* rope_sin, int64_t max_pos,
                                  const int32_t* positions, int64_t B, int64_t S, int64_t H,
                                  int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float eps,
                                  qmoe_bf16* q_out, qmoe_bf16* k_cache, qmoe_bf16* v_cache,
                                  float* workspace, qmoe_stream_t stream) {
  QMOE_REQUIRE(wqkv && q_norm_w && k_norm_w && rope_cos && rope_sin && k_cache && v_cache &&
                   (B == 0 || S == 0 || (x && positions && q_out)),
               "qmoe_qkv_norm_rope: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_qkv_norm_rope: head_dim must be 128 (D=%lld)", (long long)D);
  QMOE_REQUIRE(H > 0 && H % 64 == 0, "qmoe_qkv_norm_rope: H %% 64 != 0");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq + 2 * Hkv < 65536,
               "qmoe_qkv_norm_rope: bad head counts");
  QMOE_REQUIRE(B >= 0 && S >= 0 && B * S < (1ll << 31), "qmoe_qkv_norm_rope: bad B/S");
  QMOE_REQUIRE(S_max > 0 && max_pos > 0, "qmoe_qkv_norm_rope: bad S_max/max_pos");
  const int64_t T = B * S;
  if (T == 0) return QMOE_OK;
  const int max_p = int(std::min<int64_t>(max_pos, 1ll << 30));
  if (qkv_decode_path(T, H)) {
    QMOE_REQUIRE(workspace, "qmoe_qkv_norm_rope: T <= 16 needs the workspace");
    const int64_t N = (Hq + 2 * Hkv) * HD;
    int rc = gemm_launch(x, H, wqkv, T, N, H, QMOE_GEMM_STORE_F32, workspace, N, as_stream(stream));
    if (rc) return rc;
    hipLaunchKernelGGL(qkv_finish_kernel, dim3(unsigned(Hq + 2 * Hkv), unsigned(T)), dim3(64), 0,
                       as_stream(stream), workspace, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, int(T), int(S),
                       int(Hq), int(Hkv), int(S_max), max_p, eps, q_out, k_cache, v_cache);
    return hip_status("qmoe_qkv_norm_rope(finish)");
  }
  // 128 x 640 tiles on the wide pipeline once they fill every CU at least
  // once (their 32-bit operand offsets need both operands below 2 GiB)
  if ((T + QkvWide::BN - 1) / QkvWide::BN * (((Hq + 2 * Hkv) * HD + QkvWide::BM - 1) / QkvWide::BM) >= 256 &&
      T * H * 2 < (1ll << 31) && (Hq + 2 * Hkv) * HD * H * 2 < (1ll << 31))
    return qkv_wide_launch(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, T, S, H, Hq, Hkv, S_max,
                           max_p, eps, q_out, k_cache, v_cache, as_stream(stream));
  if (T >= QKV_PIPE_MIN_T && H % 64 == 0 && T * H * 2 < (1ll << 32)) {
    // 256-row tiles once they give every CU a workgroup; below that 128-row
    // tiles, two per CU, while they fill the CUs.  Fewer tiles than CUs: one
    // workgroup per CU with four stages in flight, 64-row tiles while those
    // fit in one round, else 128-row ones (the GEMM alone at N = 5120, K =
    // 2048: 384 tokens 19.0 -> 17.5 us, 640 tokens 29.4 -> 23.2 us against
    // 64-row tiles two per CU, which need two rounds from 512 tokens on)
    const int64_t NH = Hq + 2 * Hkv;
    if ((T + 255) / 256 * NH >= 256)
      return qkv_pipe_launch<pipe::Pipe<256, 128, 64, 2>, 1>(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin,
                                                              positions, T, S, H, Hq, Hkv, S_max, max_p, eps, q_out,
                                                              k_cache, v_cache, as_stream(stream));
    if ((T + 127) / 128 * NH >= 256)
      return qkv_pipe_launch<pipe::Pipe<128, 128, 64, 2>, 2>(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin,
                                                              positions, T, S, H, Hq, Hkv, S_max, max_p, eps, q_out,
                                                              k_cache, v_cache, as_stream(stream));
    if ((T + 63) / 64 * NH <= current_device_cus())
      return qkv_pipe_launch<pipe::Pipe<64, 128, 64, 4>, 1>(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin,
                                                             positions, T, S, H, Hq, Hkv, S_max, max_p, eps, q_out,
                                                             k_cache, v_cache, as_stream(stream));
    return qkv_pipe_launch<pipe::Pipe<128, 128, 64, 4>, 1>(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin,
                                                            positions, T, S, H, Hq, Hkv, S_max, max_p, eps, q_out,
                                                            k_cache, v_cache, as_stream(stream));
  }
  dim3 grid(unsigned(Hq + 2 * Hkv), unsigned((T + tile::BM - 1) / tile::BM));
  hipLaunchKernelGGL(qkv_norm_rope_kernel, grid, dim3(256), 0, as_stream(stream), x, wqkv, q_norm_w,
                     k_norm_w, rope_cos, rope_sin, positions, int(T), int(S), int(H), int(Hq),
                     int(Hkv), int(S_max), max_p, eps, q_out, k_cache, v_cache);
  return hip_status("qmoe_qkv_norm_rope");
}

extern "C" int qmoe_qkv_finish(const float* qkv, const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                               const float* rope_cos, const float* rope_sin, int64_t max_pos,
                               const int32_t* positions, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                               int64_t D, int64_t S_max, float eps, qmoe_bf16* q_out, qmoe_bf16* k_cache,
                               qmoe_bf16* v_cache, qmoe_stream_t stream) {
  QMOE_REQUIRE(q_norm_w && k_norm_w && rope_cos && rope_sin && k_cache && v_cache &&
                   (B == 0 || S == 0 || (qkv && positions && q_out)),
               "qmoe_qkv_finish: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_qkv_finish: head_dim must be 128 (D=%lld)", (long long)D);
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq + 2 * Hkv < 65536, "qmoe_qkv_finish: bad head counts");
  QMOE_REQUIRE(B >= 0 && S >= 0 && B * S <= QKV_DEC_MAX_T, "qmoe_qkv_finish: need B*S <= 16");
  QMOE_REQUIRE(S_max > 0 && max_pos > 0, "qmoe_qkv_finish: bad S_max/max_pos");
  const int64_t T = B * S;
  if (T == 0) return QMOE_OK;
  const int max_p = int(std::min<int64_t>(max_pos, 1ll << 30));
  hipLaunchKernelGGL(qkv_finish_kernel, dim3(unsigned(Hq + 2 * Hkv), unsigned(T)), dim3(64), 0, as_stream(stream), qkv,
                     q_norm_w, k_norm_w, rope_cos, rope_sin, positions, int(T), int(S), int(Hq), int(Hkv),
                     int(S_max), max_p, eps, q_out, k_cache, v_cache);
  return hip_status("qmoe_qkv_finish");
}

namespace qmoe {
// Key splits of the prefill launch: the smallest kt_split (64-key tiles per
// workgroup, at least 2) whose split grid still fits one workgroup per CU,
// for grids below the CU count with a host-known start, when it takes at
// least AP_SPLIT_MIN_GAIN key steps off the longest tile (a split costs
// about three steps: the partial's store, the count and the merge); 0 (no
// split) otherwise.  *grid gets the launch's workgroup count.
constexpr int AP_SPLIT_MIN_GAIN = 4;
static int ap_kt_split(int64_t B, int64_t S, int64_t Hq, int64_t start, bool host_start, int64_t* grid) {
  const int64_t n_qt = (S + AP_QT - 1) / AP_QT, base = n_qt * Hq * B, cus = current_device_cus();
  *grid = base;
  if (!host_start || base >= cus) return 0;
  auto n_kt = [&](int64_t t) { return (start + std::min((t + 1) * AP_QT, S) + AP_KT - 1) / AP_KT; };
  for (int64_t spt = 2; spt <= n_kt(n_qt - 1) - AP_SPLIT_MIN_GAIN; ++spt) {
    int64_t total = 0;
    for (int64_t t = 0; t < n_qt; ++t) total += (n_kt(t) + spt - 1) / spt * Hq * B;
    if (total <= cus && (n_kt(n_qt - 1) + spt - 1) / spt <= AP_MAX_SPLITS) {
      *grid = total;
      return int(spt);
    }
  }
  return 0;
}

// Counter bytes at the head of the prefill workspace (256-byte aligned).
static int64_t ap_cnt_bytes(int64_t B, int64_t S, int64_t Hq) {
  return ((S + AP_QT - 1) / AP_QT * Hq * B * 4 + 255) / 256 * 256;
}

static int ap_launch(const char* fn, const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                     int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, int64_t start,
                     const int32_t* start_dev, float scale, void* ws, int64_t ws_bytes, qmoe_bf16* out,
                     qmoe_stream_t stream) {
  QMOE_REQUIRE(k_cache && v_cache && (B == 0 || S == 0 || (q && out)), "%s: null pointer", fn);
  QMOE_REQUIRE(D == HD, "%s: head_dim must be 128", fn);
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq < 65536, "%s: bad heads", fn);
  QMOE_REQUIRE(B >= 0 && B < 65536 && S >= 0 && S <= S_max && start >= 0 && start + S <= S_max,
               "%s: need 0 <= start and start + S <= S_max", fn);
  QMOE_REQUIRE(S_max <= AP_MAX_SMAX, "%s: S_max must be <= %d", fn, AP_MAX_SMAX);
  QMOE_REQUIRE(ws_bytes >= 0 && (ws != nullptr || ws_bytes == 0), "%s: bad workspace", fn);
  if (B == 0 || S == 0) return QMOE_OK;
  QMOE_REQUIRE((S + AP_QT - 1) / AP_QT * Hq * B < (1ll << 31), "%s: grid too large", fn);
  int64_t grid = 0;
  ApSplit sp{0, nullptr, nullptr};
  if (ws) {
    const int kt_split = ap_kt_split(B, S, Hq, start, start_dev == nullptr, &grid);
    const int64_t cb = ap_cnt_bytes(B, S, Hq);
    if (kt_split > 0 && ws_bytes >= cb + grid * AP_PREC * 4) {
      sp.kt_split = kt_split;
      sp.cnt = static_cast<int32_t*>(ws);
      sp.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + cb);
    }
  }
  if (sp.kt_split == 0) grid = (S + AP_QT - 1) / AP_QT * Hq * B;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(unsigned(grid)), dim3(256), 0, as_stream(stream), q, k_cache,
                     v_cache, int(B), int(S), int(Hq), int(Hkv), int(S_max), int(start), start_dev, scale_log2,
                     out, sp);
  return hip_status(fn);
}
}  // namespace qmoe

extern "C" int qmoe_attn_prefill(const qmoe_bf16* q, const qmoe_bf16* k_cache,
                                 const qmoe_bf16* v_cache, int64_t B, int64_t S, int64_t Hq,
                                 int64_t Hkv, int64_t D, int64_t S_max, int64_t start, float scale,
                                 qmoe_bf16* out, qmoe_stream_t stream) {
  return qmoe::ap_launch("qmoe_attn_prefill", q, k_cache, v_cache, B, S, Hq, Hkv, D, S_max, start, nullptr, scale,
                         nullptr, 0, out, stream);
}

extern "C" int64_t qmoe_attn_prefill_workspace(int64_t B, int64_t S, int64_t Hq, int64_t D) {
  if (B < 0 || S < 0 || Hq <= 0 || D != qmoe::HD) return -1;
  return qmoe::ap_cnt_bytes(B, S, Hq) + int64_t(qmoe::current_device_cus()) * qmoe::AP_PREC * 4;
}

extern "C" int qmoe_attn_prefill_ws(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                                    int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max,
                                    int64_t start, float scale, void* workspace, int64_t workspace_bytes,
                                    qmoe_bf16* out, qmoe_stream_t stream) {
  return qmoe::ap_launch("qmoe_attn_prefill_ws", q, k_cache, v_cache, B, S, Hq, Hkv, D, S_max, start, nullptr,
                         scale, workspace, workspace_bytes, out, stream);
}

extern "C" int qmoe_attn_prefill_at(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                                    int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max,
                                    const int32_t* start, float scale, qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(start || B == 0 || S == 0, "qmoe_attn_prefill_at: null pointer");
  return qmoe::ap_launch("qmoe_attn_prefill_at", q, k_cache, v_cache, B, S, Hq, Hkv, D, S_max, 0, start, scale,
                         nullptr, 0, out, stream);
}

extern "C" int64_t qmoe_attn_decode_workspace(int64_t B, int64_t Hq, int64_t D, int64_t S_max) {
  const int64_t nsplit = (S_max + AD_WKEYS - 1) / AD_WKEYS;  // the most partials: one wave per split
  return B * Hq * nsplit * (D + 4);
}

// Waves per split workgroup: four (one merged partial per 256 keys) when the
// step has many 64-key waves, i.e. the batch x kv heads and the cache
// capacity are both large, or when the cache alone holds 64 or more waves'
// keys (at batch 1 and context 8000 the merge of 129 one-wave partials per
// head costs more than the wider splits save: 20.7 -> 13.3 us a step; at
// context 800 one wave per split stays ahead, 8.8 against 10.2 us); one
// otherwise.  Chosen from the cache shape, not from max_ctx, so a
// bucket-sized launch and a full-capacity launch split the keys alike and
// give the same bits.
static int ad_subs(int64_t B, int64_t Hkv, int64_t S_max) {
  const int64_t waves = (S_max + AD_WKEYS - 1) / AD_WKEYS;
  return (waves >= 64 || (B * Hkv >= 16 && waves * B * Hkv >= 2048)) ? AD_MAX_SUBS : 1;
}

// B query rows; chunk_start / qpb as in ad_ctx (nullptr / 1: one query per batch row).
// fin.raw != nullptr: the fused decode (q == nullptr, ctx_len == fin.positions).
static int attn_decode_launch(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                              const int32_t* ctx_len, const int32_t* chunk_start, int64_t qpb, int64_t B,
                              int64_t Hq, int64_t Hkv, int64_t S_max, int64_t max_ctx, float scale,
                              float* partial, qmoe_bf16* out, hipStream_t s, const AdFinish& fin = AdFinish{}) {
  if (B == 0) return QMOE_OK;
  const int subs = ad_subs(chunk_start ? B / qpb : B, Hkv, S_max);
  const int split_keys = subs * AD_WKEYS;
  const int nsplit = int((max_ctx + split_keys - 1) / split_keys);
  const dim3 grid{unsigned(nsplit), unsigned(Hkv), unsigned(B)};
  const bool fused = fin.raw != nullptr;
#define QMOE_AD_SPLIT(SUBS, FUSED)                                                                                 \
  hipLaunchKernelGGL((attn_decode_split_kernel<SUBS, FUSED>), grid, dim3(SUBS * 64), 0, s, q, k_cache, v_cache,   \
                     ctx_len, chunk_start, int(qpb), int(Hq), int(Hkv), int(S_max), int(max_ctx), nsplit, scale, \
                     partial, fin)
  if (subs == 1) {
    if (fused)
      QMOE_AD_SPLIT(1, true);
    else
      QMOE_AD_SPLIT(1, false);
  } else {
    if (fused)
      QMOE_AD_SPLIT(AD_MAX_SUBS, true);
    else
      QMOE_AD_SPLIT(AD_MAX_SUBS, false);
  }
#undef QMOE_AD_SPLIT
  int rc = hip_status("qmoe_attn_decode(split)");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(unsigned(B * Hq)), dim3(HD), 0, s, partial, ctx_len,
                     chunk_start, int(qpb), int(S_max), int(Hq), int(max_ctx), nsplit, split_keys,
                     fused ? fin.max_pos : 0, out);
  return hip_status("qmoe_attn_decode(merge)");
}

extern "C" int qmoe_attn_decode(const qmoe_bf16* q, const qmoe_bf16* k_cache,
                                const qmoe_bf16* v_cache, const int32_t* ctx_len, int64_t B,
                                int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float scale,
                                float* partial, qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(k_cache && v_cache && (B == 0 || (q && ctx_len && partial && out)), "qmoe_attn_decode: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_decode: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= AD_MAX_G && Hkv < 65536,
               "qmoe_attn_decode: need Hq %% Hkv == 0 and Hq / Hkv <= 16");
  QMOE_REQUIRE(B >= 0 && B < 65536 && S_max > 0 && S_max < (1ll << 30), "qmoe_attn_decode: bad B/S_max");
  return attn_decode_launch(q, k_cache, v_cache, ctx_len, nullptr, 1, B, Hq, Hkv, S_max, S_max, scale, partial, out,
                            as_stream(stream));
}

extern "C" int qmoe_attn_decode_bucket(const qmoe_bf16* q, const qmoe_bf16* k_cache,
                                       const qmoe_bf16* v_cache, const int32_t* ctx_len, int64_t B,
                                       int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, int64_t max_ctx,
                                       float scale, float* partial, qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(k_cache && v_cache && (B == 0 || (q && ctx_len && partial && out)),
               "qmoe_attn_decode_bucket: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_decode_bucket: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= AD_MAX_G && Hkv < 65536,
               "qmoe_attn_decode_bucket: need Hq %% Hkv == 0 and Hq / Hkv <= 16");
  QMOE_REQUIRE(B >= 0 && B < 65536 && S_max > 0 && S_max < (1ll << 30), "qmoe_attn_decode_bucket: bad B/S_max");
  QMOE_REQUIRE(max_ctx > 0 && max_ctx <= S_max, "qmoe_attn_decode_bucket: need 0 < max_ctx <= S_max");
  return attn_decode_launch(q, k_cache, v_cache, ctx_len, nullptr, 1, B, Hq, Hkv, S_max, max_ctx, scale, partial, out,
                            as_stream(stream));
}

extern "C" int qmoe_attn_decode_fused(const float* qkv, const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                                      const float* rope_cos, const float* rope_sin, int64_t max_pos,
                                      const int32_t* positions, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t S_max, int64_t max_ctx, float eps, float scale, qmoe_bf16* k_cache,
                                      qmoe_bf16* v_cache, float* partial, qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(q_norm_w && k_norm_w && rope_cos && rope_sin && k_cache && v_cache &&
                   (B == 0 || (qkv && positions && partial && out)),
               "qmoe_attn_decode_fused: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_decode_fused: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= AD_MAX_G && Hkv < 65536 && Hq + 2 * Hkv < 65536,
               "qmoe_attn_decode_fused: need Hq %% Hkv == 0 and Hq / Hkv <= 16");
  QMOE_REQUIRE(B >= 0 && B < 65536 && S_max > 0 && S_max < (1ll << 30), "qmoe_attn_decode_fused: bad B/S_max");
  QMOE_REQUIRE(max_ctx > 0 && max_ctx <= S_max, "qmoe_attn_decode_fused: need 0 < max_ctx <= S_max");
  QMOE_REQUIRE(max_pos > 0, "qmoe_attn_decode_fused: bad max_pos");
  AdFinish fin{qkv, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, int(std::min<int64_t>(max_pos, 1ll << 30)),
               eps, k_cache, v_cache};
  return attn_decode_launch(nullptr, k_cache, v_cache, positions, nullptr, 1, B, Hq, Hkv, S_max, max_ctx, scale,
                            partial, out, as_stream(stream), fin);
}

extern "C" int qmoe_attn_decode_chunk(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                                      const int32_t* start, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                                      int64_t D, int64_t S_max, float scale, float* partial, qmoe_bf16* out,
                                      qmoe_stream_t stream) {
  QMOE_REQUIRE(k_cache && v_cache && (B == 0 || (q && start && partial && out)), "qmoe_attn_decode_chunk: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_decode_chunk: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= AD_MAX_G && Hkv < 65536,
               "qmoe_attn_decode_chunk: need Hq %% Hkv == 0 and Hq / Hkv <= 16");
  QMOE_REQUIRE(B >= 0 && S > 0 && B * S < 65536 && S_max >= S && S_max < (1ll << 30),
               "qmoe_attn_decode_chunk: bad B/S/S_max");
  return attn_decode_launch(q, k_cache, v_cache, nullptr, start, S, B * S, Hq, Hkv, S_max, S_max, scale, partial,
                            out, as_stream(stream));
}
