// The whole MoE block at decode shape (T <= 8 tokens) in three launches:
//
//   block_logits_kernel     [optional post-attention RMSNorm] + router logits:
//                           E single-wave workgroups, one router row each (in
//                           registers); every wave normalises the few token
//                           rows itself, workgroup 0 also stores them.  No
//                           workgroup waits on another: cross-workgroup
//                           counters serialise at about 20 ns per workgroup
//                           on one address, which is what this avoids.
//   block_gateup_kernel     every workgroup first runs softmax/top-k per token
//                           on the T*E logits (exact DPP selection, the same
//                           answer everywhere; workgroup (0,0) publishes it).
//                           The workgroup's active-expert index then selects
//                           its expert from the set of chosen experts (a
//                           bitmask built from the few top-k ids) and its token
//                           rows are the (t, j) pairs routed there, so no
//                           permutation pass is needed.  Gate/up rows are
//                           streamed once into registers; SwiGLU in fp32:
//                           act[t*k+j, i].
//   block_down_combine_kernel  one workgroup per 8 output columns h (one per
//                           wave; 8 waves keep enough loads in flight per CU)
//                           over all (t, j) pairs: out[t,h] = residual +
//                           sum_j w[t,j] * act[t*k+j] . W2[e(t,j), h], summed in
//                           fixed j order (deterministic; no atomics).
//
// HBM traffic is the touched experts' weights (U * 3 * H * I * 2 bytes) plus
// the router (E * H * 2); everything else is a few KB.
#include "decode_util.hpp"
#include "topk_impl.hpp"

namespace qmoe {

constexpr int BLK_MAX_T = 8;
constexpr int BLK_MAX_PAIRS = 64;         // T * k
constexpr int BLK_DOWN_ROWS = 8;          // output columns per down workgroup (1 per wave)
constexpr int BLK_PAIR_GROUP = 8;         // (t, j) pairs whose W2 rows are loaded together
constexpr int BLK_ACT_LDS_FLOATS = 8192;  // act staged in LDS when T*k*I fits (32 KB)

// ------------------------------------------------------------------ router logits
// One wave per router row e.  Each lane owns H/64 positions of the token row
// (HC chunks of 8 at c*512 + 8*lane), so the optional RMSNorm is a wave
// reduction over registers: no LDS, no barrier, no cross-workgroup traffic.
// Workgroup 0 also stores the normalised bf16 rows for the gate/up kernel.
template <int HC>
__global__ __launch_bounds__(64) void block_logits_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ h, const uint16_t* __restrict__ rms_w,
    float eps, const uint16_t* __restrict__ w_router, const float* __restrict__ bias, int T, int H,
    int E, float* __restrict__ logits, uint16_t* __restrict__ x_out) {
  const int lane = threadIdx.x, e = blockIdx.x;
  u32x4 wr[HC];
#pragma unroll
  for (int c = 0; c < HC; ++c) wr[c] = ld_stream(w_router + int64_t(e) * H + c * 512 + lane * 8);
  const float b = bias ? bias[e] : 0.0f;
  for (int r = 0; r < T; ++r) {
    float xf[HC][8];
    if (h) {
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        const float4* hp = reinterpret_cast<const float4*>(h + int64_t(r) * H + c * 512 + lane * 8);
        const float4 v0 = hp[0], v1 = hp[1];
        xf[c][0] = v0.x; xf[c][1] = v0.y; xf[c][2] = v0.z; xf[c][3] = v0.w;
        xf[c][4] = v1.x; xf[c][5] = v1.y; xf[c][6] = v1.z; xf[c][7] = v1.w;
#pragma unroll
        for (int q = 0; q < 8; ++q) ss += xf[c][q] * xf[c][q];
      }
      const float rr = rsqrtf(wave_sum(ss) / float(H) + eps);
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        float wf[8];
        unpack8(*reinterpret_cast<const u32x4*>(rms_w + c * 512 + lane * 8), wf);
        u32x4 o;
        o.x = pack_bf16x2(wf[0] * (xf[c][0] * rr), wf[1] * (xf[c][1] * rr));
        o.y = pack_bf16x2(wf[2] * (xf[c][2] * rr), wf[3] * (xf[c][3] * rr));
        o.z = pack_bf16x2(wf[4] * (xf[c][4] * rr), wf[5] * (xf[c][5] * rr));
        o.w = pack_bf16x2(wf[6] * (xf[c][6] * rr), wf[7] * (xf[c][7] * rr));
        unpack8(o, xf[c]);  // the router sees the bf16 normed row, as the experts do
        if (e == 0) *reinterpret_cast<u32x4*>(x_out + int64_t(r) * H + c * 512 + lane * 8) = o;
      }
    } else {
#pragma unroll
      for (int c = 0; c < HC; ++c)
        unpack8(ld16(x + int64_t(r) * H + c * 512 + lane * 8), xf[c]);
    }
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      opaque(wr[c]);
      acc += dot8(wr[c], xf[c]);
    }
    acc = wave_sum(acc);
    if (lane == 0) logits[int64_t(r) * E + e] = acc + b;
  }
}

// ------------------------------------------------------------------ gate/up
template <int HC>
__global__ __launch_bounds__(256) void block_gateup_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ logits, int E,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    const uint16_t* __restrict__ w13, int T, int H, int I, int k, float* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [min(T*k,16)][H]
  __shared__ float s_log[BLK_MAX_T * ROUTER_MAX_E];
  __shared__ int32_t s_idx[BLK_MAX_PAIRS];
  __shared__ float s_w[BLK_MAX_PAIRS];
  __shared__ uint32_t s_mask[ROUTER_MAX_E / 32];
  __shared__ int32_t s_list[BLK_MAX_PAIRS];
  __shared__ int s_e, s_n;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int npairs = T * k;
  // every workgroup selects the experts itself from the T*E logits (same
  // inputs, same deterministic selection), so no workgroup waits on another
  for (int q = t; q < T * E; q += 256) s_log[q] = logits[q];
  if (t < ROUTER_MAX_E / 32) s_mask[t] = 0u;
  __syncthreads();
  for (int tok = wave; tok < T; tok += 4)
    topk_softmax_wave(s_log + tok * E, E, k, s_idx + tok * k, s_w + tok * k);
  __syncthreads();
  if (t < npairs) {
    const int ee = s_idx[t];
    atomicOr(&s_mask[ee >> 5], 1u << (ee & 31));
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      topk_idx[t] = ee;
      topk_w[t] = s_w[t];
    }
  }
  __syncthreads();
  if (t == 0) {
    int a = blockIdx.x, ex = -1;
    for (int wd = 0; wd < ROUTER_MAX_E / 32 && ex < 0; ++wd) {
      uint32_t m = s_mask[wd];
      const int c = __popc(m);
      if (a < c) {
        for (int q = 0; q < a; ++q) m &= m - 1;  // drop the a lowest set bits
        ex = wd * 32 + __ffs(m) - 1;
      } else {
        a -= c;
      }
    }
    s_e = ex;
  }
  __syncthreads();
  const int e = s_e;
  if (e < 0) return;
  const int i_base = blockIdx.y * 8 + wave * 2;
  const int grp = i_base / 32, off = i_base % 32;
  const uint16_t* we = w13 + int64_t(e) * 2 * I * H;
  u32x4 w[4][HC];  // gate i_base, gate i_base+1, up i_base, up i_base+1
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int prow = grp * 64 + (r < 2 ? 0 : 32) + off + (r & 1);
    const uint16_t* p = we + int64_t(prow) * H + lane * 8;
#pragma unroll
    for (int c = 0; c < HC; ++c) w[r][c] = ld_stream(p + c * 512);
  }
  if (wave == 0) {
    const bool hit = lane < npairs && s_idx[lane] == e;
    const unsigned long long m = __ballot(hit);
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (hit) s_list[__popcll(m & lt)] = lane;
    if (lane == 0) s_n = __popcll(m);
  }
  __syncthreads();
  const int n_all = s_n;
  for (int c0 = 0; c0 < n_all; c0 += DEC_TOK_CHUNK) {
    const int n = min(DEC_TOK_CHUNK, n_all - c0);
    if (c0 > 0) __syncthreads();
    const int hch = H / 8;
    for (int q = t; q < n * hch; q += 256) {
      const int j = q / hch, kc = q - j * hch;
      const int64_t row = s_list[c0 + j] / k;
      *reinterpret_cast<u32x4*>(xs + j * H + kc * 8) = ld16(x + row * H + kc * 8);
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        float xf[8];
        unpack8(*reinterpret_cast<const u32x4*>(xs + j * H + c * 512 + lane * 8), xf);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          opaque(w[r][c]);
          acc[r] += dot8(w[r][c], xf);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = wave_sum(acc[r]);
      if (lane < 2) {
        const float g = lane ? acc[1] : acc[0];
        const float u = lane ? acc[3] : acc[2];
        act[int64_t(s_list[c0 + j]) * I + i_base + lane] = silu(g) * u;
      }
    }
  }
}

// ------------------------------------------------------------------ down + combine
template <int IC>
__global__ __launch_bounds__(64 * BLK_DOWN_ROWS) void block_down_combine_kernel(
    const float* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_w,
    const float* residual, int T, int H, int I, int k, float* out) {
  __shared__ int32_t s_idx[BLK_MAX_PAIRS];
  __shared__ float s_w[BLK_MAX_PAIRS];
  __shared__ __attribute__((aligned(16))) float s_act[BLK_ACT_LDS_FLOATS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int npairs = T * k;
  const int hrow = blockIdx.x * BLK_DOWN_ROWS + wave;
  const int ichunks = I / 8;
  // first group's W2 rows go out before anything else (expert ids read directly)
  u32x4 w[BLK_PAIR_GROUP][IC];
  auto load_group = [&](int p0) {
#pragma unroll
    for (int g = 0; g < BLK_PAIR_GROUP; ++g) {
      const int p = p0 + g;
      const int e = p < npairs ? topk_idx[p] : 0;
      const uint16_t* rowp = w2 + (int64_t(e) * H + hrow) * I;
#pragma unroll
      for (int c = 0; c < IC; ++c) {
        const int ch = lane + 64 * c;
        w[g][c] = (p < npairs && ch < ichunks) ? ld_stream(rowp + ch * 8) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  load_group(0);
  if (t < npairs) {
    s_idx[t] = topk_idx[t];
    s_w[t] = topk_w[t];
  }
  const bool act_lds = npairs * I <= BLK_ACT_LDS_FLOATS;
  if (act_lds) {
    for (int q = t; q < npairs * I / 4; q += 64 * BLK_DOWN_ROWS)
      reinterpret_cast<float4*>(s_act)[q] = reinterpret_cast<const float4*>(act)[q];
  }
  __syncthreads();
  float run = 0.0f;  // running weighted sum of the current token (wave-uniform)
  for (int p0 = 0; p0 < npairs; p0 += BLK_PAIR_GROUP) {
    if (p0 > 0) load_group(p0);
#pragma unroll
    for (int g = 0; g < BLK_PAIR_GROUP; ++g) {
      const int p = p0 + g;
      if (p < npairs) {
        const float* ap = act_lds ? s_act + p * I : act + int64_t(p) * I;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < IC; ++c) {
          const int ch = lane + 64 * c;
          if (ch < ichunks) {
            const float4 a0 = reinterpret_cast<const float4*>(ap + ch * 8)[0];
            const float4 a1 = reinterpret_cast<const float4*>(ap + ch * 8)[1];
            const float x8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            acc += dot8(w[g][c], x8);
          }
        }
        acc = wave_sum(acc);
        const int j = p % k;
        run = (j == 0) ? s_w[p] * acc : fmaf(s_w[p], acc, run);
        if (j == k - 1 && lane == 0) {
          const int64_t o = int64_t(p / k) * H + hrow;
          out[o] = (residual ? residual[o] : 0.0f) + run;
        }
      }
    }
  }
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_moe_decode_block(const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w,
                                     float eps, const qmoe_bf16* w_router, const float* bias,
                                     const qmoe_bf16* w13, const qmoe_bf16* w2,
                                     const float* residual, int64_t T, int64_t H, int64_t I,
                                     int64_t E, int64_t k, float* logits, int32_t* topk_idx,
                                     float* topk_w, float* act, int32_t* sync, qmoe_bf16* x_out,
                                     float* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(w_router && w13 && w2 && logits && topk_idx && topk_w && act && out,
               "qmoe_moe_decode_block: null pointer");
  (void)sync;  // reserved: the launches no longer synchronise through memory
  QMOE_REQUIRE((x != nullptr) != (h != nullptr), "qmoe_moe_decode_block: pass exactly one of x and h");
  QMOE_REQUIRE(!h || (rms_w && x_out), "qmoe_moe_decode_block: h needs rms_w and x_out");
  QMOE_REQUIRE(T >= 0 && T <= BLK_MAX_T, "qmoe_moe_decode_block: T must be <= 8 (T=%lld)", (long long)T);
  QMOE_REQUIRE(E > 0 && E <= ROUTER_MAX_E && k > 0 && k <= ROUTER_MAX_K && k <= E && T * k <= BLK_MAX_PAIRS,
               "qmoe_moe_decode_block: need E <= 256, k <= min(16, E), T*k <= 64");
  QMOE_REQUIRE(H >= 512 && H <= 4096 && H % 512 == 0 && (H / 512 & (H / 512 - 1)) == 0,
               "qmoe_moe_decode_block: H must be 512, 1024, 2048 or 4096");
  QMOE_REQUIRE(I % 32 == 0 && I > 0 && I <= 1536, "qmoe_moe_decode_block: I must be a multiple of 32, <= 1536");
  QMOE_REQUIRE(eps >= 0.0f, "qmoe_moe_decode_block: eps < 0");
  if (T == 0) return QMOE_OK;
  hipStream_t s = as_stream(stream);
  const uint16_t* xin = h ? x_out : x;
  const size_t shm1 = size_t(std::min<int64_t>(T * k, DEC_TOK_CHUNK)) * H * 2;
  dim3 g1(unsigned(std::min<int64_t>(E, T * k)), unsigned(I / 8));
  switch (H / 512) {
#define QMOE_BLK(HC)                                                                              \
  case HC:                                                                                        \
    hipLaunchKernelGGL(block_logits_kernel<HC>, dim3(unsigned(E)), dim3(64), 0, s, x, h, rms_w,    \
                       eps, w_router, bias, int(T), int(H), int(E), logits, x_out);               \
    if (int rc = hip_status("qmoe_moe_decode_block(router)")) return rc;                          \
    hipLaunchKernelGGL(block_gateup_kernel<HC>, g1, dim3(256), shm1, s, xin, logits, int(E),      \
                       topk_idx, topk_w, w13, int(T), int(H), int(I), int(k), act);               \
    break;
    QMOE_BLK(1)
    QMOE_BLK(2)
    QMOE_BLK(4)
    QMOE_BLK(8)
#undef QMOE_BLK
  }
  if (int rc = hip_status("qmoe_moe_decode_block(gate_up)")) return rc;
  dim3 g2(unsigned(H / BLK_DOWN_ROWS));
  switch (int((I / 8 + 63) / 64)) {
#define QMOE_DC(IC)                                                                               \
  case IC:                                                                                        \
    hipLaunchKernelGGL(block_down_combine_kernel<IC>, g2, dim3(64 * BLK_DOWN_ROWS), 0, s, act, w2, \
                       topk_idx, topk_w, residual, int(T), int(H), int(I), int(k), out);          \
    break;
    QMOE_DC(1)
    QMOE_DC(2)
    QMOE_DC(3)
#undef QMOE_DC
  }
  return hip_status("qmoe_moe_decode_block(down)");
}
