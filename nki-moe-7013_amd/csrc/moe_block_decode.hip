// The whole MoE block at decode shape (T <= 8 tokens) in three launches:
//
//   block_router_kernel     [optional post-attention RMSNorm] + router logits:
//                           ceil(E/4) workgroups, one wave per router row (kept
//                           in registers); every workgroup normalises the few
//                           token rows itself, workgroup 0 also stores them.
//                           The last workgroup to arrive (device-scope counter,
//                           re-armed by that workgroup) runs softmax/top-k per
//                           token.  Only ceil(E/4) = 32 workgroups fence, which
//                           keeps the serialised fence cost to about 2 us.
//   block_gateup_kernel     the workgroup's active-expert index selects its
//                           expert from the set of chosen experts (a bitmask
//                           built from the few top-k ids) and its token rows are
//                           the (t, j) pairs routed there, so no permutation
//                           pass is needed.  Gate/up rows are streamed once into
//                           registers; SwiGLU in fp32: act[t*k+j, i].
//   block_down_combine_kernel  one workgroup per 4 output columns h (one per
//                           wave) over all (t, j) pairs: out[t,h] = residual +
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
constexpr int BLK_DOWN_ROWS = 4;          // output columns per down workgroup (1 per wave)
constexpr int BLK_PAIR_GROUP = 8;         // (t, j) pairs whose W2 rows are loaded together
constexpr int BLK_ACT_LDS_FLOATS = 8192;  // act staged in LDS when T*k*I fits (32 KB)

// ------------------------------------------------------------------ router + top-k
template <int HC>
__global__ __launch_bounds__(256) void block_router_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ h, const uint16_t* __restrict__ rms_w,
    float eps, const uint16_t* __restrict__ w_router, const float* __restrict__ bias, int T, int H,
    int E, int k, float* logits, uint16_t* __restrict__ x_out, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, int32_t* sync) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [T][H]
  __shared__ float red[BLK_MAX_T][4];
  __shared__ int s_last;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int e = blockIdx.x * 4 + wave;
  u32x4 wr[HC];
  if (e < E) {
#pragma unroll
    for (int c = 0; c < HC; ++c) wr[c] = ld16(w_router + int64_t(e) * H + c * 512 + lane * 8);
  }
  if (h) {
    // fused RMSNorm: pass 1 sums of squares, pass 2 normalise (rows are L2-hot)
#pragma unroll
    for (int r = 0; r < BLK_MAX_T; ++r) {
      if (r < T) {
        float ss = 0.0f;
        for (int c = t; c < H / 4; c += 256) {
          const float4 v = reinterpret_cast<const float4*>(h + int64_t(r) * H)[c];
          ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[r][wave] = ss;
      }
    }
    __syncthreads();
    for (int r = 0; r < T; ++r) {
      const float rr = rsqrtf((red[r][0] + red[r][1] + red[r][2] + red[r][3]) / float(H) + eps);
      for (int c = t; c < H / 4; c += 256) {
        const float4 v = reinterpret_cast<const float4*>(h + int64_t(r) * H)[c];
        const uint2 wv = reinterpret_cast<const uint2*>(rms_w)[c];
        uint2 o;
        o.x = pack_bf16x2(bf16_lo(wv.x) * (v.x * rr), bf16_hi(wv.x) * (v.y * rr));
        o.y = pack_bf16x2(bf16_lo(wv.y) * (v.z * rr), bf16_hi(wv.y) * (v.w * rr));
        reinterpret_cast<uint2*>(xs + r * H)[c] = o;
        if (blockIdx.x == 0) reinterpret_cast<uint2*>(x_out + int64_t(r) * H)[c] = o;
      }
    }
  } else {
    stage_rows_bf16(xs, x, nullptr, 0, T, H);
  }
  __syncthreads();
  if (e < E) {
    const float b = bias ? bias[e] : 0.0f;
    for (int r = 0; r < T; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        opaque(wr[c]);
        float xf[8];
        unpack8(*reinterpret_cast<const u32x4*>(xs + r * H + c * 512 + lane * 8), xf);
        acc += dot8(wr[c], xf);
      }
      acc = wave_sum(acc);
      if (lane == 0) logits[int64_t(r) * E + e] = acc + b;
    }
  }
  // the last workgroup to arrive selects the experts
  __threadfence();
  __syncthreads();
  if (t == 0) s_last = (atomicAdd(sync, 1) == int(gridDim.x) - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  // stage each token's logits in LDS with vector loads, then rank them there
  float* s_log = reinterpret_cast<float*>(xs);  // T*E floats <= 8 KB, fits in the x staging area
  for (int q = t; q < T * E; q += 256) s_log[q] = logits[q];
  __syncthreads();
  for (int tok = wave; tok < T; tok += 4)
    topk_softmax_wave(s_log + tok * E, E, k, topk_idx + tok * k, topk_w + tok * k);
  if (t == 0) *sync = 0;  // every workgroup has arrived: re-arm
}

// ------------------------------------------------------------------ gate/up
template <int HC>
__global__ __launch_bounds__(256) void block_gateup_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ topk_idx,
    const uint16_t* __restrict__ w13, int T, int H, int I, int k, float* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [min(T*k,16)][H]
  __shared__ int32_t s_idx[BLK_MAX_PAIRS];
  __shared__ uint32_t s_mask[ROUTER_MAX_E / 32];
  __shared__ int32_t s_list[BLK_MAX_PAIRS];
  __shared__ int s_e, s_n;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int npairs = T * k;
  if (t < ROUTER_MAX_E / 32) s_mask[t] = 0u;
  __syncthreads();
  if (t < npairs) {
    const int ee = topk_idx[t];
    s_idx[t] = ee;
    atomicOr(&s_mask[ee >> 5], 1u << (ee & 31));
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
__global__ __launch_bounds__(256) void block_down_combine_kernel(
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
    for (int q = t; q < npairs * I / 4; q += 256)
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
  QMOE_REQUIRE(w_router && w13 && w2 && logits && topk_idx && topk_w && act && sync && out,
               "qmoe_moe_decode_block: null pointer");
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
  const size_t shm0 = std::max<size_t>(size_t(T) * H * 2, size_t(T) * E * 4);
  dim3 g0(unsigned((E + 3) / 4));
  const size_t shm1 = size_t(std::min<int64_t>(T * k, DEC_TOK_CHUNK)) * H * 2;
  dim3 g1(unsigned(std::min<int64_t>(E, T * k)), unsigned(I / 8));
  switch (H / 512) {
#define QMOE_BLK(HC)                                                                              \
  case HC:                                                                                        \
    hipLaunchKernelGGL(block_router_kernel<HC>, g0, dim3(256), shm0, s, x, h, rms_w, eps,         \
                       w_router, bias, int(T), int(H), int(E), int(k), logits, x_out, topk_idx,   \
                       topk_w, sync);                                                             \
    if (int rc = hip_status("qmoe_moe_decode_block(router)")) return rc;                          \
    hipLaunchKernelGGL(block_gateup_kernel<HC>, g1, dim3(256), shm1, s, xin, topk_idx, w13,       \
                       int(T), int(H), int(I), int(k), act);                                      \
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
    hipLaunchKernelGGL(block_down_combine_kernel<IC>, g2, dim3(256), 0, s, act, w2, topk_idx,      \
                       topk_w, residual, int(T), int(H), int(I), int(k), out);                    \
    break;
    QMOE_DC(1)
    QMOE_DC(2)
    QMOE_DC(3)
#undef QMOE_DC
  }
  return hip_status("qmoe_moe_decode_block(down)");
}
