// The whole MoE block at decode shape (T <= 8 tokens) in three launches:
//
//   block_logits_kernel     [optional post-attention RMSNorm] + router logits:
//                           E workgroups of T waves, one router row each (in
//                           registers); wave r normalises token row r itself,
//                           workgroup 0 also stores the rows.  No
//                           workgroup waits on another: cross-workgroup
//                           counters serialise at about 20 ns per workgroup
//                           on one address, which is what this avoids.
//   block_expert_kernel     BLK_WGS workgroups.  Each first runs softmax/top-k
//                           per token on the T*E logits (exact DPP selection,
//                           the same answer everywhere; workgroup 0 publishes
//                           it) and lists the touched experts in ascending id.
//                           The work items are (touched expert u, slice s of
//                           BLK_SLICE intermediate units); workgroup g takes
//                           items g, g + BLK_WGS, ...  An item streams the
//                           slice's gate and up rows (2 * 8 rows of H) and the
//                           expert's down block w2[e][s] (H x 8, contiguous in
//                           the blocked layout) once, computes the 8 SwiGLU
//                           outputs per routed token (times the routing
//                           weight), and adds their down product to the
//                           workgroup's running partial output in registers.
//                           The next item's weights are in flight while the
//                           current one is computed.  No workgroup waits on
//                           another: the gate/up -> down dependency stays
//                           inside the item.
//   block_reduce_kernel     out[t,h] = residual[t,h] + sum_g partial[g][t][h],
//                           g in a fixed order (deterministic; no atomics).
//
// HBM traffic is the touched experts' weights (U * 3 * H * I * 2 bytes) plus
// the router (E * H * 2); the partials are BLK_WGS * T * H * 4 bytes (2 MB at
// T = 1), written once and read once.
#include <atomic>
#include <mutex>

#include "decode_util.hpp"
#include "topk_impl.hpp"

namespace qmoe {

constexpr int BLK_MAX_T = 8;
constexpr int BLK_MAX_PAIRS = 64;  // T * k
constexpr int BLK_SLICE = QMOE_W2_BLOCK;  // intermediate units per work item
constexpr int BLK_WGS = QMOE_DECODE_BLOCK_WGS;
constexpr int BLK_RED_WAVES = 8;

static_assert(BLK_SLICE == 8, "an item is 4 waves x 2 units");

// ------------------------------------------------------------------ router logits
// One workgroup per router row e, one wave per token row (T <= 8 waves: the
// rows' loads and reductions run side by side, not one after another).  Each
// lane owns H/64 positions of the token row (HC chunks of 8 at c*512 + 8*lane),
// so the optional RMSNorm is a wave reduction over registers: no LDS, no
// barrier, no cross-workgroup traffic.  Every wave loads the router row; the
// concurrent misses on one line merge in L2, so HBM still sees it once.
// Workgroup 0 also stores the normalised bf16 rows for the expert kernel.
template <int HC>
__global__ __launch_bounds__(64 * BLK_MAX_T) void block_logits_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ h, const uint16_t* __restrict__ rms_w,
    float eps, const uint16_t* __restrict__ w_router, const float* __restrict__ bias, int T, int H,
    int E, float* __restrict__ logits, uint16_t* __restrict__ x_out) {
  const int lane = threadIdx.x & 63, e = blockIdx.x;
  u32x4 wr[HC], wn[HC];
#pragma unroll
  for (int c = 0; c < HC; ++c) wr[c] = ld_stream(w_router + int64_t(e) * H + c * 512 + lane * 8);
#pragma unroll
  for (int c = 0; c < HC; ++c)  // the norm weights go out with the router row
    wn[c] = h ? ld16(rms_w + c * 512 + lane * 8) : u32x4{0u, 0u, 0u, 0u};
  const float b = bias ? bias[e] : 0.0f;
  for (int r = threadIdx.x >> 6; r < T; r += blockDim.x >> 6) {
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
        unpack8(wn[c], wf);
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

// ------------------------------------------------------------------ experts
// Weights of one work item held by one thread: gate rows i, i+1 and up rows
// i, i+1 (i = s*8 + 2*wave) as HC 16-byte chunks each (lane*8 + c*512), and
// DQ = H/256 down rows h = tid + 256*q, 8 bf16 (the slice) each.
template <int HC>
struct ItemRegs {
  u32x4 g[4][HC];
  u32x4 d[2 * HC];
};

// GR item groups of 4 waves per workgroup; group r of workgroup g takes
// items g*GR + r, then + gridDim.x*GR, ...  PF: the next item's loads are
// issued before the current item is computed (two register sets).
template <int HC, int MT, int GR, bool PF>
__global__ __launch_bounds__(256 * GR) void block_expert_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ logits, int E, int k,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w, const uint16_t* __restrict__ w13,
    const uint16_t* __restrict__ w2b, int T, int H, int I, float* __restrict__ partial) {
  constexpr int DQ = 2 * HC;  // H / 256
  constexpr int NT = 256 * GR;
  // dynamic LDS: x rows [T][H] bf16, then (GR > 1) the group-combine buffer [T][H] f32
  extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];
  __shared__ float s_log[BLK_MAX_T * ROUTER_MAX_E];
  __shared__ int32_t s_idx[BLK_MAX_PAIRS];
  __shared__ float s_w[BLK_MAX_PAIRS];
  __shared__ float s_wt[ROUTER_MAX_E][BLK_MAX_T];  // routing weight of (e, t) where routed
  __shared__ uint32_t s_tm[ROUTER_MAX_E];          // bit t: token t is routed to expert e
  __shared__ int32_t s_uexp[ROUTER_MAX_E];         // touched experts, ascending
  __shared__ int s_wcnt[4];
  __shared__ __attribute__((aligned(16))) float s_act[GR][2][MT][BLK_SLICE];
  const int tid = threadIdx.x, grp = tid >> 8, gt = tid & 255, lane = tid & 63, wave = gt >> 6;
  float* s_red = reinterpret_cast<float*>(s_x + T * H);

  // logits and x rows: every load issued before the first LDS store
  float lg[(BLK_MAX_T * ROUTER_MAX_E + NT - 1) / NT];
#pragma unroll
  for (int i = 0; i < (BLK_MAX_T * ROUTER_MAX_E + NT - 1) / NT; ++i) {
    const int q = tid + NT * i;
    lg[i] = q < T * E ? logits[q] : 0.0f;
  }
  stage16<NT, (BLK_MAX_T * 4096 / 8 + NT - 1) / NT>(reinterpret_cast<u32x4*>(s_x), T * H / 8,
                                                    [&](int q) { return x + int64_t(q) * 8; });
#pragma unroll
  for (int i = 0; i < (BLK_MAX_T * ROUTER_MAX_E + NT - 1) / NT; ++i) {
    const int q = tid + NT * i;
    if (q < T * E) s_log[q] = lg[i];
  }
  for (int q = tid; q < E; q += NT) s_tm[q] = 0u;
  __syncthreads();
  for (int t = tid >> 6; t < T; t += NT / 64)
    topk_softmax_wave(s_log + t * E, E, k, s_idx + t * k, s_w + t * k);
  __syncthreads();
  if (tid < T * k) {
    const int e = s_idx[tid], t = tid / k;
    atomicOr(&s_tm[e], 1u << t);
    s_wt[e][t] = s_w[tid];
    if (blockIdx.x == 0) {
      topk_idx[tid] = e;
      topk_w[tid] = s_w[tid];
    }
  }
  __syncthreads();
  // compact the touched experts in ascending id (E <= 256: waves 0-3, one
  // thread per expert id)
  const bool used = tid < E && s_tm[tid] != 0u;
  const unsigned long long used_m = __ballot(used);
  if (tid < 256 && lane == 0) s_wcnt[wave] = __popcll(used_m);
  __syncthreads();
  if (used) {
    int base = 0;
    for (int w = 0; w < wave; ++w) base += s_wcnt[w];
    s_uexp[base + __popcll(used_m & ((1ull << lane) - 1ull))] = tid;
  }
  __syncthreads();
  const int U = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
  const int NS = I / BLK_SLICE;
  const int n_items = U * NS;
  const int stride = int(gridDim.x) * GR;

  float part[MT][DQ];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int q = 0; q < DQ; ++q) part[t][q] = 0.0f;

  auto load = [&](int it, ItemRegs<HC>& r) {
    const int u = it / NS, s = it - u * NS;
    const int e = s_uexp[u];
    const int i0 = s * BLK_SLICE + 2 * wave;  // this wave's two units (same 32-group)
    const uint16_t* we = w13 + int64_t(e) * 2 * I * H;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int prow = (i0 / QMOE_W13_GROUP) * 2 * QMOE_W13_GROUP + (q < 2 ? 0 : QMOE_W13_GROUP) +
                       (i0 % QMOE_W13_GROUP) + (q & 1);
      const uint16_t* p = we + int64_t(prow) * H + lane * 8;
#pragma unroll
      for (int c = 0; c < HC; ++c) r.g[q][c] = ld_stream(p + c * 512);
    }
    const uint16_t* wd = w2b + (int64_t(e) * NS + s) * H * BLK_SLICE + gt * BLK_SLICE;
#pragma unroll
    for (int q = 0; q < DQ; ++q) r.d[q] = ld_stream(wd + q * 256 * BLK_SLICE);
  };

  // One named barrier per group would be ideal; the whole workgroup's
  // barrier is used instead, so every group runs the same number of
  // compute steps (n_steps below) and idle groups still reach it.
  auto compute = [&](int it, ItemRegs<HC>& r, int buf, bool live) {
    const int e = live ? s_uexp[it / NS] : 0;
    const uint32_t tm = live ? s_tm[e] : 0u;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < T && ((tm >> t) & 1u)) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < HC; ++c) {
          float xf[8];
          unpack8(*reinterpret_cast<const u32x4*>(s_x + t * H + c * 512 + lane * 8), xf);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            opaque(r.g[q][c]);
            acc[q] += dot8(r.g[q][c], xf);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = wave_sum(acc[q]);
        if (lane == 0) {
          const float wt = s_wt[e][t];
          s_act[grp][buf][t][2 * wave] = silu(acc[0]) * acc[2] * wt;
          s_act[grp][buf][t][2 * wave + 1] = silu(acc[1]) * acc[3] * wt;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < T && ((tm >> t) & 1u)) {
        const float4 a0 = *reinterpret_cast<const float4*>(&s_act[grp][buf][t][0]);
        const float4 a1 = *reinterpret_cast<const float4*>(&s_act[grp][buf][t][4]);
        const float a8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int q = 0; q < DQ; ++q) {
          opaque(r.d[q]);
          part[t][q] += dot8(r.d[q], a8);
        }
      }
    }
    // Every register of the item counts as consumed here, on every path:
    // otherwise the refill two items later waits (WAW) on loads issued after
    // these, which serialises the stream.
    if (live) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int c = 0; c < HC; ++c) opaque(r.g[q][c]);
#pragma unroll
      for (int q = 0; q < DQ; ++q) opaque(r.d[q]);
    }
  };

  // items of this group: first, first + stride, ...; all groups loop n_steps
  // times (the most any group has) so the workgroup barriers match up.
  const int first = int(blockIdx.x) * GR + grp;
  const int first0 = int(blockIdx.x) * GR;  // group 0 has the most items
  const int n_steps = first0 < n_items ? (n_items - first0 + stride - 1) / stride : 0;
  ItemRegs<HC> ra;
  if constexpr (PF) {
    ItemRegs<HC> rb;
    int it = first;
    if (it < n_items) load(it, ra);
    for (int st = 0; st < n_steps; st += 2) {
      const int it2 = it + stride;
      if (it2 < n_items) load(it2, rb);
      compute(it, ra, 0, it < n_items);
      if (st + 1 >= n_steps) break;
      const int it3 = it2 + stride;
      if (it3 < n_items) load(it3, ra);
      compute(it2, rb, 1, it2 < n_items);
      it = it3;
    }
  } else {
    int it = first;
    for (int st = 0; st < n_steps; ++st, it += stride) {
      if (it < n_items) load(it, ra);
      compute(it, ra, st & 1, it < n_items);
    }
  }

  // combine the groups in a fixed order (group 0 + 1 + 2 ...), then store
  if constexpr (GR > 1) {
    for (int r = 1; r < GR; ++r) {
      if (grp == r) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
          if (t < T)
#pragma unroll
            for (int q = 0; q < DQ; ++q) s_red[t * H + q * 256 + gt] = part[t][q];
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
          if (t < T)
#pragma unroll
            for (int q = 0; q < DQ; ++q) part[t][q] += s_red[t * H + q * 256 + gt];
      }
      __syncthreads();
    }
  }
  if (grp == 0) {
    float* pp = partial + int64_t(blockIdx.x) * T * H + gt;
#pragma unroll
    for (int t = 0; t < MT; ++t)
      if (t < T)
#pragma unroll
        for (int q = 0; q < DQ; ++q) pp[t * H + q * 256] = part[t][q];
  }
}

// ------------------------------------------------------------------ reduce
// One workgroup per (64 columns, token): wave w sums partials g = w, w + 8,
// ... in order; the 8 wave sums are added in wave order.
// All BLK_WGS / BLK_RED_WAVES loads of a lane are issued before the first add.
__global__ __launch_bounds__(64 * BLK_RED_WAVES) void block_reduce_kernel(
    const float* __restrict__ partial, const float* residual, int T, int H, float* out) {
  constexpr int PER = BLK_WGS / BLK_RED_WAVES;
  static_assert(PER * BLK_RED_WAVES == BLK_WGS, "partials per wave");
  __shared__ float s_sum[BLK_RED_WAVES][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane, t = blockIdx.y;
  const float* p = partial + int64_t(t) * H + h;
  const int64_t stride = int64_t(T) * H;
  const int64_t o = int64_t(t) * H + h;
  const float res = (wave == 0 && residual) ? residual[o] : 0.0f;  // requested with the partials
  float v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) v[q] = p[int64_t(wave + q * BLK_RED_WAVES) * stride];
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < PER; ++q) acc += v[q];
  s_sum[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float v = s_sum[0][lane];
#pragma unroll
    for (int w = 1; w < BLK_RED_WAVES; ++w) v += s_sum[w][lane];
    out[o] = res + v;
  }
}

}  // namespace qmoe

namespace qmoe {

template <int HC, int MT, int GR, bool PF>
static void launch_expert_cfg(const uint16_t* x, const float* logits, int64_t E, int64_t k,
                              int32_t* topk_idx, float* topk_w, const uint16_t* w13,
                              const uint16_t* w2b, int64_t T, int64_t H, int64_t I, float* partial,
                              hipStream_t s) {
  auto fn = block_expert_kernel<HC, MT, GR, PF>;
  const size_t shm = size_t(T) * H * 2 + (GR > 1 ? size_t(T) * H * 4 : 0);
  static const bool attr = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(fn, dim3(BLK_WGS), dim3(256 * GR), shm, s, x, logits, int(E), int(k), topk_idx,
                     topk_w, w13, w2b, int(T), int(H), int(I), partial);
}

// T = 1: three item groups per workgroup (12 waves per CU; at the MoE shape
// every group gets exactly one item, so the whole 76 MB is requested at once).
// T <= 8: register budget of the 8-token accumulators allows two groups
// (one for H = 4096).
template <int HC>
static void launch_block_experts(const uint16_t* x, const float* logits, int64_t E, int64_t k,
                                 int32_t* topk_idx, float* topk_w, const uint16_t* w13,
                                 const uint16_t* w2b, int64_t T, int64_t H, int64_t I,
                                 float* partial, hipStream_t s) {
  if (T == 1)
    launch_expert_cfg<HC, 1, (HC <= 4 ? 3 : 1), (HC > 4)>(x, logits, E, k, topk_idx, topk_w, w13,
                                                          w2b, T, H, I, partial, s);
  else
    launch_expert_cfg<HC, BLK_MAX_T, (HC <= 4 ? 2 : 1), false>(x, logits, E, k, topk_idx, topk_w,
                                                               w13, w2b, T, H, I, partial, s);
}

// Argument checks shared by both entry points (everything but the partials).
static int check_block_args(const char* fn, const qmoe_bf16* x, const float* h,
                            const qmoe_bf16* rms_w, float eps, const qmoe_bf16* w_router,
                            const qmoe_bf16* w13, const qmoe_bf16* w2, int64_t T, int64_t H,
                            int64_t I, int64_t E, int64_t k, const float* logits,
                            const int32_t* topk_idx, const float* topk_w, const qmoe_bf16* x_out,
                            const float* out) {
  QMOE_REQUIRE(w_router && w13 && w2 && logits && topk_idx && topk_w && out, "%s: null pointer", fn);
  QMOE_REQUIRE((x != nullptr) != (h != nullptr), "%s: pass exactly one of x and h", fn);
  QMOE_REQUIRE(!h || (rms_w && x_out), "%s: h needs rms_w and x_out", fn);
  QMOE_REQUIRE(T >= 0 && T <= BLK_MAX_T, "%s: T must be <= 8 (T=%lld)", fn, (long long)T);
  QMOE_REQUIRE(E > 0 && E <= ROUTER_MAX_E && k > 0 && k <= ROUTER_MAX_K && k <= E && T * k <= BLK_MAX_PAIRS,
               "%s: need E <= 256, k <= min(16, E), T*k <= 64", fn);
  QMOE_REQUIRE(H >= 512 && H <= 4096 && H % 512 == 0 && (H / 512 & (H / 512 - 1)) == 0,
               "%s: H must be 512, 1024, 2048 or 4096", fn);
  QMOE_REQUIRE(I % QMOE_W13_GROUP == 0 && I > 0 && I <= 1536, "%s: I must be a multiple of 32, <= 1536",
               fn);
  QMOE_REQUIRE(eps >= 0.0f, "%s: eps < 0", fn);
  return QMOE_OK;
}

// The three launches, on validated arguments; `partial` holds BLK_WGS * T * H
// floats, every one of which the expert kernel overwrites before the reduce
// reads it (no clearing needed between calls).
static int run_block(const char* fn, const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w,
                     float eps, const qmoe_bf16* w_router, const float* bias, const qmoe_bf16* w13,
                     const qmoe_bf16* w2, const float* residual, int64_t T, int64_t H, int64_t I,
                     int64_t E, int64_t k, float* logits, int32_t* topk_idx, float* topk_w,
                     float* partial, qmoe_bf16* x_out, float* out, hipStream_t s) {
  if (T == 0) return QMOE_OK;
  const uint16_t* xin = h ? x_out : x;
  switch (H / 512) {
#define QMOE_BLK(HC)                                                                              \
  case HC:                                                                                        \
    hipLaunchKernelGGL(block_logits_kernel<HC>, dim3(unsigned(E)), dim3(unsigned(64 * T)), 0, s, x, \
                       h, rms_w, eps, w_router, bias, int(T), int(H), int(E), logits, x_out);     \
    if (int rc = hip_status(fn)) return rc;                                                       \
    launch_block_experts<HC>(xin, logits, E, k, topk_idx, topk_w, w13, w2, T, H, I, partial, s);  \
    break;
    QMOE_BLK(1)
    QMOE_BLK(2)
    QMOE_BLK(4)
    QMOE_BLK(8)
#undef QMOE_BLK
  }
  if (int rc = hip_status(fn)) return rc;
  hipLaunchKernelGGL(block_reduce_kernel, dim3(unsigned(H / 64), unsigned(T)), dim3(64 * BLK_RED_WAVES),
                     0, s, partial, residual, int(T), int(H), out);
  return hip_status(fn);
}

// ------------------------------------------------------------------ allocation-free variant
// The partials of qmoe_moe_decode_block_noalloc live in this fixed array of
// the library's device memory (16 MiB; each GPU holds its own copy until the
// process ends).  Host code never passes `scratch` itself to a kernel: on the
// host that name is only a stand-in, so its device address is looked up once
// per device with hipGetSymbolAddress and kept in g_scratch.
constexpr int64_t BLK_NOALLOC_FLOATS = int64_t(BLK_WGS) * QMOE_DECODE_BLOCK_NOALLOC_MAX_TH;
static __device__ __align__(256) float scratch[BLK_NOALLOC_FLOATS];

constexpr int SCRATCH_MAX_DEVICES = 64;
static std::atomic<float*> g_scratch[SCRATCH_MAX_DEVICES];
static std::mutex g_scratch_mu;

// Device address of the current device's `scratch` (resolved on the first
// call on that device, with that device current).
static int scratch_on_current_device(const char* fn, float** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(QMOE_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  QMOE_REQUIRE(dev >= 0 && dev < SCRATCH_MAX_DEVICES, "%s: device %d beyond %d", fn, dev,
               SCRATCH_MAX_DEVICES);
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr)
        return fail(QMOE_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                    hipGetErrorString(e));
      p = static_cast<float*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return QMOE_OK;
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int64_t qmoe_moe_decode_block_workspace(int64_t T, int64_t H) {
  if (T < 0 || H < 0) return -1;
  return int64_t(BLK_WGS) * T * H * int64_t(sizeof(float));
}

extern "C" int qmoe_moe_decode_block(const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w,
                                     float eps, const qmoe_bf16* w_router, const float* bias,
                                     const qmoe_bf16* w13, const qmoe_bf16* w2,
                                     const float* residual, int64_t T, int64_t H, int64_t I,
                                     int64_t E, int64_t k, float* logits, int32_t* topk_idx,
                                     float* topk_w, void* workspace, int64_t workspace_bytes,
                                     qmoe_bf16* x_out, float* out, qmoe_stream_t stream) {
  const char* fn = "qmoe_moe_decode_block";
  if (int rc = check_block_args(fn, x, h, rms_w, eps, w_router, w13, w2, T, H, I, E, k, logits,
                                topk_idx, topk_w, x_out, out))
    return rc;
  QMOE_REQUIRE(workspace, "%s: null workspace", fn);
  QMOE_REQUIRE(workspace_bytes >= qmoe_moe_decode_block_workspace(T, H),
               "%s: workspace of %lld bytes < %lld", fn, (long long)workspace_bytes,
               (long long)qmoe_moe_decode_block_workspace(T, H));
  return run_block(fn, x, h, rms_w, eps, w_router, bias, w13, w2, residual, T, H, I, E, k, logits,
                   topk_idx, topk_w, static_cast<float*>(workspace), x_out, out, as_stream(stream));
}

extern "C" int qmoe_moe_decode_block_noalloc(const qmoe_bf16* x, const float* h,
                                             const qmoe_bf16* rms_w, float eps,
                                             const qmoe_bf16* w_router, const float* bias,
                                             const qmoe_bf16* w13, const qmoe_bf16* w2,
                                             const float* residual, int64_t T, int64_t H,
                                             int64_t I, int64_t E, int64_t k, float* logits,
                                             int32_t* topk_idx, float* topk_w, qmoe_bf16* x_out,
                                             float* out, qmoe_stream_t stream) {
  const char* fn = "qmoe_moe_decode_block_noalloc";
  if (int rc = check_block_args(fn, x, h, rms_w, eps, w_router, w13, w2, T, H, I, E, k, logits,
                                topk_idx, topk_w, x_out, out))
    return rc;
  QMOE_REQUIRE(T * H <= QMOE_DECODE_BLOCK_NOALLOC_MAX_TH,
               "%s: T*H = %lld exceeds the static scratch limit of %d (T <= 8 at H = 2048)", fn,
               (long long)(T * H), QMOE_DECODE_BLOCK_NOALLOC_MAX_TH);
  float* partial = nullptr;
  if (int rc = scratch_on_current_device(fn, &partial)) return rc;
  return run_block(fn, x, h, rms_w, eps, w_router, bias, w13, w2, residual, T, H, I, E, k, logits,
                   topk_idx, topk_w, partial, x_out, out, as_stream(stream));
}
