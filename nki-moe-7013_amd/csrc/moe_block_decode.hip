// The whole MoE block at decode shape (T <= 8 tokens).  At T = 1 and the
// Qwen3-30B-A3B shape it is one launch (block_fused_kernel, below); otherwise
// three:
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

// ------------------------------------------------------------------ fused T = 1 block
// The whole block in one launch for one token at the Qwen3-30B-A3B shape
// (H = 2048, I = 768, k = 8, E <= 256).  256 workgroups of 12 waves, one per
// CU and all resident at once (the host checks the CU count):
//   router   wave w < 8 of workgroup g < E / 8 computes router logit 8g + w;
//            the workgroup publishes its 8 logits together (8 copies, one
//            per XCD; one 64-byte store each); wave 0 of every workgroup
//            collects the E logits from its XCD's copy.
//   top-k    wave 0, on the logits in registers (k rounds of a DPP max).
//   gate/up  workgroup g = (j, m), j = g / 32 the rank of its expert, m =
//            g % 32: the 24 units [24m, 24m + 24) of expert j, wave w units
//            24m + 2w and + 1 (four rows of H).  Each wave publishes its two
//            SwiGLU outputs times the routing weight.
//   handoff  wave 0 collects expert j's 768 activations and shares them in
//   1        LDS.
//   down     rows [64m, 64m + 64) of expert j over all 768 units: wave w
//            blocks 8w .. 8w + 7 of the 96 8-unit blocks, lane l row 64m + l
//            (one 16-byte chunk of the blocked layout per block; 1 KB
//            contiguous per instruction).  The down loads go out once the
//            wave's gate/up rows are in, so the gate/up traffic that handoff
//            1 waits for goes first and the handoff runs under the down
//            traffic.  Each thread sums its row over the wave's blocks, the
//            workgroup the 12 waves in order.
//   handoff  the 64 row sums are published; workgroup (j, m) collects rows
//   2        64m + 8j .. + 8 from the 8 workgroups (0..7, m) (all on one
//            XCD) and writes residual + the sum over the experts in rank
//            order.
// Every exchanged value carries its call's tag, so no fence or flag orders
// data against a signal: a reader polls (relaxed agent-scope atomics) until
// every word it needs carries the tag of the current call.  The call number
// is each workgroup's own counter in the workspace header, read and advanced
// once per call by that workgroup alone (all of them run once per call, so
// the counters stay equal).  Logits are 64-bit (tag, value) words; the
// SwiGLU outputs are fp32 rounded to 19 mantissa bits with a 4-bit tag (call
// number mod 15, plus 1) in the low bits, two per 64-bit word, which halves
// the words polled; the reader clears the tag bits.  Waits give up after
// FB_SPIN polls: the workgroup then sets the header's status word and writes
// NaN to its output rows, and every wait of the call still ends, so the
// launch drains.
constexpr int FB_WGS = QMOE_DECODE_BLOCK_WGS;
constexpr int FB_WAVES = 12, FB_THREADS = 64 * FB_WAVES;
constexpr int FB_H = 2048, FB_I = 768, FB_K = 8, FB_HC = FB_H / 512;
constexpr int FB_GPE = FB_WGS / FB_K;                // workgroups per expert rank: 32
constexpr int FB_UNITS = FB_I / FB_GPE;               // SwiGLU units per workgroup: 24
constexpr int FB_ROWS = FB_H / FB_GPE;                // down rows per workgroup: 64
constexpr int FB_BLOCKS = FB_I / QMOE_W2_BLOCK;       // 8-unit blocks of the down matrix: 96
constexpr int FB_DBLK = FB_BLOCKS / FB_WAVES;         // down blocks per wave: 8
static_assert(FB_UNITS == 2 * FB_WAVES, "two units per wave");
static_assert(FB_DBLK * FB_WAVES == FB_BLOCKS && FB_ROWS == 64, "one row per lane, 8 blocks per wave");
constexpr int FB_SPIN = 1 << 15;  // polls (each a memory round trip) before a wait gives up
// workspace header, in 32-bit words
constexpr int FBW_EPOCH = 0;          // u32[FB_WGS]: calls run by workgroup g
constexpr int FBW_STATUS = FB_WGS;    // u32: nonzero once a wait gave up
constexpr int FBW_LOGIT = 1024;       // u64 [8 XCD copies][ROUTER_MAX_E], FBW_LOGIT_REP words apart
constexpr int FBW_LOGIT_REP = 1056;
constexpr int FBW_ACT = 10240;        // u64 [FB_K][FB_I / 2]: two tagged SwiGLU outputs each
constexpr int FBW_PART = 16384;       // u64 [FB_GPE][FB_K][FB_ROWS]: tagged row sums
constexpr int FBW_END = FBW_PART + 2 * FB_GPE * FB_K * FB_ROWS;
constexpr int64_t FB_HEADER_BYTES = QMOE_DECODE_BLOCK_STATE_BYTES;
static_assert(FBW_STATUS * 4 == QMOE_DECODE_BLOCK_STATUS_OFFSET, "status word as the header says");
static_assert(FBW_LOGIT + 8 * FBW_LOGIT_REP <= FBW_ACT && 2 * ROUTER_MAX_E <= FBW_LOGIT_REP &&
                  FBW_ACT + FB_K * FB_I <= FBW_PART && int64_t(FBW_END) * 4 <= FB_HEADER_BYTES,
              "header layout");

__device__ __forceinline__ uint64_t ld_agent64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fb_tag32(uint32_t ep) { return ep % 0xffffffffu + 1u; }
__device__ __forceinline__ uint32_t fb_tag4(uint32_t ep) { return ep % 15u + 1u; }
// fp32 -> 19-bit mantissa (round to nearest, ties away) with tag t in bits 0-3;
// NaN becomes the default quiet NaN, which survives the reader's masking.
__device__ __forceinline__ uint32_t fb_selftag(float v, uint32_t t) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t a = b & 0x7fffffffu;
  const uint32_t r = a > 0x7f800000u ? 0x7fc00000u : (a == 0x7f800000u ? b : b + 8u);
  return (r & ~15u) | t;
}
__device__ __forceinline__ float fb_untag(uint32_t w) { return __uint_as_float(w & ~15u); }
__device__ __forceinline__ bool fb_has_tag4(uint64_t v, uint32_t t) {
  return (uint32_t(v) & 15u) == t && (uint32_t(v >> 32) & 15u) == t;
}
// Order-preserving key of a logit (NaN ranks as -inf); every key of a valid
// logit is >= key(-inf) = 0x007fffff, so 0 marks padding.
__device__ __forceinline__ uint32_t fb_key(float l) {
  const uint32_t b = __float_as_uint(l != l ? -INFINITY : l);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float fb_unkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// bf16(rmsnorm(h) * w) of one H = 512 * HC row by one wave: lane l holds
// elements c * 512 + 8 l .. + 8 (c < HC) as packed bf16.
template <int HC>
__device__ __forceinline__ void norm_row_wave(const float* __restrict__ h, const uint16_t* __restrict__ w,
                                              float eps, int H, u32x4* xb) {
  const int lane = threadIdx.x & 63;
  u32x4 wn[HC];
  float xf[HC][8];
#pragma unroll
  for (int c = 0; c < HC; ++c) wn[c] = ld16(w + c * 512 + lane * 8);
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    const float4* hp = reinterpret_cast<const float4*>(h + c * 512 + lane * 8);
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
    xb[c].x = pack_bf16x2(wf[0] * (xf[c][0] * rr), wf[1] * (xf[c][1] * rr));
    xb[c].y = pack_bf16x2(wf[2] * (xf[c][2] * rr), wf[3] * (xf[c][3] * rr));
    xb[c].z = pack_bf16x2(wf[4] * (xf[c][4] * rr), wf[5] * (xf[c][5] * rr));
    xb[c].w = pack_bf16x2(wf[6] * (xf[c][6] * rr), wf[7] * (xf[c][7] * rr));
  }
}

// Top-k of one token by one wave, keys in registers: lane l holds the order
// keys (fb_key) of logits l + 64 j, j < J, 0 for padding.  k rounds of one
// DPP max; the round's winner is the lowest index holding the max key (read
// from the ballots of the J registers in index order), which is then cleared:
// the selection and tie rule of the other top-k kernels.  Lane 0 writes the
// winner of round r to s_idx[r] and its key to s_top[r].
template <int J>
__device__ __forceinline__ void fb_topk_wave(uint32_t (&key)[J], int k, int32_t* s_idx, uint32_t* s_top) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < ROUTER_MAX_K; ++r) {
    if (r < k) {
      uint32_t best = key[0];
#pragma unroll
      for (int j = 1; j < J; ++j) best = max(best, key[j]);
      best = dpp_max_u32_wave(best);
      int win = -1;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const unsigned long long msk = __ballot(key[j] == best);
        if (win < 0 && msk != 0ull) win = 64 * j + __builtin_ctzll(msk);
      }
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (lane + 64 * j == win) key[j] = 0u;
      if (lane == 0) {
        s_idx[r] = win;
        s_top[r] = best;
      }
    }
  }
}

__global__ __launch_bounds__(FB_THREADS) void block_fused_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ h, const uint16_t* __restrict__ rms_w,
    float eps, const uint16_t* __restrict__ w_router, const float* __restrict__ bias, int E,
    const uint16_t* __restrict__ w13, const uint16_t* __restrict__ w2b, const float* residual,
    float* __restrict__ logits, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    uint32_t* __restrict__ ws, uint16_t* __restrict__ x_out, float* out) {
  constexpr int HC = FB_HC, H = FB_H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = blockIdx.x;
  const int j = g / FB_GPE, m = g % FB_GPE;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[FB_H];
  __shared__ int32_t s_idx[FB_K];
  __shared__ uint32_t s_top[FB_K];  // keys of the selected logits, by rank
  __shared__ __attribute__((aligned(16))) float s_act[FB_I];
  __shared__ float s_red[FB_WAVES][FB_ROWS];
  __shared__ float s_fin[64];
  __shared__ float s_plog[FB_K];
  __shared__ uint32_t s_ep;
  __shared__ int s_fail;
  uint64_t* const logit_x = reinterpret_cast<uint64_t*>(ws + FBW_LOGIT);
  uint64_t* const act_x = reinterpret_cast<uint64_t*>(ws + FBW_ACT);
  uint64_t* const part_x = reinterpret_cast<uint64_t*>(ws + FBW_PART);
  const int out_row = m * FB_ROWS + FB_K * j + tid;  // rows this workgroup finishes (tid < 8)
  const float res = (tid < FB_K && residual) ? residual[out_row] : 0.0f;

  // ---- router: workgroup p < ceil(E / 8) computes logits 8p .. 8p + 7, one
  // per wave, and publishes them together (one 64-byte store per XCD copy)
  constexpr int LJ = ROUTER_MAX_E / 64;
  const int e_r = FB_K * g + wave;  // the router row of this wave, if any
  const bool prod = wave < FB_K && e_r < E;
  uint32_t ep0 = 0u;  // wave 0: this workgroup's call count
  if (wave == 0) {
    if (lane == 0) ep0 = __hip_atomic_load(ws + FBW_EPOCH + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ep0 = __builtin_amdgcn_readfirstlane(ep0);
  }
  if (wave == 0 || prod) {
    u32x4 wr[HC];
    if (prod)
#pragma unroll
      for (int c = 0; c < HC; ++c) wr[c] = ld_stream(w_router + int64_t(e_r) * H + c * 512 + lane * 8);
    u32x4 xb[HC];
    if (h) {
      norm_row_wave<HC>(h, rms_w, eps, H, xb);
      if (g == 0 && wave == 0)
#pragma unroll
        for (int c = 0; c < HC; ++c) *reinterpret_cast<u32x4*>(x_out + c * 512 + lane * 8) = xb[c];
    } else {
#pragma unroll
      for (int c = 0; c < HC; ++c) xb[c] = ld16(x + c * 512 + lane * 8);
    }
    if (wave == 0)
#pragma unroll
      for (int c = 0; c < HC; ++c) *reinterpret_cast<u32x4*>(s_x + c * 512 + lane * 8) = xb[c];
    if (prod) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        float xf[8];
        unpack8(xb[c], xf);
        opaque(wr[c]);
        acc += dot8(wr[c], xf);
      }
      acc = wave_sum(acc) + (bias ? bias[e_r] : 0.0f);
      if (lane == 0) {
        logits[e_r] = acc;
        s_plog[wave] = acc;
      }
    }
  }
  lds_barrier();
  if (wave == 0) {
    bool fail = false;
    uint32_t key[LJ];
    {
      const uint32_t t32 = fb_tag32(ep0);
      if (lane < FB_K && FB_K * g + lane < E) {
        const uint64_t v = (uint64_t(t32) << 32) | __float_as_uint(s_plog[lane]);
#pragma unroll
        for (int r = 0; r < 8; ++r) st_agent64(logit_x + r * (FBW_LOGIT_REP / 2) + FB_K * g + lane, v);
      }
      const uint64_t* src = logit_x + xcc_id() * (FBW_LOGIT_REP / 2);
      uint64_t v[LJ];
      bool ok;
      int n = 0;
      do {
#pragma unroll
        for (int i = 0; i < LJ; ++i) v[i] = lane + 64 * i < E ? ld_agent64(src + lane + 64 * i) : 0ull;
        ok = true;
#pragma unroll
        for (int i = 0; i < LJ; ++i) ok = ok && (lane + 64 * i >= E || uint32_t(v[i] >> 32) == t32);
      } while (__ballot(!ok) != 0ull && ++n < FB_SPIN);
      fail = __ballot(!ok) != 0ull;
#pragma unroll
      for (int i = 0; i < LJ; ++i) key[i] = lane + 64 * i < E ? fb_key(__uint_as_float(uint32_t(v[i]))) : 0u;
    }
    if (E <= 64) {
      uint32_t k1[1] = {key[0]};
      fb_topk_wave<1>(k1, FB_K, s_idx, s_top);
    } else if (E <= 128) {
      uint32_t k2[2] = {key[0], key[1]};
      fb_topk_wave<2>(k2, FB_K, s_idx, s_top);
    } else {
      fb_topk_wave<4>(key, FB_K, s_idx, s_top);
    }
    if (lane == 0) {
      __hip_atomic_store(ws + FBW_EPOCH + g, ep0 + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_ep = ep0;
      s_fail = fail ? 1 : 0;
    }
  }
  lds_barrier();
  const uint32_t ep = s_ep;
  // ---- routing weights exp(l_r - l_0) / sum over the k chosen, summed over
  // lanes 0..k-1 in the wave-sum's fixed order; every wave computes them
  const float pr = lane < FB_K ? expf(fb_unkey(s_top[lane]) - fb_unkey(s_top[0])) : 0.0f;
  const float wsum = wave_sum(pr);
  const float wt = __shfl(pr, j) / wsum;  // the weight of this workgroup's gate/up expert
  if (g == 0 && tid < FB_K) {
    topk_idx[tid] = s_idx[tid];
    topk_w[tid] = pr / wsum;
  }
  const int e = s_idx[j];

  // ---- gate and up rows of the wave's two units
  const int u0 = m * FB_UNITS + 2 * wave;  // even: u0 and u0 + 1 share a packed 32-row group
  const uint16_t* we = w13 + int64_t(e) * 2 * FB_I * H;
  u32x4 gu[4][HC];  // gate u0, gate u0 + 1, up u0, up u0 + 1
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int prow = (u0 / QMOE_W13_GROUP) * 2 * QMOE_W13_GROUP + (q < 2 ? 0 : QMOE_W13_GROUP) +
                     (u0 % QMOE_W13_GROUP) + (q & 1);
#pragma unroll
    for (int c = 0; c < HC; ++c) gu[q][c] = ld_stream(we + int64_t(prow) * H + c * 512 + lane * 8);
  }

  // ---- SwiGLU of the wave's two units -> published
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    float xf[8];
    unpack8(*reinterpret_cast<const u32x4*>(s_x + c * 512 + lane * 8), xf);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      opaque(gu[q][c]);
      acc[q] += dot8(gu[q][c], xf);
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = wave_sum(acc[q]);
  const uint32_t t4 = fb_tag4(ep);
  if (lane == 0) {
    const float a0 = silu(acc[0]) * acc[2] * wt, a1 = silu(acc[1]) * acc[3] * wt;
    st_agent64(act_x + j * (FB_I / 2) + m * (FB_UNITS / 2) + wave,
               uint64_t(fb_selftag(a0, t4)) | (uint64_t(fb_selftag(a1, t4)) << 32));
  }

  // ---- down rows 64m + lane of expert j, blocks 8w .. 8w + 7
  const uint16_t* wd =
      w2b + ((int64_t(e) * FB_BLOCKS + FB_DBLK * wave) * H + m * FB_ROWS + lane) * QMOE_W2_BLOCK;
  u32x4 dn[FB_DBLK];
#pragma unroll
  for (int b = 0; b < FB_DBLK; ++b) dn[b] = ld_stream(wd + int64_t(b) * H * QMOE_W2_BLOCK);

  // ---- handoff 1: wave 0 collects expert j's 768 activations (first poll
  // once the wave's own rows are in: by then most are published)
  if (wave == 0) {
    constexpr int AJ = FB_I / 2 / 64;  // 6 words per lane
    const uint64_t* src = act_x + j * (FB_I / 2);
    uint64_t v[AJ];
    bool ok;
    int n = 0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    do {
      if (n > 0) __builtin_amdgcn_s_sleep(4);
#pragma unroll
      for (int i = 0; i < AJ; ++i) v[i] = ld_agent64(src + lane + 64 * i);
      ok = true;
#pragma unroll
      for (int i = 0; i < AJ; ++i) ok = ok && fb_has_tag4(v[i], t4);
    } while (__ballot(!ok) != 0ull && ++n < FB_SPIN);
    if (__ballot(!ok) != 0ull && lane == 0) s_fail = 1;
#pragma unroll
    for (int i = 0; i < AJ; ++i) {
      const int a = 2 * (lane + 64 * i);
      *reinterpret_cast<float2*>(s_act + a) = float2{fb_untag(uint32_t(v[i])), fb_untag(uint32_t(v[i] >> 32))};
    }
  }
  lds_barrier();

  // ---- down product: each thread its row over the wave's 8 blocks
  float y = 0.0f;
#pragma unroll
  for (int b = 0; b < FB_DBLK; ++b) {
    const float* ap = s_act + (FB_DBLK * wave + b) * QMOE_W2_BLOCK;  // same address in every lane
    const float4 p0 = *reinterpret_cast<const float4*>(ap);
    const float4 p1 = *reinterpret_cast<const float4*>(ap + 4);
    const float a8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    opaque(dn[b]);
    y += dot8(dn[b], a8);
  }
  s_red[wave][lane] = y;
  lds_barrier();

  // ---- handoff 2: the 12 waves in order -> published; rows 64m + 8j .. + 8
  // collected from the 8 experts' workgroups and summed in rank order
  if (wave == 0) {
    const uint32_t t32 = fb_tag32(ep);
    float v = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < FB_WAVES; ++w) v += s_red[w][lane];
    st_agent64(part_x + (m * FB_K + j) * FB_ROWS + lane, (uint64_t(t32) << 32) | __float_as_uint(v));
    const uint64_t* src = part_x + (m * FB_K + (lane >> 3)) * FB_ROWS + FB_K * j + (lane & 7);
    uint64_t q;
    bool ok;
    int n = 0;
    do {
      q = ld_agent64(src);
      ok = uint32_t(q >> 32) == t32;
    } while (__ballot(!ok) != 0ull && ++n < FB_SPIN);
    if (__ballot(!ok) != 0ull && lane == 0) s_fail = 1;
    s_fin[lane] = __uint_as_float(uint32_t(q));
  }
  lds_barrier();
  if (tid < FB_K) {
    float s = s_fin[tid];
#pragma unroll
    for (int x8 = 1; x8 < FB_K; ++x8) s += s_fin[FB_K * x8 + tid];
    out[out_row] = s_fail ? __builtin_nanf("") : res + s;
  }
  if (tid == 0 && s_fail) __hip_atomic_store(ws + FBW_STATUS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  QMOE_REQUIRE(w_router && w13 && w2 && (T == 0 || (logits && topk_idx && topk_w && out)), "%s: null pointer", fn);
  QMOE_REQUIRE(T == 0 || (x != nullptr) != (h != nullptr), "%s: pass exactly one of x and h", fn);
  QMOE_REQUIRE(!h || (rms_w && (T == 0 || x_out)), "%s: h needs rms_w and x_out", fn);
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

// The single-launch form covers one token at the shape it is built for, with
// all FB_WGS workgroups resident at once (one per CU).
static bool fused_block_applies(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  return T == 1 && H == FB_H && I == FB_I && k == FB_K && E <= ROUTER_MAX_E &&
         current_device_cus() >= FB_WGS;
}

// The launches, on validated arguments.  `workspace` starts with
// FB_HEADER_BYTES of call-to-call state (zero before the first call; used by
// the fused T = 1 launch only), then BLK_WGS * T * H floats of partials,
// every one of which the expert kernel overwrites before the reduce reads it.
static int run_block(const char* fn, const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w,
                     float eps, const qmoe_bf16* w_router, const float* bias, const qmoe_bf16* w13,
                     const qmoe_bf16* w2, const float* residual, int64_t T, int64_t H, int64_t I,
                     int64_t E, int64_t k, float* logits, int32_t* topk_idx, float* topk_w,
                     void* workspace, qmoe_bf16* x_out, float* out, hipStream_t s) {
  if (T == 0) return QMOE_OK;
  uint32_t* header = static_cast<uint32_t*>(workspace);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + FB_HEADER_BYTES);
  const uint16_t* xin = h ? x_out : x;
  if (fused_block_applies(T, H, I, E, k)) {
    hipLaunchKernelGGL(block_fused_kernel, dim3(FB_WGS), dim3(FB_THREADS), 0, s, x, h, rms_w, eps, w_router,
                       bias, int(E), w13, w2, residual, logits, topk_idx, topk_w, header, x_out, out);
    return hip_status(fn);
  }
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
constexpr int64_t BLK_NOALLOC_FLOATS =
    FB_HEADER_BYTES / 4 + int64_t(BLK_WGS) * QMOE_DECODE_BLOCK_NOALLOC_MAX_TH;
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
  return FB_HEADER_BYTES + int64_t(BLK_WGS) * T * H * int64_t(sizeof(float));
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
                   topk_idx, topk_w, workspace, x_out, out, as_stream(stream));
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
