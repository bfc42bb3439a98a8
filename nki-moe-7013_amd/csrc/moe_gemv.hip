// Decode-shape expert MLPs (T <= 64 tokens): HBM-bound GEMV form.
//
// Every expert touched by at least one token has its weights streamed from
// HBM exactly once; the (few) token rows routed to it are applied to the
// weights while they sit in registers.
//
//   phase 1  act[s, i]   = silu(x[tok(s)] . Wg[e,i]) * (x[tok(s)] . Wu[e,i])   (fp32)
//   phase 2  y_slot[s,h] = act[s] . W2[e,h]                                   (fp32)
//
// Grid: (active-expert slot, row group).  A workgroup whose active slot is
// beyond the number of touched experts (meta[1]) exits at once, so the grid
// can be sized on the host as min(E, T*k) without knowing the routing.
//
// Phase 1 row mapping.  w13 is packed in groups of 64 rows (32 gate rows then
// the 32 matching up rows).  A workgroup covers 16 intermediate units
// i0 = 16*blockIdx.y; wave w owns units i0 + 4w + [0, 4): 4 gate rows and the
// 4 matching up rows, each 2*H bytes, held in registers (H/512 16-byte loads
// per row per lane).
//
// Phase 2 row mapping.  A workgroup covers 32 output rows h; wave w owns 8.
// A row of W2 is I bf16 = I/8 16-byte chunks; lane l loads chunks l, l+64, ...
#include "common.hpp"

namespace qmoe {

constexpr int GV_TOK_CHUNK = 16;   // token rows staged in LDS at a time
constexpr int GV_MAX_H = 4096;     // register budget: H/512 chunks per row
constexpr int GV_MAX_I = 1536;     // I/512 chunks per W2 row (ceil)

template <int HC>  // HC = H / 512 (16-byte chunks per lane per row)
__global__ __launch_bounds__(256) void moe_gateup_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ slot_token,
    const int32_t* __restrict__ active, const int32_t* __restrict__ meta, int H, int I,
    float* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [GV_TOK_CHUNK][H]
  if (int(blockIdx.x) >= meta[1]) return;
  const int e = active[blockIdx.x];
  const int s0 = offsets[e], s1 = offsets[e + 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int i_base = blockIdx.y * 16 + wave * 4;  // first intermediate unit of this wave
  const int grp = i_base / 32, off = i_base % 32;
  const uint16_t* we = w13 + int64_t(e) * 2 * I * H;
  // rows: 0..3 gate units i_base+r, 4..7 up units i_base+r
  u32x4 w[8][HC];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int prow = grp * 64 + (r < 4 ? 0 : 32) + off + (r & 3);
    const uint16_t* p = we + int64_t(prow) * H + lane * 8;
#pragma unroll
    for (int c = 0; c < HC; ++c) w[r][c] = ld_stream(p + c * 512);
  }
  for (int c0 = s0; c0 < s1; c0 += GV_TOK_CHUNK) {
    const int n = min(GV_TOK_CHUNK, s1 - c0);
    __syncthreads();
    const int hch = H / 8;
    for (int q = t; q < n * hch; q += 256) {
      const int j = q / hch, kc = q - j * hch;
      *reinterpret_cast<u32x4*>(xs + j * H + kc * 8) =
          ld16(x + int64_t(slot_token[c0 + j]) * H + kc * 8);
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      float acc[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + j * H + c * 512 + lane * 8);
        float x8[8] = {bf16_lo(xv.x), bf16_hi(xv.x), bf16_lo(xv.y), bf16_hi(xv.y),
                       bf16_lo(xv.z), bf16_hi(xv.z), bf16_lo(xv.w), bf16_hi(xv.w)};
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[r] += dot8(w[r][c], x8);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = wave_sum(acc[r]);
      if (lane < 4) {
        // lane r writes unit i_base + r (select without dynamic register indexing)
        float g = acc[0], u = acc[4];
#pragma unroll
        for (int r = 1; r < 4; ++r)
          if (lane == r) {
            g = acc[r];
            u = acc[4 + r];
          }
        act[int64_t(c0 + j) * I + i_base + lane] = silu(g) * u;
      }
    }
  }
}

template <int IC>  // IC = ceil(I / 512)
__global__ __launch_bounds__(256) void moe_down_gemv_kernel(
    const float* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, int H, int I, float* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(16))) float as[];  // [GV_TOK_CHUNK][I]
  if (int(blockIdx.x) >= meta[1]) return;
  const int e = active[blockIdx.x];
  const int s0 = offsets[e], s1 = offsets[e + 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h_base = blockIdx.y * 32 + wave * 8;
  const int ichunks = I / 8;
  const uint16_t* we = w2 + int64_t(e) * H * I;
  u32x4 w[8][IC];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const uint16_t* p = we + int64_t(h_base + r) * I;
#pragma unroll
    for (int c = 0; c < IC; ++c) {
      const int ch = lane + 64 * c;
      w[r][c] = (ch < ichunks) ? ld_stream(p + ch * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  for (int c0 = s0; c0 < s1; c0 += GV_TOK_CHUNK) {
    const int n = min(GV_TOK_CHUNK, s1 - c0);
    __syncthreads();
    const int i4 = I / 4;
    for (int q = t; q < n * i4; q += 256) {
      const int j = q / i4, c = q - j * i4;
      reinterpret_cast<float4*>(as + j * I)[c] =
          reinterpret_cast<const float4*>(act + int64_t(c0 + j) * I)[c];
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      float acc[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < IC; ++c) {
        const int ch = lane + 64 * c;
        if (ch < ichunks) {
          const float4 a0 = reinterpret_cast<const float4*>(as + j * I + ch * 8)[0];
          const float4 a1 = reinterpret_cast<const float4*>(as + j * I + ch * 8)[1];
          const float x8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
          for (int r = 0; r < 8; ++r) acc[r] += dot8(w[r][c], x8);
        }
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = wave_sum(acc[r]);
      if (lane < 8) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < 8; ++r)
          if (lane == r) v = acc[r];
        y_slot[int64_t(c0 + j) * H + h_base + lane] = v;
      }
    }
  }
}

}  // namespace qmoe

extern "C" int qmoe_moe_experts_gemv(const qmoe_bf16* x, const qmoe_bf16* w13,
                                     const qmoe_bf16* w2, const int32_t* offsets,
                                     const int32_t* slot_token, const int32_t* active,
                                     const int32_t* meta, int64_t T, int64_t H, int64_t I,
                                     int64_t E, int64_t k, float* act, float* y_slot,
                                     qmoe_stream_t stream) {
  using namespace qmoe;
  QMOE_REQUIRE(x && w13 && w2 && offsets && slot_token && active && meta && act && y_slot,
               "qmoe_moe_experts_gemv: null pointer");
  QMOE_REQUIRE(T >= 0 && T <= 64, "qmoe_moe_experts_gemv: T must be <= 64 (T=%lld)", (long long)T);
  QMOE_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= E, "qmoe_moe_experts_gemv: bad E/k");
  QMOE_REQUIRE(H % 512 == 0 && H <= GV_MAX_H, "qmoe_moe_experts_gemv: H must be a multiple of 512, <= 4096");
  QMOE_REQUIRE(I % 32 == 0 && I <= GV_MAX_I, "qmoe_moe_experts_gemv: I must be a multiple of 32, <= 1536");
  if (T == 0) return QMOE_OK;
  hipStream_t s = as_stream(stream);
  const unsigned nact = unsigned(std::min<int64_t>(E, T * k));
  // rows of one expert <= T*k (a token may list an expert twice via the seams)
  const int64_t stage_rows = std::min<int64_t>(T * k, GV_TOK_CHUNK);
  const size_t shm1 = size_t(stage_rows) * H * 2;
  dim3 g1(nact, unsigned(I / 16));
  switch (H / 512) {
#define QMOE_GU(HC)                                                                          \
  case HC:                                                                                   \
    hipLaunchKernelGGL(moe_gateup_gemv_kernel<HC>, g1, dim3(256), shm1, s, x, w13, offsets,  \
                       slot_token, active, meta, int(H), int(I), act);                      \
    break;
    QMOE_GU(1)
    QMOE_GU(2)
    QMOE_GU(4)
    QMOE_GU(8)
#undef QMOE_GU
    default:
      return fail(QMOE_ERR_INVALID, "qmoe_moe_experts_gemv: unsupported H=%lld", (long long)H);
  }
  int rc = hip_status("qmoe_moe_experts_gemv(gate_up)");
  if (rc) return rc;
  const size_t shm2 = size_t(stage_rows) * I * 4;
  dim3 g2(nact, unsigned(H / 32));
  const int ic = int((I / 8 + 63) / 64);
  switch (ic) {
#define QMOE_DN(IC)                                                                           \
  case IC:                                                                                    \
    hipLaunchKernelGGL(moe_down_gemv_kernel<IC>, g2, dim3(256), shm2, s, act, w2, offsets,    \
                       active, meta, int(H), int(I), y_slot);                                 \
    break;
    QMOE_DN(1)
    QMOE_DN(2)
    QMOE_DN(3)
#undef QMOE_DN
    default:
      return fail(QMOE_ERR_INVALID, "qmoe_moe_experts_gemv: unsupported I=%lld", (long long)I);
  }
  return hip_status("qmoe_moe_experts_gemv(down)");
}
