// Decode-shape expert MLPs driven by dispatch metadata (T <= 64 tokens):
// HBM-bound GEMVs, each touched expert's weights streamed from HBM once.
//
//   moe_gateup_gemv_kernel   act[s,i] = silu(x.Wg[e,i]) * (x.Wu[e,i]) (fp32).
//                            The expert's gate/up rows go into registers and are
//                            applied to the expert's (few) token rows staged in LDS.
//   moe_down_gemv_kernel     y_slot[s,h] = act[s].W2[e,h] (fp32), from the blocked
//                            w2 layout [E][I/8][H][8] (one column per thread).
//
// Grid: (active-expert slot, row group); slots beyond the number of touched
// experts (meta[1]) exit at once, so the host sizes the grid as min(E, T*k)
// without knowing the routing.  (The T <= 8 fused block is moe_block_decode.hip.)
//
// The token loop keeps the weight registers opaque to the optimiser: without
// that, the loop-invariant bf16 -> fp32 unpacking is hoisted out of the loop,
// doubling the live registers, and the weight loads get serialised.
#include "decode_util.hpp"

namespace qmoe {

// ================================================================== gate/up
// Workgroup: 8 intermediate units (i0 = 8*blockIdx.y); wave w: units i0+2w,
// i0+2w+1 = 2 gate rows + the 2 matching up rows of the packed w13.
template <int HC>
__global__ __launch_bounds__(256) void moe_gateup_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ slot_token,
    const int32_t* __restrict__ active, const int32_t* __restrict__ meta, int H, int I,
    float* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [DEC_TOK_CHUNK][H]
  if (int(blockIdx.x) >= meta[1]) return;
  const int e = active[blockIdx.x];
  const int s0 = offsets[e], s1 = offsets[e + 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int i_base = blockIdx.y * 8 + wave * 2;
  const int grp = i_base / 32, off = i_base % 32;
  const uint16_t* we = w13 + int64_t(e) * 2 * I * H;
  u32x4 w[4][HC];  // rows: gate i_base, gate i_base+1, up i_base, up i_base+1
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int prow = grp * 64 + (r < 2 ? 0 : 32) + off + (r & 1);
    const uint16_t* p = we + int64_t(prow) * H + lane * 8;
#pragma unroll
    for (int c = 0; c < HC; ++c) w[r][c] = ld_stream(p + c * 512);
  }
  for (int c0 = s0; c0 < s1; c0 += DEC_TOK_CHUNK) {
    const int n = min(DEC_TOK_CHUNK, s1 - c0);
    __syncthreads();
    stage_rows_bf16(xs, x, slot_token, c0, n, H);
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
        act[int64_t(c0 + j) * I + i_base + lane] = silu(g) * u;
      }
    }
  }
}

// ================================================================== down
// Workgroup: (active-expert slot, 256 output columns).  Thread t owns column
// h = 256*blockIdx.y + t and walks the expert's I/8 blocks of the blocked w2
// ([I/8][H][8]): each 16-byte load is that column's 8 weights of one block,
// so a wave's load is 1 KB contiguous and no cross-lane reduction is needed.
// DOWN_NB blocks are loaded per batch; the expert's token rows (act, f32) are
// staged in LDS DEC_TOK_CHUNK at a time.
template <int NB>
__global__ __launch_bounds__(256) void moe_down_gemv_kernel(
    const float* __restrict__ act, const uint16_t* __restrict__ w2b,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, int H, int I, float* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(16))) float as[];  // [DEC_TOK_CHUNK][I]
  if (int(blockIdx.x) >= meta[1]) return;
  const int e = active[blockIdx.x];
  const int s0 = offsets[e], s1 = offsets[e + 1];
  const int t = threadIdx.x;
  const int h = blockIdx.y * 256 + t;
  const int NS = I / QMOE_W2_BLOCK;
  const uint16_t* wp = w2b + (int64_t(e) * NS * H + h) * QMOE_W2_BLOCK;
  for (int c0 = s0; c0 < s1; c0 += DEC_TOK_CHUNK) {
    const int n = min(DEC_TOK_CHUNK, s1 - c0);
    __syncthreads();
    const int i4 = I / 4;
    for (int q = t; q < n * i4; q += 256) {
      const int j = q / i4, c = q - j * i4;
      reinterpret_cast<float4*>(as + j * I)[c] =
          reinterpret_cast<const float4*>(act + int64_t(c0 + j) * I)[c];
    }
    __syncthreads();
    float acc[DEC_TOK_CHUNK];
#pragma unroll
    for (int j = 0; j < DEC_TOK_CHUNK; ++j) acc[j] = 0.0f;
    for (int b0 = 0; b0 < NS; b0 += NB) {
      u32x4 w[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b)
        w[b] = (b0 + b < NS) ? ld_stream(wp + int64_t(b0 + b) * H * QMOE_W2_BLOCK) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < DEC_TOK_CHUNK; ++j) {
        if (j < n) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            if (b0 + b < NS) {
              const float4 a0 = reinterpret_cast<const float4*>(as + j * I + (b0 + b) * 8)[0];
              const float4 a1 = reinterpret_cast<const float4*>(as + j * I + (b0 + b) * 8)[1];
              const float x8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
              opaque(w[b]);
              acc[j] += dot8(w[b], x8);
            }
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < DEC_TOK_CHUNK; ++j)
      if (j < n) y_slot[int64_t(c0 + j) * H + h] = acc[j];
  }
}

// ================================================================== launchers
static int check_dec_shapes(const char* fn, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  QMOE_REQUIRE(T >= 0 && T <= DEC_MAX_T, "%s: T must be <= 64 (T=%lld)", fn, (long long)T);
  QMOE_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= E, "%s: bad E/k", fn);
  QMOE_REQUIRE(H % 512 == 0 && H >= 512 && H <= 4096 && (H / 512 & (H / 512 - 1)) == 0,
               "%s: H must be 512, 1024, 2048 or 4096 (H=%lld)", fn, (long long)H);
  QMOE_REQUIRE(I % 32 == 0 && I > 0 && I <= 1536, "%s: I must be a multiple of 32, <= 1536", fn);
  return QMOE_OK;
}

static int launch_experts(const uint16_t* x, const uint16_t* w13, const uint16_t* w2,
                          const int32_t* offsets, const int32_t* slot_token, const int32_t* active,
                          const int32_t* meta, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                          float* act, float* y_slot, hipStream_t s) {
  const unsigned nact = unsigned(std::min<int64_t>(E, T * k));
  // rows of one expert <= T*k (a token may list an expert twice via the seams)
  const int64_t stage_rows = std::min<int64_t>(T * k, DEC_TOK_CHUNK);
  const size_t shm1 = size_t(stage_rows) * H * 2;
  dim3 g1(nact, unsigned(I / 8));
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
  }
  int rc = hip_status("moe experts (gate_up)");
  if (rc) return rc;
  const size_t shm2 = size_t(stage_rows) * I * 4;
  dim3 g2(nact, unsigned(H / 256));
  hipLaunchKernelGGL(moe_down_gemv_kernel<DOWN_NB>, g2, dim3(256), shm2, s, act, w2, offsets, active,
                     meta, int(H), int(I), y_slot);
  return hip_status("moe experts (down)");
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_moe_experts_gemv(const qmoe_bf16* x, const qmoe_bf16* w13,
                                     const qmoe_bf16* w2, const int32_t* offsets,
                                     const int32_t* slot_token, const int32_t* active,
                                     const int32_t* meta, int64_t T, int64_t H, int64_t I,
                                     int64_t E, int64_t k, float* act, float* y_slot,
                                     qmoe_stream_t stream) {
  QMOE_REQUIRE(x && w13 && w2 && offsets && slot_token && active && meta && act && y_slot,
               "qmoe_moe_experts_gemv: null pointer");
  int rc = check_dec_shapes("qmoe_moe_experts_gemv", T, H, I, E, k);
  if (rc) return rc;
  if (T == 0) return QMOE_OK;
  return launch_experts(x, w13, w2, offsets, slot_token, active, meta, T, H, I, E, k, act, y_slot,
                        as_stream(stream));
}

