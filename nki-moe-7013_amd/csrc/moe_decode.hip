// Decode-shape expert MLPs driven by dispatch metadata (T <= 64 tokens):
// HBM-bound GEMVs, each touched expert's weights streamed from HBM once.
//
//   moe_gateup_gemv_kernel   act[s,i] = silu(x.Wg[e,i]) * (x.Wu[e,i]) (fp32).
//                            The expert's gate/up rows go into registers and are
//                            applied to the expert's (few) token rows staged in LDS.
//   moe_down_mfma_kernel     y_slot[s,h] = bf16(act[s]).W2[e,h] (fp32 accumulation)
//                            on MFMA, from the blocked w2 layout [E][I/8][H][8].
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

// Token rows of gate/up staged in LDS at a time: small enough that several
// workgroups share a CU, so each new workgroup's dependent first loads
// (routing metadata, then its expert's rows) overlap the others' weight
// streams.  4 rows (16 KB at H = 2048) leave room for five workgroups per
// CU; 16 rows (64 KB) allowed two and made the gate/up pass 1.4x slower at
// T = 64.
#ifndef QMOE_GU_TOK_CHUNK
#define QMOE_GU_TOK_CHUNK 4
#endif
constexpr int GU_TOK_CHUNK = QMOE_GU_TOK_CHUNK;

// ================================================================== gate/up
// Workgroup: 8 intermediate units (i0 = 8*blockIdx.y); wave w: units i0+2w,
// i0+2w+1 = 2 gate rows + the 2 matching up rows of the packed w13.
template <int HC, int TC>
__global__ __launch_bounds__(256) void moe_gateup_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ slot_token,
    const int32_t* __restrict__ active, const int32_t* __restrict__ meta, int H, int I,
    float* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [TC][H]
  // both requested before the branch (active has E >= gridDim.x entries)
  const int n_active = meta[1], e = active[blockIdx.x];
  if (int(blockIdx.x) >= n_active) return;
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
  for (int c0 = s0; c0 < s1; c0 += TC) {
    const int n = min(TC, s1 - c0);
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
// Workgroup: (active-expert slot, 64 output columns); wave w owns the 16
// columns h = 64*blockIdx.y + 16*w + l%16 and computes, on
// v_mfma_f32_16x16x32_bf16, y[token][h] for up to 16 of the expert's tokens
// at a time:
//   A (16 x 32): the tokens' fp32 SwiGLU activations as two bf16 parts,
//       hi = bf16(a) and lo = bf16(a - hi), one MFMA each (rows past the
//       expert's count are zeros), staged in LDS; lane l -> token l % 16, k
//       offset (l / 16) * 8.  hi + lo carries 16 significant bits, so the
//       product keeps the fp32-activation accuracy of this path;
//   B (16 x 32): the weights, lane l -> column l % 16 and the 8 units of
//       blocked-w2 block 4*ks + l/16 ([I/8][H][8]: 16 contiguous bytes, so
//       the 16 columns of one block are 256 contiguous bytes).
// The weights stream in batches of DN_KB k-steps with the next batch in
// flight.
constexpr int DN_KB = 8;                // k-steps of 32 per weight batch
constexpr int DN_COLS = 64;             // output columns per workgroup
constexpr int DN_ROWS = 16;             // tokens per MFMA pass

__global__ __launch_bounds__(256) void moe_down_mfma_kernel(
    const float* __restrict__ act, const uint16_t* __restrict__ w2b,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, int H, int I, float* __restrict__ y_slot) {
  extern __shared__ __attribute__((aligned(16))) uint16_t as[];  // hi, lo: [2][DN_ROWS][I + 8] bf16
  const int n_active = meta[1], e = active[blockIdx.x];  // both requested before the branch
  if (int(blockIdx.x) >= n_active) return;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 15, kq = lane >> 4;
  const int h = blockIdx.y * DN_COLS + wave * 16 + col;
  const int NS = I / QMOE_W2_BLOCK, KS = I / 32, ald = I + 8;
  const int nkb = (KS + DN_KB - 1) / DN_KB;
  // block kb = 4*ks + kq of column h: w2b[((e*NS + kb)*H + h)*8 .. +8]
  const uint16_t* wp = w2b + ((int64_t(e) * NS + kq) * H + h) * QMOE_W2_BLOCK;
  const int64_t ks_stride = int64_t(4) * H * QMOE_W2_BLOCK;
  u32x4 wa[2][DN_KB];
  auto load = [&](u32x4 (&dst)[DN_KB], int kb) {
#pragma unroll
    for (int u = 0; u < DN_KB; ++u) {
      const int ks = kb * DN_KB + u;
      dst[u] = ks < KS ? ld_stream(wp + ks * ks_stride) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  const int s0 = offsets[e], s1 = offsets[e + 1];
  for (int c0 = s0; c0 < s1; c0 += DN_ROWS) {
    const int n = min(DN_ROWS, s1 - c0);
    load(wa[0], 0);
    __syncthreads();  // the previous pass's fragment reads are done
    // act rows -> bf16 hi / lo parts in LDS; 4 floats per chunk, all loads
    // before the stores
    const int i4 = I / 4, total = DN_ROWS * i4;
    constexpr int SI = 6;
    for (int q0 = t; q0 < total; q0 += 256 * SI) {
      float4 v[SI];
#pragma unroll
      for (int u = 0; u < SI; ++u) {
        const int q = q0 + u * 256, j = q / i4, c = q - j * i4;
        v[u] = (q < total && j < n) ? reinterpret_cast<const float4*>(act + int64_t(c0 + j) * I)[c]
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (int u = 0; u < SI; ++u) {
        const int q = q0 + u * 256, j = q / i4, c = q - j * i4;
        if (q < total) {
          const uint32_t h01 = pack_bf16x2(v[u].x, v[u].y), h23 = pack_bf16x2(v[u].z, v[u].w);
          *reinterpret_cast<uint2*>(as + j * ald + c * 4) = make_uint2(h01, h23);
          *reinterpret_cast<uint2*>(as + (DN_ROWS + j) * ald + c * 4) =
              make_uint2(pack_bf16x2(v[u].x - bf16_lo(h01), v[u].y - bf16_hi(h01)),
                         pack_bf16x2(v[u].z - bf16_lo(h23), v[u].w - bf16_hi(h23)));
        }
      }
    }
    __syncthreads();
    f32x4 acc = f32x4{};
    const uint16_t* ap = as + col * ald + kq * 8;
    auto step = [&](const u32x4 (&src)[DN_KB], int kb) {
#pragma unroll
      for (int u = 0; u < DN_KB; ++u) {
        const int ks = kb * DN_KB + u;
        if (ks < KS) {
          const u32x4 ahi = *reinterpret_cast<const u32x4*>(ap + ks * 32);
          const u32x4 alo = *reinterpret_cast<const u32x4*>(ap + DN_ROWS * ald + ks * 32);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ahi),
                                                        __builtin_bit_cast(bf16x8, src[u]), acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, alo),
                                                        __builtin_bit_cast(bf16x8, src[u]), acc, 0, 0, 0);
        }
      }
    };
    for (int kb = 0; kb < nkb; kb += 2) {
      if (kb + 1 < nkb) load(wa[1], kb + 1);
      step(wa[0], kb);
      if (kb + 1 < nkb) {
        if (kb + 2 < nkb) load(wa[0], kb + 2);
        step(wa[1], kb + 1);
      }
    }
    // lane l holds column h and tokens kq*4 + 0..3
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = kq * 4 + r;
      if (j < n) y_slot[int64_t(c0 + j) * H + h] = acc[r];
    }
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
  const size_t shm1 = size_t(std::min<int64_t>(T * k, GU_TOK_CHUNK)) * H * 2;
  dim3 g1(nact, unsigned(I / 8));
  switch (H / 512) {
#define QMOE_GU(HC)                                                                                  \
  case HC:                                                                                           \
    hipLaunchKernelGGL((moe_gateup_gemv_kernel<HC, GU_TOK_CHUNK>), g1, dim3(256), shm1, s, x, w13,   \
                       offsets, slot_token, active, meta, int(H), int(I), act);                     \
    break;
    QMOE_GU(1)
    QMOE_GU(2)
    QMOE_GU(4)
    QMOE_GU(8)
#undef QMOE_GU
  }
  int rc = hip_status("moe experts (gate_up)");
  if (rc) return rc;
  const size_t shm2 = size_t(2 * DN_ROWS) * (I + 8) * 2;
  dim3 g2(nact, unsigned(H / DN_COLS));
  hipLaunchKernelGGL(moe_down_mfma_kernel, g2, dim3(256), shm2, s, act, w2, offsets, active, meta, int(H),
                     int(I), y_slot);
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
  QMOE_REQUIRE(w13 && w2 && offsets && active && meta && (T == 0 || (x && slot_token && act && y_slot)),
               "qmoe_moe_experts_gemv: null pointer");
  int rc = check_dec_shapes("qmoe_moe_experts_gemv", T, H, I, E, k);
  if (rc) return rc;
  if (T == 0) return QMOE_OK;
  return launch_experts(x, w13, w2, offsets, slot_token, active, meta, T, H, I, E, k, act, y_slot,
                        as_stream(stream));
}

