// Token embedding gather and greedy argmax over the lm_head logits: the two
// steps either side of the layer stack in every decode step.
//
//   embed_gather_kernel   out[i] = float(table[ids[i]]) (bf16 row -> fp32
//                         residual stream).  An id outside [0, V) writes a
//                         zero row and raises err[0] = 1: nothing traps, and
//                         the caller checks the flag on the host.
//   argmax_partial_kernel / argmax_final_kernel
//                         greedy token per row in two launches: ARGMAX_PARTS
//                         workgroups per row each reduce a contiguous slice
//                         to (value, index), then one workgroup per row
//                         reduces the parts.  No semaphores and no memset, so
//                         the pair replays correctly inside a HIP graph.
//                         Ties resolve to the lowest index and NaN ranks
//                         above every number (first NaN wins), as
//                         torch.argmax does.
#include "common.hpp"

namespace qmoe {

constexpr int ARGMAX_PARTS = 256;
constexpr int ARGMAX_THREADS = 256;

// Order-preserving key: larger value -> larger key; NaN above +inf.  Packed
// with the complemented index so that a max over the 64-bit key picks the
// largest value and, among equal values, the lowest index.
__device__ __forceinline__ uint64_t argmax_key(float v, int64_t idx) {
  uint32_t b = __float_as_uint(v);
  uint32_t ord;
  if (v != v)
    ord = 0xffffffffu;
  else
    ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (uint64_t(ord) << 32) | uint64_t(~uint32_t(idx));
}

__device__ __forceinline__ uint64_t u64max(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t block_max_u64(uint64_t k, uint64_t* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = uint32_t(k), hi = uint32_t(k >> 32);
    const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(hi), o, 64))) << 32) |
                           uint32_t(__shfl_xor(int(lo), o, 64));
    k = u64max(k, other);
  }
  if (lane == 0) red[wave] = k;
  __syncthreads();
  uint64_t m = red[0];
  for (int w = 1; w < int(blockDim.x) / 64; ++w) m = u64max(m, red[w]);
  return m;
}

__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_partial_kernel(const float* __restrict__ x,
                                                                        int64_t n, int64_t ldx,
                                                                        uint64_t* __restrict__ part) {
  __shared__ uint64_t red[ARGMAX_THREADS / 64];
  const int row = blockIdx.y, p = blockIdx.x;
  const int64_t chunk = (n + ARGMAX_PARTS - 1) / ARGMAX_PARTS;
  const int64_t b0 = int64_t(p) * chunk, b1 = min(n, b0 + chunk);
  const float* xr = x + int64_t(row) * ldx;
  uint64_t k = 0;  // below every real key (index complement of -1 never wins)
  for (int64_t i = b0 + threadIdx.x; i < b1; i += ARGMAX_THREADS) k = u64max(k, argmax_key(xr[i], i));
  k = block_max_u64(k, red);
  if (threadIdx.x == 0) part[int64_t(row) * ARGMAX_PARTS + p] = k;
}

__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_final_kernel(const uint64_t* __restrict__ part,
                                                                      int64_t* __restrict__ out) {
  __shared__ uint64_t red[ARGMAX_THREADS / 64];
  const int row = blockIdx.x;
  uint64_t k = 0;
  for (int i = threadIdx.x; i < ARGMAX_PARTS; i += ARGMAX_THREADS)
    k = u64max(k, part[int64_t(row) * ARGMAX_PARTS + i]);
  k = block_max_u64(k, red);
  if (threadIdx.x == 0) out[row] = int64_t(~uint32_t(k & 0xffffffffu));
}

__global__ __launch_bounds__(256) void embed_gather_kernel(const uint16_t* __restrict__ table,
                                                           int64_t V, int H,
                                                           const int64_t* __restrict__ ids,
                                                           float* __restrict__ out,
                                                           int32_t* __restrict__ err) {
  const int i = blockIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < V;
  if (!ok && threadIdx.x == 0) err[0] = 1;
  const uint16_t* src = table + (ok ? id : 0) * int64_t(H);
  float* dst = out + int64_t(i) * H;
  for (int c = threadIdx.x; c < H / 4; c += 256) {
    const uint2 v = reinterpret_cast<const uint2*>(src)[c];
    reinterpret_cast<float4*>(dst)[c] =
        ok ? make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y)) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int64_t qmoe_argmax_workspace(int64_t rows) {
  return rows < 0 ? -1 : rows * ARGMAX_PARTS * int64_t(sizeof(uint64_t));
}

extern "C" int qmoe_argmax(const float* x, int64_t rows, int64_t n, int64_t ldx, void* workspace,
                           int64_t workspace_bytes, int64_t* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(rows == 0 || (x && workspace && out), "qmoe_argmax: null pointer");
  QMOE_REQUIRE(rows >= 0 && rows < 65536 && n > 0 && n < (1ll << 31) && ldx >= n,
               "qmoe_argmax: bad rows/n/ldx");
  QMOE_REQUIRE(workspace_bytes >= qmoe_argmax_workspace(rows), "qmoe_argmax: workspace too small");
  if (rows == 0) return QMOE_OK;
  hipStream_t s = as_stream(stream);
  uint64_t* part = static_cast<uint64_t*>(workspace);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(ARGMAX_PARTS, unsigned(rows)), dim3(ARGMAX_THREADS), 0,
                     s, x, n, ldx, part);
  if (int rc = hip_status("qmoe_argmax(partial)")) return rc;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(unsigned(rows)), dim3(ARGMAX_THREADS), 0, s, part, out);
  return hip_status("qmoe_argmax(final)");
}

extern "C" int qmoe_embed(const qmoe_bf16* table, int64_t V, int64_t H, const int64_t* ids, int64_t n,
                          float* out, int32_t* err, qmoe_stream_t stream) {
  QMOE_REQUIRE(table && err && (n == 0 || (ids && out)), "qmoe_embed: null pointer");
  QMOE_REQUIRE(V > 0 && H > 0 && H % 4 == 0 && H < (1 << 24), "qmoe_embed: bad V/H (H %% 4 == 0)");
  QMOE_REQUIRE(n >= 0 && n < (1ll << 31), "qmoe_embed: bad n");
  if (n == 0) return QMOE_OK;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(unsigned(n)), dim3(256), 0, as_stream(stream), table, V,
                     int(H), ids, out, err);
  return hip_status("qmoe_embed");
}
