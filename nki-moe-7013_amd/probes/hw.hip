// Measurement probes (not part of the product ABI): hardware ceilings that the
// kernel designs are held against.  bench.py runs them and reports the
// results in its `measured_peaks`.
//
//   qmoe_probe_empty    a kernel that does nothing: back-to-back launches of
//                       it in a HIP graph give the cost of a kernel boundary.
//   qmoe_probe_stream   every workgroup (256 threads) reads its contiguous
//                       share of a buffer with 16-byte loads, 8 in flight per
//                       thread: the HBM read rate at a given workgroup count.
//   qmoe_probe_l2       every wave reads 8 KB runs of a 512 KB buffer (L2
//                       resident after the first pass), into VGPRs or into
//                       LDS through `buffer_load_dwordx4 ... lds` (the DMA
//                       the GEMM pipelines use): the L2 -> CU rate.
// All offsets stay inside the buffers; the only global stores are guarded by
// conditions the data never meets (they keep the loads live).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t L2_BYTES = 512 * 1024;

__global__ void empty_kernel() {}

__global__ __launch_bounds__(256) void stream_kernel(const uint8_t* __restrict__ src, int64_t bytes,
                                                     unsigned* __restrict__ out) {
  // workgroup share: whole 4 KB pages, the last workgroup takes the rest
  const int64_t pages = bytes >> 12, per = (pages + gridDim.x - 1) / gridDim.x;
  const int64_t p0 = int64_t(blockIdx.x) * per, p1 = p0 + per < pages ? p0 + per : pages;
  u32x4 acc{0u, 0u, 0u, 0u};
  // one round: 8 loads per thread = 8 x 4 KB = 32 KB per workgroup
  for (int64_t p = p0; p < p1; p += 8) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t off = (p + j) * 4096 + threadIdx.x * 16;
      v[j] = p + j < p1 ? *reinterpret_cast<const u32x4*>(src + off) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) out[blockIdx.x] = 1u;
}

__device__ __forceinline__ i32x4 make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(p);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(b)));
  r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(b >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane(int(bytes));
  r.w = 0x00020000;
  return r;
}

// 64 lanes x 16 bytes from rsrc + voff (per lane) into LDS at M0 + 16 * lane
__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voff, i32x4 rsrc) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(rsrc)
      : "memory");
}

// Each wave: `iters` rounds of 8 x 1 KB reads (8 KB) at an 8 KB-aligned run of
// the buffer; DMA into a private two-round LDS ring (16 KB per wave) with one
// round in flight, or loads into VGPRs.
template <bool DMA>
__global__ __launch_bounds__(256) void l2_kernel(const uint8_t* __restrict__ src, int iters,
                                                 unsigned* __restrict__ out) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const uint32_t base = (blockIdx.x * 4096u + uint32_t(wave) * 1024u) % L2_BYTES;
  if constexpr (DMA) {
    const i32x4 r = make_rsrc(src, L2_BYTES);
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem)) + uint32_t(wave) * 16384u;
    for (int it = 0; it < iters; ++it) {
      const uint32_t b = (base + uint32_t(it) * 8192u) % L2_BYTES;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        dma16(lds0 + uint32_t(it & 1) * 8192u + j * 1024u, (b + j * 1024u + lane * 16u) % L2_BYTES, r);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (smem[threadIdx.x] == 0xAB && smem[threadIdx.x + 1] == 0xCD) out[blockIdx.x] = 1u;
  } else {
    u32x4 acc{0u, 0u, 0u, 0u};
    for (int it = 0; it < iters; ++it) {
      const uint32_t b = (base + uint32_t(it) * 8192u) % L2_BYTES;
      u32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = *reinterpret_cast<const u32x4*>(src + (b + j * 1024u + lane * 16u) % L2_BYTES);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc ^= v[j];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) out[blockIdx.x] = 1u;
  }
}
}  // namespace

// Returns 0, or the HIP error code of the launch (1 for bad arguments).
extern "C" int qmoe_probe_empty(int blocks, void* stream) {
  if (blocks <= 0) return 1;
  hipLaunchKernelGGL(empty_kernel, dim3(unsigned(blocks)), dim3(64), 0, reinterpret_cast<hipStream_t>(stream));
  return int(hipGetLastError());
}

// src: `bytes` readable bytes (a multiple of 4096); out: unsigned [blocks].
extern "C" int qmoe_probe_stream(const void* src, int64_t bytes, int blocks, unsigned* out, void* stream) {
  if (!src || !out || blocks <= 0 || bytes <= 0 || bytes % 4096) return 1;
  hipLaunchKernelGGL(stream_kernel, dim3(unsigned(blocks)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint8_t*>(src), bytes, out);
  return int(hipGetLastError());
}

// src: 512 KB; out: unsigned [blocks].  Bytes read: blocks * 4 waves * iters * 8 KB.
extern "C" int qmoe_probe_l2(const void* src, int blocks, int iters, int dma, unsigned* out, void* stream) {
  if (!src || !out || blocks <= 0 || iters <= 0) return 1;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dma) {
    static const bool attr = [] {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(l2_kernel<true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
      return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(l2_kernel<true>, dim3(unsigned(blocks)), dim3(256), 65536, s,
                       reinterpret_cast<const uint8_t*>(src), iters, out);
  } else {
    hipLaunchKernelGGL(l2_kernel<false>, dim3(unsigned(blocks)), dim3(256), 0, s,
                       reinterpret_cast<const uint8_t*>(src), iters, out);
  }
  return int(hipGetLastError());
}
