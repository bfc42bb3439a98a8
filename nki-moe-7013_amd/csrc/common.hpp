// Shared device/host helpers for libqmoe (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "qmoe_capi.h"

namespace qmoe {

// ---------------------------------------------------------------- errors
// Records a printf-style message in the thread-local last-error buffer and
// returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Compute units of the current device (queried once per device; 0 when the
// query fails).
int current_device_cus();

inline int hip_status(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(QMOE_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
  return QMOE_OK;
}

#define QMOE_REQUIRE(cond, ...)                              \
  do {                                                       \
    if (!(cond)) return ::qmoe::fail(QMOE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(qmoe_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------- types
typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// Round-to-nearest-even float -> bf16 bit pattern (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}

// dot of 8 bf16 (packed in a u32x4) with 8 floats
__device__ __forceinline__ float dot8(const u32x4& w, const float* x) {
  float s = bf16_lo(w.x) * x[0];
  s = fmaf(bf16_hi(w.x), x[1], s);
  s = fmaf(bf16_lo(w.y), x[2], s);
  s = fmaf(bf16_hi(w.y), x[3], s);
  s = fmaf(bf16_lo(w.z), x[4], s);
  s = fmaf(bf16_hi(w.z), x[5], s);
  s = fmaf(bf16_lo(w.w), x[6], s);
  s = fmaf(bf16_hi(w.w), x[7], s);
  return s;
}

// acc + dot of 8 bf16 pairs, both operands packed (u32x4 = 8 bf16): four
// v_dot2c_f32_bf16 (each adds lo*lo + hi*hi to the fp32 accumulator; the
// bf16 products are exact in fp32).  No unpacking of either operand.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                         acc, false);
}
__device__ __forceinline__ float dot8_bf16(const u32x4& a, const u32x4& b, float acc) {
  acc = dot2_bf16(a.x, b.x, acc);
  acc = dot2_bf16(a.y, b.y, acc);
  acc = dot2_bf16(a.z, b.z, acc);
  return dot2_bf16(a.w, b.w, acc);
}

// ---------------------------------------------------------------- reductions (wave64)
// DPP-based: row_shr 1/2/4/8 leave each 16-lane row's total in its lane 15,
// row_bcast:15 / row_bcast:31 fold the rows so lane 63 holds the wave total,
// which readlane broadcasts.  Each step is a VALU op with a DPP modifier (a few
// cycles), unlike __shfl_xor, which goes through ds_bpermute.
#define QMOE_DPP_ROW_SHR(n) (0x110 + (n))
#define QMOE_DPP_ROW_BCAST15 0x142
#define QMOE_DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xf, BOUND_ZERO));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<QMOE_DPP_ROW_SHR(1), 0xf, true>(0.0f, v);
  v += dpp_mov<QMOE_DPP_ROW_SHR(2), 0xf, true>(0.0f, v);
  v += dpp_mov<QMOE_DPP_ROW_SHR(4), 0xf, true>(0.0f, v);
  v += dpp_mov<QMOE_DPP_ROW_SHR(8), 0xf, true>(0.0f, v);
  v += dpp_mov<QMOE_DPP_ROW_BCAST15, 0xa, false>(0.0f, v);
  v += dpp_mov<QMOE_DPP_ROW_BCAST31, 0xc, false>(0.0f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_SHR(1), 0xf, false>(v, v));
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_SHR(2), 0xf, false>(v, v));
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_SHR(4), 0xf, false>(v, v));
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_SHR(8), 0xf, false>(v, v));
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_BCAST15, 0xa, false>(v, v));
  v = fmaxf(v, dpp_mov<QMOE_DPP_ROW_BCAST31, 0xc, false>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Workgroup barrier for LDS traffic: waits for the wave's own LDS (and
// scalar) operations only.  __syncthreads() also waits for every global load
// and store the wave has outstanding (its fence), which puts a memory round
// trip on the critical path wherever a write-through store precedes it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The XCD (accelerator complex die, one of 8, each with its own L2) the
// calling wave runs on.
__device__ __forceinline__ int xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return int(v & 7);
}

// Non-temporal 16-byte load for weights that are streamed once.
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

}  // namespace qmoe
