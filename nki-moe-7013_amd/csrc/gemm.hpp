// Internal launcher shared by the entry points that need a plain GEMM.
#pragma once
#include "common.hpp"

namespace qmoe {
// C = A . B^T (see qmoe_gemm in qmoe_capi.h).
int gemm_launch(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N,
                int64_t K, int mode, void* C, int64_t ldc, hipStream_t s);
// Split-K partial products part[slice][M][N] (f32) of C = A . B^T without the
// reduction: *splits = the slice count launched, 0 when the problem is not
// split (too many tiles or K too short) or part_bytes is too small (nothing
// launched; the caller computes C another way).  gemm_splitk_bytes = the
// workspace such a call needs (0: never split).
int gemm_splitk_slices(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N, int64_t K,
                       float* part, int64_t part_bytes, int* splits, hipStream_t s);
int64_t gemm_splitk_bytes(int64_t M, int64_t N, int64_t K);
// C[N] = bf16(rmsnorm(h)) . B^T for one fp32 row h (see qmoe_gemv_rmsnorm).
int gemv_rmsnorm_launch(const float* h, const uint16_t* rms_w, float eps, const uint16_t* B, int64_t N,
                        int64_t K, int mode, void* C, hipStream_t s);
}  // namespace qmoe

namespace qmoe {
// Router logits (GEMM) + per-token top-k (see qmoe_router_topk_ws; a null
// workspace: no split-K).
int router_launch(const uint16_t* x, const uint16_t* w_router, const float* bias, int64_t T,
                  int64_t H, int64_t E, int64_t k, int32_t* topk_idx, float* topk_w, float* logits,
                  void* workspace, int64_t workspace_bytes, hipStream_t s);
// Dispatch metadata (see qmoe_moe_permute).
int permute_launch(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E, int64_t tile_m,
                   int64_t max_tiles, int32_t* counts, int32_t* offsets, int32_t* slot_token,
                   int32_t* token_slot, int32_t* active, int32_t* tiles, int32_t* meta,
                   hipStream_t s);
}  // namespace qmoe
