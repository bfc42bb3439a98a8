// Internal launcher shared by the entry points that need a plain GEMM.
#pragma once
#include "common.hpp"

namespace qmoe {
// C = A . B^T (see qmoe_gemm in qmoe_capi.h).
int gemm_launch(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t M, int64_t N,
                int64_t K, int mode, void* C, int64_t ldc, hipStream_t s);
}  // namespace qmoe
