// Residual GEMMs through hipBLASLt (blaslt.cpp).
#pragma once

#include "kernels.hpp"

namespace s1 {

// Rows from which the model hands its unsplit residual GEMMs to hipBLASLt (setting blaslt).
constexpr int LT_MIN_M = 2048;

// C[M, N] f32 += A[M, K] . W[N, K]^T (+ bias[N]), the arithmetic of gemm_launch with EPI_RESID
// and no split, enqueued on `st`. Returns false, enqueuing nothing, when hipBLASLt offers no
// algorithm without workspace for the shape (the caller then runs gemm_launch). Thread-safe.
bool lt_resid_gemm(const GemmArgs& g, hipStream_t st);

}  // namespace s1
