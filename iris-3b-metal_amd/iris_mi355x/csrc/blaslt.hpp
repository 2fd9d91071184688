// Plain BF16 GEMMs on hipBLASLt for the shapes listed in blaslt.hip (host-side interface).
#pragma once
#include "iris_common.hpp"

namespace iris {

// whether F.linear of these sizes (m rows, n outputs, k inputs) is one of the measured shapes
bool blaslt_wanted(int m, int n, int k);

// C[m, n] = A[m, k] W[n, k]^T (+ bias[n], FP32), BF16 output, on hipBLASLt; false when this path
// declines (set-up failed, or a new problem met during graph capture) and nothing was launched
bool blaslt_linear(const bf16* a, const bf16* w, const float* bias, bf16* c, int m, int n, int k, long lda, long ldb,
                   long ldc, hipStream_t stream);

}  // namespace iris
