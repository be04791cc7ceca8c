// Batched prefill: Y[m] = W X[m] with gemv_quant semantics per row.
// First version: one decode-GEMV launch per activation row.
#include "uq_internal.h"

namespace uq {

hipError_t launch_gemm(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s) {
    for (int m = 0; m < M; m++) {
        hipError_t e = launch_gemv(w, X + (size_t)m * w.dim_in, Y + (size_t)m * w.dim_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace uq
