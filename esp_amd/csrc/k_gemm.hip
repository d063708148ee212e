// Projection GEMM dispatch: C[M,N] = A[M,K] . W[N,K]^T.
#include "common.hpp"
#include "kernels_extra.hpp"

namespace esp {

bool gemm_mfma_ok(Dt wt, const GemmArgs &a);
void launch_gemm_mfma(GemmEpi epi, const GemmArgs &a, float *ws, size_t ws_bytes, hipStream_t s);

// bf16 weights go to the matrix cores (activations split into bf16 hi + lo);
// f32 weights and unaligned shapes use the vector-ALU kernel.
void launch_gemm(Dt wt, GemmEpi epi, const GemmArgs &a, hipStream_t s) {
    if (a.defer_splits) *a.defer_splits = 0;
    if (a.M <= 0 || a.N <= 0) return;
    if (gemm_mfma_ok(wt, a)) launch_gemm_mfma(epi, a, a.ws, a.ws ? a.ws_bytes : 0, s);
    else if (a.kdup) fail(ESP_BACKEND, "doubled-K GEMM: operands outside the matrix-core form");
    else launch_gemm_simple(wt, epi, a, s);
}

}  // namespace esp
