// Projection GEMM dispatch: C[M,N] = A[M,K] . W[N,K]^T.
#include "common.hpp"
#include "kernels_extra.hpp"

namespace esp {

void launch_gemm(Dt wt, GemmEpi epi, const GemmArgs &a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return;
    launch_gemm_simple(wt, epi, a, s);
}

}  // namespace esp
