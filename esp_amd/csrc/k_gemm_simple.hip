// Generic tiled projection GEMM, C[M,N] = A[M,K] . W[N,K]^T with f32
// accumulation on the vector ALUs. It serves the f32 weight format (where
// every product must stay f32) and shapes the MFMA kernel does not tile.
#include "common.hpp"
#include "dev.hpp"

namespace esp {

constexpr int SG_BM = 64, SG_BN = 64, SG_BK = 16;

template <typename AT, typename WT, int EPI>
__global__ void __launch_bounds__(256) gemm_simple_k(GemmArgs a) {
    constexpr int NW = EPI == GEMM_SWIGLU ? 2 : 1;
    __shared__ float As[SG_BK][SG_BM + 4];
    __shared__ float Ws[NW][SG_BK][SG_BN + 4];
    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    const int n0 = blockIdx.x * SG_BN;
    int m0, mend, grp;
    if (!group_tile(a.grp_offs, a.grp_n, a.M, blockIdx.y, SG_BM, m0, mend, grp)) return;
    const AT *A = (const AT *)a.a;
    const size_t woff = (size_t)grp * a.grp_w_stride;
    const WT *Wm[2] = {(const WT *)a.w + woff, (const WT *)a.w2 + woff};
    float acc[NW][4][4];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[w][i][j] = 0.f;
    for (int k0 = 0; k0 < a.K; k0 += SG_BK) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int e = tid + i * 256;  // 0..1023
            int r = e / SG_BK, kk = e % SG_BK;
            int gm = m0 + r, gk = k0 + kk;
            float av = 0.f;
            if (gm < mend && gk < a.K) {
                size_t ai = (size_t)gm * a.K + gk;
                av = a.a_lo ? bf2f(((const uint16_t *)a.a)[ai]) + bf2f(((const uint16_t *)a.a_lo)[ai])
                            : ld(A, ai);
            }
            As[kk][r] = av;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                int gn = n0 + r;
                Ws[w][kk][r] = (gn < a.N && gk < a.K) ? ld(Wm[w], (size_t)gn * a.K + gk) : 0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < SG_BK; ++kk) {
            float av[4], wv[NW][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int j = 0; j < 4; ++j) wv[w][j] = Ws[w][kk][tx * 4 + j];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[w][i][j] += av[i] * wv[w][j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int gm = m0 + ty * 4 + i;
        if (gm >= mend) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int gn = n0 + tx * 4 + j;
            if (gn >= a.N) continue;
            if (EPI == GEMM_SWIGLU) {
                float y = silu(acc[0][i][j]) * acc[NW - 1][i][j];
                size_t ci = (size_t)gm * a.ldc + gn;
                if (a.c_lo) {
                    uint16_t h = f2bf(y);
                    ((uint16_t *)a.c)[ci] = h;
                    ((uint16_t *)a.c_lo)[ci] = f2bf(y - bf2f(h));
                } else {
                    st((AT *)a.c, ci, y);
                }
            } else {
                float v = a.bias ? acc[0][i][j] + a.bias[gn] : acc[0][i][j];
                float *c = (float *)a.c + (size_t)gm * a.ldc + gn;
                if (EPI == GEMM_RESIDUAL) *c = *c + v;
                else *c = v;
            }
        }
    }
}

template <typename AT, typename WT>
static void simple_dispatch(GemmEpi epi, const GemmArgs &a, hipStream_t s) {
    dim3 grid((a.N + SG_BN - 1) / SG_BN,
              (a.M + SG_BM - 1) / SG_BM + (a.grp_offs ? a.grp_n : 0));
    if (epi == GEMM_STORE) gemm_simple_k<AT, WT, GEMM_STORE><<<grid, 256, 0, s>>>(a);
    else if (epi == GEMM_RESIDUAL) gemm_simple_k<AT, WT, GEMM_RESIDUAL><<<grid, 256, 0, s>>>(a);
    else gemm_simple_k<AT, WT, GEMM_SWIGLU><<<grid, 256, 0, s>>>(a);
}

void launch_gemm_simple(Dt wt, GemmEpi epi, const GemmArgs &a, hipStream_t s) {
    if (wt == DT_BF16) simple_dispatch<float, uint16_t>(epi, a, s);
    else simple_dispatch<float, float>(epi, a, s);
}

}  // namespace esp
