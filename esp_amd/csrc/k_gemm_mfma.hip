// Prefill projection GEMM on the CDNA4 matrix cores:
//   C[M,N] (f32) = A[M,K] (f32 activations) . W[N,K]^T (bf16 weights)
// The activations arrive split into two bf16 planes, hi = bf16(a) and
// lo = bf16(a - hi) (a = hi + lo + O(2^-17 a)), written that way by the
// kernel that produced them; both parts are multiplied against the same bf16
// weight fragment with v_mfma_f32_32x32x16_bf16, accumulating in f32. Every
// product is exact, so the result keeps f32-level accuracy on bf16 MFMA.
//
// Block tile 128 x (NB x BN) x 32, four waves in a 2 x 2 arrangement; each
// wave owns 64 rows x NB*BN/2 weight columns. The wide form has 128 columns
// per wave (2 x 4 MFMA blocks of 32 x 32): BN = 256 for one weight matrix,
// or BN = 128 each for the gate and up matrices of SWIGLU, whose tiles share
// the A fragments; it keeps LDS reads at 512 bytes per MFMA (A costs 4 bytes
// per element as two planes). Grids too small to fill the chip with it use
// the narrow form (half the columns per block). A and W tiles are staged through LDS (rows padded to
// 80 bytes) from register prefetches issued one k-tile ahead. Epilogues:
// STORE (+bias), RESIDUAL (+=), SWIGLU (out = silu(g) * u).
#include <cstdlib>
#include <utility>

#include "common.hpp"
#include "dev.hpp"
#include "kernels_extra.hpp"

namespace esp {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v_t __attribute__((ext_vector_type(2)));

constexpr int MF_BM = 128, MF_BK = 32, MF_LD = MF_BK + 8;
constexpr int MF_CPR = MF_BK / 8;  // 16-byte chunks per tile row
constexpr int MF_A_ELEMS = MF_BM * MF_LD;  // one A plane (bf16) per buffer
// NJ = 32-column MFMA blocks per wave and weight matrix; BN = 64 * NJ
template <int NJ> constexpr int mf_b_elems() { return 64 * NJ * MF_LD; }

template <int NB, int NJ> constexpr size_t mfma_lds_bytes() {
    return (size_t)(2 * MF_A_ELEMS + NB * mf_b_elems<NJ>()) * 2;
}

// Split-K: blockIdx.z = k-split; each split writes raw f32 sums for its K
// range to ws[z][M][N] (x NB planes) and mfma_reduce_k adds the splits in
// order and applies the epilogue, so results do not depend on timing.
constexpr int MF_PARTIAL = 16;

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
    return (uint32_t)lo | ((uint32_t)hi << 16);
}

// XCD-aware tile order: workgroups are dispatched round-robin over the 8
// XCDs (linear id % 8), so XCD x is given the contiguous tile range
// [x*per, (x+1)*per) of a column-major tile order (row tiles fastest). Each
// weight tile is then fetched into one XCD's L2 and reused by every row tile
// that XCD runs, instead of being pulled into all eight L2s.
constexpr int MF_XCDS = 8;

template <int EPI, int NB, int NJ>
__global__ void __launch_bounds__(256, 2) gemm_mfma_k(GemmArgs g, float *ws, int k_per_split,
                                                     int mt, int nt) {
    constexpr int BN = 64 * NJ, B_ELEMS = mf_b_elems<NJ>();
    extern __shared__ uint16_t lds[];
    uint16_t *sA = lds;                          // [hi/lo][BM*LD]
    uint16_t *sB = lds + 2 * MF_A_ELEMS;         // [nb][BN*LD]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int total = mt * nt, per = (total + MF_XCDS - 1) / MF_XCDS;
    const int tile = (blockIdx.x % MF_XCDS) * per + blockIdx.x / MF_XCDS;
    if (tile >= total) return;
    int m0, M, grp;  // M: end of this tile's group (rows >= M are not computed)
    if (!group_tile(g.grp_offs, g.grp_n, g.M, tile % mt, MF_BM, m0, M, grp)) return;
    const int n0 = (tile / mt) * BN;
    const size_t woff = (size_t)grp * g.grp_w_stride;
    const uint16_t *Ah = (const uint16_t *)g.a, *Al = (const uint16_t *)g.a_lo;
    const uint16_t *Wm[2] = {(const uint16_t *)g.w + woff, (const uint16_t *)g.w2 + woff};
    const int N = g.N, K = g.K;

    f32x16_t acc[NB][2][NJ];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[b][i][j][e] = 0.f;

    constexpr int ACH = MF_BM * MF_CPR / 256, BCH = BN * MF_CPR / 256;  // chunks per thread
    u32x4v_t ra[2][ACH];  // [hi/lo][chunk]
    u32x4v_t rb[NB][BCH];
    const int kbeg = blockIdx.z * k_per_split;
    const int kend = min(K, kbeg + k_per_split);
    auto load_tile = [&](int kt) {
        const int kb = kbeg + kt * MF_BK;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int i = 0; i < ACH; ++i) {
                int idx = tid + 256 * i;  // chunks of 8 bf16 (128 x BK tile)
                int row = idx / MF_CPR, k = kb + (idx % MF_CPR) * 8;
                int gm = m0 + row;
                const uint16_t *src = p ? Al : Ah;
                if (gm < M && k + 7 < kend) {
                    ra[p][i] = *(const u32x4v_t *)(src + (size_t)gm * K + k);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = (gm < M && k + q < kend) ? src[(size_t)gm * K + k + q] : 0;
                    ra[p][i] = u32x4v_t{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                                        pack2(e[6], e[7])};
                }
            }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < BCH; ++i) {
                int idx = tid + 256 * i;  // chunks of 8 bf16 (BN x BK tile)
                int row = idx / MF_CPR, k = kb + (idx % MF_CPR) * 8;
                int gn = n0 + row;
                if (gn < N && k + 7 < kend) {
                    rb[b][i] = __builtin_nontemporal_load(
                        (const u32x4v_t *)(Wm[b] + (size_t)gn * K + k));
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = (gn < N && k + q < kend) ? Wm[b][(size_t)gn * K + k + q] : 0;
                    rb[b][i] = u32x4v_t{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                                        pack2(e[6], e[7])};
                }
            }
    };
    auto store_tile = [&]() {
        uint16_t *ah = sA;
        uint16_t *al = sA + MF_A_ELEMS;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int i = 0; i < ACH; ++i) {
                int idx = tid + 256 * i;
                int row = idx / MF_CPR, k = (idx % MF_CPR) * 8;
                *(u32x4v_t *)((p ? al : ah) + row * MF_LD + k) = ra[p][i];
            }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            uint16_t *bb = sB + b * B_ELEMS;
#pragma unroll
            for (int i = 0; i < BCH; ++i) {
                int idx = tid + 256 * i;
                int row = idx / MF_CPR, k = (idx % MF_CPR) * 8;
                *(u32x4v_t *)(bb + row * MF_LD + k) = rb[b][i];
            }
        }
    };
    auto compute = [&]() {
        const uint16_t *ah = sA;
        const uint16_t *al = sA + MF_A_ELEMS;
#pragma unroll
        for (int ks = 0; ks < MF_BK / 16; ++ks) {
            const int koff = ks * 16 + (lane >> 5) * 8;
            bf16x8_t fh[2], fl[2], fb[NB][NJ];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                int r = wm * 64 + i * 32 + (lane & 31);
                fh[i] = *(const bf16x8_t *)(ah + r * MF_LD + koff);
                fl[i] = *(const bf16x8_t *)(al + r * MF_LD + koff);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    int r = wn * (BN / 2) + j * 32 + (lane & 31);
                    fb[b][j] = *(const bf16x8_t *)(sB + b * B_ELEMS + r * MF_LD + koff);
                }
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[i], fb[b][j], acc[b][i][j], 0, 0, 0);
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[i], fb[b][j], acc[b][i][j], 0, 0, 0);
                    }
        }
    };

    // single LDS buffer (more blocks per CU hide latency); the next tile's
    // global loads are in flight in registers while this tile computes
    const int KT = (kend - kbeg + MF_BK - 1) / MF_BK;
    if (KT > 0) load_tile(0);
    for (int kt = 0; kt < KT; ++kt) {
        store_tile();
        __syncthreads();
        if (kt + 1 < KT) load_tile(kt + 1);
        compute();
        __syncthreads();
    }

    // epilogue: lane holds column (lane & 31) of each 32 x 32 block, rows
    // (e / 4) * 8 + (lane >> 5) * 4 + e % 4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
            if (col >= N) continue;
            if (EPI == MF_PARTIAL) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                    if (row >= M) continue;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        ws[(((size_t)blockIdx.z * NB + b) * g.M + row) * N + col] = acc[b][i][j][e];
                }
                continue;
            }
            const float bias = (EPI != GEMM_SWIGLU && g.bias) ? g.bias[col] : 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                if (row >= M) continue;
                float *c = (float *)g.c + (size_t)row * g.ldc + col;
                if (EPI == GEMM_SWIGLU) {
                    const float y = silu(acc[0][i][j][e]) * acc[NB - 1][i][j][e];
                    if (g.c_lo) {
                        const size_t ci = (size_t)row * g.ldc + col;
                        uint16_t h = f2bf(y);
                        ((uint16_t *)g.c)[ci] = h;
                        ((uint16_t *)g.c_lo)[ci] = f2bf(y - bf2f(h));
                    } else {
                        *c = y;
                    }
                } else {
                    float v = g.bias ? acc[0][i][j][e] + bias : acc[0][i][j][e];
                    if (EPI == GEMM_RESIDUAL) *c = *c + v;
                    else *c = v;
                }
            }
        }
}

template <int EPI, int NB>
__global__ void __launch_bounds__(256) mfma_reduce_k(GemmArgs g, const float *ws, int splits) {
    const size_t MN = (size_t)g.M * g.N;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < MN;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(idx / g.N), col = (int)(idx % g.N);
        float v[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            // up to eight split partials in flight per batch, summed in split order
            float t = 0.f;
            if (splits <= 4) {
                for (int z = 0; z < splits; ++z) t += ws[((size_t)z * NB + b) * MN + idx];
                v[b] = t;
                continue;
            }
            for (int z0 = 0; z0 < splits; z0 += 8) {
                float pz[8];
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    pz[q] = z0 + q < splits ? ws[((size_t)(z0 + q) * NB + b) * MN + idx] : 0.f;
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (z0 + q < splits) t += pz[q];
            }
            v[b] = t;
        }
        float *c = (float *)g.c + (size_t)row * g.ldc + col;
        if (EPI == GEMM_SWIGLU) {
            const float y = silu(v[0]) * v[NB - 1];
            if (g.c_lo) {
                const size_t ci = (size_t)row * g.ldc + col;
                uint16_t h = f2bf(y);
                ((uint16_t *)g.c)[ci] = h;
                ((uint16_t *)g.c_lo)[ci] = f2bf(y - bf2f(h));
            } else {
                *c = y;
            }
        } else {
            float y = g.bias ? v[0] + g.bias[col] : v[0];
            if (EPI == GEMM_RESIDUAL) *c = *c + y;
            else *c = y;
        }
    }
}

// mfma_reduce_k over four consecutive columns per thread (N and ldc
// multiples of 4): 16-byte partial loads, every split's load of the group in
// flight before the sums, and the same per-element arithmetic (splits
// summed from 0 in split order, then the epilogue).
template <int EPI, int NB>
__global__ void __launch_bounds__(256) mfma_reduce4_k(GemmArgs g, const float *ws, int splits) {
    const size_t MN = (size_t)g.M * g.N, MN4 = MN / 4;
    for (size_t q = blockIdx.x * (size_t)blockDim.x + threadIdx.x; q < MN4;
         q += (size_t)gridDim.x * blockDim.x) {
        const size_t idx = q * 4;
        const int row = (int)(idx / g.N), col = (int)(idx % g.N);
        float4 v[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int z0 = 0; z0 < splits; z0 += 8) {
                float4 pz[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < splits) pz[u] = *(const float4 *)(ws + ((size_t)(z0 + u) * NB + b) * MN + idx);
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < splits) {
                        t.x += pz[u].x;
                        t.y += pz[u].y;
                        t.z += pz[u].z;
                        t.w += pz[u].w;
                    }
            }
            v[b] = t;
        }
        const size_t ci = (size_t)row * g.ldc + col;
        if (EPI == GEMM_SWIGLU) {
            const float y[4] = {silu(v[0].x) * v[NB - 1].x, silu(v[0].y) * v[NB - 1].y,
                                silu(v[0].z) * v[NB - 1].z, silu(v[0].w) * v[NB - 1].w};
            if (g.c_lo) {
                uint16_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    h[e] = f2bf(y[e]);
                    l[e] = f2bf(y[e] - bf2f(h[e]));
                }
                *(uint2 *)((uint16_t *)g.c + ci) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
                *(uint2 *)((uint16_t *)g.c_lo + ci) = make_uint2(pack2(l[0], l[1]), pack2(l[2], l[3]));
            } else {
                *(float4 *)((float *)g.c + ci) = make_float4(y[0], y[1], y[2], y[3]);
            }
        } else {
            float4 y = v[0];
            if (g.bias) {
                const float4 bb = *(const float4 *)(g.bias + col);
                y.x += bb.x;
                y.y += bb.y;
                y.z += bb.z;
                y.w += bb.w;
            }
            float4 *c = (float4 *)((float *)g.c + ci);
            if (EPI == GEMM_RESIDUAL) {
                const float4 o = *c;
                y.x = o.x + y.x;
                y.y = o.y + y.y;
                y.z = o.z + y.z;
                y.w = o.w + y.w;
            }
            *c = y;
        }
    }
}

// ---------------------------------------------------------------------------
// Streamed form (K a multiple of 32): the same 128 x 256 block tile, but the
// A planes and weight rows go global -> LDS directly (global_load_lds, 16
// bytes per lane) through a ring of LDS_STAGES stages of 32 keys, issued
// LDS_STAGES - 1 stages ahead, so no registers stage the tiles and global
// latency is covered by three stages of MFMA work. One barrier per stage.
// Each tile row is 64 bytes (four 16-byte chunks); chunk c of row r sits at
// slot c ^ ((r >> 2) & 3). ds_read_b128 serves 16 lanes per cycle from 64
// four-byte banks, so the 16 rows a quarter-wave reads (same chunk) must
// land on 16 distinct 16-byte slots mod 256 bytes; rows r, r+4, r+8, r+12
// share r & 3 and the XOR separates them (measured: no bank conflicts). Rows past M or N re-read the
// last valid row (their results are dropped by the epilogue).
constexpr int LS_BK = 32;
constexpr int LS_ROWB = LS_BK * 2;                 // bytes per tile row

// BMW waves along M (block rows 64 * BMW) x 2 along N, BROWS weight rows
// per stage (all matrices), STG stages: 128-row blocks with 256 weight rows
// keep two stages (64 KB) so two blocks share a CU; 256-row blocks (eight
// waves) keep three (144 KB); one row tile (M <= 128) uses 64 weight rows
// per matrix and three stages, and 129-1023 rows 128 weight rows per
// matrix and three stages (the stage count and tile widths for these row
// ranges were chosen by measurement on the C5 and C2 shapes).
template <int BMW, int BROWS = 256, int STG = (BMW == 2 ? 2 : 3)> struct LsForm {
    static constexpr int BM = 64 * BMW, NT = 128 * BMW;
    static constexpr int A = BM * LS_ROWB;                       // one A plane per stage
    static constexpr int STAGE = 2 * A + BROWS * LS_ROWB;
    static constexpr int STAGES = STG;
    static constexpr size_t LDS = (size_t)STAGES * STAGE;
    static constexpr int QB = BROWS / (32 * BMW);                // weight loads per wave and stage
    static constexpr int LPS = 4 + QB;                           // loads per wave and stage
    static_assert(QB >= 1 && QB * 32 * BMW == BROWS, "weight rows must split over the waves");
};

// s_waitcnt immediate for vmcnt(n) (n & 15 in bits 3:0, n >> 4 in bits 15:14)
constexpr int vm_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

__device__ __forceinline__ int ls_swz(int r) { return (r >> 2) & 3; }

typedef const void __attribute__((address_space(1))) *gptr_t;
typedef void __attribute__((address_space(3))) *lptr_t;

// PROD: NP more waves per block issue every direct load of the tiles (the
// 2 x BMW MFMA waves issue no vector memory instructions), each a fixed
// 1 / NP of every stage's load instructions: a producer waits for its loads
// of a stage, meets the MFMA waves at the stage barrier and issues its
// share of the stage that reuses the slot just freed.
//
// DUP: the doubled-K packed form (GemmArgs::kdup): A keys past kdup read
// the planes again from key 0, and stages past kdup skip the lo products.
template <int EPI, int NB, int BMW, int BROWS = 256, int STG = (BMW == 2 ? 2 : 3), bool PROD = false,
          bool DUP = false, int NP = 1>
__global__ void __launch_bounds__(128 * BMW + (PROD ? 64 * NP : 0), (BMW == 2 && STG == 2) ? 2 : 1)
    gemm_lds_k(GemmArgs g, float *ws, int k_per_split, int mt, int nt) {
    using F = LsForm<BMW, BROWS, STG>;
    constexpr int BN = BROWS / NB;     // weight columns per matrix
    constexpr int NJ = BN / 64;        // 32-column MFMA blocks per wave and matrix
    constexpr int STAGES = F::STAGES;
    constexpr int NMW = 2 * BMW;       // MFMA waves
    static_assert(!PROD || (BN % 16) == 0, "a producer instruction's 16 weight rows share a matrix");
    extern __shared__ __attribute__((aligned(16))) char lds_s[];
    // wave index in an SGPR: the LDS bases of the direct loads (M0) stay scalar
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int total = mt * nt, per = (total + MF_XCDS - 1) / MF_XCDS;
    const int tile = (blockIdx.x % MF_XCDS) * per + blockIdx.x / MF_XCDS;
    if (tile >= total) return;
    int m0, M, grp;  // M: end of this tile's group (rows >= M are not computed)
    // row / column tile of this range position: bands of g.band column tiles
    const int bw = g.band > 1 ? min(g.band, nt) : 1, bsz = mt * bw, bnd = tile / bsz, idx = tile - bnd * bsz;
    const int cw = min(bw, nt - bnd * bw), rt = idx / cw, ct = bnd * bw + idx % cw;
    if (!group_tile(g.grp_offs, g.grp_n, g.M, rt, F::BM, m0, M, grp)) return;
    const int n0 = ct * BN;
    const size_t woff = (size_t)grp * g.grp_w_stride;
    const int N = g.N, K = g.K;
    const int kbeg = blockIdx.z * k_per_split;
    const int KT = (min(K, kbeg + k_per_split) - kbeg) / LS_BK;
    // A row stride and the A key of stage kt (block-uniform)
    const int lda = DUP ? g.kdup : K;
    auto akey = [&](int kt) {
        const int k = kbeg + kt * LS_BK;
        return DUP && k >= g.kdup ? k - g.kdup : k;
    };

    // this lane's global sources: A plane p, wave-instruction q covers LDS
    // slots (wave*2+q)*64 + lane; weights: (wave*QB+q)*64 + lane
    const uint16_t *asrc[2][2], *bsrc[F::QB];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int sl = (wave * 2 + q) * 64 + lane, r = sl >> 2, kc = (sl & 3) ^ ls_swz(r);
        const size_t off = (size_t)min(m0 + r, M - 1) * lda + kc * 8;
        asrc[0][q] = (const uint16_t *)g.a + off;
        asrc[1][q] = (const uint16_t *)g.a_lo + off;
    }
#pragma unroll
    for (int q = 0; q < F::QB; ++q) {
        const int sl = (wave * F::QB + q) * 64 + lane, r = sl >> 2, kc = (sl & 3) ^ ls_swz(r);
        const int b = r / BN, n = min(n0 + r % BN, N - 1);
        bsrc[q] = (const uint16_t *)(b ? g.w2 : g.w) + woff + (size_t)n * K + kbeg + kc * 8;
    }
    auto issue = [&](int kt) {
        char *base = lds_s + (kt % STAGES) * F::STAGE;
        const int ko = kt * LS_BK, ka = akey(kt);
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                __builtin_amdgcn_global_load_lds((gptr_t)(asrc[p][q] + ka),
                                                 (lptr_t)(base + p * F::A + (wave * 2 + q) * 1024), 16, 0, 0);
#pragma unroll
        for (int q = 0; q < F::QB; ++q)
            __builtin_amdgcn_global_load_lds((gptr_t)(bsrc[q] + ko),
                                             (lptr_t)(base + 2 * F::A + (wave * F::QB + q) * 1024), 16, 0, 0);
    };

    if constexpr (PROD) {
        if (wave >= NMW) {  // producer wave pw: its share (1 / NP) of every stage's slots
            constexpr int AQ = 2 * NMW / NP, BQ = F::QB * NMW / NP;  // its instructions per A plane / for B
            constexpr int LP = 2 * AQ + BQ;                           // its loads per stage
            static_assert((2 * NMW) % NP == 0 && (F::QB * NMW) % NP == 0, "producers share the slots evenly");
            static_assert(LP < 64, "one stage's loads must fit the vmcnt counter");
            const int pw = wave - NMW;
            int aoff[AQ], boff[BQ];
#pragma unroll
            for (int j = 0; j < AQ; ++j) {
                const int q = pw + NP * j;
                const int sl = q * 64 + lane, r = sl >> 2, kc = (sl & 3) ^ ls_swz(r);
                aoff[j] = (int)((size_t)min(m0 + r, M - 1) * lda + kc * 8);
            }
#pragma unroll
            for (int j = 0; j < BQ; ++j) {
                const int q = pw + NP * j;
                const int sl = q * 64 + lane, r = sl >> 2, kc = (sl & 3) ^ ls_swz(r);
                boff[j] = (int)((size_t)min(n0 + r % BN, N - 1) * K + kbeg + kc * 8);
            }
            const uint16_t *pa = (const uint16_t *)g.a, *pl = (const uint16_t *)g.a_lo;
            const uint16_t *pw0 = (const uint16_t *)g.w + woff, *pw1 = (const uint16_t *)g.w2 + woff;
            auto pissue = [&](int kt) {
                char *base = lds_s + (kt % STAGES) * F::STAGE;
                const int ko = kt * LS_BK, ka = akey(kt);
#pragma unroll
                for (int j = 0; j < AQ; ++j) {
                    const int q = pw + NP * j;
                    __builtin_amdgcn_global_load_lds((gptr_t)(pa + aoff[j] + ka), (lptr_t)(base + q * 1024), 16, 0, 0);
                    __builtin_amdgcn_global_load_lds((gptr_t)(pl + aoff[j] + ka), (lptr_t)(base + F::A + q * 1024), 16, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < BQ; ++j) {  // rows [16 q, 16 q + 16): gate rows, then up rows
                    const int q = pw + NP * j;
                    const uint16_t *pw_ = q * 16 < BN ? pw0 : pw1;
                    __builtin_amdgcn_global_load_lds((gptr_t)(pw_ + boff[j] + ko), (lptr_t)(base + 2 * F::A + q * 1024), 16, 0, 0);
                }
            };
#pragma unroll
            for (int st = 0; st < STAGES - 1; ++st)
                if (st < KT) pissue(st);
            for (int kt = 0; kt < KT; ++kt) {
                const int later = min(STAGES - 2, KT - 1 - kt);
                static_assert(STAGES == 3, "the producer keeps one later stage in flight");
                if (later >= 1) __builtin_amdgcn_s_waitcnt(vm_imm(LP));
                else __builtin_amdgcn_s_waitcnt(vm_imm(0));
                __builtin_amdgcn_s_barrier();
                if (kt + STAGES - 1 < KT) pissue(kt + STAGES - 1);
            }
            return;
        }
    }

    f32x16_t acc[NB][2][NJ];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[b][i][j][e] = 0.f;

    if constexpr (!PROD) {
#pragma unroll
        for (int st = 0; st < STAGES - 1; ++st)
            if (st < KT) issue(st);
    }
    for (int kt = 0; kt < KT; ++kt) {
        // this stage's loads are done once at most (later stages issued) x LPS remain
        if constexpr (!PROD) {
            const int later = min(STAGES - 2, KT - 1 - kt);
            static_assert(STAGES <= 6 && 4 * F::LPS < 64, "vmcnt waits below cover up to 4 later stages");
            if (later >= 4) __builtin_amdgcn_s_waitcnt(vm_imm(4 * F::LPS));
            else if (later == 3) __builtin_amdgcn_s_waitcnt(vm_imm(3 * F::LPS));
            else if (later == 2) __builtin_amdgcn_s_waitcnt(vm_imm(2 * F::LPS));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vm_imm(F::LPS));
            else __builtin_amdgcn_s_waitcnt(vm_imm(0));
        }
        // every wave's loads of stage kt landed; stage kt-1 is free. A bare
        // s_barrier: a fenced __syncthreads would wait for every stage in flight
        __builtin_amdgcn_s_barrier();
        if constexpr (!PROD) {
            if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1);
        }
        const char *base = lds_s + (kt % STAGES) * F::STAGE;
        const char *ah = base, *al = base + F::A, *bb = base + 2 * F::A;
        // the doubled-K form's second half multiplies the weights' lo part
        // by the hi plane only
        const bool lo_on = !DUP || kbeg + kt * LS_BK < g.kdup;
        // Form with register room (no producer wave: at most two waves per
        // SIMD): both 16-deep k-steps' fragments are read before their
        // MFMAs, and the schedule interleaves the second step's LDS reads
        // with the first step's MFMAs, so only the first reads' latency is
        // exposed per stage (at most 12 reads in flight: lgkmcnt counts
        // 15). The producer form (up to three waves per SIMD, ~170
        // registers) reads each step's fragments just before its MFMAs.
        constexpr int KS = LS_BK / 16;
        static_assert(KS == 2, "two k-steps per stage");
        if constexpr (!PROD) {
            constexpr int RD = 4 + NB * NJ;      // LDS reads per k-step
            constexpr int MF = 2 * NB * 2 * NJ;  // MFMAs per k-step
            bf16x8_t fh[KS][2], fl[KS][2], fb[KS][NB][NJ];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int c = 2 * ks + (lane >> 5);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int r = wm * 64 + i * 32 + (lane & 31);
                    const int off = r * LS_ROWB + ((c ^ ls_swz(r)) << 4);
                    fh[ks][i] = *(const bf16x8_t *)(ah + off);
                    fl[ks][i] = *(const bf16x8_t *)(al + off);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int r = b * BN + wn * (BN / 2) + j * 32 + (lane & 31);
                        fb[ks][b][j] = *(const bf16x8_t *)(bb + r * LS_ROWB + ((c ^ ls_swz(r)) << 4));
                    }
            }
            // hi products of every accumulator, then the lo ones:
            // consecutive MFMAs never chain on one accumulator
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    if (p && !lo_on) break;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
#pragma unroll
                        for (int i = 0; i < 2; ++i)
#pragma unroll
                            for (int j = 0; j < NJ; ++j)
                                acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                    p ? fl[ks][i] : fh[ks][i], fb[ks][b][j], acc[b][i][j], 0, 0, 0);
                }
            // step 0's reads, then step 0's MFMAs with one of step 1's reads
            // after every MF / RD of them, then step 1's MFMAs (the one-row-
            // tile form, 5 reads for 4 MFMAs, keeps the default order)
            if constexpr (MF % RD == 0) {
                __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
#pragma unroll
                for (int q = 0; q < RD; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, MF / RD, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int c = 2 * ks + (lane >> 5);
                bf16x8_t fh[2], fl[2], fb[NB][NJ];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int r = wm * 64 + i * 32 + (lane & 31);
                    const int off = r * LS_ROWB + ((c ^ ls_swz(r)) << 4);
                    fh[i] = *(const bf16x8_t *)(ah + off);
                    fl[i] = *(const bf16x8_t *)(al + off);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int r = b * BN + wn * (BN / 2) + j * 32 + (lane & 31);
                        fb[b][j] = *(const bf16x8_t *)(bb + r * LS_ROWB + ((c ^ ls_swz(r)) << 4));
                    }
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < NJ; ++j) {
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[i], fb[b][j], acc[b][i][j], 0, 0, 0);
                            if (lo_on)
                                acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[i], fb[b][j], acc[b][i][j], 0, 0, 0);
                        }
            }
        }
    }

    // epilogue: lane holds column (lane & 31) of each 32 x 32 block, rows
    // (e / 4) * 8 + (lane >> 5) * 4 + e % 4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
            if (col >= N) continue;
            if (EPI == MF_PARTIAL) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                    if (row >= M) continue;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        ws[(((size_t)blockIdx.z * NB + b) * g.M + row) * N + col] = acc[b][i][j][e];
                }
                continue;
            }
            const float bias = (EPI != GEMM_SWIGLU && g.bias) ? g.bias[col] : 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                if (row >= M) continue;
                float *c = (float *)g.c + (size_t)row * g.ldc + col;
                if (EPI == GEMM_SWIGLU) {
                    const float y = silu(acc[0][i][j][e]) * acc[NB - 1][i][j][e];
                    if (g.c_lo) {
                        const size_t ci = (size_t)row * g.ldc + col;
                        uint16_t h = f2bf(y);
                        ((uint16_t *)g.c)[ci] = h;
                        ((uint16_t *)g.c_lo)[ci] = f2bf(y - bf2f(h));
                    } else {
                        *c = y;
                    }
                } else {
                    float v = g.bias ? acc[0][i][j][e] + bias : acc[0][i][j][e];
                    if (EPI == GEMM_RESIDUAL) *c = *c + v;
                    else *c = v;
                }
            }
        }
}

static int g_cus = 0;

// The split-K reduction launch: four columns per thread when the shapes
// and pointers allow 16-byte access, else one.
template <int EPI, int NB>
static void launch_reduce(const GemmArgs &a, const float *ws, int splits, hipStream_t s) {
    const size_t mn = (size_t)a.M * a.N;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool v4 = a.N % 4 == 0 && a.ldc % 4 == 0 && al16(ws) && al16(a.c) &&
                    (!a.c_lo || al16(a.c_lo)) && (!a.bias || al16(a.bias));
    if (v4) {
        const int rblocks = (int)std::min<size_t>((mn / 4 + 255) / 256, (size_t)g_cus * 8);
        mfma_reduce4_k<EPI, NB><<<rblocks, 256, 0, s>>>(a, ws, splits);
        return;
    }
    const int rblocks = (int)std::min<size_t>((mn + 255) / 256, (size_t)g_cus * 8);
    mfma_reduce_k<EPI, NB><<<rblocks, 256, 0, s>>>(a, ws, splits);
}

// min_ks: smallest k range a split may get (the weight tile each block
// streams shrinks with it, so skinny row counts use short splits to put the
// weight stream on every CU)
template <int EPI, int NB, int NJ>
static void mfma_launch_nj(const GemmArgs &a, float *ws, size_t ws_bytes, hipStream_t s,
                           int min_ks = 512) {
    constexpr size_t shm = mfma_lds_bytes<NB, NJ>();
    constexpr int BN = 64 * NJ;
    const int gx = (a.N + BN - 1) / BN,
              gy = (a.M + MF_BM - 1) / MF_BM + (a.grp_offs ? a.grp_n : 0);
    const int blocks = MF_XCDS * ((gx * gy + MF_XCDS - 1) / MF_XCDS);
    // split K until the grid covers the chip twice
    int splits = 1;
    while (gx * gy * splits < 2 * g_cus && a.K / (splits * 2) >= min_ks &&
           (size_t)(splits * 2) * NB * a.M * a.N * 4 <= ws_bytes)
        splits *= 2;
    int kps = (a.K + splits - 1) / splits;
    kps = (kps + MF_BK - 1) / MF_BK * MF_BK;
    if (splits == 1) {
        gemm_mfma_k<EPI, NB, NJ><<<dim3(blocks, 1, 1), 256, shm, s>>>(a, nullptr, a.K, gy, gx);
        return;
    }
    gemm_mfma_k<MF_PARTIAL, NB, NJ><<<dim3(blocks, 1, splits), 256, shm, s>>>(a, ws, kps, gy, gx);
    if (a.defer_splits) {
        *a.defer_splits = splits;
        return;
    }
    launch_reduce<EPI, NB>(a, ws, splits, s);
}

template <int EPI, int NB, int BMW, int BROWS = 256, int STG = (BMW == 2 ? 2 : 3), bool DUP = false>
static void lds_launch(const GemmArgs &a, float *ws, size_t ws_bytes, hipStream_t s,
                       int want_blocks, int min_ks = 512) {
    using F = LsForm<BMW, BROWS, STG>;
    constexpr int BN = BROWS / NB;
    static bool attr = false;
    if (!attr) {
        ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_lds_k<EPI, NB, BMW, BROWS, STG, false, DUP>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)F::LDS));
        ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_lds_k<MF_PARTIAL, NB, BMW, BROWS, STG, false, DUP>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)F::LDS));
        attr = true;
    }
    const int gx = (a.N + BN - 1) / BN,
              gy = (a.M + F::BM - 1) / F::BM + (a.grp_offs ? a.grp_n : 0);
    const int blocks = MF_XCDS * ((gx * gy + MF_XCDS - 1) / MF_XCDS);
    int splits = 1;
    while (gx * gy * splits < want_blocks && a.K / (splits * 2) >= min_ks &&
           (size_t)(splits * 2) * NB * a.M * a.N * 4 <= ws_bytes)
        splits *= 2;
    // 256-row tiles of one weight matrix take the producer form (measured on
    // MI355X at the 8B prefill shapes: down 522 -> 502 us, o 159 -> 152 us;
    // gate/up pairs showed no gain and keep 128-row blocks)
    constexpr bool prod = BMW == 4 && NB == 1 && BROWS == 256 && STG == 3;
    // Fewer splits where the extra blocks only add a partial round: with
    // `slots` blocks resident on the chip, s splits take ceil(tiles s /
    // slots) rounds of K / s keys, so s is halved while that is no slower
    // (the partial sums and their reduction then go away). The 2048-row
    // q/k/v+LoRA projection of the 8B shape (200 tiles) runs unsplit instead
    // of as 400 half-K blocks plus a reduction.
    // Conversely a grid of between one and two rounds (the grouped expert
    // down_proj of the MoE prefill: 384 tiles at most on 256 slots) takes
    // two splits, 1.5 rounds of the full K instead of 2 (for grouped
    // launches the tile count is the bound the grid is sized for).
    {
        static int per_cu = 0;
        if (!per_cu) {
            const void *k = reinterpret_cast<const void *>(gemm_lds_k<MF_PARTIAL, NB, BMW, BROWS, STG, prod, DUP, prod ? 4 : 1>);
            ESP_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)F::LDS));
            ESP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, F::NT + (prod ? 64 * 4 : 0), F::LDS));
            if (per_cu <= 0) per_cu = 1;
        }
        const long long tiles = (long long)gx * gy, slots = (long long)per_cu * g_cus;
        auto rounds = [&](int sp) { return (tiles * sp + slots - 1) / slots; };
        if (!a.grp_offs)
            while (splits > 1 && 2 * rounds(splits / 2) <= rounds(splits)) splits /= 2;
        if (splits == 1 && tiles > slots && tiles < 2 * slots && rounds(2) < 2 * rounds(1) &&
            a.K / 2 >= min_ks && (size_t)2 * NB * a.M * a.N * 4 <= ws_bytes)
            splits = 2;
    }
    int kps = (a.K + splits - 1) / splits;
    kps = (kps + LS_BK - 1) / LS_BK * LS_BK;
    // Tile order: each XCD's range walks bands of four weight-column tiles
    // (row tiles within a band), so the blocks resident on one XCD share
    // both activation and weight strips in its L2 instead of spanning every
    // row tile of one or two column tiles. Measured on the 8B prefill shapes
    // (with the four producer waves below, against column-major order and
    // one producer): q/k/v 236 -> 212 us, down 505 -> 484, o 144 -> 141,
    // gate/up 1015 -> 978 at 2048 rows; 7-11% at 4096 rows.
    GemmArgs ab = a;
    ab.band = 4;
    if constexpr (prod) {
        // four producer waves each issue a quarter of every stage's direct
        // loads: one wave kept at most one stage (48 loads, under the 63 of
        // vmcnt) in flight ahead of the barrier
        auto go = [&](auto npc) {
            constexpr int NPV = decltype(npc)::value;
            static bool pattr = false;
            if (!pattr) {
                ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_lds_k<EPI, NB, BMW, BROWS, STG, true, DUP, NPV>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)F::LDS));
                ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_lds_k<MF_PARTIAL, NB, BMW, BROWS, STG, true, DUP, NPV>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)F::LDS));
                pattr = true;
            }
            if (splits == 1) {
                gemm_lds_k<EPI, NB, BMW, BROWS, STG, true, DUP, NPV><<<dim3(blocks, 1, 1), F::NT + 64 * NPV, F::LDS, s>>>(ab, nullptr, a.K, gy, gx);
                return;
            }
            gemm_lds_k<MF_PARTIAL, NB, BMW, BROWS, STG, true, DUP, NPV><<<dim3(blocks, 1, splits), F::NT + 64 * NPV, F::LDS, s>>>(ab, ws, kps, gy, gx);
            if (a.defer_splits) {
                *a.defer_splits = splits;
                return;
            }
            launch_reduce<EPI, NB>(a, ws, splits, s);
        };
        go(std::integral_constant<int, 4>{});
        return;
    }
    if (splits == 1) {
        gemm_lds_k<EPI, NB, BMW, BROWS, STG, false, DUP><<<dim3(blocks, 1, 1), F::NT, F::LDS, s>>>(ab, nullptr, a.K, gy, gx);
        return;
    }
    gemm_lds_k<MF_PARTIAL, NB, BMW, BROWS, STG, false, DUP><<<dim3(blocks, 1, splits), F::NT, F::LDS, s>>>(ab, ws, kps, gy, gx);
    if (a.defer_splits) {
        *a.defer_splits = splits;
        return;
    }
    launch_reduce<EPI, NB>(a, ws, splits, s);
}

// ---------------------------------------------------------------------------
// Skinny streamed form (one row tile of M <= 32 * RB rows, no groups): each
// block owns 32 * NW weight columns per matrix and one k range. The
// activation rows of each 32-key stage go global -> LDS (direct loads into a
// ring of D + 1 stages, read by every wave); each wave streams the weight
// rows of its own 32 columns global -> registers, D stages ahead, and
// multiplies them by all 32 * RB rows. The weights then need no LDS room or
// LDS bandwidth, and the bytes in flight per CU (NW * D * NB * 2 KB per
// block) are set by registers, not by the stage ring. The k range of a block
// is a multiple of D stages: every stage of a steady group issues stage
// kt + D unconditionally and the last group issues none, so every vmcnt wait
// is an exact constant (conditional loads would make the compiler wait for
// all loads in flight at each group's first use).
template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F> __device__ __forceinline__ void static_for(F &&f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

template <int EPI, int NB, int RB, int NW, int D>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
    gemm_skinny_k(GemmArgs g, float *ws, int k_per_split) {
    constexpr int ROWS = 32 * RB;
    constexpr int APL = ROWS * LS_ROWB;  // one A plane of a stage
    constexpr int AST = 2 * APL;         // one stage (hi + lo planes)
    constexpr int AQ = 4 * RB;           // 1 KB direct loads per stage
    static_assert(AQ % NW == 0, "the stage's A loads split evenly over the waves");
    constexpr int LA = AQ / NW;          // A loads per wave and stage
    constexpr int LPS = LA + 2 * NB;     // loads per wave and stage
    static_assert(D >= 2 && (D - 1) * LPS < 64, "waits count up to D - 1 later stages");
    extern __shared__ __attribute__((aligned(16))) char lds_s[];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int M = g.M, N = g.N, K = g.K;
    const int n0 = blockIdx.x * 32 * NW;
    const int kbeg = blockIdx.z * k_per_split;
    const int KT = (min(K, kbeg + k_per_split) - kbeg) / LS_BK;  // a multiple of D

    // A: wave-instruction q covers slots (q mod 2RB) * 64 + lane of plane
    // q / 2RB (16 rows x 4 chunks, chunk c of row r at slot c ^ swz(r));
    // rows past M re-read row M - 1
    const uint16_t *asrc[LA];
    int adst[LA];
#pragma unroll
    for (int j = 0; j < LA; ++j) {
        const int q = wave * LA + j, p = q / (2 * RB), qq = q % (2 * RB);
        const int sl = qq * 64 + lane, r = sl >> 2, kc = (sl & 3) ^ ls_swz(r);
        asrc[j] = (const uint16_t *)(p ? g.a_lo : g.a) + (size_t)min(r, M - 1) * K + kbeg + kc * 8;
        adst[j] = p * APL + qq * 1024;
    }
    // weights: the MFMA B-operand layout, lane = (column lane & 31, keys
    // 8 * (lane >> 5) .. + 8 of each 16-key step); columns past N re-read N - 1
    const uint16_t *wsrc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int n = min(n0 + wave * 32 + (lane & 31), N - 1);
        wsrc[b] = (const uint16_t *)(b ? g.w2 : g.w) + (size_t)n * K + kbeg + (lane >> 5) * 8;
    }
    auto issue_a = [&](int kt, int slot) {
        char *base = lds_s + slot * AST;
#pragma unroll
        for (int j = 0; j < LA; ++j)
            __builtin_amdgcn_global_load_lds((gptr_t)(asrc[j] + kt * LS_BK), (lptr_t)(base + adst[j]), 16, 0, 0);
    };
    auto issue_w = [&](int kt, bf16x8_t (&r)[NB][2]) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) r[b][ks] = *(const bf16x8_t *)(wsrc[b] + kt * LS_BK + ks * 16);
    };

    f32x16_t acc[NB][RB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[b][i][e] = 0.f;

    auto stage = [&](int slot, int nslot, bf16x8_t (&w)[NB][2], auto later_c, auto more_c, int kt) {
        constexpr int LATER = decltype(later_c)::value;
        constexpr bool MORE = decltype(more_c)::value;
        // this stage's loads are done once at most LATER stages' remain
        __builtin_amdgcn_s_waitcnt(vm_imm(LATER * LPS));
        // every wave's A loads of this stage landed; the previous slot is free
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MORE) issue_a(kt + D, nslot);
        __builtin_amdgcn_sched_barrier(0);
        const char *ah = lds_s + slot * AST, *al = ah + APL;
        // a k-step's fragment reads, then its MFMAs (both k-steps' reads
        // first when the registers allow: one matrix)
        constexpr int KG = NB == 1 ? 2 : 1;
#pragma unroll
        for (int g0 = 0; g0 < 2; g0 += KG) {
            bf16x8_t fh[KG][RB], fl[KG][RB];
#pragma unroll
            for (int kk = 0; kk < KG; ++kk) {
                const int c = 2 * (g0 + kk) + (lane >> 5);
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    const int r = i * 32 + (lane & 31);
                    const int off = r * LS_ROWB + ((c ^ ls_swz(r)) << 4);
                    fh[kk][i] = *(const bf16x8_t *)(ah + off);
                    fl[kk][i] = *(const bf16x8_t *)(al + off);
                }
            }
            // hi products of every accumulator, then the lo ones
#pragma unroll
            for (int kk = 0; kk < KG; ++kk) {
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < RB; ++i)
                        acc[b][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[kk][i], w[b][g0 + kk], acc[b][i], 0, 0, 0);
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < RB; ++i)
                        acc[b][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[kk][i], w[b][g0 + kk], acc[b][i], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * KG * RB, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * KG * RB * NB, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MORE) issue_w(kt + D, w);
        __builtin_amdgcn_sched_barrier(0);
    };

    // prologue: stages 0 .. D-1, A then weights per stage
    bf16x8_t wr[D][NB][2];
#pragma unroll
    for (int s = 0; s < D; ++s) {
        issue_a(s, s);
        issue_w(s, wr[s]);
    }
    int kt = 0, aslot = 0;  // aslot: ring slot of stage kt (D + 1 slots)
    for (; kt + D < KT; kt += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int nslot = aslot == 0 ? D : aslot - 1;  // (kt + s + D) mod (D + 1)
            stage(aslot, nslot, wr[s], std::integral_constant<int, D - 1>{}, std::true_type{}, kt + s);
            aslot = aslot == D ? 0 : aslot + 1;
        }
    }
    // last group: no further loads; stage s waits for D - 1 - s later stages
    static_for<D>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        stage(aslot, 0, wr[s], std::integral_constant<int, D - 1 - s>{}, std::false_type{}, kt + s);
        aslot = aslot == D ? 0 : aslot + 1;
    });

    // epilogue: lane holds column (lane & 31) of each 32 x 32 block, rows
    // (e / 4) * 8 + (lane >> 5) * 4 + e % 4
    const int col = n0 + wave * 32 + (lane & 31);
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
            if (row >= M) continue;
            if (EPI == MF_PARTIAL) {
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    ws[(((size_t)blockIdx.z * NB + b) * M + row) * N + col] = acc[b][i][e];
                continue;
            }
            float *c = (float *)g.c + (size_t)row * g.ldc + col;
            if (EPI == GEMM_SWIGLU) {
                const float y = silu(acc[0][i][e]) * acc[NB - 1][i][e];
                if (g.c_lo) {
                    const size_t ci = (size_t)row * g.ldc + col;
                    uint16_t h = f2bf(y);
                    ((uint16_t *)g.c)[ci] = h;
                    ((uint16_t *)g.c_lo)[ci] = f2bf(y - bf2f(h));
                } else {
                    *c = y;
                }
            } else {
                float v = g.bias ? acc[0][i][e] + g.bias[col] : acc[0][i][e];
                if (EPI == GEMM_RESIDUAL) *c = *c + v;
                else *c = v;
            }
        }
}

// k split as for the streamed form; each split's range is a multiple of
// D stages (K % (32 D) == 0 is checked by the caller)
template <int EPI, int NB, int RB, int NW, int D>
static void skinny_launch(const GemmArgs &a, float *ws, size_t ws_bytes, hipStream_t s,
                          int want_blocks, int min_ks) {
    constexpr size_t LDSB = (size_t)(D + 1) * 2 * 32 * RB * LS_ROWB;
    static bool attr = false;
    if (!attr) {
        ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_skinny_k<EPI, NB, RB, NW, D>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDSB));
        ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_skinny_k<MF_PARTIAL, NB, RB, NW, D>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDSB));
        attr = true;
    }
    constexpr int BN = 32 * NW, KU = LS_BK * D;
    if (a.K % KU != 0 || a.M > 32 * RB) fail(ESP_BACKEND, "skinny GEMM: shape outside the form");
    const int gx = (a.N + BN - 1) / BN;
    int splits = 1;
    while (gx * splits < want_blocks && a.K / (splits * 2) >= min_ks &&
           (size_t)(splits * 2) * NB * a.M * a.N * 4 <= ws_bytes)
        splits *= 2;
    int kps = (a.K + splits - 1) / splits;
    kps = (kps + KU - 1) / KU * KU;
    splits = (a.K + kps - 1) / kps;
    if (splits == 1) {
        gemm_skinny_k<EPI, NB, RB, NW, D><<<dim3(gx, 1, 1), 64 * NW, LDSB, s>>>(a, nullptr, a.K);
        return;
    }
    gemm_skinny_k<MF_PARTIAL, NB, RB, NW, D><<<dim3(gx, 1, splits), 64 * NW, LDSB, s>>>(a, ws, kps);
    if (a.defer_splits) {
        *a.defer_splits = splits;
        return;
    }
    launch_reduce<EPI, NB>(a, ws, splits, s);
}

template <int EPI> static void mfma_launch(const GemmArgs &a, float *ws, size_t ws_bytes,
                                           hipStream_t s) {
    constexpr int NB = EPI == GEMM_SWIGLU ? 2 : 1;
    constexpr int NJW = 4 / NB;  // wide form: 128 weight columns per wave
    if (!g_cus) {
        int dev = 0;
        ESP_HIP(hipGetDevice(&dev));
        ESP_HIP(hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (g_cus <= 0) g_cus = 256;
    }
    const long long wide_tiles = (long long)((a.N + 64 * NJW - 1) / (64 * NJW)) * ((a.M + MF_BM - 1) / MF_BM);
    // long row counts (prefill of >= 1024 tokens) take the LDS-streamed form:
    // 256-row blocks for one weight matrix, 128-row blocks for gate/up pairs
    if (a.K % LS_BK == 0 && a.M >= 1024) {
        if (a.kdup) {
            if (a.K != 2 * a.kdup || a.kdup % LS_BK) fail(ESP_BACKEND, "doubled-K GEMM: K must be 2 kdup");
            if (NB == 1) lds_launch<EPI, NB, 4, 256, 3, true>(a, ws, ws_bytes, s, g_cus);
            else lds_launch<EPI, NB, 2, 256, 2, true>(a, ws, ws_bytes, s, 2 * g_cus);
            return;
        }
        if (NB == 1) lds_launch<EPI, NB, 4>(a, ws, ws_bytes, s, g_cus);
        else lds_launch<EPI, NB, 2>(a, ws, ws_bytes, s, 2 * g_cus);
        return;
    }
    if (a.kdup) fail(ESP_BACKEND, "doubled-K GEMM: only the streamed form of >= 1024 rows takes it");
    if (a.M <= MF_BM && !a.grp_offs) {
        // skinny streamed form (measured on MI355X, 1B / 8B shapes): a
        // weight matrix wide enough to fill the chip with one k range (the
        // 128256-column output head) takes 256 columns per block, two
        // stages ahead (64 rows: 240 -> 138 us); 64 rows or fewer take 128
        // columns per block, four stages ahead (16 rows: down 18.0 -> 12.3
        // us, gate/up 26.1 -> 19.7 us). 65 - 128 rows of narrower matrices
        // keep the streamed form below, which measured faster there.
        const bool wide = (a.N + 255) / 256 >= g_cus;
        if (wide && a.K % (LS_BK * 2) == 0) {
            if (a.M <= 64) skinny_launch<EPI, NB, 2, 8, 2>(a, ws, ws_bytes, s, g_cus, 256);
            else skinny_launch<EPI, NB, 4, 8, 2>(a, ws, ws_bytes, s, g_cus, 256);
            return;
        }
        if (a.M <= 64 && a.K % (LS_BK * 4) == 0) {
            skinny_launch<EPI, NB, 2, 4, 4>(a, ws, ws_bytes, s, g_cus, 256);
            return;
        }
    }
    if (a.K % LS_BK == 0 && a.M <= MF_BM && !getenv("ESP_SKINNY_REG")) {
        // one row tile (decode batches, forced blocks): 64 weight columns per
        // matrix, three stages (60 KB of LDS; measured on the C5 step: 3.28
        // -> 3.19 ms against six stages), k splits down to 256 keys
        lds_launch<EPI, NB, 2, 64 * NB, 3>(a, ws, ws_bytes, s, g_cus, 256);
        return;
    }
    if (a.K % LS_BK == 0 && a.M > MF_BM && a.M < 1024 && !getenv("ESP_MID_REG")) {
        // 129 - 1023 rows (grammar-forced spans in a batch, short prompts):
        // the streamed form, 128-row tiles of 128 weight rows per matrix,
        // three stages (measured on the C5 grammar batch: 4.87 -> 4.47 ms
        // per step against the register-staged tiles; 64 weight rows and
        // six stages 4.55, the 256-row prefill tiles 4.80).
        // ESP_MID_REG=1 keeps the register-staged form, for comparison.
        lds_launch<EPI, NB, 2, 128 * NB, 3>(a, ws, ws_bytes, s, g_cus, 256);
        return;
    }
    if (a.M <= MF_BM) {
        // 64-column register-staged tiles, k splits down to 128 keys
        mfma_launch_nj<EPI, NB, 1>(a, ws, ws_bytes, s, 128);
        return;
    }
    if (wide_tiles >= g_cus) mfma_launch_nj<EPI, NB, NJW>(a, ws, ws_bytes, s);
    else mfma_launch_nj<EPI, NB, NJW / 2>(a, ws, ws_bytes, s);
}

bool gemm_mfma_ok(Dt wt, const GemmArgs &a) {
    return wt == DT_BF16 && a.a_lo && a.K % 8 == 0 && a.K >= 32 && ((uintptr_t)a.a % 16) == 0 &&
           ((uintptr_t)a.a_lo % 16) == 0 && ((uintptr_t)a.w % 16) == 0 &&
           (!a.w2 || ((uintptr_t)a.w2 % 16) == 0);
}

void launch_gemm_mfma(GemmEpi epi, const GemmArgs &a, float *ws, size_t ws_bytes, hipStream_t s) {
    if (epi == GEMM_STORE) mfma_launch<GEMM_STORE>(a, ws, ws_bytes, s);
    else if (epi == GEMM_RESIDUAL) mfma_launch<GEMM_RESIDUAL>(a, ws, ws_bytes, s);
    else mfma_launch<GEMM_SWIGLU>(a, ws, ws_bytes, s);
}

}  // namespace esp
