// Causal GQA attention for a block of consecutive query rows of one sequence
// (prefill and long forced blocks) on the CDNA4 matrix cores.
//
// attention.rs:345-397 computes softmax((q.k)/sqrt(hd) + mask) . v with the
// causal rule `key > past + query` and the sliding rule `pos - key >= window`;
// this kernel evaluates the same function tile by tile with an online
// softmax (running max / sum per query row), never materialising scores.
//
// Precision: with an f32 cache, q, k, v and the probabilities p are split
// into bf16 hi + lo parts (both round-to-nearest-even); each product uses
// three bf16 MFMAs (hi.hi + hi.lo + lo.hi) accumulating in f32, which keeps
// ~16 mantissa bits of each operand. With an f16 cache (F16), k and v are
// exact f16 operands and only q and p are split, into f16 hi + lo: two f16
// MFMAs per product (k.q_hi + k.q_lo, v.p_hi + v.p_lo), ~22 bits of q and p,
// and one LDS plane per tile instead of two.
//
// Layout: a wave owns 32 query rows of one query head and computes the
// transposed products S^T = K Q^T and O^T = V^T P^T with
// v_mfma_f32_32x32x16_bf16. In the accumulator layout lane l holds column
// l%32 (= its query row) and, in register i, row (i/4)*8 + (l/32)*4 + i%4
// (= a key of the tile, or an output dim). So:
//  * the softmax max / sum over a tile's 32 keys is 16 values in-lane plus
//    one exchange with lane l^32;
//  * the per-row rescale of O^T is one factor per lane;
//  * the 16 probabilities a lane holds are already the B operand of the
//    P.V product, provided the V^T operand reads keys in the same order:
//    B k-slot 8*(l/32)+e of k-step kk is register kk*8+e, i.e. key
//    (2*kk + e/4)*8 + (l/32)*4 + e%4 -- two runs of four consecutive keys.
// K tiles are staged as [key][dim] and V tiles as V^T [dim][key], both
// bf16 hi/lo planes in LDS.
//
// Schedule: a workgroup of eight waves takes a 128-row query block; waves
// 0-3 (key group 0) take the even 32-key tiles and waves 4-7 (group 1) the
// odd ones, so each SIMD runs two waves of the block. A step stages two
// tiles (one per group) into one of two LDS buffer pairs while the other
// pair is multiplied: one barrier per step, the next step's f32 rows in
// registers during the products. Each group keeps its own running max,
// sum and output rows; group 1 hands its partial rows to group 0 through
// LDS at the end. The running max moves only when a tile's max passes it
// by more than 8 (log2 units), so the output rescale is rare and the
// probabilities stay below 2^8. A workgroup takes query block nqb-1-i and
// then block i, so every workgroup sees about the same number of tiles.
#include <type_traits>

#include "common.hpp"
#include "dev.hpp"
#include "flash.hpp"

namespace esp {

typedef __bf16 fbf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 fbf16x2_t __attribute__((ext_vector_type(2)));
typedef float ff32x16_t __attribute__((ext_vector_type(16)));
typedef float ff32x4_t __attribute__((ext_vector_type(4)));
typedef float ff32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t fu32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t fu32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 ff16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 ff16x2_t __attribute__((ext_vector_type(2)));

constexpr int FA_BQ = 128, FA_BK = 32, FA_WQ = 32, FA_XCDS = 8;

template <int HD, bool F16 = false> struct FaLds {
    static constexpr int KLD = HD + 8;     // K rows [key][dim] (16-bit), padded
    static constexpr int VLD = FA_BK + 4;  // V^T rows [dim][key] (16-bit), padded
    static constexpr int K_ELEMS = FA_BK * KLD;
    static constexpr int V_ELEMS = HD * VLD;
    static constexpr int PLANES = F16 ? 1 : 2;  // hi (+ lo) per operand
    static constexpr int BUF = PLANES * (K_ELEMS + V_ELEMS);  // 16-bit elements per tile buffer
    static constexpr size_t tiles = (size_t)4 * BUF * 2;       // two steps x two tiles
    static constexpr size_t merge = (size_t)4 * (HD / 32 * 16 + 2) * 64 * 4;  // key group 1's partial rows
    static constexpr size_t bytes = tiles > merge ? tiles : merge;
    static constexpr int KCH = FA_BK * HD / 8 / 256;  // 8-dim K chunks per thread
    static constexpr int VCH = FA_BK * HD / 8 / 256;  // 4-key x 2-dim V units per thread
};

// two floats -> {packed bf16 hi pair, packed bf16 lo pair} (x = hi + lo)
__device__ __forceinline__ fu32x2_t split2(float x, float y) {
    ff32x2_t v = {x, y};
    fbf16x2_t h = __builtin_convertvector(v, fbf16x2_t);
    ff32x2_t r = v - __builtin_convertvector(h, ff32x2_t);
    return fu32x2_t{__builtin_bit_cast(uint32_t, h),
                    __builtin_bit_cast(uint32_t, __builtin_convertvector(r, fbf16x2_t))};
}

// two floats -> {packed f16 hi pair, packed f16 lo pair} (x = hi + lo)
__device__ __forceinline__ fu32x2_t split2h(float x, float y) {
    ff32x2_t v = {x, y};
    ff16x2_t h = __builtin_convertvector(v, ff16x2_t);
    ff32x2_t r = v - __builtin_convertvector(h, ff32x2_t);
    return fu32x2_t{__builtin_bit_cast(uint32_t, h),
                    __builtin_bit_cast(uint32_t, __builtin_convertvector(r, ff16x2_t))};
}

__device__ __forceinline__ void split8h(ff32x4_t x0, ff32x4_t x1, ff16x8_t &h, ff16x8_t &l) {
    const fu32x2_t a = split2h(x0[0], x0[1]), b = split2h(x0[2], x0[3]);
    const fu32x2_t c = split2h(x1[0], x1[1]), d = split2h(x1[2], x1[3]);
    h = __builtin_bit_cast(ff16x8_t, fu32x4_t{a[0], b[0], c[0], d[0]});
    l = __builtin_bit_cast(ff16x8_t, fu32x4_t{a[1], b[1], c[1], d[1]});
}

// eight floats -> bf16x8 hi and lo operands
__device__ __forceinline__ void split8(ff32x4_t x0, ff32x4_t x1, fbf16x8_t &h, fbf16x8_t &l) {
    const fu32x2_t a = split2(x0[0], x0[1]), b = split2(x0[2], x0[3]);
    const fu32x2_t c = split2(x1[0], x1[1]), d = split2(x1[2], x1[3]);
    h = __builtin_bit_cast(fbf16x8_t, fu32x4_t{a[0], b[0], c[0], d[0]});
    l = __builtin_bit_cast(fbf16x8_t, fu32x4_t{a[1], b[1], c[1], d[1]});
}


// One 128-row query block `qb` of query head `qh` (kv head `kvh`).
template <int HD, bool F16>
__device__ __forceinline__ void flash_block(const FlashArgs &a, int qb, int qh, int kvh, uint16_t *fl) {
    typedef FaLds<HD, F16> Ly;
    typedef typename std::conditional<F16, ff16x8_t, fbf16x8_t>::type op8_t;  // MFMA operand
    constexpr int NKS = HD / 16;  // k-steps over head dims for S^T
    constexpr int NDT = HD / 32;  // 32-row output dim tiles of O^T
    constexpr int ES = F16 ? 2 : 4;  // bytes per cached element
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int half = lane >> 5, col = lane & 31;
    const int qw = wave & 3, kg = wave >> 2, ltid = tid & 255;  // query slice, key group
    const int q0 = qb * FA_BQ;                       // first row of the block
    const int wq0 = q0 + qw * FA_WQ;                 // first row of this wave
    const float c2 = 1.4426950408889634f / sqrtf((float)HD);  // log2(e)/sqrt(hd)

    // Q^T fragments (B operand): lane holds query row wq0 + col, dims
    // ks*16 + half*8 .. +8
    op8_t qfh[NKS], qfl[NKS];
    {
        const int r = wq0 + col;
        const float *qrow = a.q + (size_t)r * a.nq * HD + (size_t)qh * HD + half * 8;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            ff32x4_t x0 = {0.f, 0.f, 0.f, 0.f}, x1 = x0;
            if (r < a.M) {
                x0 = *(const ff32x4_t *)(qrow + ks * 16);
                x1 = *(const ff32x4_t *)(qrow + ks * 16 + 4);
            }
            if constexpr (F16) split8h(x0, x1, qfh[ks], qfl[ks]);
            else split8(x0, x1, qfh[ks], qfl[ks]);
        }
    }
    const int qp = a.p0 + wq0 + col;  // this lane's query position
    float m = -INFINITY, lsum = 0.f;
    ff32x16_t o[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.f;

    const int last_row = min(a.M, q0 + FA_BQ) - 1;
    const int kv_hi = a.p0 + last_row + 1;  // exclusive
    int kv_lo = a.window > 0 ? max(0, a.p0 + q0 - a.window + 1) : 0;
    kv_lo = kv_lo / FA_BK * FA_BK;
    const char *kbase = (const char *)a.kv +
                        ((size_t)a.seq * a.seq_stride + (size_t)kvh * a.head_stride) * ES;
    const char *vbase = kbase + (size_t)a.kv_half_stride * ES;

    // this thread's staging units, as byte offsets within a tile: 8 dims of
    // one key per K chunk; 2 dims x 4 consecutive keys per V unit
    uint32_t koff[Ly::KCH], voff[Ly::VCH];
    int kkey[Ly::KCH], vkey[Ly::VCH];
#pragma unroll
    for (int c = 0; c < Ly::KCH; ++c) {
        const int idx = ltid + c * 256;
        kkey[c] = idx / (HD / 8);
        koff[c] = (uint32_t)((kkey[c] * HD + (idx % (HD / 8)) * 8) * ES);
    }
#pragma unroll
    for (int c = 0; c < Ly::VCH; ++c) {
        const int idx = ltid + c * 256;
        vkey[c] = (idx / (HD / 2)) * 4;
        voff[c] = (uint32_t)((vkey[c] * HD + (idx % (HD / 2)) * 2) * ES);
    }

    // register staging of one tile (keys at or beyond kv_hi read as zero)
    ff32x4_t kreg[Ly::KCH][2];
    ff32x2_t vreg[Ly::VCH][4];
    fu32x4_t kreg16[Ly::KCH];
    uint32_t vreg16[Ly::VCH][4];
    auto load_tile = [&](int k0) {
        const char *kt = kbase + (size_t)k0 * HD * ES, *vt = vbase + (size_t)k0 * HD * ES;
        if (k0 + FA_BK <= kv_hi) {  // whole tile in range (uniform)
#pragma unroll
            for (int c = 0; c < Ly::KCH; ++c) {
                const char *p = kt + koff[c];
                if constexpr (F16) kreg16[c] = *(const fu32x4_t *)p;
                else {
                    kreg[c][0] = *(const ff32x4_t *)p;
                    kreg[c][1] = *(const ff32x4_t *)(p + 16);
                }
            }
#pragma unroll
            for (int c = 0; c < Ly::VCH; ++c) {
                const char *p = vt + voff[c];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (F16) vreg16[c][j] = *(const uint32_t *)(p + j * HD * ES);
                    else vreg[c][j] = *(const ff32x2_t *)(p + j * HD * ES);
                }
            }
            return;
        }
#pragma unroll
        for (int c = 0; c < Ly::KCH; ++c) {
            const char *p = kt + koff[c];
            const bool in = k0 + kkey[c] < kv_hi;
            if constexpr (F16) {
                kreg16[c] = fu32x4_t{0u, 0u, 0u, 0u};
                if (in) kreg16[c] = *(const fu32x4_t *)p;
            } else {
                kreg[c][0] = kreg[c][1] = ff32x4_t{0.f, 0.f, 0.f, 0.f};
                if (in) {
                    kreg[c][0] = *(const ff32x4_t *)p;
                    kreg[c][1] = *(const ff32x4_t *)(p + 16);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < Ly::VCH; ++c) {
            const char *p = vt + voff[c];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool in = k0 + vkey[c] + j < kv_hi;
                if constexpr (F16) {
                    vreg16[c][j] = 0u;
                    if (in) vreg16[c][j] = *(const uint32_t *)(p + j * HD * ES);
                } else {
                    vreg[c][j] = ff32x2_t{0.f, 0.f};
                    if (in) vreg[c][j] = *(const ff32x2_t *)(p + j * HD * ES);
                }
            }
        }
    };
    // K tile -> [key][dim] planes, V tile -> V^T [dim][key] planes of buffer b
    auto store_tile = [&](int b) {
        uint16_t *Kh = fl + b * Ly::BUF, *Kl = Kh + Ly::K_ELEMS;  // Kl, Vl: f32 cache only
        uint16_t *Vh = Kh + Ly::PLANES * Ly::K_ELEMS, *Vl = Vh + Ly::V_ELEMS;
#pragma unroll
        for (int c = 0; c < Ly::KCH; ++c) {
            const int idx = ltid + c * 256, key = idx / (HD / 8), d = (idx % (HD / 8)) * 8;
            if constexpr (F16) {
                *(fu32x4_t *)(Kh + key * Ly::KLD + d) = kreg16[c];
            } else {
                fbf16x8_t h, l;
                split8(kreg[c][0], kreg[c][1], h, l);
                *(fbf16x8_t *)(Kh + key * Ly::KLD + d) = h;
                *(fbf16x8_t *)(Kl + key * Ly::KLD + d) = l;
            }
        }
#pragma unroll
        for (int c = 0; c < Ly::VCH; ++c) {
            const int idx = ltid + c * 256, dp = idx % (HD / 2), kq = idx / (HD / 2);
            // dims 2dp and 2dp+1, keys kq*4 .. +4
            const int o0 = (2 * dp) * Ly::VLD + kq * 4;
            if constexpr (F16) {
                // each u32 holds (dim 2dp, dim 2dp+1) of one key
                const uint32_t *v = vreg16[c];
                *(fu32x2_t *)(Vh + o0) = fu32x2_t{(v[0] & 0xffffu) | (v[1] << 16),
                                                  (v[2] & 0xffffu) | (v[3] << 16)};
                *(fu32x2_t *)(Vh + o0 + Ly::VLD) = fu32x2_t{(v[0] >> 16) | (v[1] & 0xffff0000u),
                                                            (v[2] >> 16) | (v[3] & 0xffff0000u)};
            } else {
                const fu32x2_t a = split2(vreg[c][0][0], vreg[c][1][0]), b = split2(vreg[c][2][0], vreg[c][3][0]);
                const fu32x2_t e = split2(vreg[c][0][1], vreg[c][1][1]), f = split2(vreg[c][2][1], vreg[c][3][1]);
                *(fu32x2_t *)(Vh + o0) = fu32x2_t{a[0], b[0]};
                *(fu32x2_t *)(Vl + o0) = fu32x2_t{a[1], b[1]};
                *(fu32x2_t *)(Vh + o0 + Ly::VLD) = fu32x2_t{e[0], f[0]};
                *(fu32x2_t *)(Vl + o0 + Ly::VLD) = fu32x2_t{e[1], f[1]};
            }
        }
    };

    // Steps of two tiles: key group g multiplies tile 2i+g of step i from
    // buffer pair i%2 while step i+1 is converted into the other pair; one
    // barrier per step. Each group keeps its own running max / sum / output
    // for its tiles; the two are merged at the end.
    load_tile(kv_lo + kg * FA_BK);
    store_tile(kg);
    __syncthreads();
    if (kv_lo + 2 * FA_BK < kv_hi) load_tile(kv_lo + 2 * FA_BK + kg * FA_BK);
    int buf = 0;
    for (int ks0 = kv_lo; ks0 < kv_hi; ks0 += 2 * FA_BK) {
        const int k0 = ks0 + kg * FA_BK;
        if (k0 < kv_hi) {
            const uint16_t *Kh = fl + (buf * 2 + kg) * Ly::BUF, *Kl = Kh + Ly::K_ELEMS;
            const uint16_t *Vh = Kh + Ly::PLANES * Ly::K_ELEMS, *Vl = Vh + Ly::V_ELEMS;
            // S^T = K Q^T: 32 keys x this wave's 32 queries
            ff32x16_t sacc;
    #pragma unroll
            for (int i = 0; i < 16; ++i) sacc[i] = 0.f;
    #pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const int off = col * Ly::KLD + ks * 16 + half * 8;
                if constexpr (F16) {
                    const ff16x8_t kh = *(const ff16x8_t *)(Kh + off);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qfh[ks], sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qfl[ks], sacc, 0, 0, 0);
                } else {
                    fbf16x8_t kh = *(const fbf16x8_t *)(Kh + off);
                    fbf16x8_t kl = *(const fbf16x8_t *)(Kl + off);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qfh[ks], sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qfh[ks], sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qfl[ks], sacc, 0, 0, 0);
                }
            }
            // scale; mask only tiles that cross the diagonal / window / end
            const bool full = k0 + FA_BK - 1 <= a.p0 + wq0 && k0 + FA_BK <= kv_hi &&
                              (a.window <= 0 || a.p0 + wq0 + FA_WQ - 1 - k0 < a.window);
    #pragma unroll
            for (int i = 0; i < 16; ++i) sacc[i] *= c2;
            if (!full) {
    #pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = k0 + (i >> 2) * 8 + half * 4 + (i & 3);
                    const bool ok = (key <= qp) & (key < kv_hi) & ((a.window <= 0) | (qp - key < a.window));
                    sacc[i] = ok ? sacc[i] : -INFINITY;
                }
            }
            float mx = sacc[0];
    #pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sacc[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            // The running max moves only when a tile's max passes it by more
            // than 8 (log2 units): the probabilities stay below 2^8, and the
            // rescale of the output accumulators is rare.
            const float mn = mx > m + 8.f ? mx : m;
            const float msub = mn == -INFINITY ? 0.f : mn;
            float ps = 0.f;
    #pragma unroll
            for (int i = 0; i < 16; ++i) {
                sacc[i] = __builtin_amdgcn_exp2f(sacc[i] - msub);
                ps += sacc[i];
            }
            ps += __shfl_xor(ps, 32, 64);
            if (__any(mn != m)) {
                const float alpha = __builtin_amdgcn_exp2f(m - msub);
                lsum *= alpha;
    #pragma unroll
                for (int t = 0; t < NDT; ++t)
    #pragma unroll
                    for (int i = 0; i < 16; ++i) o[t][i] *= alpha;
            }
            lsum += ps;
            m = mn;
            // P^T as B operands (hi / lo) of the two 16-key steps
            op8_t ph[2], pl[2];
    #pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const ff32x4_t p0 = {sacc[kk * 8], sacc[kk * 8 + 1], sacc[kk * 8 + 2], sacc[kk * 8 + 3]};
                const ff32x4_t p1 = {sacc[kk * 8 + 4], sacc[kk * 8 + 5], sacc[kk * 8 + 6], sacc[kk * 8 + 7]};
                if constexpr (F16) split8h(p0, p1, ph[kk], pl[kk]);
                else split8(p0, p1, ph[kk], pl[kk]);
            }
            // O^T += V^T P^T
    #pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int ka = (2 * kk) * 8 + half * 4, kb = ka + 8;
    #pragma unroll
                for (int t = 0; t < NDT; ++t) {
                    const int vo = (t * 32 + col) * Ly::VLD;
                    fu32x2_t h0 = *(const fu32x2_t *)(Vh + vo + ka), h1 = *(const fu32x2_t *)(Vh + vo + kb);
                    if constexpr (F16) {
                        const ff16x8_t vh = __builtin_bit_cast(ff16x8_t, fu32x4_t{h0[0], h0[1], h1[0], h1[1]});
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph[kk], o[t], 0, 0, 0);
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl[kk], o[t], 0, 0, 0);
                    } else {
                        fu32x2_t l0 = *(const fu32x2_t *)(Vl + vo + ka), l1 = *(const fu32x2_t *)(Vl + vo + kb);
                        fbf16x8_t vh = __builtin_bit_cast(fbf16x8_t, fu32x4_t{h0[0], h0[1], h1[0], h1[1]});
                        fbf16x8_t vl = __builtin_bit_cast(fbf16x8_t, fu32x4_t{l0[0], l0[1], l1[0], l1[1]});
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph[kk], o[t], 0, 0, 0);
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph[kk], o[t], 0, 0, 0);
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl[kk], o[t], 0, 0, 0);
                    }
                }
            }
        }
        // next step into the other buffer pair (its previous contents were
        // consumed before the last barrier), then the barrier that publishes it
        if (ks0 + 2 * FA_BK < kv_hi) store_tile((buf ^ 1) * 2 + kg);
        __syncthreads();
        if (ks0 + 4 * FA_BK < kv_hi) load_tile(ks0 + 4 * FA_BK + kg * FA_BK);
        buf ^= 1;
    }
    // merge: key group 1 publishes its partial rows, group 0 combines them
    float *xo = (float *)fl + (size_t)qw * (NDT * 16 + 2) * 64 + lane;
    if (kg == 1) {
        xo[0] = m;
        xo[64] = lsum;
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) xo[(2 + t * 16 + i) * 64] = o[t][i];
    }
    __syncthreads();
    if (kg == 1) return;
    const float m1 = xo[0], l1 = xo[64];
    const float mn = fmaxf(m, m1), msub = mn == -INFINITY ? 0.f : mn;
    const float a0 = __builtin_amdgcn_exp2f(m - msub), a1 = __builtin_amdgcn_exp2f(m1 - msub);
    const float inv = 1.f / (lsum * a0 + l1 * a1);
    // normalise and store: lane -> query row wq0 + col; register i -> dim
    // t*32 + (i/4)*8 + half*4 + i%4 (runs of four consecutive dims)
    const int r = wq0 + col;
    if (r >= a.M) return;
    const size_t rowo = (size_t)r * a.nq * HD + (size_t)qh * HD + half * 4;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const size_t idx = rowo + t * 32 + g * 8;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = g * 4 + e;
                v[e] = (o[t][i] * a0 + xo[(2 + t * 16 + i) * 64] * a1) * inv;
            }
            if (a.out_lo) {
                const fu32x2_t x = split2(v[0], v[1]), y = split2(v[2], v[3]);
                *(fu32x2_t *)((uint16_t *)a.out + idx) = fu32x2_t{x[0], y[0]};
                *(fu32x2_t *)(a.out_lo + idx) = fu32x2_t{x[1], y[1]};
            } else {
                *(ff32x4_t *)(a.out + idx) = ff32x4_t{v[0], v[1], v[2], v[3]};
            }
        }
}

template <int HD, bool F16>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) flash_attn_k(FlashArgs a, int nqb) {
    extern __shared__ uint16_t fl[];
    // Work: a group is (pair of query blocks, kv head); its G query heads run
    // on one XCD (workgroups are dealt to the XCDs round-robin by linear id)
    // so they share K/V tiles in that XCD's L2.
    const int npair = (nqb + 1) / 2;
    const int G = a.nq / a.nkv, ngroups = npair * a.nkv;
    const int xcd = blockIdx.x % FA_XCDS, slot = blockIdx.x / FA_XCDS;
    const int gi = (slot / G) * FA_XCDS + xcd;
    if (gi >= ngroups) return;
    const int pr = gi / a.nkv, kvh = gi % a.nkv;
    const int qh = kvh * G + slot % G;
    flash_block<HD, F16>(a, nqb - 1 - pr, qh, kvh, fl);
    if (pr != nqb - 1 - pr) {
        __syncthreads();  // the first block's merge rows are read
        flash_block<HD, F16>(a, pr, qh, kvh, fl);
    }
}

bool flash_ok(int hd) { return hd == 64 || hd == 128; }

template <int HD, bool F16> static void flash_launch(const FlashArgs &a, int nqb, int blocks, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        ESP_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(flash_attn_k<HD, F16>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)FaLds<HD, F16>::bytes));
        attr = true;
    }
    flash_attn_k<HD, F16><<<blocks, 512, FaLds<HD, F16>::bytes, s>>>(a, nqb);
}

void launch_flash(const FlashArgs &a, hipStream_t s) {
    if (a.M <= 0) return;
    if (a.nkv <= 0 || a.nq % a.nkv != 0) fail(ESP_BACKEND, "flash attention: bad head grouping");
    const int nqb = (a.M + FA_BQ - 1) / FA_BQ;
    const int G = a.nq / a.nkv, ngroups = (nqb + 1) / 2 * a.nkv;
    const int blocks = ((ngroups + FA_XCDS - 1) / FA_XCDS) * FA_XCDS * G;
    if (a.hd == 64) {
        if (a.kv_f16) flash_launch<64, true>(a, nqb, blocks, s);
        else flash_launch<64, false>(a, nqb, blocks, s);
    } else if (a.hd == 128) {
        if (a.kv_f16) flash_launch<128, true>(a, nqb, blocks, s);
        else flash_launch<128, false>(a, nqb, blocks, s);
    } else {
        fail(ESP_BACKEND, "flash attention: unsupported head_dim");
    }
}

}  // namespace esp
