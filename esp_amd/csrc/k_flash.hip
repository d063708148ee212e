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
// bf16 hi/lo planes in LDS; the next tile's f32 rows are loaded into
// registers while the current tile is multiplied.
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
    static constexpr size_t bytes = (size_t)PLANES * (K_ELEMS + V_ELEMS) * 2;
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

template <int HD, bool F16>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) flash_attn_k(FlashArgs a, int nqb) {
    typedef FaLds<HD, F16> Ly;
    typedef typename std::conditional<F16, ff16x8_t, fbf16x8_t>::type op8_t;  // MFMA operand
    constexpr int NKS = HD / 16;  // k-steps over head dims for S^T
    constexpr int NDT = HD / 32;  // 32-row output dim tiles of O^T
    constexpr int ES = F16 ? 2 : 4;  // bytes per cached element
    extern __shared__ uint16_t fl[];
    uint16_t *Kh = fl, *Kl = Kh + Ly::K_ELEMS;  // Kl, Vl: f32 cache only
    uint16_t *Vh = fl + Ly::PLANES * Ly::K_ELEMS, *Vl = Vh + Ly::V_ELEMS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int half = lane >> 5, col = lane & 31;

    // Work order: groups (query block, kv head) longest query block first;
    // the G query heads of a group run on one XCD (workgroups are dealt to
    // the XCDs round-robin by linear id) so they share K/V tiles in its L2.
    const int G = a.nq / a.nkv, ngroups = nqb * a.nkv;
    const int xcd = blockIdx.x % FA_XCDS, slot = blockIdx.x / FA_XCDS;
    const int gi = (slot / G) * FA_XCDS + xcd;
    if (gi >= ngroups) return;
    const int qb = nqb - 1 - gi / a.nkv, kvh = gi % a.nkv;
    const int qh = kvh * G + slot % G;
    const int q0 = qb * FA_BQ;                       // first row of the block
    const int wq0 = q0 + wave * FA_WQ;               // first row of this wave
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

    // register staging of one tile (rows beyond kv_hi are zero): 8 dims of a
    // key per K chunk; 2 dims x 4 keys per V unit
    ff32x4_t kreg[Ly::KCH][2];
    ff32x2_t vreg[Ly::VCH][4];
    fu32x4_t kreg16[Ly::KCH];
    uint32_t vreg16[Ly::VCH][4];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int c = 0; c < Ly::KCH; ++c) {
            const int idx = tid + c * 256, key = idx / (HD / 8), d = (idx % (HD / 8)) * 8;
            const int t = k0 + key;
            const char *p = kbase + ((size_t)t * HD + d) * ES;
            if constexpr (F16) {
                kreg16[c] = fu32x4_t{0u, 0u, 0u, 0u};
                if (t < kv_hi) kreg16[c] = *(const fu32x4_t *)p;
            } else {
                kreg[c][0] = kreg[c][1] = ff32x4_t{0.f, 0.f, 0.f, 0.f};
                if (t < kv_hi) {
                    kreg[c][0] = *(const ff32x4_t *)p;
                    kreg[c][1] = *(const ff32x4_t *)(p + 16);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < Ly::VCH; ++c) {
            const int idx = tid + c * 256, dp = idx % (HD / 2), kq = idx / (HD / 2);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = k0 + kq * 4 + j;
                const char *p = vbase + ((size_t)t * HD + dp * 2) * ES;
                if constexpr (F16) {
                    vreg16[c][j] = 0u;
                    if (t < kv_hi) vreg16[c][j] = *(const uint32_t *)p;
                } else {
                    vreg[c][j] = ff32x2_t{0.f, 0.f};
                    if (t < kv_hi) vreg[c][j] = *(const ff32x2_t *)p;
                }
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int c = 0; c < Ly::KCH; ++c) {
            const int idx = tid + c * 256, key = idx / (HD / 8), d = (idx % (HD / 8)) * 8;
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
            const int idx = tid + c * 256, dp = idx % (HD / 2), kq = idx / (HD / 2);
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

    if (kv_lo < kv_hi) load_tile(kv_lo);
    for (int k0 = kv_lo; k0 < kv_hi; k0 += FA_BK) {
        __syncthreads();  // previous tile fully consumed
        store_tile();
        __syncthreads();
        if (k0 + FA_BK < kv_hi) load_tile(k0 + FA_BK);  // in flight during the products

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
        // mask (only tiles that cross the diagonal / window / end), online softmax
        const bool full = k0 + FA_BK - 1 <= a.p0 + wq0 && k0 + FA_BK <= kv_hi &&
                          (a.window <= 0 || a.p0 + wq0 + FA_WQ - 1 - k0 < a.window);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = sacc[i] * c2;
            if (!full) {
                const int key = k0 + (i >> 2) * 8 + half * 4 + (i & 3);
                const bool ok = key <= qp && key < kv_hi && (a.window <= 0 || qp - key < a.window);
                s = ok ? s : -INFINITY;
            }
            sacc[i] = s;
            mx = fmaxf(mx, s);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(m, mx);
        const float msub = mn == -INFINITY ? 0.f : mn;
        const float alpha = exp2f(m - msub);
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sacc[i] = exp2f(sacc[i] - msub);
            ps += sacc[i];
        }
        ps += __shfl_xor(ps, 32, 64);
        lsum = lsum * alpha + ps;
        m = mn;
        if (__any(alpha != 1.f)) {
#pragma unroll
            for (int t = 0; t < NDT; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[t][i] *= alpha;
        }
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
    // normalise and store: lane -> query row wq0 + col; register i -> dim
    // t*32 + (i/4)*8 + half*4 + i%4 (runs of four consecutive dims)
    const int r = wq0 + col;
    if (r >= a.M) return;
    const float inv = 1.f / lsum;
    const size_t rowo = (size_t)r * a.nq * HD + (size_t)qh * HD + half * 4;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const size_t idx = rowo + t * 32 + g * 8;
            const float v0 = o[t][g * 4] * inv, v1 = o[t][g * 4 + 1] * inv;
            const float v2 = o[t][g * 4 + 2] * inv, v3 = o[t][g * 4 + 3] * inv;
            if (a.out_lo) {
                const fu32x2_t x = split2(v0, v1), y = split2(v2, v3);
                *(fu32x2_t *)((uint16_t *)a.out + idx) = fu32x2_t{x[0], y[0]};
                *(fu32x2_t *)(a.out_lo + idx) = fu32x2_t{x[1], y[1]};
            } else {
                *(ff32x4_t *)(a.out + idx) = ff32x4_t{v0, v1, v2, v3};
            }
        }
}

bool flash_ok(int hd) { return hd == 64 || hd == 128; }

void launch_flash(const FlashArgs &a, hipStream_t s) {
    if (a.M <= 0) return;
    if (a.nkv <= 0 || a.nq % a.nkv != 0) fail(ESP_BACKEND, "flash attention: bad head grouping");
    const int nqb = (a.M + FA_BQ - 1) / FA_BQ;
    const int G = a.nq / a.nkv, ngroups = nqb * a.nkv;
    const int blocks = ((ngroups + FA_XCDS - 1) / FA_XCDS) * FA_XCDS * G;
    if (a.hd == 64) {
        if (a.kv_f16) flash_attn_k<64, true><<<blocks, 256, FaLds<64, true>::bytes, s>>>(a, nqb);
        else flash_attn_k<64, false><<<blocks, 256, FaLds<64>::bytes, s>>>(a, nqb);
    } else if (a.hd == 128) {
        if (a.kv_f16) flash_attn_k<128, true><<<blocks, 256, FaLds<128, true>::bytes, s>>>(a, nqb);
        else flash_attn_k<128, false><<<blocks, 256, FaLds<128>::bytes, s>>>(a, nqb);
    } else {
        fail(ESP_BACKEND, "flash attention: unsupported head_dim");
    }
}

}  // namespace esp
