// Causal GQA attention for a block of consecutive query rows of one sequence
// (prefill and long forced blocks) on the CDNA4 matrix cores.
//
// attention.rs:345-397 computes softmax((q.k)/sqrt(hd) + mask) . v with the
// causal rule `key > past + query` and the sliding rule `pos - key >= window`;
// this kernel evaluates the same function tile by tile with an online
// softmax (running max / sum per query row), never materialising scores.
//
// Precision: q, k, v (f32 in the cache) and the probabilities p are split
// into bf16 hi + lo parts; each product uses three bf16 MFMAs (hi.hi +
// hi.lo + lo.hi), accumulating in f32, which keeps ~16 mantissa bits of
// each operand.
//
// Layout: block = 4 waves x 32 query rows (128 rows) of one query head;
// key tiles of 32 are staged in LDS (K rows as [key][dim], V transposed as
// [dim][key]); S = Q K^T comes out of v_mfma_f32_32x32x16_bf16 with lane
// l holding key column l%32 and query rows (i/4)*8 + (l/32)*4 + i%4 in
// register i, so the softmax reductions are 32-lane butterflies and the
// per-row rescale of the output accumulators uses the same register map.
// P is re-laid through LDS as the A operand of O += P V.
#include "common.hpp"
#include "dev.hpp"
#include "flash.hpp"

namespace esp {

typedef __bf16 fbf16x8_t __attribute__((ext_vector_type(8)));
typedef float ff32x16_t __attribute__((ext_vector_type(16)));
typedef float ff32x4_t __attribute__((ext_vector_type(4)));

constexpr int FA_BQ = 128, FA_BK = 32, FA_WQ = 32;

template <int HD> struct FaLds {
    static constexpr int KLD = HD + 8;     // K rows (bf16), padded
    static constexpr int VLD = FA_BK + 8;  // V^T rows (bf16), padded
    static constexpr int PLD = FA_BK + 8;  // P rows (bf16), padded
    static constexpr int K_ELEMS = FA_BK * KLD;
    static constexpr int V_ELEMS = HD * VLD;
    static constexpr int P_ELEMS = FA_WQ * PLD;
    static constexpr size_t bytes = (size_t)(2 * K_ELEMS + 2 * V_ELEMS + 4 * 2 * P_ELEMS) * 2;
};

__device__ __forceinline__ void split_bf16(float v, uint16_t &h, uint16_t &l) {
    h = f2bf(v);
    l = f2bf(v - bf2f(h));
}

template <int HD>
__global__ void __launch_bounds__(256) flash_attn_k(FlashArgs a) {
    typedef FaLds<HD> Ly;
    constexpr int NKS = HD / 16;  // k-steps over head dims for S
    constexpr int NDT = HD / 32;  // 32-wide output dim tiles
    extern __shared__ uint16_t fl[];
    uint16_t *Kh = fl, *Kl = Kh + Ly::K_ELEMS;
    uint16_t *Vh = Kl + Ly::K_ELEMS, *Vl = Vh + Ly::V_ELEMS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    uint16_t *Ph = Vl + Ly::V_ELEMS + wave * 2 * Ly::P_ELEMS, *Pl = Ph + Ly::P_ELEMS;
    const int qh = blockIdx.y, G = a.nq / a.nkv, kvh = qh / G;
    const int q0 = blockIdx.x * FA_BQ;               // first row of the block
    const int wq0 = q0 + wave * FA_WQ;               // first row of this wave
    const float scale = sqrtf((float)HD);
    const int half = lane >> 5, col = lane & 31;

    // Q fragments (A operand): lane holds row wq0 + col, dims ks*16 + half*8 .. +8
    fbf16x8_t qfh[NKS], qfl[NKS];
    {
        const int r = wq0 + col;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            uint16_t h[8], l[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float v = r < a.M ? a.q[(size_t)r * a.nq * HD + (size_t)qh * HD + ks * 16 + half * 8 + e] : 0.f;
                split_bf16(v, h[e], l[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                qfh[ks][e] = __builtin_bit_cast(__bf16, h[e]);
                qfl[ks][e] = __builtin_bit_cast(__bf16, l[e]);
            }
        }
    }
    // per-register query row and position
    int qpos[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) qpos[i] = a.p0 + wq0 + (i >> 2) * 8 + half * 4 + (i & 3);
    float m[16], lsum[16];
    ff32x16_t o[NDT];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        m[i] = -INFINITY;
        lsum[i] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.f;

    const int last_row = min(a.M, q0 + FA_BQ) - 1;
    const int kv_hi = a.p0 + last_row + 1;  // exclusive
    int kv_lo = a.window > 0 ? max(0, a.p0 + q0 - a.window + 1) : 0;
    kv_lo = kv_lo / FA_BK * FA_BK;
    const float *kbase = a.kv + (size_t)a.seq * a.seq_stride + (size_t)kvh * a.head_stride;
    const float *vbase = kbase + a.kv_half_stride;

    for (int k0 = kv_lo; k0 < kv_hi; k0 += FA_BK) {
        __syncthreads();  // previous tile fully consumed
        // stage K [key][dim] and V^T [dim][key] as bf16 hi/lo
        for (int idx = tid; idx < FA_BK * HD / 4; idx += 256) {
            const int key = idx / (HD / 4), d = (idx % (HD / 4)) * 4;
            const int t = k0 + key;
            ff32x4_t kv4 = {0.f, 0.f, 0.f, 0.f}, vv4 = {0.f, 0.f, 0.f, 0.f};
            if (t < kv_hi) {
                kv4 = *(const ff32x4_t *)(kbase + (size_t)t * HD + d);
                vv4 = *(const ff32x4_t *)(vbase + (size_t)t * HD + d);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint16_t h, l;
                split_bf16(kv4[e], h, l);
                Kh[key * Ly::KLD + d + e] = h;
                Kl[key * Ly::KLD + d + e] = l;
                split_bf16(vv4[e], h, l);
                Vh[(d + e) * Ly::VLD + key] = h;
                Vl[(d + e) * Ly::VLD + key] = l;
            }
        }
        __syncthreads();
        // S = Q K^T for this wave's 32 rows x 32 keys
        ff32x16_t sacc;
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const int off = col * Ly::KLD + ks * 16 + half * 8;
            fbf16x8_t kh = *(const fbf16x8_t *)(Kh + off);
            fbf16x8_t kl = *(const fbf16x8_t *)(Kl + off);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qfh[ks], kh, sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qfh[ks], kl, sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qfl[ks], kh, sacc, 0, 0, 0);
        }
        // scale, mask, online softmax (per query row = per register)
        const int key = k0 + col;
        float alpha[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int qp = qpos[i];
            const bool ok = key <= qp && key < kv_hi && (a.window <= 0 || qp - key < a.window);
            float s = ok ? sacc[i] / scale : -INFINITY;
            float mx = s;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            const float mn = fmaxf(m[i], mx);
            const float al = mn == -INFINITY ? 1.f : __expf(m[i] - mn);
            const float p = s == -INFINITY ? 0.f : __expf(s - mn);
            float ps = p;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) ps += __shfl_xor(ps, off, 64);
            lsum[i] = lsum[i] * al + ps;
            m[i] = mn;
            alpha[i] = al;
            sacc[i] = p;
        }
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[t][i] *= alpha[i];
        // P -> LDS as [query row][key] (hi/lo), then read A fragments
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = (i >> 2) * 8 + half * 4 + (i & 3);
            uint16_t h, l;
            split_bf16(sacc[i], h, l);
            Ph[r * Ly::PLD + col] = h;
            Pl[r * Ly::PLD + col] = l;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < FA_BK / 16; ++kk) {
            const int poff = col * Ly::PLD + kk * 16 + half * 8;
            fbf16x8_t ph = *(const fbf16x8_t *)(Ph + poff);
            fbf16x8_t pl = *(const fbf16x8_t *)(Pl + poff);
#pragma unroll
            for (int t = 0; t < NDT; ++t) {
                const int voff = (t * 32 + col) * Ly::VLD + kk * 16 + half * 8;
                fbf16x8_t vh = *(const fbf16x8_t *)(Vh + voff);
                fbf16x8_t vl = *(const fbf16x8_t *)(Vl + voff);
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ph, vh, o[t], 0, 0, 0);
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ph, vl, o[t], 0, 0, 0);
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pl, vh, o[t], 0, 0, 0);
            }
        }
    }
    // normalise and store: register i -> row (i/4)*8 + half*4 + i%4, dim t*32 + col
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = wq0 + (i >> 2) * 8 + half * 4 + (i & 3);
        if (r >= a.M) continue;
        const float inv_l = lsum[i];
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
            const size_t idx = (size_t)r * a.nq * HD + (size_t)qh * HD + t * 32 + col;
            const float v = o[t][i] / inv_l;
            if (a.out_lo) {
                uint16_t h = f2bf(v);
                ((uint16_t *)a.out)[idx] = h;
                a.out_lo[idx] = f2bf(v - bf2f(h));
            } else {
                a.out[idx] = v;
            }
        }
    }
}

bool flash_ok(int hd) { return hd == 64 || hd == 128; }

void launch_flash(const FlashArgs &a, hipStream_t s) {
    dim3 grid((a.M + FA_BQ - 1) / FA_BQ, a.nq);
    if (a.hd == 64) {
        flash_attn_k<64><<<grid, 256, FaLds<64>::bytes, s>>>(a);
    } else if (a.hd == 128) {
        flash_attn_k<128><<<grid, 256, FaLds<128>::bytes, s>>>(a);
    } else {
        fail(ESP_BACKEND, "flash attention: unsupported head_dim");
    }
}

}  // namespace esp
