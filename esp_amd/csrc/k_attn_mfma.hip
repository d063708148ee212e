// Decode attention of many rows (batched decode, forced blocks) on the CDNA4
// matrix cores: the same function as attn_decode_k without key splits
// (attention.rs:345-397: softmax(q.k / sqrt(hd) + causal / window mask) . v
// over the row's cached keys), for batches whose (row, kv head) units fill
// the chip on their own.
//
// One wave per (row group, kv head) unit: a group is up to 16 / G rows of
// one sequence at consecutive positions (a forced block's rows), so the
// group's key tiles are read once; its rows' G query heads are the 16
// columns of v_mfma_f32_16x16x32 products (column c = row c / G, head c % G;
// unused columns are zero), each column masked to its own row's keys:
//   S^T = K Q^T   A = K (16 keys x 32 dims), B = Q^T
//   O^T = V^T P^T A = V^T (16 dims x 32 keys, through LDS), B = P^T
// In the 16 x 16 accumulator layout lane l holds column l % 16 (= its query
// head) and rows 4 (l / 16) + i, i < 4. So the running max, sum and output
// rescale of a head live in the lanes of that column, and the probabilities
// a lane holds for its keys 16 h + 4 (l / 16) + i of a 32-key tile are
// exactly the B operand k-slots 8 (l / 16) + 4 h + i of the P.V product,
// provided the V^T operand reads the keys in that order (two runs of four
// consecutive keys per lane). The K operand's dims are permuted the same
// way in Q: k-step s, k-slot 8 (l / 16) + j holds dim (l / 16) hd/4 + 8 s + j,
// so each lane loads hd/4 consecutive dims of its key row.
//
// Precision as the prefill kernel (k_flash.hip): with an f16 cache, k and v
// are exact f16 operands and q and p are split into f16 hi + lo (two
// products); with an f32 cache q, k, v and p are split into bf16 hi + lo and
// each product takes three MFMAs (hi.hi + hi.lo + lo.hi). The running max
// moves only when a tile's max passes it by more than 8 (log2 units), so the
// probabilities stay below 2^8. Tiles are double-buffered in registers: the
// next tile's loads are issued before the current tile is used; they are
// buffer loads whose range check covers the whole offset (the tile start is
// part of the per-lane offset), so keys at or past the row's end read as 0
// and nothing past the unit's rows is fetched.
#include <type_traits>

#include "common.hpp"
#include "decode.hpp"
#include "dev.hpp"

namespace esp {

typedef _Float16 am_h8 __attribute__((ext_vector_type(8)));
typedef __bf16 am_b8 __attribute__((ext_vector_type(8)));
typedef float am_f4 __attribute__((ext_vector_type(4)));
typedef float am_f2 __attribute__((ext_vector_type(2)));
typedef uint32_t am_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t am_u2 __attribute__((ext_vector_type(2)));

constexpr int AM_BK = 32;          // keys per tile
constexpr int AM_VLD = AM_BK + 4;  // V^T row stride in LDS (16-bit elements)

template <int HD, bool F16> struct AmShape {
    static constexpr int KD = HD / 4;                  // dims per lane of a key row
    static constexpr int KS = HD / 32;                 // k-steps of the S product
    static constexpr int KL = F16 ? KD / 8 : KD / 4;   // 16-byte K loads per lane and 16-key half
    static constexpr int DP = HD / 2;                  // dim pairs of a row
    static constexpr int VU = AM_BK * DP / 4 / 64;     // (4 keys x 2 dims) V units per lane
    static constexpr int PLANES = F16 ? 1 : 2;         // V^T planes (hi, lo)
    static constexpr int LDSW = PLANES * HD * AM_VLD;  // 16-bit elements per wave
    typedef typename std::conditional<F16, uint32_t, am_u2>::type VW;  // one key's two dims
};

template <int HD, bool F16> struct AmTile {
    using S = AmShape<HD, F16>;
    am_u4 k[2][S::KL];               // [16-key half][load]
    typename S::VW v[S::VU][4];      // [unit][key of the quad]
};

typedef __bf16 am_b2 __attribute__((ext_vector_type(2)));
typedef _Float16 am_h2 __attribute__((ext_vector_type(2)));

// f32 pair -> {packed hi pair, packed lo pair} (x = hi + lo, both RNE) in
// bf16 (f32 cache operands) or f16 (q and p over an f16 cache)
__device__ __forceinline__ am_u2 am_split_bf(float x, float y) {
    const am_f2 v = {x, y};
    const am_b2 h = __builtin_convertvector(v, am_b2);
    const am_f2 r = v - __builtin_convertvector(h, am_f2);
    return am_u2{__builtin_bit_cast(uint32_t, h), __builtin_bit_cast(uint32_t, __builtin_convertvector(r, am_b2))};
}
__device__ __forceinline__ am_u2 am_split_h(float x, float y) {
    const am_f2 v = {x, y};
    const am_h2 h = __builtin_convertvector(v, am_h2);
    const am_f2 r = v - __builtin_convertvector(h, am_f2);
    return am_u2{__builtin_bit_cast(uint32_t, h), __builtin_bit_cast(uint32_t, __builtin_convertvector(r, am_h2))};
}

// One unit per block (one wave), so a batch's units spread over every CU:
// four units per block put the C5 step's 576 units on 144 CUs, and splitting
// a unit's tiles over two or four waves (merged through LDS) measured slower
// than one wave per unit.
template <int HD, bool F16>
__global__ void __launch_bounds__(64) attn_rows_mfma_k(AttnDecodeArgs a) {
    using S = AmShape<HD, F16>;
    using T = AmTile<HD, F16>;
    constexpr int ES = F16 ? 2 : 4;
    __shared__ __attribute__((aligned(16))) uint16_t lds[S::LDSW];
    // the unit, its row range and the buffer descriptors are wave-uniform
    const int lane = threadIdx.x & 63;
    const int unit = blockIdx.x;
    if (unit >= (a.grp ? a.ngrp : a.M) * a.nkv) return;
    const int g = unit % a.nkv, gi = unit / a.nkv;
    const int G = a.nq / a.nkv;
    const int col = lane & 15, grp = lane >> 4;
    // the unit's rows: one group of nr consecutive positions of a sequence
    // (or a single row); column col is row j = col / G, query head col % G
    int r0 = gi, nr = 1;
    if (a.grp) {
        const int e = a.grp[gi];
        r0 = e & 0xffff;
        nr = e >> 16;
    }
    const int j = col / G, hq = col % G;
    const bool cvalid = j < nr;
    const int row_c = r0 + (cvalid ? j : 0);
    const int seq = a.seq1 >= 0 ? a.seq1 : a.row_seq[r0];
    const int pos_c = a.row_pos[row_c];  // this lane's row
    const int pos0 = a.row_pos[r0], posn = a.row_pos[r0 + nr - 1];
    const int lo_c = a.window > 0 ? max(0, pos_c - a.window + 1) : 0;
    const int hi_c = min(pos_c + 1, a.max_t);
    // the key range every column needs: [lo of the first row, end of the last)
    const int lo = a.window > 0 ? max(0, pos0 - a.window + 1) : 0;
    const int hi = min(posn + 1, a.max_t);
    const char *kb = (const char *)a.kv + ((size_t)seq * a.seq_stride + (size_t)g * a.head_stride) * ES;
    const char *vb = kb + (size_t)a.kv_half_stride * ES;
    uint16_t *vt = lds;

    // q of this lane's head (zero columns past G), pre-split
    am_u4 qh[S::KS], ql[S::KS];
    {
        const float *qr = a.q + (size_t)row_c * a.nq * HD + (size_t)(g * G + hq) * HD + grp * S::KD;
#pragma unroll
        for (int s = 0; s < S::KS; ++s) {
            const am_f4 x0 = *(const am_f4 *)(qr + 8 * s), x1 = *(const am_f4 *)(qr + 8 * s + 4);
            float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            if (!cvalid) {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const am_u2 hl = F16 ? am_split_h(x[2 * j], x[2 * j + 1]) : am_split_bf(x[2 * j], x[2 * j + 1]);
                qh[s][j] = hl[0];
                ql[s][j] = hl[1];
            }
        }
    }

    // Tile loads are buffer loads over this unit's K and V rows [0, hi):
    // keys past the row's range read as 0 (and are masked below). The tile
    // start is added to each lane's constant row offset (the per-lane offset
    // is what the range check compares with the descriptor's size; the
    // scalar offset is left 0).
    constexpr int ROWB = HD * ES;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void *)kb, (short)0, hi * ROWB, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void *)vb, (short)0, hi * ROWB, 0x00020000);
    // K: half h, lane key 16 h + col, dims grp * KD ..; V unit u: dims
    // 2 dp, 2 dp + 1 of keys 4 kq .. 4 kq + 3
    const int dp = lane % S::DP;
    auto vkq = [&](int u) { return u * (64 / S::DP) + lane / S::DP; };
    int kofs[2], vofs[S::VU];
#pragma unroll
    for (int h = 0; h < 2; ++h) kofs[h] = (16 * h + col) * ROWB + grp * S::KD * ES;
#pragma unroll
    for (int u = 0; u < S::VU; ++u) vofs[u] = 4 * vkq(u) * ROWB + 2 * dp * ES;
    auto load = [&](T &b, int t0) {
        const int so = t0 * ROWB;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < S::KL; ++q)
                b.k[h][q] = __builtin_bit_cast(am_u4, __builtin_amdgcn_raw_buffer_load_b128(rk, so + kofs[h] + 16 * q, 0, 0));
#pragma unroll
        for (int u = 0; u < S::VU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (F16)
                    b.v[u][e] = __builtin_amdgcn_raw_buffer_load_b32(rv, so + vofs[u] + e * ROWB, 0, 0);
                else
                    b.v[u][e] = __builtin_bit_cast(am_u2, __builtin_amdgcn_raw_buffer_load_b64(rv, so + vofs[u] + e * ROWB, 0, 0));
            }
    };

    const float cscale = 1.4426950408889634f / sqrtf((float)HD);  // log2(e) / sqrt(hd)
    float m = -INFINITY, l = 0.f;
    am_f4 o[HD / 16];
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) o[d] = am_f4{0.f, 0.f, 0.f, 0.f};

    auto tile = [&](const T &b, int t0) {
        // V^T into this wave's LDS planes: [dim][key], keys 4 kq .. + 3 per write
#pragma unroll
        for (int u = 0; u < S::VU; ++u) {
            const int kq = vkq(u);
            if constexpr (F16) {
                const uint32_t w0 = b.v[u][0], w1 = b.v[u][1], w2 = b.v[u][2], w3 = b.v[u][3];
                const am_u2 d0 = {(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
                const am_u2 d1 = {(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
                *(am_u2 *)(vt + (2 * dp) * AM_VLD + 4 * kq) = d0;
                *(am_u2 *)(vt + (2 * dp + 1) * AM_VLD + 4 * kq) = d1;
            } else {
                uint32_t h0[4], l0[4];  // per key: (dim 2dp, dim 2dp+1) hi / lo pairs
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const am_u2 hl = am_split_bf(__uint_as_float(b.v[u][e][0]), __uint_as_float(b.v[u][e][1]));
                    h0[e] = hl[0];
                    l0[e] = hl[1];
                }
#pragma unroll
                for (int pl = 0; pl < 2; ++pl) {
                    const uint32_t *w = pl ? l0 : h0;
                    const am_u2 d0 = {(w[0] & 0xffffu) | (w[1] << 16), (w[2] & 0xffffu) | (w[3] << 16)};
                    const am_u2 d1 = {(w[0] >> 16) | (w[1] & 0xffff0000u), (w[2] >> 16) | (w[3] & 0xffff0000u)};
                    uint16_t *plane = vt + pl * HD * AM_VLD;
                    *(am_u2 *)(plane + (2 * dp) * AM_VLD + 4 * kq) = d0;
                    *(am_u2 *)(plane + (2 * dp + 1) * AM_VLD + 4 * kq) = d1;
                }
            }
        }
        // S^T for the two 16-key halves
        am_f4 sa[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            sa[h] = am_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < S::KS; ++s) {
                if constexpr (F16) {
                    const am_h8 kf = __builtin_bit_cast(am_h8, b.k[h][s]);
                    sa[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(am_h8, qh[s]), sa[h], 0, 0, 0);
                    sa[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(am_h8, ql[s]), sa[h], 0, 0, 0);
                } else {
                    am_u4 kh, kl;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const am_u4 x = b.k[h][2 * s + j];
                        const am_u2 a0 = am_split_bf(__uint_as_float(x[0]), __uint_as_float(x[1]));
                        const am_u2 a1 = am_split_bf(__uint_as_float(x[2]), __uint_as_float(x[3]));
                        kh[2 * j] = a0[0];
                        kl[2 * j] = a0[1];
                        kh[2 * j + 1] = a1[0];
                        kl[2 * j + 1] = a1[1];
                    }
                    const am_b8 khb = __builtin_bit_cast(am_b8, kh), klb = __builtin_bit_cast(am_b8, kl);
                    sa[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khb, __builtin_bit_cast(am_b8, qh[s]), sa[h], 0, 0, 0);
                    sa[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khb, __builtin_bit_cast(am_b8, ql[s]), sa[h], 0, 0, 0);
                    sa[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klb, __builtin_bit_cast(am_b8, qh[s]), sa[h], 0, 0, 0);
                }
            }
        }
        // online softmax in log2 units; keys past the row's range weigh 0
        float sc[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = t0 + 16 * h + 4 * grp + i;
                sc[4 * h + i] = key >= lo_c && key < hi_c ? sa[h][i] * cscale : -INFINITY;
            }
        float mx = sc[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) mx = fmaxf(mx, sc[k]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = mx > m + 8.f ? mx : m;
        if (__any(mn != m)) {
            const float al = mn != m ? __builtin_amdgcn_exp2f(m - mn) : 1.f;  // m = -inf: 0
            l *= al;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d) o[d] *= al;
            m = mn;
        }
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            p[k] = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[k] - m);
            l += p[k];
        }
        // P^T operand: k-slot 8 grp + 4 h + i = key 16 h + 4 grp + i
        am_u4 ph, pl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const am_u2 hl = F16 ? am_split_h(p[2 * j], p[2 * j + 1]) : am_split_bf(p[2 * j], p[2 * j + 1]);
            ph[j] = hl[0];
            pl[j] = hl[1];
        }
        // O^T += V^T P^T per 16-dim tile; V^T k-slots read in the same key order
#pragma unroll
        for (int d = 0; d < HD / 16; ++d) {
            const uint16_t *r0 = vt + (d * 16 + col) * AM_VLD + 4 * grp;
            am_u4 vh;
            {
                const am_u2 x0 = *(const am_u2 *)r0, x1 = *(const am_u2 *)(r0 + 16);
                vh = am_u4{x0[0], x0[1], x1[0], x1[1]};
            }
            if constexpr (F16) {
                const am_h8 va = __builtin_bit_cast(am_h8, vh);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, __builtin_bit_cast(am_h8, ph), o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, __builtin_bit_cast(am_h8, pl), o[d], 0, 0, 0);
            } else {
                const uint16_t *r1 = r0 + HD * AM_VLD;
                const am_u2 y0 = *(const am_u2 *)r1, y1 = *(const am_u2 *)(r1 + 16);
                const am_u4 vl = {y0[0], y0[1], y1[0], y1[1]};
                const am_b8 vhb = __builtin_bit_cast(am_b8, vh), vlb = __builtin_bit_cast(am_b8, vl);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhb, __builtin_bit_cast(am_b8, ph), o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhb, __builtin_bit_cast(am_b8, pl), o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vlb, __builtin_bit_cast(am_b8, ph), o[d], 0, 0, 0);
            }
        }
    };

    // tiles alternate between two register buffers; every prefetch is
    // issued (a tile past the last key reads zeros), so the waits are exact
    T b0, b1;
    int t = lo;
    load(b0, t);
    while (true) {
        load(b1, t + AM_BK);
        tile(b0, t);
        t += AM_BK;
        if (t >= hi) break;
        load(b0, t + AM_BK);
        tile(b1, t);
        t += AM_BK;
        if (t >= hi) break;
    }
    // the head's sum over the four lane groups, then O / sum
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!cvalid) return;
    const size_t ob = (size_t)row_c * a.nq * HD + (size_t)(g * G + hq) * HD;
#pragma unroll
    for (int d = 0; d < HD / 16; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = o[d][i] / l;
            const size_t idx = ob + d * 16 + 4 * grp + i;
            if (a.out_lo) {
                const uint16_t h = f2bf(v);
                ((uint16_t *)a.out)[idx] = h;
                a.out_lo[idx] = f2bf(v - bf2f(h));
            } else {
                a.out[idx] = v;
            }
        }
}

bool attn_rows_mfma_ok(const AttnDecodeArgs &a) {
    const int G = a.nkv > 0 ? a.nq / a.nkv : 0;
    if (a.lora_on || a.n_split != 1 || G < 1 || G > 16 || a.nq % a.nkv) return false;
    return (a.hd == 64) || (a.hd == 128 && a.kv_f16);
}

void launch_attn_rows_mfma(const AttnDecodeArgs &a, hipStream_t s) {
    if (!attn_rows_mfma_ok(a)) fail(ESP_BACKEND, "attn_rows_mfma: unsupported shape");
    if (a.max_t < 1) fail(ESP_BACKEND, "attn_rows_mfma: empty key range");
    const long long units = (long long)(a.grp ? a.ngrp : a.M) * a.nkv;
    const unsigned blocks = (unsigned)units;
    if (a.hd == 64) {
        if (a.kv_f16) attn_rows_mfma_k<64, true><<<blocks, 64, 0, s>>>(a);
        else attn_rows_mfma_k<64, false><<<blocks, 64, 0, s>>>(a);
    } else {
        attn_rows_mfma_k<128, true><<<blocks, 64, 0, s>>>(a);
    }
}

}  // namespace esp
