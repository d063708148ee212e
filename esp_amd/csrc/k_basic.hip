// Bandwidth-bound kernels of the decoder forward: embedding gather, RMSNorm,
// the QKV epilogue (LoRA B-add, QK-norm, RoPE, KV append) and split-K
// attention over the per-sequence cache.
#include "common.hpp"
#include "dev.hpp"

namespace esp {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ embed
// model.rs:57-62 TokenEmbedding::forward — gather rows of [V, H].
template <typename WT>
__global__ void __launch_bounds__(256) embed_k(const WT *E, const int32_t *ids, int H, float *h) {
    int m = blockIdx.x;
    const WT *row = E + (size_t)ids[m] * H;
    for (int j = threadIdx.x; j < H; j += blockDim.x) h[(size_t)m * H + j] = ld(row, j);
}

void launch_embed(Dt wt, const void *embed, const int32_t *ids, int M, int H, float *h,
                  hipStream_t s) {
    if (wt == DT_BF16)
        embed_k<uint16_t><<<M, 256, 0, s>>>((const uint16_t *)embed, ids, H, h);
    else
        embed_k<float><<<M, 256, 0, s>>>((const float *)embed, ids, H, h);
}

// ---------------------------------------------------------------- rmsnorm
// burn-nn RmsNorm (built at layer.rs:27-33): y = x / sqrt(mean(x^2) + eps) * gamma.
template <typename OT, bool SPLIT>
__global__ void __launch_bounds__(256) rmsnorm_k(const float *x, const float *gamma, float eps,
                                                 int H, OT *out, const int32_t *row_index) {
    __shared__ float red[16];
    int m = blockIdx.x;
    int src = row_index ? row_index[m] : m;
    const float *xr = x + (size_t)src * H;
    float ss = 0.f;
    for (int j = threadIdx.x; j < H; j += blockDim.x) ss += xr[j] * xr[j];
    ss = block_sum(ss, red);
    float rms = sqrtf(ss / (float)H + eps);
    const size_t plane = (size_t)gridDim.x * H;
    for (int j = threadIdx.x; j < H; j += blockDim.x) {
        float y = (xr[j] / rms) * gamma[j];
        if (SPLIT) st_split((uint16_t *)out, plane, (size_t)m * H + j, y);
        else st(out, (size_t)m * H + j, y);
    }
}

// One wave per row for rows up to 4096 wide: the row and the norm weights
// stay in registers (NQ four-element pieces per lane, 16-byte loads issued
// together), the sum of squares is a wave reduction, and the output goes out
// four elements per store.
template <typename OT, bool SPLIT, int NQ>
__global__ void __launch_bounds__(256) rmsnorm_wave_k(const float *x, const float *gamma, float eps, int M,
                                                      int H, OT *out, const int32_t *row_index) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const int src = row_index ? row_index[m] : m;
    const float *xr = x + (size_t)src * H;
    f32x4 v[NQ], gv[NQ];  // the row and the norm weights, loaded together
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int j = (lane + 64 * i) * 4;
        v[i] = j < H ? *(const f32x4 *)(xr + j) : f32x4{0.f, 0.f, 0.f, 0.f};
        gv[i] = j < H ? *(const f32x4 *)(gamma + j) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)H + eps);
    const size_t plane = (size_t)M * H;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int j = (lane + 64 * i) * 4;
        if (j >= H) continue;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (v[i][e] / rms) * gv[i][e];
        const size_t o = (size_t)m * H + j;
        if (SPLIT) {
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hi[e] = f2bf(y[e]);
                lo[e] = f2bf(y[e] - bf2f(hi[e]));
            }
            *(uint2 *)((uint16_t *)out + o) = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            *(uint2 *)((uint16_t *)out + plane + o) =
                make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
        } else if (sizeof(OT) == 2) {
            uint16_t b[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) b[e] = f2bf(y[e]);
            *(uint2 *)((uint16_t *)out + o) = make_uint2(b[0] | ((uint32_t)b[1] << 16), b[2] | ((uint32_t)b[3] << 16));
        } else {
            *(f32x4 *)((float *)out + o) = f32x4{y[0], y[1], y[2], y[3]};
        }
    }
}

template <typename OT, bool SPLIT>
static bool rmsnorm_wave(const float *x, const float *gamma, float eps, int M, int H, OT *out,
                         const int32_t *row_index, hipStream_t s) {
    if (H % 4 || H > 4096) return false;
    const int nq = (H / 4 + 63) / 64;
    const int blocks = (M + 3) / 4;
    if (nq <= 2) rmsnorm_wave_k<OT, SPLIT, 2><<<blocks, 256, 0, s>>>(x, gamma, eps, M, H, out, row_index);
    else if (nq <= 4) rmsnorm_wave_k<OT, SPLIT, 4><<<blocks, 256, 0, s>>>(x, gamma, eps, M, H, out, row_index);
    else if (nq <= 8) rmsnorm_wave_k<OT, SPLIT, 8><<<blocks, 256, 0, s>>>(x, gamma, eps, M, H, out, row_index);
    else rmsnorm_wave_k<OT, SPLIT, 16><<<blocks, 256, 0, s>>>(x, gamma, eps, M, H, out, row_index);
    return true;
}

void launch_rmsnorm(const float *x, const float *gamma, float eps, int M, int H, Dt out_dt,
                    void *out, const int32_t *row_index, hipStream_t s) {
    if (out_dt == DT_SPLIT && rmsnorm_wave<uint16_t, true>(x, gamma, eps, M, H, (uint16_t *)out, row_index, s)) return;
    if (out_dt == DT_BF16 && rmsnorm_wave<uint16_t, false>(x, gamma, eps, M, H, (uint16_t *)out, row_index, s)) return;
    if (out_dt == DT_F32 && rmsnorm_wave<float, false>(x, gamma, eps, M, H, (float *)out, row_index, s)) return;
    if (out_dt == DT_SPLIT)
        rmsnorm_k<uint16_t, true><<<M, 256, 0, s>>>(x, gamma, eps, H, (uint16_t *)out, row_index);
    else if (out_dt == DT_BF16)
        rmsnorm_k<uint16_t, false><<<M, 256, 0, s>>>(x, gamma, eps, H, (uint16_t *)out, row_index);
    else
        rmsnorm_k<float, false><<<M, 256, 0, s>>>(x, gamma, eps, H, (float *)out, row_index);
}

// Split-K partial sums of a RESIDUAL projection fused with the RMSNorm that
// follows it (layer.rs:120-151: the o_proj residual before post-attention
// norm, the down_proj residual before the next layer's input norm). One
// block per row; thread t owns elements 4 (t + 256 i) .. + 4. The partials
// are summed from 0 in split order, eight loads in flight, then + bias and
// added to x, exactly as the GEMM reduction does; the norm is then that of
// rmsnorm_k on the new row.
template <typename OT, bool SPLIT, int NQ>
__global__ void __launch_bounds__(256) resid_norm_k(const float *ws, int splits, int M, int H,
                                                    const float *bias, float *x, const float *gamma,
                                                    float eps, OT *out) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const size_t MH = (size_t)M * H;
    f32x4 v[NQ], gv[NQ];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int j = (tid + 256 * i) * 4;
        v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (j >= H) continue;
        // gamma now, with the partials: no memory wait after the barrier
        gv[i] = *(const f32x4 *)(gamma + j);
        const size_t o = (size_t)m * H + j;
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
        for (int z0 = 0; z0 < splits; z0 += 8) {
            f32x4 pz[8];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                pz[q] = z0 + q < splits ? *(const f32x4 *)(ws + (size_t)(z0 + q) * MH + o) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (z0 + q < splits) t += pz[q];
        }
        if (bias) t = t + *(const f32x4 *)(bias + j);
        const f32x4 xv = *(const f32x4 *)(x + o) + t;
        *(f32x4 *)(x + o) = xv;
        v[i] = xv;
        ss += xv[0] * xv[0] + xv[1] * xv[1] + xv[2] * xv[2] + xv[3] * xv[3];
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int j = (tid + 256 * i) * 4;
        if (j >= H) continue;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (v[i][e] / rms) * gv[i][e];
        const size_t o = (size_t)m * H + j;
        if (SPLIT) {
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hi[e] = f2bf(y[e]);
                lo[e] = f2bf(y[e] - bf2f(hi[e]));
            }
            *(uint2 *)((uint16_t *)out + o) = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            *(uint2 *)((uint16_t *)out + MH + o) =
                make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
        } else {
            *(f32x4 *)((float *)out + o) = f32x4{y[0], y[1], y[2], y[3]};
        }
    }
}

bool resid_norm_ok(int H) { return H > 0 && H % 4 == 0 && H <= 8192; }

void launch_resid_norm(const float *ws, int splits, int M, int H, const float *bias, float *x,
                       const float *gamma, float eps, Dt out_dt, void *out, hipStream_t s) {
    if (!resid_norm_ok(H) || splits < 1 || (out_dt != DT_SPLIT && out_dt != DT_F32))
        fail(ESP_BACKEND, "resid_norm: unsupported shape");
    const int nq = (H / 4 + 255) / 256;
#define RN_LAUNCH(NQ_)                                                                                    \
    do {                                                                                                  \
        if (out_dt == DT_SPLIT)                                                                           \
            resid_norm_k<uint16_t, true, NQ_><<<M, 256, 0, s>>>(ws, splits, M, H, bias, x, gamma, eps,    \
                                                                 (uint16_t *)out);                        \
        else                                                                                              \
            resid_norm_k<float, false, NQ_><<<M, 256, 0, s>>>(ws, splits, M, H, bias, x, gamma, eps,      \
                                                               (float *)out);                             \
    } while (0)
    if (nq <= 1) RN_LAUNCH(1);
    else if (nq <= 2) RN_LAUNCH(2);
    else if (nq <= 4) RN_LAUNCH(4);
    else RN_LAUNCH(8);
#undef RN_LAUNCH
}

// ----------------------------------------------------------------- rope_kv
// attention.rs:306-326: q/k/v projections (+bias, + unmerged LoRA as in
// lora.rs:93-97), optional QK RMSNorm over head_dim (:312-319), split-half
// RoPE at the row's absolute position (:99-123), then K/V appended to the
// cache (:126-148). General form (any head_dim up to 256, mixed adapter
// ranks): a block owns a group of heads (one thread per head element) and
// up to ROPE_ROWS consecutive token rows: every row's loads
// are issued before any is used, each thread's LoRA-B row (first ROPE_BREG
// ranks) is loaded once into registers, and the rows' LoRA t values are
// staged in LDS.
constexpr int ROPE_BREG = 32, ROPE_ROWS = 16;

template <typename WT, typename KT>
__global__ void __launch_bounds__(256) rope_kv_k(RopeKvArgs a, int rows_per_block, int t_lo, int t_n) {
    extern __shared__ float sh[];  // [rows][heads_per_block * hd] values, then [rows][t_n] LoRA t
    const int hd = a.hd, half = hd / 2;
    const int hpi = blockDim.x / hd, bw = hpi * hd;
    float *tsh = sh + (size_t)rows_per_block * bw;
    const int total = a.nq + 2 * a.nkv;
    const int qw = a.nq * hd, kvw = a.nkv * hd;
    KT *cache = (KT *)a.kv;
    const int lh = threadIdx.x / hd, head = blockIdx.y * hpi + lh, d = threadIdx.x % hd;
    const bool active = lh < hpi && head < total;
    int target = 0, col = 0, off = 0;
    if (active) {
        target = head < a.nq ? 0 : (head < a.nq + a.nkv ? 1 : 2);
        off = target == 0 ? 0 : (target == 1 ? qw : qw + kvw);
        col = off + (head - (target == 0 ? 0 : (target == 1 ? a.nq : a.nq + a.nkv))) * hd + d;
    }
    const int m0 = blockIdx.x * rows_per_block;
    const int nr = min(a.rows.M - m0, rows_per_block);

    // issue every load of the block's rows
    for (int i = threadIdx.x; i < nr * t_n; i += blockDim.x)
        tsh[i] = a.qkv[(size_t)(m0 + i / t_n) * a.ldq + t_lo + i % t_n];
    float x[ROPE_ROWS];
#pragma unroll
    for (int r = 0; r < ROPE_ROWS; ++r)
        x[r] = active && r < nr ? a.qkv[(size_t)(m0 + r) * a.ldq + col] : 0.f;
    const WT *B = active ? (const WT *)a.lora_b[target] : nullptr;
    const int rank = B ? a.lora_rank[target] : 0;
    float breg[ROPE_BREG];
#pragma unroll
    for (int i = 0; i < ROPE_BREG; ++i) breg[i] = i < rank ? ld(B, (size_t)(col - off) * rank + i) : 0.f;
    __syncthreads();

    // LoRA: x += scale * B t
    if (rank) {
        const int tcol = a.lora_t_col[target] - t_lo;
        const float sc = a.lora_scale[target];
#pragma unroll
        for (int r = 0; r < ROPE_ROWS; ++r) {
            if (r >= nr) continue;
            const float *t = tsh + r * t_n + tcol;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ROPE_BREG; ++i)
                if (i < rank) acc += breg[i] * t[i];
            for (int i = ROPE_BREG; i < rank; ++i) acc += ld(B, (size_t)(col - off) * rank + i) * t[i];
            x[r] = x[r] + acc * sc;
        }
    }
    if (active) {
#pragma unroll
        for (int r = 0; r < ROPE_ROWS; ++r)
            if (r < nr) sh[r * bw + lh * hd + d] = x[r];
    }
    // QK RMSNorm over each head's hd values
    const float *g = active && target < 2 ? (target == 0 ? a.q_norm : a.k_norm) : nullptr;
    if (a.q_norm || a.k_norm) {
        __syncthreads();
        if (g) {
#pragma unroll
            for (int r = 0; r < ROPE_ROWS; ++r) {
                if (r >= nr) continue;
                const float *v = sh + r * bw + lh * hd;
                float ss = 0.f;
                for (int i = 0; i < hd; ++i) ss += v[i] * v[i];
                const float rms = sqrtf(ss / (float)hd + a.eps);
                x[r] = (x[r] / rms) * g[d];
            }
        }
        __syncthreads();
        if (g) {
#pragma unroll
            for (int r = 0; r < ROPE_ROWS; ++r)
                if (r < nr) sh[r * bw + lh * hd + d] = x[r];
        }
    }
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int r = 0; r < ROPE_ROWS; ++r) {
        if (r >= nr) continue;
        const int m = m0 + r;
        const int pos = a.rows.row_pos[m];
        const int seq = a.rows.row_seq[m];
        if (target < 2) {
            const float *v = sh + r * bw + lh * hd;
            const float rot = d < half ? -v[d + half] : v[d - half];
            const float y = x[r] * a.rope_cos[(size_t)pos * hd + d] + rot * a.rope_sin[(size_t)pos * hd + d];
            if (target == 0) {
                a.q_out[(size_t)m * qw + head * hd + d] = y;
            } else {
                const int kh = head - a.nq;
                st(cache, (size_t)seq * a.seq_stride + (size_t)kh * a.head_stride + (size_t)pos * hd + d, y);
            }
        } else {
            const int vh = head - a.nq - a.nkv;
            st(cache, (size_t)seq * a.seq_stride + a.kv_half_stride + (size_t)vh * a.head_stride +
                          (size_t)pos * hd + d, x[r]);
        }
    }
}


// Pair form (head_dim 64 or 128, every adapter of the layer of rank R or
// none): a thread owns the RoPE pair (d, d + hd/2) of one head, so the
// rotation needs no exchange. A head is one wave (hd 128) or half of one
// (hd 64, the query and kv head counts even, so the two heads of a wave
// share their target): the target (q, k or v) and the row's LoRA t values
// are wave-uniform, and the QK RMSNorm is a reduction within the head's
// lanes. B's two rows per thread sit in registers. Rows go RK2_RB at a
// time, every load of a batch issued before its first use.
constexpr int RK2_RB = 8;

template <int R, typename WT> __device__ __forceinline__ void rk2_brow(const WT *B, size_t row, float *b) {
    if constexpr (sizeof(WT) == 2) {
        const uint4 *p = (const uint4 *)((const uint16_t *)B + row * R);
#pragma unroll
        for (int k = 0; k < R / 8; ++k) {
            const uint4 u = p[k];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) b[k * 8 + e] = __uint_as_float((e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu) << 16);
        }
    } else {
        const float4 *p = (const float4 *)((const float *)B + row * R);
#pragma unroll
        for (int k = 0; k < R / 4; ++k) {
            const float4 u = p[k];
            b[k * 4] = u.x; b[k * 4 + 1] = u.y; b[k * 4 + 2] = u.z; b[k * 4 + 3] = u.w;
        }
    }
}

template <typename WT, typename KT, int R, int HD>
__global__ void __launch_bounds__(256) rope_kv2_k(const RopeKvArgs a, int rows_per_block) {
    constexpr int HALF = HD / 2, HPB = 256 / HALF;  // lanes per head, heads per block
    const int p = threadIdx.x % HALF;
    const int head = blockIdx.y * HPB + threadIdx.x / HALF;
    const int total = a.nq + 2 * a.nkv;
    if (head >= total) return;  // no barriers below
    const int target = __builtin_amdgcn_readfirstlane(head < a.nq ? 0 : (head < a.nq + a.nkv ? 1 : 2));
    const int hbase = target == 0 ? 0 : (target == 1 ? a.nq : a.nq + a.nkv);
    const int qw = a.nq * HD, kvw = a.nkv * HD;
    const int off = target == 0 ? 0 : (target == 1 ? qw : qw + kvw);
    const int hl = head - hbase;  // head within its target
    const int c0 = off + hl * HD + p, c1 = c0 + HALF;
    const float *__restrict__ qkv = a.qkv;
    const float *__restrict__ part = a.part;
    const float *__restrict__ cs = a.rope_cos;
    const float *__restrict__ sn = a.rope_sin;
    const int32_t *__restrict__ rpos = a.rows.row_pos;
    const int32_t *__restrict__ rseq = a.rows.row_seq;
    KT *__restrict__ cache = (KT *)a.kv;

    const WT *B = R ? (const WT *)a.lora_b[target] : nullptr;
    const bool lora = R && B && a.lora_rank[target] == R;
    const int tcol = a.lora_t_col[target];
    const float lsc = a.lora_scale[target];
    float b0[R ? R : 1], b1[R ? R : 1];
    if constexpr (R > 0) {
        if (lora) {
            rk2_brow<R>(B, (size_t)(c0 - off), b0);
            rk2_brow<R>(B, (size_t)(c1 - off), b1);
        }
    }
    const float *g = target == 0 ? a.q_norm : (target == 1 ? a.k_norm : nullptr);
    const float g0 = g ? g[p] : 0.f, g1 = g ? g[p + HALF] : 0.f;

    const int m0 = blockIdx.x * rows_per_block;
    const int nr = min(a.rows.M - m0, rows_per_block);
    for (int rb = 0; rb < nr; rb += RK2_RB) {
        float x0[RK2_RB], x1[RK2_RB];
        int pos[RK2_RB], sq[RK2_RB];
#pragma unroll
        for (int r = 0; r < RK2_RB; ++r) {
            const int m = m0 + min(rb + r, nr - 1);
            if (!part) {
                x0[r] = qkv[(size_t)m * a.ldq + c0];
                x1[r] = qkv[(size_t)m * a.ldq + c1];
            }
            pos[r] = rpos[m];
            sq[r] = rseq[m];
        }
        if (part) {
            // the projection's split-K partials, summed from 0 in split order
            // (eight loads in flight), then + bias, as the GEMM reduction does
            const size_t MN = (size_t)a.rows.M * a.ldq;
#pragma unroll
            for (int r = 0; r < RK2_RB; ++r) {
                const int m = m0 + min(rb + r, nr - 1);
                float t0 = 0.f, t1 = 0.f;
                if (rb + r < nr) {  // block-uniform
                    const float *__restrict__ p = part + (size_t)m * a.ldq;
                    for (int z0 = 0; z0 < a.splits; z0 += 8) {
                        float p0[8], p1[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            const size_t zo = (size_t)min(z0 + q, a.splits - 1) * MN;
                            p0[q] = p[zo + c0];
                            p1[q] = p[zo + c1];
                        }
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            if (z0 + q < a.splits) {
                                t0 += p0[q];
                                t1 += p1[q];
                            }
                    }
                    if (a.part_bias) {
                        t0 = t0 + a.part_bias[c0];
                        t1 = t1 + a.part_bias[c1];
                    }
                }
                x0[r] = t0;
                x1[r] = t1;
            }
        }
        // LoRA: x += scale * B t (the row's t values are uniform loads)
        if constexpr (R > 0) {
            if (lora) {
#pragma unroll
                for (int r = 0; r < RK2_RB; ++r) {
                    const int m = m0 + min(rb + r, nr - 1);
                    const float *__restrict__ t = qkv + (size_t)m * a.ldq + tcol;
                    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        const float ti = t[i];
                        acc0 += b0[i] * ti;
                        acc1 += b1[i] * ti;
                    }
                    x0[r] = x0[r] + acc0 * lsc;
                    x1[r] = x1[r] + acc1 * lsc;
                }
            }
        }
        // QK RMSNorm over the head's values: a reduction within its lanes
        if (g) {
#pragma unroll
            for (int r = 0; r < RK2_RB; ++r) {
                float ss = x0[r] * x0[r] + x1[r] * x1[r];
#pragma unroll
                for (int o = HALF / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, HALF);
                const float rms = sqrtf(ss / (float)HD + a.eps);
                x0[r] = (x0[r] / rms) * g0;
                x1[r] = (x1[r] / rms) * g1;
            }
        }
#pragma unroll
        for (int r = 0; r < RK2_RB; ++r) {
            if (rb + r >= nr) break;
            const int m = m0 + rb + r;
            if (target < 2) {
                const size_t tb = (size_t)pos[r] * HD + p;
                const float y0 = x0[r] * cs[tb] + (-x1[r]) * sn[tb];
                const float y1 = x1[r] * cs[tb + HALF] + x0[r] * sn[tb + HALF];
                if (target == 0) {
                    float *q = a.q_out + (size_t)m * qw + head * HD;
                    q[p] = y0;
                    q[p + HALF] = y1;
                } else {
                    const size_t ci = (size_t)sq[r] * a.seq_stride + (size_t)hl * a.head_stride + (size_t)pos[r] * HD + p;
                    st(cache, ci, y0);
                    st(cache, ci + HALF, y1);
                }
            } else {
                const size_t ci = (size_t)sq[r] * a.seq_stride + a.kv_half_stride + (size_t)hl * a.head_stride +
                                  (size_t)pos[r] * HD + p;
                st(cache, ci, x0[r]);
                st(cache, ci + HALF, x1[r]);
            }
        }
    }
}

template <typename WT, typename KT, int HD>
static bool rope_kv2_launch(const RopeKvArgs &a, hipStream_t s) {
    constexpr int HPB = 256 / (HD / 2);
    if (HD == 64 && (a.nq % 2 || a.nkv % 2)) return false;  // two heads per wave share a target
    int rank = 0;
    for (int j = 0; j < 3; ++j) {
        if (!a.lora_b[j] || !a.lora_rank[j]) continue;
        if (rank && a.lora_rank[j] != rank) return false;
        rank = a.lora_rank[j];
    }
    // rows per block: measured at the C3 prefill (2048 rows, LoRA on q/v) 32 /
    // 16 / 8 / 4 rows: 41.7 / 39.1 / 36.2 / 45.4 us per launch
    const int rpb = a.rows.M >= 128 ? 8 : 1;
    dim3 grid((a.rows.M + rpb - 1) / rpb, (a.nq + 2 * a.nkv + HPB - 1) / HPB);
    switch (rank) {
    case 0: rope_kv2_k<WT, KT, 0, HD><<<grid, 256, 0, s>>>(a, rpb); return true;
    case 8: rope_kv2_k<WT, KT, 8, HD><<<grid, 256, 0, s>>>(a, rpb); return true;
    case 16: rope_kv2_k<WT, KT, 16, HD><<<grid, 256, 0, s>>>(a, rpb); return true;
    case 32: rope_kv2_k<WT, KT, 32, HD><<<grid, 256, 0, s>>>(a, rpb); return true;
    default: return false;
    }
}

bool rope_kv_fusable(Dt wt, Dt kvdt, int hd, int nq, int nkv, bool lora) {
    const bool dts = (wt == DT_BF16 && (kvdt == DT_F16 || kvdt == DT_F32)) || (wt == DT_F32 && kvdt == DT_F32);
    return dts && !lora && (hd == 128 || (hd == 64 && nq % 2 == 0 && nkv % 2 == 0));
}

void launch_rope_kv(Dt wt, Dt kvdt, const RopeKvArgs &a, hipStream_t s) {
    if (a.hd > 256) fail(ESP_UNSUPPORTED, "head_dim: values above 256 are not implemented");
    if (a.part) {
        bool lora = false;
        for (int j = 0; j < 3; ++j) lora |= a.lora_b[j] && a.lora_rank[j];
        if (!rope_kv_fusable(wt, kvdt, a.hd, a.nq, a.nkv, lora) || a.splits < 1)
            fail(ESP_BACKEND, "rope_kv: split-K partials need the pair form");
    }
    bool done = false;
    if (a.hd == 128) {
        if (wt == DT_BF16 && kvdt == DT_F16) done = rope_kv2_launch<uint16_t, _Float16, 128>(a, s);
        else if (wt == DT_BF16 && kvdt == DT_F32) done = rope_kv2_launch<uint16_t, float, 128>(a, s);
        else if (wt == DT_F32 && kvdt == DT_F32) done = rope_kv2_launch<float, float, 128>(a, s);
    } else if (a.hd == 64) {
        if (wt == DT_BF16 && kvdt == DT_F16) done = rope_kv2_launch<uint16_t, _Float16, 64>(a, s);
        else if (wt == DT_BF16 && kvdt == DT_F32) done = rope_kv2_launch<uint16_t, float, 64>(a, s);
        else if (wt == DT_F32 && kvdt == DT_F32) done = rope_kv2_launch<float, float, 64>(a, s);
    }
    if (done) return;
    if (a.part) fail(ESP_BACKEND, "rope_kv: split-K partials need the pair form");
    const int hpi = 256 / a.hd;
    // contiguous span of LoRA t columns read by this layer
    int t_lo = 0, t_hi = 0;
    bool any = false;
    for (int j = 0; j < 3; ++j) {
        if (!a.lora_b[j] || !a.lora_rank[j]) continue;
        const int c0 = a.lora_t_col[j], c1 = c0 + a.lora_rank[j];
        t_lo = any ? std::min(t_lo, c0) : c0;
        t_hi = any ? std::max(t_hi, c1) : c1;
        any = true;
    }
    const int t_n = t_hi - t_lo;
    const size_t per_row = sizeof(float) * ((size_t)hpi * a.hd + t_n);
    const size_t lds_cap = 64 * 1024;
    if (per_row > lds_cap) fail(ESP_UNSUPPORTED, "lora: total adapter rank too large for one layer");
    int rpb = a.rows.M >= 1024 ? ROPE_ROWS : (a.rows.M >= 128 ? 4 : 1);
    while (rpb > 1 && rpb * per_row > lds_cap) rpb /= 2;
    const size_t shm = rpb * per_row;
    dim3 grid((a.rows.M + rpb - 1) / rpb, (a.nq + 2 * a.nkv + hpi - 1) / hpi);
    if (wt == DT_BF16 && kvdt == DT_F16)
        rope_kv_k<uint16_t, _Float16><<<grid, 256, shm, s>>>(a, rpb, t_lo, t_n);
    else if (wt == DT_BF16 && kvdt == DT_F32)
        rope_kv_k<uint16_t, float><<<grid, 256, shm, s>>>(a, rpb, t_lo, t_n);
    else if (wt == DT_F32 && kvdt == DT_F32)
        rope_kv_k<float, float><<<grid, 256, shm, s>>>(a, rpb, t_lo, t_n);
    else
        fail(ESP_BACKEND, "rope_kv: unsupported dtype pair");
}

// --------------------------------------------------------------- attention
// attention.rs:345-397: softmax((q.k)/sqrt(hd) + mask) . v, with the causal
// rule `key > past + query` and the sliding rule `pos - key >= window`
// (:362-368). GQA: q head i reads kv head i / group (:333-343), served here
// by one block per (row, kv head, key split) without materialising copies.
// Partials (running max, sum, unnormalised output) are merged by
// attn_reduce_k.
constexpr int ATT_KT = 32;  // keys per LDS tile

template <typename KT>
__global__ void __launch_bounds__(256) attn_split_k(AttnArgs a) {
    extern __shared__ float sm[];
    const int split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;
    const int hd = a.hd, G = a.nq / a.nkv;
    const int pos = a.rows.row_pos[row], seq = a.rows.row_seq[row];
    int lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
    int hi = pos + 1;
    lo = max(lo, split * a.split_len);
    hi = min(hi, (split + 1) * a.split_len);
    float *qs = sm;                        // [G][hd]
    float *ks = qs + G * hd;               // [KT][hd+1]
    float *vs = ks + ATT_KT * (hd + 1);    // [KT][hd]
    float *ss = vs + ATT_KT * hd;          // [G][KT]
    float *mrow = ss + G * ATT_KT;         // [G] running max
    float *lrow = mrow + G;                // [G] running sum
    float *alpha = lrow + G;               // [G] rescale for this tile
    const int tid = threadIdx.x;
    const size_t pbase = (((size_t)row * a.nq + (size_t)g * G) * a.n_split + split) * (hd + 2);
    if (lo >= hi) {
        for (int i = tid; i < G * (hd + 2); i += blockDim.x) {
            int j = i / (hd + 2), c = i % (hd + 2);
            float *p = a.part + pbase + (size_t)j * a.n_split * (hd + 2);
            p[c] = c == 0 ? -INFINITY : 0.f;
        }
        return;
    }
    const float scale = sqrtf((float)hd);
    const float *qrow = a.q + (size_t)row * a.nq * hd + (size_t)g * G * hd;
    for (int i = tid; i < G * hd; i += blockDim.x) qs[i] = qrow[i];
    if (tid < G) {
        mrow[tid] = -INFINITY;
        lrow[tid] = 0.f;
    }
    // each thread owns outputs (j, d) = o, o + 256, ...
    constexpr int MAXO = 8;  // G*hd <= 2048
    float acc[MAXO];
#pragma unroll
    for (int i = 0; i < MAXO; ++i) acc[i] = 0.f;
    const KT *kbase = (const KT *)a.kv + (size_t)seq * a.seq_stride + (size_t)g * a.head_stride;
    const KT *vbase = kbase + a.kv_half_stride;
    for (int t0 = lo; t0 < hi; t0 += ATT_KT) {
        const int nt = min(ATT_KT, hi - t0);
        __syncthreads();
        for (int i = tid; i < nt * hd; i += blockDim.x) {
            int t = i / hd, d = i % hd;
            ks[t * (hd + 1) + d] = ld(kbase, (size_t)(t0 + t) * hd + d);
            vs[t * hd + d] = ld(vbase, (size_t)(t0 + t) * hd + d);
        }
        __syncthreads();
        for (int i = tid; i < G * ATT_KT; i += blockDim.x) {
            int j = i / ATT_KT, t = i % ATT_KT;
            float s = -INFINITY;
            if (t < nt) {
                float dot = 0.f;
                for (int d = 0; d < hd; ++d) dot += qs[j * hd + d] * ks[t * (hd + 1) + d];
                s = dot / scale;
            }
            ss[j * ATT_KT + t] = s;
        }
        __syncthreads();
        if (tid < G) {
            float mx = mrow[tid];
            for (int t = 0; t < nt; ++t) mx = fmaxf(mx, ss[tid * ATT_KT + t]);
            float al = __expf(mrow[tid] - mx);
            float l = lrow[tid] * al;
            for (int t = 0; t < nt; ++t) {
                float p = __expf(ss[tid * ATT_KT + t] - mx);
                ss[tid * ATT_KT + t] = p;
                l += p;
            }
            mrow[tid] = mx;
            lrow[tid] = l;
            alpha[tid] = al;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < MAXO; ++i) {
            int o = tid + i * blockDim.x;
            if (o < G * hd) {
                int j = o / hd, d = o % hd;
                float v = acc[i] * alpha[j];
                for (int t = 0; t < nt; ++t) v += ss[j * ATT_KT + t] * vs[t * hd + d];
                acc[i] = v;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MAXO; ++i) {
        int o = tid + i * blockDim.x;
        if (o < G * hd) {
            int j = o / hd, d = o % hd;
            a.part[pbase + (size_t)j * a.n_split * (hd + 2) + 2 + d] = acc[i];
        }
    }
    if (tid < G) {
        float *p = a.part + pbase + (size_t)tid * a.n_split * (hd + 2);
        p[0] = mrow[tid];
        p[1] = lrow[tid];
    }
}

template <typename OT, bool SPLIT>
__global__ void __launch_bounds__(256) attn_reduce_k(AttnArgs a, OT *out) {
    const int qh = blockIdx.x, row = blockIdx.y;
    const int hd = a.hd;
    const float *p = a.part + ((size_t)row * a.nq + qh) * a.n_split * (hd + 2);
    float mx = -INFINITY;
    for (int s = 0; s < a.n_split; ++s) mx = fmaxf(mx, p[(size_t)s * (hd + 2)]);
    float l = 0.f;
    for (int s = 0; s < a.n_split; ++s) {
        float ms = p[(size_t)s * (hd + 2)];
        if (ms != -INFINITY) l += p[(size_t)s * (hd + 2) + 1] * __expf(ms - mx);
    }
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float v = 0.f;
        for (int s = 0; s < a.n_split; ++s) {
            float ms = p[(size_t)s * (hd + 2)];
            if (ms != -INFINITY) v += p[(size_t)s * (hd + 2) + 2 + d] * __expf(ms - mx);
        }
        const size_t i = (size_t)row * a.nq * hd + (size_t)qh * hd + d;
        if (SPLIT) st_split((uint16_t *)out, (size_t)a.rows.M * a.nq * hd, i, v / l);
        else st(out, i, v / l);
    }
}

void launch_attention(Dt kvdt, const AttnArgs &a, hipStream_t s) {
    const int G = a.nq / a.nkv;
    if (G * a.hd > 8 * 256) fail(ESP_UNSUPPORTED, "attention: group*head_dim above 2048");
    size_t shm = sizeof(float) * ((size_t)G * a.hd + ATT_KT * (a.hd + 1) + ATT_KT * a.hd +
                                  (size_t)G * ATT_KT + 3 * G);
    dim3 grid(a.n_split, a.nkv, a.rows.M);
    if (kvdt != DT_F16 && kvdt != DT_F32) fail(ESP_BACKEND, "attention: unsupported cache type");
    if (shm > 64 * 1024) {
        static bool set[2] = {false, false};
        int i = kvdt == DT_F16;
        if (!set[i]) {
            ESP_HIP(hipFuncSetAttribute(i ? (const void *)attn_split_k<_Float16>
                                          : (const void *)attn_split_k<float>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
            set[i] = true;
        }
    }
    if (kvdt == DT_F16)
        attn_split_k<_Float16><<<grid, 256, shm, s>>>(a);
    else
        attn_split_k<float><<<grid, 256, shm, s>>>(a);
    dim3 g2(a.nq, a.rows.M);
    int th = a.hd >= 64 ? 64 * ((a.hd + 63) / 64) : 64;
    if (th > 256) th = 256;
    if (a.out_dt == DT_SPLIT)
        attn_reduce_k<uint16_t, true><<<g2, th, 0, s>>>(a, (uint16_t *)a.out);
    else if (a.out_dt == DT_BF16)
        attn_reduce_k<uint16_t, false><<<g2, th, 0, s>>>(a, (uint16_t *)a.out);
    else
        attn_reduce_k<float, false><<<g2, th, 0, s>>>(a, (float *)a.out);
}

// ------------------------------------------------------------ generation
// Device-side token hand-off for the captured decode step. gen[0] = token
// fed to the next step, gen[1] = step index, gen[3] = its position,
// gen[8 + i] = i-th generated id.
__global__ void gen_step_k(const uint32_t *picked, int32_t *gen) {
    int32_t t = (int32_t)picked[0];
    gen[0] = t;
    gen[8 + gen[1]] = t;
    gen[1] += 1;
    gen[3] += 1;
}

void launch_gen_step(const uint32_t *picked, int32_t *gen, hipStream_t s) {
    gen_step_k<<<1, 1, 0, s>>>(picked, gen);
}

}  // namespace esp
