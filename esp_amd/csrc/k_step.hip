// Persistent single-token decode step: one launch runs the embedding lookup,
// every layer and the head of a decode step for one row (model.rs:502-539,
// layer.rs:115-151, attention.rs:306-403 at one position).
//
// The grid is one round of resident blocks. Phases are separated by a grid
// barrier (group counters, then one global counter and a generation word);
// data handed from one phase to the next is written with agent-scope
// (write-through) stores and read with agent-scope loads, so no L2 of any
// XCD can serve a stale copy. Every GEMV phase issues its first weight loads
// before it waits at the barrier that precedes it, so the weight stream of
// the next projection is already in flight while the grid synchronises.
//
// Phases per layer: [LoRA t = A.norm(h)] -> q/k/v + RoPE + K/V append ->
// attention over key splits -> merge of the splits -> o_proj (+h) ->
// gate/up SwiGLU -> down_proj (+h); then the head with a greedy argmax.
// The arithmetic of each phase follows the single-kernel decode path
// (k_decode.hip): per-row dot products over four K quarters summed in wave
// order, online softmax per key chunk, split partials merged in split order.
#include "common.hpp"
#include "decode.hpp"
#include "decode_dev.hpp"
#include "dev.hpp"
#include "step.hpp"

namespace esp {

typedef unsigned long long u64_t;

__device__ __forceinline__ unsigned ldu_agent(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stu_agent(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned addu_agent(unsigned *p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// two floats with one agent-scope 8-byte load (p 8-byte aligned)
__device__ __forceinline__ void ld_agent2(const float *p, float &x, float &y) {
    const u64_t v = __hip_atomic_load((const u64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    x = __uint_as_float((unsigned)v);
    y = __uint_as_float((unsigned)(v >> 32));
}
__device__ __forceinline__ f32x4_t ld_agent4(const float *p) {
    float x0, x1, x2, x3;
    ld_agent2(p, x0, x1);
    ld_agent2(p + 2, x2, x3);
    return f32x4_t{x0, x1, x2, x3};
}

// ------------------------------------------------------------ grid barrier
// bar words: [0] groups arrived, [1] generation, [2] error, [32 + 32 g]
// arrivals of block group g (blockIdx % SB_GROUPS; one 128-byte line each).
// A wait longer than SB_TIMEOUT (wall clock, 100 MHz) sets the error word
// and every block leaves the kernel at its next barrier.
constexpr int SB_GROUPS = 8;
constexpr u64_t SB_TIMEOUT = 200000000ull;  // 2 s

__device__ __forceinline__ bool grid_sync(unsigned *bar) {
    __shared__ unsigned quit;
    wait_stores();  // this wave's stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned nb = gridDim.x, grp = blockIdx.x % SB_GROUPS;
        const unsigned gsize = (nb - grp + SB_GROUPS - 1) / SB_GROUPS;
        const unsigned gen = ldu_agent(bar + 1);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // generation read before arriving
        bool last = false;
        if (addu_agent(bar + 32 + 32 * grp, 1u) == gsize - 1) {
            stu_agent(bar + 32 + 32 * grp, 0u);
            wait_stores();  // group counter reset before the global arrival
            last = addu_agent(bar, 1u) == SB_GROUPS - 1;
        }
        if (last) {
            stu_agent(bar, 0u);
            wait_stores();
            stu_agent(bar + 1, gen + 1);
        } else {
            const u64_t t0 = wall_clock64();
            while (ldu_agent(bar + 1) == gen) {
                __builtin_amdgcn_s_sleep(1);
                if (ldu_agent(bar + 2) || wall_clock64() - t0 > SB_TIMEOUT) {
                    stu_agent(bar + 2, 1u);
                    break;
                }
            }
        }
        quit = ldu_agent(bar + 2);
    }
    __syncthreads();
    return quit != 0;
}

// ------------------------------------------------------------ GEMV phases
struct GemvP {
    const uint16_t *w, *w2;  // weight rows (SWIGLU: gate, up)
    const float *x;          // input vector (written by an earlier phase)
    const float *gamma;      // nullable: fused RMSNorm of x
    const float *bias;       // nullable
    float *y;
    int units, K;
    const StepLayer *ly;     // QKVROPE: bias / LoRA of the layer
    float *kvl;              // QKVROPE: layer base of the cache
};

struct StepShared {
    float red[DG_MAX_IT][4][DG_WAVES];
    float ssq[DG_WAVES];
    float best_v[DG_WAVES];
    int best_i[DG_WAVES];
};

template <int EPI, int NCH> constexpr int step_rb() {
    return RowsPerUnit<EPI>::v == 2 ? (NCH <= 2 ? 2 : 1) : (NCH <= 2 ? 4 : (NCH <= 4 ? 2 : 1));
}

template <int EPI, int NCH> struct GemvPhase {
    static constexpr int RB = step_rb<EPI, NCH>();
    static constexpr int RU = RowsPerUnit<EPI>::v, R = RB * RU;
    Chunk<uint16_t> wc[R][NCH];

    __device__ __forceinline__ void load(const StepArgs &a, const GemvP &p, int u0) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int kq = p.K / DG_WAVES, nch = kq / 8, k0 = wave * kq;
        const uint16_t *rp[R];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int u = min(u0 + r, p.units - 1);
            if (EPI == DG_SWIGLU) {
                rp[r * 2] = p.w + (size_t)u * p.K;
                rp[r * 2 + 1] = p.w2 + (size_t)u * p.K;
            } else if (EPI == DG_QKVROPE) {
                const int half = a.hd / 2, head = u / half, d = u % half;
                const int row = head * a.hd + d;
                rp[r * 2] = p.w + (size_t)row * p.K;
                rp[r * 2 + 1] = p.w + (size_t)(row + half) * p.K;
            } else {
                rp[r] = p.w + (size_t)u * p.K;
            }
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int ch = lane + 64 * c;
            if (ch < nch) {
#pragma unroll
                for (int r = 0; r < R; ++r) wc[r][c].load(rp[r] + k0 + ch * 8);
            }
        }
    }

    __device__ __forceinline__ void prefetch(const StepArgs &a, const GemvP &p) {
        if ((int)blockIdx.x * RB < p.units) load(a, p, blockIdx.x * RB);
    }

    __device__ __forceinline__ void epilogue(const StepArgs &a, const GemvP &p, int u, const float *y,
                                             float &bv, int &bi) {
        if (EPI == DG_STORE) {
            st_agent(p.y + u, p.bias ? y[0] + p.bias[u] : y[0]);
        } else if (EPI == DG_RESID) {
            const float v = p.bias ? y[0] + p.bias[u] : y[0];
            st_agent(p.y + u, ld_agent(p.y + u) + v);
        } else if (EPI == DG_SWIGLU) {
            st_agent(p.y + u, silu(y[0]) * y[1]);
        } else if (EPI == DG_HEAD) {
            p.y[u] = y[0];
            if (y[0] > bv || (y[0] == bv && u < bi)) {
                bv = y[0];
                bi = u;
            }
        } else {  // DG_QKVROPE
            const int hd = a.hd, half = hd / 2, head = u / half, d = u % half;
            const int r0 = head * hd + d, r1 = r0 + half;
            float v0 = y[0], v1 = y[1];
            if (p.bias) {
                v0 = v0 + p.bias[r0];
                v1 = v1 + p.bias[r1];
            }
            const StepLayer &ly = *p.ly;
            if (ly.lora_rows) {  // unmerged LoRA, before RoPE (lora.rs:93-97)
                const int j = head < a.nq ? 0 : (head < a.nq + a.nkv ? 1 : 2);
                if (ly.lora_b[j]) {
                    const uint16_t *B = (const uint16_t *)ly.lora_b[j];
                    const int rank = ly.lora_rank[j];
                    const int off = j == 0 ? 0 : (j == 1 ? a.nq * hd : (a.nq + a.nkv) * hd);
                    const float *t = a.t + ly.lora_t_col[j];
                    float c0 = 0.f, c1 = 0.f;
                    for (int i = 0; i < rank; ++i) {
                        const float ti = ld_agent(t + i);
                        c0 += bf2f(B[(size_t)(r0 - off) * rank + i]) * ti;
                        c1 += bf2f(B[(size_t)(r1 - off) * rank + i]) * ti;
                    }
                    v0 = v0 + c0 * ly.lora_scale[j];
                    v1 = v1 + c1 * ly.lora_scale[j];
                }
            }
            const int pos = a.row_pos[0], seq = a.row_seq[0];
            const float *cs = a.rope_cos + (size_t)pos * hd;
            const float *sn = a.rope_sin + (size_t)pos * hd;
            if (head < a.nq + a.nkv) {
                const float o0 = v0 * cs[d] + (-v1) * sn[d];
                const float o1 = v1 * cs[d + half] + v0 * sn[d + half];
                if (head < a.nq) {
                    st_agent(a.q + r0, o0);
                    st_agent(a.q + r1, o1);
                } else {
                    float *kc = p.kvl + (size_t)seq * a.seq_stride +
                                (size_t)(head - a.nq) * a.head_stride + (size_t)pos * hd;
                    st_agent(kc + d, o0);
                    st_agent(kc + d + half, o1);
                }
            } else {
                float *vc = p.kvl + (size_t)seq * a.seq_stride + a.kv_half_stride +
                            (size_t)(head - a.nq - a.nkv) * a.head_stride + (size_t)pos * hd;
                st_agent(vc + d, v0);
                st_agent(vc + d + half, v1);
            }
        }
    }

    __device__ __forceinline__ void run(const StepArgs &a, const GemvP &p, StepShared &sm) {
        const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
        const int K = p.K, kq = K / DG_WAVES, nch = kq / 8, k0 = wave * kq;
        float xr[NCH][8];
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int ch = lane + 64 * c;
            if (ch < nch) {
                const float *xp = p.x + k0 + ch * 8;
#pragma unroll
                for (int i = 0; i < 4; ++i) ld_agent2(xp + 2 * i, xr[c][2 * i], xr[c][2 * i + 1]);
#pragma unroll
                for (int i = 0; i < 8; ++i) ss += xr[c][i] * xr[c][i];
            }
        }
        if (p.gamma) {
            ss = wave_sum(ss);
            if (lane == 0) sm.ssq[wave] = ss;
            __syncthreads();
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < DG_WAVES; ++w) tot += sm.ssq[w];
            const float rms = sqrtf(tot / (float)K + a.eps);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int ch = lane + 64 * c;
                if (ch < nch) {
                    const float *g = p.gamma + k0 + ch * 8;
#pragma unroll
                    for (int i = 0; i < 8; ++i) xr[c][i] = (xr[c][i] / rms) * g[i];
                }
            }
        }
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        const int stride = gridDim.x * RB;
        int u0 = blockIdx.x * RB;
        while (u0 < p.units) {  // rounds of at most DG_MAX_IT iterations
            const int ubase = u0;
            int it = 0;
            for (; it < DG_MAX_IT && u0 < p.units; ++it, u0 += stride) {
                float acc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const int ch = lane + 64 * c;
                    if (ch < nch) {
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[r] += wc[r][c].dot(xr[c]);
                    }
                }
                if (u0 + stride < p.units) load(a, p, u0 + stride);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float v = wave_sum_uniform(acc[r]);
                    if (lane == 0) sm.red[it][r][wave] = v;
                }
            }
            __syncthreads();
            for (int e = tid; e < it * RB; e += blockDim.x) {
                const int ii = e / RB, r = e % RB;
                const int u = ubase + ii * stride + r;
                if (u >= p.units) continue;
                float y[RU];
#pragma unroll
                for (int j = 0; j < RU; ++j) {
                    float t = 0.f;
#pragma unroll
                    for (int w = 0; w < DG_WAVES; ++w) t += sm.red[ii][r * RU + j][w];
                    y[j] = t;
                }
                epilogue(a, p, u, y, bv, bi);
            }
            __syncthreads();
        }
        if (EPI == DG_HEAD) {  // this block's best (value, lowest id)
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (lane == 0) {
                sm.best_v[wave] = bv;
                sm.best_i[wave] = bi;
            }
            __syncthreads();
            if (tid == 0) {
                float b = sm.best_v[0];
                int bj = sm.best_i[0];
                for (int w = 1; w < DG_WAVES; ++w)
                    if (sm.best_v[w] > b || (sm.best_v[w] == b && sm.best_i[w] < bj)) {
                        b = sm.best_v[w];
                        bj = sm.best_i[w];
                    }
                st_agent(a.part_v + blockIdx.x, b);
                st_agent(a.part_i + blockIdx.x, bj);
            }
        }
    }
};

// prefetch the phase's first weights, wait for the previous phase, run
template <int EPI, int NCH>
__device__ __forceinline__ bool gemv_step(const StepArgs &a, const GemvP &p, StepShared &sm) {
    GemvPhase<EPI, NCH> ph;
    ph.prefetch(a, p);
    if (grid_sync(a.bar)) return true;
    ph.run(a, p, sm);
    return false;
}

// Widths up to 8192 (4 chunks per lane) for every phase; the residual
// phases (o_proj, down_proj: K = query width or ffn width) also up to 16384.
template <int EPI>
__device__ __forceinline__ bool gemv_phase(const StepArgs &a, const GemvP &p, int nch, StepShared &sm) {
    switch (nch) {
        case 1: return gemv_step<EPI, 1>(a, p, sm);
        case 2: return gemv_step<EPI, 2>(a, p, sm);
        case 4: return gemv_step<EPI, 4>(a, p, sm);
        default: return gemv_step<EPI, EPI == DG_RESID ? DG_MAXC : 4>(a, p, sm);
    }
}

// ------------------------------------------------------------ attention
// keys whose K/V loads a block issues at once (fewer for 8-head groups,
// whose q and accumulators take twice the registers)
template <int GM> constexpr int step_att_chunk() { return GM <= 4 ? 64 : 32; }
// Key split `split` of kv head g for the row: as attn_decode_k, with q read
// by agent loads and the row's own key/value (written this step) too.
template <int HD, int GM>
__device__ __forceinline__ void attn_item(const StepArgs &a, const float *kvl, int window, int split, int g) {
    constexpr int NW = 4;
    constexpr int DPL = 8, LPK = HD / DPL, KPW = 64 / LPK, NS = step_att_chunk<GM>() / (NW * KPW);
    constexpr int STRIDE = HD + ATT_PART_PAD;
    __shared__ float wm[NW][GM], wl[NW][GM];
    __shared__ float wacc[NW][GM][HD];
    const int G = a.nq / a.nkv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp = lane / LPK, sub = lane % LPK;
    const int pos = a.row_pos[0], seq = a.row_seq[0];
    int lo = window > 0 ? max(0, pos - window + 1) : 0;
    int hi = pos + 1;
    lo = max(lo, split * a.split_len);
    hi = min(hi, (split + 1) * a.split_len);
    const float inv_scale = 1.f / sqrtf((float)HD);
    float q[GM][DPL];
    const float *qrow = a.q + (size_t)g * G * HD + sub * DPL;
#pragma unroll
    for (int j = 0; j < GM; ++j)
        if (j < G) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ld_agent2(qrow + (size_t)j * HD + 2 * i, q[j][2 * i], q[j][2 * i + 1]);
        }
    float m[GM], l[GM], acc[GM][DPL];
#pragma unroll
    for (int j = 0; j < GM; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
    }
    const float *kb = kvl + (size_t)seq * a.seq_stride + (size_t)g * a.head_stride + sub * DPL;
    const float *vb = kb + a.kv_half_stride;
    for (int c0 = lo; c0 < hi; c0 += NS * NW * KPW) {
        f32x4_t kk[NS][2], vv[NS][2];
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const int t = c0 + st * NW * KPW + wave * KPW + grp;
            kk[st][0] = kk[st][1] = vv[st][0] = vv[st][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (t < hi && t != pos) {
                kk[st][0] = *(const f32x4_t *)(kb + (size_t)t * HD);
                kk[st][1] = *(const f32x4_t *)(kb + (size_t)t * HD + 4);
                vv[st][0] = *(const f32x4_t *)(vb + (size_t)t * HD);
                vv[st][1] = *(const f32x4_t *)(vb + (size_t)t * HD + 4);
            } else if (t == pos && t < hi) {  // written by this step's q/k/v phase
                const float *kp = kb + (size_t)t * HD, *vp = vb + (size_t)t * HD;
                kk[st][0] = ld_agent4(kp);
                kk[st][1] = ld_agent4(kp + 4);
                vv[st][0] = ld_agent4(vp);
                vv[st][1] = ld_agent4(vp + 4);
            }
        }
#pragma unroll
        for (int j = 0; j < GM; ++j) {
            if (j >= G) break;
            float sc[NS];
            float mx = m[j];
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) d += q[j][e] * kk[st][0][e];
#pragma unroll
                for (int e = 0; e < 4; ++e) d += q[j][4 + e] * kk[st][1][e];
                d = group_sum<LPK>(d);
                const int t = c0 + st * NW * KPW + wave * KPW + grp;
                sc[st] = t < hi ? d * inv_scale : -INFINITY;
                mx = fmaxf(mx, sc[st]);
            }
            if (mx == -INFINITY) continue;
            const float al = __expf(m[j] - mx);
            l[j] *= al;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[j][e] *= al;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const float pr = __expf(sc[st] - mx);
                l[j] += pr;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][e] += pr * vv[st][0][e];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][4 + e] += pr * vv[st][1][e];
            }
            m[j] = mx;
        }
    }
    // merge the key groups of the wave, then the waves; publish the partial
#pragma unroll
    for (int j = 0; j < GM; ++j) {
        if (j >= G) break;
#pragma unroll
        for (int o = LPK; o < 64; o <<= 1) {
            const float om = __shfl_xor(m[j], o, 64), ol = __shfl_xor(l[j], o, 64);
            const float mn = fmaxf(m[j], om);
            const float s1 = mn == -INFINITY ? 0.f : __expf(m[j] - mn);
            const float s2 = mn == -INFINITY ? 0.f : __expf(om - mn);
            l[j] = l[j] * s1 + ol * s2;
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float oa = __shfl_xor(acc[j][i], o, 64);
                acc[j][i] = acc[j][i] * s1 + oa * s2;
            }
            m[j] = mn;
        }
        if (grp == 0) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) wacc[wave][j][sub * DPL + i] = acc[j][i];
            if (sub == 0) {
                wm[wave][j] = m[j];
                wl[wave][j] = l[j];
            }
        }
    }
    __syncthreads();
    for (int o = tid; o < G * HD; o += blockDim.x) {
        const int j = o / HD, d = o % HD;
        float mx = -INFINITY;
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wm[w][j]);
        float L = 0.f, v = 0.f;
        for (int w = 0; w < NW; ++w) {
            const float sc = mx == -INFINITY ? 0.f : __expf(wm[w][j] - mx);
            L += wl[w][j] * sc;
            v += wacc[w][j][d] * sc;
        }
        float *pp = a.part + ((size_t)(g * G + j) * a.n_split + split) * STRIDE;
        st_agent(pp + ATT_PART_PAD + d, v);
        if (d == 0) {
            st_agent(pp, mx);
            st_agent(pp + 1, L);
        }
    }
    __syncthreads();  // LDS reused by the block's next item
}

// Merge of the splits of query head qh in split order (deterministic).
template <int HD>
__device__ __forceinline__ void merge_item(const StepArgs &a, int qh) {
    constexpr int STRIDE = HD + ATT_PART_PAD;
    constexpr int MB = 32;
    __shared__ float mm[ATT_MAX_SPLIT_STEP], ww[ATT_MAX_SPLIT_STEP];
    __shared__ float LL;
    const int tid = threadIdx.x, ns = a.n_split;
    const float *pb = a.part + (size_t)qh * ns * STRIDE;
    for (int i = tid; i < ns; i += blockDim.x) {
        mm[i] = ld_agent(pb + (size_t)i * STRIDE);
        ww[i] = ld_agent(pb + (size_t)i * STRIDE + 1);
    }
    __syncthreads();
    if (tid < 64) {
        const int s0 = tid, s1 = tid + 64;  // ns <= 128
        const float m0 = s0 < ns ? mm[s0] : -INFINITY, m1 = s1 < ns ? mm[s1] : -INFINITY;
        const float mx = wave_max(fmaxf(m0, m1));
        const float w0 = m0 == -INFINITY ? 0.f : __expf(m0 - mx);
        const float w1 = m1 == -INFINITY ? 0.f : __expf(m1 - mx);
        const float L = wave_sum((s0 < ns ? ww[s0] * w0 : 0.f) + (s1 < ns ? ww[s1] * w1 : 0.f));
        if (s0 < ns) ww[s0] = w0;
        if (s1 < ns) ww[s1] = w1;
        if (tid == 0) LL = L;
    }
    __syncthreads();
    for (int d = tid; d < HD; d += blockDim.x) {
        const float *p0 = pb + ATT_PART_PAD + d;
        float v = 0.f;
        for (int sp0 = 0; sp0 < ns; sp0 += MB) {
            float t0[MB];
#pragma unroll
            for (int q = 0; q < MB; ++q) t0[q] = sp0 + q < ns ? ld_agent(p0 + (size_t)(sp0 + q) * STRIDE) : 0.f;
#pragma unroll
            for (int q = 0; q < MB; ++q)
                if (sp0 + q < ns) v += t0[q] * ww[sp0 + q];
        }
        st_agent(a.attn + (size_t)qh * HD + d, v / LL);
    }
    __syncthreads();
}

// ------------------------------------------------------------ the step
template <int HD, int GM>
__global__ void __launch_bounds__(DG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) step_k(StepArgs a) {
    __shared__ StepShared sm;
    const int H = a.H, qw = a.nq * a.hd;
    // embedding row (model.rs:514)
    {
        const int tok = a.ids[0];
        const uint16_t *e = (const uint16_t *)a.embed + (size_t)tok * H;
        for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < H; k += gridDim.x * blockDim.x)
            st_agent(a.h + k, bf2f(e[k]));
    }
    for (int l = 0; l < a.L; ++l) {
        const StepLayer *ly = a.layers + l;
        float *kvl = a.kv + (size_t)l * a.layer_stride;
        const int qkv_n = qw + 2 * a.nkv * a.hd;
        if (ly->lora_rows) {  // t = A . norm(h) for the LoRA targets
            GemvP p{};
            p.w = (const uint16_t *)ly->qkv + (size_t)qkv_n * H;
            p.x = a.h;
            p.gamma = ly->in_norm;
            p.y = a.t;
            p.units = ly->lora_rows;
            p.K = H;
            if (gemv_phase<DG_STORE>(a, p, a.nch_h, sm)) return;
        }
        {
            GemvP p{};
            p.w = (const uint16_t *)ly->qkv;
            p.x = a.h;
            p.gamma = ly->in_norm;
            p.bias = ly->qkv_bias;
            p.units = qkv_n / 2;
            p.K = H;
            p.ly = ly;
            p.kvl = kvl;
            if (gemv_phase<DG_QKVROPE>(a, p, a.nch_h, sm)) return;
        }
        if (grid_sync(a.bar)) return;
        for (int it = blockIdx.x; it < a.n_split * a.nkv; it += gridDim.x)
            attn_item<HD, GM>(a, kvl, ly->window, it % a.n_split, it / a.n_split);
        if (grid_sync(a.bar)) return;
        for (int qh = blockIdx.x; qh < a.nq; qh += gridDim.x) merge_item<HD>(a, qh);
        {
            GemvP p{};
            p.w = (const uint16_t *)ly->o;
            p.x = a.attn;
            p.bias = ly->o_bias;
            p.y = a.h;
            p.units = H;
            p.K = qw;
            if (gemv_phase<DG_RESID>(a, p, a.nch_q, sm)) return;
        }
        {
            GemvP p{};
            p.w = (const uint16_t *)ly->gate;
            p.w2 = (const uint16_t *)ly->up;
            p.x = a.h;
            p.gamma = ly->post_norm;
            p.y = a.act;
            p.units = a.F;
            p.K = H;
            if (gemv_phase<DG_SWIGLU>(a, p, a.nch_h, sm)) return;
        }
        {
            GemvP p{};
            p.w = (const uint16_t *)ly->down;
            p.x = a.act;
            p.y = a.h;
            p.units = H;
            p.K = a.F;
            if (gemv_phase<DG_RESID>(a, p, a.nch_f, sm)) return;
        }
    }
    {  // final RMSNorm + head (model.rs:531-538, 661-665) with the block argmax
        GemvP p{};
        p.w = (const uint16_t *)a.head;
        p.x = a.h;
        p.gamma = a.final_norm;
        p.y = a.logits;
        p.units = a.V;
        p.K = H;
        if (gemv_phase<DG_HEAD>(a, p, a.nch_h, sm)) return;
    }
    if (!a.picked) return;
    if (grid_sync(a.bar)) return;
    if (blockIdx.x != 0) return;
    // greedy id: block partials in block order (lowest id on ties)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float b = -INFINITY;
    int bj = 0x7fffffff;
    for (int k = tid; k < (int)gridDim.x; k += blockDim.x) {
        const float v = ld_agent(a.part_v + k);
        const int i = ld_agent(a.part_i + k);
        if (v > b || (v == b && i < bj)) {
            b = v;
            bj = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(b, o, 64);
        const int oi = __shfl_xor(bj, o, 64);
        if (ov > b || (ov == b && oi < bj)) {
            b = ov;
            bj = oi;
        }
    }
    if (lane == 0) {
        sm.best_v[wave] = b;
        sm.best_i[wave] = bj;
    }
    __syncthreads();
    if (tid == 0) {
        b = sm.best_v[0];
        bj = sm.best_i[0];
        for (int w = 1; w < DG_WAVES; ++w)
            if (sm.best_v[w] > b || (sm.best_v[w] == b && sm.best_i[w] < bj)) {
                b = sm.best_v[w];
                bj = sm.best_i[w];
            }
        if (bj == 0x7fffffff) bj = 0;
        a.picked[0] = (uint32_t)bj;
        if (a.gen) {  // device-loop hand-off: next token, step count, position
            int32_t *gn = a.gen;
            gn[0] = bj;
            gn[8 + gn[1]] = bj;
            gn[1] += 1;
            gn[3] += 1;
        }
    }
}

// ------------------------------------------------------------ host side
static int step_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        ESP_HIP(hipGetDevice(&dev));
        ESP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus <= 0) cus = 256;
    }
    return cus;
}

template <int HD, int GM> static int step_blocks() {
    static int per_cu = 0;
    if (!per_cu) {
        ESP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(step_k<HD, GM>), DG_THREADS, 0));
        if (per_cu <= 0) per_cu = 1;
    }
    int nb = per_cu * step_cus();
    return nb > DG_MAX_PART ? DG_MAX_PART : nb;
}

static int step_blocks_for(int hd, int G) {
    if (hd == 64) return G <= 4 ? step_blocks<64, 4>() : step_blocks<64, 8>();
    return G <= 4 ? step_blocks<128, 4>() : step_blocks<128, 8>();
}

static bool nch_ok(int K) {
    // K split in four quarters of 8-element chunks, at most DG_MAXC per lane
    return K % 32 == 0 && K / 32 <= 64 * DG_MAXC;
}

int step_nch(int K) {
    const int n = (K / DG_WAVES / 8 + 63) / 64;
    return n <= 1 ? 1 : (n <= 2 ? 2 : (n <= 4 ? 4 : DG_MAXC));
}

bool step_ok(int hd, int G, int H, int qw, int F, bool qk_norm, bool moe, Dt wt) {
    return wt == DT_BF16 && !qk_norm && !moe && (hd == 64 || hd == 128) && G >= 1 && G <= 8 &&
           nch_ok(H) && step_nch(H) <= 4 && nch_ok(qw) && nch_ok(F);
}

int step_attn_splits(int hd, int G, int nkv, int max_t, int *split_len) {
    const int cap = ATT_MAX_SPLIT_STEP;
    int ns = step_blocks_for(hd, G) / (nkv > 0 ? nkv : 1);
    ns = ns < 1 ? 1 : (ns > cap ? cap : ns);
    int len = (max_t + ns - 1) / ns;
    len = len < 32 ? 32 : (len + 31) / 32 * 32;
    ns = (max_t + len - 1) / len;
    if (ns < 1) ns = 1;
    *split_len = len;
    return ns;
}

void launch_step(const StepArgs &a, int G, hipStream_t s) {
    if (a.n_split > ATT_MAX_SPLIT_STEP) fail(ESP_BACKEND, "decode step: too many key splits");
    const int nb = step_blocks_for(a.hd, G);
    if (nb < SB_GROUPS) fail(ESP_BACKEND, "decode step: grid too small for the barrier");
    if (a.hd == 64) {
        if (G <= 4) step_k<64, 4><<<nb, DG_THREADS, 0, s>>>(a);
        else step_k<64, 8><<<nb, DG_THREADS, 0, s>>>(a);
    } else {
        if (G <= 4) step_k<128, 4><<<nb, DG_THREADS, 0, s>>>(a);
        else step_k<128, 8><<<nb, DG_THREADS, 0, s>>>(a);
    }
}

}  // namespace esp
