// Single-token (decode) kernels, built to stream weights at HBM rate with as
// few dispatches per layer as the data dependencies allow.
//
// decode_gemv_k: y = W x for one input row. A block owns RB output rows (or
// row pairs); its four waves split K into contiguous quarters, each lane
// keeping its slice of x (optionally RMS-normalised) in registers for the
// whole grid-stride loop, so x is read once per block while weight rows
// stream with 16-byte loads. Epilogues fuse what follows the projection:
//   RESID   h[n] += y (+bias)                      (o_proj, down_proj)
//   SWIGLU  act[n] = silu(g_n) * u_n               (gate/up pairs)
//   QKVROPE q/k/v rows in split-half pairs (d, d+hd/2): +bias, RoPE at the
//           row's position, q -> f32 buffer, k/v appended to the cache
//   HEAD    logits[n] (+ greedy argmax, lowest id on ties, reduced by the
//           last block to finish; optionally hands the token to the next
//           captured step: gen[0] = id, gen[8+step] = id, step++, pos++)
//
// attn_decode_k: causal GQA attention for one query row per (kv head, key
// split), online softmax in registers; the last split to finish for a
// (row, kv head) merges the partials in split order (deterministic).
#include "common.hpp"
#include "dev.hpp"
#include "decode.hpp"
#include "decode_dev.hpp"

namespace esp {

// NCH = 8-element chunks per lane and row in this wave's quarter of K
// (K <= 4 * 64 * 8 * NCH). The first iteration's weight loads are issued
// before x is read and normalised, and each iteration issues the next
// one's loads before reducing its own sums.
template <typename WT, int EPI, int RB, int NCH>
__global__ void __launch_bounds__(DG_THREADS) decode_gemv_k(DecodeGemvArgs a) {
    constexpr int RU = RowsPerUnit<EPI>::v;
    constexpr int R = RB * RU;  // weight rows per block iteration
    __shared__ float red[DG_MAX_IT][R][DG_WAVES];
    __shared__ float ssq[DG_WAVES];
    __shared__ float best_v[DG_WAVES];
    __shared__ int best_i[DG_WAVES];
    __shared__ int last;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int K = a.K, kq = K / DG_WAVES, nch = kq / 8;  // chunks in this wave's quarter
    const int k0 = wave * kq;
    const WT *W = (const WT *)a.w;
    const WT *W2 = (const WT *)a.w2;
    const int units = EPI == DG_QKVROPE ? a.N / 2 : a.N;

    Chunk<WT> wc[R][NCH];
    auto load_rows = [&](int u0) {
        const WT *rp[R];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            int u = min(u0 + r, units - 1);
            if (EPI == DG_SWIGLU) {
                rp[r * 2] = W + (size_t)u * K;
                rp[r * 2 + 1] = W2 + (size_t)u * K;
            } else if (EPI == DG_QKVROPE) {
                int half = a.hd / 2, head = u / half, d = u % half;
                int row = head * a.hd + d;
                rp[r * 2] = W + (size_t)row * K;
                rp[r * 2 + 1] = W + (size_t)(row + half) * K;
            } else {
                rp[r] = W + (size_t)u * K;
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
    };
    if ((int)blockIdx.x * RB < units) load_rows(blockIdx.x * RB);

    // ---- x slice in registers (+ fused RMSNorm)
    float xr[NCH][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        int ch = lane + 64 * c;
        if (ch < nch) {
            const float *xp = a.x + k0 + ch * 8;
            f32x4_t p0 = *(const f32x4_t *)xp, p1 = *(const f32x4_t *)(xp + 4);
            xr[c][0] = p0.x; xr[c][1] = p0.y; xr[c][2] = p0.z; xr[c][3] = p0.w;
            xr[c][4] = p1.x; xr[c][5] = p1.y; xr[c][6] = p1.z; xr[c][7] = p1.w;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += xr[c][i] * xr[c][i];
        }
    }
    if (a.gamma) {
        ss = wave_sum(ss);
        if (lane == 0) ssq[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < DG_WAVES; ++w) tot += ssq[w];
        const float rms = sqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            int ch = lane + 64 * c;
            if (ch < nch) {
                const float *g = a.gamma + k0 + ch * 8;
#pragma unroll
                for (int i = 0; i < 8; ++i) xr[c][i] = (xr[c][i] / rms) * g[i];
            }
        }
    }
    // ---- stream rows; each wave parks its sums in LDS (no barrier)
    int iters = 0;
    for (int u0 = blockIdx.x * RB; u0 < units; u0 += gridDim.x * RB, ++iters) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            int ch = lane + 64 * c;
            if (ch < nch) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] += wc[r][c].dot(xr[c]);
            }
        }
        if (u0 + gridDim.x * RB < units) load_rows(u0 + gridDim.x * RB);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum_uniform(acc[r]);
            if (lane == 0) red[iters][r][wave] = v;
        }
    }
    __syncthreads();
    // ---- epilogues: thread t handles unit (iteration t / RB, row t % RB)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int e = tid; e < iters * RB; e += blockDim.x) {
        const int it = e / RB, r = e % RB;
        const int u = blockIdx.x * RB + it * gridDim.x * RB + r;
        if (u >= units) continue;
        float y[RU];
#pragma unroll
        for (int j = 0; j < RU; ++j) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < DG_WAVES; ++w) t += red[it][r * RU + j][w];
            y[j] = t;
        }
        if (EPI == DG_RESID) {
            float v = a.bias ? y[0] + a.bias[u] : y[0];
            a.y[u] = a.y[u] + v;
        } else if (EPI == DG_STORE) {
            a.y[u] = a.bias ? y[0] + a.bias[u] : y[0];
        } else if (EPI == DG_HEAD) {
            a.y[u] = y[0];
            if (y[0] > bv || (y[0] == bv && u < bi)) {
                bv = y[0];
                bi = u;
            }
        } else if (EPI == DG_SWIGLU) {
            a.y[u] = silu(y[0]) * y[1];
        } else {  // DG_QKVROPE
            const int hd = a.hd, half = hd / 2, head = u / half, d = u % half;
            const int r0 = head * hd + d, r1 = r0 + half;
            float v0 = y[0], v1 = y[1];
            if (a.bias) {
                v0 = v0 + a.bias[r0];
                v1 = v1 + a.bias[r1];
            }
            if (a.lora_t) {  // unmerged LoRA, before RoPE (lora.rs:93-97)
                const int j = head < a.nq ? 0 : (head < a.nq + a.nkv ? 1 : 2);
                if (a.lora_b[j]) {
                    const WT *B = (const WT *)a.lora_b[j];
                    const int rank = a.lora_rank[j];
                    const int off = j == 0 ? 0 : (j == 1 ? a.nq * hd : (a.nq + a.nkv) * hd);
                    const float *t = a.lora_t + a.lora_t_col[j];
                    float c0 = 0.f, c1 = 0.f;
                    for (int i = 0; i < rank; ++i) {
                        c0 += ld(B, (size_t)(r0 - off) * rank + i) * t[i];
                        c1 += ld(B, (size_t)(r1 - off) * rank + i) * t[i];
                    }
                    v0 = v0 + c0 * a.lora_scale[j];
                    v1 = v1 + c1 * a.lora_scale[j];
                }
            }
            const int pos = a.row_pos[0], seq = a.row_seq[0];
            const float *cs = a.rope_cos + (size_t)pos * hd;
            const float *sn = a.rope_sin + (size_t)pos * hd;
            if (head < a.nq + a.nkv) {
                float o0 = v0 * cs[d] + (-v1) * sn[d];
                float o1 = v1 * cs[d + half] + v0 * sn[d + half];
                if (head < a.nq) {
                    a.q_out[r0] = o0;
                    a.q_out[r1] = o1;
                } else {
                    float *kc = a.kv + (size_t)seq * a.seq_stride +
                                (size_t)(head - a.nq) * a.head_stride + (size_t)pos * hd;
                    kc[d] = o0;
                    kc[d + half] = o1;
                }
            } else {
                float *vc = a.kv + (size_t)seq * a.seq_stride + a.kv_half_stride +
                            (size_t)(head - a.nq - a.nkv) * a.head_stride + (size_t)pos * hd;
                vc[d] = v0;
                vc[d + half] = v1;
            }
        }
    }
    if (EPI != DG_HEAD || !a.ticket) return;
    // ---- greedy argmax across blocks: partial per block, last block reduces
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        best_v[wave] = bv;
        best_i[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float b = best_v[0];
        int bj = best_i[0];
        for (int w = 1; w < DG_WAVES; ++w)
            if (best_v[w] > b || (best_v[w] == b && best_i[w] < bj)) {
                b = best_v[w];
                bj = best_i[w];
            }
        st_agent(a.part_v + blockIdx.x, b);
        st_agent(a.part_i + blockIdx.x, bj);
        wait_stores();
        int t = atomicAdd(a.ticket, 1);
        last = t == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    // last block: reduce the partials in block order (deterministic)
    float b = -INFINITY;
    int bj = 0x7fffffff;
    constexpr int PER = DG_MAX_PART / DG_THREADS;
    float pvs[PER];
    int pis[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {  // independent loads, issued together
        int k = tid + q * DG_THREADS;
        pvs[q] = k < (int)gridDim.x ? ld_agent(a.part_v + k) : -INFINITY;
        pis[q] = k < (int)gridDim.x ? ld_agent(a.part_i + k) : 0x7fffffff;
    }
#pragma unroll
    for (int q = 0; q < PER; ++q)
        if (pvs[q] > b || (pvs[q] == b && pis[q] < bj)) {
            b = pvs[q];
            bj = pis[q];
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(b, o, 64);
        int oi = __shfl_xor(bj, o, 64);
        if (ov > b || (ov == b && oi < bj)) {
            b = ov;
            bj = oi;
        }
    }
    if (lane == 0) {
        best_v[wave] = b;
        best_i[wave] = bj;
    }
    __syncthreads();
    if (tid == 0) {
        b = best_v[0];
        bj = best_i[0];
        for (int w = 1; w < DG_WAVES; ++w)
            if (best_v[w] > b || (best_v[w] == b && best_i[w] < bj)) {
                b = best_v[w];
                bj = best_i[w];
            }
        if (bj == 0x7fffffff) bj = 0;
        a.picked[0] = (uint32_t)bj;
        if (a.gen) {
            int32_t *g = a.gen;
            g[0] = bj;
            g[8 + g[1]] = bj;
            g[1] += 1;
            g[3] += 1;
        }
        *a.ticket = 0;
    }
}

template <typename WT, int EPI, int RB, int NCH>
static void dg_launch_nch(const DecodeGemvArgs &a, int cus, hipStream_t s) {
    static int per_cu = 0;  // resident blocks per CU for this instance
    if (!per_cu) {
        ESP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(decode_gemv_k<WT, EPI, RB, NCH>), DG_THREADS, 0));
        if (per_cu <= 0) per_cu = 1;
    }
    const int units = EPI == DG_QKVROPE ? a.N / 2 : a.N;
    const int groups = (units + RB - 1) / RB;
    // one round of resident blocks, every block doing the same number of
    // iterations
    const int cap = cus * per_cu;
    int iters = (groups + cap - 1) / cap;
    const int need = (groups + DG_MAX_IT - 1) / DG_MAX_IT;  // LDS slots per block
    int blocks = (groups + iters - 1) / iters;
    if (blocks < need) blocks = need;
    if (EPI == DG_HEAD && a.ticket && blocks > DG_MAX_PART)
        fail(ESP_UNSUPPORTED, "decode head: vocabulary above the argmax partial capacity");
    decode_gemv_k<WT, EPI, RB, NCH><<<blocks, DG_THREADS, 0, s>>>(a);
}

template <typename WT, int EPI>
static void dg_launch(const DecodeGemvArgs &a, int cus, hipStream_t s) {
    // Measured on MI355X: two rows per block (more blocks in flight) beats
    // larger row blocks with more loads per lane at every decode shape.
    const int nch = (a.K / DG_WAVES / 8 + 63) / 64;  // chunks per lane and row
    if (nch <= 1) dg_launch_nch<WT, EPI, 2, 1>(a, cus, s);
    else if (nch <= 2) dg_launch_nch<WT, EPI, 2, 2>(a, cus, s);
    else if (nch <= 4) dg_launch_nch<WT, EPI, 2, 4>(a, cus, s);
    else dg_launch_nch<WT, EPI, 2, DG_MAXC>(a, cus, s);
}

bool decode_gemv_ok(int K) { return K % 32 == 0 && K / 32 <= 64 * DG_MAXC; }

void launch_decode_gemv(Dt wt, int epi, const DecodeGemvArgs &a, hipStream_t s) {
    if (!decode_gemv_ok(a.K)) fail(ESP_BACKEND, "decode_gemv: unsupported width");
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        ESP_HIP(hipGetDevice(&dev));
        ESP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus <= 0) cus = 256;
    }
#define DG_CASE(E)                                                   \
    case E:                                                          \
        if (wt == DT_BF16) dg_launch<uint16_t, E>(a, cus, s);        \
        else dg_launch<float, E>(a, cus, s);                         \
        break;
    switch (epi) {
        DG_CASE(DG_STORE)
        DG_CASE(DG_RESID)
        DG_CASE(DG_SWIGLU)
        DG_CASE(DG_QKVROPE)
        DG_CASE(DG_HEAD)
        default: fail(ESP_BACKEND, "decode_gemv: bad epilogue");
    }
#undef DG_CASE
}

// ------------------------------------------------------------ attention

constexpr int ATT_MAX_SPLIT = 128;
constexpr int ATT_WAVES = 4;     // waves per attention block
constexpr int ATT_CHUNK = 128;  // keys whose K/V loads a block issues at once
constexpr int ATT_PSTRIDE_PAD = ATT_PART_PAD;  // partial row: m, l, 2 pad, acc[hd]

// One block per (key split, kv head, row). A key is covered by a group of
// hd/8 lanes (8 dims each), so a wave scores 64*8/hd keys per step and a
// dot product is finished with DPP swaps inside the group. A chunk of
// ATT_CHUNK keys has all its K/V loads issued before any score is formed,
// and the softmax update is done once per chunk (one exp per key). GM is
// the largest query-head group the instance serves (4 or 8).
template <int HD, int GM>
__global__ void __launch_bounds__(ATT_WAVES * 64) attn_decode_k(AttnDecodeArgs a) {
    constexpr int NW = ATT_WAVES;
    constexpr int DPL = 8;               // dims per lane
    constexpr int LPK = HD / DPL;        // lanes per key
    constexpr int KPW = 64 / LPK;        // keys per wave per step
    constexpr int NS = ATT_CHUNK / (NW * KPW);  // steps per chunk
    constexpr int GMAX = GM;
    constexpr int STRIDE = HD + ATT_PSTRIDE_PAD;
    __shared__ float wm[NW][GMAX], wl[NW][GMAX];
    __shared__ float wacc[NW][GMAX][HD];
    __shared__ int last;
    const int split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;
    const int G = a.nq / a.nkv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp = lane / LPK, sub = lane % LPK;
    const int pos = a.row_pos[row], seq = a.row_seq[row];
    int lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
    int hi = pos + 1;
    lo = max(lo, split * a.split_len);
    hi = min(hi, (split + 1) * a.split_len);
    const float inv_scale = 1.f / sqrtf((float)HD);
    // q for the group's heads: this lane's 8 dims
    float q[GMAX][DPL];
    const float *qrow = a.q + (size_t)row * a.nq * HD + (size_t)g * G * HD + sub * DPL;
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
        if (j < G) {
            const f32x4_t v0 = *(const f32x4_t *)(qrow + (size_t)j * HD);
            const f32x4_t v1 = *(const f32x4_t *)(qrow + (size_t)j * HD + 4);
            q[j][0] = v0.x; q[j][1] = v0.y; q[j][2] = v0.z; q[j][3] = v0.w;
            q[j][4] = v1.x; q[j][5] = v1.y; q[j][6] = v1.z; q[j][7] = v1.w;
        }
    float m[GMAX], l[GMAX], acc[GMAX][DPL];
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
    }
    const float *kb = a.kv + (size_t)seq * a.seq_stride + (size_t)g * a.head_stride + sub * DPL;
    const float *vb = kb + a.kv_half_stride;
    for (int c0 = lo; c0 < hi; c0 += ATT_CHUNK) {
        f32x4_t kk[NS][2], vv[NS][2];
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const int t = c0 + st * NW * KPW + wave * KPW + grp;
            kk[st][0] = kk[st][1] = vv[st][0] = vv[st][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (t < hi) {
                kk[st][0] = *(const f32x4_t *)(kb + (size_t)t * HD);
                kk[st][1] = *(const f32x4_t *)(kb + (size_t)t * HD + 4);
                vv[st][0] = *(const f32x4_t *)(vb + (size_t)t * HD);
                vv[st][1] = *(const f32x4_t *)(vb + (size_t)t * HD + 4);
            }
        }
#pragma unroll
        for (int j = 0; j < GMAX; ++j) {
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
            if (mx == -INFINITY) continue;  // no key of this lane's group in the chunk yet
            const float al = __expf(m[j] - mx);
            l[j] *= al;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[j][e] *= al;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const float p = __expf(sc[st] - mx);
                l[j] += p;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][e] += p * vv[st][0][e];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][4 + e] += p * vv[st][1][e];
            }
            m[j] = mx;
        }
    }
    // merge the KPW key groups of the wave (lanes with equal `sub`)
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
        if (j >= G) break;
#pragma unroll
        for (int o = LPK; o < 64; o <<= 1) {
            float om = __shfl_xor(m[j], o, 64), ol = __shfl_xor(l[j], o, 64);
            float mn = fmaxf(m[j], om);
            float s1 = mn == -INFINITY ? 0.f : __expf(m[j] - mn);
            float s2 = mn == -INFINITY ? 0.f : __expf(om - mn);
            l[j] = l[j] * s1 + ol * s2;
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                float oa = __shfl_xor(acc[j][i], o, 64);
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
    // merge the waves; write this split's partial (m, l, -, -, acc[HD]) per head
    for (int o = tid; o < G * HD; o += blockDim.x) {
        int j = o / HD, d = o % HD;
        float mx = -INFINITY;
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wm[w][j]);
        float L = 0.f, v = 0.f;
        for (int w = 0; w < NW; ++w) {
            float sc = mx == -INFINITY ? 0.f : __expf(wm[w][j] - mx);
            L += wl[w][j] * sc;
            v += wacc[w][j][d] * sc;
        }
        if (a.n_split == 1) {  // single split: normalise directly
            a.out[(size_t)row * a.nq * HD + (size_t)(g * G + j) * HD + d] = v / L;
            continue;
        }
        float *p = a.part + (((size_t)row * a.nq + (size_t)g * G + j) * a.n_split + split) * STRIDE;
        st_agent(p + ATT_PSTRIDE_PAD + d, v);
        if (d == 0) {
            st_agent(p, mx);
            st_agent(p + 1, L);
        }
    }
    if (a.n_split == 1) return;
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        int *tk = a.ticket + (size_t)row * a.nkv + g;
        int t = atomicAdd(tk, 1);
        last = t == a.n_split - 1;
        if (last) *tk = 0;
    }
    __syncthreads();
    if (!last) return;
    // Merge in the last block. Split maxima / sums go to LDS; each head's
    // weights exp(m_s - max) and total are reduced across one wave; then
    // every thread issues its partial loads (up to 32 splits x 2 outputs)
    // at once and weights them in split order, so the result is
    // deterministic.
    __shared__ float mm[GMAX][ATT_MAX_SPLIT], ww[GMAX][ATT_MAX_SPLIT], LL[GMAX];
    const int ns = a.n_split;
    const float *pb = a.part + ((size_t)row * a.nq + (size_t)g * G) * ns * STRIDE;
    for (int i = tid; i < G * ns; i += blockDim.x) {
        const int j = i / ns, sp = i % ns;
        mm[j][sp] = ld_agent(pb + ((size_t)j * ns + sp) * STRIDE);
        ww[j][sp] = ld_agent(pb + ((size_t)j * ns + sp) * STRIDE + 1);
    }
    __syncthreads();
    for (int j = wave; j < G; j += NW) {
        const int s0 = lane, s1 = lane + 64;  // ns <= 128
        const float m0 = s0 < ns ? mm[j][s0] : -INFINITY, m1 = s1 < ns ? mm[j][s1] : -INFINITY;
        const float mx = wave_max(fmaxf(m0, m1));
        const float w0 = m0 == -INFINITY ? 0.f : __expf(m0 - mx);
        const float w1 = m1 == -INFINITY ? 0.f : __expf(m1 - mx);
        const float L = wave_sum((s0 < ns ? ww[j][s0] * w0 : 0.f) + (s1 < ns ? ww[j][s1] * w1 : 0.f));
        if (s0 < ns) ww[j][s0] = w0;
        if (s1 < ns) ww[j][s1] = w1;
        if (lane == 0) LL[j] = L;
    }
    __syncthreads();
    constexpr int MB = 32;  // splits per load batch
    for (int o0 = tid; o0 < G * HD; o0 += 2 * blockDim.x) {
        const int o1 = o0 + blockDim.x;
        const bool has1 = o1 < G * HD;
        const int j0 = o0 / HD, d0 = o0 % HD, j1 = has1 ? o1 / HD : j0, d1 = has1 ? o1 % HD : d0;
        const float *p0 = pb + (size_t)j0 * ns * STRIDE + ATT_PSTRIDE_PAD + d0;
        const float *p1 = pb + (size_t)j1 * ns * STRIDE + ATT_PSTRIDE_PAD + d1;
        float v0 = 0.f, v1 = 0.f;
        for (int sp0 = 0; sp0 < ns; sp0 += MB) {
            float t0[MB], t1[MB];
#pragma unroll
            for (int q = 0; q < MB; ++q) {
                t0[q] = sp0 + q < ns ? ld_agent(p0 + (size_t)(sp0 + q) * STRIDE) : 0.f;
                t1[q] = has1 && sp0 + q < ns ? ld_agent(p1 + (size_t)(sp0 + q) * STRIDE) : 0.f;
            }
#pragma unroll
            for (int q = 0; q < MB; ++q) {
                if (sp0 + q < ns) {
                    v0 += t0[q] * ww[j0][sp0 + q];
                    v1 += t1[q] * ww[j1][sp0 + q];
                }
            }
        }
        a.out[(size_t)row * a.nq * HD + (size_t)(g * G + j0) * HD + d0] = v0 / LL[j0];
        if (has1) a.out[(size_t)row * a.nq * HD + (size_t)(g * G + j1) * HD + d1] = v1 / LL[j1];
    }
}

bool attn_decode_ok(int hd, int G) { return (hd == 64 || hd == 128) && G <= 8; }

template <int HD, int GM> static int attn_resident_blocks() {
    static int per_cu = 0;
    if (!per_cu) {
        ESP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(attn_decode_k<HD, GM>), ATT_WAVES * 64, 0));
        if (per_cu <= 0) per_cu = 1;
    }
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        ESP_HIP(hipGetDevice(&dev));
        ESP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus <= 0) cus = 256;
    }
    return per_cu * cus;
}

// Key splits for one decode row: as many splits as keep every (split, kv
// head) block resident at once (one round of blocks), at most 64 (hd 128)
// or 128 (hd 64) since the merge re-reads every split's partial; split
// lengths are multiples of 32 keys, and a split up to ATT_CHUNK keys is
// read in one round of loads.
int attn_decode_splits(int hd, int nkv, int G, int max_t, int *split_len) {
    int slots = hd == 64 ? (G <= 4 ? attn_resident_blocks<64, 4>() : attn_resident_blocks<64, 8>())
                         : (G <= 4 ? attn_resident_blocks<128, 4>() : attn_resident_blocks<128, 8>());
    const int cap = hd == 64 ? ATT_MAX_SPLIT : ATT_MAX_SPLIT / 2;
    int ns = slots / (nkv > 0 ? nkv : 1);
    ns = ns < 1 ? 1 : (ns > cap ? cap : ns);
    int len = (max_t + ns - 1) / ns;
    len = len < 32 ? 32 : (len + 31) / 32 * 32;
    ns = (max_t + len - 1) / len;
    if (ns < 1) ns = 1;
    *split_len = len;
    return ns;
}

void launch_attn_decode(const AttnDecodeArgs &a, hipStream_t s) {
    const int G = a.nq / a.nkv;
    if (!attn_decode_ok(a.hd, G)) fail(ESP_BACKEND, "attn_decode: unsupported head shape");
    dim3 grid(a.n_split, a.nkv, a.M);
    if (a.n_split > ATT_MAX_SPLIT) fail(ESP_BACKEND, "attn_decode: too many key splits");
    if (a.hd == 64) {
        if (G <= 4) attn_decode_k<64, 4><<<grid, ATT_WAVES * 64, 0, s>>>(a);
        else attn_decode_k<64, 8><<<grid, ATT_WAVES * 64, 0, s>>>(a);
    } else {
        if (G <= 4) attn_decode_k<128, 4><<<grid, ATT_WAVES * 64, 0, s>>>(a);
        else attn_decode_k<128, 8><<<grid, ATT_WAVES * 64, 0, s>>>(a);
    }
}

}  // namespace esp
