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
#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <vector>

#include "common.hpp"
#include "dev.hpp"
#include "decode.hpp"
#include "decode_dev.hpp"
#include "attn_dev.hpp"

namespace esp {

// NCH = 8-element chunks per lane and row in this wave's share (1 / NW) of K
// (K <= NW * 64 * 8 * NCH). The first iteration's weight loads are issued
// before x is read and normalised, and each iteration issues the next
// one's loads before reducing its own sums.
template <typename WT, int EPI, int RB, int NCH, int NW = DG_WAVES>
__global__ void __launch_bounds__(NW * 64) decode_gemv_k(DecodeGemvArgs a) {
    constexpr int RU = RowsPerUnit<EPI>::v;
    constexpr int R = RB * RU;  // weight rows per block iteration
    __shared__ float red[DG_MAX_IT][R][NW];
    __shared__ float ssq[NW];
    __shared__ float best_v[NW];
    __shared__ int best_i[NW];
    __shared__ int last;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int CW = Chunk<WT>::W;  // weights per chunk
    const int K = a.K, kq = K / NW, nch = kq / CW;  // chunks in this wave's quarter
    const int k0 = wave * kq;
    const void *W = a.w;
    const void *W2 = a.w2;
    size_t ex0 = 0;  // element offset of the routed expert (RESID)
    if ((EPI == DG_RESID || EPI == DG_STORE) && a.ex_sel)  // one routed expert's rows
        ex0 = (size_t)min(max(a.ex_sel[a.ex_slot], 0), a.ex_count - 1) * a.ex_stride;
    // QKVROPE: N/2 rotary pairs, then the LoRA A rows in pairs
    const int units = EPI == DG_QKVROPE ? a.N / 2 + (a.lora_rows + 1) / 2 : a.N;

    Chunk<WT> wc[R][NCH];
    auto load_rows = [&](int u0) {
        const void *rb[R];    // matrix of each row (gate or up for SWIGLU)
        const float *rs[R];   // its block scales (packed formats)
        size_t ro[R];         // element offset of the row's first weight
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            int u = min(u0 + r, units - 1);
            if (EPI == DG_SWIGLU) {
                size_t off = (size_t)u * K;
                if (a.ex_sel) {  // (slot, row) of a routed expert
                    const int j = u / a.ex_rows, e = min(max(a.ex_sel[j], 0), a.ex_count - 1);
                    off = (size_t)e * a.ex_stride + (size_t)(u - j * a.ex_rows) * K;
                }
                rb[r * 2] = W;
                rb[r * 2 + 1] = W2;
                rs[r * 2] = a.ws;
                rs[r * 2 + 1] = a.ws2;
                ro[r * 2] = ro[r * 2 + 1] = off;
            } else if (EPI == DG_QKVROPE) {
                rb[r * 2] = rb[r * 2 + 1] = W;
                rs[r * 2] = rs[r * 2 + 1] = a.ws;
                if (u < a.N / 2) {
                    int half = a.hd / 2, head = u / half, d = u % half;
                    int row = head * a.hd + d;
                    ro[r * 2] = (size_t)row * K;
                    ro[r * 2 + 1] = (size_t)(row + half) * K;
                } else {  // LoRA A rows 2i, 2i + 1 (the last one clamped)
                    const int i = 2 * (u - a.N / 2);
                    ro[r * 2] = (size_t)(a.N + i) * K;
                    ro[r * 2 + 1] = (size_t)(a.N + min(i + 1, a.lora_rows - 1)) * K;
                }
            } else {
                rb[r] = W;
                rs[r] = a.ws;
                ro[r] = ex0 + (size_t)u * K;
            }
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int ch = lane + 64 * c;
            if (ch < nch) {
#pragma unroll
                for (int r = 0; r < R; ++r) wc[r][c].load_at(rb[r], ro[r] + k0 + ch * CW, rs[r]);
            }
        }
    };
    if ((int)blockIdx.x * RB < units) load_rows(blockIdx.x * RB);

    // ---- x slice in registers (+ fused RMSNorm)
    float xr[NCH][CW];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        int ch = lane + 64 * c;
        if (ch < nch) {
            const float *xp = a.x + k0 + ch * CW;
#pragma unroll
            for (int q = 0; q < CW / 4; ++q) {
                const f32x4_t p = *(const f32x4_t *)(xp + 4 * q);
                xr[c][4 * q] = p.x;
                xr[c][4 * q + 1] = p.y;
                xr[c][4 * q + 2] = p.z;
                xr[c][4 * q + 3] = p.w;
            }
        }
    }
    // The epilogue's memory operands for this thread's unit (the residual
    // row and bias; the rotary row at the decode position), loaded here so
    // they arrive with the first weight rows instead of as dependent round
    // trips (position, then the rope row) after the last ones. Thread t owns
    // epilogue unit t (at most DG_MAX_IT * RB <= blockDim.x units per block).
    const int n_it = (int)blockIdx.x * RB < units
                         ? (units - (int)blockIdx.x * RB + (int)gridDim.x * RB - 1) / ((int)gridDim.x * RB)
                         : 0;
    const int pe_u = (int)blockIdx.x * RB + (tid / RB) * (int)gridDim.x * RB + tid % RB;
    const bool pe = tid < n_it * RB && pe_u < units;
    float pf[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (EPI == DG_RESID && pe) {
        pf[0] = a.y[pe_u];
        if (a.bias) pf[1] = a.bias[pe_u];
    } else if (EPI == DG_QKVROPE && pe && pe_u < a.N / 2) {
        const int half = a.hd / 2, head = pe_u / half, d = pe_u % half;
        const int r0 = head * a.hd + d;
        if (a.bias) {
            pf[0] = a.bias[r0];
            pf[1] = a.bias[r0 + half];
        }
        if (head < a.nq + a.nkv) {
            const size_t ro = (size_t)a.row_pos[0] * a.hd + d;
            pf[2] = a.rope_cos[ro];
            pf[3] = a.rope_cos[ro + half];
            pf[4] = a.rope_sin[ro];
            pf[5] = a.rope_sin[ro + half];
        }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (lane + 64 * c < nch) {
#pragma unroll
            for (int i = 0; i < CW; ++i) ss += xr[c][i] * xr[c][i];
        }
    }
    if (a.gamma) {
        ss = wave_sum(ss);
        if (lane == 0) ssq[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) tot += ssq[w];
        const float rms = sqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            int ch = lane + 64 * c;
            if (ch < nch) {
                const float *g = a.gamma + k0 + ch * CW;
#pragma unroll
                for (int i = 0; i < CW; ++i) xr[c][i] = (xr[c][i] / rms) * g[i];
            }
        }
    }
    // per-chunk input sums (the packed formats' bias term; unused otherwise)
    float xs[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        xs[c] = 0.f;
        if (WPacked<WT>::v) {
#pragma unroll
            for (int i = 0; i < CW; ++i) xs[c] += xr[c][i];
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
                for (int r = 0; r < R; ++r) acc[r] += wc[r][c].dot(xr[c], xs[c]);
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
            for (int w = 0; w < NW; ++w) t += red[it][r * RU + j][w];
            y[j] = t;
        }
        const bool mine = e == tid;  // the unit whose operands were prefetched
        if (EPI == DG_RESID) {
            float v = a.bias ? y[0] + (mine ? pf[1] : a.bias[u]) : y[0];
            if (a.ex_w) v = v * a.ex_w[a.ex_slot];
            if (a.sig_scale) v = v * (1.f / (1.f + expf(-a.sig_scale[0])));
            a.y[u] = (mine ? pf[0] : a.y[u]) + v;
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
            if (u >= a.N / 2) {  // LoRA t = A . norm(x), stored as is
                const int i = 2 * (u - a.N / 2);
                a.lora_t_out[i] = y[0];
                if (i + 1 < a.lora_rows) a.lora_t_out[i + 1] = y[1];
                continue;
            }
            const int hd = a.hd, half = hd / 2, head = u / half, d = u % half;
            const int r0 = head * hd + d, r1 = r0 + half;
            float v0 = y[0], v1 = y[1];
            if (a.bias) {
                v0 = v0 + (mine ? pf[0] : a.bias[r0]);
                v1 = v1 + (mine ? pf[1] : a.bias[r1]);
            }
            const int pos = a.row_pos[0], seq = a.row_seq[0];
            const float *cs = a.rope_cos + (size_t)pos * hd;
            const float *sn = a.rope_sin + (size_t)pos * hd;
            if (head < a.nq + a.nkv) {
                const float c0 = mine ? pf[2] : cs[d], c1 = mine ? pf[3] : cs[d + half];
                const float s0 = mine ? pf[4] : sn[d], s1 = mine ? pf[5] : sn[d + half];
                float o0 = v0 * c0 + (-v1) * s0;
                float o1 = v1 * c1 + v0 * s1;
                if (head < a.nq) {
                    a.q_out[r0] = o0;
                    a.q_out[r1] = o1;
                } else {
                    const size_t i = (size_t)seq * a.seq_stride +
                                     (size_t)(head - a.nq) * a.head_stride + (size_t)pos * hd + d;
                    if (a.kv_f16) {
                        st((_Float16 *)a.kv, i, o0);
                        st((_Float16 *)a.kv, i + half, o1);
                    } else {
                        ((float *)a.kv)[i] = o0;
                        ((float *)a.kv)[i + half] = o1;
                    }
                }
            } else {
                const size_t i = (size_t)seq * a.seq_stride + a.kv_half_stride +
                                 (size_t)(head - a.nq - a.nkv) * a.head_stride + (size_t)pos * hd + d;
                if (a.kv_f16) {
                    st((_Float16 *)a.kv, i, v0);
                    st((_Float16 *)a.kv, i + half, v1);
                } else {
                    ((float *)a.kv)[i] = v0;
                    ((float *)a.kv)[i + half] = v1;
                }
            }
        }
    }
    if (EPI == DG_QKVROPE && a.rope_row && blockIdx.x == 0) {
        const size_t ro = (size_t)a.row_pos[0] * a.hd;
        for (int d = tid; d < a.hd; d += blockDim.x) {
            a.rope_row[d] = a.rope_cos[ro + d];
            a.rope_row[a.hd + d] = a.rope_sin[ro + d];
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
        for (int w = 1; w < NW; ++w)
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
    constexpr int PER = DG_MAX_PART / (NW * 64);
    float pvs[PER];
    int pis[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {  // independent loads, issued together
        int k = tid + q * (NW * 64);
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
        for (int w = 1; w < NW; ++w)
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

template <typename WT, int EPI, int RB, int NCH, int NW = DG_WAVES>
static void dg_launch_nch(const DecodeGemvArgs &a, int cus, hipStream_t s) {
    static int per_cu = 0;  // resident blocks per CU for this instance
    if (!per_cu) {
        ESP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(decode_gemv_k<WT, EPI, RB, NCH, NW>), NW * 64, 0));
        if (per_cu <= 0) per_cu = 1;
    }
    const int units = EPI == DG_QKVROPE ? a.N / 2 + (a.lora_rows + 1) / 2 : a.N;
    const int groups = (units + RB - 1) / RB;
    // One round of resident blocks, every block doing the same number of
    // iterations. Packed rows are 1/2 (q8) or 1/4 (q4) of the bf16 bytes, so
    // a block's fixed work (reading x, the fused RMSNorm, the reductions)
    // weighs more: at most four resident blocks per CU, each looping over
    // more rows.
    // Measured at the C3 shape (decode tok/s, q8 / q4): no cap 399 / 446,
    // caps 2 / 3 / 4 / 5 / 6: 412 / 443, 410 / 452, 412 / 461, 408 / 454,
    // 400 / 445; the head keeps the full round (q4: 68.0 vs 72.2 us).
    const int cap = cus * ((WPacked<WT>::v && EPI != DG_HEAD) ? std::min(per_cu, 4) : per_cu);
    int iters = (groups + cap - 1) / cap;
    const int need = (groups + DG_MAX_IT - 1) / DG_MAX_IT;  // LDS slots per block
    int blocks = (groups + iters - 1) / iters;
    if (blocks < need) blocks = need;
    if (EPI == DG_HEAD && a.ticket && blocks > DG_MAX_PART)
        fail(ESP_UNSUPPORTED, "decode head: vocabulary above the argmax partial capacity");
    decode_gemv_k<WT, EPI, RB, NCH, NW><<<blocks, NW * 64, 0, s>>>(a);
}

template <typename WT, int EPI>
static void dg_launch(const DecodeGemvArgs &a, int cus, hipStream_t s) {
    // Measured on MI355X: two rows per block (more blocks in flight) beats
    // one or four rows per block at the 4k-wide projection shapes (below:
    // one row per block for bf16 rows up to 2k).
    const int nch = (a.K / DG_WAVES / Chunk<WT>::W + 63) / 64;  // chunks per lane and row
    // the head over a short K (one chunk per lane) streams best with four
    // rows per block (measured at H 2048: 90.6 vs 97.4 us for 128256 rows)
    if (EPI == DG_HEAD && nch <= 1) {
        dg_launch_nch<WT, EPI, 4, 1>(a, cus, s);
        return;
    }
    // bf16 rows wider than 4k (down_proj at F 8192 and 14336): eight waves
    // split K, half the chunks per lane (at F 14336 four instead of eight:
    // 111 instead of 155 VGPRs, four waves per SIMD instead of three).
    // Measured: C3 decode 3.35 -> 3.30 ms per token (seven waves, exactly
    // four chunks per lane, 3.32 ms); C2 decode (F 8192) 1296 -> 1317 tok/s
    // over the four-wave form, and 1328 -> 1334 on another box with two
    // chunks per lane allocated instead of four. ESP_DG_4W=1 keeps the
    // four-wave form, for comparison.
    if (std::is_same<WT, uint16_t>::value && nch > 2 && a.K % (8 * 64) == 0 && !getenv("ESP_DG_4W")) {
        if ((a.K / 8 / 8 + 63) / 64 <= 2) dg_launch_nch<WT, EPI, 2, 2, 8>(a, cus, s);
        else dg_launch_nch<WT, EPI, 2, DG_MAXC / 2, 8>(a, cus, s);
        return;
    }
    // bf16 rows of 2k-4k (K 4096: two chunks per lane with four waves) for
    // the q/k/v, o, gate/up and head projections: eight waves, one chunk per
    // lane (more waves in flight per CU, each with half the registers).
    // Measured at C3 / C4 decode (tok/s): 302.6-302.9 -> 308.7-309.2 and
    // 1376-1378 -> 1402-1413; gate/up alone 306.4-307.6 (its launch 40.6 ->
    // 38.7 us); the C3 head 165.0 -> 160.8 us (four rows per block: 169.2).
    if constexpr (std::is_same<WT, uint16_t>::value &&
                  (EPI == DG_SWIGLU || EPI == DG_QKVROPE || EPI == DG_RESID || EPI == DG_HEAD)) {
        if (nch == 2 && a.K % (8 * 64) == 0 && !getenv("ESP_DG_4W")) {
            dg_launch_nch<WT, EPI, 2, 1, 8>(a, cus, s);
            return;
        }
    }
    // bf16 rows up to 2k (one chunk per lane: the 1B shape's q/k/v, o and
    // gate/up): one row (pair) per block, more blocks in flight. Measured at
    // C2 decode: 1324.2-1324.8 -> 1334.2-1334.7 tok/s (three or four rows
    // per block: 1320 / 1290).
    if constexpr (std::is_same<WT, uint16_t>::value &&
                  (EPI == DG_SWIGLU || EPI == DG_QKVROPE || EPI == DG_RESID)) {
        if (nch == 1) {
            dg_launch_nch<WT, EPI, 1, 1>(a, cus, s);
            return;
        }
    }
    // Packed down_proj rows wider than 8k split K over eight waves the same
    // way: at most two 16-weight chunks per lane (K <= 16384). Measured at
    // the C3 shape (K 14336): q8 decode 384.8 -> 401.4 tok/s, q4 432.7 ->
    // 444.8.
    if constexpr (WPacked<WT>::v && EPI == DG_RESID) {
        if (nch > 2 && a.K % (8 * Chunk<WT>::W) == 0 && !getenv("ESP_DG_4W")) {
            dg_launch_nch<WT, EPI, 2, 2, 8>(a, cus, s);
            return;
        }
    }
    if (nch <= 1) dg_launch_nch<WT, EPI, 2, 1>(a, cus, s);
    else if (nch <= 2) dg_launch_nch<WT, EPI, 2, 2>(a, cus, s);
    else if (nch <= 4) dg_launch_nch<WT, EPI, 2, 4>(a, cus, s);
    else dg_launch_nch<WT, EPI, 2, DG_MAXC>(a, cus, s);
}

bool decode_gemv_ok(int K) { return K % 32 == 0 && K / 32 <= 64 * DG_MAXC; }

// Packed formats read chunks of 16 weights: each wave's quarter of K must
// hold whole chunks.
bool decode_gemv_packed_ok(Dt wt, int K) {
    return decode_gemv_ok(K) && (!dt_packed(wt) || K % (DG_WAVES * 16) == 0);
}

void launch_decode_gemv(Dt wt, int epi, const DecodeGemvArgs &a, hipStream_t s) {
    if (!decode_gemv_ok(a.K) || (dt_packed(wt) && !decode_gemv_packed_ok(wt, a.K)))
        fail(ESP_BACKEND, "decode_gemv: unsupported width");
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
        else if (wt == DT_Q8) dg_launch<q8_t, E>(a, cus, s);         \
        else if (wt == DT_Q4) dg_launch<q4_t, E>(a, cus, s);         \
        else dg_launch<float, E>(a, cus, s);                         \
        break;
    if ((wt == DT_Q8 || wt == DT_Q4) && (!a.ws || (epi == DG_SWIGLU && !a.ws2) || a.ex_sel))
        fail(ESP_BACKEND, "decode_gemv: packed weights need their block scales (no routed experts)");
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

__device__ __forceinline__ void att_store(const AttnDecodeArgs &a, size_t i, float v) {
    if (a.out_lo) {
        const uint16_t h = f2bf(v);
        ((uint16_t *)a.out)[i] = h;
        a.out_lo[i] = f2bf(v - bf2f(h));
    } else {
        a.out[i] = v;
    }
}

// One block of ATT_WAVES waves per (key split, kv head, row): a 1-D grid
// whose block -> work mapping depends on the merge protocol (below). A key
// is covered by a group of hd/8 lanes; lane `sub` of the group holds dims
// [4 sub, 4 sub + 4) and [hd/2 + 4 sub, hd/2 + 4 sub + 4), so each 16-byte
// load of the group covers a contiguous hd/2 * 4 bytes of the key row, and
// a dot product is finished with DPP swaps inside the group. The loads of
// the first two chunks of the split (both buffers) are issued right after
// q's, before the row's position is known: they cover the split's planned
// range (clamped to max_t, the plan's key bound; lanes past the range re-read
// its last key) and keys past the position are masked afterwards, so the
// position read and the K/V stream overlap. The softmax update runs once per chunk (one exp per key).
// The key groups of a wave merge through lane-pair swaps, the waves through
// LDS; the last split to finish for a (row, kv head) merges the partials in
// split order (deterministic), each thread one output with every partial
// load of a batch in flight at once.
//
// Merge protocol. With xcd_nx > 0, the splits of one (row, kv head) are
// blocks whose linear ids share the residue mod xcd_nx; the dispatcher deals
// the blocks of a launch to the XCDs round-robin (from a rotating first
// XCD), so they all run on one XCD and exchange partials through its L2:
// plain stores, then L1-bypassing loads in the merging block. With
// xcd_nx == 0 the partials go through agent-scope (write-through) stores and
// loads instead, which any placement tolerates.
template <int HD, int GM, bool XCD, int NW = ATT_WAVES, bool F16 = false>
__global__ void __launch_bounds__(NW * 64) attn_decode_k(AttnDecodeArgs a) {
    typedef typename KvSlice<F16>::T KR;
    constexpr int ES = F16 ? 2 : 4;  // bytes per cached element
    constexpr int NT = NW * 64;
    constexpr int DPL = 8;               // dims per lane
    constexpr int LPK = HD / DPL;        // lanes per key
    constexpr int KPW = 64 / LPK;        // keys per wave per step
    constexpr int STEP = NW * KPW;       // keys per block step
    // Key chunks are double-buffered: the next chunk's loads are in flight
    // while the current one is consumed. Steps per buffer, measured on
    // MI355X: the narrow (4-wave, many-row) form at the C5 batch 65.0 us per
    // launch with two (66.4 with three, 69.9 with five, 70.7 single-
    // buffered with five); the 8-wave form three over an f32 cache (C2
    // decode 1327 vs 1287-1312 tok/s single-buffered with five) and two over
    // an f16 cache (163 VGPRs, three waves per SIMD: 15.2 vs 16.4 us per
    // launch at hd 128, 4096 keys, 32 splits).
    constexpr int NS = (NW == 4 || F16) ? 2 : 3;  // steps per chunk
    constexpr int CH = NS * STEP;        // keys per chunk
    constexpr int HALF = HD / 2;
    constexpr int STRIDE = HD + ATT_PART_PAD;
    __shared__ float wm[NW][GM], wl[NW][GM];
    __shared__ __attribute__((aligned(16))) float wacc[NW][GM][HD];
    __shared__ int last;
    const int ns = a.n_split, U = a.M * a.nkv;
    int unit, split;
    {
        const int b = blockIdx.x;
        if (XCD && !a.misplace) {
            const int x = b % a.xcd_nx, i = b / a.xcd_nx;
            unit = x + a.xcd_nx * (i / ns);
            split = i % ns;
        } else {
            unit = b / ns;
            split = b % ns;
        }
        if (unit >= U) return;  // padding block of a short residue class
    }
    const int g = unit % a.nkv, row = unit / a.nkv;
    const int G = a.nq / a.nkv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp = lane / LPK, sub = lane % LPK;
    const int seq = a.seq1 >= 0 ? a.seq1 : a.row_seq[row];
    const int s0 = split * a.split_len;
    const int s1 = min(s0 + a.split_len, a.max_t);
    const char *kb = (const char *)a.kv +
                     ((size_t)seq * a.seq_stride + (size_t)g * a.head_stride + sub * 4) * ES;
    const char *vb = kb + (size_t)a.kv_half_stride * ES;
    KR kk[NS][2], vv[NS][2];
    KR kk2[NS][2], vv2[NS][2];  // the second buffer
    // lanes past the chunk end re-read its last key (masked later)
    auto issue = [&](KR (&K)[NS][2], KR (&V)[NS][2], int c0, int c1) {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            if (c0 + st * STEP < c1) {  // block-uniform
                const int t = min(c0 + st * STEP + wave * KPW + grp, c1 - 1);
                K[st][0] = __builtin_nontemporal_load((const KR *)(kb + (size_t)t * HD * ES));
                K[st][1] = __builtin_nontemporal_load((const KR *)(kb + ((size_t)t * HD + HALF) * ES));
                V[st][0] = __builtin_nontemporal_load((const KR *)(vb + (size_t)t * HD * ES));
                V[st][1] = __builtin_nontemporal_load((const KR *)(vb + ((size_t)t * HD + HALF) * ES));
            }
        }
    };
    // q for the group's heads: this lane's 8 dims
    float q[GM][DPL];
    const float *qrow = a.q + (size_t)row * a.nq * HD + (size_t)g * G * HD + sub * 4;
#pragma unroll
    for (int j = 0; j < GM; ++j)
        if (j < G) {
            const f32x4_t v0 = *(const f32x4_t *)(qrow + (size_t)j * HD);
            const f32x4_t v1 = *(const f32x4_t *)(qrow + (size_t)j * HD + HALF);
            q[j][0] = v0.x; q[j][1] = v0.y; q[j][2] = v0.z; q[j][3] = v0.w;
            q[j][4] = v1.x; q[j][5] = v1.y; q[j][6] = v1.z; q[j][7] = v1.w;
        }
    // Fast LoRA path: this thread's delta outputs o = tid + k NT, k < KO
    // (head j = o / HD, dim d = o % HD; rows of the key and value heads
    // whatever the position), B rows (rank <= 16) and the lane's rope dims
    // loaded before the first keys, so they return first.
    constexpr bool FASTOK = GM <= 4;  // eight heads per kv head would spill
    constexpr int KO = FASTOK ? ((GM + 2) * HD + NT - 1) / NT : 1;
    const bool fast = FASTOK && a.lora_on && a.lora_fast;  // block-uniform
    u32x4_t lb[KO][2];
    f32x4_t rr[4];  // cos lo, cos hi, sin lo, sin hi at this lane's dims
    // A wave's outputs share their head (HD is a multiple of 64), so the
    // target and its kernel arguments are wave-uniform (scalar reads).
    auto lsel = [&](int tg, auto p0, auto p1, auto p2) { return tg == 0 ? p0 : tg == 1 ? p1 : p2; };
    if (fast) {
#pragma unroll
        for (int k = 0; k < KO; ++k) {
            lb[k][0] = lb[k][1] = u32x4_t{0u, 0u, 0u, 0u};
            const int o = tid + k * NT;
            const int j = __builtin_amdgcn_readfirstlane(o / HD), d = o % HD;
            if (j >= G + 2) continue;
            const int tg = j < G ? 0 : j - G + 1;
            const void *bp = lsel(tg, a.lora_b[0], a.lora_b[1], a.lora_b[2]);
            if (!bp) continue;
            const size_t brow = j < G ? (size_t)(g * G + j) * HD + d : (size_t)g * HD + d;
            const int rank = lsel(tg, a.lora_rank[0], a.lora_rank[1], a.lora_rank[2]);
            const u32x4_t *B = (const u32x4_t *)((const uint16_t *)bp + brow * rank);
            lb[k][0] = B[0];
            if (rank > 8) lb[k][1] = B[1];
        }
        rr[0] = *(const f32x4_t *)(a.rope_row + sub * 4);
        rr[1] = *(const f32x4_t *)(a.rope_row + HALF + sub * 4);
        rr[2] = *(const f32x4_t *)(a.rope_row + HD + sub * 4);
        rr[3] = *(const f32x4_t *)(a.rope_row + HD + HALF + sub * 4);
    }
    issue(kk, vv, s0, min(s0 + CH, s1));
    if (s0 + CH < s1) issue(kk2, vv2, s0 + CH, min(s0 + 2 * CH, s1));
    const int pos = a.row_pos[row];
    // Unmerged LoRA of a single decode row: c = scale * B t for the group's
    // query heads (and, in the block whose split holds the new key, for this
    // kv head's key and value rows), one (head, dim) per thread into LDS;
    // each lane then adds its dims' rotated deltas to q, and keeps the new
    // key / value row's deltas for the patch in consume().
    __shared__ float lc[GM + 2][HD];
    float kd[DPL], vd[DPL];
    bool kv_patch = false;
    if (fast) {
        const bool own = pos >= s0 && pos < s1;
#pragma unroll
        for (int k = 0; k < KO; ++k) {
            const int o = tid + k * NT;
            const int j = __builtin_amdgcn_readfirstlane(o / HD), d = o % HD;
            if (j >= G + 2) break;
            const int tg = j < G ? 0 : j - G + 1;
            float c = 0.f;
            if (lsel(tg, a.lora_b[0], a.lora_b[1], a.lora_b[2])) {
                const float *t = lsel(tg, a.lora_t[0], a.lora_t[1], a.lora_t[2]);
                const int rank = lsel(tg, a.lora_rank[0], a.lora_rank[1], a.lora_rank[2]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if (h * 8 >= rank) break;
                    const u32x4_t b = lb[k][h];
                    const float *tt = t + 8 * h;
                    c += __uint_as_float(b.x << 16) * tt[0] + __uint_as_float(b.x & 0xffff0000u) * tt[1] +
                         __uint_as_float(b.y << 16) * tt[2] + __uint_as_float(b.y & 0xffff0000u) * tt[3] +
                         __uint_as_float(b.z << 16) * tt[4] + __uint_as_float(b.z & 0xffff0000u) * tt[5] +
                         __uint_as_float(b.w << 16) * tt[6] + __uint_as_float(b.w & 0xffff0000u) * tt[7];
                }
                c = c * lsel(tg, a.lora_scale[0], a.lora_scale[1], a.lora_scale[2]);
            }
            lc[j][d] = c;
        }
        lds_barrier();
        auto rot = [&](const float *c, float *out) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x0 = c[sub * 4 + e], x1 = c[HALF + sub * 4 + e];
                out[e] = x0 * rr[0][e] + (-x1) * rr[2][e];
                out[4 + e] = x1 * rr[1][e] + x0 * rr[3][e];
            }
        };
#pragma unroll
        for (int j = 0; j < GM; ++j) {
            if (j >= G) break;
            float dq[DPL];
            rot(lc[j], dq);
#pragma unroll
            for (int e = 0; e < DPL; ++e) q[j][e] += dq[e];
        }
        if (own && (a.lora_b[1] || a.lora_b[2])) {
            kv_patch = true;
            rot(lc[G], kd);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vd[e] = lc[G + 1][sub * 4 + e];
                vd[4 + e] = lc[G + 1][HALF + sub * 4 + e];
            }
        }
    } else if (a.lora_on) {  // block-uniform
        const bool own = pos >= s0 && pos < s1;
        for (int o = tid; o < (G + 2) * HD; o += NT) {
            const int j = o / HD, d = o % HD;
            if (j >= G && !own) continue;
            const int tg = j < G ? 0 : j - G + 1;
            const size_t brow = j < G ? (size_t)(g * G + j) * HD + d : (size_t)g * HD + d;
            float c = 0.f;
            if (a.lora_b[tg]) {
                const int rank = a.lora_rank[tg];
                const float *t = a.lora_t[tg];
                if (a.lora_vec) {  // bf16 rows of 8k values, 16-byte aligned rows and t
                    const uint4 *B = (const uint4 *)((const uint16_t *)a.lora_b[tg] + brow * rank);
                    const f32x4_t *t4 = (const f32x4_t *)t;
#pragma unroll 4
                    for (int i = 0; i < rank / 8; ++i) {
                        const uint4 b = B[i];
                        const f32x4_t ta = t4[2 * i], tb = t4[2 * i + 1];
                        c += __uint_as_float(b.x << 16) * ta.x + __uint_as_float(b.x & 0xffff0000u) * ta.y +
                             __uint_as_float(b.y << 16) * ta.z + __uint_as_float(b.y & 0xffff0000u) * ta.w +
                             __uint_as_float(b.z << 16) * tb.x + __uint_as_float(b.z & 0xffff0000u) * tb.y +
                             __uint_as_float(b.w << 16) * tb.z + __uint_as_float(b.w & 0xffff0000u) * tb.w;
                    }
                } else if (a.lora_b_f32) {
                    const float *B = (const float *)a.lora_b[tg] + brow * rank;
                    for (int i = 0; i < rank; ++i) c += B[i] * t[i];
                } else {
                    const uint16_t *B = (const uint16_t *)a.lora_b[tg] + brow * rank;
                    for (int i = 0; i < rank; ++i) c += bf2f(B[i]) * t[i];
                }
                c = c * a.lora_scale[tg];
            }
            lc[j][d] = c;
        }
        const float *cs = a.rope_cos + (size_t)pos * HD + sub * 4;
        const float *sn = a.rope_sin + (size_t)pos * HD + sub * 4;
        const f32x4_t c_lo = *(const f32x4_t *)cs, c_hi = *(const f32x4_t *)(cs + HALF);
        const f32x4_t s_lo = *(const f32x4_t *)sn, s_hi = *(const f32x4_t *)(sn + HALF);
        __syncthreads();
        // RoPE of the delta pair (d, d + HD/2), as the QKV epilogue rotates y
        auto rot = [&](const float *c, float *out) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x0 = c[sub * 4 + e], x1 = c[HALF + sub * 4 + e];
                out[e] = x0 * c_lo[e] + (-x1) * s_lo[e];
                out[4 + e] = x1 * c_hi[e] + x0 * s_hi[e];
            }
        };
#pragma unroll
        for (int j = 0; j < GM; ++j) {
            if (j >= G) break;
            float dq[DPL];
            rot(lc[j], dq);
#pragma unroll
            for (int e = 0; e < DPL; ++e) q[j][e] += dq[e];
        }
        if (own && (a.lora_b[1] || a.lora_b[2])) {
            kv_patch = true;
            rot(lc[G], kd);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vd[e] = lc[G + 1][sub * 4 + e];
                vd[4 + e] = lc[G + 1][HALF + sub * 4 + e];
            }
        }
    }
    int lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
    int hi = min(pos + 1, a.max_t);
    lo = max(lo, s0);
    hi = min(hi, s1);
    const float inv_scale = 1.f / sqrtf((float)HD);
    float m[GM], l[GM], acc[GM][DPL];
#pragma unroll
    for (int j = 0; j < GM; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
    }
    // one chunk's keys [c0, c1) from a register buffer
    // Keys and values are widened to f32 one step at a time (scores from K,
    // then the V accumulation), so no chunk is held twice in registers.
    auto consume = [&](KR (&kr)[NS][2], KR (&vr)[NS][2], int c0, int c1) {
        bool ok[NS];
        float sc[GM][NS];
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const int t = c0 + st * STEP + wave * KPW + grp;
            ok[st] = t >= lo && t < c1;
            if (kv_patch && t == pos && c0 + st * STEP < c1) {
                // the new key's LoRA deltas, kept in the cache for later steps
                f32x4_t k0 = kv_f32(kr[st][0]), k1 = kv_f32(kr[st][1]);
                f32x4_t v0 = kv_f32(vr[st][0]), v1 = kv_f32(vr[st][1]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    k0[e] += kd[e];
                    k1[e] += kd[4 + e];
                    v0[e] += vd[e];
                    v1[e] += vd[4 + e];
                }
                char *kw = (char *)kb + (size_t)pos * HD * ES, *vw = (char *)vb + (size_t)pos * HD * ES;
                if constexpr (F16) {  // what the cache holds is what every later step reads
                    kr[st][0] = kv_f16(k0);
                    kr[st][1] = kv_f16(k1);
                    vr[st][0] = kv_f16(v0);
                    vr[st][1] = kv_f16(v1);
                } else {
                    kr[st][0] = k0;
                    kr[st][1] = k1;
                    vr[st][0] = v0;
                    vr[st][1] = v1;
                }
                *(KR *)kw = kr[st][0];
                *(KR *)(kw + HALF * ES) = kr[st][1];
                *(KR *)vw = vr[st][0];
                *(KR *)(vw + HALF * ES) = vr[st][1];
            }
            if (c0 + st * STEP < c1) {  // block-uniform
                const f32x4_t k0 = kv_f32(kr[st][0]), k1 = kv_f32(kr[st][1]);
#pragma unroll
                for (int j = 0; j < GM; ++j) {
                    if (j >= G) break;
                    const float d0 = q[j][0] * k0[0] + q[j][1] * k0[1];
                    const float d1 = q[j][2] * k0[2] + q[j][3] * k0[3];
                    const float d2 = q[j][4] * k1[0] + q[j][5] * k1[1];
                    const float d3 = q[j][6] * k1[2] + q[j][7] * k1[3];
                    const float d = group_sum<LPK>((d0 + d1) + (d2 + d3));
                    sc[j][st] = ok[st] ? d * inv_scale : -INFINITY;
                }
            } else {
#pragma unroll
                for (int j = 0; j < GM; ++j) sc[j][st] = -INFINITY;
            }
        }
        // online-softmax update per head; sc becomes the weights p (0 for a
        // head with no key of this lane's group in the chunk yet)
#pragma unroll
        for (int j = 0; j < GM; ++j) {
            if (j >= G) break;
            float mx = m[j];
#pragma unroll
            for (int st = 0; st < NS; ++st) mx = fmaxf(mx, sc[j][st]);
            if (mx == -INFINITY) {
#pragma unroll
                for (int st = 0; st < NS; ++st) sc[j][st] = 0.f;
                continue;
            }
            const float al = __expf(m[j] - mx);
            l[j] *= al;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[j][e] *= al;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[j][st] = __expf(sc[j][st] - mx);
                l[j] += sc[j][st];
            }
            m[j] = mx;
        }
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            if (c0 + st * STEP >= c1) continue;  // block-uniform
            const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
            // unread or unwritten rows contribute nothing (their weight is 0)
            const f32x4_t v0 = ok[st] ? kv_f32(vr[st][0]) : z, v1 = ok[st] ? kv_f32(vr[st][1]) : z;
#pragma unroll
            for (int j = 0; j < GM; ++j) {
                if (j >= G) break;
                const float pw = sc[j][st];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][e] += pw * v0[e];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[j][4 + e] += pw * v1[e];
            }
        }
    };
    // Chunks alternate between the buffers. Both first chunks were issued
    // before q and the position were read; a buffer is refilled with the
    // chunk two ahead right after it has been consumed. Loads cover the
    // split's planned range (keys past the row's position are masked), so
    // chunk k always starts at s0 + k CH.
    for (int c0 = s0; c0 < hi;) {
        const int c1 = min(c0 + CH, hi);
        consume(kk, vv, c0, c1);
        if (c1 >= hi) break;
        if (c0 + 2 * CH < s1) issue(kk, vv, c0 + 2 * CH, min(c0 + 3 * CH, s1));
        const int c2 = min(c1 + CH, hi);
        consume(kk2, vv2, c1, c2);
        if (c2 >= hi) break;
        if (c1 + 2 * CH < s1) issue(kk2, vv2, c1 + 2 * CH, min(c1 + 3 * CH, s1));
        c0 = c2;
    }
    // merge the KPW key groups of the wave: lane pairs at distance LPK .. 32
    att_wave_merge<LPK, GM>(G, m, l, acc);
    if (grp == 0) {
#pragma unroll
        for (int j = 0; j < GM; ++j) {
            if (j >= G) break;
            *(f32x4_t *)&wacc[wave][j][sub * 4] = f32x4_t{acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
            *(f32x4_t *)&wacc[wave][j][HALF + sub * 4] = f32x4_t{acc[j][4], acc[j][5], acc[j][6], acc[j][7]};
            if (sub == 0) {
                wm[wave][j] = m[j];
                wl[wave][j] = l[j];
            }
        }
    }
    __syncthreads();
    // merge the waves; write this split's partial (m, l, -, -, acc[HD]) per head
    for (int o = tid; o < G * HD; o += NT) {
        const int j = o / HD, d = o % HD;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wm[w][j]);
        float L = 0.f, v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float sc = mx == -INFINITY ? 0.f : __expf(wm[w][j] - mx);
            L += wl[w][j] * sc;
            v += wacc[w][j][d] * sc;
        }
        if (ns == 1) {  // single split: normalise directly
            att_store(a, (size_t)row * a.nq * HD + (size_t)(g * G + j) * HD + d, v / L);
            continue;
        }
        float *p = a.part + (((size_t)row * a.nq + (size_t)g * G + j) * ns + split) * STRIDE;
        if (XCD) {
            p[ATT_PART_PAD + d] = v;
            if (d == 0) {
                p[0] = mx;
                p[1] = L;
            }
        } else {
            st_agent(p + ATT_PART_PAD + d, v);
            if (d == 0) {
                st_agent(p, mx);
                st_agent(p + 1, L);
            }
        }
    }
    if (ns == 1) return;
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        // one device-scope add counts the split and the XCD it ran on
        const unsigned xcc = XCD ? __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 7u : 0u;
        unsigned long long *tk = a.ticket + unit;
        const unsigned long long t = atomicAdd(tk, 1ull + (1ull << (8 + 7 * xcc)));
        last = (int)(t & 0xffu) == ns - 1;
        if (last) {
            *tk = 0;
            // every earlier split must have run on this block's XCD, or its
            // plain stores may still sit in another XCD's L2
            if (XCD && (int)((t >> (8 + 7 * xcc)) & 0x7fu) != ns - 1) atomicOr(a.xcd_err, 1);
        }
    }
    __syncthreads();
    if (!last) return;
    // Merge in the last block, splits in batches of ATT_MB: each thread owns
    // one output of one head and issues its partial loads of the batch
    // first; the batch's (m, l) pairs are read once into LDS meanwhile. A
    // running maximum carries across batches; splits are summed in order
    // (deterministic). Offsets past the last split are clamped (their weight
    // is zero), so the loads carry no predicates.
    __shared__ float bm_[GM][ATT_MB], bl_[GM][ATT_MB];
    const float *pb = a.part + ((size_t)row * a.nq + (size_t)g * G) * ns * STRIDE;
    // L1-bypassing (sc0) loads of this unit's partial rows
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)pb, (short)0, G * ns * STRIDE * (int)sizeof(float), 0x00020000);
    auto ld1 = [&](int off) -> float {
        if (XCD) return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off * 4, 0, 1));
        return ld_agent(pb + off);
    };
    auto ld2 = [&](int off, float &x, float &y) {
        if (XCD) {
            const auto r = __builtin_amdgcn_raw_buffer_load_b64(rs, off * 4, 0, 1);
            x = __uint_as_float(r[0]);
            y = __uint_as_float(r[1]);
        } else {
            x = ld_agent(pb + off);
            y = ld_agent(pb + off + 1);
        }
    };
    for (int o = tid; o < ((G * HD + NT - 1) / NT) * NT; o += NT) {
        const bool own = o < G * HD;  // wave-uniform
        const int j = own ? o / HD : 0, d = own ? o % HD : 0;
        float M = -INFINITY, L = 0.f, V = 0.f;
        for (int sp0 = 0; sp0 < ns; sp0 += ATT_MB) {
            float tv[ATT_MB];
            if (own) {
#pragma unroll
                for (int q = 0; q < ATT_MB; ++q)
                    tv[q] = ld1((j * ns + min(sp0 + q, ns - 1)) * STRIDE + ATT_PART_PAD + d);
            }
            __syncthreads();  // previous batch's (m, l) reads are done
            if (tid < G * ATT_MB) {
                const int jj = tid / ATT_MB, q = tid % ATT_MB;
                float mv, lv;
                ld2((jj * ns + min(sp0 + q, ns - 1)) * STRIDE, mv, lv);
                bm_[jj][q] = sp0 + q < ns ? mv : -INFINITY;
                bl_[jj][q] = lv;
            }
            __syncthreads();
            if (!own) continue;
            float bmax = M;
#pragma unroll
            for (int q = 0; q < ATT_MB; ++q) bmax = fmaxf(bmax, bm_[j][q]);
            if (bmax == -INFINITY) continue;
            const float r = __expf(M - bmax);
            L *= r;
            V *= r;
#pragma unroll
            for (int q = 0; q < ATT_MB; ++q) {
                const float w = __expf(bm_[j][q] - bmax);
                L += bl_[j][q] * w;
                V += tv[q] * w;
            }
            M = bmax;
        }
        if (own) att_store(a, (size_t)row * a.nq * HD + (size_t)g * G * HD + o, V / L);
    }
}

bool attn_decode_ok(int hd, int G) { return (hd == 64 || hd == 128) && G <= 8; }

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        ESP_HIP(hipGetDevice(&dev));
        ESP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus <= 0) cus = 256;
    }
    return cus;
}

// Key splits for M decode rows over max_t cached keys: about one block per
// CU in total (rows x kv heads x splits), but no split shorter than one block
// step while the rows alone do not fill the chip; split lengths are
// multiples of the keys one wave covers per step; at most ATT_MAX_SPLIT
// splits.
// A single row at head_dim 64 over at most 2048 keys (the 1B shape's
// decode): four-wave blocks, about one per two CUs. Measured at C2 decode
// (~640 keys): 1336-1337 -> 1345.6-1346.4 tok/s (block targets 256 / 512:
// 1343-1344 / 1342-1343).
static bool att_short_row(int hd, int M, int max_t) { return hd == 64 && M == 1 && max_t <= 2048; }

int attn_decode_splits(int hd, int nkv, int G, int M, int max_t, int *split_len) {
    (void)G;
    const bool shrt = att_short_row(hd, M, max_t);
    const int kpw = 64 * 8 / hd, step = (shrt ? 4 : ATT_WAVES) * kpw;
    const int target = shrt ? device_cus() / 2 : device_cus();
    const long long base = (long long)M * (nkv > 0 ? nkv : 1);
    int ns = (int)((target + base - 1) / base);
    ns = std::min(ns, (max_t + step - 1) / step);
    ns = std::max(1, std::min(ns, ATT_MAX_SPLIT));
    int len = (max_t + ns - 1) / ns;
    len = std::max(kpw, (len + kpw - 1) / kpw * kpw);
    ns = (max_t + len - 1) / len;
    if (ns < 1) ns = 1;
    *split_len = len;
    return ns;
}

// Probe of the dispatch order the XCD-local merge relies on: in every
// launch, blocks whose linear ids share a residue mod the XCD count run on
// one XCD. Checked once per process on the current device over launches of
// several sizes; any mismatch selects the agent-scope merge.
__global__ void xcc_probe_k(int32_t *out) {
    const unsigned x = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20);  // HW_REG_XCC_ID[3:0]
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)x;
}

static int g_xcd_off = 0;  // set once a launch reported a split across XCDs

void attn_xcd_disable() { g_xcd_off = 1; }

int attn_xcd_mode() {
    static int mode = -1;
    if (g_xcd_off) return 0;
    if (mode < 0) {
        int dev = 0, nx = 0;
        ESP_HIP(hipGetDevice(&dev));
        if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || nx < 1) nx = 0;
        mode = 0;
        if (nx == 1) {
            mode = 1;
        } else if (nx > 1) {
            const int sizes[4] = {7, 256, 1000, 4099};
            int32_t *d = nullptr;
            ESP_HIP(hipMalloc(&d, 4099 * sizeof(int32_t)));
            std::vector<int32_t> h(4099);
            bool ok = true;
            for (int rep = 0; rep < 16 && ok; ++rep) {
                const int nb = sizes[rep % 4];
                xcc_probe_k<<<nb, 64>>>(d);
                ESP_HIP(hipMemcpy(h.data(), d, nb * sizeof(int32_t), hipMemcpyDeviceToHost));
                for (int b = nx; b < nb && ok; ++b) ok = h[b] == h[b % nx];
            }
            ESP_HIP(hipFree(d));
            mode = ok ? nx : 0;
        }
    }
    const char *e = getenv("ESP_ATT_XCD");
    if (e && e[0] == '0') return 0;
    return mode;
}

void launch_attn_decode(const AttnDecodeArgs &a0, hipStream_t s) {
    AttnDecodeArgs a = a0;
    const int G = a.nq / a.nkv;
    if (!attn_decode_ok(a.hd, G)) fail(ESP_BACKEND, "attn_decode: unsupported head shape");
    if (a.n_split > ATT_MAX_SPLIT) fail(ESP_BACKEND, "attn_decode: too many key splits");
    if (a.max_t < 1 || (long long)a.n_split * a.split_len < a.max_t)
        fail(ESP_BACKEND, "attn_decode: key splits do not cover max_t");
    const long long U = (long long)a.M * a.nkv;
    if (a.n_split > 1 && U > ATT_MAX_TICKETS)
        fail(ESP_BACKEND, "attn_decode: too many (row, kv head) merges");
    {
        // batches whose units fill the chip without key splits: matrix cores
        // (ESP_ATT_MFMA=0 keeps the vector form, for comparison)
        const char *am = getenv("ESP_ATT_MFMA");
        const long long Ur = (long long)(a.grp ? a.ngrp : a.M) * a.nkv;  // its units: row groups
        if (Ur >= device_cus() && attn_rows_mfma_ok(a) && !(am && am[0] == '0')) {
            launch_attn_rows_mfma(a, s);
            return;
        }
    }
    a.xcd_nx = a.n_split > 1 ? attn_xcd_mode() : 0;
    {
        const char *mp = getenv("ESP_ATT_XCD_MISPLACE");
        a.misplace = a.xcd_nx > 0 && mp && mp[0] == '1';
    }
    long long nb = a.xcd_nx > 0 ? (long long)a.xcd_nx * ((U + a.xcd_nx - 1) / a.xcd_nx) * a.n_split
                                : U * a.n_split;
    if (nb > 0x7fffffffLL) fail(ESP_BACKEND, "attn_decode: grid too large");
    dim3 grid((unsigned)nb);
    // Many rows (batched decode) already fill the chip without key splits:
    // four-wave blocks then let two blocks share a CU, so one block's loads
    // overlap the other's scores across the chunks of a long split. A short
    // single row at head_dim 64 takes them too (att_short_row).
    const bool narrow = att_short_row(a.hd, a.M, a.max_t) ||
                        (U >= device_cus() && a.split_len > 2 * ATT_WAVES * 64 * 8 / a.hd);
#define ATT_LAUNCH_T(HD_, GM_, F16_)                                                           \
    do {                                                                                   \
        if (narrow) {                                                                      \
            if (a.xcd_nx > 0) attn_decode_k<HD_, GM_, true, 4, F16_><<<grid, 4 * 64, 0, s>>>(a);   \
            else attn_decode_k<HD_, GM_, false, 4, F16_><<<grid, 4 * 64, 0, s>>>(a);              \
        } else if (a.xcd_nx > 0) {                                                         \
            attn_decode_k<HD_, GM_, true, ATT_WAVES, F16_><<<grid, ATT_WAVES * 64, 0, s>>>(a);      \
        } else {                                                                           \
            attn_decode_k<HD_, GM_, false, ATT_WAVES, F16_><<<grid, ATT_WAVES * 64, 0, s>>>(a);     \
        }                                                                                  \
    } while (0)
#define ATT_LAUNCH(HD_, GM_)                       \
    do {                                           \
        if (a.kv_f16) ATT_LAUNCH_T(HD_, GM_, true); \
        else ATT_LAUNCH_T(HD_, GM_, false);        \
    } while (0)
    if (a.hd == 64) {
        if (G <= 4) ATT_LAUNCH(64, 4);
        else ATT_LAUNCH(64, 8);
    } else {
        if (G <= 4) ATT_LAUNCH(128, 4);
        else ATT_LAUNCH(128, 8);
    }
#undef ATT_LAUNCH
#undef ATT_LAUNCH_T
}

}  // namespace esp
