// Routed experts (moe.rs:135-256): fp32 softmax router, top-k by
// probability with ties to the lower expert id, optional renormalisation,
// per-expert row grouping, and the combine that adds each token's expert
// outputs in ascending expert order before the sigmoid-gated shared expert.
#include "common.hpp"
#include "dev.hpp"
#include "kernels_extra.hpp"

namespace esp {

// Top-k of one row per thread over the whole grid. A row whose softmax is
// not finite (status 2) or whose top-k mass is not positive (status 3) marks
// its selections with -status for the grouping pass.
__device__ void route_row(const RouteArgs &a, int t) {
    const int E = a.E, k = a.k;
    const float *l = a.logits + (size_t)t * E;
    float mx = -INFINITY;
    for (int e = 0; e < E; ++e) mx = fmaxf(mx, l[e]);
    float sum = 0.f;
    for (int e = 0; e < E; ++e) sum += expf(l[e] - mx);
    bool bad = false;
    for (int e = 0; e < E; ++e) bad |= !isfinite(expf(l[e] - mx) / sum);
    if (bad) {
        for (int j = 0; j < k; ++j) a.sel[(size_t)t * k + j] = -2;
        return;
    }
    // top-k by (probability desc, id asc) (moe.rs:166)
    int chosen[8];
    float prob[8];
    for (int j = 0; j < k; ++j) {
        int best = -1;
        float bp = 0.f;
        for (int e = 0; e < E; ++e) {
            bool used = false;
            for (int i = 0; i < j; ++i) used |= chosen[i] == e;
            if (used) continue;
            float p = expf(l[e] - mx) / sum;
            if (best < 0 || p > bp) {
                best = e;
                bp = p;
            }
        }
        chosen[j] = best;
        prob[j] = bp;
    }
    float mass = 1.0f;
    if (a.norm_topk) {
        mass = 0.f;
        for (int j = 0; j < k; ++j) mass += prob[j];
    }
    if (!isfinite(mass) || mass <= 0.f) {
        for (int j = 0; j < k; ++j) a.sel[(size_t)t * k + j] = -3;
        return;
    }
    // store ascending by expert id
    for (int j = 0; j < k; ++j) {
        int rank = 0;
        for (int i = 0; i < k; ++i) rank += chosen[i] < chosen[j];
        a.sel[(size_t)t * k + rank] = chosen[j];
        a.w[(size_t)t * k + rank] = prob[j] / mass;
    }
}

// route_row for one row by a whole wave (E <= 64): lane e computes expert
// e's exponential and probability, the max and the sum (in expert order, as
// route_row adds them) come from the lanes' values, and lane 0 picks the
// top-k from the probabilities in LDS. Same values as route_row, with one
// exponential per expert instead of 2 + k.
__device__ void route_row_wave(const RouteArgs &a, int t, float *pr, int *ssel = nullptr) {
    const int E = a.E, k = a.k, lane = threadIdx.x & 63;
    const float *l = a.logits + (size_t)t * E;
    const float x = lane < E ? l[lane] : -INFINITY;
    float mx = -INFINITY;
    for (int e = 0; e < E; ++e) mx = fmaxf(mx, __shfl(x, e, 64));
    const float ex = lane < E ? expf(x - mx) : 0.f;
    float sum = 0.f;
    for (int e = 0; e < E; ++e) sum += __shfl(ex, e, 64);
    const float p = ex / sum;
    const bool bad = __any(lane < E && !isfinite(p));
    if (bad) {
        if (lane < k) {
            a.sel[(size_t)t * k + lane] = -2;
            if (ssel) ssel[t * k + lane] = -2;
        }
        return;
    }
    if (lane < E) pr[lane] = p;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane != 0) return;
    int chosen[8];
    float prob[8];
    for (int j = 0; j < k; ++j) {
        int best = -1;
        float bp = 0.f;
        for (int e = 0; e < E; ++e) {
            bool used = false;
            for (int i = 0; i < j; ++i) used |= chosen[i] == e;
            if (used) continue;
            const float q = pr[e];
            if (best < 0 || q > bp) {
                best = e;
                bp = q;
            }
        }
        chosen[j] = best;
        prob[j] = bp;
    }
    float mass = 1.0f;
    if (a.norm_topk) {
        mass = 0.f;
        for (int j = 0; j < k; ++j) mass += prob[j];
    }
    if (!isfinite(mass) || mass <= 0.f) {
        for (int j = 0; j < k; ++j) {
            a.sel[(size_t)t * k + j] = -3;
            if (ssel) ssel[t * k + j] = -3;
        }
        return;
    }
    for (int j = 0; j < k; ++j) {
        int rank = 0;
        for (int i = 0; i < k; ++i) rank += chosen[i] < chosen[j];
        a.sel[(size_t)t * k + rank] = chosen[j];
        a.w[(size_t)t * k + rank] = prob[j] / mass;
        if (ssel) ssel[t * k + rank] = chosen[j];
    }
}

// Decode-sized routing (up to 16 rows, 64 selections and 64 experts): one
// wave takes the rows in turn and then groups the selections from its LDS
// copy with ballots (counts per expert, ranks from the lanes below), the
// same offsets, grouped rows and tokens as route_group.
__global__ void __launch_bounds__(64) route_small_k(RouteArgs a) {
    __shared__ float pr[64];
    __shared__ int ssel[64];
    const int lane = threadIdx.x, E = a.E, k = a.k, R = a.M * k;
    for (int t = 0; t < a.M; ++t) route_row_wave(a, t, pr, ssel);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int sv = lane < R ? ssel[lane] : E;  // E: no selection
    int status = max(0, -sv);
    for (int o = 32; o >= 1; o >>= 1) status = max(status, __shfl_xor(status, o, 64));
    if (status) {
        if (lane == 0) {
            for (int e = 0; e <= E; ++e) a.offs[e] = 0;
            a.offs[E + 1] = status;
            if (a.err) atomicMax(a.err, status);
            if (a.err && a.step) atomicMin(a.err + 1, (a.step[0] << 2) | status);
        }
        if (lane < R) {
            a.slot[lane] = lane;
            a.perm[lane] = lane / k;
        }
        return;
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    int start = 0, my = 0;
    for (int e = 0; e < E; ++e) {
        const unsigned long long m = __ballot(sv == e);
        if (lane == 0) a.offs[e] = start;
        if (sv == e) my = start + __popcll(m & below);
        start += __popcll(m);
    }
    if (lane == 0) {
        a.offs[E] = start;
        a.offs[E + 1] = 0;
    }
    if (lane < R) {
        a.slot[lane] = my;
        a.perm[my] = lane / k;
    }
}

__global__ void __launch_bounds__(256) route_topk_k(RouteArgs a) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < a.M) route_row(a, t);
}

// Grouping of all selections by one block: the failure status of any row,
// then the expert offsets, the grouped row of each selection and the token
// of each grouped row.
__device__ void route_group(const RouteArgs &a) {
    const int E = a.E, k = a.k;
    const int R = a.M * k;
    const int nt = blockDim.x, tid = threadIdx.x;
    __shared__ int status;
    if (tid == 0) status = 0;
    __syncthreads();
    const int per = (R + nt - 1) / nt, b0 = min(R, tid * per), b1 = min(R, b0 + per);
    constexpr int EMAX = 32;  // experts handled by the parallel forms
    constexpr int PF = 16;    // selections per thread held in registers
    // register form (up to 4096 selections): the thread's range is loaded
    // once, counted per expert, scanned across the block with wave prefix
    // sums and placed; it computes the same ranks as the forms below
    const bool fast = E <= EMAX && per <= PF && nt == 256;
    int sv[PF];
    {
        int st = 0;
        if (fast) {
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                sv[j] = b0 + j < b1 ? a.sel[b0 + j] : E;  // E: no selection
                st = max(st, -sv[j]);
            }
        } else {
            for (int i = b0; i < b1; ++i) st = max(st, -a.sel[i]);
        }
        if (st > 0) atomicMax(&status, st);
    }
    __syncthreads();
    if (status) {
        // No expert gets a row; the grouped rows and the combine still index
        // in bounds (identity slots). The sticky word reports the layer's
        // failure to the host at the end of the forward.
        if (tid == 0) {
            for (int e = 0; e <= E; ++e) a.offs[e] = 0;
            a.offs[E + 1] = status;
            if (a.err) atomicMax(a.err, status);
            if (a.err && a.step) atomicMin(a.err + 1, (a.step[0] << 2) | status);
        }
        for (int i = tid; i < R; i += nt) {
            a.slot[i] = i;
            a.perm[i] = i / k;
        }
        return;
    }
    // Stable grouping: selection i = t*k + j (token-major) gets the rank of
    // i among the selections of its expert. Each thread counts a contiguous
    // range of selections per expert, an exclusive scan over threads gives
    // every range its start, and the ranges are then placed in parallel:
    // rows of an expert stay in token order.
    __shared__ int tc[EMAX][257];
    __shared__ int eoff[257];
    if (fast) {
        __shared__ int wtot[EMAX][4];
        const int lane = tid & 63, wv = tid >> 6;
        for (int e = 0; e < E; ++e) {
            int v = 0;
#pragma unroll
            for (int j = 0; j < PF; ++j) v += sv[j] == e;
            int x = v;  // inclusive prefix over the wave's threads
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(x, o, 64);
                if (lane >= o) x += y;
            }
            tc[e][tid] = x - v;
            if (lane == 63) wtot[e][wv] = x;
        }
        __syncthreads();
        if (tid == 0) {
            int acc = 0;
            for (int e = 0; e < E; ++e) {
                a.offs[e] = acc;
                eoff[e] = acc;
                for (int w = 0; w < 4; ++w) {
                    const int c = wtot[e][w];
                    wtot[e][w] = acc - eoff[e];
                    acc += c;
                }
            }
            a.offs[E] = acc;
            a.offs[E + 1] = 0;
        }
        __syncthreads();
        for (int e = 0; e < E; ++e) tc[e][tid] += eoff[e] + wtot[e][wv];
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            if (b0 + j >= b1) break;
            const int c = tc[sv[j]][tid]++;
            a.perm[c] = (b0 + j) / k;
            a.slot[b0 + j] = c;
        }
        return;
    }
    if (E <= EMAX) {
        const int nact = (R + per - 1) / per;  // threads holding selections
        for (int e = 0; e < E; ++e) tc[e][tid] = 0;
        for (int i = b0; i < b1; ++i) tc[a.sel[i]][tid] += 1;
        __syncthreads();
        if (tid < E) {  // exclusive scan of expert tid's counts over threads
            int acc = 0;
            for (int t = 0; t < nact; ++t) {
                const int c = tc[tid][t];
                tc[tid][t] = acc;
                acc += c;
            }
            eoff[tid] = acc;  // expert total
        }
        __syncthreads();
        if (tid == 0) {
            int acc = 0;
            for (int e = 0; e < E; ++e) {
                const int c = eoff[e];
                eoff[e] = acc;
                a.offs[e] = acc;
                acc += c;
            }
            a.offs[E] = acc;
            a.offs[E + 1] = 0;
        }
        __syncthreads();
        int run[EMAX];
        for (int e = 0; e < E; ++e) run[e] = eoff[e] + tc[e][tid];
        for (int i = b0; i < b1; ++i) {
            const int e = a.sel[i];
            int c = 0;
            for (int q = 0; q < E; ++q)
                if (q == e) c = run[q]++;
            a.perm[c] = i / k;
            a.slot[i] = c;
        }
        return;
    }
    __shared__ int cnt[257];
    for (int e = tid; e < E; e += nt) {
        int c = 0;
        for (int i = 0; i < R; ++i) c += a.sel[i] == e;
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            a.offs[e] = acc;
            int c = cnt[e];
            cnt[e] = acc;
            acc += c;
        }
        a.offs[E] = acc;
        a.offs[E + 1] = 0;
    }
    __syncthreads();
    for (int e = tid; e < E; e += nt) {
        int c = cnt[e];
        for (int i = 0; i < R; ++i)
            if (a.sel[i] == e) {
                a.perm[c] = i / k;
                a.slot[i] = c;
                ++c;
            }
    }
}

__global__ void __launch_bounds__(256) route_group_k(RouteArgs a) { route_group(a); }

// Up to 256 rows (decode, short batches): one block, one launch; up to 16
// rows of at most 64 experts take a wave per row.
__global__ void __launch_bounds__(256) route_k(RouteArgs a) {
    __shared__ float pr[4][64];
    const int wave = threadIdx.x >> 6;
    if (a.M <= 16 && a.E <= 64) {
        for (int t = wave; t < a.M; t += 4) route_row_wave(a, t, pr[wave]);
    } else if ((int)threadIdx.x < a.M) {
        route_row(a, threadIdx.x);
    }
    __syncthreads();
    route_group(a);
}

// More rows: the rows' top-k over the grid, one row per thread (one block
// walking the 2048 rows of a MoE prefill layer took 134 us), then the
// grouping in one block.
void launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.E > 256 || a.k > 8) fail(ESP_UNSUPPORTED, "config.experts: more than 256 experts or top-k above 8");
    if (a.M <= 16 && a.M * a.k <= 64 && a.E <= 64) {
        route_small_k<<<1, 64, 0, s>>>(a);
        return;
    }
    if (a.M <= 256) {
        route_k<<<1, 256, 0, s>>>(a);
        return;
    }
    route_topk_k<<<(a.M + 255) / 256, 256, 0, s>>>(a);
    route_group_k<<<1, 256, 0, s>>>(a);
}

template <typename T>
__global__ void __launch_bounds__(256) gather_k(const T *src, const int32_t *perm, int H, T *dst) {
    int r = blockIdx.x;
    const T *s = src + (size_t)perm[r] * H;
    for (int j = threadIdx.x; j < H; j += blockDim.x) dst[(size_t)r * H + j] = s[j];
}

void launch_gather_rows(Dt dt, const void *src, const int32_t *perm, int rows, int H, void *dst,
                        hipStream_t s) {
    if (!rows) return;
    if (dt == DT_BF16) gather_k<uint16_t><<<rows, 256, 0, s>>>((const uint16_t *)src, perm, H, (uint16_t *)dst);
    else gather_k<float><<<rows, 256, 0, s>>>((const float *)src, perm, H, (float *)dst);
}

// One thread per (token, hidden element): every load of a thread is
// independent, so a single decode row costs one memory round trip.
__global__ void __launch_bounds__(256) combine_k(CombineArgs a) {
    const int t = blockIdx.x, d = blockIdx.y * blockDim.x + threadIdx.x;
    if (d >= a.H) return;
    float out = 0.f;
    for (int j = 0; j < a.k; ++j) {
        float y = a.y[(size_t)a.slot[(size_t)t * a.k + j] * a.H + d];
        out = out + y * a.w[(size_t)t * a.k + j];
    }
    if (a.ys) {
        const float g = 1.0f / (1.0f + expf(-a.sg[t]));
        out = out + g * a.ys[(size_t)t * a.H + d];
    }
    a.h[(size_t)t * a.H + d] += out;
}

void launch_combine(const CombineArgs &a, hipStream_t s) {
    combine_k<<<dim3(a.M, (a.H + 255) / 256), 256, 0, s>>>(a);
}

// --------------------------------------------------------------- fills

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename T>
__global__ void __launch_bounds__(256) fill_normal_k(T *dst, size_t n, uint64_t seed, float sd) {
    size_t pairs = (n + 1) / 2;
    for (size_t p = blockIdx.x * (size_t)blockDim.x + threadIdx.x; p < pairs;
         p += (size_t)gridDim.x * blockDim.x) {
        uint64_t base = seed + 0x9E3779B97F4A7C15ull * (2 * p);
        uint64_t x1 = mix64(base + 0x9E3779B97F4A7C15ull);
        uint64_t x2 = mix64(base + 2 * 0x9E3779B97F4A7C15ull);
        float u1 = ((float)(x1 >> 40) + 1.0f) * (1.0f / 16777216.0f);
        float u2 = (float)(x2 >> 40) * (1.0f / 16777216.0f);
        float r = sqrtf(-2.0f * logf(u1));
        float sv, cv;
        sincosf(6.2831853071795864f * u2, &sv, &cv);
        st(dst, 2 * p, r * cv * sd);
        if (2 * p + 1 < n) st(dst, 2 * p + 1, r * sv * sd);
    }
}

void launch_fill_normal(Dt dt, void *dst, size_t n, uint64_t seed, float sd, hipStream_t s) {
    if (!n) return;
    size_t pairs = (n + 1) / 2;
    int blocks = (int)std::min<size_t>((pairs + 255) / 256, 65536);
    if (dt == DT_BF16) fill_normal_k<uint16_t><<<blocks, 256, 0, s>>>((uint16_t *)dst, n, seed, sd);
    else fill_normal_k<float><<<blocks, 256, 0, s>>>((float *)dst, n, seed, sd);
}

__global__ void fill_const_k(float *dst, size_t n, float v) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = v;
}

void launch_fill_const(float *dst, size_t n, float v, hipStream_t s) {
    if (!n) return;
    int blocks = (int)std::min<size_t>((n + 255) / 256, 65536);
    fill_const_k<<<blocks, 256, 0, s>>>(dst, n, v);
}

__global__ void fill_bits_k(uint16_t *dst, size_t n, uint16_t b) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = b;
}

void launch_fill_bits(uint16_t *dst, size_t n, uint16_t bits, hipStream_t s) {
    if (!n) return;
    int blocks = (int)std::min<size_t>((n + 255) / 256, 65536);
    fill_bits_k<<<blocks, 256, 0, s>>>(dst, n, bits);
}

// ------------------------------------------------- packed weight formats

// out[i] = q_i * scale[i / 32]: the weight value the packed formats define
// (weight_format.rs:390-397).
template <bool Q4>
__global__ void __launch_bounds__(256) dequant_k(const void *values, const float *scales,
                                                 size_t n, float *out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        int q;
        if (Q4) {
            const uint8_t b = ((const uint8_t *)values)[i >> 1];
            q = ((int)((unsigned)b << (28 - 4 * (int)(i & 1)))) >> 28;
        } else {
            q = ((const int8_t *)values)[i];
        }
        out[i] = (float)q * scales[i >> 5];
    }
}

void launch_dequant(Dt wt, const void *values, const float *scales, size_t n, float *out,
                    hipStream_t s) {
    if (!n) return;
    int blocks = (int)std::min<size_t>((n + 255) / 256, 65536);
    if (wt == DT_Q4) dequant_k<true><<<blocks, 256, 0, s>>>(values, scales, n, out);
    else dequant_k<false><<<blocks, 256, 0, s>>>(values, scales, n, out);
}

// A packed projection [N, K] as the two bf16 planes of a doubled-K matrix
// for the matrix cores: row n = [hi(w) | lo(w)] with w = q * scale (f32,
// the format's definition), hi = bf16(w), lo = bf16(w - hi), so hi + lo
// holds w to ~2^-17 relative. Multiplied against activation rows
// [a_hi | a_hi] (hi plane) and [a_lo | 0] (lo plane), the bf16 GEMM sums
// a_hi w_hi + a_lo w_hi + a_hi w_lo over the original K.
// Eight consecutive weights of a row per thread (K % 8 == 0): one 8- or
// 4-byte load of the values and one scale, two 16-byte stores (hi and lo
// halves of the row); the same per-element arithmetic as one weight per
// thread, which moved two bytes per store and ran at ~2 TB/s.
template <bool Q4>
__global__ void __launch_bounds__(256) dequant_split_k(const void *values, const float *scales,
                                                       size_t N, size_t K, uint16_t *out) {
    const size_t chunks = N * K / 8;
    for (size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x; c < chunks;
         c += (size_t)gridDim.x * blockDim.x) {
        const size_t i = c * 8;
        int q[8];
        if (Q4) {
            const uint32_t b = *(const uint32_t *)((const uint8_t *)values + (i >> 1));
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = ((int)(b << (28 - 4 * j))) >> 28;
        } else {
            const uint2 b = *(const uint2 *)((const int8_t *)values + i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                q[j] = (int)(int8_t)(b.x >> (8 * j));
                q[4 + j] = (int)(int8_t)(b.y >> (8 * j));
            }
        }
        const float sc = scales[i >> 5];
        uint32_t h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float w0 = (float)q[2 * j] * sc, w1 = (float)q[2 * j + 1] * sc;
            const uint16_t h0 = f2bf(w0), h1 = f2bf(w1);
            h[j] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            l[j] = (uint32_t)f2bf(w0 - bf2f(h0)) | ((uint32_t)f2bf(w1 - bf2f(h1)) << 16);
        }
        const size_t n = i / K, k = i - n * K;
        *(uint4 *)(out + n * 2 * K + k) = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4 *)(out + n * 2 * K + K + k) = make_uint4(l[0], l[1], l[2], l[3]);
    }
}

void launch_dequant_split(Dt wt, const void *values, const float *scales, size_t N, size_t K,
                          uint16_t *out, hipStream_t s) {
    if (!N || !K) return;
    if (K % 8) fail(ESP_BACKEND, "dequant_split: K must be a multiple of 8");
    int blocks = (int)std::min<size_t>((N * K / 8 + 255) / 256, 65536);
    if (wt == DT_Q4) dequant_split_k<true><<<blocks, 256, 0, s>>>(values, scales, N, K, out);
    else dequant_split_k<false><<<blocks, 256, 0, s>>>(values, scales, N, K, out);
}

// Split activation planes [M, K] widened for the doubled-K product above:
// hi2 = [hi | hi], lo2 = [lo | 0], both [M, 2K]; four bf16 per lane.
__global__ void __launch_bounds__(256) widen_split_k(const uint16_t *hi, const uint16_t *lo,
                                                     size_t M, size_t K, uint16_t *hi2,
                                                     uint16_t *lo2) {
    const size_t q = K / 4, n_all = M * q;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n_all;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t m = i / q, c = (i - m * q) * 4;
        const uint2 h = *(const uint2 *)(hi + m * K + c);
        const uint2 l = *(const uint2 *)(lo + m * K + c);
        *(uint2 *)(hi2 + m * 2 * K + c) = h;
        *(uint2 *)(hi2 + m * 2 * K + K + c) = h;
        *(uint2 *)(lo2 + m * 2 * K + c) = l;
        *(uint2 *)(lo2 + m * 2 * K + K + c) = make_uint2(0u, 0u);
    }
}

void launch_widen_split(const uint16_t *hi, const uint16_t *lo, size_t M, size_t K, uint16_t *hi2,
                        uint16_t *lo2, hipStream_t s) {
    if (!M || !K) return;
    if (K % 4) fail(ESP_BACKEND, "widen_split: K must be a multiple of 4");
    int blocks = (int)std::min<size_t>((M * K / 4 + 255) / 256, 65536);
    widen_split_k<<<blocks, 256, 0, s>>>(hi, lo, M, K, hi2, lo2);
}

// weight_format.rs:150-183, one thread per 32-input block: scale = peak /
// max (1 for an all-zero block, at least the smallest normal f32), q =
// round-half-away(v / scale) clamped to [-max, max]; q4 packs two per byte,
// the even input in the low nibble.
template <bool Q4>
__global__ void __launch_bounds__(256) quantize_k(const float *src, size_t blocks, void *values,
                                                  float *scales) {
    const float qmax = Q4 ? 7.f : 127.f;
    for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < blocks;
         b += (size_t)gridDim.x * blockDim.x) {
        const float *v = src + b * 32;
        float peak = 0.f;
        for (int i = 0; i < 32; ++i) peak = fmaxf(peak, fabsf(v[i]));
        const float scale = peak == 0.f ? 1.f : fmaxf(peak / qmax, 1.17549435e-38f);
        scales[b] = scale;
        if (Q4) {
            uint8_t *o = (uint8_t *)values + b * 16;
            for (int i = 0; i < 32; i += 2) {
                const int q0 = (int)fminf(fmaxf(roundf(v[i] / scale), -qmax), qmax);
                const int q1 = (int)fminf(fmaxf(roundf(v[i + 1] / scale), -qmax), qmax);
                o[i / 2] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
            }
        } else {
            int8_t *o = (int8_t *)values + b * 32;
            for (int i = 0; i < 32; ++i)
                o[i] = (int8_t)(int)fminf(fmaxf(roundf(v[i] / scale), -qmax), qmax);
        }
    }
}

void launch_quantize(Dt wt, const float *src, size_t rows, size_t cols, void *values,
                     float *scales, hipStream_t s) {
    const size_t blocks = rows * cols / 32;
    if (!blocks) return;
    int grid = (int)std::min<size_t>((blocks + 255) / 256, 65536);
    if (wt == DT_Q4) quantize_k<true><<<grid, 256, 0, s>>>(src, blocks, values, scales);
    else quantize_k<false><<<grid, 256, 0, s>>>(src, blocks, values, scales);
}

}  // namespace esp
