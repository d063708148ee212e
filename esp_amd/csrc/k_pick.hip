// Token choice over device-resident logits rows: the grammar bitmask
// (constraint.rs:277-297), greedy argmax with the lowest id winning ties
// (generate.rs:70-79, provider.rs:808-815), and the seeded temperature /
// nucleus sampler (sample.rs:83-121) reproduced step for step: f32 weights
// exp((l - max) * (1/T)), a descending sort with ties by ascending id,
// sequential f32 prefix sums for the nucleus cut and the kept mass, one
// splitmix64 draw, and the subtract-walk.
#include <algorithm>
#include <cstdlib>

#include "common.hpp"
#include "dev.hpp"

namespace esp {

constexpr int PICK_THREADS = 1024;
constexpr int PICK_LDS_CAP = 16384;  // candidates sorted in LDS (8 B each)
// Rows listing more ids than this (every id not masked to -inf) take the
// bucketed path; up to it the weights go straight into the LDS sort and one
// lane runs the sequential sums. The bucketed path's parallel sums win
// beyond a few thousand ids: measured on MI355X at the C5 step (64 rows of
// ~6.4k allowed ids out of 128256), the in-block path for every row took
// pick_k to 470 us per launch (3.19 ms per step) against 2.98 ms per step
// with this bound.
constexpr int PICK_DIRECT_MAX = 2048;

struct Cand {
    float w;
    int32_t id;
};

// Descending weight, ascending id; sentinels (w < 0) last.
__device__ __forceinline__ bool before(Cand a, Cand b) {
    if (a.w != b.w) return a.w > b.w;
    return a.id < b.id;
}

// Sampled rows with more candidates than the LDS sort holds are finished
// by three more kernels. pick_k buckets the candidates by the top bits of
// their f32 weight (bits 30..17: exponent and six mantissa bits; larger
// bucket = larger weight) and writes them bucket by bucket in descending
// bucket order; pick_bsort_k sorts each bucket in LDS, one wave per bucket
// up to PB_WAVE_CAP candidates and one block per larger bucket
// (pick_bsort_big_k sorts, one at a time, the rare buckets larger than
// LDS); pick_chain_k then runs the sequential f32 sums and the draw over
// the sorted list.
constexpr int PB_BITS = 14;
constexpr int PB_BINS = 1 << PB_BITS;
constexpr int PB_WAVE_CAP = 1024;  // buckets up to this size are sorted by one wave
__device__ __forceinline__ int wbucket(float w) {
    return (int)((__float_as_uint(w) >> (31 - PB_BITS)) & (PB_BINS - 1));
}

struct PickRow {
    int C;         // candidates (positive weights)
    int zmax;      // largest zero-weight id, -1 if none
    int deferred;  // 1: finished by pick_chain_k
    int flags;
};

// Per-call scratch: [n][cap] sorted candidates | [n][cap] weights (first
// pick_k's list of the ids it weighs, then the sorted weights) |
// big-bucket temp [cap] | [n][PB_BINS] bucket start | [n][PB_BINS] bucket
// count | [n] PickRow | small, medium and big bucket lists [n * PB_BINS]
// each | counters [4] (small, big, medium).
struct PickScratch {
    Cand *cand, *temp;
    float *wts;
    int *bstart, *bcount;
    PickRow *info;
    uint32_t *work, *med, *big, *counts;
    int cap;
};

__host__ __device__ inline int pick_cap(int V) {
    int c = 1;
    while (c < V + 1) c <<= 1;
    return c;
}

__host__ __device__ inline PickScratch pick_layout(void *base, int n, int V) {
    PickScratch p;
    p.cap = pick_cap(V);
    char *b = (char *)base;
    p.cand = (Cand *)b;
    b += (size_t)n * p.cap * sizeof(Cand);
    p.wts = (float *)b;
    b += (size_t)n * p.cap * sizeof(float);
    p.temp = (Cand *)b;
    b += (size_t)p.cap * sizeof(Cand);
    p.bstart = (int *)b;
    b += (size_t)n * PB_BINS * 4;
    p.bcount = (int *)b;
    b += (size_t)n * PB_BINS * 4;
    p.info = (PickRow *)b;
    b += (size_t)n * sizeof(PickRow);
    p.work = (uint32_t *)b;
    b += (size_t)n * PB_BINS * 4;
    p.med = (uint32_t *)b;
    b += (size_t)n * PB_BINS * 4;
    p.big = (uint32_t *)b;
    b += (size_t)n * PB_BINS * 4;
    p.counts = (uint32_t *)b;
    return p;
}

// Exclusive prefix sum over the block (blockDim.x a multiple of 64, at
// most 32 waves); *total receives the block sum. tmp: LDS, >= 33 ints.
__device__ int block_excl_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) tmp[wv] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int w = 0; w < nw; ++w) {
            const int t = tmp[w];
            tmp[w] = run;
            run += t;
        }
        tmp[32] = run;
    }
    __syncthreads();
    const int r = tmp[wv] + x - v;
    *total = tmp[32];
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint64_t splitmix_next(uint64_t &s) {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Bitonic sort of n (power of two) candidates; buf is LDS or global memory
// owned by this block. Each thread takes the lower elements i of its pairs
// (i, i + j) directly, so every compare-exchange is a branch-free load /
// select / store.
__device__ void bitonic(Cand *buf, int n) {
    const int half = n >> 1;
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int pi = threadIdx.x; pi < half; pi += blockDim.x) {
                const int i = ((pi & ~(j - 1)) << 1) | (pi & (j - 1)), p = i + j;
                const Cand x = buf[i], y = buf[p];
                const bool up = (i & k) == 0;  // this run sorted by `before`
                const bool swap = up ? before(y, x) : before(x, y);
                buf[i] = swap ? y : x;
                buf[p] = swap ? x : y;
            }
            __syncthreads();
        }
    }
}

// v[q] = row[i4 + q] for ids below V (row 16-byte aligned when V % 4 == 0).
__device__ __forceinline__ void load4(const float *row, int V, int i4, float (&v)[4]) {
    typedef float f4_t __attribute__((ext_vector_type(4)));
    if ((V & 3) == 0 && i4 + 3 < V) {
        const f4_t x = *(const f4_t *)(row + i4);
        v[0] = x.x;
        v[1] = x.y;
        v[2] = x.z;
        v[3] = x.w;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = i4 + q < V ? row[i4 + q] : 0.f;
    }
}

__global__ void __launch_bounds__(PICK_THREADS) pick_k(PickArgs a) {
    extern __shared__ Cand lds[];
    __shared__ float red_f[32];
    __shared__ int red_i[32];
    __shared__ int s_count, s_zmax, s_bad, s_elig, s_wbase, s_mbase, s_ncand;
    __shared__ int s_scan[33];
    const int row = blockIdx.x;
    const int V = a.V;
    const float *L = a.logits + (size_t)row * V;
    const uint32_t *bits = a.allowed ? a.allowed + (size_t)row * ((V + 31) / 32) : nullptr;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const esp_sampler *smp = a.samplers ? a.samplers + row : nullptr;
    const bool sampled = smp && smp->temperature > 0.f;
    // sampled rows list the ids whose weight pass 2 computes (every id not
    // masked to -inf), in the row's weight scratch; the later passes walk
    // that list instead of the vocabulary
    int32_t *list = sampled ? (int32_t *)(pick_layout(a.scratch, a.n, V).wts +
                                          (size_t)row * pick_cap(V))
                            : nullptr;
    if (tid == 0) {
        s_count = 0;
        s_zmax = -1;
        s_bad = 0;
        s_elig = 0;
        s_ncand = 0;
    }
    __syncthreads();
    // pass 1: mask, finiteness, greedy best and max. Each thread takes four
    // consecutive ids at a time (one 16-byte load when the row is aligned),
    // four groups in flight; ids rise along a thread's walk.
    float best = -INFINITY;
    int best_id = 0x7fffffff;
    int bad = 0, elig = 0, zmax = -1;
    const int gs = 4 * (int)blockDim.x;
    // the loop is wave-uniform (lanes past V take part with no ids), so the
    // candidate list grows by one LDS atomic per wave and iteration
    for (int j0 = 0; j0 + wv * 256 < V; j0 += 4 * gs) {
        const int i4 = j0 + tid * 4;
        float v4[4][4];
        uint32_t bw[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            load4(L, V, i4 + g * gs, v4[g]);
            bw[g] = bits && i4 + g * gs < V ? bits[(i4 + g * gs) >> 5] : 0u;
        }
        uint32_t cm = 0;  // this lane's listed ids, bit 4 g + q
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = i4 + g * gs + q;
                const bool in = i < V;
                float v = v4[g][q];
                const bool fin = isfinite(v);
                const bool allowed = bits ? ((bw[g] >> (i & 31)) & 1u) : true;
                // pass 2's value: masked or non-finite ids of a masked row are -inf
                const float v2 = bits && (!allowed || !fin) ? -INFINITY : v;
                if (in) {
                    bad |= !fin;
                    if (bits ? (!allowed || !fin) : isnan(v)) v = -INFINITY;
                    elig += (allowed && fin);
                    if (v > best || (v == best && i < best_id)) {
                        best = v;
                        best_id = i;
                    }
                }
                if (list) {
                    // weight 0 without an exp: the largest such id is the
                    // fall-through of an uncut list; every other id is listed
                    const bool cand = in && v2 != -INFINITY;
                    if (in && !cand) zmax = i;
                    cm |= (uint32_t)cand << (4 * g + q);
                }
            }
        if (list) {
            uint64_t bm[16];
            int tot = 0;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                bm[k] = __ballot((cm >> k) & 1u);
                tot += __popcll(bm[k]);
            }
            if (tot) {  // wave-uniform
                int base = 0;
                if (lane == 0) base = atomicAdd(&s_ncand, tot);
                base = __shfl(base, 0);
                const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    if ((cm >> k) & 1u) list[base + __popcll(bm[k] & below)] = i4 + (k >> 2) * gs + (k & 3);
                    base += __popcll(bm[k]);
                }
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ob = __shfl_xor(best, o, 64);
        int oi = __shfl_xor(best_id, o, 64);
        if (ob > best || (ob == best && oi < best_id)) {
            best = ob;
            best_id = oi;
        }
    }
    if (lane == 0) {
        red_f[wv] = best;
        red_i[wv] = best_id;
    }
    if (bad) atomicOr(&s_bad, 1);
    if (elig) atomicAdd(&s_elig, elig);
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
            if (red_f[w] > red_f[0] || (red_f[w] == red_f[0] && red_i[w] < red_i[0])) {
                red_f[0] = red_f[w];
                red_i[0] = red_i[w];
            }
    }
    __syncthreads();
    const float mx = red_f[0];
    uint8_t flags = (s_bad ? ESP_PICK_NONFINITE : 0) |
                    ((bits && s_elig == 0) ? ESP_PICK_NO_ELIGIBLE : 0);
    if (!sampled || (bits && s_elig == 0)) {
        if (tid == 0) {
            a.ids_out[row] = (bits && s_elig == 0) ? 0u : (uint32_t)(red_i[0] == 0x7fffffff ? 0 : red_i[0]);
            a.flags_out[row] = flags;
            if (a.state_out) a.state_out[row] = smp ? smp->state : 0;
        }
        return;
    }
    // pass 2 over the listed ids: their weights, the candidate count
    // (weights > 0) and the largest zero-weight id (pass 1's, or an exp that
    // underflows). A row listing at most direct_max ids puts its candidates
    // straight into the LDS sort (one exp per id); a longer row builds the
    // weight-bucket histogram of its candidates (the exp is recomputed, bit
    // for bit, where the scatter needs a weight again).
    const float inv_t = 1.0f / smp->temperature;
    const PickScratch ps = pick_layout(a.scratch, a.n, V);
    const int ncand = s_ncand;
    const int dmax = a.direct_max > 0 ? min(a.direct_max, PICK_LDS_CAP) : PICK_DIRECT_MAX;
    const bool direct = ncand <= dmax;  // block-uniform
    // every listed id k = tid + j * blockDim.x, eight at a time: the list
    // entries, then their logits, are loaded before any is used
    auto for_cands = [&](auto &&fn) {
        constexpr int B8 = 8;
        for (int k0 = tid; k0 < ncand; k0 += B8 * (int)blockDim.x) {
            int id[B8];
            float lg[B8];
#pragma unroll
            for (int j = 0; j < B8; ++j) {
                const int k = k0 + j * (int)blockDim.x;
                id[j] = k < ncand ? list[k] : -1;
            }
#pragma unroll
            for (int j = 0; j < B8; ++j) lg[j] = id[j] >= 0 ? L[id[j]] : 0.f;
#pragma unroll
            for (int j = 0; j < B8; ++j)
                if (id[j] >= 0) fn(id[j], (float)exp((double)((lg[j] - mx) * inv_t)));
        }
    };
    int *hist = (int *)lds, *cur = hist + PB_BINS;
    Cand *buf = lds;
    int cnt = 0;
    if (direct) {
        for_cands([&](int i, float w) {
            if (w > 0.f) buf[atomicAdd(&s_count, 1)] = Cand{w, i};
            else if (w == 0.f) zmax = max(zmax, i);
        });
    } else {
        for (int d = tid; d < PB_BINS; d += blockDim.x) hist[d] = 0;
        __syncthreads();
        for_cands([&](int i, float w) {
            if (w > 0.f) {
                ++cnt;
                atomicAdd(&hist[wbucket(w)], 1);
            } else if (w == 0.f) {
                zmax = max(zmax, i);
            }
        });
        cnt = (int)wave_sum((float)cnt);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) zmax = max(zmax, __shfl_xor(zmax, o, 64));
    if (lane == 0) {
        if (!direct) atomicAdd(&s_count, cnt);
        if (zmax >= 0) atomicMax(&s_zmax, zmax);
    }
    __syncthreads();
    const int C = s_count;
    if (C == 0) {  // every weight NaN: nothing can be drawn
        if (tid == 0) {
            a.ids_out[row] = 0;
            a.flags_out[row] = flags | ESP_PICK_NONFINITE;
            if (a.state_out) a.state_out[row] = smp->state;
        }
        return;
    }
    if (!direct) {
        // bucketed path: descending-bucket offsets, work lists, scatter.
        // Wave v owns the descending positions [1024 v, 1024 v + 1024),
        // taken 64 at a time by its lanes (consecutive LDS words).
        constexpr int SPAN = PB_BINS / (PICK_THREADS / 64);
        static_assert(SPAN * (PICK_THREADS / 64) == PB_BINS, "bucket spans");
        int hs = 0, fs = 0, ms = 0;
        for (int r = lane; r < SPAN; r += 64) {
            const int h = hist[PB_BINS - 1 - (wv * SPAN + r)];
            hs += h;
            fs += h > 0 && h <= PB_WAVE_CAP;
            ms += h > PB_WAVE_CAP && h <= PICK_LDS_CAP;
        }
        hs = (int)wave_sum((float)hs);  // < 2^24: exact in f32
        fs = (int)wave_sum((float)fs);
        ms = (int)wave_sum((float)ms);
        if (lane == 0) {
            s_scan[wv] = hs;
            s_scan[16 + wv] = fs;
        }
        if (lane == 0) red_i[wv] = ms;
        __syncthreads();
        if (tid == 0) {
            int ro = 0, rs = 0, rm = 0;
            for (int v = 0; v < PICK_THREADS / 64; ++v) {
                const int a0 = s_scan[v], a1 = s_scan[16 + v], a2 = red_i[v];
                s_scan[v] = ro;
                s_scan[16 + v] = rs;
                red_i[v] = rm;
                ro += a0;
                rs += a1;
                rm += a2;
            }
            s_wbase = rs ? (int)atomicAdd(&ps.counts[0], (uint32_t)rs) : 0;
            s_mbase = rm ? (int)atomicAdd(&ps.counts[2], (uint32_t)rm) : 0;
        }
        __syncthreads();
        int o = s_scan[wv], si = s_wbase + s_scan[16 + wv], mi = s_mbase + red_i[wv];
        int *gst = ps.bstart + (size_t)row * PB_BINS, *gct = ps.bcount + (size_t)row * PB_BINS;
        const uint32_t rb = (uint32_t)row << PB_BITS;
        for (int r0 = 0; r0 < SPAN; r0 += 64) {
            const int d = PB_BINS - 1 - (wv * SPAN + r0 + lane);
            const int h = hist[d];
            const int fsm = h > 0 && h <= PB_WAVE_CAP, fmd = h > PB_WAVE_CAP && h <= PICK_LDS_CAP;
            // wave-inclusive scans of h and the two flags
            int ph = h, pf = fsm, pm = fmd;
#pragma unroll
            for (int dd = 1; dd < 64; dd <<= 1) {
                const int y0 = __shfl_up(ph, dd), y1 = __shfl_up(pf, dd), y2 = __shfl_up(pm, dd);
                if (lane >= dd) {
                    ph += y0;
                    pf += y1;
                    pm += y2;
                }
            }
            const int start_d = o + ph - h;
            gst[d] = start_d;
            gct[d] = h;
            cur[d] = start_d;
            if (fsm) ps.work[si + pf - 1] = rb | (uint32_t)d;
            else if (fmd) ps.med[mi + pm - 1] = rb | (uint32_t)d;
            else if (h > PICK_LDS_CAP) ps.big[atomicAdd(&ps.counts[1], 1u)] = rb | (uint32_t)d;
            o += __shfl(ph, 63);
            si += __shfl(pf, 63);
            mi += __shfl(pm, 63);
        }
        __syncthreads();
        Cand *dst = ps.cand + (size_t)row * ps.cap;
        for_cands([&](int i, float w) {
            if (w > 0.f) dst[atomicAdd(&cur[wbucket(w)], 1)] = Cand{w, i};
        });
        if (tid == 0) ps.info[row] = PickRow{C, s_zmax, 1, flags};
        return;
    }
    int n2 = 1;
    while (n2 < C) n2 <<= 1;
    for (int i = C + tid; i < n2; i += blockDim.x) buf[i] = Cand{-1.f, 0x7fffffff};
    __syncthreads();
    bitonic(buf, n2);
    // LDS-resident lists go to struct-of-arrays in place (weights, then ids)
    // so the serial pass below reads four weights per load; every element is
    // read into registers before any is written back
    const bool soa = true;  // n2 <= PICK_LDS_CAP here
    float *sw = (float *)buf;
    int32_t *sid = (int32_t *)buf + n2;
    if (soa) {
        constexpr int PER = PICK_LDS_CAP / PICK_THREADS;
        Cand cr[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = q * (int)blockDim.x + tid;
            cr[q] = i < n2 ? buf[i] : Cand{0.f, 0};
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = q * (int)blockDim.x + tid;
            if (i < n2) {
                sw[i] = cr[q].w;
                sid[i] = cr[q].id;
            }
        }
        __syncthreads();
    }
    if (tid != 0) return;
    // sequential pass (sample.rs:96-120) by one lane: the f32 sums must keep
    // the reference's left-to-right order, so they stay serial; weights are
    // read eight at a time and past-the-end slots add -0.0 (an exact no-op),
    // so the adds carry no branches. The kept mass equals the nucleus prefix
    // sum (same terms, same order), so it is not summed a third time.
    constexpr int RB8 = 8;
    typedef float f4_t __attribute__((ext_vector_type(4)));
    auto w8_at = [&](int i0, float (&w8)[8], int lim, float pad) {  // i0 % 8 == 0
        float v[8];
        if (soa && n2 >= 8) {
            const int b = min(i0, n2 - 8);
            const f4_t lo = *(const f4_t *)(sw + b), hi = *(const f4_t *)(sw + b + 4);
            v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
            v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = soa ? sw[min(i0 + q, n2 - 1)] : buf[min(i0 + q, n2 - 1)].w;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) w8[q] = i0 + q < lim ? v[q] : pad;
    };
    auto id_at = [&](int i) { return soa ? sid[i] : buf[i].id; };
    // Monotone running values (positive weights) let whole batches of eight
    // be added plainly: only the batch where the nucleus mass crosses its
    // target, or where the draw crosses zero, is replayed term by term from
    // the batch's starting value (identical arithmetic, identical result).
    int keep = C;
    const float top_p = smp->top_p;
    float total = -0.0f;
    if (top_p >= 0.f) {
        float all = -0.0f;
        float nx[RB8];  // next batch in flight while this one is added
        w8_at(0, nx, C, -0.0f);
        for (int i0 = 0; i0 < C; i0 += RB8) {
            float w8[RB8];
#pragma unroll
            for (int q = 0; q < RB8; ++q) w8[q] = nx[q];
            w8_at(i0 + RB8, nx, C, -0.0f);
#pragma unroll
            for (int q = 0; q < RB8; ++q) all += w8[q];
        }
        const float p = top_p > 1.f ? 1.f : top_p;
        const float target = all * p;
        float mass = 0.0f;
        keep = 0;
        w8_at(0, nx, C, -0.0f);
        for (int i0 = 0; i0 < C; i0 += RB8) {
            float w8[RB8];
#pragma unroll
            for (int q = 0; q < RB8; ++q) w8[q] = nx[q];
            w8_at(i0 + RB8, nx, C, -0.0f);
            float m2 = mass;
#pragma unroll
            for (int q = 0; q < RB8; ++q) m2 += w8[q];
            if (m2 < target && i0 + RB8 < C) {  // no crossing inside this batch
                mass = m2;
                keep = i0 + RB8;
                continue;
            }
            for (int q = 0; q < RB8 && i0 + q < C; ++q) {
                mass += w8[q];
                keep = i0 + q + 1;
                if (mass >= target) break;
            }
            break;
        }
        if (keep < 1) keep = 1;
        total = -0.0f + mass;
    } else {
        for (int i0 = 0; i0 < keep; i0 += RB8) {
            float w8[RB8];
            w8_at(i0, w8, keep, -0.0f);
#pragma unroll
            for (int q = 0; q < RB8; ++q) total += w8[q];
        }
    }
    uint64_t state = smp->state;
    uint64_t x = splitmix_next(state);
    float u = (float)((double)(x >> 11) / 9007199254740992.0) * total;
    // fall-through value: the last element of the (truncated) sorted list
    int32_t out = (top_p < 0.f && s_zmax >= 0) ? s_zmax : (keep > 0 ? id_at(keep - 1) : 0);
    float nw[RB8];
    w8_at(0, nw, keep, 0.f);
    for (int i0 = 0; i0 < keep; i0 += RB8) {
        float w8[RB8];
#pragma unroll
        for (int q = 0; q < RB8; ++q) w8[q] = nw[q];
        w8_at(i0 + RB8, nw, keep, 0.f);
        float u2 = u;
#pragma unroll
        for (int q = 0; q < RB8; ++q) u2 -= w8[q];
        if (u2 > 0.0f && i0 + RB8 < keep) {  // the draw stays positive past this batch
            u = u2;
            continue;
        }
        int hit = -1;
        for (int q = 0; q < RB8 && i0 + q < keep; ++q) {
            u -= w8[q];
            if (u <= 0.0f) {
                hit = i0 + q;
                break;
            }
        }
        if (hit >= 0) out = id_at(hit);
        break;
    }
    a.ids_out[row] = (uint32_t)out;
    a.flags_out[row] = flags;
    if (a.state_out) a.state_out[row] = state;
}

// Clears the counters and row records of the bucketed path.
__global__ void pick_reset_k(PickScratch ps, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 4) ps.counts[i] = 0;
    if (i < n) ps.info[i] = PickRow{0, -1, 0, 0};
}

// Sorts the listed buckets in LDS by descending weight, ascending id:
// first the small ones, one wave per bucket with wave-level barriers only,
// then the medium ones (up to PICK_LDS_CAP), one block per bucket.
__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ void __launch_bounds__(PICK_THREADS) pick_bsort_k(PickScratch ps) {
    extern __shared__ Cand lds[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nwaves = PICK_THREADS / 64;
    Cand *wl = lds + wv * PB_WAVE_CAP;
    const uint32_t nsmall = ps.counts[0];
    for (uint32_t k = blockIdx.x * nwaves + wv; k < nsmall; k += gridDim.x * nwaves) {
        const uint32_t item = ps.work[k];
        const int row = (int)(item >> PB_BITS), d = (int)(item & (PB_BINS - 1));
        const int n = ps.bcount[(size_t)row * PB_BINS + d];
        Cand *g = ps.cand + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        int n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (int i = lane; i < n2; i += 64) wl[i] = i < n ? g[i] : Cand{-1.f, 0x7fffffff};
        wave_sync_lds();
        const int half = n2 >> 1;
        for (int kk = 2; kk <= n2; kk <<= 1) {
            for (int j = kk >> 1; j > 0; j >>= 1) {
                for (int pi = lane; pi < half; pi += 64) {
                    const int i = ((pi & ~(j - 1)) << 1) | (pi & (j - 1)), p = i + j;
                    const Cand x = wl[i], y = wl[p];
                    const bool up = (i & kk) == 0;
                    const bool swap = up ? before(y, x) : before(x, y);
                    wl[i] = swap ? y : x;
                    wl[p] = swap ? x : y;
                }
                wave_sync_lds();
            }
        }
        float *gw = ps.wts + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        for (int i = lane; i < n; i += 64) {
            g[i] = wl[i];
            gw[i] = wl[i].w;
        }
        wave_sync_lds();
    }
    __syncthreads();
    const uint32_t nmed = ps.counts[2];
    for (uint32_t k = blockIdx.x; k < nmed; k += gridDim.x) {
        const uint32_t item = ps.med[k];
        const int row = (int)(item >> PB_BITS), d = (int)(item & (PB_BINS - 1));
        const int n = ps.bcount[(size_t)row * PB_BINS + d];
        Cand *g = ps.cand + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        int n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (int i = threadIdx.x; i < n2; i += blockDim.x)
            lds[i] = i < n ? g[i] : Cand{-1.f, 0x7fffffff};
        __syncthreads();
        bitonic(lds, n2);
        float *gw = ps.wts + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            g[i] = lds[i];
            gw[i] = lds[i].w;
        }
        __syncthreads();
    }
}

// Buckets larger than LDS (many equal weights): sorted one after another
// through the global temp area by a single block.
__global__ void __launch_bounds__(PICK_THREADS) pick_bsort_big_k(PickScratch ps) {
    const uint32_t total = ps.counts[1];
    for (uint32_t k = 0; k < total; ++k) {
        const uint32_t item = ps.big[k];
        const int row = (int)(item >> PB_BITS), d = (int)(item & (PB_BINS - 1));
        const int n = ps.bcount[(size_t)row * PB_BINS + d];
        Cand *g = ps.cand + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        int n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (int i = threadIdx.x; i < n2; i += blockDim.x)
            ps.temp[i] = i < n ? g[i] : Cand{-1.f, 0x7fffffff};
        __syncthreads();
        bitonic(ps.temp, n2);
        float *gw = ps.wts + (size_t)row * ps.cap + ps.bstart[(size_t)row * PB_BINS + d];
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            g[i] = ps.temp[i];
            gw[i] = ps.temp[i].w;
        }
        __syncthreads();
    }
}

// The sequential tail of sample.rs:96-120 over the sorted weights of a row,
// computed exactly but in parallel. While a running f32 value x stays in
// one binade [2^k, 2^(k+1)) its grid is fixed (ulp 2^(k-23)), and
// RN(x + w) equals x plus w rounded to that grid. So a run of adds (or, for
// the draw walk, subtracts) is an integer prefix sum on the grid; the
// elements where the run must stop are the "events": a term whose grid
// rounding is an exact tie (then the rounding depends on the running
// value's parity), a result that would leave the binade (upward for sums;
// downward, judged on the term rounded up, for the walk), and, for the
// nucleus, reaching the cut target. Each event is one ordinary f32 add by
// one thread; everything between events is a block scan.
constexpr int GC_IPT = 16;                    // items per thread, max window 16384
constexpr int GC_CK = 256;                    // checkpoints kept by the total pass
constexpr int GC_SERIAL = 256;                // stretch stepped serially near events
constexpr int GC_LDS_W = 16384;               // sorted weights staged in LDS (64 KB)
constexpr uint64_t GC_HUGE = 1ull << 62;

// x > 0: x = K * 2^ue with K on the binade's integer grid [low, lim).
__device__ __forceinline__ void grid_of(float x, int &ue, uint64_t &K, uint64_t &lim,
                                        uint64_t &low) {
    const uint32_t b = __float_as_uint(x);
    const int ex = (int)((b >> 23) & 0xff);
    K = ex ? (uint64_t)((b & 0x7fffff) | 0x800000) : (uint64_t)(b & 0x7fffff);
    ue = ex ? ex - 150 : -149;
    lim = ex ? (1ull << 24) : (1ull << 23);
    low = ex ? (1ull << 23) : 0;
}

// The float with x's exponent field and grid value K (K within x's binade).
__device__ __forceinline__ float from_grid(float x, uint64_t K) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t ex = (b >> 23) & 0xff;
    return ex ? __uint_as_float(ex << 23 | (uint32_t)(K & 0x7fffff)) : __uint_as_float((uint32_t)K);
}

// w / 2^ue rounded to nearest (q, tie = exactly half) and rounded up (qc).
__device__ __forceinline__ uint64_t grid_units(uint32_t wb, int ue, bool &tie, uint64_t &qc) {
    const int ew = (int)((wb >> 23) & 0xff);
    uint64_t m = wb & 0x7fffff;
    int e;
    if (ew == 0) {
        e = -149;
    } else {
        m |= 0x800000;
        e = ew - 150;
    }
    const int sh = ue - e;
    tie = false;
    if (sh <= 0) {
        qc = -sh > 37 ? GC_HUGE : m << (-sh);
        return qc;
    }
    if (sh >= 64) {
        qc = m != 0;
        return 0;
    }
    uint64_t q = m >> sh;
    const uint64_t r = m & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    qc = q + (r != 0);
    if (r > half) ++q;
    else if (r == half) tie = true;
    return q;
}

// ceil(t / 2^ue) for t > 0, saturating.
__device__ __forceinline__ uint64_t grid_ceil(float t, int ue) {
    bool tie;
    uint64_t qc;
    (void)grid_units(__float_as_uint(t), ue, tie, qc);
    return qc;
}

// grid_units in 32 bits for the scan windows, values saturated at GC_SAT:
// a term of 2^24 grid units or more leaves the binade (or passes the walk's
// floor), so it is an event, and before a window's first event every prefix
// stays below 2^24 (no wrap-around reaches the first event).
constexpr uint32_t GC_SAT = 1u << 25;
__device__ __forceinline__ uint32_t grid_units32(uint32_t wb, int ue, bool &tie, uint32_t &qc) {
    const int ew = (int)((wb >> 23) & 0xff);
    uint32_t m = wb & 0x7fffff;
    int e;
    if (ew == 0) {
        e = -149;
    } else {
        m |= 0x800000;
        e = ew - 150;
    }
    const int sh = ue - e;
    tie = false;
    if (sh <= 0) {  // -sh >= 2 only for normal terms (m >= 2^23): >= 2^25 units
        qc = -sh >= 2 ? GC_SAT : m << (-sh);
        return qc;
    }
    if (sh >= 25) {  // m < 2^24 <= half: rounds to 0, never a tie
        qc = m != 0;
        return 0;
    }
    const uint32_t q = m >> sh, r = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    qc = q + (r != 0);
    if (r > half) return q + 1;
    tie = r == half;
    return q;
}

// Exclusive prefix sum of a u32 over the block (wrapping); *total gets the sum.
__device__ uint32_t block_scan_u32(uint32_t v, uint32_t *tmp, uint32_t *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) tmp[wv] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int w = 0; w < nw; ++w) {
            const uint32_t t = tmp[w];
            tmp[w] = run;
            run += t;
        }
        tmp[32] = run;
    }
    __syncthreads();
    const uint32_t r = tmp[wv] + x - v;
    *total = tmp[32];
    __syncthreads();
    return r;
}

template <int GC_THREADS>
__global__ void __launch_bounds__(GC_THREADS) pick_chain_k(PickArgs a, PickScratch ps) {
    __shared__ uint32_t s_tmp[33];
    __shared__ uint64_t s_pref;
    __shared__ float s_x;
    __shared__ int s_i, s_ev, s_stop;
    __shared__ float s_wev;
    __shared__ __attribute__((aligned(16))) float s_w[GC_SERIAL];
    __shared__ int ck_i[GC_CK];
    __shared__ float ck_x[GC_CK];
    __shared__ int s_nck;
    const int row = blockIdx.x;
    const PickRow info = ps.info[row];
    if (!info.deferred) return;
    const Cand *cand = ps.cand + (size_t)row * ps.cap;
    const esp_sampler smp = a.samplers[row];
    const int C = info.C;
    const int tid = threadIdx.x;
    // the sorted weights (descending), staged in LDS when they fit: every
    // round of the sums below reads a window of them
    extern __shared__ __attribute__((aligned(16))) float lw[];
    const float *w = ps.wts + (size_t)row * ps.cap;
    if (C <= GC_LDS_W) {
        for (int j = tid; j < C; j += GC_THREADS) lw[j] = w[j];
        __syncthreads();
        w = lw;
    }

    // Runs x (+= or -=) w[i] for i from i0 up to n, stopping after the
    // element where x >= target (sum with target) or x <= 0 (walk).
    // Leaves the final x in s_x and the stop index (or n) in s_i; s_stop = 1
    // when it stopped early. Records checkpoints when `record`.
    auto run = [&](bool walk, int i0, float x0, int n, bool use_target, float target,
                   bool record) {
        if (tid == 0) {
            s_x = x0;
            s_i = i0;
            s_stop = 0;
            if (record) s_nck = 0;
        }
        __syncthreads();
        for (;;) {
            const int i = s_i;
            const float x = s_x;
            if (s_stop || i >= n) break;
            if (record && tid == 0 && s_nck < GC_CK) {
                ck_i[s_nck] = i;
                ck_x[s_nck] = x;
                ++s_nck;
            }
            uint64_t K = 0, lim = 0, low = 0, T = 0;
            int ue = 0;
            // steps that surely stay on the current grid: the largest
            // remaining term is w[i]
            uint64_t D = 0;
            if (x > 0.f) {
                grid_of(x, ue, K, lim, low);
                if (use_target) T = grid_ceil(target, ue);
                bool t;
                uint64_t qc;
                const uint64_t qi = grid_units(__float_as_uint(w[i]), ue, t, qc);
                if (!walk) {
                    uint64_t room = lim - K - 1;
                    if (use_target) room = min(room, T > K ? T - K - 1 : 0);
                    D = room / (qi ? qi : 1);
                } else {
                    const uint64_t fl = low ? low : 1;
                    D = K > fl ? (K - fl) / (qc ? qc : 1) : 0;
                }
            }
            if (D < GC_SERIAL) {
                // a short stretch of ordinary f32 steps from LDS-staged terms
                const int len = min(GC_SERIAL, n - i);
                for (int r = tid; r < len; r += GC_THREADS) s_w[r] = w[i + r];
                __syncthreads();
                if (tid == 0) {
                    // Terms are positive, so the running value is monotone
                    // (up for sums, down for the walk): a batch of eight whose
                    // end value has not reached the stop condition never
                    // reached it inside, and is added plainly; the batch that
                    // reaches it is replayed term by term from its start
                    // value (identical arithmetic either way).
                    auto reached = [&](float v) {
                        return walk ? v <= 0.0f : (use_target && v >= target);
                    };
                    float y = x;
                    int k = 0, stop = 0;
                    for (; k + 8 <= len; k += 8) {
                        const float4 b0 = *(const float4 *)&s_w[k];
                        const float4 b1 = *(const float4 *)&s_w[k + 4];
                        float z = y;
                        if (!walk) {
                            z += b0.x; z += b0.y; z += b0.z; z += b0.w;
                            z += b1.x; z += b1.y; z += b1.z; z += b1.w;
                        } else {
                            z -= b0.x; z -= b0.y; z -= b0.z; z -= b0.w;
                            z -= b1.x; z -= b1.y; z -= b1.z; z -= b1.w;
                        }
                        if (!reached(z)) {
                            y = z;
                            continue;
                        }
                        stop = 1;
                        break;
                    }
                    // the reaching batch (stop) or the tail past the last
                    // whole batch, term by term
                    const int end = stop ? k + 8 : len;
                    stop = 0;
                    for (; k < end; ++k) {
                        y = walk ? y - s_w[k] : y + s_w[k];
                        if (reached(y)) {
                            stop = 1;
                            break;
                        }
                    }
                    s_x = y;
                    s_stop = stop;
                    s_i = stop ? i + k : i + len;
                }
                __syncthreads();
                continue;
            }
            int W = (int)min<uint64_t>(D, (uint64_t)GC_THREADS * GC_IPT);
            W = max(W, GC_THREADS);
            W = min(W, n - i);
            const int ipt = (W + GC_THREADS - 1) / GC_THREADS;
            const int base = i + tid * ipt;
            // 32-bit grid values (see grid_units32); the bounds below lim
            const uint32_t K32 = (uint32_t)K, lim32 = (uint32_t)lim, low32 = (uint32_t)(low ? low : 1);
            const uint32_t T32 = (uint32_t)min<uint64_t>(T, lim);
            uint32_t q[GC_IPT], qc[GC_IPT];
            float wv[GC_IPT];
            bool tie[GC_IPT];
            uint32_t lsum = 0;
#pragma unroll
            for (int r = 0; r < GC_IPT; ++r) {
                const int j = base + r;
                q[r] = qc[r] = 0;
                tie[r] = false;
                wv[r] = 0.f;
                if (r < ipt && j < i + W) {
                    wv[r] = w[j];
                    q[r] = grid_units32(__float_as_uint(wv[r]), ue, tie[r], qc[r]);
                    lsum += q[r];
                }
            }
            uint32_t tot;
            uint32_t E = block_scan_u32(lsum, s_tmp, &tot);
            if (tid == 0) s_ev = 0x7fffffff;
            __syncthreads();
            int mine = 0x7fffffff;
            uint32_t mine_pref = 0;
            float mine_w = 0.f;
#pragma unroll
            for (int r = 0; r < GC_IPT; ++r) {
                const int j = base + r;
                if (r < ipt && j < i + W && mine == 0x7fffffff) {
                    bool ev = tie[r];
                    if (!walk) ev = ev || K32 + E + q[r] >= lim32 || (use_target && K32 + E + q[r] >= T32);
                    else ev = ev || E + qc[r] + low32 > K32;
                    if (ev) {
                        mine = j - i;
                        mine_pref = E;
                        mine_w = wv[r];
                    } else {
                        E += q[r];
                    }
                }
            }
            if (mine != 0x7fffffff) atomicMin(&s_ev, mine);
            __syncthreads();
            const int e = s_ev;
            if (e != 0x7fffffff && mine == e) {
                s_pref = mine_pref;
                s_wev = mine_w;
            }
            __syncthreads();
            if (tid == 0) {
                const uint64_t P = e == 0x7fffffff ? tot : s_pref;
                float y = from_grid(x, walk ? K - P : K + P);
                int k = e == 0x7fffffff ? i + W : i + e, stop = 0;
                if (e != 0x7fffffff) {
                    // the event term, as one ordinary f32 step
                    if (!walk) {
                        y += s_wev;
                        stop = use_target && y >= target;
                    } else {
                        y -= s_wev;
                        stop = y <= 0.0f;
                    }
                    if (!stop) ++k;
                }
                s_x = y;
                s_i = k;
                s_stop = stop;
            }
            __syncthreads();
        }
    };

    // pass 1: the total over every candidate (Rust's f32 sum starts at -0.0)
    run(false, 0, -0.0f, C, false, 0.f, true);
    const float total = s_x;
    int keep = C;
    float kept = total;
    const float top_p = smp.top_p;
    if (top_p >= 0.f) {
        const float p = top_p > 1.f ? 1.f : top_p;
        const float target = total * p;
        // restart from the last checkpoint still below the target
        int c = 0;
        const int nck = s_nck;
        while (c + 1 < nck && ck_x[c + 1] < target) ++c;
        const int i0 = nck ? ck_i[c] : 0;
        const float x0 = nck ? ck_x[c] : -0.0f;
        __syncthreads();
        run(false, i0, x0, C, true, target, false);
        keep = s_stop ? s_i + 1 : C;
        kept = -0.0f + s_x;
    }
    // pass 2: the draw walks the kept prefix
    uint64_t state = smp.state;
    const uint64_t x = splitmix_next(state);
    const float u = (float)((double)(x >> 11) / 9007199254740992.0) * kept;
    __syncthreads();
    run(true, 0, u, keep, false, 0.f, false);
    const int hit = s_stop ? s_i : -1;
    if (tid == 0) {
        int out;
        if (hit >= 0) out = cand[hit].id;
        else out = (top_p < 0.f && info.zmax >= 0) ? info.zmax : cand[keep - 1].id;
        a.ids_out[row] = (uint32_t)out;
        a.flags_out[row] = (uint8_t)info.flags;
        if (a.state_out) a.state_out[row] = state;
    }
}

size_t pick_scratch_bytes(int n, int V) {
    const size_t cap = (size_t)pick_cap(V);
    return (size_t)n * cap * (sizeof(Cand) + sizeof(float)) + cap * sizeof(Cand) +
           (size_t)n * PB_BINS * 4 * 5 + (size_t)n * sizeof(PickRow) + 64;
}

void launch_pick(const PickArgs &a, hipStream_t s) {
    static bool attr = false;
    size_t shm = sizeof(Cand) * PICK_LDS_CAP;
    if (!attr) {
        ESP_HIP(hipFuncSetAttribute((const void *)pick_k,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
        ESP_HIP(hipFuncSetAttribute((const void *)pick_bsort_k,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
        attr = true;
    }
    const bool sampled = a.samplers != nullptr;
    PickArgs ak = a;
    {
        // ESP_PICK_DIRECT_MAX lowers the in-block path's row length (comparisons)
        static const int dm = [] {
            const char *e = getenv("ESP_PICK_DIRECT_MAX");
            return e ? std::max(1, std::min(atoi(e), PICK_LDS_CAP)) : PICK_DIRECT_MAX;
        }();
        ak.direct_max = dm;
    }
    PickScratch ps{};
    if (sampled) {
        if (a.scratch_bytes < pick_scratch_bytes(a.n, a.V))
            fail(ESP_BACKEND, "pick: sampling scratch too small");
        ps = pick_layout(a.scratch, a.n, a.V);
        pick_reset_k<<<(a.n + 2 + 255) / 256, 256, 0, s>>>(ps, a.n);
    }
    pick_k<<<a.n, PICK_THREADS, shm, s>>>(ak);
    if (sampled) {
        pick_bsort_k<<<256, PICK_THREADS, shm, s>>>(ps);
        pick_bsort_big_k<<<1, PICK_THREADS, 0, s>>>(ps);
        // ESP_PICK_CHAIN_THREADS: the chain kernel's block size (comparisons)
        static const int ct = [] {
            const char *e = getenv("ESP_PICK_CHAIN_THREADS");
            const int v = e ? atoi(e) : 1024;
            return v == 256 || v == 512 ? v : 1024;
        }();
        static bool cattr = false;
        constexpr int lw = GC_LDS_W * 4;
        if (!cattr) {
            ESP_HIP(hipFuncSetAttribute((const void *)pick_chain_k<256>, hipFuncAttributeMaxDynamicSharedMemorySize, lw));
            ESP_HIP(hipFuncSetAttribute((const void *)pick_chain_k<512>, hipFuncAttributeMaxDynamicSharedMemorySize, lw));
            ESP_HIP(hipFuncSetAttribute((const void *)pick_chain_k<1024>, hipFuncAttributeMaxDynamicSharedMemorySize, lw));
            cattr = true;
        }
        if (ct == 256) pick_chain_k<256><<<a.n, 256, lw, s>>>(a, ps);
        else if (ct == 512) pick_chain_k<512><<<a.n, 512, lw, s>>>(a, ps);
        else pick_chain_k<1024><<<a.n, 1024, lw, s>>>(a, ps);
    }
}

}  // namespace esp
