// Token choice over device-resident logits rows: the grammar bitmask
// (constraint.rs:277-297), greedy argmax with the lowest id winning ties
// (generate.rs:70-79, provider.rs:808-815), and the seeded temperature /
// nucleus sampler (sample.rs:83-121) reproduced step for step: f32 weights
// exp((l - max) * (1/T)), a descending sort with ties by ascending id,
// sequential f32 prefix sums for the nucleus cut and the kept mass, one
// splitmix64 draw, and the subtract-walk.
#include "common.hpp"
#include "dev.hpp"

namespace esp {

constexpr int PICK_THREADS = 1024;
constexpr int PICK_LDS_CAP = 16384;  // candidates sorted in LDS (8 B each)

struct Cand {
    float w;
    int32_t id;
};

// Descending weight, ascending id; sentinels (w < 0) last.
__device__ __forceinline__ bool before(Cand a, Cand b) {
    if (a.w != b.w) return a.w > b.w;
    return a.id < b.id;
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

__global__ void __launch_bounds__(PICK_THREADS) pick_k(PickArgs a) {
    extern __shared__ Cand lds[];
    __shared__ float red_f[32];
    __shared__ int red_i[32];
    __shared__ int s_count, s_zmax, s_bad, s_elig;
    const int row = blockIdx.x;
    const int V = a.V;
    const float *L = a.logits + (size_t)row * V;
    const uint32_t *bits = a.allowed ? a.allowed + (size_t)row * ((V + 31) / 32) : nullptr;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) {
        s_count = 0;
        s_zmax = -1;
        s_bad = 0;
        s_elig = 0;
    }
    __syncthreads();
    // pass 1: mask, finiteness, greedy best and max
    float best = -INFINITY;
    int best_id = 0x7fffffff;
    int bad = 0, elig = 0;
    for (int i = tid; i < V; i += blockDim.x) {
        float v = L[i];
        bool fin = isfinite(v);
        bad |= !fin;
        bool allowed = bits ? ((bits[i >> 5] >> (i & 31)) & 1u) : true;
        if (bits ? (!allowed || !fin) : isnan(v)) v = -INFINITY;
        elig += (allowed && fin);
        if (v > best || (v == best && i < best_id)) {
            best = v;
            best_id = i;
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
    const esp_sampler *smp = a.samplers ? a.samplers + row : nullptr;
    const bool sampled = smp && smp->temperature > 0.f;
    if (!sampled || (bits && s_elig == 0)) {
        if (tid == 0) {
            a.ids_out[row] = (bits && s_elig == 0) ? 0u : (uint32_t)(red_i[0] == 0x7fffffff ? 0 : red_i[0]);
            a.flags_out[row] = flags;
            if (a.state_out) a.state_out[row] = smp ? smp->state : 0;
        }
        return;
    }
    // pass 2: weights and candidate compaction
    const float inv_t = 1.0f / smp->temperature;
    Cand *gbuf = (Cand *)((char *)a.scratch + (size_t)row * (size_t)((V + 1) * sizeof(Cand)) * 2);
    // count candidates first to choose LDS or global storage; the largest
    // zero-weight id (the fall-through of an uncut list) is a block max
    int cnt = 0, zmax = -1;
    for (int i = tid; i < V; i += blockDim.x) {
        float v = L[i];
        bool allowed = bits ? ((bits[i >> 5] >> (i & 31)) & 1u) : true;
        if (bits && (!allowed || !isfinite(v))) v = -INFINITY;
        float w = v == -INFINITY ? 0.f : (float)exp((double)((v - mx) * inv_t));
        if (w > 0.f) ++cnt;
        else if (w == 0.f) zmax = i;  // ids rise along this thread's stride
    }
    cnt = (int)wave_sum((float)cnt);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) zmax = max(zmax, __shfl_xor(zmax, o, 64));
    if (lane == 0) {
        atomicAdd(&s_count, cnt);
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
    int n2 = 1;
    while (n2 < C) n2 <<= 1;
    Cand *buf = n2 <= PICK_LDS_CAP ? lds : gbuf;
    __syncthreads();
    if (tid == 0) s_count = 0;
    __syncthreads();
    for (int i = tid; i < V; i += blockDim.x) {
        float v = L[i];
        bool allowed = bits ? ((bits[i >> 5] >> (i & 31)) & 1u) : true;
        if (bits && (!allowed || !isfinite(v))) v = -INFINITY;
        float w = v == -INFINITY ? 0.f : (float)exp((double)((v - mx) * inv_t));
        if (w > 0.f) {
            int slot = atomicAdd(&s_count, 1);
            buf[slot] = Cand{w, i};
        }
    }
    __syncthreads();
    for (int i = C + tid; i < n2; i += blockDim.x) buf[i] = Cand{-1.f, 0x7fffffff};
    __syncthreads();
    bitonic(buf, n2);
    // LDS-resident lists go to struct-of-arrays in place (weights, then ids)
    // so the serial pass below reads four weights per load; every element is
    // read into registers before any is written back
    const bool soa = n2 <= PICK_LDS_CAP;
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

size_t pick_scratch_bytes(int n, int V) {
    return (size_t)n * (size_t)((V + 1) * sizeof(Cand)) * 2;
}

void launch_pick(const PickArgs &a, hipStream_t s) {
    static bool attr = false;
    size_t shm = sizeof(Cand) * PICK_LDS_CAP;
    if (!attr) {
        ESP_HIP(hipFuncSetAttribute((const void *)pick_k,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
        attr = true;
    }
    pick_k<<<a.n, PICK_THREADS, shm, s>>>(a);
}

}  // namespace esp
