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
// owned by this block.
__device__ void bitonic(Cand *buf, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += blockDim.x) {
                int p = i ^ j;
                if (p > i) {
                    Cand x = buf[i], y = buf[p];
                    bool up = (i & k) == 0;  // this run sorted by `before`
                    bool swap = up ? before(y, x) : before(x, y);
                    if (swap) {
                        buf[i] = y;
                        buf[p] = x;
                    }
                }
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
    // count candidates first to choose LDS or global storage
    int cnt = 0;
    for (int i = tid; i < V; i += blockDim.x) {
        float v = L[i];
        bool allowed = bits ? ((bits[i >> 5] >> (i & 31)) & 1u) : true;
        if (bits && (!allowed || !isfinite(v))) v = -INFINITY;
        float arg = (v - mx) * inv_t;
        float w = (float)exp((double)arg);
        if (w > 0.f) ++cnt;
        else if (w == 0.f) atomicMax(&s_zmax, i);
    }
    cnt = (int)wave_sum((float)cnt);
    if (lane == 0) atomicAdd(&s_count, cnt);
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
        float w = (float)exp((double)((v - mx) * inv_t));
        if (w > 0.f) {
            int slot = atomicAdd(&s_count, 1);
            buf[slot] = Cand{w, i};
        }
    }
    __syncthreads();
    for (int i = C + tid; i < n2; i += blockDim.x) buf[i] = Cand{-1.f, 0x7fffffff};
    __syncthreads();
    bitonic(buf, n2);
    if (tid != 0) return;
    // sequential pass (sample.rs:96-120)
    int keep = C;
    const float top_p = smp->top_p;
    if (top_p >= 0.f) {
        float total = -0.0f;
        for (int i = 0; i < C; ++i) total += buf[i].w;
        float p = top_p > 1.f ? 1.f : top_p;
        float target = total * p;
        float mass = 0.0f;
        keep = 0;
        for (int i = 0; i < C; ++i) {
            mass += buf[i].w;
            keep = i + 1;
            if (mass >= target) break;
        }
        if (keep < 1) keep = 1;
    }
    float total = -0.0f;
    for (int i = 0; i < keep; ++i) total += buf[i].w;
    uint64_t state = smp->state;
    uint64_t x = splitmix_next(state);
    float u = (float)((double)(x >> 11) / 9007199254740992.0) * total;
    // fall-through value: the last element of the (truncated) sorted list
    int32_t out = (top_p < 0.f && s_zmax >= 0) ? s_zmax : (keep > 0 ? buf[keep - 1].id : 0);
    for (int i = 0; i < keep; ++i) {
        u -= buf[i].w;
        if (u <= 0.0f) {
            out = buf[i].id;
            break;
        }
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
