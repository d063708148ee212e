// Device helpers of the split-K decode attention (k_decode.hip): split
// limits, lane-pair exchanges of online-softmax states, the cache's 4-dim
// slices, and a barrier that does not wait for loads in flight.
#pragma once

#include "decode_dev.hpp"

namespace esp {

constexpr int ATT_MAX_SPLIT = 128;
constexpr int ATT_WAVES = 8;      // waves per attention block (two per SIMD)
constexpr int ATT_MB = 32;        // splits whose partials one merge batch loads at once

// Both values of the lane pair (lane, lane ^ X), lower lane first, in every
// lane of the pair: X = 32 and 16 with the gfx950 permlane swaps, X = 8 with
// a DPP rotate by 8 inside each 16-lane row.
template <int X> __device__ __forceinline__ void lane_pair(float v, float &lo, float &hi) {
    if constexpr (X == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else if constexpr (X == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        static_assert(X == 8, "lane_pair: X = 8, 16 or 32");
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
        const bool low = (threadIdx.x & 8) == 0;
        lo = low ? v : o;
        hi = low ? o : v;
    }
}

// Merges the online-softmax states (m, l, acc[8]) of the key groups of a
// wave (lane pairs at distance LPK .. 32): the wave's maximum per head first
// (max over the pairs), then each group's state rescaled to it once (one
// exp per head and lane), then plain sums over the pairs, lower lane first,
// so every lane of a pair holds the same result. Against merging the pairs
// as online-softmax states level by level (two exps per head and level) this
// measured C2 decode 1345-1360 -> 1358-1374 tok/s and C3 309.8-310.3 ->
// 311.2-313.0 tok/s (three alternating pairs of runs on one box).
template <int LPK, int GM>
__device__ __forceinline__ void att_wave_merge(int G, float (&m)[GM], float (&l)[GM], float (&acc)[GM][8]) {
    auto pmax = [](float v) {
        float a, b;
        if constexpr (LPK <= 8) { lane_pair<8>(v, a, b); v = fmaxf(a, b); }
        if constexpr (LPK <= 16) { lane_pair<16>(v, a, b); v = fmaxf(a, b); }
        lane_pair<32>(v, a, b);
        return fmaxf(a, b);
    };
    auto psum = [](float v) {
        float a, b;
        if constexpr (LPK <= 8) { lane_pair<8>(v, a, b); v = a + b; }
        if constexpr (LPK <= 16) { lane_pair<16>(v, a, b); v = a + b; }
        lane_pair<32>(v, a, b);
        return a + b;
    };
#pragma unroll
    for (int j = 0; j < GM; ++j) {
        if (j >= G) break;
        const float mx = pmax(m[j]);
        const float w = mx == -INFINITY ? 0.f : __expf(m[j] - mx);
        l[j] = psum(l[j] * w);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = psum(acc[j][i] * w);
        m[j] = mx;
    }
}

// Keys and values as 4-dim slices: f32x4 (f32 cache) or four f16 in a u32x2.
template <bool F16> struct KvSlice { typedef f32x4_t T; };
template <> struct KvSlice<true> { typedef u32x2_t T; };
__device__ __forceinline__ f32x4_t kv_f32(f32x4_t x) { return x; }
__device__ __forceinline__ f32x4_t kv_f32(u32x2_t x) {
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    return __builtin_convertvector(__builtin_bit_cast(h4_t, x), f32x4_t);
}
__device__ __forceinline__ u32x2_t kv_f16(f32x4_t x) {
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(u32x2_t, __builtin_convertvector(x, h4_t));
}

// LDS stores visible to the other waves of the block, with no wait on the
// vector-memory loads in flight (a fenced __syncthreads waits for every one).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace esp
