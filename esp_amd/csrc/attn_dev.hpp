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

// Merges the online-softmax states (m, l, acc[8]) of lane pairs (lane, lane ^ X).
template <int X, int GM>
__device__ __forceinline__ void att_pair_merge(int G, float (&m)[GM], float (&l)[GM], float (&acc)[GM][8]) {
#pragma unroll
    for (int j = 0; j < GM; ++j) {
        if (j >= G) break;
        float m0, m1, l0, l1;
        lane_pair<X>(m[j], m0, m1);
        lane_pair<X>(l[j], l0, l1);
        const float mn = fmaxf(m0, m1);
        const float w0 = mn == -INFINITY ? 0.f : __expf(m0 - mn);
        const float w1 = mn == -INFINITY ? 0.f : __expf(m1 - mn);
        l[j] = l0 * w0 + l1 * w1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float a0, a1;
            lane_pair<X>(acc[j][i], a0, a1);
            acc[j][i] = a0 * w0 + a1 * w1;
        }
        m[j] = mn;
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
