// Device helpers of the single-token kernels (k_decode.hip): cross-block
// hand-off stores and loads, and the packed weight formats.
#pragma once

#include "common.hpp"
#include "dev.hpp"

namespace esp {

constexpr int DG_THREADS = 256;
constexpr int DG_WAVES = 4;
constexpr int DG_MAXC = 8;  // max 8-element chunks per lane per row (K <= 4*64*8*8 = 16384)

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Cross-block hand-off without flushing L2: partials are written with
// agent-scope (write-through) stores, the writer waits for its stores to
// complete (s_waitcnt vmcnt(0)) before taking a ticket, and the last block
// reads the partials with agent-scope loads.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_agent(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Packed projection weights (decoder/weight_format.rs:138-223): signed
// integers along K in each [out, in] row, one f32 scale per 32 inputs;
// weight = q * scale. q8: one byte per weight. q4: two per byte, the even
// input in the low nibble.
struct q8_t {
    int8_t v;
};
struct q4_t {
    uint8_t v;
};
template <typename WT> struct WPacked { static constexpr bool v = false; };
template <> struct WPacked<q8_t> { static constexpr bool v = true; };
template <> struct WPacked<q4_t> { static constexpr bool v = true; };

// Chunk<WT>: W consecutive weights of one row and their dot product with W
// f32 inputs. load_at(base, e, scales) reads weights e .. e+W-1 of a
// row-major matrix (e a multiple of W; scales used by packed formats).
template <typename WT> struct Chunk;
template <> struct Chunk<uint16_t> {  // 8 bf16 = 16 bytes
    static constexpr int W = 8;  // weights per chunk
    u32x4_t v;
    __device__ __forceinline__ void load(const uint16_t *p) {
        v = __builtin_nontemporal_load((const u32x4_t *)p);
    }
    __device__ __forceinline__ void load_at(const void *base, size_t e, const float *) {
        load((const uint16_t *)base + e);
    }
    __device__ __forceinline__ float dot(const float *x) const {
        float s = 0.f;
        s += __uint_as_float(v.x << 16) * x[0];
        s += __uint_as_float(v.x & 0xffff0000u) * x[1];
        s += __uint_as_float(v.y << 16) * x[2];
        s += __uint_as_float(v.y & 0xffff0000u) * x[3];
        s += __uint_as_float(v.z << 16) * x[4];
        s += __uint_as_float(v.z & 0xffff0000u) * x[5];
        s += __uint_as_float(v.w << 16) * x[6];
        s += __uint_as_float(v.w & 0xffff0000u) * x[7];
        return s;
    }
    __device__ __forceinline__ float dot(const float *x, float) const { return dot(x); }
};
template <> struct Chunk<float> {  // 8 f32 = 2 x 16 bytes
    static constexpr int W = 8;
    f32x4_t a, b;
    __device__ __forceinline__ void load(const float *p) {
        a = __builtin_nontemporal_load((const f32x4_t *)p);
        b = __builtin_nontemporal_load((const f32x4_t *)p + 1);
    }
    __device__ __forceinline__ void load_at(const void *base, size_t e, const float *) {
        load((const float *)base + e);
    }
    __device__ __forceinline__ float dot(const float *x) const {
        float s = 0.f;
        s += a.x * x[0];
        s += a.y * x[1];
        s += a.z * x[2];
        s += a.w * x[3];
        s += b.x * x[4];
        s += b.y * x[5];
        s += b.z * x[6];
        s += b.w * x[7];
        return s;
    }
    __device__ __forceinline__ float dot(const float *x, float) const { return dot(x); }
};

// Packed chunks hold 16 weights (16 bytes of q8, 8 of q4) inside one
// 32-input scale block. The signed values are biased to unsigned bytes / nibbles
// (xor 0x80 / 0x8) so each converts to f32 in one instruction; the bias
// comes back once per chunk through xsum, the sum of the chunk's inputs:
// sum q x = sum (q + b) x - b * xsum.
template <> struct Chunk<q8_t> {
    static constexpr int W = 16;
    u32x4_t v;
    float sc;
    __device__ __forceinline__ void load_at(const void *base, size_t e, const float *scales) {
        v = __builtin_nontemporal_load((const u32x4_t *)((const int8_t *)base + e));
        sc = scales[e >> 5];
    }
    __device__ __forceinline__ float dot(const float *x, float xsum) const {
        float s = 0.f;
        const unsigned d[4] = {v.x ^ 0x80808080u, v.y ^ 0x80808080u, v.z ^ 0x80808080u,
                               v.w ^ 0x80808080u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s += (float)(d[j] & 0xff) * x[4 * j];
            s += (float)((d[j] >> 8) & 0xff) * x[4 * j + 1];
            s += (float)((d[j] >> 16) & 0xff) * x[4 * j + 2];
            s += (float)(d[j] >> 24) * x[4 * j + 3];
        }
        return (s - 128.f * xsum) * sc;
    }
};
template <> struct Chunk<q4_t> {  // 16 q4 weights = 8 bytes (all 64 lanes busy at K 4096)
    static constexpr int W = 16;
    u32x2_t v;
    float sc;
    __device__ __forceinline__ void load_at(const void *base, size_t e, const float *scales) {
        v = __builtin_nontemporal_load((const u32x2_t *)((const uint8_t *)base + (e >> 1)));
        sc = scales[e >> 5];
    }
    __device__ __forceinline__ float dot(const float *x, float xsum) const {
        float s = 0.f;
        const unsigned d[2] = {v.x ^ 0x88888888u, v.y ^ 0x88888888u};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned lo = d[j] & 0x0f0f0f0fu, hi = (d[j] >> 4) & 0x0f0f0f0fu;
            // byte b of dword j holds weights 8j + 2b (low) and 8j + 2b + 1 (high)
            s += (float)(lo & 0xff) * x[8 * j];
            s += (float)(hi & 0xff) * x[8 * j + 1];
            s += (float)((lo >> 8) & 0xff) * x[8 * j + 2];
            s += (float)((hi >> 8) & 0xff) * x[8 * j + 3];
            s += (float)((lo >> 16) & 0xff) * x[8 * j + 4];
            s += (float)((hi >> 16) & 0xff) * x[8 * j + 5];
            s += (float)(lo >> 24) * x[8 * j + 6];
            s += (float)(hi >> 24) * x[8 * j + 7];
        }
        return (s - 8.f * xsum) * sc;
    }
};

// rows handled per unit: SWIGLU and QKVROPE units are row pairs
template <int EPI> struct RowsPerUnit { static constexpr int v = 1; };
template <> struct RowsPerUnit<DG_SWIGLU> { static constexpr int v = 2; };
template <> struct RowsPerUnit<DG_QKVROPE> { static constexpr int v = 2; };

constexpr int DG_MAX_IT = 64;  // grid-stride iterations per block

// Sum over all 64 lanes, returned wave-uniform: DPP sums inside each
// 16-lane row, then the four row sums read out in a fixed order.
__device__ __forceinline__ float wave_sum_uniform(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    const int b = __builtin_bit_cast(int, v);
    return ((__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
             __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32))) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
}

// Sum over aligned groups of N lanes (N = 8 or 16) with DPP lane swaps:
// quad xor 1, quad xor 2, half-row mirror (8 lanes), row mirror (16 lanes).
template <int N> __device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16, "group_sum: 8 or 16 lanes");
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    if (N == 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
}

}  // namespace esp
