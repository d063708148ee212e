// Device-side helpers shared by the kernel files (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esp {

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// f32 -> bf16 bits, round to nearest even (quiet NaN preserved).
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <typename T> __device__ __forceinline__ float ld(const T *p, size_t i);
template <> __device__ __forceinline__ float ld<float>(const float *p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<uint16_t>(const uint16_t *p, size_t i) {
    return bf2f(p[i]);
}

template <> __device__ __forceinline__ float ld<_Float16>(const _Float16 *p, size_t i) {
    return (float)p[i];
}

template <typename T> __device__ __forceinline__ void st(T *p, size_t i, float v);
template <> __device__ __forceinline__ void st<float>(float *p, size_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<uint16_t>(uint16_t *p, size_t i, float v) {
    p[i] = f2bf(v);
}
// f32 -> f16, round to nearest even
template <> __device__ __forceinline__ void st<_Float16>(_Float16 *p, size_t i, float v) {
    p[i] = (_Float16)v;
}

// Store x into a split (hi/lo bf16 planes) matrix; `plane` = elements per plane.
__device__ __forceinline__ void st_split(uint16_t *base, size_t plane, size_t i, float x) {
    uint16_t h = f2bf(x);
    base[i] = h;
    base[plane + i] = f2bf(x - bf2f(h));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` needs 16 floats.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    int nw = blockDim.x >> 6;
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

// Row tile `slot` of a GEMM launch with tiles of BM rows. One group (offs
// == nullptr): rows [slot * BM, M). Grouped: slots run through the groups in
// order, ceil(n_e / BM) per group e of offs[e+1] - offs[e] rows (offsets
// clamped into [0, M] and made ascending, so a corrupt table stays in
// bounds); gives the tile's first row, its group's row end and the group,
// or false past the last tile. Uniform across the block (scalar loads).
__device__ __forceinline__ bool group_tile(const int32_t *offs, int n_groups, int M, int slot,
                                           int BM, int &m0, int &mend, int &grp) {
    if (!offs) {
        m0 = slot * BM;
        mend = M;
        grp = 0;
        return m0 < M;
    }
    int acc = 0, prev = min(max(offs[0], 0), M);
    for (int e = 0; e < n_groups; ++e) {
        const int nx = min(max(offs[e + 1], prev), M);
        const int tiles = (nx - prev + BM - 1) / BM;
        if (slot < acc + tiles) {
            m0 = prev + (slot - acc) * BM;
            mend = nx;
            grp = e;
            return true;
        }
        acc += tiles;
        prev = nx;
    }
    return false;
}

}  // namespace esp
