// Device pass over one staged layer block (streaming.hpp): finiteness of
// every tensor (tensors.rs:22-66), finite positive block scales of packed
// projections (weight_format.rs:225-273), and the exact widening of bf16 /
// f16 artifact tensors into the block's f32 regions.
//
// HBM-bound: one read of every checked byte plus one f32 write per widened
// element. Each descriptor gets its own row of workgroups (blockIdx.y);
// lanes take 16 bytes at a time, so a wave reads 1 KiB per step. Region
// starts are 256-byte aligned by construction (the staging plan pads them);
// the element tail past the last full 16-byte group, and any region whose
// start is not 16-byte aligned, is taken one element per lane.
#include <limits.h>

#include "common.hpp"
#include "streaming.hpp"

namespace esp {

namespace {

__device__ inline uint32_t bf16_bad(uint32_t h) { return (h & 0x7f80u) == 0x7f80u; }
__device__ inline uint32_t f16_bad(uint32_t h) { return (h & 0x7c00u) == 0x7c00u; }
__device__ inline uint32_t f32_bad(uint32_t u) { return (u & 0x7f800000u) == 0x7f800000u; }
__device__ inline uint32_t scale_bad(uint32_t u) {
    // finite and > 0: sign clear, not zero, exponent not all ones
    return (u >> 31) | (uint32_t)(u == 0u) | f32_bad(u);
}
__device__ inline float f16_to_f32(uint32_t h) {
    _Float16 v;
    const unsigned short b = (unsigned short)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

__global__ void __launch_bounds__(256) stream_check_k(StreamChecks c, int *bad) {
    const StreamCheck d = c.d[blockIdx.y];
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nthr = (uint64_t)gridDim.x * blockDim.x;
    uint32_t err = 0;
    // 16-byte groups only where source and destination are both aligned
    // (a fused region's later tensors may not be); otherwise every element
    // takes the one-per-lane path
    const bool al = ((uintptr_t)d.src % 16 == 0) && ((uintptr_t)d.dst % 16 == 0);
    if (d.op == SC_BF16 || d.op == SC_BF16_F32 || d.op == SC_F16_F32) {
        // 2-byte elements, 8 per 16-byte group
        const uint4 *src = (const uint4 *)d.src;
        const uint64_t groups = al ? d.n / 8 : 0;
        for (uint64_t g = tid; g < groups; g += nthr) {
            const uint4 v = src[g];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            if (d.op == SC_BF16) {
                for (int k = 0; k < 4; ++k) err |= bf16_bad(w[k] & 0xffffu) | bf16_bad(w[k] >> 16);
                continue;
            }
            float f[8];
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = w[k] & 0xffffu, hi = w[k] >> 16;
                if (d.op == SC_BF16_F32) {
                    err |= bf16_bad(lo) | bf16_bad(hi);
                    f[2 * k] = __uint_as_float(lo << 16);
                    f[2 * k + 1] = __uint_as_float(hi << 16);
                } else {
                    err |= f16_bad(lo) | f16_bad(hi);
                    f[2 * k] = f16_to_f32(lo);
                    f[2 * k + 1] = f16_to_f32(hi);
                }
            }
            float4 *o = (float4 *)(d.dst + g * 8);
            o[0] = make_float4(f[0], f[1], f[2], f[3]);
            o[1] = make_float4(f[4], f[5], f[6], f[7]);
        }
        const unsigned short *s16 = (const unsigned short *)d.src;
        for (uint64_t i = groups * 8 + tid; i < d.n; i += nthr) {
            const uint32_t h = s16[i];
            if (d.op == SC_BF16) err |= bf16_bad(h);
            else if (d.op == SC_BF16_F32) {
                err |= bf16_bad(h);
                d.dst[i] = __uint_as_float(h << 16);
            } else {
                err |= f16_bad(h);
                d.dst[i] = f16_to_f32(h);
            }
        }
    } else {
        // 4-byte elements (SC_F32, SC_SCALES), 4 per group
        const uint4 *src = (const uint4 *)d.src;
        const bool sc = d.op == SC_SCALES;
        const uint64_t groups = al ? d.n / 4 : 0;
        for (uint64_t g = tid; g < groups; g += nthr) {
            const uint4 v = src[g];
            if (sc) err |= scale_bad(v.x) | scale_bad(v.y) | scale_bad(v.z) | scale_bad(v.w);
            else err |= f32_bad(v.x) | f32_bad(v.y) | f32_bad(v.z) | f32_bad(v.w);
        }
        const uint32_t *s32 = (const uint32_t *)d.src;
        for (uint64_t i = groups * 4 + tid; i < d.n; i += nthr)
            err |= sc ? scale_bad(s32[i]) : f32_bad(s32[i]);
    }
    if (err) atomicMin(bad, d.tag);
}

}  // namespace

void launch_stream_check(const StreamChecks &c, int *bad, hipStream_t s) {
    if (c.n <= 0) return;
    // 128 workgroups per region: the largest projection (a few hundred MB)
    // streams at full HBM rate, the small norms cost one short wave each
    dim3 grid(128, (unsigned)c.n);
    hipLaunchKernelGGL(stream_check_k, grid, dim3(256), 0, s, c, bad);
    ESP_HIP(hipGetLastError());
}

}  // namespace esp
