// Single-row projections (decode): y = W x streamed from HBM at full width.
// Weight rows stay in HF [out, in] order, so each output is one contiguous
// row read with 16-byte loads; the input row lives in LDS as f32 (optionally
// RMS-normalised on the way in, which removes a separate norm launch).
#include "common.hpp"
#include "dev.hpp"

namespace esp {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / 64;

template <typename WT> struct Vec16;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <> struct Vec16<uint16_t> {
    static constexpr int N = 8;
    typedef u32x4_t raw;
    __device__ static void unpack(raw r, float *o) {
        o[0] = __uint_as_float(r.x << 16);
        o[1] = __uint_as_float(r.x & 0xffff0000u);
        o[2] = __uint_as_float(r.y << 16);
        o[3] = __uint_as_float(r.y & 0xffff0000u);
        o[4] = __uint_as_float(r.z << 16);
        o[5] = __uint_as_float(r.z & 0xffff0000u);
        o[6] = __uint_as_float(r.w << 16);
        o[7] = __uint_as_float(r.w & 0xffff0000u);
    }
};
template <> struct Vec16<float> {
    static constexpr int N = 4;
    typedef f32x4_t raw;
    __device__ static void unpack(raw r, float *o) {
        o[0] = r.x;
        o[1] = r.y;
        o[2] = r.z;
        o[3] = r.w;
    }
};

// Loads the (optionally normalised) input row into LDS.
__device__ __forceinline__ void gemv_stage_x(const GemvArgs &a, float *xs, float *red) {
    if (a.gamma) {
        float ss = 0.f;
        for (int k = threadIdx.x; k < a.K; k += blockDim.x) ss += a.x[k] * a.x[k];
        ss = block_sum(ss, red);
        float rms = sqrtf(ss / (float)a.K + a.eps);
        for (int k = threadIdx.x; k < a.K; k += blockDim.x) xs[k] = (a.x[k] / rms) * a.gamma[k];
    } else {
        for (int k = threadIdx.x; k < a.K; k += blockDim.x) xs[k] = a.x[k];
    }
    __syncthreads();
}

// dot(row_r, xs) for R weight rows at once (R independent load streams per
// lane keep enough bytes in flight), reduced across the wave.
template <typename WT, int R, bool VEC>
__device__ __forceinline__ void gemv_rows(const WT *const *rowp, int K, const float *xs,
                                          float *out) {
    const int lane = threadIdx.x & 63;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    int kdone = 0;
    if (VEC) {
        typedef Vec16<WT> V;
        const int nv = K / V::N;
#pragma unroll 4
        for (int c = lane; c < nv; c += 64) {
            typename V::raw raw[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
                raw[r] = __builtin_nontemporal_load((const typename V::raw *)rowp[r] + c);
            float xv[V::N];
#pragma unroll
            for (int i = 0; i < V::N; ++i) xv[i] = xs[c * V::N + i];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float w[V::N];
                V::unpack(raw[r], w);
#pragma unroll
                for (int i = 0; i < V::N; ++i) acc[r] += w[i] * xv[i];
            }
        }
        kdone = nv * V::N;
    }
    for (int k = kdone + lane; k < K; k += 64) {
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += ld(rowp[r], (size_t)k) * xs[k];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) out[r] = wave_sum(acc[r]);
}

template <typename WT, int EPI, bool VEC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_k(GemvArgs a) {
    extern __shared__ float xs[];
    __shared__ float red[16];
    gemv_stage_x(a, xs, red);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const WT *W = (const WT *)a.w;
    if (EPI == GEMV_SWIGLU) {
        const WT *W2 = (const WT *)a.w2;
        for (int n = blockIdx.x * GEMV_WAVES + wave; n < a.N; n += gridDim.x * GEMV_WAVES) {
            const WT *rp[2] = {W + (size_t)n * a.K, W2 + (size_t)n * a.K};
            float gu[2];
            gemv_rows<WT, 2, VEC>(rp, a.K, xs, gu);
            if (lane == 0) a.y[n] = silu(gu[0]) * gu[1];
        }
        return;
    }
    constexpr int R = 2;
    for (int n0 = (blockIdx.x * GEMV_WAVES + wave) * R; n0 < a.N;
         n0 += gridDim.x * GEMV_WAVES * R) {
        const WT *rp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) rp[r] = W + (size_t)min(n0 + r, a.N - 1) * a.K;
        float v[R];
        gemv_rows<WT, R, VEC>(rp, a.K, xs, v);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int n = n0 + r;
                if (n >= a.N) break;
                float y = a.bias ? v[r] + a.bias[n] : v[r];
                if (EPI == GEMV_RESIDUAL) a.y[n] = a.y[n] + y;
                else a.y[n] = y;
            }
        }
    }
}

template <typename WT, int EPI>
static void gemv_launch(const GemvArgs &a, hipStream_t s) {
    int dev_cus = 256;
    int rows_per_block = GEMV_WAVES * (EPI == GEMV_SWIGLU ? 1 : 2);
    int blocks = (a.N + rows_per_block - 1) / rows_per_block;
    int cap = 4 * dev_cus;
    if (blocks > cap) blocks = cap;
    size_t shm = sizeof(float) * (size_t)a.K;
    static bool attr_set[2] = {false, false};
    if (shm > 64 * 1024) {
        for (int v = 0; v < 2; ++v)
            if (!attr_set[v]) {
                ESP_HIP(hipFuncSetAttribute(
                    v ? (const void *)gemv_k<WT, EPI, true> : (const void *)gemv_k<WT, EPI, false>,
                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 256));
                attr_set[v] = true;
            }
    }
    bool vec = (a.K * sizeof(WT)) % 16 == 0 && ((uintptr_t)a.w % 16) == 0 &&
               (!a.w2 || ((uintptr_t)a.w2 % 16) == 0);
    if (vec)
        gemv_k<WT, EPI, true><<<blocks, GEMV_THREADS, shm, s>>>(a);
    else
        gemv_k<WT, EPI, false><<<blocks, GEMV_THREADS, shm, s>>>(a);
}

void launch_gemv(Dt wt, GemvEpi epi, const GemvArgs &a, hipStream_t s) {
    if ((size_t)a.K * 4 > 160 * 1024) fail(ESP_UNSUPPORTED, "gemv: input width above 40960");
    if (wt == DT_BF16) {
        if (epi == GEMV_STORE) gemv_launch<uint16_t, GEMV_STORE>(a, s);
        else if (epi == GEMV_RESIDUAL) gemv_launch<uint16_t, GEMV_RESIDUAL>(a, s);
        else gemv_launch<uint16_t, GEMV_SWIGLU>(a, s);
    } else {
        if (epi == GEMV_STORE) gemv_launch<float, GEMV_STORE>(a, s);
        else if (epi == GEMV_RESIDUAL) gemv_launch<float, GEMV_RESIDUAL>(a, s);
        else gemv_launch<float, GEMV_SWIGLU>(a, s);
    }
}

}  // namespace esp
