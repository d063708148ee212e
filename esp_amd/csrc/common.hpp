// Internal declarations shared by the host runtime and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/esp_hip.h"

namespace esp {

struct Error {
    esp_status code;
    std::string msg;
};

[[noreturn]] inline void fail(esp_status code, std::string msg) { throw Error{code, std::move(msg)}; }

#define ESP_HIP(x)                                                                         \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess)                                                              \
            ::esp::fail(ESP_BACKEND, std::string(#x) + ": " + hipGetErrorString(e_));     \
    } while (0)

typedef uint16_t bf16_t;  // raw bf16 bits in host code

// Element kinds. DT_SPLIT is an f32 activation matrix stored as two bf16
// planes of the same shape, hi = bf16(x) then lo = bf16(x - hi), so matrix
// cores can consume it exactly (R x C matrix: hi[r*C+c], lo[R*C + r*C+c]).
// DT_Q8 / DT_Q4: packed projection weights, signed 8- or 4-bit integers
// along K with one f32 scale per 32 inputs (values, then the scales).
// DT_F16: IEEE binary16 (the K/V cache of the bf16 and packed formats).
enum Dt { DT_F32 = 0, DT_BF16 = 1, DT_SPLIT = 2, DT_Q8 = 3, DT_Q4 = 4, DT_F16 = 5 };

inline size_t dt_size(Dt d) { return d == DT_BF16 || d == DT_F16 ? 2 : 4; }
inline bool dt_packed(Dt d) { return d == DT_Q8 || d == DT_Q4; }
// bytes of the packed values of n weights (n a multiple of 32)
inline size_t packed_value_bytes(Dt d, size_t n) { return d == DT_Q8 ? n : n / 2; }

// ---------------------------------------------------------------------------
// Kernel launch interfaces (implemented in the .hip files). Every launcher
// takes the stream explicitly; shapes are validated by the caller.

// Row descriptors of one forward: token row r belongs to sequence
// row_seq[r] at absolute position row_pos[r].
struct Rows {
    const int32_t *ids;      // [M]
    const int32_t *row_seq;  // [M]
    const int32_t *row_pos;  // [M]
    int M;
    int seq1 = -1;           // >= 0: every row belongs to this sequence
    // nullable: groups of consecutive rows of one sequence (consecutive
    // positions), row0 | (rows << 16) each, for attention kernels that read
    // a sequence's keys once per group
    const int32_t *grp = nullptr;
    int ngrp = 0;
    int grp_rows = 0;        // rows per full group
};

// h[M,H] (f32) = embed[ids[m]] (wt)
void launch_embed(Dt wt, const void *embed, const int32_t *ids, int M, int H, float *h,
                  hipStream_t s);

// out[M,H] (dt out) = x / sqrt(mean(x^2)+eps) * gamma ; rows selected by
// row_index (nullable = identity).
// x[m] += bias + sum_z ws[z][m] (the split-K partials of a RESIDUAL
// projection, summed in split order as the GEMM reduction does), then
// out = RMSNorm(x[m]) * gamma in out_dt (DT_SPLIT: hi/lo planes of M rows).
// H <= 8192, H % 4 == 0 (resid_norm_ok).
bool resid_norm_ok(int H);
void launch_resid_norm(const float *ws, int splits, int M, int H, const float *bias, float *x,
                       const float *gamma, float eps, Dt out_dt, void *out, hipStream_t s);
void launch_rmsnorm(const float *x, const float *gamma, float eps, int M, int H, Dt out_dt,
                    void *out, const int32_t *row_index, hipStream_t s);

// GEMV (one input row): y = W x with the input RMS-normalised on the fly
// when gamma != nullptr. Epilogue kinds below.
enum GemvEpi { GEMV_STORE = 0, GEMV_RESIDUAL = 1, GEMV_SWIGLU = 2 };
struct GemvArgs {
    const void *w;     // [N, K] wt (SWIGLU: gate rows)
    const void *w2;    // SWIGLU: up rows [N, K]
    const float *x;    // [K] f32
    const float *gamma;  // nullable: fused RMSNorm of x
    float eps;
    const float *bias;   // nullable [N]
    float *y;            // STORE/SWIGLU: out [N]; RESIDUAL: y[n] += result
    int N, K;
};
void launch_gemv(Dt wt, GemvEpi epi, const GemvArgs &a, hipStream_t s);

// GEMM (several input rows): C[M,N] = A[M,K] * W[N,K]^T with f32 activations
// A, weights W in the model format, f32 accumulation.
enum GemmEpi { GEMM_STORE = 0, GEMM_RESIDUAL = 1, GEMM_SWIGLU = 2 };
struct GemmArgs {
    const void *a;     // [M, K] act: f32, or the hi plane of a split matrix
    const void *a_lo;  // lo plane of a split A (nullable = A is f32)
    const void *w;     // [N, K] wt
    const void *w2;    // SWIGLU up rows
    const float *bias; // nullable [N]
    void *c;           // STORE: f32 [M, ldc]; RESIDUAL: f32 +=; SWIGLU: f32 [M, ldc] or hi plane
    void *c_lo;        // SWIGLU only: lo plane of a split output (nullable = f32 out)
    int M, N, K, ldc;
    float *ws;         // nullable split-K workspace
    size_t ws_bytes;
    // Grouped launch (routed experts): the M rows are grp_n consecutive
    // groups with row offsets grp_offs[0..grp_n] (device, ascending, written
    // by the router on the stream, never read by the host); group e
    // multiplies W + e * grp_w_stride (and W2 likewise, elements). The grid
    // is sized for ceil(M / tile rows) + grp_n row tiles; the ones past the
    // groups' last tile exit. nullptr = one group of M rows.
    const int32_t *grp_offs;
    int grp_n;
    long long grp_w_stride;
    // Nullable host word. When set, a launch that splits K leaves the
    // partial sums in ws ([splits][M][N] f32) and stores the split count
    // here instead of running the reduction and epilogue (the consumer sums
    // them, in split order); a launch without splits applies the epilogue and
    // stores 0.
    int *defer_splits;
    // Doubled-K packed form (0 = off; the streamed GEMM of >= 1024 rows
    // only): the weights are [N, K] rows [hi | lo] with K = 2 kdup, the A
    // planes stay [M, kdup] and are read again for keys kdup .. K, and the
    // lo plane multiplies only keys below kdup, so the products are
    // a_hi w_hi + a_lo w_hi + a_hi w_lo without a widened copy of A.
    int kdup;
    // Tile order of the streamed GEMM (set by its launcher): the XCD-major
    // tile ranges walk bands of this many weight-column tiles, row tiles
    // within a band (1 = column-major).
    int band;
};
void launch_gemm(Dt wt, GemmEpi epi, const GemmArgs &a, hipStream_t s);

// QKV post-processing: LoRA B-adds, optional QK RMSNorm, RoPE at each row's
// position, K/V append into the cache, q written as f32 [M, nq, hd].
struct RopeKvArgs {
    const float *qkv;   // [M, ldq] raw projection (+bias): q | k | v | lora t
    int ldq;
    float *q_out;       // [M, nq*hd] f32
    const float *rope_cos, *rope_sin;  // [max_pos, hd]
    const float *q_norm, *k_norm;      // nullable [hd]
    float eps;
    // LoRA: t for target j at qkv column lora_t_col[j] (rank lora_rank[j]),
    // B_j [out, rank] (wt), scale lora_scale[j]; targets 0 q, 1 k, 2 v.
    const void *lora_b[3];
    int lora_t_col[3], lora_rank[3];
    float lora_scale[3];
    Rows rows;
    void *kv;           // cache base (kv dt)
    long long seq_stride, layer_stride, kv_half_stride, head_stride;  // elements
    int nq, nkv, hd;
    // Nullable: the q/k/v projection's split-K partial sums [splits][M][ldq]
    // (qkv is then unread), summed in split order, + part_bias (nullable).
    // Pair form only (rope_kv_fusable).
    const float *part;
    int splits;
    const float *part_bias;
};
// Whether launch_rope_kv takes `part` for these shapes: the pair form's
// dtype pairs, head_dim 64 (even head counts) or 128, and no LoRA adapter
// (its t columns are read raw).
bool rope_kv_fusable(Dt wt, Dt kvdt, int hd, int nq, int nkv, bool lora);
void launch_rope_kv(Dt wt, Dt kvdt, const RopeKvArgs &a, hipStream_t s);

// Attention over the cache for each row (causal, optional sliding window).
struct AttnArgs {
    const float *q;     // [M, nq*hd] f32 (post RoPE)
    const void *kv;     // cache base
    long long seq_stride, layer_stride, kv_half_stride, head_stride;
    Rows rows;
    int nq, nkv, hd, window;  // window 0 = none
    float *part;        // scratch partials
    int n_split, split_len;
    void *out;          // [M, nq*hd] out dt (DT_SPLIT: planes of M rows)
    Dt out_dt;
};
void launch_attention(Dt kvdt, const AttnArgs &a, hipStream_t s);

// Token pick over logits rows.
struct PickArgs {
    const float *logits;  // [n, V]
    int n, V;
    const uint32_t *allowed;  // nullable [n, ceil(V/32)]
    const esp_sampler *samplers;  // nullable device copy [n]
    uint32_t *ids_out;     // [n]
    uint8_t *flags_out;    // [n]
    uint64_t *state_out;   // [n] advanced sampler states
    void *scratch;         // sampling scratch
    size_t scratch_bytes;
    int direct_max;        // set by launch_pick: rows with more listed ids take the bucketed path
};
void launch_pick(const PickArgs &a, hipStream_t s);
size_t pick_scratch_bytes(int n, int V);
// esp_pick_noalloc: the pick over device inputs and outputs with all scratch
// in the library's fixed device array (k_pick_fixed.hip).
void launch_pick_fixed(int device, const float *logits, int n, int V, const uint32_t *allowed_dev,
                       esp_sampler *samplers_dev, uint32_t *ids_dev, uint8_t *flags_dev,
                       hipStream_t s);

// Packed weights: out[i] = q_i * scale[i / 32] in f32 (n a multiple of 32).
// Packed [N, K] -> bf16 [N, 2K] rows [hi(q*scale) | lo(q*scale)], and split
// activation planes [M, K] -> [M, 2K] ([hi | hi], [lo | 0]): the doubled-K
// form of a packed projection for the bf16 matrix-core GEMM.
void launch_dequant_split(Dt wt, const void *values, const float *scales, size_t N, size_t K,
                          uint16_t *out, hipStream_t s);
void launch_widen_split(const uint16_t *hi, const uint16_t *lo, size_t M, size_t K, uint16_t *hi2,
                        uint16_t *lo2, hipStream_t s);
void launch_dequant(Dt wt, const void *values, const float *scales, size_t n, float *out,
                    hipStream_t s);
// decoder/weight_format.rs:150-183 on the device: rows x cols f32 (cols a
// multiple of 32) to packed values + block scales.
void launch_quantize(Dt wt, const float *src, size_t rows, size_t cols, void *values,
                     float *scales, hipStream_t s);

// Device-side generation hand-off (see k_basic.hip).
void launch_gen_step(const uint32_t *picked, int32_t *gen, hipStream_t s);

}  // namespace esp
