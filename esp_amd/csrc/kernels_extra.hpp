// Launchers for the fill, routed-expert and GEMM helper kernels.
#pragma once

#include "common.hpp"

namespace esp {

struct Model;
struct Kv;
struct LayerW;

// value[i] = std * N(0,1) from a splitmix64 counter stream and Box-Muller.
void launch_fill_normal(Dt dt, void *dst, size_t n, uint64_t seed, float std, hipStream_t s);
void launch_fill_const(float *dst, size_t n, float v, hipStream_t s);
void launch_fill_bits(uint16_t *dst, size_t n, uint16_t bits, hipStream_t s);

void launch_gemm_simple(Dt wt, GemmEpi epi, const GemmArgs &a, hipStream_t s);

// moe.rs:156-181 routing on the device.
struct RouteArgs {
    const float *logits;  // [M, E]
    int M, E, k;
    int norm_topk;
    int32_t *sel;    // [M, k] selected experts, ascending id
    float *w;        // [M, k] matching weights
    int32_t *offs;   // [E + 1] expert row offsets; offs[E + 1] = status
    int32_t *perm;   // [M * k] token of each grouped row
    int32_t *slot;   // [M, k] grouped row of each selection
    int32_t *err;    // nullable sticky status word: max(2 non-finite router, 3 bad top-k mass)
    // nullable: the device generation loop's step counter (emitted tokens so
    // far); a failing route then also records min(step << 2 | status) in err[1]
    const int32_t *step;
};
void launch_route(const RouteArgs &a, hipStream_t s);
void launch_gather_rows(Dt dt, const void *src, const int32_t *perm, int rows, int H, void *dst,
                        hipStream_t s);
struct CombineArgs {
    const float *y;      // [M * k, H] grouped expert outputs
    const int32_t *slot; // [M, k]
    const float *w;      // [M, k]
    const float *ys;     // nullable [M, H] shared expert output
    const float *sg;     // nullable [M] shared gate logit
    float *h;            // [M, H] residual stream (+=)
    int M, k, H;
};
void launch_combine(const CombineArgs &a, hipStream_t s);

void moe_block(Model &m, Kv &kv, LayerW &w, int Mc, hipStream_t s, int l);
// one decode row through the routed experts without host round trips
bool moe_decode_ok(const Model &m);
void moe_decode(Model &m, Kv &kv, LayerW &w, hipStream_t s);

}  // namespace esp
