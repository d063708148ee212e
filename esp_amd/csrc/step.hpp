// Persistent single-token decode step (k_step.hip).
#pragma once

#include "common.hpp"

namespace esp {

// Per-layer weights as the step kernel reads them (device array).
struct StepLayer {
    const void *qkv;          // [qkv_rows, H] q | k | v | LoRA-A rows
    const float *qkv_bias;    // [qkv_rows] or null
    const float *in_norm, *post_norm;
    const void *o;            // [H, qw]
    const float *o_bias;      // [H] or null
    const void *gate, *up, *down;
    const void *lora_b[3];    // B_j [out_j, rank_j] (targets q, k, v) or null
    int lora_rank[3], lora_t_col[3];
    float lora_scale[3];
    int lora_rows;            // LoRA-A rows after q | k | v (0 = none)
    int window;               // sliding window (0 = none)
};

struct StepArgs {
    const StepLayer *layers;
    int L, H, F, V, nq, nkv, hd;
    float eps;
    const void *embed, *head;
    const float *final_norm;
    const float *rope_cos, *rope_sin;
    // the row: token id, sequence, position (device)
    const int32_t *ids, *row_seq, *row_pos;
    // f32 KV cache: [seq][layer][K|V][kv head][max_ctx][hd]
    float *kv;
    long long seq_stride, layer_stride, kv_half_stride, head_stride;
    // scratch vectors
    float *h, *t, *q, *attn, *act, *part, *logits;
    int n_split, split_len;
    int nch_h, nch_q, nch_f;  // 8-element chunks per lane for K = H, qw, F
    // head argmax (gen nullable: logits only)
    float *part_v;
    int32_t *part_i;
    uint32_t *picked;
    int32_t *gen;
    unsigned *bar;  // barrier state, STEP_BAR_WORDS zeroed words
};

constexpr int STEP_BAR_WORDS = 512;
constexpr int ATT_MAX_SPLIT_STEP = 128;  // key splits the step kernel merges

// 8-element chunks per lane for a GEMV phase of width K (1, 2, 4 or 8)
int step_nch(int K);

// The step kernel serves bf16 dense models with head_dim 64 or 128, query
// groups up to 8, no QK norm, and widths its GEMV phases cover.
bool step_ok(int hd, int G, int H, int qw, int F, bool qk_norm, bool moe, Dt wt);
// Splits of the attention phase for `max_t` keys (resident blocks / kv heads).
int step_attn_splits(int hd, int G, int nkv, int max_t, int *split_len);
void launch_step(const StepArgs &a, int G, hipStream_t s);

}  // namespace esp
