/*
 * esp_oracle.h — CPU restatement of esp's llama-family decoder forward
 * (the burn-ndarray "f32 corridor": every weight widened exactly to f32,
 * all arithmetic in f32).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the
 * HIP path in esp_amd/ and the CPU baseline timed by bench.py. Nothing
 * in the product (esp_amd/, include/) may link, load or call it.
 *
 * Reference files restated (paths relative to merely-made/esp,
 * crates/esp/src/infer/decoder/):
 *   config.rs:158-180      RopeScaling::apply
 *   attention.rs:58-124    LlamaRotaryEncoding::{with_scaling, apply}
 *   attention.rs:126-153   LayerKvCache::append
 *   attention.rs:292-404   DecoderAttention::forward_cached_chunked
 *   layer.rs:115-153       DecoderLayer::forward_cached_chunked
 *   moe.rs:76-90,135-256   Expert / DecoderMlp::forward
 *   model.rs:502-666       try_forward_cached_last / forward_cached_hidden
 *   lora.rs:93-97          add_delta
 *   generate.rs:70-79      argmax_last; provider.rs:808-815 constrained greedy
 *   sample.rs:21-121       SplitMix64, Sampler::{sample, skip_draws}
 *   constraint.rs:277-297  Constraint::mask
 */
#ifndef ESP_ORACLE_H
#define ESP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1 };

typedef struct {
    const void *data; /* NULL = absent */
    int32_t dtype;    /* ORC_F32 or ORC_BF16 (raw little-endian bf16 bits) */
    int32_t pad;
} orc_tensor;

/* Per-layer tensor slots, HF [out, in] orientation for projections. */
enum {
    ORC_IN_NORM = 0,
    ORC_Q, ORC_K, ORC_V, ORC_O,
    ORC_Q_BIAS, ORC_K_BIAS, ORC_V_BIAS, ORC_O_BIAS,
    ORC_Q_NORM, ORC_K_NORM,
    ORC_POST_NORM,
    ORC_GATE, ORC_UP, ORC_DOWN,               /* dense MLP */
    ORC_ROUTER, ORC_SHARED_GATE,              /* MoE router [E,H], shared gate [1,H] */
    ORC_SH_GATE, ORC_SH_UP, ORC_SH_DOWN,      /* MoE shared expert (absent = none) */
    ORC_LAYER_SLOTS
};

typedef struct {
    int32_t hidden, layers, n_heads, n_kv_heads, head_dim, ffn, vocab, max_pos;
    float rms_eps;
    int32_t qkv_bias, o_bias, qk_norm;
    int32_t n_experts, top_k, moe_ffn, shared_ffn, norm_topk;
    const int32_t *layer_is_moe;  /* [layers] */
    const int32_t *layer_window;  /* [layers]; 0 = no sliding window */
    const float *rope_cos;        /* [max_pos, head_dim] (orc_rope_table) */
    const float *rope_sin;
    orc_tensor embed, final_norm, lm_head; /* lm_head.data NULL = tied */
    const orc_tensor *layer;      /* [layers][ORC_LAYER_SLOTS] */
    const orc_tensor *experts;    /* [layers][n_experts][3] gate, up, down; may be NULL */
} orc_model;

typedef struct orc_kv orc_kv;

/* RoPE table, attention.rs:58-95 + config.rs:158-180.
 * scaling: 0 none, 1 linear(factor), 2 llama3(factor, low, high, orig). */
void orc_rope_table(int max_pos, int head_dim, float theta, int scaling,
                    float factor, float low_freq, float high_freq, int orig_max,
                    float *cos_out, float *sin_out);

orc_kv *orc_kv_create(const orc_model *m, int max_ctx);
void orc_kv_destroy(orc_kv *kv);
int orc_kv_position(const orc_kv *kv);
/* Fill the whole cache with seeded values and set its position (timing of
 * long-context decode without running the prefill). */
void orc_kv_fill_synthetic(orc_kv *kv, int position, uint64_t seed);

/* model.rs:502-539: forward `n` ids at the cache position, extend the
 * cache, write last-position logits [vocab] (f32). all_logits (nullable)
 * receives [n, vocab] logits for every position (test-only convenience).
 * Returns 0, or -1 for empty / over-window input (model.rs:548-556),
 * -2 for a non-finite router row (moe.rs:162-164), -3 for invalid top-k
 * mass (moe.rs:175-177), -4 allocation failure. */
int orc_forward_last(const orc_model *m, orc_kv *kv, const int32_t *ids, int n,
                     float *logits_out, float *all_logits);

/* lora.rs:93-97: out[o][i] = base[o][i] + (sum_r A[r][i] * B[o][r]) * scale,
 * HF orientation, A [rank, in], B [out, rank], all f32 (base may be bf16). */
void orc_lora_merge(orc_tensor base, const float *a, const float *b, int out_f,
                    int in_f, int rank, float scale, float *merged);

/* generate.rs:70-79 and provider.rs:808-815: greedy, lowest id wins ties. */
int32_t orc_argmax(const float *row, int n);

/* constraint.rs:277-297 with an allowed-token bitmask (bit id of word id/32):
 * disallowed or non-finite -> -inf. Returns number of eligible tokens. */
int orc_mask(float *row, int n, const uint32_t *allowed_bits);

/* sample.rs:21-52 splitmix64 */
uint64_t orc_splitmix64_next(uint64_t *state);
/* sample.rs:64-69 */
uint64_t orc_skip_draws(uint64_t state, uint64_t draws);
/* sample.rs:83-121; ties in the sort are ordered by ascending id.
 * top_p < 0 means None. Advances *state by one draw. */
int32_t orc_sample(const float *row, int n, float temperature, float top_p, uint64_t *state);

/* Test-input generator: splitmix64 counter stream + Box-Muller,
 * value[i] = std * N(0,1); out is f32 or bf16 (round-to-nearest-even). */
void orc_fill_normal(uint64_t seed, size_t n, float std, int dtype, void *out);

void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
