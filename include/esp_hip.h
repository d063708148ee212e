/*
 * esp_hip.h — C ABI of the MI355X (gfx950) llama-family decoder forward.
 *
 * This is the drop-in boundary for esp's model-execution seam. Each entry
 * point names the reference interface it replaces (paths relative to
 * merely-made/esp, crates/esp/src/infer/). Plain pointers and sizes only;
 * no C++ exception crosses the boundary; every call returns an esp_status
 * whose values are 1:1 with the reference's InferError variants
 * (provider.rs:160-183), with the message available from esp_last_error.
 *
 * Threading: a model is immutable after load and may be shared by threads.
 * A KV handle binds one HIP stream and is owned by one caller at a time
 * (the reference's `&mut KvCache`). Calls are synchronous: when one returns,
 * its outputs are in host memory (or, for device-resident logits, complete
 * on the KV handle's stream).
 */
#ifndef ESP_HIP_H
#define ESP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* InferError (provider.rs:160-183) as status codes. */
typedef enum esp_status {
    ESP_OK = 0,
    ESP_PROMPT_TOO_LONG = 1,   /* PromptTooLong { length, limit } */
    ESP_MODEL_NOT_LOADED = 2,  /* ModelNotLoaded */
    ESP_INTERRUPTED = 3,       /* Interrupted */
    ESP_BACKEND = 4,           /* Backend(String): a HIP failure */
    ESP_STAGE_UNAVAILABLE = 5, /* StageUnavailable(String) */
    ESP_INVALID_REQUEST = 6,   /* InvalidRequest(String) */
    ESP_INVALID_CONFIG = 7,    /* InvalidConfig(String) */
    ESP_INVALID_WEIGHTS = 8,   /* InvalidWeights(String) */
    ESP_UNSUPPORTED = 9        /* Unsupported { feature, detail }: "feature: detail" */
} esp_status;

/* Weight storage/compute format (decoder/weight_format.rs:22-32):
 * F32 widens every checkpoint tensor to f32 (the reference's default
 * corridor); BF16 keeps bf16 weights in HBM, bf16 MFMA inputs, f32
 * accumulation and an f32 residual stream; its artifacts must be BF16
 * (weight_format.rs:283-291). Q8_BLOCK32 / Q4_BLOCK32
 * ("q8-k32-f32-scale-f16-shared-v1" / "q4-..."): every projection is a U8
 * tensor of packed signed 8- or 4-bit values along K plus one f32 scale per
 * 32 inputs (weight_format.rs:138-223, 225-273), every other tensor F16;
 * decode GEMVs read the packed bytes and dequantize in registers,
 * activations stay f32. Dense llama-family layers only (no routed experts,
 * no unmerged LoRA: ESP_UNSUPPORTED). */
typedef enum esp_format {
    ESP_FORMAT_F32 = 0,
    ESP_FORMAT_BF16 = 1,
    ESP_FORMAT_Q8_BLOCK32 = 2,
    ESP_FORMAT_Q4_BLOCK32 = 3
} esp_format;

typedef enum esp_rope_scaling {
    ESP_ROPE_NONE = 0,
    ESP_ROPE_LINEAR = 1, /* config.rs:158-160 */
    ESP_ROPE_LLAMA3 = 2  /* config.rs:161-178 */
} esp_rope_scaling;

/* Parsed decoder geometry: DecoderConfig (decoder/config.rs:322-363) with
 * its derived values (config.rs:433-490) already resolved by the host. */
typedef struct esp_config {
    uint32_t vocab_size;
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_hidden_layers;
    uint32_t num_attention_heads;
    uint32_t num_key_value_heads; /* kv_heads() */
    uint32_t head_dim;            /* head_dim() */
    uint32_t max_position_embeddings;
    float rms_norm_eps;
    float rope_theta;
    uint32_t rope_scaling; /* esp_rope_scaling */
    float rope_factor;
    float rope_low_freq_factor;
    float rope_high_freq_factor;
    uint32_t rope_original_max_position_embeddings;
    uint32_t tie_word_embeddings;
    uint32_t qkv_bias;    /* qkv_bias() */
    uint32_t output_bias; /* output_bias() */
    uint32_t qk_norm;     /* qk_norm() */
    const uint32_t *layer_window; /* [layers] layer_window(i), 0 = none; NULL = none */
    /* Routed experts (MoeConfig, config.rs:37-48); num_experts 0 = dense. */
    uint32_t num_experts;
    uint32_t num_experts_per_tok;
    uint32_t moe_intermediate_size;
    uint32_t shared_expert_intermediate_size; /* 0 = no shared expert */
    uint32_t norm_topk_prob;
    const uint8_t *layer_is_moe; /* [layers] layer_is_moe(i); NULL = none */
    uint32_t format;             /* esp_format */
} esp_config;

/* One PEFT LoRA adapter (decoder/lora.rs:99-217), applied unmerged as
 * y += scale * B (A x) for each targeted attention projection. */
typedef struct esp_lora {
    uint32_t rank;
    float scale;          /* alpha / rank * selection scale (lora.rs:194) */
    uint32_t target_mask; /* bit 0 q_proj, 1 k_proj, 2 v_proj, 3 o_proj */
    const uint8_t *safetensors; /* base_model.model.model.layers.{i}.self_attn.{m}.lora_{A,B}.weight */
    size_t safetensors_len;
} esp_lora;

/* Sampler state (decoder/sample.rs:56-122). temperature <= 0 selects
 * greedy (generate.rs:70-79; constrained greedy provider.rs:808-815);
 * top_p < 0 means None. `state` is the splitmix64 state: seed plus
 * 0x9E3779B97F4A7C15 * draws (sample.rs:64-69); esp_pick advances it by
 * one draw for each sampled row. */
typedef struct esp_sampler {
    float temperature;
    float top_p;
    uint64_t state;
} esp_sampler;

/* esp_pick per-row flags */
#define ESP_PICK_NONFINITE 1u   /* the row held NaN/inf logits (provider.rs:219-240) */
#define ESP_PICK_NO_ELIGIBLE 2u /* no finite allowed token (constraint.rs:292-294) */

typedef struct esp_model esp_model;
typedef struct esp_kv esp_kv;

/* Thread-local message of the last failing call on this thread. Returns
 * the full message length; copies at most len-1 bytes plus a NUL. */
size_t esp_last_error(char *buf, size_t len);

/* decoder/loader.rs:573-580 load_decoder_from_bytes + model.rs:166-194
 * DecoderModel::from_loaded (+ lora.rs:260-307 when adapters are given).
 * `safetensors` holds HF-named tensors (loader.rs:36-64); it is borrowed
 * for the duration of the call only. Unconsumed tensors are refused
 * (loader.rs:277-308); lm_head.weight may be absent only when tied
 * (loader.rs:438-446). Weights are staged into HBM on the current device. */
esp_status esp_model_load(const esp_config *config, const uint8_t *safetensors, size_t len,
                          const esp_lora *adapters, uint32_t n_adapters, esp_model **out);
/* Synthetic model of the given geometry (no reference counterpart; used by
 * benchmarks and large-shape tests): every projection, expert and
 * embedding is N(0, std) from a seeded device generator, norms are 1 and
 * biases 0. lora_rank > 0 adds unmerged LoRA on the projections in
 * lora_mask (bit 0 q, 1 k, 2 v) with A ~ N(0, lora_a_std),
 * B ~ N(0, lora_b_std) and the given scale. */
esp_status esp_model_create_synthetic(const esp_config *config, uint64_t seed, float std,
                                      uint32_t lora_rank, uint32_t lora_mask, float lora_a_std,
                                      float lora_b_std, float lora_scale, esp_model **out);
esp_status esp_model_destroy(esp_model *model);
/* Bytes of HBM the model's weights occupy. */
esp_status esp_model_weight_bytes(const esp_model *model, uint64_t *bytes);

/* model.rs:476-483 DecoderModel::new_cache, for `batch` independent
 * sequences of up to `max_ctx` positions each (max_ctx <=
 * max_position_embeddings). Contiguous per-sequence f32 keys and values
 * (every weight format). */
esp_status esp_kv_create(esp_model *model, uint32_t batch, uint32_t max_ctx, esp_kv **out);
/* esp_kv_create with options. ESP_KV_F16 (bf16 weights only, else
 * ESP_UNSUPPORTED): keys and values stored as IEEE half, half the cache
 * bytes. No reference counterpart: the reference's cache holds the
 * activation dtype. Half precision stays within the bf16-config tolerance
 * of the f32 corridor on 16-layer 1B-shape models but not on 32-layer
 * 8B-shape ones (CPU emulation of random-init models), so it is for
 * callers that trade that margin for cache capacity and bandwidth. */
#define ESP_KV_F16 1u
esp_status esp_kv_create_ex(esp_model *model, uint32_t batch, uint32_t max_ctx, uint32_t flags,
                            esp_kv **out);
esp_status esp_kv_destroy(esp_kv *kv);
/* Forget sequence `seq` (or every sequence when seq == UINT32_MAX). */
esp_status esp_kv_reset(esp_kv *kv, uint32_t seq);
/* model.rs:676-681 KvCache::position */
esp_status esp_kv_position(const esp_kv *kv, uint32_t seq, uint32_t *position);
/* The HIP stream (hipStream_t) this KV handle's work runs on. */
esp_status esp_kv_stream(const esp_kv *kv, void **stream);
/* Device address of the last forward's logits rows on this handle
 * (row-major f32 [n_rows][vocab], valid until the next forward; NULL and 0
 * before any forward), so a caller can read or post-process scores in
 * place on the handle's stream before esp_pick. Stands where the reference
 * hands its logits tensor to the provider (model.rs:502-539 return value,
 * provider.rs:744-760 row read); the provider's test-only score faults
 * (provider.rs:70-71, 755-762) are injected through it. */
esp_status esp_kv_logits(esp_kv *kv, float **rows_dev, uint32_t *n_rows);
/* (esp_kv_logits returns once the last forward on the handle has finished.) */

/* model.rs:502-539 try_forward_cached_last for one sequence: consume `n`
 * ids at the sequence's position, extend its cache, and leave the
 * last-position logits (f32, [vocab]) device-resident as row 0 for
 * esp_pick; also copy them to `logits_out` when it is non-NULL.
 * Empty, out-of-vocabulary or over-window input -> ESP_INVALID_REQUEST
 * (model.rs:548-556) and the cache is unchanged. */
esp_status esp_forward_last(esp_model *model, esp_kv *kv, uint32_t seq, const int32_t *ids,
                            uint32_t n, float *logits_out);

/* The same forward for several sequences at once: sequence seqs[i]
 * consumes seq_lens[i] ids (ids concatenated in order). Decode steps are
 * seq_len 1; grammar-forced spans are short blocks over a warm cache
 * (provider.rs:865-872). Each sequence's result equals its own
 * esp_forward_last. Last-position logits land as rows 0..n_seqs-1.
 * Without logits_out the call may return while the pass still runs on the
 * handle's stream (esp_kv_stream): every later call on the handle is
 * ordered after it, esp_kv_logits waits for it, and a device failure of the
 * pass is reported by the next call that waits (esp_pick). Passes that must
 * read back a status (routed experts, streamed layers, split-merging
 * attention) still finish before returning. */
esp_status esp_forward_batch(esp_model *model, esp_kv *kv, uint32_t n_seqs, const uint32_t *seqs,
                             const uint32_t *seq_lens, const int32_t *ids, float *logits_out);

/* Token choice over the device-resident logits rows of the last forward
 * on this KV handle (generate.rs:30-44 TokenPicker::pick,
 * provider.rs:807-816). allowed_bits (nullable) holds one bitmask of
 * ceil(vocab/32) u32 words per row (bit id%32 of word id/32 = allowed);
 * with a mask, disallowed or non-finite logits become -inf
 * (constraint.rs:277-297). samplers (nullable = greedy for every row).
 * ids_out[n_rows]; flags_out[n_rows] (nullable) gets ESP_PICK_* bits.
 * Returns ESP_INVALID_REQUEST if a masked row has no eligible token. */
esp_status esp_pick(esp_kv *kv, uint32_t n_rows, const uint32_t *allowed_bits,
                    esp_sampler *samplers, uint32_t *ids_out, uint8_t *flags_out);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory: code under HIP stream capture, serving loops and harnesses that
 * forbid hipMalloc. esp_pick with every input and output in device memory
 * and no device allocation, synchronisation or host copy: allowed_bits_dev
 * (nullable) as esp_pick's allowed_bits; samplers_dev (nullable) whose
 * sampled rows' states advance in place, exactly as esp_pick advances
 * them (not for a row with no eligible token); ids_dev[n_rows];
 * flags_dev[n_rows] (nullable) gets the ESP_PICK_* bits. It is enqueued on
 * the KV handle's stream and returns without waiting, so a row with no
 * eligible token is reported only in flags_dev. All scratch lives in one
 * fixed device array of ESP_PICK_NOALLOC_SCRATCH_BYTES per GPU (held from
 * library load until the process ends); rows x vocabulary needing more
 * (about 30 MiB for 16 sampled rows of a 128256-token vocabulary) ->
 * ESP_INVALID_REQUEST. Calls that overlap on one GPU race on that array. */
#define ESP_PICK_NOALLOC_SCRATCH_BYTES (32u << 20)
esp_status esp_pick_noalloc(esp_kv *kv, uint32_t n_rows, const uint32_t *allowed_bits_dev,
                            esp_sampler *samplers_dev, uint32_t *ids_dev, uint8_t *flags_dev);

/* generate.rs:134-170 try_generate_ids_with + TokenPicker::Greedy, run on
 * the device: prefill `prompt`, then up to max_new greedy steps, stopping
 * at (and excluding) any id in `eos`. Writes generated ids to out_ids and
 * their count to n_out; at most min(max_new, W - n_prompt + 1) ids, where
 * W = min(the KV handle's max_ctx, max_position_embeddings), so out_ids
 * needs that many slots (any max_new, up to UINT32_MAX, is accepted). A
 * run that yields that many ids without eos while max_new asks for more
 * fails as the reference's next forward past the window does. The
 * per-step token never leaves the device; decode steps replay one
 * captured HIP graph in chunks of 4, 8, 16, 32 and then 64 forwards, the
 * host checking the new ids for eos between chunks, so an early eos ends
 * the call after at most the rest of its chunk. A router failure counts
 * only in a forward the reference runs (one feeding a token before eos). */
esp_status esp_generate_greedy(esp_model *model, esp_kv *kv, uint32_t seq, const int32_t *prompt,
                               uint32_t n_prompt, uint32_t max_new, const int32_t *eos,
                               uint32_t n_eos, int32_t *out_ids, uint32_t *n_out);

/* ---- Layer streaming (decoder/streaming.rs, model.rs:196-415) ---- */

/* streaming.rs:172-201 StreamingOptions; every field must be positive
 * (validate, :195-201). query_chunk bounds the reference's per-chunk
 * attention; this library's attention is row-independent, so it is
 * checked and kept but does not change results. */
typedef struct esp_streaming_options {
    uint64_t query_chunk;      /* reference default 32 */
    uint64_t max_layer_bytes;  /* reference default 256 MiB */
    uint64_t max_shared_bytes; /* reference default 1 GiB */
} esp_streaming_options;

/* streaming.rs:17-37 LayerSource::read_layer in fill form. Copy layer
 * `index`'s verified safetensors artifact into `dst` (pinned host memory
 * owned by the library, `cap` bytes, cap <= limit) and set *len to its
 * size. An artifact larger than `limit` is refused before it is read
 * (return ESP_INVALID_WEIGHTS); one larger than `cap` but within `limit`
 * is reported by setting *len without copying (the library refuses it: it
 * cannot be the declared block). Any other non-zero return fails the
 * forward with that status and no position advances. The library calls it
 * on the thread running the forward, one call at a time. */
typedef esp_status (*esp_layer_read_fn)(void *user, uint32_t index, uint64_t limit, uint8_t *dst,
                                        uint64_t cap, uint64_t *len);
/* streaming.rs:26-66 LayerSource::read_expert in the same fill form: the
 * artifact of routed expert `expert` of layer `layer`, holding exactly
 * model.layers.{layer}.mlp.experts.{expert}.{gate,up,down}_proj.weight
 * (loader.rs:137-168). NULL = the source has no expert reader
 * (ESP_INVALID_WEIGHTS "layer source has no expert reader" when a routed
 * layer runs). */
typedef esp_status (*esp_expert_read_fn)(void *user, uint32_t layer, uint32_t expert,
                                         uint64_t limit, uint8_t *dst, uint64_t cap, uint64_t *len);
typedef struct esp_layer_source {
    esp_layer_read_fn read_layer;
    void *user;
    esp_expert_read_fn read_expert; /* nullable */
} esp_layer_source;

/* provider.rs:370-426 from_layer_source_with_format + model.rs:268-312
 * DecoderModel::from_layer_source_with_format. `shared` holds only
 * model.embed_tokens.weight, model.norm.weight and (unless tied)
 * lm_head.weight; it is borrowed for the call. shared_len above
 * max_shared_bytes -> ESP_INVALID_WEIGHTS "shared artifact exceeds its byte
 * limit"; any other tensor name -> "unexpected tensor in shared artifact".
 * Each forward then reads every layer through `source` (model.rs:556-646):
 * the artifact must hold exactly model.layers.{i}.* of the declared block
 * (loader.rs:830-848), is staged into HBM on a copy stream while the
 * previous layer computes, and is checked on the device (dtype admission,
 * finiteness, packed block scales) before its results are used. A routed
 * layer's artifact holds its core (attention, norms, router, shared expert:
 * loader.rs:66-85); its experts are read per forward through read_expert,
 * only those the router chose, in ascending order (moe.rs:183-243), each
 * staged while the previous one computes. Routed experts run in the f32
 * and bf16 formats (packed -> ESP_UNSUPPORTED). `source` is copied; its
 * `user` must outlive the model. */
esp_status esp_model_load_streamed(const esp_config *config, const uint8_t *shared,
                                   size_t shared_len, const esp_layer_source *source,
                                   const esp_streaming_options *options, esp_model **out);

/* model.rs:336-362 with_layer_cache: keep a first-fit subset (at most 128
 * layers) of streamed layers resident in HBM within `budget` bytes of
 * payload (counted as the reference does: 4 bytes per element of every
 * tensor in the artifact). budget 0 turns the cache off. A model that does
 * not stream -> ESP_INVALID_CONFIG. */
esp_status esp_model_layer_cache(esp_model *model, uint64_t budget);

/* model.rs:384-415 with_resident_layers: read every layer once through
 * the source, and every routed expert once through read_expert
 * (loader.rs:196-210), and keep all of them in HBM; the model then no
 * longer streams. A model that does not stream is left unchanged. */
esp_status esp_model_resident_layers(esp_model *model);

/* streaming.rs:228-252 StreamingReadStats (logical verified reads) and
 * :210-220 DeviceLayerCacheStats. `streamed` is 0 (and every other field
 * 0) for a model that does not stream (model.rs:314-333 returns None). */
typedef struct esp_streaming_stats {
    uint32_t streamed;
    uint32_t device_cache; /* 1 when a device layer cache is set */
    uint64_t layer_reads, encoded_bytes_read, largest_encoded_layer;
    uint64_t cache_hits, cache_misses, retained_payload_bytes, payload_budget_bytes;
    uint64_t cached_layers;
    /* streaming.rs:242-252, 305-312: routed experts read per forward */
    uint64_t expert_reads, expert_encoded_bytes_read, largest_encoded_expert;
} esp_streaming_stats;
esp_status esp_model_streaming_stats(const esp_model *model, esp_streaming_stats *out);

/* ---- Stage chain (decoder/stage.rs) ---- */

typedef struct esp_stage esp_stage;

/* stage.rs:301-372 DecoderStage::from_source (+ :384-413 with_output when
 * `shared` is non-NULL): layers first..end-1 read once through `source`
 * (artifacts named model.layers.{i}.*, checked as esp_model_load_streamed
 * checks them) and kept in HBM, with a one-sequence KV cache of max_ctx
 * positions (0 = max_position_embeddings). Only the final range
 * (end == num_hidden_layers) may take `shared`, whose final norm and head
 * it then owns. first >= end or end beyond the model -> ESP_INVALID_CONFIG
 * "empty or out-of-model stage range". */
esp_status esp_stage_create(const esp_config *config, uint32_t first, uint32_t end,
                            const esp_layer_source *source, const esp_streaming_options *options,
                            const uint8_t *shared, size_t shared_len, uint32_t max_ctx,
                            esp_stage **out);
esp_status esp_stage_destroy(esp_stage *stage);

/* stage.rs:471-527 StageExecutor::forward: hidden [seq, hidden_size] f32
 * (host memory, the f32 hidden wire's values) at absolute positions
 * start..start+seq. start 0 restarts the stage's cache; otherwise start
 * must equal the stage's position and seq must be 1, and a stage whose
 * last forward failed refuses until a restart (ESP_INVALID_REQUEST "stage
 * KV position mismatch; restart from checkpoint"). `out` receives the
 * hidden rows [seq, hidden_size], or for a stage with the output head the
 * last position's logits [vocab_size] (f32). */
esp_status esp_stage_forward(esp_stage *stage, const float *hidden, uint32_t seq, uint32_t start,
                             float *out);

/* ---- Constrained decoding (decoder/constraint.rs) ----
 * A vocabulary holds the byte string of every token id of a byte-level
 * tokenizer; a constraint is one request's compiled output grammar plus its
 * active automaton state. A constraint is owned by one caller at a time; a
 * vocabulary may be shared by many constraints and threads. */
typedef struct esp_vocab esp_vocab;
typedef struct esp_constraint esp_constraint;

/* The token table constraint.rs:119-154 derives from a ByteLevel
 * tokenizer: token i is bytes[offsets[i] .. offsets[i+1]] for i <
 * n_tokens, where n_tokens is the model's vocabulary size. An empty token
 * (added tokens, ids the tokenizer lacks, pieces outside the byte
 * alphabet) is never allowed. */
esp_status esp_vocab_create(const uint8_t *bytes, const uint32_t *offsets, uint32_t n_tokens,
                            esp_vocab **out);
esp_status esp_vocab_destroy(esp_vocab *vocab);

/* constraint.rs:56-157 Constraint::new. grammar_json is an OutputGrammar
 * (provider.rs:55-75) in its serde form, e.g.
 * {"kind":"sequence","items":[{"kind":"literal","value":"{\"v\":"},
 * {"kind":"json_string","max_bytes":8},{"kind":"literal","value":"}"}]}.
 * Bounds as the reference: nesting depth 24, 100000 states, 262144 literal
 * bytes, JSON string bound 1..4096, 1..64 choice alternatives
 * (ESP_INVALID_REQUEST). The constraint keeps its own reference to the
 * vocabulary, so the vocabulary may be destroyed first. */
esp_status esp_constraint_create(const esp_vocab *vocab, const char *grammar_json, size_t len,
                                 esp_constraint **out);
esp_status esp_constraint_destroy(esp_constraint *c);
/* constraint.rs:261-273 accept: advance by one token; an empty or
 * unknown token, or one the grammar refuses, is ESP_INVALID_REQUEST and
 * leaves the state unchanged. */
esp_status esp_constraint_accept(esp_constraint *c, uint32_t token);
/* constraint.rs:256-260 complete: the grammar may end here. */
esp_status esp_constraint_complete(const esp_constraint *c, uint8_t *complete);
/* constraint.rs:296-318, the byte half of `forced`: the unique-byte
 * continuation of the active state (at most 4096 bytes, cut back to valid
 * UTF-8). The caller tokenises it and checks that the ids' bytes
 * round-trip (constraint.rs:319-343). `len` receives the length; `out`
 * needs `cap` >= len (4096 always suffices). */
esp_status esp_constraint_forced_bytes(const esp_constraint *c, uint8_t *out, uint32_t cap,
                                       uint32_t *len);
/* constraint.rs:277-297 mask, its eligibility half, on the device: bit
 * id%32 of word id/32 is set iff token id is non-empty and leaves the
 * grammar alive. Runs on `stream` (hipStream_t, NULL = default); the
 * ceil(n_tokens/32) words go to allowed_dev (device, nullable) and/or
 * allowed_host (host, nullable). Returns after the mask is complete. */
esp_status esp_constraint_mask(esp_constraint *c, void *stream, uint32_t *allowed_dev,
                               uint32_t *allowed_host);
/* provider.rs:740-817 with the mask built on the device: esp_pick where
 * row i's mask is constraints[i]'s (NULL = unconstrained row). Disallowed
 * or non-finite logits become -inf; a row with no eligible token sets
 * ESP_PICK_NO_ELIGIBLE and the call returns ESP_INVALID_REQUEST
 * (constraint.rs:292-294). Constraint states are not advanced: the caller
 * accepts the picked ids (constraint.rs:261). */
esp_status esp_pick_constrained(esp_kv *kv, uint32_t n_rows, esp_constraint *const *constraints,
                                esp_sampler *samplers, uint32_t *ids_out, uint8_t *flags_out);

/* Kernel timing (measurement support, no reference counterpart): while
 * enabled, every launch of the named kernel family records HIP events on
 * its stream; read returns launches and total milliseconds since enable.
 * The family "attn_xcd_fallback" counts (always, time 0) the forwards
 * computed again because a decode-attention launch found a (row, kv
 * head)'s key splits on several XCDs, after which the process uses the
 * agent-scope merge. "greedy_forwards" counts (always) the decode
 * forwards esp_generate_greedy issues. The name "attn_xcd_mode" reads (launches) the
 * merge the decode attention uses on the current device: 0 agent-scope,
 * 1 a single XCD, N > 1 XCD-local over N XCDs. */
esp_status esp_profile_enable(const char *kernel, int enable);
esp_status esp_profile_read(const char *kernel, uint64_t *launches, double *total_ms);

/* Library/build identification. */
const char *esp_version(void);

#ifdef __cplusplus
}
#endif
#endif
