// extern "C" entry points of include/esp_hip.h. No exception crosses this
// boundary: every failure becomes an esp_status plus a thread-local message.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "decode.hpp"
#include "kernels_extra.hpp"
#include "profile.hpp"
#include "constraint.hpp"
#include "runtime.hpp"
#include "streaming.hpp"

namespace esp {
Model *load_model(const esp_config *cfg, const uint8_t *bytes, size_t len,
                  const esp_lora *adapters, uint32_t n_adapters);
Model *synthetic_model(const esp_config *cfg, uint64_t seed, float std, uint32_t lora_rank,
                       uint32_t lora_mask, float lora_a_std, float lora_b_std, float lora_scale);
Kv *create_kv(Model *m, uint32_t batch, uint32_t max_ctx, bool f16);
void decode_step_dev(Model &m, Kv &kv, int seq, int max_t, int32_t *gen);
void moe_check(Kv &kv);
void moe_steps_reset(Kv &kv);
void moe_check_steps(Kv &kv, uint32_t n);
bool xcd_merge_failed(Kv &kv);
void launch_gen_step(const uint32_t *picked, int32_t *gen, hipStream_t s);
}  // namespace esp

using namespace esp;

static thread_local std::string g_err;

template <typename F> static esp_status guard(F &&f) {
    try {
        f();
        g_err.clear();
        return ESP_OK;
    } catch (const Error &e) {
        g_err = e.msg;
        return e.code;
    } catch (const std::bad_alloc &) {
        g_err = "host allocation failed";
        return ESP_BACKEND;
    } catch (const std::exception &e) {
        g_err = e.what();
        return ESP_BACKEND;
    } catch (...) {
        g_err = "unknown failure";
        return ESP_BACKEND;
    }
}

extern "C" {

size_t esp_last_error(char *buf, size_t len) {
    if (buf && len) {
        size_t n = std::min(len - 1, g_err.size());
        memcpy(buf, g_err.data(), n);
        buf[n] = 0;
    }
    return g_err.size();
}

const char *esp_version(void) { return "esp-mi355x 0.1 (gfx950)"; }

esp_status esp_model_load(const esp_config *config, const uint8_t *safetensors, size_t len,
                          const esp_lora *adapters, uint32_t n_adapters, esp_model **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        if (n_adapters && !adapters) fail(ESP_INVALID_REQUEST, "null adapter array");
        *out = (esp_model *)load_model(config, safetensors, len, adapters, n_adapters);
    });
}

esp_status esp_model_create_synthetic(const esp_config *config, uint64_t seed, float std,
                                      uint32_t lora_rank, uint32_t lora_mask, float lora_a_std,
                                      float lora_b_std, float lora_scale, esp_model **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        *out = (esp_model *)synthetic_model(config, seed, std, lora_rank, lora_mask, lora_a_std,
                                            lora_b_std, lora_scale);
    });
}

esp_status esp_model_load_streamed(const esp_config *config, const uint8_t *shared,
                                   size_t shared_len, const esp_layer_source *source,
                                   const esp_streaming_options *options, esp_model **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        *out = (esp_model *)load_streamed_model(config, shared, shared_len, source, options);
    });
}

esp_status esp_model_layer_cache(esp_model *model, uint64_t budget) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        Model &m = *(Model *)model;
        if (!m.st) {
            if (budget == 0) return;  // model.rs:337-340
            fail(ESP_INVALID_CONFIG, "device layer caching requires a dense f32 indexed model");
        }
        std::lock_guard<std::recursive_mutex> lk(m.st->mu);
        stream_set_cache(m, budget);
    });
}

esp_status esp_model_resident_layers(esp_model *model) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        Model &m = *(Model *)model;
        if (!m.st) return;
        std::shared_ptr<Streamer> keep = m.st;  // outlives the switch to resident layers
        std::lock_guard<std::recursive_mutex> lk(keep->mu);
        stream_make_resident(m);
    });
}

esp_status esp_model_streaming_stats(const esp_model *model, esp_streaming_stats *out) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        if (!out) fail(ESP_INVALID_REQUEST, "null output");
        const Model &m = *(const Model *)model;
        std::shared_ptr<Streamer> keep = m.st;
        if (!keep) {
            stream_stats(m, out);
            return;
        }
        std::lock_guard<std::recursive_mutex> lk(keep->mu);
        stream_stats(m, out);
    });
}

}  // extern "C"

// One stage of a layer-range chain: its resident layers, its own
// one-sequence KV cache and the position rules of stage.rs:471-527.
struct esp_stage {
    std::unique_ptr<Model> model;
    std::unique_ptr<Kv> kv;
    bool head = false;
    int position = 0;
    bool failed = false;
    std::mutex mu;
    ~esp_stage() {
        (void)hipDeviceSynchronize();
        kv.reset();  // before the model it refers to
    }
};

extern "C" {

esp_status esp_stage_create(const esp_config *config, uint32_t first, uint32_t end,
                            const esp_layer_source *source, const esp_streaming_options *options,
                            const uint8_t *shared, size_t shared_len, uint32_t max_ctx,
                            esp_stage **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        std::unique_ptr<esp_stage> st(new esp_stage());
        st->model.reset(load_stage_model(config, first, end, source, options, shared, shared_len));
        st->head = shared != nullptr;
        const uint32_t ctx = max_ctx ? max_ctx : config->max_position_embeddings;
        st->kv.reset(create_kv(st->model.get(), 1, ctx, false));
        *out = st.release();
    });
}

esp_status esp_stage_destroy(esp_stage *stage) {
    return guard([&] { delete stage; });
}

esp_status esp_stage_forward(esp_stage *stage, const float *hidden, uint32_t seq, uint32_t start,
                             float *out) {
    return guard([&] {
        if (!stage) fail(ESP_MODEL_NOT_LOADED, "stage not loaded");
        esp_stage &st = *stage;
        Model &m = *st.model;
        if (!hidden || !out || seq == 0 || (uint64_t)start + seq > m.cfg.max_position_embeddings ||
            (uint64_t)start + seq > (uint64_t)st.kv->max_ctx)
            fail(ESP_INVALID_REQUEST, "stage hidden shape, dtype or context");
        std::lock_guard<std::mutex> lk(st.mu);
        if (start == 0) {  // a fresh generation rebuilds the stage's cache
            st.position = 0;
            st.failed = false;
        }
        if (st.failed || st.position != (int)start || (start != 0 && seq != 1))
            fail(ESP_INVALID_REQUEST, "stage KV position mismatch; restart from checkpoint");
        st.failed = true;  // a partial failure invalidates the cache until a prefill
        forward_hidden(m, *st.kv, hidden, (int)seq, (int)start, out, st.head);
        st.position += (int)seq;
        st.failed = false;
    });
}

esp_status esp_model_destroy(esp_model *model) {
    return guard([&] {
        if (model) {
            (void)hipDeviceSynchronize();
            delete (Model *)model;
        }
    });
}

esp_status esp_model_weight_bytes(const esp_model *model, uint64_t *bytes) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        if (bytes) *bytes = ((const Model *)model)->weight_bytes;
    });
}

esp_status esp_kv_create(esp_model *model, uint32_t batch, uint32_t max_ctx, esp_kv **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        *out = (esp_kv *)create_kv((Model *)model, batch, max_ctx, false);
    });
}

esp_status esp_kv_create_ex(esp_model *model, uint32_t batch, uint32_t max_ctx, uint32_t flags,
                            esp_kv **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "null output handle");
        *out = nullptr;
        if (flags & ~(uint32_t)ESP_KV_F16) fail(ESP_INVALID_REQUEST, "kv: unknown flags");
        *out = (esp_kv *)create_kv((Model *)model, batch, max_ctx, (flags & ESP_KV_F16) != 0);
    });
}

esp_status esp_kv_destroy(esp_kv *kv) {
    return guard([&] {
        if (kv) {
            Kv *k = (Kv *)kv;
            (void)hipStreamSynchronize(k->stream);
            delete k;
        }
    });
}

esp_status esp_kv_reset(esp_kv *kv, uint32_t seq) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        Kv *k = (Kv *)kv;
        if (seq == UINT32_MAX) std::fill(k->pos.begin(), k->pos.end(), 0);
        else if (seq < (uint32_t)k->batch) k->pos[seq] = 0;
        else fail(ESP_INVALID_REQUEST, "sequence index out of range");
    });
}

esp_status esp_kv_position(const esp_kv *kv, uint32_t seq, uint32_t *position) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        const Kv *k = (const Kv *)kv;
        if (seq >= (uint32_t)k->batch) fail(ESP_INVALID_REQUEST, "sequence index out of range");
        if (position) *position = (uint32_t)k->pos[seq];
    });
}

esp_status esp_kv_stream(const esp_kv *kv, void **stream) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        if (stream) *stream = (void *)((const Kv *)kv)->stream;
    });
}

esp_status esp_kv_logits(esp_kv *kv, float **rows_dev, uint32_t *n_rows) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        Kv &k = *(Kv *)kv;
        ESP_HIP(hipStreamSynchronize(k.stream));  // the last forward has finished
        if (rows_dev) *rows_dev = k.logits_rows ? k.logits.as<float>() : nullptr;
        if (n_rows) *n_rows = (uint32_t)k.logits_rows;
    });
}

// the forward may still be in flight on the handle's (non-blocking) stream
static void copy_logits(Kv &kv, int rows, float *out) {
    if (!out) return;
    ESP_HIP(hipMemcpyAsync(out, kv.logits.p, (size_t)rows * kv.model->V * 4, hipMemcpyDeviceToHost, kv.stream));
    ESP_HIP(hipStreamSynchronize(kv.stream));
}

esp_status esp_forward_last(esp_model *model, esp_kv *kv, uint32_t seq, const int32_t *ids,
                            uint32_t n, float *logits_out) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        if (!n || !ids) fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
        Kv &k = *(Kv *)kv;
        if (k.model != (Model *)model) fail(ESP_INVALID_REQUEST, "kv handle belongs to another model");
        forward(*(Model *)model, k, 1, &seq, &n, ids);
        copy_logits(k, 1, logits_out);
    });
}

esp_status esp_forward_batch(esp_model *model, esp_kv *kv, uint32_t n_seqs, const uint32_t *seqs,
                             const uint32_t *seq_lens, const int32_t *ids, float *logits_out) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        if (!n_seqs || !seqs || !seq_lens || !ids)
            fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
        Kv &k = *(Kv *)kv;
        if (k.model != (Model *)model) fail(ESP_INVALID_REQUEST, "kv handle belongs to another model");
        forward(*(Model *)model, k, (int)n_seqs, seqs, seq_lens, ids);
        copy_logits(k, (int)n_seqs, logits_out);
    });
}

}  // extern "C"

// esp_pick and esp_pick_constrained: masks come from the host
// (allowed_bits) or are computed on the device from constraints (cs).
static void pick_rows(Kv &k, uint32_t n_rows, const uint32_t *allowed_bits,
                      esp_constraint *const *cs, esp_sampler *samplers, uint32_t *ids_out,
                      uint8_t *flags_out) {
    if (!n_rows || (int)n_rows > k.logits_rows)
        fail(ESP_INVALID_REQUEST, "pick: rows exceed the logits of the last forward");
    if (!ids_out) fail(ESP_INVALID_REQUEST, "pick: null ids_out");
    const int V = k.model->V, words = (V + 31) / 32;
    std::vector<Constraint *> rows_c, con;
    std::vector<uint32_t *> con_mask;
    if (cs) {
        for (uint32_t i = 0; i < n_rows; ++i) {
            Constraint *c = (Constraint *)cs[i];
            if (c && (int)c->vocab->n != V)
                fail(ESP_INVALID_REQUEST, "constraint vocabulary does not match the model");
            rows_c.push_back(c);
        }
    }
    const bool masked = allowed_bits || cs;
    const size_t mask_b = masked ? (size_t)n_rows * words * 4 : 0;
    const size_t smp_b = samplers ? (size_t)n_rows * sizeof(esp_sampler) : 0;
    const size_t out_b = (size_t)n_rows * (4 + 1 + 8) + 64;
    size_t off_mask = 0, off_smp = (mask_b + 255) / 256 * 256,
           off_out = off_smp + (smp_b + 255) / 256 * 256;
    k.pick_io.ensure(off_out + out_b);
    char *io = (char *)k.pick_io.p;
    hipStream_t s = k.stream;
    // pinned staging with the device layout: [mask | samplers | ids, states, flags]
    if (k.pick_pinned_bytes < off_out + out_b) {
        if (k.pick_pinned) ESP_HIP(hipHostFree(k.pick_pinned));
        k.pick_pinned = nullptr;
        k.pick_pinned_bytes = 0;
        ESP_HIP(hipHostMalloc(&k.pick_pinned, off_out + out_b, hipHostMallocDefault));
        k.pick_pinned_bytes = off_out + out_b;
    }
    char *pin = (char *)k.pick_pinned;
    if (allowed_bits) memcpy(pin + off_mask, allowed_bits, mask_b);
    if (smp_b) memcpy(pin + off_smp, samplers, smp_b);
    // One upload of what the host supplies (constraint rows are written on
    // the device), on the pick stream: the previous pick's kernels and
    // readback of `io` and `pin` are complete (it synchronized), and nothing
    // of the forward still running on `s` touches them, so the copy overlaps
    // that forward; `s` waits for it before the pick kernels.
    if (allowed_bits || smp_b) {
        if (!k.pick_stream) {
            ESP_HIP(hipStreamCreateWithFlags(&k.pick_stream, hipStreamNonBlocking));
            ESP_HIP(hipEventCreateWithFlags(&k.pick_up, hipEventDisableTiming));
        }
        if (allowed_bits)
            ESP_HIP(hipMemcpyAsync(io, pin, off_smp + smp_b, hipMemcpyHostToDevice, k.pick_stream));
        else
            ESP_HIP(hipMemcpyAsync(io + off_smp, pin + off_smp, smp_b, hipMemcpyHostToDevice, k.pick_stream));
        ESP_HIP(hipEventRecord(k.pick_up, k.pick_stream));
        ESP_HIP(hipStreamWaitEvent(s, k.pick_up, 0));
    }
    if (cs) {
        uint32_t *m = (uint32_t *)(io + off_mask);
        for (uint32_t i = 0; i < n_rows; ++i) {
            if (rows_c[i]) {
                con.push_back(rows_c[i]);
                con_mask.push_back(m + (size_t)i * words);
            } else {
                ESP_HIP(hipMemsetAsync(m + (size_t)i * words, 0xff, (size_t)words * 4, s));
            }
        }
        if (!k.cmask) k.cmask = std::make_shared<MaskCtx>();
        Prof p("cmask", s);
        run_cmask(*k.cmask, con.data(), con_mask.data(), (int)con.size(), s);
    }
    bool any_sampled = false;
    for (uint32_t i = 0; samplers && i < n_rows; ++i) any_sampled |= samplers[i].temperature > 0.f;
    size_t scr = any_sampled ? pick_scratch_bytes((int)n_rows, V) : 0;
    k.pick_scratch.ensure(scr ? scr : 64);
    PickArgs a{};
    a.logits = k.logits.as<float>();
    a.n = (int)n_rows;
    a.V = V;
    a.allowed = mask_b ? (const uint32_t *)(io + off_mask) : nullptr;
    // rows with temperature 0 are greedy: without a sampled row the
    // sampler path (and its scratch) is not used at all
    a.samplers = smp_b && any_sampled ? (const esp_sampler *)(io + off_smp) : nullptr;
    uint32_t *d_ids = (uint32_t *)(io + off_out);
    uint64_t *d_state = (uint64_t *)(io + off_out + (size_t)n_rows * 4 + 8 - ((size_t)n_rows * 4) % 8);
    uint8_t *d_flags = (uint8_t *)(d_state + n_rows);
    a.ids_out = d_ids;
    a.flags_out = d_flags;
    a.state_out = d_state;
    a.scratch = k.pick_scratch.p;
    a.scratch_bytes = k.pick_scratch.bytes;
    {
        Prof p("pick", s);
        launch_pick(a, s);
    }
    // one readback of ids, states and flags (contiguous in the io buffer)
    const size_t res_b = (size_t)((char *)(d_flags + n_rows) - (char *)d_ids);
    ESP_HIP(hipMemcpyAsync(pin + off_out, d_ids, res_b, hipMemcpyDeviceToHost, s));
    if (!con.empty()) check_cmask(*k.cmask, s);
    ESP_HIP(hipStreamSynchronize(s));
    memcpy(ids_out, pin + off_out, (size_t)n_rows * 4);
    const uint64_t *states = (const uint64_t *)(pin + off_out + ((char *)d_state - (char *)d_ids));
    const uint8_t *flags = (const uint8_t *)(pin + off_out + ((char *)d_flags - (char *)d_ids));
    bool none = false;
    for (uint32_t i = 0; i < n_rows; ++i) {
        if (flags_out) flags_out[i] = flags[i];
        if (samplers && samplers[i].temperature > 0.f && !(flags[i] & ESP_PICK_NO_ELIGIBLE))
            samplers[i].state = states[i];
        none |= (flags[i] & ESP_PICK_NO_ELIGIBLE) != 0;
    }
    if (none) fail(ESP_INVALID_REQUEST, "output grammar has no finite eligible token");
}

extern "C" {

esp_status esp_pick(esp_kv *kv, uint32_t n_rows, const uint32_t *allowed_bits,
                    esp_sampler *samplers, uint32_t *ids_out, uint8_t *flags_out) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        pick_rows(*(Kv *)kv, n_rows, allowed_bits, nullptr, samplers, ids_out, flags_out);
    });
}

esp_status esp_pick_noalloc(esp_kv *kv, uint32_t n_rows, const uint32_t *allowed_bits_dev,
                            esp_sampler *samplers_dev, uint32_t *ids_dev, uint8_t *flags_dev) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        Kv &k = *(Kv *)kv;
        if (!n_rows || (int)n_rows > k.logits_rows)
            fail(ESP_INVALID_REQUEST, "pick: rows exceed the logits of the last forward");
        if (!ids_dev) fail(ESP_INVALID_REQUEST, "pick: null ids_out");
        launch_pick_fixed(k.model->device, k.logits.as<float>(), (int)n_rows, k.model->V,
                          allowed_bits_dev, samplers_dev, ids_dev, flags_dev, k.stream);
    });
}

esp_status esp_pick_constrained(esp_kv *kv, uint32_t n_rows, esp_constraint *const *constraints,
                                esp_sampler *samplers, uint32_t *ids_out, uint8_t *flags_out) {
    return guard([&] {
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        if (!constraints) fail(ESP_INVALID_REQUEST, "pick: null constraints");
        pick_rows(*(Kv *)kv, n_rows, nullptr, constraints, samplers, ids_out, flags_out);
    });
}

// ------------------------------------------------------------ constraints

struct esp_vocab {
    std::shared_ptr<Vocab> v;
};

esp_status esp_vocab_create(const uint8_t *bytes, const uint32_t *offsets, uint32_t n_tokens,
                            esp_vocab **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "vocab: null out");
        *out = nullptr;
        if (!offsets || !n_tokens) fail(ESP_INVALID_REQUEST, "vocab: empty token table");
        if (offsets[0] != 0) fail(ESP_INVALID_REQUEST, "vocab: offsets must start at 0");
        auto v = std::make_shared<Vocab>();
        v->n = n_tokens;
        v->off.assign(offsets, offsets + n_tokens + 1);
        for (uint32_t i = 0; i < n_tokens; ++i) {
            if (v->off[i + 1] < v->off[i]) fail(ESP_INVALID_REQUEST, "vocab: offsets decrease");
            v->max_len = std::max(v->max_len, v->off[i + 1] - v->off[i]);
        }
        if (v->off[n_tokens] && !bytes) fail(ESP_INVALID_REQUEST, "vocab: null bytes");
        v->bytes.assign(bytes, bytes + v->off[n_tokens]);
        *out = new esp_vocab{std::move(v)};
    });
}

esp_status esp_vocab_destroy(esp_vocab *vocab) {
    return guard([&] { delete vocab; });
}

esp_status esp_constraint_create(const esp_vocab *vocab, const char *grammar_json, size_t len,
                                 esp_constraint **out) {
    return guard([&] {
        if (!out) fail(ESP_INVALID_REQUEST, "constraint: null out");
        *out = nullptr;
        if (!vocab) fail(ESP_INVALID_REQUEST, "constraint: null vocabulary");
        *out = (esp_constraint *)new Constraint(vocab->v, grammar_json, len);
    });
}

esp_status esp_constraint_destroy(esp_constraint *c) {
    return guard([&] { delete (Constraint *)c; });
}

esp_status esp_constraint_accept(esp_constraint *c, uint32_t token) {
    return guard([&] {
        if (!c) fail(ESP_INVALID_REQUEST, "null constraint");
        ((Constraint *)c)->accept(token);
    });
}

esp_status esp_constraint_complete(const esp_constraint *c, uint8_t *complete) {
    return guard([&] {
        if (!c || !complete) fail(ESP_INVALID_REQUEST, "null constraint");
        *complete = ((const Constraint *)c)->complete() ? 1 : 0;
    });
}

esp_status esp_constraint_forced_bytes(const esp_constraint *c, uint8_t *out, uint32_t cap,
                                       uint32_t *len) {
    return guard([&] {
        if (!c || !len) fail(ESP_INVALID_REQUEST, "null constraint");
        std::vector<uint8_t> b = ((const Constraint *)c)->forced_bytes();
        *len = (uint32_t)b.size();
        if (b.size() > cap || (!out && !b.empty()))
            fail(ESP_INVALID_REQUEST, "forced bytes exceed the output buffer");
        if (!b.empty()) memcpy(out, b.data(), b.size());
    });
}

esp_status esp_constraint_mask(esp_constraint *c, void *stream, uint32_t *allowed_dev,
                               uint32_t *allowed_host) {
    return guard([&] {
        if (!c) fail(ESP_INVALID_REQUEST, "null constraint");
        Constraint &k = *(Constraint *)c;
        hipStream_t s = (hipStream_t)stream;
        const size_t words = ((size_t)k.vocab->n + 31) / 32;
        uint32_t *m = allowed_dev;
        DevMem tmp;
        if (!m) {
            tmp.alloc(words * 4);
            m = tmp.as<uint32_t>();
        }
        Constraint *one = &k;
        {
            Prof p("cmask", s);
            run_cmask(k.ctx, &one, &m, 1, s);
        }
        if (allowed_host)
            ESP_HIP(hipMemcpyAsync(allowed_host, m, words * 4, hipMemcpyDeviceToHost, s));
        check_cmask(k.ctx, s);
    });
}

esp_status esp_generate_greedy(esp_model *model, esp_kv *kv, uint32_t seq, const int32_t *prompt,
                               uint32_t n_prompt, uint32_t max_new, const int32_t *eos,
                               uint32_t n_eos, int32_t *out_ids, uint32_t *n_out) {
    return guard([&] {
        if (!model) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
        if (!kv) fail(ESP_INVALID_REQUEST, "null kv handle");
        if (!prompt || !n_prompt) fail(ESP_INVALID_REQUEST, "prompt must not be empty");
        Model &m = *(Model *)model;
        Kv &k = *(Kv *)kv;
        if (k.model != &m) fail(ESP_INVALID_REQUEST, "kv handle belongs to another model");
        if (seq >= (uint32_t)k.batch) fail(ESP_INVALID_REQUEST, "sequence index out of range");
        // The reference grows its cache and refuses only a forward that
        // would pass the window (model.rs:547-556): generation that stops at
        // eos before then succeeds. So only the decode forwards that fit run
        // (token i, 1-based, is fed at position n_prompt + i - 1); if no eos
        // comes among the tokens they yield, the next forward is the one the
        // reference refuses.
        const long long lim =
            std::min<long long>(k.max_ctx, (long long)m.cfg.max_position_embeddings);
        if ((long long)n_prompt > lim)
            fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
        const uint32_t fit =
            max_new ? (uint32_t)std::min<long long>((long long)max_new - 1, lim - n_prompt) : 0;
        const uint32_t gen_n = max_new ? fit + 1 : 0;  // tokens the fitting forwards yield
        const long long last_pos = (long long)n_prompt + fit;
        auto finish = [&](uint32_t n) {
            // the KV holds exactly the fed tokens: every emitted id but the
            // last of a full-length run (generate.rs:154-168)
            k.pos[seq] = (int)(n_prompt + std::min<uint32_t>(n, max_new - 1));
            if (n == gen_n && gen_n < max_new)
                fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
            if (n_out) *n_out = n;
        };
        // One pass of the generation; true when a decode-attention launch
        // found its splits on several XCDs (the XCD-local merge is then off
        // for the process and the pass runs again).
        auto pass = [&]() -> bool {
        if (n_out) *n_out = 0;
        k.pos[seq] = 0;  // generate.rs:141 new_cache per generation
        forward(m, k, 1, &seq, &n_prompt, prompt);
        if (max_new == 0) return false;
        hipStream_t s = k.stream;
        // gen layout: [0] fed token, [1] step, [2] row_seq, [3] row_pos, [8..] list
        // (gen_n <= the context window + 1 slots: only the fitting forwards'
        // tokens are ever written)
        DevMem gen((8 + (size_t)gen_n) * 4);
        int32_t *g = gen.as<int32_t>();
        int32_t init[4] = {0, 0, (int32_t)seq, (int32_t)n_prompt - 1};
        ESP_HIP(hipMemcpyAsync(g, init, sizeof(init), hipMemcpyHostToDevice, s));
        // first token from the prefill logits
        PickArgs a{};
        a.logits = k.logits.as<float>();
        a.n = 1;
        a.V = m.V;
        k.pick_io.ensure(64);
        a.ids_out = (uint32_t *)k.pick_io.p;
        a.flags_out = (uint8_t *)k.pick_io.p + 16;
        launch_pick(a, s);
        launch_gen_step(a.ids_out, g, s);
        const int max_t = (int)last_pos;
        // Streamed layers that all sit in the device layer cache read
        // nothing more: such a model replays the captured decode step like
        // a resident one, and its hit counter is set afterwards to the
        // forwards the reference takes (one per emitted token before the
        // last, generate.rs:154-168).
        // The streamer's lock is taken before its cache is inspected and held
        // to the end, so no other call can evict a layer in between.
        std::shared_ptr<Streamer> keep = m.st;
        std::unique_lock<std::recursive_mutex> st_lk;
        if (keep) st_lk = std::unique_lock<std::recursive_mutex>(keep->mu);
        // (routed experts are read per forward even for cached layers, so such
        // a model keeps the host-driven loop)
        std::shared_ptr<Streamer> cached_st =
            keep && (int)keep->cache.size() == m.L && !m.E ? keep : nullptr;
        const uint64_t hits0 = cached_st ? cached_st->hits : 0;
        auto is_eos = [&](int32_t id) {
            for (uint32_t e = 0; e < n_eos; ++e)
                if (id == eos[e]) return true;
            return false;
        };
        if (keep && !cached_st) {
            // Streamed layers are read between kernels: one host-driven step
            // per token, stopping at eos (generate.rs:154-168) so no layer
            // is read for a step the reference does not take.
            uint32_t n = 0;
            for (uint32_t i = 0; i < gen_n; ++i) {
                int32_t id = 0;
                ESP_HIP(hipMemcpyAsync(&id, g + 8 + i, 4, hipMemcpyDeviceToHost, s));
                ESP_HIP(hipStreamSynchronize(s));
                stream_check(m);
                if (is_eos(id)) break;
                if (out_ids) out_ids[n] = id;
                ++n;
                if (i + 1 < gen_n) {
                    prof_count("greedy_forwards");
                    decode_step_dev(m, k, (int)seq, max_t, g);
                }
            }
            if (xcd_merge_failed(k)) return true;
            finish(n);
            return false;
        }
        // Every layer kind routes and groups on the device (MoE included), so
        // the decode step is captured once and replayed, in chunks of 4, 8,
        // 16, 32, then 64 forwards: between chunks the host reads the new
        // ids and stops at eos (generate.rs:154-168), so the forwards run are
        // those the reference runs plus at most the rest of the last chunk.
        // ESP_GRAPHS=0 replays eagerly (profilers).
        const char *env = getenv("ESP_GRAPHS");
        const bool capturable = !(env && env[0] == '0');
        struct Exec {
            hipGraphExec_t x = nullptr;
            ~Exec() {
                if (x) (void)hipGraphExecDestroy(x);
            }
        } exec;
        moe_steps_reset(k);
        std::vector<int32_t> list(gen_n);
        uint32_t seen = 0, avail = 1, fwd = 0, n = gen_n, chunk = 4;
        // reads list[seen, avail): true once an eos or the last fitting
        // token has been seen
        auto scan = [&]() -> bool {
            ESP_HIP(hipMemcpyAsync(list.data() + seen, g + 8 + seen, (size_t)(avail - seen) * 4,
                                   hipMemcpyDeviceToHost, s));
            ESP_HIP(hipStreamSynchronize(s));
            for (; seen < avail; ++seen)
                if (is_eos(list[seen])) {
                    n = seen;
                    return true;
                }
            return avail == gen_n;
        };
        while (!scan()) {
            uint32_t c = std::min(chunk, fit - fwd);
            chunk = std::min<uint32_t>(chunk * 2, 64);
            for (uint32_t i = 0; i < c; ++i) prof_count("greedy_forwards");
            fwd += c;
            avail += c;
            if (fwd == c) {
                decode_step_dev(m, k, (int)seq, max_t, g);  // eager: sizes every scratch buffer
                --c;
            }
            if (c && capturable && !exec.x) {
                hipGraph_t graph = nullptr;
                ESP_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
                g_capturing = true;
                try {
                    decode_step_dev(m, k, (int)seq, max_t, g);
                } catch (...) {
                    g_capturing = false;
                    (void)hipStreamEndCapture(s, &graph);
                    if (graph) (void)hipGraphDestroy(graph);
                    throw;
                }
                g_capturing = false;
                ESP_HIP(hipStreamEndCapture(s, &graph));
                hipError_t ie = hipGraphInstantiate(&exec.x, graph, nullptr, nullptr, 0);
                (void)hipGraphDestroy(graph);
                ESP_HIP(ie);
            }
            for (uint32_t i = 0; i < c; ++i) {
                if (exec.x) ESP_HIP(hipGraphLaunch(exec.x, s));
                else decode_step_dev(m, k, (int)seq, max_t, g);
            }
        }
        if (xcd_merge_failed(k)) return true;
        if (out_ids)
            for (uint32_t i = 0; i < n; ++i) out_ids[i] = list[i];
        moe_check_steps(k, n);  // a forward the reference runs whose router failed
        if (cached_st) {
            stream_check(m);
            const uint64_t fw = std::min<uint64_t>(n, max_new - 1);
            cached_st->hits = hits0 + fw * (uint64_t)m.L;
        }
        finish(n);
        return false;
        };
        const StreamMark mark = stream_mark(m);
        if (!pass()) return;
        stream_rewind(m, mark);
        if (pass())
            fail(ESP_BACKEND, "decode attention: split placement check failed with the agent-scope merge");
    });
}

esp_status esp_profile_enable(const char *kernel, int enable) {
    return guard([&] {
        if (!kernel) fail(ESP_INVALID_REQUEST, "null kernel name");
        prof_enable(kernel, enable);
    });
}

esp_status esp_profile_read(const char *kernel, uint64_t *launches, double *total_ms) {
    return guard([&] {
        if (!kernel) fail(ESP_INVALID_REQUEST, "null kernel name");
        unsigned long long n = 0;
        if (!strcmp(kernel, "attn_xcd_mode")) {  // the decode attention's merge mode
            n = (unsigned long long)attn_xcd_mode();
            if (total_ms) *total_ms = 0.0;
        } else {
            prof_read(kernel, &n, total_ms);
        }
        if (launches) *launches = n;
    });
}

}  // extern "C"
