// Host runtime of the MI355X decoder: weight staging into HBM, per-sequence
// KV caches, the layer-by-layer forward over token rows, token choice and
// the device-resident greedy loop. Every public entry point is in
// esp_abi.cpp; this file holds the machinery.
#include "runtime.hpp"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <set>

#include "decode.hpp"
#include "flash.hpp"
#include "kernels_extra.hpp"
#include "profile.hpp"
#include "safetensors.hpp"
#include "streaming.hpp"

namespace esp {

// words of Kv::tickets (128-byte multiple)
// [0, 2 * ATT_MAX_TICKETS): 64-bit attention merge tickets; then the head
// ticket, the XCD placement flag, the argmax partials and the picked id
static const int kHeadTicket = 2 * ATT_MAX_TICKETS;
static const int kXcdErr = kHeadTicket + 4;
static const int kTicketWords = (kHeadTicket + 8 + 2 * DG_MAX_PART + 8 + 31) / 32 * 32;

struct Rows;

Kv::~Kv() {
    if (gen_exec) (void)hipGraphExecDestroy(gen_exec);
    if (pinned) (void)hipHostFree(pinned);
    if (pick_pinned) (void)hipHostFree(pick_pinned);
    if (pick_up) (void)hipEventDestroy(pick_up);
    if (pick_stream) (void)hipStreamDestroy(pick_stream);
    if (stream) (void)hipStreamDestroy(stream);
}

// ------------------------------------------------------------------ RoPE
// decoder/config.rs:158-180 RopeScaling::apply
static float rope_scale(const esp_config &c, float freq) {
    if (c.rope_scaling == ESP_ROPE_LINEAR) return freq / c.rope_factor;
    if (c.rope_scaling == ESP_ROPE_LLAMA3) {
        const float tau = 6.28318530717958647692f;
        float wavelength = tau / freq;
        float original = (float)c.rope_original_max_position_embeddings;
        if (wavelength < original / c.rope_high_freq_factor) return freq;
        if (wavelength > original / c.rope_low_freq_factor) return freq / c.rope_factor;
        float smooth = (original / wavelength - c.rope_low_freq_factor) /
                       (c.rope_high_freq_factor - c.rope_low_freq_factor);
        return (1.0f - smooth) * freq / c.rope_factor + smooth * freq;
    }
    return freq;
}

// decoder/attention.rs:58-95: the host f32 table [max_pos, hd], each half
// duplicated (cos/sin of position * inverse frequency).
static void build_rope(const esp_config &c, std::vector<float> &cs, std::vector<float> &sn) {
    const int hd = (int)c.head_dim, half = hd / 2, mp = (int)c.max_position_embeddings;
    cs.assign((size_t)mp * hd, 0.f);
    sn.assign((size_t)mp * hd, 0.f);
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i)
        inv[i] = rope_scale(c, 1.0f / powf(c.rope_theta, (float)(2 * i) / (float)hd));
    for (int p = 0; p < mp; ++p)
        for (int i = 0; i < half; ++i) {
            float angle = (float)p * inv[i];
            float cv = cosf(angle), sv = sinf(angle);
            cs[(size_t)p * hd + i] = cs[(size_t)p * hd + half + i] = cv;
            sn[(size_t)p * hd + i] = sn[(size_t)p * hd + half + i] = sv;
        }
}

// --------------------------------------------------------------- staging

static void validate_config(const esp_config &c) {
    if (!c.vocab_size || !c.hidden_size || !c.intermediate_size || !c.num_hidden_layers ||
        !c.num_attention_heads || !c.num_key_value_heads || !c.head_dim ||
        !c.max_position_embeddings)
        fail(ESP_INVALID_CONFIG, "zero, non-finite or overflowing decoder dimensions/settings");
    if (c.num_attention_heads % c.num_key_value_heads)
        fail(ESP_INVALID_CONFIG, "num_attention_heads not divisible by num_key_value_heads");
    if (c.head_dim % 2) fail(ESP_INVALID_CONFIG, "head_dim must be even for rotary encoding");
    if (!(c.rms_norm_eps > 0.f) || !isfinite(c.rms_norm_eps) || !(c.rope_theta > 0.f) ||
        !isfinite(c.rope_theta))
        fail(ESP_INVALID_CONFIG, "zero, non-finite or overflowing decoder dimensions/settings");
    if (c.format > ESP_FORMAT_Q4_BLOCK32)
        fail(ESP_INVALID_CONFIG, "unknown weight format " + std::to_string(c.format));
    if (c.head_dim > 256) fail(ESP_UNSUPPORTED, "head_dim: values above 256 are not implemented");
    if (c.num_attention_heads / c.num_key_value_heads * c.head_dim > 2048)
        fail(ESP_UNSUPPORTED, "attention: query group x head_dim above 2048 is not implemented");
    if (c.num_experts) {
        if (!c.num_experts_per_tok || c.num_experts_per_tok > c.num_experts ||
            !c.moe_intermediate_size)
            fail(ESP_UNSUPPORTED,
                 "config.experts: invalid expert count, routing, intermediate size or sparse-layer "
                 "selection");
        if (c.num_experts > 256) fail(ESP_UNSUPPORTED, "config.experts: more than 256 experts");
        if (c.num_experts_per_tok > 8) fail(ESP_UNSUPPORTED, "config.experts: top-k above 8");
    }
}

static void init_model_shape(Model &m, const esp_config &c) {
    m.cfg = c;
    m.cfg.layer_window = nullptr;
    m.cfg.layer_is_moe = nullptr;
    m.wt = c.format == ESP_FORMAT_BF16 ? DT_BF16
         : c.format == ESP_FORMAT_Q8_BLOCK32 ? DT_Q8
         : c.format == ESP_FORMAT_Q4_BLOCK32 ? DT_Q4 : DT_F32;
    m.et = dt_packed(m.wt) ? DT_F32 : m.wt;
    m.ht = m.wt;
    m.H = c.hidden_size;
    m.L = c.num_hidden_layers;
    m.nq = c.num_attention_heads;
    m.nkv = c.num_key_value_heads;
    m.hd = c.head_dim;
    m.F = c.intermediate_size;
    m.V = c.vocab_size;
    m.qw = m.nq * m.hd;
    m.kvw = m.nkv * m.hd;
    m.E = c.num_experts;
    m.topk = c.num_experts_per_tok;
    m.Fe = c.moe_intermediate_size;
    m.Fs = c.shared_expert_intermediate_size;
    m.norm_topk = c.norm_topk_prob != 0;
    m.layers.assign(m.L, LayerW());
    for (int l = 0; l < m.L; ++l) {
        m.layers[l].window = c.layer_window ? (int)c.layer_window[l] : 0;
        m.layers[l].moe = m.E && c.layer_is_moe && c.layer_is_moe[l];
    }
    ESP_HIP(hipGetDevice(&m.device));
}

// Packed formats (weight_format.rs:138-223) run dense llama-family layers:
// every projection input width a multiple of 32 within the decode GEMV.
static void check_packed(const Model &m, uint32_t n_adapters) {
    if (!dt_packed(m.wt)) return;
    const char *id = m.wt == DT_Q8 ? "weight format q8-k32-f32-scale-f16-shared-v1"
                                   : "weight format q4-k32-f32-scale-f16-shared-v1";
    if (m.E) fail(ESP_UNSUPPORTED, std::string(id) + ": routed experts are not implemented");
    if (n_adapters) fail(ESP_UNSUPPORTED, std::string(id) + ": unmerged LoRA is not implemented");
    for (int k : {m.H, m.qw, m.F}) {
        if (k % 32)
            fail(ESP_INVALID_WEIGHTS, "weight format: packed projection input width " +
                                          std::to_string(k) + " must be divisible by 32");
        if (!decode_gemv_packed_ok(m.wt, k))
            fail(ESP_UNSUPPORTED, std::string(id) + ": projection input width " +
                                      std::to_string(k) + " (the decode kernels need a multiple of 64, "
                                      "at most 16384)");
    }
}

static void upload(void *dst, const void *src, size_t bytes) {
    ESP_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
}

static void stage_rope(Model &m) {
    std::vector<float> cs, sn;
    build_rope(m.cfg, cs, sn);
    m.rope_cos = (float *)m.alloc(cs.size() * 4);
    m.rope_sin = (float *)m.alloc(sn.size() * 4);
    upload(m.rope_cos, cs.data(), cs.size() * 4);
    upload(m.rope_sin, sn.data(), sn.size() * 4);
}

static inline float half_to_f32(uint16_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 0x1f, f = h & 0x3ff;
    uint32_t out;
    if (e == 0) {
        if (f == 0) out = s << 31;
        else {
            int ee = -1;
            do {
                ++ee;
                f <<= 1;
            } while (!(f & 0x400));
            out = (s << 31) | ((uint32_t)(127 - 15 - ee) << 23) | ((f & 0x3ff) << 13);
        }
    } else if (e == 31) {
        out = (s << 31) | 0x7f800000u | (f << 13);
    } else {
        out = (s << 31) | ((e + 127 - 15) << 23) | (f << 13);
    }
    float r;
    memcpy(&r, &out, 4);
    return r;
}

// The named tensor with exactly `shape` (tensors.rs:22-66 messages).
const StTensor &expect_tensor(const std::map<std::string, StTensor> &t, const std::string &name,
                              const std::vector<uint64_t> &shape) {
    auto it = t.find(name);
    if (it == t.end()) fail(ESP_INVALID_WEIGHTS, "missing tensor: " + name);
    if (it->second.shape != shape) {
        std::string e = "weight format: expected [";
        for (size_t i = 0; i < shape.size(); ++i) e += (i ? ", " : "") + std::to_string(shape[i]);
        e += "], got [";
        for (size_t i = 0; i < it->second.shape.size(); ++i)
            e += (i ? ", " : "") + std::to_string(it->second.shape[i]);
        fail(ESP_INVALID_WEIGHTS, e + "] for " + name);
    }
    return it->second;
}

// Dtype admission of one non-packed tensor (weight_format.rs:110-133,
// 283-291): bf16 models take BF16 projections, the packed formats F16 for
// every tensor that is not a packed projection; force_f32 tensors (norms,
// biases) of unpacked models may be F32, BF16 or F16.
void check_tensor_dtype(const Model &m, const std::string &name, const StTensor &s,
                        bool force_f32) {
    if ((m.wt == DT_BF16 && !force_f32 && s.dtype != "BF16") ||
        (dt_packed(m.wt) && s.dtype != "F16"))
        fail(ESP_INVALID_WEIGHTS, "weight format: artifact dtype disagrees with declared format (" +
                                      name + ")");
    if (s.dtype != "F32" && s.dtype != "BF16" && s.dtype != "F16")
        fail(ESP_INVALID_WEIGHTS, "weight format: cannot import " + s.dtype + " (" + name + ")");
}

// The header side of a packed projection [rows, cols]
// (weight_format.rs:225-273): a U8 tensor whose shape is its byte count.
// Returns whether the byte count is the packed values plus the f32 block
// scales; the scales themselves are checked by the caller.
bool check_packed_header(const Model &m, const std::string &name, const StTensor &s,
                         uint64_t rows, uint64_t cols) {
    if (s.dtype != "U8")
        fail(ESP_INVALID_WEIGHTS, "weight format: unpacked projection in a quantized row (" +
                                      name + ")");
    if (cols % 32)
        fail(ESP_INVALID_WEIGHTS, "weight format: packed projection input width must be "
                                  "divisible by 32");
    const size_t n = rows * cols, vb = packed_value_bytes(m.wt, n), sb = n / 32 * 4;
    if (s.shape.size() != 1 || s.shape[0] != s.bytes)
        fail(ESP_INVALID_WEIGHTS, "weight format: packed buffer must have its encoded "
                                  "byte-count shape");
    return s.bytes == vb + sb;
}

// Reads checkpoint tensors into a host staging vector in the model's
// format, checking shape, dtype admission and finiteness
// (decoder/weight_format.rs:110-133, 225-315; tensors.rs:22-66).
struct Stager {
    Model &m;
    const std::map<std::string, StTensor> &t;
    std::set<std::string> consumed;

    const StTensor &get(const std::string &name, std::vector<uint64_t> shape) {
        const StTensor &s = expect_tensor(t, name, shape);
        consumed.insert(name);
        return s;
    }
    bool has(const std::string &name) const { return t.count(name) != 0; }

    // Append the tensor's elements (converted) to `out` as the model dtype
    // (or f32 when force_f32).
    void read(const std::string &name, std::vector<uint64_t> shape, std::vector<uint8_t> &out,
              bool force_f32 = false) {
        const StTensor &s = get(name, shape);
        size_t n = 1;
        for (auto d : shape) n *= d;
        Dt dst = force_f32 || dt_packed(m.wt) ? DT_F32 : m.wt;
        check_tensor_dtype(m, name, s, force_f32);
        size_t base = out.size();
        out.resize(base + n * dt_size(dst));
        uint8_t *o = out.data() + base;
        for (size_t i = 0; i < n; ++i) {
            float v;
            if (s.dtype == "F32") memcpy(&v, s.data + 4 * i, 4);
            else if (s.dtype == "BF16") {
                uint32_t u = (uint32_t)(s.data[2 * i] | (s.data[2 * i + 1] << 8)) << 16;
                memcpy(&v, &u, 4);
            } else if (s.dtype == "F16") {
                v = half_to_f32((uint16_t)(s.data[2 * i] | (s.data[2 * i + 1] << 8)));
            } else {
                fail(ESP_INVALID_WEIGHTS, "weight format: cannot import " + s.dtype + " (" + name + ")");
            }
            if (!isfinite(v)) fail(ESP_INVALID_WEIGHTS, "weight format: non-finite weight in " + name);
            if (dst == DT_F32) memcpy(o + 4 * i, &v, 4);
            else {
                uint16_t b = (uint16_t)(s.data[2 * i] | (s.data[2 * i + 1] << 8));
                memcpy(o + 2 * i, &b, 2);
            }
        }
    }
    // A packed projection [rows, cols] (weight_format.rs:225-273): a U8
    // tensor whose shape is its byte count, the packed values then the
    // f32 block scales, every scale finite and positive. Appends to vals
    // and scales.
    void read_packed(const std::string &name, uint64_t rows, uint64_t cols,
                     std::vector<uint8_t> &vals, std::vector<uint8_t> &scales) {
        auto it = t.find(name);
        if (it == t.end()) fail(ESP_INVALID_WEIGHTS, "missing tensor: " + name);
        const StTensor &s = it->second;
        const size_t n = rows * cols, vb = packed_value_bytes(m.wt, n), sb = n / 32 * 4;
        bool ok = check_packed_header(m, name, s, rows, cols);
        for (size_t i = 0; ok && i < n / 32; ++i) {
            float sc;
            memcpy(&sc, s.data + vb + 4 * i, 4);
            ok = isfinite(sc) && sc > 0.f;
        }
        if (!ok)
            fail(ESP_INVALID_WEIGHTS, "weight format: packed projection byte count or block scales "
                                      "are invalid (" + name + ")");
        consumed.insert(name);
        vals.insert(vals.end(), s.data, s.data + vb);
        scales.insert(scales.end(), s.data + vb, s.data + vb + sb);
    }
    // values then scales in one allocation; *scales_out points at the scales
    void *packed(const std::vector<uint8_t> &vals, const std::vector<uint8_t> &scales,
                 const float **scales_out) {
        std::vector<uint8_t> all(vals);
        size_t pad = (256 - all.size() % 256) % 256;  // 256-byte aligned scales
        all.resize(all.size() + pad, 0);
        const size_t off = all.size();
        all.insert(all.end(), scales.begin(), scales.end());
        char *d = (char *)to_device(all);
        *scales_out = (const float *)(d + off);
        return d;
    }
    void *proj(const std::string &name, uint64_t rows, uint64_t cols, const float **scales_out) {
        if (!dt_packed(m.wt)) return tensor(name, {rows, cols});
        std::vector<uint8_t> v, sc;
        read_packed(name, rows, cols, v, sc);
        return packed(v, sc, scales_out);
    }
    void *to_device(const std::vector<uint8_t> &host) {
        void *d = m.alloc(host.size());
        upload(d, host.data(), host.size());
        return d;
    }
    void *tensor(const std::string &name, std::vector<uint64_t> shape, bool force_f32 = false) {
        std::vector<uint8_t> h;
        read(name, shape, h, force_f32);
        return to_device(h);
    }
};

static void refuse_unconsumed(const Stager &s) {
    std::vector<std::string> left;
    for (auto &kv : s.t) {
        const std::string &n = kv.first;
        if (s.consumed.count(n)) continue;
        if (n.size() >= 20 && n.compare(n.size() - 20, 20, ".rotary_emb.inv_freq") == 0) continue;
        left.push_back(n);
    }
    if (left.empty()) return;
    std::sort(left.begin(), left.end());
    const std::string &first = left[0];
    // decoder/loader.rs:257-275 why_unconsumed
    std::string why;
    auto ends = [&](const char *suf) {
        size_t k = strlen(suf);
        return first.size() >= k && first.compare(first.size() - k, k, suf) == 0;
    };
    if (ends(".bias")) why = "this bias is not declared by the decoder configuration";
    else if (first.find("q_norm") != std::string::npos || first.find("k_norm") != std::string::npos)
        why = "this head norm is not declared by the decoder configuration";
    else if (first.find("experts") != std::string::npos ||
             first.find("block_sparse_moe") != std::string::npos || ends(".mlp.gate.weight"))
        why = "this expert or router is not declared by the decoder configuration";
    else if (first.find("norm") != std::string::npos)
        why = "normalization layers beyond the Llama block's two per layer are not implemented";
    else why = "the Llama-block decoder does not consume this tensor";
    fail(ESP_UNSUPPORTED, "tensor " + first + ": " + why + "; " + std::to_string(left.size()) +
                              " unconsumed tensor(s) in this checkpoint");
}

static const char *kTargets[4] = {"q_proj", "k_proj", "v_proj", "o_proj"};

Model *load_model(const esp_config *cfg, const uint8_t *bytes, size_t len,
                  const esp_lora *adapters, uint32_t n_adapters) {
    if (!cfg) fail(ESP_INVALID_CONFIG, "null config");
    validate_config(*cfg);
    std::unique_ptr<Model> mp(new Model());
    Model &m = *mp;
    init_model_shape(m, *cfg);
    check_packed(m, n_adapters);
    auto tensors = parse_safetensors(bytes, len);
    Stager s{m, tensors, {}};
    const uint64_t H = m.H, qw = m.qw, kvw = m.kvw, hd = m.hd;

    // adapters: parse each; per target the ranks stack in adapter order
    std::vector<std::map<std::string, StTensor>> ad_t(n_adapters);
    int rank_sum[4] = {0, 0, 0, 0};
    float tscale[4] = {0, 0, 0, 0};
    for (uint32_t a = 0; a < n_adapters; ++a) {
        const esp_lora &ad = adapters[a];
        if (!ad.rank || !isfinite(ad.scale))
            fail(ESP_INVALID_CONFIG, "adapter " + std::to_string(a) +
                                         ": PEFT rank must be positive and alpha finite");
        if (ad.target_mask & 8u)
            fail(ESP_UNSUPPORTED, "adapter o_proj: unmerged LoRA on o_proj is not implemented");
        if (m.E) fail(ESP_UNSUPPORTED, "MoE adapters/training: expert routing is inference-only");
        ad_t[a] = parse_safetensors(ad.safetensors, ad.safetensors_len);
        int nt = 0;
        for (int j = 0; j < 3; ++j)
            if (ad.target_mask & (1u << j)) {
                ++nt;
                if (rank_sum[j] && tscale[j] != ad.scale)
                    fail(ESP_UNSUPPORTED, "adapters: stacked adapters on one projection must share "
                                          "a scale");
                rank_sum[j] += ad.rank;
                tscale[j] = ad.scale;
            }
        if (ad_t[a].size() != (size_t)m.L * nt * 2)
            fail(ESP_INVALID_WEIGHTS, "adapter " + std::to_string(a) +
                                          ": adapter tensor count mismatch: expected " +
                                          std::to_string((size_t)m.L * nt * 2) + ", got " +
                                          std::to_string(ad_t[a].size()));
    }
    const int lora_total = rank_sum[0] + rank_sum[1] + rank_sum[2];

    for (int l = 0; l < m.L; ++l) {
        LayerW &w = m.layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        w.in_norm = (float *)s.tensor(p + "input_layernorm.weight", {H}, true);
        w.post_norm = (float *)s.tensor(p + "post_attention_layernorm.weight", {H}, true);
        // fused q | k | v | LoRA-A rows (loader.rs:508-535 read order)
        std::vector<uint8_t> qkv, qkv_sc;
        if (dt_packed(m.wt)) {
            s.read_packed(p + "self_attn.q_proj.weight", qw, H, qkv, qkv_sc);
            s.read_packed(p + "self_attn.k_proj.weight", kvw, H, qkv, qkv_sc);
            s.read_packed(p + "self_attn.v_proj.weight", kvw, H, qkv, qkv_sc);
        } else {
            s.read(p + "self_attn.q_proj.weight", {qw, H}, qkv);
            s.read(p + "self_attn.k_proj.weight", {kvw, H}, qkv);
            s.read(p + "self_attn.v_proj.weight", {kvw, H}, qkv);
        }
        w.qkv_rows = (int)(qw + 2 * kvw) + lora_total;
        int tcol = (int)(qw + 2 * kvw);
        for (int j = 0; j < 3; ++j) {
            if (!rank_sum[j]) continue;
            uint64_t outf = j == 0 ? qw : kvw;
            std::vector<uint8_t> bcat((size_t)outf * rank_sum[j] * dt_size(m.wt));
            int roff = 0;
            for (uint32_t a = 0; a < n_adapters; ++a) {
                if (!(adapters[a].target_mask & (1u << j))) continue;
                uint64_t r = adapters[a].rank;
                Stager sa{m, ad_t[a], {}};
                std::string pre = "base_model.model.model.layers." + std::to_string(l) +
                                  ".self_attn." + kTargets[j];
                sa.read(pre + ".lora_A.weight", {r, H}, qkv);
                std::vector<uint8_t> b;
                sa.read(pre + ".lora_B.weight", {outf, r}, b);
                size_t es = dt_size(m.wt);
                for (uint64_t o = 0; o < outf; ++o)
                    memcpy(bcat.data() + ((size_t)o * rank_sum[j] + roff) * es,
                           b.data() + (size_t)o * r * es, r * es);
                roff += (int)r;
            }
            w.lora_b[j] = s.to_device(bcat);
            w.lora_rank[j] = rank_sum[j];
            w.lora_t_col[j] = tcol;
            w.lora_scale[j] = tscale[j];
            tcol += rank_sum[j];
        }
        w.qkv = dt_packed(m.wt) ? s.packed(qkv, qkv_sc, &w.qkv_s) : s.to_device(qkv);
        if (cfg->qkv_bias) {
            std::vector<uint8_t> b;
            s.read(p + "self_attn.q_proj.bias", {qw}, b, true);
            s.read(p + "self_attn.k_proj.bias", {kvw}, b, true);
            s.read(p + "self_attn.v_proj.bias", {kvw}, b, true);
            b.resize((size_t)w.qkv_rows * 4, 0);
            w.qkv_bias = (float *)s.to_device(b);
        }
        w.o = s.proj(p + "self_attn.o_proj.weight", H, qw, &w.o_s);
        if (cfg->output_bias) w.o_bias = (float *)s.tensor(p + "self_attn.o_proj.bias", {H}, true);
        if (cfg->qk_norm) {
            w.q_norm = (float *)s.tensor(p + "self_attn.q_norm.weight", {hd}, true);
            w.k_norm = (float *)s.tensor(p + "self_attn.k_norm.weight", {hd}, true);
        }
        if (!w.moe) {
            uint64_t F = m.F;
            w.gate = s.proj(p + "mlp.gate_proj.weight", F, H, &w.gate_s);
            w.up = s.proj(p + "mlp.up_proj.weight", F, H, &w.up_s);
            w.down = s.proj(p + "mlp.down_proj.weight", H, F, &w.down_s);
        } else {
            uint64_t E = m.E, Fe = m.Fe, Fs = m.Fs;
            w.router = s.tensor(p + "mlp.gate.weight", {E, H});
            if (Fs) {
                w.shared_gate = s.tensor(p + "mlp.shared_expert_gate.weight", {1, H});
                w.sh_gate = s.tensor(p + "mlp.shared_expert.gate_proj.weight", {Fs, H});
                w.sh_up = s.tensor(p + "mlp.shared_expert.up_proj.weight", {Fs, H});
                w.sh_down = s.tensor(p + "mlp.shared_expert.down_proj.weight", {H, Fs});
            }
            std::vector<uint8_t> g, u, d;
            for (uint64_t e = 0; e < E; ++e) {
                std::string ep = p + "mlp.experts." + std::to_string(e) + ".";
                s.read(ep + "gate_proj.weight", {Fe, H}, g);
                s.read(ep + "up_proj.weight", {Fe, H}, u);
                s.read(ep + "down_proj.weight", {H, Fe}, d);
            }
            w.ex_gate = s.to_device(g);
            w.ex_up = s.to_device(u);
            w.ex_down = s.to_device(d);
        }
    }
    m.embed = s.tensor("model.embed_tokens.weight", {(uint64_t)m.V, H});
    m.final_norm = (float *)s.tensor("model.norm.weight", {H}, true);
    if (s.has("lm_head.weight")) {
        m.head = s.proj("lm_head.weight", (uint64_t)m.V, H, &m.head_s);
    } else if (cfg->tie_word_embeddings) {
        m.head = m.embed;  // model.rs:167-169 tied head
        m.ht = m.et;
    } else {
        fail(ESP_INVALID_WEIGHTS, "lm_head.weight missing but tie_word_embeddings is false");
    }
    refuse_unconsumed(s);
    stage_rope(m);
    return mp.release();
}

Model *load_streamed_model(const esp_config *cfg, const uint8_t *shared, size_t len,
                           const esp_layer_source *source, const esp_streaming_options *opt) {
    if (!cfg) fail(ESP_INVALID_CONFIG, "null config");
    if (!source || !source->read_layer) fail(ESP_INVALID_REQUEST, "null layer source");
    // provider.rs:381-387 (StreamingOptions::validate, streaming.rs:195-201)
    if (!opt || !opt->query_chunk || !opt->max_layer_bytes || !opt->max_shared_bytes)
        fail(ESP_INVALID_CONFIG, "streaming limits must be positive");
    if (len > opt->max_shared_bytes)
        fail(ESP_INVALID_WEIGHTS, "shared artifact exceeds its byte limit");
    validate_config(*cfg);
    std::unique_ptr<Model> mp(new Model());
    Model &m = *mp;
    init_model_shape(m, *cfg);
    std::map<std::string, StTensor> tensors;
    try {
        tensors = parse_safetensors(shared, len);
    } catch (const Error &e) {
        fail(ESP_INVALID_WEIGHTS, "shared tensors: " + e.msg);
    }
    for (auto &kv : tensors)  // provider.rs:394-405
        if (kv.first != "model.embed_tokens.weight" && kv.first != "model.norm.weight" &&
            kv.first != "lm_head.weight")
            fail(ESP_INVALID_WEIGHTS, "unexpected tensor in shared artifact");
    check_packed(m, 0);
    // the geometry every staged block binds (scratch buffers are sized from it)
    for (auto &w : m.layers) w.qkv_rows = m.qw + 2 * m.kvw;
    Stager s{m, tensors, {}};
    const uint64_t H = m.H;
    m.embed = s.tensor("model.embed_tokens.weight", {(uint64_t)m.V, H});
    m.final_norm = (float *)s.tensor("model.norm.weight", {H}, true);
    if (s.has("lm_head.weight")) {
        m.head = s.proj("lm_head.weight", (uint64_t)m.V, H, &m.head_s);
    } else if (cfg->tie_word_embeddings) {
        m.head = m.embed;
        m.ht = m.et;
    } else {
        fail(ESP_INVALID_WEIGHTS, "lm_head.weight missing but tie_word_embeddings is false");
    }
    stage_rope(m);
    streamer_init(m, *source, *opt);
    return mp.release();
}

Model *load_stage_model(const esp_config *cfg, uint32_t first, uint32_t end,
                        const esp_layer_source *source, const esp_streaming_options *opt,
                        const uint8_t *shared, size_t shared_len) {
    if (!cfg) fail(ESP_INVALID_CONFIG, "null config");
    if (!source || !source->read_layer) fail(ESP_INVALID_REQUEST, "null layer source");
    if (first >= end || end > cfg->num_hidden_layers)  // stage.rs:28-35
        fail(ESP_INVALID_CONFIG, "empty or out-of-model stage range");
    if (!opt || !opt->query_chunk || !opt->max_layer_bytes || !opt->max_shared_bytes)
        fail(ESP_INVALID_CONFIG, "streaming limits must be positive");
    validate_config(*cfg);
    esp_config c = *cfg;  // the range as a model of its own
    c.num_hidden_layers = end - first;
    if (cfg->layer_window) c.layer_window = cfg->layer_window + first;
    if (cfg->layer_is_moe) c.layer_is_moe = cfg->layer_is_moe + first;
    std::unique_ptr<Model> mp(new Model());
    Model &m = *mp;
    init_model_shape(m, c);
    check_packed(m, 0);
    for (auto &w : m.layers) w.qkv_rows = m.qw + 2 * m.kvw;
    if (shared) {  // stage.rs:384-413 with_output: the final range owns norm and head
        if (end != cfg->num_hidden_layers)
            fail(ESP_INVALID_WEIGHTS, "only the final stage may own the output head");
        if (shared_len > opt->max_shared_bytes)
            fail(ESP_INVALID_WEIGHTS, "shared artifact exceeds its byte limit");
        std::map<std::string, StTensor> tensors;
        try {
            tensors = parse_safetensors(shared, shared_len);
        } catch (const Error &e) {
            fail(ESP_INVALID_WEIGHTS, "shared tensors: " + e.msg);
        }
        for (auto &kv : tensors)
            if (kv.first != "model.embed_tokens.weight" && kv.first != "model.norm.weight" &&
                kv.first != "lm_head.weight")
                fail(ESP_INVALID_WEIGHTS, "unexpected tensor in shared artifact");
        Stager s{m, tensors, {}};
        const uint64_t H = m.H;
        m.final_norm = (float *)s.tensor("model.norm.weight", {H}, true);
        if (s.has("lm_head.weight")) {  // an untied embedding is not kept
            m.head = s.proj("lm_head.weight", (uint64_t)m.V, H, &m.head_s);
        } else if (cfg->tie_word_embeddings) {
            m.embed = s.tensor("model.embed_tokens.weight", {(uint64_t)m.V, H});
            m.head = m.embed;
            m.ht = m.et;
        } else {
            fail(ESP_INVALID_WEIGHTS, "lm_head.weight missing but tie_word_embeddings is false");
        }
    }
    stage_rope(m);
    streamer_init(m, *source, *opt, (int)first);
    {
        std::shared_ptr<Streamer> keep = m.st;
        std::lock_guard<std::recursive_mutex> lk(keep->mu);
        stream_make_resident(m);
    }
    return mp.release();
}

// Synthetic model: every projection / embedding N(0, std) from a seeded
// device generator, norms 1, biases 0 (bench and large-shape tests).
Model *synthetic_model(const esp_config *cfg, uint64_t seed, float std, uint32_t lora_rank,
                       uint32_t lora_mask, float lora_a_std, float lora_b_std,
                       float lora_scale) {
    if (!cfg) fail(ESP_INVALID_CONFIG, "null config");
    validate_config(*cfg);
    if (lora_mask & 8u) fail(ESP_UNSUPPORTED, "adapter o_proj: unmerged LoRA on o_proj is not implemented");
    std::unique_ptr<Model> mp(new Model());
    Model &m = *mp;
    init_model_shape(m, *cfg);
    check_packed(m, lora_rank && lora_mask ? 1 : 0);
    uint64_t tensor_id = 0;
    auto rnd_dt = [&](size_t n, float sd, Dt dt) {
        void *p = m.alloc(n * dt_size(dt));
        launch_fill_normal(dt, p, n, seed * 0x100000001B3ull + (++tensor_id), sd, nullptr);
        return p;
    };
    auto rnd = [&](size_t n, float sd) { return rnd_dt(n, sd, m.wt); };
    // a projection: N(0, std) weights, quantized on the device for the
    // packed formats (values, 256-byte aligned block scales)
    DevMem tmp;
    auto prj = [&](size_t rows, size_t cols, float sd, const float **sc) -> void * {
        if (!dt_packed(m.wt)) return rnd(rows * cols, sd);
        tmp.ensure(rows * cols * 4);
        launch_fill_normal(DT_F32, tmp.p, rows * cols, seed * 0x100000001B3ull + (++tensor_id), sd,
                           nullptr);
        const size_t vb = (packed_value_bytes(m.wt, rows * cols) + 255) / 256 * 256;
        char *p = (char *)m.alloc(vb + rows * cols / 32 * 4);
        launch_quantize(m.wt, tmp.as<float>(), rows, cols, p, (float *)(p + vb), nullptr);
        ESP_HIP(hipStreamSynchronize(nullptr));  // tmp is reused
        *sc = (const float *)(p + vb);
        return p;
    };
    auto cst = [&](size_t n, float v) {
        float *p = (float *)m.alloc(n * 4);
        launch_fill_const(p, n, v, nullptr);
        return p;
    };
    const size_t H = m.H;
    int rank_t[3] = {0, 0, 0};
    int lora_total = 0;
    for (int j = 0; j < 3; ++j)
        if (lora_mask & (1u << j)) {
            rank_t[j] = (int)lora_rank;
            lora_total += (int)lora_rank;
        }
    for (int l = 0; l < m.L; ++l) {
        LayerW &w = m.layers[l];
        w.in_norm = cst(H, 1.f);
        w.post_norm = cst(H, 1.f);
        w.qkv_rows = m.qw + 2 * m.kvw + lora_total;
        size_t base_rows = m.qw + 2 * m.kvw;
        if (dt_packed(m.wt)) {
            w.qkv = prj(base_rows, H, std, &w.qkv_s);
        } else {
            w.qkv = m.alloc((size_t)w.qkv_rows * H * dt_size(m.wt));
            launch_fill_normal(m.wt, w.qkv, base_rows * H, seed * 0x100000001B3ull + (++tensor_id),
                               std, nullptr);
        }
        int tcol = (int)base_rows;
        for (int j = 0; j < 3; ++j) {
            if (!rank_t[j]) continue;
            char *a = (char *)w.qkv + (size_t)tcol * H * dt_size(m.wt);
            launch_fill_normal(m.wt, a, (size_t)rank_t[j] * H, seed * 0x100000001B3ull + (++tensor_id),
                               lora_a_std, nullptr);
            size_t outf = j == 0 ? m.qw : m.kvw;
            w.lora_b[j] = rnd(outf * rank_t[j], lora_b_std);
            w.lora_rank[j] = rank_t[j];
            w.lora_t_col[j] = tcol;
            w.lora_scale[j] = lora_scale;
            tcol += rank_t[j];
        }
        if (cfg->qkv_bias) w.qkv_bias = cst(w.qkv_rows, 0.f);
        w.o = prj(H, m.qw, std, &w.o_s);
        if (cfg->output_bias) w.o_bias = cst(H, 0.f);
        if (cfg->qk_norm) {
            w.q_norm = cst(m.hd, 1.f);
            w.k_norm = cst(m.hd, 1.f);
        }
        if (!w.moe) {
            w.gate = prj(m.F, H, std, &w.gate_s);
            w.up = prj(m.F, H, std, &w.up_s);
            w.down = prj(H, m.F, std, &w.down_s);
        } else {
            w.router = rnd((size_t)m.E * H, std);
            if (m.Fs) {
                w.shared_gate = rnd(H, std);
                w.sh_gate = rnd((size_t)m.Fs * H, std);
                w.sh_up = rnd((size_t)m.Fs * H, std);
                w.sh_down = rnd((size_t)H * m.Fs, std);
            }
            w.ex_gate = rnd((size_t)m.E * m.Fe * H, std);
            w.ex_up = rnd((size_t)m.E * m.Fe * H, std);
            w.ex_down = rnd((size_t)m.E * H * m.Fe, std);
        }
    }
    m.embed = rnd_dt((size_t)m.V * H, std, m.et);
    if (cfg->tie_word_embeddings) {
        m.head = m.embed;
        m.ht = m.et;
    } else {
        m.head = prj(m.V, H, std, &m.head_s);
    }
    m.final_norm = cst(H, 1.f);
    stage_rope(m);
    ESP_HIP(hipDeviceSynchronize());
    return mp.release();
}

// ------------------------------------------------------------------- KV

Kv *create_kv(Model *m, uint32_t batch, uint32_t max_ctx, bool f16) {
    if (!m) fail(ESP_MODEL_NOT_LOADED, "model not loaded");
    if (!batch || !max_ctx || max_ctx > m->cfg.max_position_embeddings)
        fail(ESP_INVALID_REQUEST, "kv: batch must be positive and max_ctx within "
                                  "max_position_embeddings");
    if (f16 && m->wt != DT_BF16)
        fail(ESP_UNSUPPORTED, "kv: half-precision keys and values need bf16 weights");
    std::unique_ptr<Kv> kv(new Kv());
    kv->model = m;
    kv->batch = (int)batch;
    kv->max_ctx = (int)max_ctx;
    // f32 keys and values by default. The f16 cache (bf16 weights, on
    // request) halves the bytes; a CPU emulation of the f32 corridor kept it
    // within the bf16-config tolerance on 16-layer 1B-shape models (0.32-0.44
    // of the bound) but not on 32-layer 8B-shape ones (1.3-1.6x).
    kv->dt = f16 ? DT_F16 : DT_F32;
    kv->head_stride = (long long)max_ctx * m->hd;
    kv->half_stride = kv->head_stride * m->nkv;
    kv->layer_stride = kv->half_stride * 2;
    kv->seq_stride = kv->layer_stride * m->L;
    kv->cache.alloc((size_t)kv->seq_stride * batch * dt_size(kv->dt));
    kv->pos.assign(batch, 0);
    ESP_HIP(hipStreamCreateWithFlags(&kv->stream, hipStreamNonBlocking));
    // [0, 4096): attention merge tickets; [4096]: head ticket; then argmax
    // partials (values, ids) and the picked id
    kv->tickets.alloc((size_t)kTicketWords * 4);
    ESP_HIP(hipMemset(kv->tickets.p, 0, kv->tickets.bytes));
    kv->rope_row.alloc((size_t)2 * m->hd * 4);
    (void)attn_xcd_mode();  // one-time dispatch probe, outside any graph capture
    return kv.release();
}

// ---------------------------------------------------------------- forward

// Byte address of layer l's block in the cache (element type kv.dt).
static void *kv_layer(Kv &kv, int l) {
    return (char *)kv.cache.p + (size_t)l * kv.layer_stride * dt_size(kv.dt);
}

static const int kMaxRows = 4096;  // token rows per pass through the layers

static void ensure_pinned(Kv &kv, size_t bytes) {
    if (kv.pinned_bytes >= bytes) return;
    if (kv.pinned) ESP_HIP(hipHostFree(kv.pinned));
    kv.pinned = nullptr;
    kv.pinned_bytes = 0;
    ESP_HIP(hipHostMalloc(&kv.pinned, bytes, hipHostMallocDefault));
    kv.pinned_bytes = bytes;
}

struct Plan {
    int n_split, split_len;
    int max_t = 0;
};

static Plan attn_plan(const Model &m, int rows, int max_t) {
    int base = rows * m.nkv;
    int want = (512 + base - 1) / base;  // aim for >= 512 blocks of >= 64 keys
    int max_split = (max_t + 63) / 64;
    int ns = std::max(1, std::min(want, max_split));
    int sl = (max_t + ns - 1) / ns;
    sl = (sl + 31) / 32 * 32;
    ns = (max_t + sl - 1) / sl;
    return Plan{ns, sl};
}

static unsigned long long *att_tickets(Kv &kv) { return kv.tickets.as<unsigned long long>(); }

// The XCD-local attention merge assumes every split of a (row, kv head)
// runs on one XCD (attn_xcd_mode's probe). Each launch checks that
// placement on the device; a violation sets this flag, read back when the
// forward's stream drains: the forward is then computed again with the
// agent-scope merge, which every placement tolerates (xcd_merge_failed).
static int32_t *xcd_err_word(Kv &kv) { return kv.tickets.as<int32_t>() + kXcdErr; }

// lo plane of a split activation buffer holding rows x cols (nullptr for f32)
static void *lo_plane(Dt act, const DevMem &b, int rows, int cols) {
    return act == DT_SPLIT ? (void *)((uint16_t *)b.p + (size_t)rows * cols) : nullptr;
}

// GEMM weight operand: packed projections are dequantized to f32 first
// (into slot 0 or 1 of kv.deq, in stream order before the GEMM reading it)
// and multiplied by the f32 GEMM.
static const void *gemm_w(Kv &kv, int slot, Dt wt, const void *w, const float *ws, size_t N,
                          size_t K) {
    if (!dt_packed(wt)) return w;
    DevMem &d = kv.deq[slot];
    d.ensure(N * K * 4);
    launch_dequant(wt, w, ws, N * K, d.as<float>(), kv.stream);
    return d.p;
}
static Dt gemm_dt(Dt wt) { return dt_packed(wt) ? DT_F32 : wt; }
// Layer GEMMs of packed models run on the matrix cores in doubled-K form:
// weights dequantized to [N, 2K] bf16 rows [hi | lo] (kernel comment in
// k_moe.hip), activations (split planes) widened to [hi | hi], [lo | 0].
static const void *gemm_w_split(Kv &kv, int slot, Dt wt, const void *w, const float *ws, size_t N,
                                size_t K) {
    if (!dt_packed(wt)) return w;
    DevMem &d = kv.deq[slot];
    d.ensure(N * K * 4);
    launch_dequant_split(wt, w, ws, N, K, d.as<uint16_t>(), kv.stream);
    return d.p;
}
static Dt layer_gemm_dt(Dt wt) { return dt_packed(wt) ? DT_BF16 : wt; }
static void widen_k(const Model &m, Kv &kv, GemmArgs &g) {
    if (!dt_packed(m.wt)) return;
    if (g.M >= 1024 && g.K % 32 == 0 && !g.grp_offs) {
        // the streamed GEMM reads the planes twice itself and skips the
        // zero lo half (GemmArgs::kdup): no widened copy, 3/4 of the MFMAs
        g.kdup = g.K;
        g.K = 2 * g.K;
        return;
    }
    const size_t M = g.M, K = g.K;
    kv.wide.ensure(M * K * 8);
    uint16_t *hi2 = kv.wide.as<uint16_t>(), *lo2 = hi2 + M * 2 * K;
    launch_widen_split((const uint16_t *)g.a, (const uint16_t *)g.a_lo, M, K, hi2, lo2, kv.stream);
    g.a = hi2;
    g.a_lo = lo2;
    g.K = (int)(2 * K);
}
// element type of LoRA B rows (packed formats carry no LoRA)
static Dt lora_dt(Dt wt) { return dt_packed(wt) ? DT_F32 : wt; }

// Split-K decode attention of Mc rows (each row its own query position)
// into kv.attn (f32), with the plan from attn_decode_splits.
// With `lora` (a single decode row whose QKV launch stored the LoRA t rows),
// the attention adds the adapters' deltas to q and to the new key/value row.
static AttnDecodeArgs attn_decode_args(Model &m, Kv &kv, const Rows &rows, int Mc, int l,
                                       const LayerW &w, const Plan &plan, Dt out_dt, bool lora) {
    AttnDecodeArgs a{};
    if (lora) {
        a.lora_on = 1;
        a.lora_b_f32 = lora_dt(m.wt) == DT_F32;
        for (int j = 0; j < 3; ++j) {
            if (!w.lora_rank[j]) continue;
            a.lora_b[j] = w.lora_b[j];
            a.lora_t[j] = kv.qkv.as<float>() + w.lora_t_col[j];
            a.lora_rank[j] = w.lora_rank[j];
            a.lora_scale[j] = w.lora_scale[j];
        }
        a.rope_cos = m.rope_cos;
        a.rope_sin = m.rope_sin;
        a.lora_vec = !a.lora_b_f32;
        for (int j = 0; j < 3; ++j)
            if (w.lora_rank[j] && (w.lora_rank[j] % 8 || w.lora_t_col[j] % 4)) a.lora_vec = 0;
        // the QKV launch copied the position's rope rows (single decode row)
        a.lora_fast = a.lora_vec && Mc == 1 && kv.rope_row.p && m.hd % 64 == 0;
        for (int j = 0; j < 3; ++j)
            if (w.lora_rank[j] > 16) a.lora_fast = 0;
        a.rope_row = kv.rope_row.as<float>();
    }
    a.q = kv.q.as<float>();
    a.kv = kv_layer(kv, l);
    a.kv_f16 = kv.dt == DT_F16;
    a.seq_stride = kv.seq_stride;
    a.kv_half_stride = kv.half_stride;
    a.head_stride = kv.head_stride;
    a.row_pos = rows.row_pos;
    a.row_seq = rows.row_seq;
    a.seq1 = rows.seq1;
    a.grp = rows.grp;
    a.ngrp = rows.ngrp;
    a.M = Mc;
    a.nq = m.nq;
    a.nkv = m.nkv;
    a.hd = m.hd;
    a.window = w.window;
    a.max_t = plan.max_t;
    a.n_split = plan.n_split;
    a.split_len = plan.split_len;
    a.part = kv.part.as<float>();
    a.ticket = att_tickets(kv);
    a.xcd_err = xcd_err_word(kv);
    a.out = kv.attn.as<float>();
    a.out_lo = (uint16_t *)lo_plane(out_dt, kv.attn, Mc, m.qw);
    return a;
}

static void attn_decode_rows(Model &m, Kv &kv, const Rows &rows, int Mc, int l, const LayerW &w,
                             const Plan &plan, Dt out_dt = DT_F32, bool lora = false) {
    AttnDecodeArgs a = attn_decode_args(m, kv, rows, Mc, l, w, plan, out_dt, lora);
    if (plan.n_split > 1) kv.att_merged = true;
    launch_attn_decode(a, kv.stream);
}

// Whether Mc rows take the split-K decode attention kernel.
static bool use_attn_decode(const Model &m, const Kv &kv, int Mc) {
    return (kv.dt == DT_F32 || kv.dt == DT_F16) && attn_decode_ok(m.hd, m.nq / m.nkv) &&
           (long long)Mc * m.nkv <= ATT_MAX_TICKETS;
}

// One layer for a single token row with the decode kernels: fused
// QKV+RoPE+KV-append (when the layer has no QK norm; a LoRA layer first
// computes its t = A.norm(x) rows), split-K attention with in-kernel merge,
// and norm-fused projections.
static void run_layer_decode(Model &m, Kv &kv, const Rows &rows, LayerW &w, int l,
                             const Plan &plan) {
    hipStream_t s = kv.stream;
    const int H = m.H;
    void *kvl = kv_layer(kv, l);
    const bool lora = w.lora_rank[0] || w.lora_rank[1] || w.lora_rank[2];
    const bool attn_fast = attn_decode_ok(m.hd, m.nq / m.nkv);
    // LoRA deltas ride the decode attention, so a LoRA layer takes the fused
    // QKV launch only when that attention runs
    if (!w.q_norm && decode_gemv_ok(H) && (!lora || attn_fast)) {
        const int qkv_n = m.qw + 2 * m.kvw;
        DecodeGemvArgs g{};
        g.w = w.qkv;
        g.ws = w.qkv_s;
        g.x = kv.h.as<float>();
        g.gamma = w.in_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.bias = w.qkv_bias;
        g.N = m.qw + 2 * m.kvw;
        g.K = H;
        g.rope_cos = m.rope_cos;
        g.rope_sin = m.rope_sin;
        g.row_pos = rows.row_pos;
        g.row_seq = rows.row_seq;
        g.q_out = kv.q.as<float>();
        g.kv = kvl;
        g.kv_f16 = kv.dt == DT_F16;
        g.seq_stride = kv.seq_stride;
        g.kv_half_stride = kv.half_stride;
        g.head_stride = kv.head_stride;
        g.nq = m.nq;
        g.nkv = m.nkv;
        g.hd = m.hd;
        if (lora) {  // t = A . norm(x) rows, in their qkv-buffer columns
            g.lora_rows = w.qkv_rows - qkv_n;
            g.lora_t_out = kv.qkv.as<float>() + qkv_n;
            g.rope_row = kv.rope_row.as<float>();
        }
        Prof p("gemv_qkv", s);
        launch_decode_gemv(m.wt, DG_QKVROPE, g, s);
    } else {
        if (decode_gemv_ok(H)) {
            DecodeGemvArgs g{};
            g.w = w.qkv;
            g.ws = w.qkv_s;
            g.x = kv.h.as<float>();
            g.gamma = w.in_norm;
            g.eps = m.cfg.rms_norm_eps;
            g.bias = w.qkv_bias;
            g.y = kv.qkv.as<float>();
            g.N = w.qkv_rows;
            g.K = H;
            Prof p("gemv_qkv", s);
            launch_decode_gemv(m.wt, DG_STORE, g, s);
        } else {
            GemvArgs g{};
            g.w = w.qkv;
            g.x = kv.h.as<float>();
            g.gamma = w.in_norm;
            g.eps = m.cfg.rms_norm_eps;
            g.bias = w.qkv_bias;
            g.y = kv.qkv.as<float>();
            g.N = w.qkv_rows;
            g.K = H;
            Prof p("gemv", s);
            launch_gemv(m.wt, GEMV_STORE, g, s);
        }
        RopeKvArgs r{};
        r.qkv = kv.qkv.as<float>();
        r.ldq = w.qkv_rows;
        r.q_out = kv.q.as<float>();
        r.rope_cos = m.rope_cos;
        r.rope_sin = m.rope_sin;
        r.q_norm = w.q_norm;
        r.k_norm = w.k_norm;
        r.eps = m.cfg.rms_norm_eps;
        for (int j = 0; j < 3; ++j) {
            r.lora_b[j] = w.lora_b[j];
            r.lora_t_col[j] = w.lora_t_col[j];
            r.lora_rank[j] = w.lora_rank[j];
            r.lora_scale[j] = w.lora_scale[j];
        }
        r.rows = rows;
        r.kv = kvl;
        r.seq_stride = kv.seq_stride;
        r.layer_stride = kv.layer_stride;
        r.kv_half_stride = kv.half_stride;
        r.head_stride = kv.head_stride;
        r.nq = m.nq;
        r.nkv = m.nkv;
        r.hd = m.hd;
        Prof p("rope_kv", s);
        launch_rope_kv(lora_dt(m.wt), kv.dt, r, s);
    }
    if (attn_fast) {
        Prof p("attention", s);
        attn_decode_rows(m, kv, rows, 1, l, w, plan, DT_F32,
                         lora && !w.q_norm && decode_gemv_ok(H));
    } else {
        AttnArgs a{};
        a.q = kv.q.as<float>();
        a.kv = kvl;
        a.seq_stride = kv.seq_stride;
        a.layer_stride = kv.layer_stride;
        a.kv_half_stride = kv.half_stride;
        a.head_stride = kv.head_stride;
        a.rows = rows;
        a.nq = m.nq;
        a.nkv = m.nkv;
        a.hd = m.hd;
        a.window = w.window;
        a.part = kv.part.as<float>();
        a.n_split = plan.n_split;
        a.split_len = plan.split_len;
        a.out = kv.attn.p;
        a.out_dt = DT_F32;
        Prof p("attention", s);
        launch_attention(kv.dt, a, s);
    }
    auto resid = [&](const char *fam, const void *wt, const float *ws, const float *x,
                     const float *bias, int N, int K) {
        if (decode_gemv_ok(K)) {
            DecodeGemvArgs g{};
            g.w = wt;
            g.ws = ws;
            g.x = x;
            g.bias = bias;
            g.y = kv.h.as<float>();
            g.N = N;
            g.K = K;
            Prof p(fam, s);
            launch_decode_gemv(m.wt, DG_RESID, g, s);
        } else {
            GemvArgs g{};
            g.w = wt;
            g.x = x;
            g.bias = bias;
            g.y = kv.h.as<float>();
            g.N = N;
            g.K = K;
            Prof p(fam, s);
            launch_gemv(m.wt, GEMV_RESIDUAL, g, s);
        }
    };
    resid("gemv_o", w.o, w.o_s, kv.attn.as<float>(), w.o_bias, H, m.qw);
    if (w.moe) {
        if (moe_decode_ok(m) && w.ex_gate) moe_decode(m, kv, w, s);
        else moe_block(m, kv, w, 1, s, l);
        return;
    }
    if (decode_gemv_ok(H)) {
        DecodeGemvArgs g{};
        g.w = w.gate;
        g.w2 = w.up;
        g.ws = w.gate_s;
        g.ws2 = w.up_s;
        g.x = kv.h.as<float>();
        g.gamma = w.post_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = kv.act.as<float>();
        g.N = m.F;
        g.K = H;
        Prof p("gemv_mlp", s);
        launch_decode_gemv(m.wt, DG_SWIGLU, g, s);
    } else {
        GemvArgs g{};
        g.w = w.gate;
        g.w2 = w.up;
        g.x = kv.h.as<float>();
        g.gamma = w.post_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = kv.act.as<float>();
        g.N = m.F;
        g.K = H;
        Prof p("gemv_mlp", s);
        launch_gemv(m.wt, GEMV_SWIGLU, g, s);
    }
    resid("gemv_down", w.down, w.down_s, kv.act.as<float>(), nullptr, H, m.F);
}

// One pass of `Mc` rows (already on the device at `rows`) through all layers.
// `x_is_gemv` selects the single-row decode kernels.
// A run of chunk rows that are consecutive positions of one sequence.
struct Seg {
    int seq, row0, len, p0;
};

static void run_layers(Model &m, Kv &kv, const Rows &rows, int Mc, int max_t, int one_seq = -1,
                       int p0 = 0, const std::vector<Seg> *segs = nullptr) {
    hipStream_t s = kv.stream;
    const bool single = Mc == 1;
    // activations keep f32 precision; bf16 models hand them to the matrix
    // cores as split hi/lo bf16 planes, f32 models as plain f32
    const Dt act = m.wt == DT_BF16 || dt_packed(m.wt) ? DT_SPLIT : DT_F32;
    const int H = m.H;
    const bool dec_attn = use_attn_decode(m, kv, Mc);
    Plan plan = attn_plan(m, Mc, max_t);
    if (dec_attn)
        plan.n_split = attn_decode_splits(m.hd, m.nkv, m.nq / m.nkv, Mc, max_t, &plan.split_len);
    plan.max_t = max_t;
    kv.part.ensure((size_t)Mc * m.nq * plan.n_split * (m.hd + ATT_PART_PAD) * 4);
    // a streamed layer's block stays reserved until its kernels are queued
    struct Release {
        Model &m;
        Kv &kv;
        ~Release() {
            if (m.st) stream_release(m, kv);
        }
    };
    // Split-K partial sums are consumed by the kernel that follows the
    // projection when it can take them (bf16 activations): the q/k/v sums by
    // the rotary/KV kernel, the o_proj and down_proj residual sums by a row
    // kernel that also applies the next RMSNorm (post-attention, or the next
    // resident layer's input norm: `pre_normed`).
    bool pre_normed = false;
    for (int l = 0; l < m.L; ++l) {
        LayerW staged;
        if (m.st) staged = stream_acquire(m, kv, l);
        Release rel{m, kv};
        LayerW &w = m.st ? staged : m.layers[l];
        if (single) {
            run_layer_decode(m, kv, rows, w, l, plan);
            continue;
        }
        bool lora_any = false;
        for (int j = 0; j < 3; ++j) lora_any |= w.lora_b[j] && w.lora_rank[j];
        int qkv_splits = 0, o_splits = 0;
        // ---- attention block (layer.rs:120-131)
        if (single) {
            GemvArgs g{};
            g.w = w.qkv;
            g.x = kv.h.as<float>();
            g.gamma = w.in_norm;
            g.eps = m.cfg.rms_norm_eps;
            g.bias = w.qkv_bias;
            g.y = kv.qkv.as<float>();
            g.N = w.qkv_rows;
            g.K = H;
            Prof p("gemv", s);
            launch_gemv(m.wt, GEMV_STORE, g, s);
        } else {
            if (!pre_normed) {
                Prof p("rmsnorm", s);
                launch_rmsnorm(kv.h.as<float>(), w.in_norm, m.cfg.rms_norm_eps, Mc, H, act,
                               kv.xn.p, nullptr, s);
            }
            GemmArgs g{};
            g.ws = kv.gemm_ws.as<float>();
            g.ws_bytes = kv.gemm_ws.bytes;
            g.a = kv.xn.p;
            g.a_lo = lo_plane(act, kv.xn, Mc, H);
            g.w = gemm_w_split(kv, 0, m.wt, w.qkv, w.qkv_s, w.qkv_rows, H);
            g.bias = w.qkv_bias;
            g.c = kv.qkv.p;
            g.M = Mc;
            g.N = w.qkv_rows;
            g.K = H;
            g.ldc = w.qkv_rows;
            if (act == DT_SPLIT && rope_kv_fusable(lora_dt(m.wt), kv.dt, m.hd, m.nq, m.nkv, lora_any))
                g.defer_splits = &qkv_splits;
            Prof p("gemm_qkv", s);
            widen_k(m, kv, g);
            launch_gemm(layer_gemm_dt(m.wt), GEMM_STORE, g, s);
        }
        pre_normed = false;
        {
            RopeKvArgs r{};
            r.qkv = kv.qkv.as<float>();
            r.ldq = w.qkv_rows;
            r.q_out = kv.q.as<float>();
            r.rope_cos = m.rope_cos;
            r.rope_sin = m.rope_sin;
            r.q_norm = w.q_norm;
            r.k_norm = w.k_norm;
            r.eps = m.cfg.rms_norm_eps;
            for (int j = 0; j < 3; ++j) {
                r.lora_b[j] = w.lora_b[j];
                r.lora_t_col[j] = w.lora_t_col[j];
                r.lora_rank[j] = w.lora_rank[j];
                r.lora_scale[j] = w.lora_scale[j];
            }
            r.rows = rows;
            r.kv = kv_layer(kv, l);
            r.seq_stride = kv.seq_stride;
            r.layer_stride = kv.layer_stride;
            r.kv_half_stride = kv.half_stride;
            r.head_stride = kv.head_stride;
            r.nq = m.nq;
            r.nkv = m.nkv;
            r.hd = m.hd;
            if (qkv_splits > 1) {
                r.part = kv.gemm_ws.as<float>();
                r.splits = qkv_splits;
                r.part_bias = w.qkv_bias;
            }
            Prof p("rope_kv", s);
            launch_rope_kv(lora_dt(m.wt), kv.dt, r, s);
        }
        bool seg_flash = segs && !segs->empty() && act == DT_SPLIT && flash_ok(m.hd);
        for (size_t i = 0; seg_flash && i < segs->size(); ++i) seg_flash = (*segs)[i].len >= 16;
        if (seg_flash) {
            // several sequences' prompt blocks: the tiled MFMA attention per block
            uint16_t *lo = (uint16_t *)lo_plane(act, kv.attn, Mc, m.qw);
            Prof p("attention", s);
            for (const Seg &g : *segs) {
                FlashArgs f{};
                f.q = kv.q.as<float>() + (size_t)g.row0 * m.qw;
                f.kv = kv_layer(kv, l);
                f.kv_f16 = kv.dt == DT_F16;
                f.seq_stride = kv.seq_stride;
                f.kv_half_stride = kv.half_stride;
                f.head_stride = kv.head_stride;
                f.seq = g.seq;
                f.p0 = g.p0;
                f.M = g.len;
                f.nq = m.nq;
                f.nkv = m.nkv;
                f.hd = m.hd;
                f.window = w.window;
                // f32 rows, or the hi plane's bf16 rows when split
                f.out = lo ? (float *)(kv.attn.as<uint16_t>() + (size_t)g.row0 * m.qw)
                           : kv.attn.as<float>() + (size_t)g.row0 * m.qw;
                f.out_lo = lo ? lo + (size_t)g.row0 * m.qw : nullptr;
                launch_flash(f, s);
            }
        } else if (one_seq >= 0 && Mc >= 16 && act == DT_SPLIT && flash_ok(m.hd)) {
            // rows are consecutive positions of one sequence: tiled MFMA attention
            FlashArgs f{};
            f.q = kv.q.as<float>();
            f.kv = kv_layer(kv, l);
            f.kv_f16 = kv.dt == DT_F16;
            f.seq_stride = kv.seq_stride;
            f.kv_half_stride = kv.half_stride;
            f.head_stride = kv.head_stride;
            f.seq = one_seq;
            f.p0 = p0;
            f.M = Mc;
            f.nq = m.nq;
            f.nkv = m.nkv;
            f.hd = m.hd;
            f.window = w.window;
            f.out = kv.attn.as<float>();
            f.out_lo = (uint16_t *)lo_plane(act, kv.attn, Mc, m.qw);
            Prof p("attention", s);
            launch_flash(f, s);
        } else if (dec_attn) {
            Prof p("attention", s);
            attn_decode_rows(m, kv, rows, Mc, l, w, plan, act);
        } else {
            AttnArgs a{};
            a.q = kv.q.as<float>();
            a.kv = kv_layer(kv, l);
            a.seq_stride = kv.seq_stride;
            a.layer_stride = kv.layer_stride;
            a.kv_half_stride = kv.half_stride;
            a.head_stride = kv.head_stride;
            a.rows = rows;
            a.nq = m.nq;
            a.nkv = m.nkv;
            a.hd = m.hd;
            a.window = w.window;
            a.part = kv.part.as<float>();
            a.n_split = plan.n_split;
            a.split_len = plan.split_len;
            a.out = kv.attn.p;
            a.out_dt = act;
            Prof p("attention", s);
            launch_attention(kv.dt, a, s);
        }
        if (single) {
            GemvArgs g{};
            g.w = w.o;
            g.x = kv.attn.as<float>();
            g.bias = w.o_bias;
            g.y = kv.h.as<float>();
            g.N = H;
            g.K = m.qw;
            Prof p("gemv", s);
            launch_gemv(m.wt, GEMV_RESIDUAL, g, s);
        } else {
            GemmArgs g{};
            g.ws = kv.gemm_ws.as<float>();
            g.ws_bytes = kv.gemm_ws.bytes;
            g.a = kv.attn.p;
            g.a_lo = lo_plane(act, kv.attn, Mc, m.qw);
            g.w = gemm_w_split(kv, 0, m.wt, w.o, w.o_s, H, m.qw);
            g.bias = w.o_bias;
            g.c = kv.h.p;
            g.M = Mc;
            g.N = H;
            g.K = m.qw;
            g.ldc = H;
            if (!w.moe && act == DT_SPLIT && resid_norm_ok(H)) g.defer_splits = &o_splits;
            Prof p("gemm_o", s);
            widen_k(m, kv, g);
            launch_gemm(layer_gemm_dt(m.wt), GEMM_RESIDUAL, g, s);
        }
        // ---- MLP block (layer.rs:147-151)
        if (w.moe) {
            moe_block(m, kv, w, Mc, s, l);
        } else if (single) {
            GemvArgs g{};
            g.w = w.gate;
            g.w2 = w.up;
            g.x = kv.h.as<float>();
            g.gamma = w.post_norm;
            g.eps = m.cfg.rms_norm_eps;
            g.y = kv.act.as<float>();
            g.N = m.F;
            g.K = H;
            {
                Prof p("gemv", s);
                launch_gemv(m.wt, GEMV_SWIGLU, g, s);
            }
            GemvArgs d{};
            d.w = w.down;
            d.x = kv.act.as<float>();
            d.y = kv.h.as<float>();
            d.N = H;
            d.K = m.F;
            Prof p("gemv", s);
            launch_gemv(m.wt, GEMV_RESIDUAL, d, s);
        } else {
            if (o_splits > 1) {
                Prof p("resid_norm", s);
                launch_resid_norm(kv.gemm_ws.as<float>(), o_splits, Mc, H, w.o_bias, kv.h.as<float>(),
                                  w.post_norm, m.cfg.rms_norm_eps, act, kv.xn.p, s);
            } else {
                Prof p("rmsnorm", s);
                launch_rmsnorm(kv.h.as<float>(), w.post_norm, m.cfg.rms_norm_eps, Mc, H, act,
                               kv.xn.p, nullptr, s);
            }
            GemmArgs g{};
            g.ws = kv.gemm_ws.as<float>();
            g.ws_bytes = kv.gemm_ws.bytes;
            g.a = kv.xn.p;
            g.a_lo = lo_plane(act, kv.xn, Mc, H);
            g.w = gemm_w_split(kv, 0, m.wt, w.gate, w.gate_s, m.F, H);
            g.w2 = gemm_w_split(kv, 1, m.wt, w.up, w.up_s, m.F, H);
            g.c = kv.act.p;
            g.c_lo = lo_plane(act, kv.act, Mc, m.F);
            g.M = Mc;
            g.N = m.F;
            g.K = H;
            g.ldc = m.F;
            {
                Prof p("gemm_mlp", s);
                widen_k(m, kv, g);
                launch_gemm(layer_gemm_dt(m.wt), GEMM_SWIGLU, g, s);
            }
            GemmArgs d{};
            d.ws = kv.gemm_ws.as<float>();
            d.ws_bytes = kv.gemm_ws.bytes;
            d.a = kv.act.p;
            d.a_lo = lo_plane(act, kv.act, Mc, m.F);
            d.w = gemm_w_split(kv, 0, m.wt, w.down, w.down_s, H, m.F);
            d.c = kv.h.p;
            d.M = Mc;
            d.N = H;
            d.K = m.F;
            d.ldc = H;
            // the next resident layer's input norm takes the partial sums
            int d_splits = 0;
            const bool next_norm = l + 1 < m.L && !m.st && act == DT_SPLIT && resid_norm_ok(H);
            if (next_norm) d.defer_splits = &d_splits;
            {
                Prof p("gemm_down", s);
                widen_k(m, kv, d);
                launch_gemm(layer_gemm_dt(m.wt), GEMM_RESIDUAL, d, s);
            }
            if (d_splits > 1) {
                Prof p("resid_norm", s);
                launch_resid_norm(kv.gemm_ws.as<float>(), d_splits, Mc, H, nullptr, kv.h.as<float>(),
                                  m.layers[l + 1].in_norm, m.cfg.rms_norm_eps, act, kv.xn.p, s);
                pre_normed = true;
            }
        }
    }
}

static void ensure_scratch(Model &m, Kv &kv, int Mc, int n_seqs) {
    const size_t H = m.H;
    int qkv_rows = 0;
    for (auto &w : m.layers) qkv_rows = std::max(qkv_rows, w.qkv_rows);
    if (qkv_rows <= 0) fail(ESP_BACKEND, "layer geometry missing: no fused q/k/v rows");
    int fmax = std::max(m.F, std::max(m.Fe, m.Fs));
    kv.h.ensure((size_t)Mc * H * 4);
    kv.xn.ensure((size_t)Mc * H * 4);
    kv.qkv.ensure((size_t)Mc * qkv_rows * 4);
    kv.q.ensure((size_t)Mc * m.qw * 4);
    kv.attn.ensure((size_t)Mc * m.qw * 4);
    kv.act.ensure((size_t)Mc * fmax * 4);
    kv.last_h.ensure((size_t)n_seqs * H * 4);
    kv.logits.ensure((size_t)std::max(n_seqs, kv.batch) * m.V * 4);
    kv.rows_dev.ensure((size_t)(4 * kMaxRows + 2 * kv.batch + 64) * 4);
    if (Mc > 1 && (m.wt == DT_BF16 || dt_packed(m.wt)))
        kv.gemm_ws.ensure((size_t)256 << 20);  // split-K partials
    if (m.E && !kv.moe_err.p) {
        kv.moe_err.ensure(64);
        launch_fill_const(kv.moe_err.as<float>(), 16, 0.f, kv.stream);
    }
}

// The sticky router status word of this KV handle (moe.rs:160-171
// refusals), raised by route_k; forward() clears it before its layers and
// reads it back with the logits.
static int32_t *moe_err_word(Kv &kv) { return kv.moe_err.as<int32_t>(); }

static void moe_fail(int32_t status) {
    if (status == 2) fail(ESP_BACKEND, "non-finite expert router");
    if (status == 3) fail(ESP_BACKEND, "invalid top-k routing mass");
    if (status) fail(ESP_BACKEND, "expert routing failed");
}

// After a forward whose status word was not read back with its results.
void moe_check(Kv &kv) {
    if (!kv.moe_err.p) return;
    int32_t st = 0;
    ESP_HIP(hipMemcpyAsync(&st, kv.moe_err.p, 4, hipMemcpyDeviceToHost, kv.stream));
    ESP_HIP(hipStreamSynchronize(kv.stream));
    moe_fail(st);
}

// Before a device-resident generation loop: no step has failed yet.
void moe_steps_reset(Kv &kv) {
    if (!kv.moe_err.p) return;
    static const int32_t none = INT32_MAX;
    ESP_HIP(hipMemcpyAsync(kv.moe_err.as<int32_t>() + 1, &none, 4, hipMemcpyHostToDevice, kv.stream));
    ESP_HIP(hipStreamSynchronize(kv.stream));
}

// After a device-resident generation loop: fail if the router failed in a
// forward the reference runs, i.e. one that fed token i < n (its step word
// is i + 1); later forwards of the last replayed chunk do not count.
void moe_check_steps(Kv &kv, uint32_t n) {
    if (!kv.moe_err.p) return;
    int32_t v = INT32_MAX;
    ESP_HIP(hipMemcpyAsync(&v, kv.moe_err.as<int32_t>() + 1, 4, hipMemcpyDeviceToHost, kv.stream));
    ESP_HIP(hipStreamSynchronize(kv.stream));
    if (v != INT32_MAX && (uint32_t)(v >> 2) <= n) moe_fail(v & 3);
}

// Head on the last row of each sequence (model.rs:531-538): final RMSNorm
// then [H] x [V, H]^T into f32 logits rows. `h_src` rows are selected by
// `row_index` (device, nullable = rows 0..n_seqs-1).
static void run_head(Model &m, Kv &kv, int n_seqs, const float *h_src, const int32_t *row_index,
                     int32_t *gen = nullptr) {
    hipStream_t s = kv.stream;
    if (n_seqs == 1 && decode_gemv_ok(m.H)) {
        int32_t *t = kv.tickets.as<int32_t>();
        DecodeGemvArgs g{};
        g.w = m.head;
        g.ws = m.head_s;
        g.x = h_src;
        g.gamma = m.final_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = kv.logits.as<float>();
        g.N = m.V;
        g.K = m.H;
        g.ticket = t + kHeadTicket;
        g.part_v = (float *)(t + kHeadTicket + 8);
        g.part_i = t + kHeadTicket + 8 + DG_MAX_PART;
        g.picked = (uint32_t *)(t + kHeadTicket + 8 + 2 * DG_MAX_PART);
        g.gen = gen;
        Prof p("gemv_head", s);
        launch_decode_gemv(m.ht, DG_HEAD, g, s);
        return;
    }
    if (n_seqs == 1) {
        GemvArgs g{};
        g.w = m.head;
        g.x = h_src;
        g.gamma = m.final_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = kv.logits.as<float>();
        g.N = m.V;
        g.K = m.H;
        Prof p("gemv", s);
        launch_gemv(m.ht, GEMV_STORE, g, s);
        return;
    }
    {
        Prof p("rmsnorm", s);
        launch_rmsnorm(h_src, m.final_norm, m.cfg.rms_norm_eps, n_seqs, m.H,
                       m.ht == DT_BF16 ? DT_SPLIT : DT_F32, kv.xn.p, row_index, s);
    }
    GemmArgs g{};
    g.ws = kv.gemm_ws.as<float>();
    g.ws_bytes = kv.gemm_ws.bytes;
    g.a = kv.xn.p;
    g.a_lo = lo_plane(m.ht == DT_BF16 ? DT_SPLIT : DT_F32, kv.xn, n_seqs, m.H);
    g.w = gemm_w(kv, 0, m.ht, m.head, m.head_s, m.V, m.H);
    g.c = kv.logits.p;
    g.M = n_seqs;
    g.N = m.V;
    g.K = m.H;
    g.ldc = m.V;
    Prof p("gemm", s);
    launch_gemm(gemm_dt(m.ht), GEMM_STORE, g, s);
}

// After a stream has drained: whether a decode-attention launch since the
// last check found a (row, kv head)'s splits on several XCDs. The flag is
// cleared and the XCD-local merge switched off for the process.
bool xcd_merge_failed(Kv &kv) {
    int32_t flag = 0;
    ESP_HIP(hipMemcpy(&flag, xcd_err_word(kv), 4, hipMemcpyDeviceToHost));
    if (!flag) return false;
    const int32_t zero = 0;
    ESP_HIP(hipMemcpy(xcd_err_word(kv), &zero, 4, hipMemcpyHostToDevice));
    attn_xcd_disable();
    prof_count("attn_xcd_fallback");
    return true;
}

static bool forward_pass(Model &m, Kv &kv, int n_seqs, const uint32_t *seqs, const uint32_t *lens,
                         const int32_t *ids);

// One forward; computed again with the agent-scope attention merge when the
// XCD-local merge's placement check failed (positions only move after a
// pass that succeeded).
void forward(Model &m, Kv &kv, int n_seqs, const uint32_t *seqs, const uint32_t *lens,
             const int32_t *ids) {
    std::unique_lock<std::recursive_mutex> streaming;
    if (m.st) streaming = std::unique_lock<std::recursive_mutex>(m.st->mu);
    const StreamMark mark = stream_mark(m);
    if (!forward_pass(m, kv, n_seqs, seqs, lens, ids)) return;
    stream_rewind(m, mark);
    if (forward_pass(m, kv, n_seqs, seqs, lens, ids))
        fail(ESP_BACKEND, "decode attention: split placement check failed with the agent-scope merge");
}

static bool forward_pass(Model &m, Kv &kv, int n_seqs, const uint32_t *seqs, const uint32_t *lens,
                         const int32_t *ids) {
    if (n_seqs <= 0) fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
    std::unique_lock<std::recursive_mutex> streaming;
    if (m.st) streaming = std::unique_lock<std::recursive_mutex>(m.st->mu);
    // validate (model.rs:548-556) before touching any state
    std::vector<int> seen(kv.batch, 0);
    long long M = 0;
    for (int i = 0; i < n_seqs; ++i) {
        if (seqs[i] >= (uint32_t)kv.batch) fail(ESP_INVALID_REQUEST, "sequence index out of range");
        if (seen[seqs[i]]++) fail(ESP_INVALID_REQUEST, "a sequence appears twice in one batch");
        long long end = (long long)kv.pos[seqs[i]] + lens[i];
        if (lens[i] == 0 || end > kv.max_ctx || end > (long long)m.cfg.max_position_embeddings)
            fail(ESP_INVALID_REQUEST, "cached input is empty or exceeds the context window");
        M += lens[i];
    }
    for (long long r = 0; r < M; ++r)
        if (ids[r] < 0 || ids[r] >= m.V) fail(ESP_INVALID_REQUEST, "token id outside the vocabulary");
    ensure_scratch(m, kv, (int)std::min<long long>(M, kMaxRows), n_seqs);
    kv.att_merged = false;
    // host row descriptors
    std::vector<int32_t> rseq(M), rpos(M);
    std::vector<int32_t> last(n_seqs);
    int max_t = 0;
    {
        long long r = 0;
        for (int i = 0; i < n_seqs; ++i) {
            for (uint32_t t = 0; t < lens[i]; ++t, ++r) {
                rseq[r] = (int32_t)seqs[i];
                rpos[r] = kv.pos[seqs[i]] + (int)t;
            }
            last[i] = (int32_t)(r - 1);
            max_t = std::max(max_t, kv.pos[seqs[i]] + (int)lens[i]);
        }
    }
    hipStream_t s = kv.stream;
    const int lastoff = 3 * kMaxRows;
    const int erroff = lastoff + kv.batch + 8;  // pinned word: the router status read back
    const int grpoff = lastoff + kv.batch + 32;  // row groups of the row attention
    ensure_pinned(kv, (size_t)(4 * kMaxRows + kv.batch + 64) * 4);
    // rows of one sequence that the matrix-core row attention serves per wave
    const int G = m.nq / m.nkv, grp_rows = G >= 1 && G <= 16 ? 16 / G : 1;
    if (kv.moe_err.p) launch_fill_const(kv.moe_err.as<float>(), 1, 0.f, s);
    int32_t *pin = (int32_t *)kv.pinned;
    int32_t *dev = kv.rows_dev.as<int32_t>();
    float *hl = kv.last_h.as<float>();
    const bool one_chunk = M <= kMaxRows;
    for (long long c0 = 0; c0 < M; c0 += kMaxRows) {
        int Mc = (int)std::min<long long>(kMaxRows, M - c0);
        ESP_HIP(hipStreamSynchronize(s));  // pinned staging buffer reuse
        memcpy(pin, ids + c0, Mc * 4);
        memcpy(pin + kMaxRows, rseq.data() + c0, Mc * 4);
        memcpy(pin + 2 * kMaxRows, rpos.data() + c0, Mc * 4);
        memcpy(pin + lastoff, last.data(), n_seqs * 4);
        // segments: runs of consecutive positions of one sequence; each is
        // cut into row groups of up to grp_rows rows
        std::vector<Seg> segs;
        int ngrp = 0;
        if (n_seqs > 1) {
            for (int r = 0; r < Mc; ++r) {
                const long long g = c0 + r;
                if (segs.empty() || rseq[g] != segs.back().seq ||
                    rpos[g] != segs.back().p0 + segs.back().len)
                    segs.push_back(Seg{rseq[g], r, 0, rpos[g]});
                segs.back().len++;
            }
            for (const Seg &sg : segs)
                for (int r = 0; r < sg.len; r += grp_rows)
                    pin[grpoff + ngrp++] = (sg.row0 + r) | (std::min(grp_rows, sg.len - r) << 16);
        }
        ESP_HIP(hipMemcpyAsync(dev, pin, (size_t)(ngrp ? grpoff + ngrp : lastoff + n_seqs) * 4,
                               hipMemcpyHostToDevice, s));
        Rows rows{dev, dev + kMaxRows, dev + 2 * kMaxRows, Mc, n_seqs == 1 ? (int)seqs[0] : -1};
        if (ngrp) {
            rows.grp = dev + grpoff;
            rows.ngrp = ngrp;
            rows.grp_rows = grp_rows;
        }
        {
            Prof p("embed", s);
            launch_embed(m.et, m.embed, rows.ids, Mc, m.H, kv.h.as<float>(), s);
        }
        if (n_seqs == 1) run_layers(m, kv, rows, Mc, max_t, (int)seqs[0], rpos[c0]);
        else run_layers(m, kv, rows, Mc, max_t, -1, 0, &segs);
        if (one_chunk) break;
        // keep the hidden state of every sequence's last row in this chunk
        for (int i = 0; i < n_seqs; ++i)
            if (last[i] >= c0 && last[i] < c0 + Mc)
                ESP_HIP(hipMemcpyAsync(hl + (size_t)i * m.H, kv.h.as<float>() + (size_t)(last[i] - c0) * m.H,
                                       (size_t)m.H * 4, hipMemcpyDeviceToDevice, s));
    }
    if (one_chunk) {
        if (n_seqs == 1) run_head(m, kv, 1, kv.h.as<float>() + (size_t)last[0] * m.H, nullptr);
        else run_head(m, kv, n_seqs, kv.h.as<float>(), dev + lastoff);
    } else {
        run_head(m, kv, n_seqs, hl, nullptr);
    }
    // The pass is left in flight (later calls on this stream, and reads of
    // the logits, are ordered after it) unless something must be read back:
    // the router status of MoE layers, a streamed layer's device checks, or
    // the placement word of a split-merging attention.
    if (kv.moe_err.p || m.st || kv.att_merged) {
        if (kv.moe_err.p)
            ESP_HIP(hipMemcpyAsync(pin + erroff, kv.moe_err.p, 4, hipMemcpyDeviceToHost, s));
        ESP_HIP(hipMemcpyAsync(pin + erroff + 1, xcd_err_word(kv), 4, hipMemcpyDeviceToHost, s));
        ESP_HIP(hipStreamSynchronize(s));
        if (m.st) stream_check(m);  // a streamed layer that failed its device checks
        if (kv.moe_err.p) moe_fail(pin[erroff]);
        if (pin[erroff + 1] && xcd_merge_failed(kv)) return true;
    }
    for (int i = 0; i < n_seqs; ++i) kv.pos[seqs[i]] += (int)lens[i];
    kv.logits_rows = n_seqs;
    return false;
}

// A stage's forward (stage.rs:471-527): `hidden` [S, H] f32 enters the
// range's first layer at absolute positions start..start+S of sequence 0;
// `out` receives the last layer's hidden rows [S, H], or with `logits` the
// final norm + head on the last row ([V] f32).
static bool forward_hidden_pass(Model &m, Kv &kv, const float *hidden, int S, int start,
                                float *out, bool logits);

void forward_hidden(Model &m, Kv &kv, const float *hidden, int S, int start, float *out,
                    bool logits) {
    if (forward_hidden_pass(m, kv, hidden, S, start, out, logits) &&
        forward_hidden_pass(m, kv, hidden, S, start, out, logits))
        fail(ESP_BACKEND, "decode attention: split placement check failed with the agent-scope merge");
}

static bool forward_hidden_pass(Model &m, Kv &kv, const float *hidden, int S, int start,
                                float *out, bool logits) {
    hipStream_t s = kv.stream;
    const int H = m.H;
    ensure_scratch(m, kv, std::min(S, kMaxRows), 1);
    if (kv.moe_err.p) launch_fill_const(kv.moe_err.as<float>(), 1, 0.f, s);
    const int lastoff = 3 * kMaxRows;
    ensure_pinned(kv, (size_t)(3 * kMaxRows + kv.batch + 64) * 4);
    int32_t *pin = (int32_t *)kv.pinned;
    int32_t *dev = kv.rows_dev.as<int32_t>();
    const int max_t = start + S;
    for (int c0 = 0; c0 < S; c0 += kMaxRows) {
        const int Mc = std::min(kMaxRows, S - c0);
        ESP_HIP(hipStreamSynchronize(s));  // pinned staging buffer reuse
        for (int r = 0; r < Mc; ++r) {
            pin[r] = 0;
            pin[kMaxRows + r] = 0;
            pin[2 * kMaxRows + r] = start + c0 + r;
        }
        pin[lastoff] = Mc - 1;
        ESP_HIP(hipMemcpyAsync(dev, pin, (size_t)(lastoff + 1) * 4, hipMemcpyHostToDevice, s));
        ESP_HIP(hipMemcpyAsync(kv.h.p, hidden + (size_t)c0 * H, (size_t)Mc * H * 4,
                               hipMemcpyHostToDevice, s));
        Rows rows{dev, dev + kMaxRows, dev + 2 * kMaxRows, Mc, 0};
        run_layers(m, kv, rows, Mc, max_t, 0, start + c0);
        if (!logits) {
            ESP_HIP(hipMemcpyAsync(out + (size_t)c0 * H, kv.h.p, (size_t)Mc * H * 4,
                                   hipMemcpyDeviceToHost, s));
        } else if (c0 + Mc == S) {
            run_head(m, kv, 1, kv.h.as<float>() + (size_t)(Mc - 1) * H, nullptr);
            ESP_HIP(hipMemcpyAsync(out, kv.logits.p, (size_t)m.V * 4, hipMemcpyDeviceToHost, s));
        }
    }
    ESP_HIP(hipStreamSynchronize(s));
    if (kv.moe_err.p) moe_check(kv);
    if (xcd_merge_failed(kv)) return true;
    kv.pos[0] = start + S;
    kv.logits_rows = logits ? 1 : 0;
    return false;
}

}  // namespace esp

namespace esp {

// One greedy decode step whose input token, position and output slot live
// in device memory (gen layout in k_basic.hip), so the step can be captured
// once and replayed: generate.rs:154-168 without the host round trip.
void decode_step_dev(Model &m, Kv &kv, int seq, int max_t, int32_t *gen) {
    hipStream_t s = kv.stream;
    ensure_scratch(m, kv, 1, 1);
    struct StepWord {
        Kv &k;
        StepWord(Kv &k_, const int32_t *w) : k(k_) { k.gen_step = w; }
        ~StepWord() { k.gen_step = nullptr; }
    } step_word(kv, gen + 1);
    Rows rows{gen, gen + 2, gen + 3, 1, seq};
    {
        Prof p("embed", s);
        launch_embed(m.et, m.embed, rows.ids, 1, m.H, kv.h.as<float>(), s);
    }
    run_layers(m, kv, rows, 1, max_t);
    if (decode_gemv_ok(m.H)) {
        run_head(m, kv, 1, kv.h.as<float>(), nullptr, gen);  // argmax + hand-off fused
        kv.logits_rows = 1;
        return;
    }
    run_head(m, kv, 1, kv.h.as<float>(), nullptr);
    kv.pick_io.ensure(64);
    PickArgs a{};
    a.logits = kv.logits.as<float>();
    a.n = 1;
    a.V = m.V;
    a.ids_out = (uint32_t *)kv.pick_io.p;
    a.flags_out = (uint8_t *)kv.pick_io.p + 16;
    {
        Prof p("pick", s);
        launch_pick(a, s);
    }
    launch_gen_step(a.ids_out, gen, s);
    kv.logits_rows = 1;
}

// Whether single-row MoE layers take the device-only decode path.
bool moe_decode_ok(const Model &m) {
    return decode_gemv_ok(m.H) && decode_gemv_ok(m.Fe) && (!m.Fs || decode_gemv_ok(m.Fs)) &&
           m.E <= 256 && m.topk <= 8;
}

// moe.rs:135-256 for one decode row, entirely on the device (capturable):
// router GEMV over RMSNorm(h), device top-k routing, one SwiGLU GEMV over
// the k selected experts' gate/up rows (expert ids read on the device) and,
// from the same pre-MoE h, the shared expert's gate and SwiGLU GEMVs; then a
// down GEMV per slot and one for the shared expert, each storing its row,
// and the combine that adds them into h in the reference's order (slots in
// ascending expert order, then the sigmoid-gated shared expert).
void moe_decode(Model &m, Kv &kv, LayerW &w, hipStream_t s) {
    const int H = m.H, E = m.E, k = m.topk;
    kv.moe_logits.ensure((size_t)E * 4);
    kv.moe_sel.ensure((size_t)k * 4);
    kv.moe_w.ensure((size_t)k * 4);
    kv.moe_slot.ensure((size_t)k * 4);
    kv.moe_offs.ensure((size_t)(E + 2) * 4);
    kv.moe_perm.ensure((size_t)k * 4);
    kv.moe_act.ensure((size_t)(k * m.Fe + m.Fs) * 4);
    kv.moe_y.ensure((size_t)k * H * 4);
    kv.moe_ys.ensure((size_t)H * 4);
    kv.moe_sg.ensure(64);
    float *act = kv.moe_act.as<float>(), *sh_act = act + (size_t)k * m.Fe;
    {
        DecodeGemvArgs r{};
        r.w = w.router;
        r.x = kv.h.as<float>();
        r.gamma = w.post_norm;
        r.eps = m.cfg.rms_norm_eps;
        r.y = kv.moe_logits.as<float>();
        r.N = E;
        r.K = H;
        Prof p("moe", s);
        launch_decode_gemv(m.wt, DG_STORE, r, s);
        RouteArgs ra{kv.moe_logits.as<float>(), 1, E, k, m.norm_topk ? 1 : 0,
                     kv.moe_sel.as<int32_t>(), kv.moe_w.as<float>(), kv.moe_offs.as<int32_t>(),
                     kv.moe_perm.as<int32_t>(), kv.moe_slot.as<int32_t>(), moe_err_word(kv), kv.gen_step};
        launch_route(ra, s);
    }
    {
        DecodeGemvArgs g{};
        g.w = w.ex_gate;
        g.w2 = w.ex_up;
        g.x = kv.h.as<float>();
        g.gamma = w.post_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = act;
        g.N = k * m.Fe;
        g.K = H;
        g.ex_sel = kv.moe_sel.as<int32_t>();
        g.ex_stride = (long long)m.Fe * H;
        g.ex_rows = m.Fe;
        g.ex_count = E;
        Prof p("gemv_mlp", s);
        launch_decode_gemv(m.wt, DG_SWIGLU, g, s);
    }
    if (m.Fs) {
        DecodeGemvArgs sg{};
        sg.w = w.shared_gate;
        sg.x = kv.h.as<float>();
        sg.gamma = w.post_norm;
        sg.eps = m.cfg.rms_norm_eps;
        sg.y = kv.moe_sg.as<float>();
        sg.N = 1;
        sg.K = H;
        DecodeGemvArgs g{};
        g.w = w.sh_gate;
        g.w2 = w.sh_up;
        g.x = kv.h.as<float>();
        g.gamma = w.post_norm;
        g.eps = m.cfg.rms_norm_eps;
        g.y = sh_act;
        g.N = m.Fs;
        g.K = H;
        Prof p("moe", s);
        launch_decode_gemv(m.wt, DG_STORE, sg, s);
        launch_decode_gemv(m.wt, DG_SWIGLU, g, s);
    }
    for (int j = 0; j < k; ++j) {
        DecodeGemvArgs d{};
        d.w = w.ex_down;
        d.x = act + (size_t)j * m.Fe;
        d.y = kv.moe_y.as<float>() + (size_t)j * H;
        d.N = H;
        d.K = m.Fe;
        d.ex_sel = kv.moe_sel.as<int32_t>();
        d.ex_stride = (long long)H * m.Fe;
        d.ex_slot = j;
        d.ex_count = E;
        Prof p("gemv_down", s);
        launch_decode_gemv(m.wt, DG_STORE, d, s);
    }
    CombineArgs c{};
    c.y = kv.moe_y.as<float>();
    c.slot = kv.moe_slot.as<int32_t>();
    c.w = kv.moe_w.as<float>();
    c.h = kv.h.as<float>();
    c.M = 1;
    c.k = k;
    c.H = H;
    if (m.Fs) {
        DecodeGemvArgs d{};
        d.w = w.sh_down;
        d.x = sh_act;
        d.y = kv.moe_ys.as<float>();
        d.N = H;
        d.K = m.Fs;
        Prof p("moe", s);
        launch_decode_gemv(m.wt, DG_STORE, d, s);
        c.ys = kv.moe_ys.as<float>();
        c.sg = kv.moe_sg.as<float>();
    }
    Prof p("moe", s);
    launch_combine(c, s);
}

// moe.rs:135-256 DecoderMlp::forward (Moe arm) for Mc rows: h += routed
// experts (+ sigmoid-gated shared expert) of RMSNorm(h). Routing, the row
// grouping, both expert GEMMs and the combine run on the device with no host
// round trip: the expert GEMMs are one grouped launch each over all experts,
// their row ranges read from the router's offsets on the device, so the
// block can be captured. A router failure is reported at the forward's end.
void moe_block(Model &m, Kv &kv, LayerW &w, int Mc, hipStream_t s, int l) {
    const Dt act = m.wt == DT_BF16 ? DT_SPLIT : DT_F32;
    const bool split = act == DT_SPLIT;
    const int H = m.H, E = m.E, k = m.topk, R = Mc * k;
    {
        Prof p("rmsnorm", s);
        launch_rmsnorm(kv.h.as<float>(), w.post_norm, m.cfg.rms_norm_eps, Mc, H, act, kv.xn.p,
                       nullptr, s);
    }
    kv.moe_logits.ensure((size_t)Mc * E * 4);
    kv.moe_sel.ensure((size_t)R * 4);
    kv.moe_w.ensure((size_t)R * 4);
    kv.moe_slot.ensure((size_t)R * 4);
    kv.moe_offs.ensure((size_t)(E + 2) * 4);
    kv.moe_perm.ensure((size_t)R * 4);
    kv.moe_x.ensure((size_t)R * H * 4);
    kv.moe_act.ensure((size_t)R * m.Fe * 4);
    kv.moe_y.ensure((size_t)R * H * 4);
    GemmArgs r{};
    r.a = kv.xn.p;
    r.a_lo = lo_plane(act, kv.xn, Mc, H);
    r.w = w.router;
    r.c = kv.moe_logits.p;
    r.M = Mc;
    r.N = E;
    r.K = H;
    r.ldc = E;
    // the router's few columns give one tile per 256 rows: K splits spread
    // it over the chip (2048 rows: 186 -> 32 us)
    r.ws = kv.gemm_ws.as<float>();
    r.ws_bytes = kv.gemm_ws.bytes;
    {
        Prof p("gemm", s);
        launch_gemm(m.wt, GEMM_STORE, r, s);
    }
    RouteArgs ra{kv.moe_logits.as<float>(), Mc, E, k, m.norm_topk ? 1 : 0,
                 kv.moe_sel.as<int32_t>(), kv.moe_w.as<float>(), kv.moe_offs.as<int32_t>(),
                 kv.moe_perm.as<int32_t>(), kv.moe_slot.as<int32_t>(), moe_err_word(kv), kv.gen_step};
    {
        Prof p("moe", s);
        launch_route(ra, s);
        if (split) {
            const uint16_t *xs = kv.xn.as<uint16_t>();
            uint16_t *xd = kv.moe_x.as<uint16_t>();
            launch_gather_rows(DT_BF16, xs, kv.moe_perm.as<int32_t>(), R, H, xd, s);
            launch_gather_rows(DT_BF16, xs + (size_t)Mc * H, kv.moe_perm.as<int32_t>(), R, H,
                               xd + (size_t)R * H, s);
        } else {
            launch_gather_rows(DT_F32, kv.xn.p, kv.moe_perm.as<int32_t>(), R, H, kv.moe_x.p, s);
        }
    }
    const size_t es = split ? 2 : 4;  // bytes per element of one plane
    char *xh = (char *)kv.moe_x.p, *ah = (char *)kv.moe_act.p;
    GemmArgs g{};
    g.ws = kv.gemm_ws.as<float>();
    g.ws_bytes = kv.gemm_ws.bytes;
    g.a = xh;
    g.a_lo = split ? xh + (size_t)R * H * es : nullptr;
    g.w = w.ex_gate;
    g.w2 = w.ex_up;
    g.c = ah;
    g.c_lo = split ? ah + (size_t)R * m.Fe * es : nullptr;
    g.M = R;
    g.N = m.Fe;
    g.K = H;
    g.ldc = m.Fe;
    g.grp_offs = kv.moe_offs.as<int32_t>();
    g.grp_n = E;
    g.grp_w_stride = (long long)m.Fe * H;
    GemmArgs d{};
    d.ws = kv.gemm_ws.as<float>();
    d.ws_bytes = kv.gemm_ws.bytes;
    d.a = g.c;
    d.a_lo = g.c_lo;
    d.w = w.ex_down;
    d.c = kv.moe_y.as<float>();
    d.M = R;
    d.N = H;
    d.K = m.Fe;
    d.ldc = H;
    d.grp_offs = g.grp_offs;
    d.grp_n = E;
    d.grp_w_stride = (long long)H * m.Fe;
    if (w.ex_gate) {
        Prof p("gemm", s);
        launch_gemm(m.wt, GEMM_SWIGLU, g, s);
        launch_gemm(m.wt, GEMM_STORE, d, s);
    } else {
        // Streamed experts (moe.rs:183-243): the router's choice comes back
        // to the host, then only the chosen experts are read, in ascending
        // order, each staged on the copy stream while the previous one's
        // GEMMs run over its own rows.
        if (!m.st) fail(ESP_BACKEND, "routed layer without experts");
        std::vector<int32_t> offs(E + 2);
        ESP_HIP(hipMemcpyAsync(offs.data(), kv.moe_offs.p, (size_t)(E + 2) * 4,
                               hipMemcpyDeviceToHost, s));
        ESP_HIP(hipStreamSynchronize(s));
        moe_fail(offs[E + 1]);
        for (int e = 0; e < E; ++e) {
            const int n = offs[e + 1] - offs[e];
            if (n <= 0) continue;
            const ExpertW x = stream_expert(m, s, l, e);
            GemmArgs ge = g, de = d;
            ge.grp_offs = de.grp_offs = nullptr;
            ge.a = xh + (size_t)offs[e] * H * es;
            ge.a_lo = split ? (char *)g.a_lo + (size_t)offs[e] * H * es : nullptr;
            ge.w = x.gate;
            ge.w2 = x.up;
            ge.c = ah + (size_t)offs[e] * m.Fe * es;
            ge.c_lo = split ? (char *)g.c_lo + (size_t)offs[e] * m.Fe * es : nullptr;
            ge.M = n;
            de.a = ge.c;
            de.a_lo = ge.c_lo;
            de.w = x.down;
            de.c = kv.moe_y.as<float>() + (size_t)offs[e] * H;
            de.M = n;
            {
                Prof p("gemm", s);
                launch_gemm(m.wt, GEMM_SWIGLU, ge, s);
                launch_gemm(m.wt, GEMM_STORE, de, s);
            }
            stream_expert_release(m, s);
        }
    }
    CombineArgs c{};
    c.y = kv.moe_y.as<float>();
    c.slot = kv.moe_slot.as<int32_t>();
    c.w = kv.moe_w.as<float>();
    c.h = kv.h.as<float>();
    c.M = Mc;
    c.k = k;
    c.H = H;
    if (m.Fs) {
        kv.moe_ys.ensure((size_t)Mc * H * 4);
        kv.moe_sg.ensure((size_t)Mc * 4);
        GemmArgs g{};
        g.ws = kv.gemm_ws.as<float>();
        g.ws_bytes = kv.gemm_ws.bytes;
        g.a = kv.xn.p;
        g.a_lo = lo_plane(act, kv.xn, Mc, H);
        g.w = w.sh_gate;
        g.w2 = w.sh_up;
        g.c = kv.act.p;
        g.c_lo = lo_plane(act, kv.act, Mc, m.Fs);
        g.M = Mc;
        g.N = m.Fs;
        g.K = H;
        g.ldc = m.Fs;
        GemmArgs d{};
        d.ws = kv.gemm_ws.as<float>();
        d.ws_bytes = kv.gemm_ws.bytes;
        d.a = kv.act.p;
        d.a_lo = g.c_lo;
        d.w = w.sh_down;
        d.c = kv.moe_ys.p;
        d.M = Mc;
        d.N = H;
        d.K = m.Fs;
        d.ldc = H;
        GemmArgs sg{};
        sg.ws = kv.gemm_ws.as<float>();
        sg.ws_bytes = kv.gemm_ws.bytes;
        sg.a = kv.xn.p;
        sg.a_lo = g.a_lo;
        sg.w = w.shared_gate;
        sg.c = kv.moe_sg.p;
        sg.M = Mc;
        sg.N = 1;
        sg.K = H;
        sg.ldc = 1;
        Prof p("gemm", s);
        launch_gemm(m.wt, GEMM_SWIGLU, g, s);
        launch_gemm(m.wt, GEMM_STORE, d, s);
        launch_gemm(m.wt, GEMM_STORE, sg, s);
        c.ys = kv.moe_ys.as<float>();
        c.sg = kv.moe_sg.as<float>();
    }
    Prof p("moe", s);
    launch_combine(c, s);
}

}  // namespace esp
