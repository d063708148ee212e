// Host side of layer streaming (streaming.hpp): the per-layer plan (names,
// shapes, dtype admission, where each tensor's bytes land), the staging
// pipeline on a copy stream, the device layer cache and the read counters.
//
// Follows crates/esp/src/infer/decoder/streaming.rs:228-322 (bounded,
// counted reads), model.rs:556-646 (read, name check, load, optional
// cache admission per layer, then run), model.rs:336-362 (first-fit cache
// of at most 128 layers within a payload budget) and model.rs:384-415
// (every layer read once and kept), with the names check of
// loader.rs:830-848.
#include "streaming.hpp"

#include <limits.h>
#include <string.h>

#include <algorithm>
#include <set>

#include "safetensors.hpp"

namespace esp {

static size_t up256(size_t x) { return (x + 255) / 256 * 256; }

Streamer::~Streamer() {
    if (copy) (void)hipStreamSynchronize(copy);
    for (int i = 0; i < 2; ++i) {
        if (stage[i]) (void)hipHostFree(stage[i]);
        if (estage[i]) (void)hipHostFree(estage[i]);
        if (copied[i]) (void)hipEventDestroy(copied[i]);
        if (freed[i]) (void)hipEventDestroy(freed[i]);
        if (ecopied[i]) (void)hipEventDestroy(ecopied[i]);
        if (efreed[i]) (void)hipEventDestroy(efreed[i]);
    }
    if (copy) (void)hipStreamDestroy(copy);
}

// Device bytes of one projection [rows, cols] and, for packed formats, the
// offset of its block scales within them.
static size_t proj_bytes(const Model &m, uint64_t rows, uint64_t cols, size_t *scales_at) {
    const size_t n = rows * cols;
    *scales_at = 0;
    if (!dt_packed(m.wt)) return n * dt_size(m.wt);
    *scales_at = up256(packed_value_bytes(m.wt, n));
    return *scales_at + n / 32 * 4;
}

static BlockLayout block_layout(const Model &m, bool moe) {
    BlockLayout b;
    size_t o = 0;
    auto f32 = [&](size_t n) {
        const size_t at = o;
        o = up256(o + n * 4);
        b.f32_elems += n;
        return at;
    };
    auto proj = [&](uint64_t rows, uint64_t cols, size_t &scales) {
        const size_t at = o;
        size_t s = 0;
        o = up256(o + proj_bytes(m, rows, cols, &s));
        scales = at + s;
        if (m.wt == DT_F32) b.f32_elems += rows * cols;
        return at;
    };
    const uint64_t H = m.H, rows = m.qw + 2 * m.kvw;
    b.in_norm = f32(H);
    b.post_norm = f32(H);
    b.qkv = proj(rows, H, b.qkv_s);
    if (m.cfg.qkv_bias) b.qkv_bias = f32(rows);
    b.o = proj(H, m.qw, b.o_s);
    if (m.cfg.output_bias) b.o_bias = f32(H);
    if (m.cfg.qk_norm) {
        b.q_norm = f32(m.hd);
        b.k_norm = f32(m.hd);
    }
    if (!moe) {
        b.gate = proj(m.F, H, b.gate_s);
        b.up = proj(m.F, H, b.up_s);
        b.down = proj(H, m.F, b.down_s);
    } else {  // routed-expert core: no packed formats (refused at load)
        size_t unused = 0;
        b.router = proj(m.E, H, unused);
        if (m.Fs) {
            b.shared_gate = proj(1, H, unused);
            b.sh_gate = proj(m.Fs, H, unused);
            b.sh_up = proj(m.Fs, H, unused);
            b.sh_down = proj(H, m.Fs, unused);
        }
    }
    b.total = o;
    return b;
}

// Bytes of one expert block: gate [Fe, H], up [Fe, H], down [H, Fe], each
// region 256-byte aligned.
static size_t expert_part(const Model &m) { return up256((size_t)m.Fe * m.H * dt_size(m.wt)); }

static const BlockLayout &layout_of(const Model &m, const Streamer &st, int l) {
    return m.layers[l].moe ? st.lay_moe : st.lay;
}

static LayerW bind(const Model &m, const BlockLayout &b, char *base, int l) {
    LayerW w;
    w.window = m.layers[l].window;
    w.moe = m.layers[l].moe;
    const bool pk = dt_packed(m.wt);
    w.in_norm = (float *)(base + b.in_norm);
    w.post_norm = (float *)(base + b.post_norm);
    w.qkv = base + b.qkv;
    w.qkv_rows = m.qw + 2 * m.kvw;
    if (m.cfg.qkv_bias) w.qkv_bias = (float *)(base + b.qkv_bias);
    w.o = base + b.o;
    if (m.cfg.output_bias) w.o_bias = (float *)(base + b.o_bias);
    if (m.cfg.qk_norm) {
        w.q_norm = (float *)(base + b.q_norm);
        w.k_norm = (float *)(base + b.k_norm);
    }
    if (w.moe) {  // experts are read per forward (ex_* stay null)
        w.router = base + b.router;
        if (m.Fs) {
            w.shared_gate = base + b.shared_gate;
            w.sh_gate = base + b.sh_gate;
            w.sh_up = base + b.sh_up;
            w.sh_down = base + b.sh_down;
        }
        return w;
    }
    w.gate = base + b.gate;
    w.up = base + b.up;
    w.down = base + b.down;
    if (pk) {
        w.qkv_s = (const float *)(base + b.qkv_s);
        w.o_s = (const float *)(base + b.o_s);
        w.gate_s = (const float *)(base + b.gate_s);
        w.up_s = (const float *)(base + b.up_s);
        w.down_s = (const float *)(base + b.down_s);
    }
    return w;
}

// loader.rs:48-85 layer_core_tensor_names: a routed-expert layer's core
// holds the router and the shared expert (when the configuration declares
// one, as the resident loader requires) in place of the dense MLP; its
// experts live in separate artifacts.
static std::vector<std::string> core_names(const Model &m, bool moe) {
    std::vector<std::string> n = {"input_layernorm.weight",
                                  "post_attention_layernorm.weight",
                                  "self_attn.q_proj.weight",
                                  "self_attn.k_proj.weight",
                                  "self_attn.v_proj.weight",
                                  "self_attn.o_proj.weight"};
    if (!moe) {
        for (const char *x : {"mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"})
            n.push_back(x);
    } else {
        n.push_back("mlp.gate.weight");
        if (m.Fs)
            for (const char *x : {"mlp.shared_expert_gate.weight", "mlp.shared_expert.gate_proj.weight",
                                  "mlp.shared_expert.up_proj.weight",
                                  "mlp.shared_expert.down_proj.weight"})
                n.push_back(x);
    }
    if (m.cfg.qkv_bias)
        for (const char *s : {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"})
            n.push_back(s);
    if (m.cfg.output_bias) n.push_back("self_attn.o_proj.bias");
    if (m.cfg.qk_norm) {
        n.push_back("self_attn.q_norm.weight");
        n.push_back("self_attn.k_norm.weight");
    }
    return n;
}

namespace {
// One host-to-device transfer of a staged artifact.
struct Piece {
    const uint8_t *src;
    size_t bytes;
    size_t dst;  // offset in the layer block, or in the raw area when `raw`
    bool raw;
};
// A check before its device addresses are known.
struct PlanCheck {
    size_t src;  // block offset, or raw offset for widening ops
    size_t dst;  // block offset of the widened f32 region
    uint64_t n;
    int op, tag;
};
struct Plan {
    std::vector<Piece> pieces;
    std::vector<PlanCheck> checks;
    std::vector<std::string> tags;
    std::vector<int> tag_scales;
    size_t raw_used = 0;
    uint64_t payload = 0;  // 4 bytes per element of every artifact tensor
};
}  // namespace

// Where every tensor of layer l's artifact goes, with the reference's
// admission checks; throws on the first refusal.
static Plan plan_layer(const Model &m, const Streamer &st,
                       const std::map<std::string, StTensor> &t, int l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    const bool moe = m.layers[l - st.first].moe;
    {
        std::set<std::string> want;
        for (auto &s : core_names(m, moe)) want.insert(p + s);
        bool same = want.size() == t.size();
        for (auto &kv : t) same = same && want.count(kv.first);
        if (!same)
            fail(ESP_INVALID_WEIGHTS, "layer " + std::to_string(l) +
                                          " tensor names do not match the declared Llama block");
    }
    Plan pl;
    for (auto &kv : t) {
        uint64_t n = 4;
        for (uint64_t d : kv.second.shape) {
            if (d && n > UINT64_MAX / d) fail(ESP_INVALID_WEIGHTS, "layer payload size overflow");
            n *= d;
        }
        if (pl.payload > UINT64_MAX - n) fail(ESP_INVALID_WEIGHTS, "layer payload size overflow");
        pl.payload += n;
    }
    const BlockLayout &b = moe ? st.lay_moe : st.lay;
    // an f32 region: in place when the artifact holds f32, else widened
    // from the raw area
    auto f32_region = [&](const StTensor &s, uint64_t n, size_t dst, int tag) {
        if (s.dtype == "F32") {
            pl.pieces.push_back({s.data, n * 4, dst, false});
            pl.checks.push_back({dst, 0, n, SC_F32, tag});
        } else {
            pl.pieces.push_back({s.data, s.bytes, pl.raw_used, true});
            pl.checks.push_back({pl.raw_used, dst, n, s.dtype == "BF16" ? SC_BF16_F32 : SC_F16_F32, tag});
            pl.raw_used = up256(pl.raw_used + s.bytes);
        }
    };
    auto tag_of = [&](const std::string &suffix, int scales) {
        pl.tags.push_back(suffix);
        pl.tag_scales.push_back(scales);
        return (int)pl.tags.size() - 1;
    };
    auto vec = [&](const char *suffix, uint64_t n, size_t dst) {
        const std::string name = p + suffix;
        const StTensor &s = expect_tensor(t, name, {n});
        check_tensor_dtype(m, name, s, true);
        f32_region(s, n, dst, tag_of(suffix, 0));
    };
    // projections of one block region in order (q | k | v share one)
    auto projs = [&](std::vector<std::pair<const char *, uint64_t>> parts, uint64_t cols,
                     size_t at, size_t scales_at) {
        size_t vo = at, so = scales_at;
        for (auto &pr : parts) {
            const std::string name = p + pr.first;
            const uint64_t rows = pr.second, n = rows * cols;
            if (dt_packed(m.wt)) {
                auto it = t.find(name);
                const StTensor &s = it->second;
                if (!check_packed_header(m, name, s, rows, cols))
                    fail(ESP_INVALID_WEIGHTS, "weight format: packed projection byte count or "
                                              "block scales are invalid (" + name + ")");
                const size_t vb = packed_value_bytes(m.wt, n), sb = n / 32 * 4;
                pl.pieces.push_back({s.data, vb, vo, false});
                pl.pieces.push_back({s.data + vb, sb, so, false});
                pl.checks.push_back({so, 0, n / 32, SC_SCALES, tag_of(pr.first, 1)});
                vo += vb;
                so += sb;
                continue;
            }
            const StTensor &s = expect_tensor(t, name, {rows, cols});
            check_tensor_dtype(m, name, s, false);
            if (m.wt == DT_BF16) {
                pl.pieces.push_back({s.data, n * 2, vo, false});
                pl.checks.push_back({vo, 0, n, SC_BF16, tag_of(pr.first, 0)});
                vo += n * 2;
            } else {
                f32_region(s, n, vo, tag_of(pr.first, 0));
                vo += n * 4;
            }
        }
    };
    const uint64_t H = m.H, qw = m.qw, kvw = m.kvw;
    vec("input_layernorm.weight", H, b.in_norm);
    vec("post_attention_layernorm.weight", H, b.post_norm);
    projs({{"self_attn.q_proj.weight", qw}, {"self_attn.k_proj.weight", kvw},
           {"self_attn.v_proj.weight", kvw}},
          H, b.qkv, b.qkv_s);
    if (m.cfg.qkv_bias) {
        vec("self_attn.q_proj.bias", qw, b.qkv_bias);
        vec("self_attn.k_proj.bias", kvw, b.qkv_bias + qw * 4);
        vec("self_attn.v_proj.bias", kvw, b.qkv_bias + (qw + kvw) * 4);
    }
    projs({{"self_attn.o_proj.weight", H}}, qw, b.o, b.o_s);
    if (m.cfg.output_bias) vec("self_attn.o_proj.bias", H, b.o_bias);
    if (m.cfg.qk_norm) {
        vec("self_attn.q_norm.weight", (uint64_t)m.hd, b.q_norm);
        vec("self_attn.k_norm.weight", (uint64_t)m.hd, b.k_norm);
    }
    if (!moe) {
        projs({{"mlp.gate_proj.weight", (uint64_t)m.F}}, H, b.gate, b.gate_s);
        projs({{"mlp.up_proj.weight", (uint64_t)m.F}}, H, b.up, b.up_s);
        projs({{"mlp.down_proj.weight", H}}, (uint64_t)m.F, b.down, b.down_s);
    } else {
        projs({{"mlp.gate.weight", (uint64_t)m.E}}, H, b.router, 0);
        if (m.Fs) {
            projs({{"mlp.shared_expert_gate.weight", 1}}, H, b.shared_gate, 0);
            projs({{"mlp.shared_expert.gate_proj.weight", (uint64_t)m.Fs}}, H, b.sh_gate, 0);
            projs({{"mlp.shared_expert.up_proj.weight", (uint64_t)m.Fs}}, H, b.sh_up, 0);
            projs({{"mlp.shared_expert.down_proj.weight", H}}, (uint64_t)m.Fs, b.sh_down, 0);
        }
    }
    if ((int)pl.checks.size() > kStreamMaxChecks) fail(ESP_BACKEND, "layer plan: too many regions");
    return pl;
}

// An expert artifact (loader.rs:137-168 load_expert): exactly the three
// projections of expert e of layer l ([Fe, H], [Fe, H], [H, Fe]), admitted
// like the layer's own projections; tag 3 * e + part.
static Plan plan_expert(const Model &m, const std::map<std::string, StTensor> &t, int l, int e) {
    const std::string p = "model.layers." + std::to_string(l) + ".mlp.experts." + std::to_string(e) + ".";
    static const char *parts[3] = {"gate_proj.weight", "up_proj.weight", "down_proj.weight"};
    {
        bool same = t.size() == 3;
        for (const char *x : parts) same = same && t.count(p + x);
        if (!same) fail(ESP_INVALID_WEIGHTS, "expert artifact names disagree with layer/expert selection");
    }
    Plan pl;
    const uint64_t H = m.H, Fe = m.Fe;
    const size_t part = expert_part(m);
    for (int i = 0; i < 3; ++i) {
        const std::string name = p + parts[i];
        const uint64_t rows = i < 2 ? Fe : H, cols = i < 2 ? H : Fe, n = rows * cols;
        const StTensor &s = expect_tensor(t, name, {rows, cols});
        check_tensor_dtype(m, name, s, false);
        const size_t dst = (size_t)i * part;
        if (m.wt == DT_BF16) {
            pl.pieces.push_back({s.data, n * 2, dst, false});
            pl.checks.push_back({dst, 0, n, SC_BF16, 3 * e + i});
        } else if (s.dtype == "F32") {
            pl.pieces.push_back({s.data, n * 4, dst, false});
            pl.checks.push_back({dst, 0, n, SC_F32, 3 * e + i});
        } else {  // f32 model, half-precision artifact: widened on the device
            pl.pieces.push_back({s.data, s.bytes, pl.raw_used, true});
            pl.checks.push_back({pl.raw_used, dst, n, s.dtype == "BF16" ? SC_BF16_F32 : SC_F16_F32,
                                 3 * e + i});
            pl.raw_used = up256(pl.raw_used + s.bytes);
        }
    }
    return pl;
}

void streamer_init(Model &m, const esp_layer_source &src, const esp_streaming_options &opt,
                   int first) {
    auto st = std::make_shared<Streamer>();
    st->first = first;
    st->src = src;
    st->opt = opt;
    st->lay = block_layout(m, false);
    st->lay_moe = block_layout(m, true);
    size_t widest = 0, f32e = 0;
    for (int l = 0; l < m.L; ++l) {
        const BlockLayout &b = layout_of(m, *st, l);
        widest = std::max(widest, b.total);
        f32e = std::max(f32e, b.f32_elems);
    }
    // The device block is at least as wide as any admissible encoding of
    // its tensors, so a valid artifact fits in the block size plus its
    // header.
    st->stage_cap = (size_t)std::min<uint64_t>(opt.max_layer_bytes, widest + (1u << 20));
    st->raw_cap = f32e * 2 + kStreamMaxChecks * 256;
    if (m.E) {
        st->eblock_bytes = 3 * expert_part(m);
        st->estage_cap = (size_t)std::min<uint64_t>(opt.max_layer_bytes, st->eblock_bytes + (1u << 20));
        st->eraw_cap = m.wt == DT_F32 ? 3 * expert_part(m) / 2 + 3 * 256 : 0;
        for (int i = 0; i < 2; ++i) {
            ESP_HIP(hipEventCreateWithFlags(&st->ecopied[i], hipEventDisableTiming));
            ESP_HIP(hipEventCreateWithFlags(&st->efreed[i], hipEventDisableTiming));
        }
        st->ebad.alloc((size_t)m.L * 4);
    }
    ESP_HIP(hipStreamCreateWithFlags(&st->copy, hipStreamNonBlocking));
    for (int i = 0; i < 2; ++i) {
        ESP_HIP(hipEventCreateWithFlags(&st->copied[i], hipEventDisableTiming));
        ESP_HIP(hipEventCreateWithFlags(&st->freed[i], hipEventDisableTiming));
    }
    st->bad.alloc((size_t)m.L * 4);
    std::vector<int> clean(m.L, INT_MAX);
    ESP_HIP(hipMemcpy(st->bad.p, clean.data(), (size_t)m.L * 4, hipMemcpyHostToDevice));
    if (st->ebad.p)
        ESP_HIP(hipMemcpy(st->ebad.p, clean.data(), (size_t)m.L * 4, hipMemcpyHostToDevice));
    m.st = st;
}

// Read layer l through the source, plan it and queue its transfer and
// device checks. The block is `perm` (a cache or resident block) or the
// slot's transient block; `compute` runs the checks and then the layer.
static LayerW stage_layer(Model &m, hipStream_t compute, int l, DevMem *perm, uint64_t *payload) {
    Streamer &st = *m.st;
    const int sl = st.next;
    st.next ^= 1;
    ESP_HIP(hipEventSynchronize(st.copied[sl]));  // this staging buffer's last transfer is done
    if (!st.stage[sl]) ESP_HIP(hipHostMalloc((void **)&st.stage[sl], st.stage_cap, hipHostMallocDefault));
    uint64_t len = 0;
    const int gl = l + st.first;  // the layer's index in the whole model
    const int rc = (int)st.src.read_layer(st.src.user, (uint32_t)gl, st.opt.max_layer_bytes,
                                          st.stage[sl], st.stage_cap, &len);
    if (rc != ESP_OK)
        fail(rc > 0 && rc <= ESP_UNSUPPORTED ? (esp_status)rc : ESP_BACKEND,
             "layer " + std::to_string(gl) + ": layer source read failed");
    if (len > st.opt.max_layer_bytes)
        fail(ESP_INVALID_WEIGHTS, "layer source exceeded its byte limit");
    if (len > st.stage_cap)
        fail(ESP_INVALID_WEIGHTS, "layer " + std::to_string(gl) + ": artifact of " +
                                      std::to_string(len) +
                                      " bytes exceeds the declared block's encoded size");
    ++st.reads;
    st.bytes += len;
    st.largest = std::max<uint64_t>(st.largest, len);
    std::map<std::string, StTensor> t;
    try {
        t = parse_safetensors(st.stage[sl], (size_t)len);
    } catch (const Error &e) {
        fail(ESP_INVALID_WEIGHTS, "layer " + std::to_string(gl) + ": " + e.msg);
    }
    Plan pl = plan_layer(m, st, t, gl);
    const int kind = m.layers[l].moe ? 1 : 0;
    if (st.tag_names[kind].empty()) {
        st.tag_names[kind] = pl.tags;
        st.tag_scales[kind] = pl.tag_scales;
    }
    *payload = pl.payload;
    const BlockLayout &lay = layout_of(m, st, l);
    if (perm) perm->alloc(lay.total);
    else if (!st.block[sl].p) st.block[sl].alloc(std::max(st.lay.total, st.lay_moe.total));
    char *base = (char *)(perm ? perm->p : st.block[sl].p);
    if (pl.raw_used && !st.raw[sl].p) st.raw[sl].alloc(st.raw_cap);
    char *raw = (char *)st.raw[sl].p;
    // the transfer waits until the layer that last used this slot is done
    ESP_HIP(hipStreamWaitEvent(st.copy, st.freed[sl], 0));
    for (const Piece &pc : pl.pieces)
        ESP_HIP(hipMemcpyAsync((pc.raw ? raw : base) + pc.dst, pc.src, pc.bytes,
                               hipMemcpyHostToDevice, st.copy));
    ESP_HIP(hipEventRecord(st.copied[sl], st.copy));
    ESP_HIP(hipStreamWaitEvent(compute, st.copied[sl], 0));
    StreamChecks c{};
    c.n = (int)pl.checks.size();
    for (int i = 0; i < c.n; ++i) {
        const PlanCheck &k = pl.checks[i];
        const bool widen = k.op == SC_BF16_F32 || k.op == SC_F16_F32;
        c.d[i].src = widen ? (const void *)(raw + k.src) : (const void *)(base + k.src);
        c.d[i].dst = widen ? (float *)(base + k.dst) : nullptr;
        c.d[i].n = k.n;
        c.d[i].op = k.op;
        c.d[i].tag = k.tag;
    }
    launch_stream_check(c, st.bad.as<int>() + l, compute);
    st.pending = true;
    st.cur_slot = sl;
    return bind(m, lay, base, l);
}

ExpertW stream_expert(Model &m, hipStream_t compute, int l, int e) {
    Streamer &st = *m.st;
    const int gl = l + st.first;
    if (!st.src.read_expert) fail(ESP_INVALID_WEIGHTS, "layer source has no expert reader");
    const int sl = st.enext;
    st.enext ^= 1;
    ESP_HIP(hipEventSynchronize(st.ecopied[sl]));  // this staging buffer's last transfer is done
    if (!st.estage[sl])
        ESP_HIP(hipHostMalloc((void **)&st.estage[sl], st.estage_cap, hipHostMallocDefault));
    uint64_t len = 0;
    const int rc = (int)st.src.read_expert(st.src.user, (uint32_t)gl, (uint32_t)e,
                                           st.opt.max_layer_bytes, st.estage[sl], st.estage_cap, &len);
    if (rc != ESP_OK)
        fail(rc > 0 && rc <= ESP_UNSUPPORTED ? (esp_status)rc : ESP_BACKEND,
             "layer " + std::to_string(gl) + " expert " + std::to_string(e) +
                 ": expert source read failed");
    if (len > st.opt.max_layer_bytes)  // moe.rs:214-218
        fail(ESP_INVALID_WEIGHTS, "expert source exceeded artifact budget");
    if (len > st.estage_cap)
        fail(ESP_INVALID_WEIGHTS, "layer " + std::to_string(gl) + " expert " + std::to_string(e) +
                                      ": artifact exceeds the declared expert's encoded size");
    ++st.ereads;
    st.ebytes += len;
    st.elargest = std::max<uint64_t>(st.elargest, len);
    std::map<std::string, StTensor> t;
    try {
        t = parse_safetensors(st.estage[sl], (size_t)len);
    } catch (const Error &err) {
        fail(ESP_INVALID_WEIGHTS, "layer " + std::to_string(gl) + " expert " + std::to_string(e) +
                                      ": " + err.msg);
    }
    Plan pl = plan_expert(m, t, gl, e);
    if (!st.eblock[sl].p) st.eblock[sl].alloc(st.eblock_bytes);
    if (pl.raw_used && !st.eraw[sl].p) st.eraw[sl].alloc(st.eraw_cap);
    char *base = (char *)st.eblock[sl].p, *raw = (char *)st.eraw[sl].p;
    // the transfer waits until the expert that last used this slot is done
    ESP_HIP(hipStreamWaitEvent(st.copy, st.efreed[sl], 0));
    for (const Piece &pc : pl.pieces)
        ESP_HIP(hipMemcpyAsync((pc.raw ? raw : base) + pc.dst, pc.src, pc.bytes,
                               hipMemcpyHostToDevice, st.copy));
    ESP_HIP(hipEventRecord(st.ecopied[sl], st.copy));
    ESP_HIP(hipStreamWaitEvent(compute, st.ecopied[sl], 0));
    StreamChecks c{};
    c.n = (int)pl.checks.size();
    for (int i = 0; i < c.n; ++i) {
        const PlanCheck &k = pl.checks[i];
        const bool widen = k.op == SC_BF16_F32 || k.op == SC_F16_F32;
        c.d[i].src = widen ? (const void *)(raw + k.src) : (const void *)(base + k.src);
        c.d[i].dst = widen ? (float *)(base + k.dst) : nullptr;
        c.d[i].n = k.n;
        c.d[i].op = k.op;
        c.d[i].tag = k.tag;
    }
    launch_stream_check(c, st.ebad.as<int>() + l, compute);
    st.pending = true;
    st.ecur = sl;
    const size_t part = expert_part(m);
    return ExpertW{base, base + part, base + 2 * part};
}

void stream_expert_release(Model &m, hipStream_t compute) {
    Streamer &st = *m.st;
    if (st.ecur >= 0) (void)hipEventRecord(st.efreed[st.ecur], compute);
    st.ecur = -1;
}

LayerW stream_acquire(Model &m, Kv &kv, int l) {
    Streamer &st = *m.st;
    for (auto &e : st.cache)
        if (e.layer == l) {
            if (st.cache_on) ++st.hits;
            st.cur_slot = -1;
            return e.w;
        }
    if (st.cache_on) ++st.misses;
    // Admission needs the artifact's payload, known once its header is
    // parsed: the layer is staged into the transient block and, when
    // admitted, copied into a kept block on the compute stream after its
    // checks.
    uint64_t payload = 0;
    LayerW w = stage_layer(m, kv.stream, l, nullptr, &payload);
    if (st.cache_on && st.cache.size() < 128 && payload <= st.budget - st.payload) {
        const BlockLayout &lay = layout_of(m, st, l);
        std::unique_ptr<DevMem> mem(new DevMem(lay.total));
        ESP_HIP(hipMemcpyAsync(mem->p, st.block[st.cur_slot].p, lay.total,
                               hipMemcpyDeviceToDevice, kv.stream));
        LayerW kept = bind(m, lay, (char *)mem->p, l);
        st.payload += payload;
        StreamEntry e;
        e.layer = l;
        e.mem = std::move(mem);
        e.w = kept;
        e.payload = payload;
        st.cache.push_back(std::move(e));
        return kept;
    }
    return w;
}

void stream_release(Model &m, Kv &kv) {
    Streamer &st = *m.st;
    if (st.cur_slot >= 0) (void)hipEventRecord(st.freed[st.cur_slot], kv.stream);
    st.cur_slot = -1;
}

void stream_check(Model &m) {
    Streamer &st = *m.st;
    if (!st.pending) return;
    st.pending = false;
    std::vector<int> bad(m.L), ebad(m.L, INT_MAX);
    ESP_HIP(hipMemcpy(bad.data(), st.bad.p, (size_t)m.L * 4, hipMemcpyDeviceToHost));
    if (st.ebad.p) ESP_HIP(hipMemcpy(ebad.data(), st.ebad.p, (size_t)m.L * 4, hipMemcpyDeviceToHost));
    for (int l = 0; l < m.L; ++l) {
        if (ebad[l] != INT_MAX) {  // an expert that failed its checks (never kept)
            std::vector<int> clean(m.L, INT_MAX);
            ESP_HIP(hipMemcpy(st.ebad.p, clean.data(), (size_t)m.L * 4, hipMemcpyHostToDevice));
            static const char *parts[3] = {"gate_proj", "up_proj", "down_proj"};
            fail(ESP_INVALID_WEIGHTS, "weight format: non-finite weight in model.layers." +
                                          std::to_string(l + st.first) + ".mlp.experts." +
                                          std::to_string(ebad[l] / 3) + "." + parts[ebad[l] % 3] +
                                          ".weight");
        }
        if (bad[l] == INT_MAX) continue;
        for (auto it = st.cache.begin(); it != st.cache.end(); ++it)
            if (it->layer == l) {  // errors are never cached (streaming.rs:101-110)
                st.payload -= it->payload;
                st.cache.erase(it);
                break;
            }
        std::vector<int> clean(m.L, INT_MAX);
        ESP_HIP(hipMemcpy(st.bad.p, clean.data(), (size_t)m.L * 4, hipMemcpyHostToDevice));
        const int tag = bad[l], kind = m.layers[l].moe ? 1 : 0;
        const std::string name = "model.layers." + std::to_string(l + st.first) + "." +
                                 (tag < (int)st.tag_names[kind].size() ? st.tag_names[kind][tag] : "?");
        if (tag < (int)st.tag_scales[kind].size() && st.tag_scales[kind][tag])
            fail(ESP_INVALID_WEIGHTS, "weight format: packed projection byte count or block scales "
                                      "are invalid (" + name + ")");
        fail(ESP_INVALID_WEIGHTS, "weight format: non-finite weight in " + name);
    }
}

void stream_set_cache(Model &m, uint64_t budget) {
    Streamer &st = *m.st;
    ESP_HIP(hipDeviceSynchronize());  // no forward still reads a cached block
    st.cache.clear();
    st.payload = st.hits = st.misses = 0;
    st.budget = budget;
    st.cache_on = budget != 0;
}

void stream_make_resident(Model &m) {
    Streamer &st = *m.st;
    ESP_HIP(hipDeviceSynchronize());
    std::vector<std::unique_ptr<DevMem>> blocks;
    std::vector<LayerW> ws;
    for (int l = 0; l < m.L; ++l) {
        blocks.emplace_back(new DevMem());
        uint64_t payload = 0;
        ws.push_back(stage_layer(m, st.copy, l, blocks.back().get(), &payload));
        ESP_HIP(hipEventRecord(st.freed[st.cur_slot], st.copy));
        st.cur_slot = -1;
        if (!ws.back().moe) continue;
        // loader.rs:196-210 ExpertMode::Resident: every expert read once and
        // kept, in the resident loader's [E][Fe][H] / [E][H][Fe] layout
        const size_t part = (size_t)m.Fe * m.H * dt_size(m.wt);
        blocks.emplace_back(new DevMem(3 * part * m.E));
        char *kept = (char *)blocks.back()->p;
        for (int e = 0; e < m.E; ++e) {
            ExpertW x = stream_expert(m, st.copy, l, e);
            for (int i = 0; i < 3; ++i)
                ESP_HIP(hipMemcpyAsync(kept + ((size_t)i * m.E + e) * part,
                                       i == 0 ? x.gate : i == 1 ? x.up : x.down, part,
                                       hipMemcpyDeviceToDevice, st.copy));
            stream_expert_release(m, st.copy);
        }
        ws.back().ex_gate = kept;
        ws.back().ex_up = kept + part * m.E;
        ws.back().ex_down = kept + 2 * part * m.E;
    }
    ESP_HIP(hipStreamSynchronize(st.copy));
    stream_check(m);
    for (int l = 0; l < m.L; ++l) {
        ws[l].window = m.layers[l].window;
        m.layers[l] = ws[l];
    }
    for (auto &b : blocks) {
        m.weight_bytes += b->bytes;
        m.mem.push_back(std::move(b));
    }
    m.st.reset();
}

StreamMark stream_mark(const Model &m) {
    StreamMark k{};
    if (!m.st) return k;
    const Streamer &st = *m.st;
    k.reads = st.reads;
    k.bytes = st.bytes;
    k.largest = st.largest;
    k.ereads = st.ereads;
    k.ebytes = st.ebytes;
    k.elargest = st.elargest;
    k.payload = st.payload;
    k.hits = st.hits;
    k.misses = st.misses;
    k.cached = st.cache.size();
    return k;
}

void stream_rewind(Model &m, const StreamMark &k) {
    if (!m.st) return;
    Streamer &st = *m.st;
    // the pass ran to its end (no check failed, so nothing was evicted): the
    // layers it admitted are the entries after the mark
    ESP_HIP(hipStreamSynchronize(st.copy));
    while (st.cache.size() > k.cached) st.cache.pop_back();
    st.reads = k.reads;
    st.bytes = k.bytes;
    st.largest = k.largest;
    st.ereads = k.ereads;
    st.ebytes = k.ebytes;
    st.elargest = k.elargest;
    st.payload = k.payload;
    st.hits = k.hits;
    st.misses = k.misses;
}

void stream_stats(const Model &m, esp_streaming_stats *o) {
    memset(o, 0, sizeof(*o));
    if (!m.st) return;
    const Streamer &st = *m.st;
    o->streamed = 1;
    o->layer_reads = st.reads;
    o->encoded_bytes_read = st.bytes;
    o->largest_encoded_layer = st.largest;
    o->expert_reads = st.ereads;
    o->expert_encoded_bytes_read = st.ebytes;
    o->largest_encoded_expert = st.elargest;
    if (st.cache_on) {
        o->device_cache = 1;
        o->cache_hits = st.hits;
        o->cache_misses = st.misses;
        o->retained_payload_bytes = st.payload;
        o->payload_budget_bytes = st.budget;
        o->cached_layers = st.cache.size();
    }
}

}  // namespace esp
