// Layer streaming: a model whose decoder layers arrive from a host-owned
// source once per forward (crates/esp/src/infer/decoder/streaming.rs,
// model.rs:196-415, loader.rs:830-848).
//
// Per layer, the host parses only the artifact's safetensors header and
// checks names, shapes and dtype admission; the tensor bytes go by DMA from
// pinned staging straight to their place in a device layer block on a copy
// stream, two blocks alternating so the next layer's transfer overlaps the
// current layer's kernels. One device pass per layer then checks finiteness
// (and packed block scales) and widens the few tensors whose artifact dtype
// differs from the device layout (norms and biases, or every tensor of an
// f32 model fed bf16 / f16 artifacts). A failed check is reported when the
// forward ends, before any position advances.
#pragma once

#include <mutex>

#include "runtime.hpp"

namespace esp {

// One region check of a staged layer block (k_stream.hip).
enum StreamOp { SC_BF16 = 0, SC_F32 = 1, SC_SCALES = 2, SC_BF16_F32 = 3, SC_F16_F32 = 4 };
struct StreamCheck {
    const void *src;  // the region itself (SC_BF16/F32/SCALES) or its raw artifact bytes
    float *dst;       // widened f32 destination (SC_*_F32), else null
    uint64_t n;       // elements
    int op;           // StreamOp
    int tag;          // reported when the check fails
};
constexpr int kStreamMaxChecks = 24;
struct StreamChecks {
    StreamCheck d[kStreamMaxChecks];
    int n;
};
// Runs every check of one layer; the smallest failing tag lands in *bad
// (atomic min; *bad starts at INT_MAX).
void launch_stream_check(const StreamChecks &c, int *bad, hipStream_t s);

// Byte offsets of one dense layer's tensors inside its device block, every
// region 256-byte aligned. Packed projections keep their values then (at
// the next 256-byte boundary) their block scales, as the resident loader
// lays them out.
struct BlockLayout {
    size_t in_norm = 0, post_norm = 0, qkv = 0, qkv_s = 0, qkv_bias = 0, o = 0, o_s = 0,
           o_bias = 0, q_norm = 0, k_norm = 0, gate = 0, gate_s = 0, up = 0, up_s = 0, down = 0,
           down_s = 0;
    // a routed-expert layer's core (loader.rs:66-85): router, shared expert
    // gate and shared expert projections in place of the dense MLP
    size_t router = 0, shared_gate = 0, sh_gate = 0, sh_up = 0, sh_down = 0;
    size_t total = 0;
    size_t f32_elems = 0;  // elements of f32 regions (bound on widening sources)
};

// One routed expert staged in HBM: [Fe, H], [Fe, H], [H, Fe] in the model's
// weight type.
struct ExpertW {
    void *gate = nullptr, *up = nullptr, *down = nullptr;
};

struct StreamEntry {
    int layer = -1;
    std::unique_ptr<DevMem> mem;
    LayerW w;
    uint64_t payload = 0;
};

struct Streamer {
    esp_layer_source src{};
    int first = 0;  // global index of local layer 0 (a stage's range start)
    esp_streaming_options opt{};
    BlockLayout lay, lay_moe;  // dense and routed-expert layer blocks
    // logical verified reads (streaming.rs:228-252)
    uint64_t reads = 0, bytes = 0, largest = 0;
    // device layer cache (model.rs:336-362, 560-646)
    bool cache_on = false;
    uint64_t budget = 0, payload = 0, hits = 0, misses = 0;
    std::vector<StreamEntry> cache;
    // the tensor suffix of each check tag (the same for every layer of one
    // kind: [0] dense, [1] routed-expert core)
    std::vector<std::string> tag_names[2];
    std::vector<int> tag_scales[2];  // 1 when the tag checks packed block scales
    // pipeline
    uint8_t *stage[2] = {nullptr, nullptr};
    size_t stage_cap = 0;
    DevMem block[2], raw[2];
    size_t raw_cap = 0;
    hipStream_t copy = nullptr;
    hipEvent_t copied[2] = {nullptr, nullptr}, freed[2] = {nullptr, nullptr};
    int next = 0, cur_slot = -1;
    bool pending = false;  // device checks queued since the last stream_check
    DevMem bad;  // int[L], INT_MAX when clean
    // routed experts (moe.rs:207-243, streaming.rs:252-260): read per forward
    // through src.read_expert for the experts the router chose, two staging
    // slots alternating on the copy stream; checks report 3 * expert + part
    // into ebad[l]
    size_t eblock_bytes = 0, estage_cap = 0, eraw_cap = 0;
    uint8_t *estage[2] = {nullptr, nullptr};
    DevMem eblock[2], eraw[2];
    hipEvent_t ecopied[2] = {nullptr, nullptr}, efreed[2] = {nullptr, nullptr};
    int enext = 0, ecur = -1;
    uint64_t ereads = 0, ebytes = 0, elargest = 0;
    DevMem ebad;  // int[L], INT_MAX when clean
    std::recursive_mutex mu;
    ~Streamer();
};

void streamer_init(Model &m, const esp_layer_source &src, const esp_streaming_options &opt,
                   int first = 0);
// The weights of layer l for a forward on kv's stream: a cached block, or
// the layer read through the source and staged into the next transient
// block. stream_release marks the end of the layer's kernels.
LayerW stream_acquire(Model &m, Kv &kv, int l);
void stream_release(Model &m, Kv &kv);
// After the forward's stream has drained: report (and evict from the
// cache) the first layer whose device checks failed.
void stream_check(Model &m);
// Expert e of local layer l, read through the source and staged for the
// kernels on `compute` (moe.rs:207-243); stream_expert_release marks the end
// of the kernels that read it.
ExpertW stream_expert(Model &m, hipStream_t compute, int l, int e);
void stream_expert_release(Model &m, hipStream_t compute);
void stream_set_cache(Model &m, uint64_t budget);
void stream_make_resident(Model &m);
void stream_stats(const Model &m, esp_streaming_stats *out);
// The read and cache counters (and cache size) before a pass that may have
// to run again; stream_rewind restores them and drops the layers the pass
// admitted, so a repeated pass counts as the one forward it stands for.
struct StreamMark {
    uint64_t reads, bytes, largest, ereads, ebytes, elargest, payload, hits, misses;
    size_t cached;
};
StreamMark stream_mark(const Model &m);
void stream_rewind(Model &m, const StreamMark &k);

}  // namespace esp
