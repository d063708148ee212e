// Host-side runtime objects behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"

namespace esp {

// One device allocation, freed with the owner.
struct DevMem {
    void *p = nullptr;
    size_t bytes = 0;
    DevMem() = default;
    explicit DevMem(size_t n) { alloc(n); }
    DevMem(const DevMem &) = delete;
    DevMem &operator=(const DevMem &) = delete;
    ~DevMem() {
        if (p) (void)hipFree(p);
    }
    void alloc(size_t n) {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
        if (n) ESP_HIP(hipMalloc(&p, n));
        bytes = n;
    }
    // Grow-only reallocation (contents not preserved).
    void ensure(size_t n) {
        if (n > bytes) alloc(n);
    }
    template <typename T> T *as() const { return (T *)p; }
};

struct MaskCtx;   // constraint.hpp
struct Streamer;  // streaming.hpp
struct StTensor;  // safetensors.hpp

struct LayerW {
    float *in_norm = nullptr, *post_norm = nullptr;
    void *qkv = nullptr;        // [qkv_rows, H]: q | k | v | LoRA-A rows (q, k, v targets)
    float *qkv_bias = nullptr;  // [qkv_rows] or null
    int qkv_rows = 0;
    // packed formats: block scales [rows, K/32] of qkv, o, gate, up, down
    const float *qkv_s = nullptr, *o_s = nullptr, *gate_s = nullptr, *up_s = nullptr,
                *down_s = nullptr;
    void *o = nullptr;          // [H, qw]
    float *o_bias = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;
    void *gate = nullptr, *up = nullptr, *down = nullptr;  // dense
    bool moe = false;
    void *router = nullptr;       // [E, H]
    void *shared_gate = nullptr;  // [1, H]
    void *sh_gate = nullptr, *sh_up = nullptr, *sh_down = nullptr;
    void *ex_gate = nullptr, *ex_up = nullptr, *ex_down = nullptr;  // [E][F][H], [E][F][H], [E][H][F]
    // unmerged LoRA (targets 0 q, 1 k, 2 v): B [out, rank], t at qkv column t_col
    void *lora_b[3] = {nullptr, nullptr, nullptr};
    int lora_rank[3] = {0, 0, 0};
    int lora_t_col[3] = {0, 0, 0};
    float lora_scale[3] = {0, 0, 0};
    int window = 0;
};

struct Model {
    esp_config cfg{};
    Dt wt = DT_F32;  // projection weight element type
    Dt et = DT_F32;  // embedding element type (and the head's when tied)
    Dt ht = DT_F32;  // head element type
    const float *head_s = nullptr;  // packed head: block scales
    int H = 0, L = 0, nq = 0, nkv = 0, hd = 0, F = 0, V = 0, qw = 0, kvw = 0;
    int E = 0, topk = 0, Fe = 0, Fs = 0;
    bool norm_topk = false;
    std::vector<LayerW> layers;
    void *embed = nullptr;  // [V, H]
    void *head = nullptr;   // [V, H] (== embed when tied)
    float *final_norm = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos, hd]
    std::vector<std::unique_ptr<DevMem>> mem;
    uint64_t weight_bytes = 0;
    int device = 0;
    // layer streaming: layers come from a host source per forward
    // (`layers` then holds only their geometry and windows)
    std::shared_ptr<Streamer> st;

    void *alloc(size_t bytes) {
        mem.emplace_back(new DevMem(bytes));
        weight_bytes += bytes;
        return mem.back()->p;
    }
};

struct Kv {
    Model *model = nullptr;
    int batch = 0, max_ctx = 0;
    Dt dt = DT_F32;
    DevMem cache;
    long long seq_stride = 0, layer_stride = 0, half_stride = 0, head_stride = 0;
    std::vector<int> pos;  // host mirror of each sequence's position
    hipStream_t stream = nullptr;
    // scratch
    DevMem rows_dev;   // ids | row_seq | row_pos | last_row  (int32)
    DevMem h, xn, qkv, q, attn, act, part, last_h, logits, pick_scratch, pick_io;
    DevMem gemm_ws;  // split-K partial sums of the prefill GEMMs
    DevMem deq[2];   // packed formats: dequantized weights of the GEMMs in flight
    DevMem wide;     // packed formats: activation planes widened to the doubled K
    DevMem tickets;  // zeroed counters for last-block merges (attention, head argmax)
    // the decode position's rope rows (cos then sin, hd floats each), written
    // by the single-row QKV launch for the attention's LoRA deltas
    DevMem rope_row;
    DevMem moe_logits, moe_sel, moe_w, moe_slot, moe_offs, moe_perm, moe_x, moe_y, moe_ys, moe_sg,
        moe_act;
    DevMem moe_err;  // sticky router status of the forward in flight (0 = ok)
    // during esp_generate_greedy's device steps: the step counter (gen[1]),
    // so a router failure records the step it happened in (moe_err[1])
    const int32_t *gen_step = nullptr;
    int logits_rows = 0;  // rows valid in `logits`
    // set when a decode attention launch of the forward in flight merged key
    // splits (its XCD placement word must then be read back)
    bool att_merged = false;
    void *pinned = nullptr;
    size_t pinned_bytes = 0;
    // esp_pick's host staging (masks and samplers in, ids / states / flags
    // out): one DMA each way instead of copies from pageable memory
    void *pick_pinned = nullptr;
    size_t pick_pinned_bytes = 0;
    // esp_pick's upload runs on its own stream (created on first use), so
    // it overlaps the forward still running on `stream`; `pick_up` orders
    // the pick kernels after it
    hipStream_t pick_stream = nullptr;
    hipEvent_t pick_up = nullptr;
    // generation graph
    hipGraphExec_t gen_exec = nullptr;
    // grammar mask buffers of esp_pick_constrained
    std::shared_ptr<MaskCtx> cmask;
    ~Kv();
};

// The forward over prepared rows; defined in runtime.cpp.
void forward(Model &m, Kv &kv, int n_seqs, const uint32_t *seqs, const uint32_t *lens,
             const int32_t *ids);

// Checkpoint admission rules shared by the resident loader and the layer
// streamer (runtime.cpp).
const StTensor &expect_tensor(const std::map<std::string, StTensor> &t, const std::string &name,
                              const std::vector<uint64_t> &shape);
void check_tensor_dtype(const Model &m, const std::string &name, const StTensor &s,
                        bool force_f32);
bool check_packed_header(const Model &m, const std::string &name, const StTensor &s,
                         uint64_t rows, uint64_t cols);
// A model whose layers stream from `source` (model.rs:196-312): only the
// shared artifact's embedding, final norm and head are staged here.
Model *load_streamed_model(const esp_config *cfg, const uint8_t *shared, size_t len,
                           const esp_layer_source *source, const esp_streaming_options *opt);
// One stage of a layer-range chain (stage.rs:280-527): layers first..end-1
// read once from `source` and kept resident; with `shared`, the final
// norm and output head.
Model *load_stage_model(const esp_config *cfg, uint32_t first, uint32_t end,
                        const esp_layer_source *source, const esp_streaming_options *opt,
                        const uint8_t *shared, size_t shared_len);
void forward_hidden(Model &m, Kv &kv, const float *hidden, int S, int start, float *out,
                    bool logits);

}  // namespace esp
