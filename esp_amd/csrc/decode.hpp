// Single-token decode kernels (k_decode.hip).
#pragma once

#include "common.hpp"

namespace esp {

enum DecodeEpi { DG_STORE = 0, DG_RESID = 1, DG_SWIGLU = 2, DG_QKVROPE = 3, DG_HEAD = 4 };
constexpr int DG_MAX_PART = 2048;  // argmax partials (blocks) of the head GEMV

struct DecodeGemvArgs {
    const void *w, *w2;   // [N, K] weight rows (SWIGLU: gate, up)
    const float *ws, *ws2;  // packed formats: [N, K/32] block scales of w, w2
    const float *x;       // [K] input row
    const float *gamma;   // nullable: fused RMSNorm of x
    float eps;
    const float *bias;    // nullable
    float *y;             // STORE/HEAD: out; RESID: +=; SWIGLU: act
    int N, K;
    // QKVROPE
    const float *rope_cos, *rope_sin;
    const int32_t *row_pos, *row_seq;  // device, one row
    float *q_out;
    void *kv;             // layer base of the cache (f16 when kv_f16, else f32)
    int kv_f16;
    long long seq_stride, kv_half_stride, head_stride;
    int nq, nkv, hd;
    // QKVROPE unmerged LoRA: the lora_rows rows after the q/k/v rows (the
    // adapters' A rows) are projected in the same launch and stored, not
    // rotated, to lora_t_out (t = A . norm(x)); the decode attention then adds
    // scale * B t (lora.rs:93-97) to q, k and v.
    int lora_rows;
    float *lora_t_out;
    // QKVROPE, nullable: block 0 also copies the rope rows at the row's
    // position here (cos then sin, hd floats each), so the attention that
    // follows reads them from a fixed address instead of after the position
    float *rope_row;
    // routed experts (moe.rs:135-256, one row): with ex_sel set, SWIGLU
    // units are (slot, row) pairs, slot = unit / ex_rows, reading expert
    // ex_sel[slot] (clamped to [0, ex_count)) of the [E][rows][K] tensors;
    // RESID and STORE read expert ex_sel[ex_slot]; RESID scales by
    // ex_w[ex_slot] when ex_w is set.
    const int32_t *ex_sel;
    const float *ex_w;
    long long ex_stride;   // elements between consecutive experts
    int ex_rows, ex_slot, ex_count;
    const float *sig_scale;  // nullable (RESID): y *= sigmoid(*sig_scale)
    // HEAD argmax
    float *part_v;
    int32_t *part_i;
    int32_t *ticket;      // nullable = no argmax
    uint32_t *picked;
    int32_t *gen;         // nullable: device-loop token hand-off
};

bool decode_gemv_ok(int K);
bool decode_gemv_packed_ok(Dt wt, int K);
void launch_decode_gemv(Dt wt, int epi, const DecodeGemvArgs &a, hipStream_t s);

struct AttnDecodeArgs {
    const float *q;       // [M, nq*hd]
    const void *kv;       // layer base of the cache (f16 when kv_f16, else f32)
    int kv_f16;
    long long seq_stride, kv_half_stride, head_stride;
    const int32_t *row_pos, *row_seq;
    int seq1;             // >= 0: every row belongs to this sequence (row_seq unread)
    int M, nq, nkv, hd, window;
    int max_t;            // plan bound: every row's position is below it
    int n_split, split_len;
    float *part;          // [M, nq, n_split, hd + 4]
    // [M, nkv] zero-initialised merge tickets: bits 0-7 count the splits
    // that arrived, bits 8 + 7x the ones that ran on XCD x
    unsigned long long *ticket;
    int32_t *xcd_err;     // set to 1 when a unit's splits ran on several XCDs
    // set by the launcher from ESP_ATT_XCD_MISPLACE=1: blocks take the
    // linear (unit, split) order under the XCD-local protocol, so the
    // placement check fires (exercises the fallback; every access stays
    // in bounds)
    int misplace;
    float *out;           // [M, nq*hd] f32, or the bf16 hi plane when out_lo is set
    uint16_t *out_lo;     // nullable: bf16 lo plane (split activation output)
    int xcd_nx;           // set by the launcher: merge protocol (0 = agent scope)
    // Unmerged LoRA of a single decode row (M == 1), targets 0 q, 1 k, 2 v:
    // with lora_on, q gets + RoPE_pos(scale_q * B_q t_q) when loaded, and the
    // key row at the row's position gets + RoPE_pos(scale_k * B_k t_k) and its
    // value row + scale_v * B_v t_v, written back to the cache by the block
    // whose split holds that position (lora.rs:93-97; RoPE is linear, so
    // RoPE(y + d) = RoPE(y) + RoPE(d)). lora_b[j] null = target j untouched.
    int lora_on, lora_b_f32;
    int lora_vec;           // bf16 B, every rank a multiple of 8, every t 16-byte aligned
    const void *lora_b[3];  // [rows, rank] bf16 (or f32 when lora_b_f32)
    const float *lora_t[3];
    int lora_rank[3];
    float lora_scale[3];
    const float *rope_cos, *rope_sin;  // [max_pos, hd]
    // With lora_fast (lora_vec, every rank <= 16, rope_row set): the deltas'
    // operands (B rows, the rope rows copied by the QKV launch) are loaded
    // before the block's first keys and the deltas are exchanged through LDS
    // without waiting for those keys.
    int lora_fast;
    const float *rope_row;
    // nullable (attn_rows_mfma_k only): row groups (Rows::grp); one unit
    // per (group, kv head) instead of per (row, kv head)
    const int32_t *grp;
    int ngrp;
};

bool attn_decode_ok(int hd, int G);
// The matrix-core form of attn_decode_k for batches without key splits
// (k_attn_mfma.hip): one wave per (row, kv head), up to 16 query heads per
// kv head, hd 64 (f16 or f32 cache) or 128 (f16 cache), no LoRA.
bool attn_rows_mfma_ok(const AttnDecodeArgs &a);
void launch_attn_rows_mfma(const AttnDecodeArgs &a, hipStream_t s);
// key splits and keys per split for M decode rows over max_t cached keys
int attn_decode_splits(int hd, int nkv, int G, int M, int max_t, int *split_len);
constexpr int ATT_MAX_TICKETS = 4096;  // (row, kv head) merge tickets at the start of Kv::tickets
constexpr int ATT_PART_PAD = 4;  // partial row = hd + ATT_PART_PAD floats
void launch_attn_decode(const AttnDecodeArgs &a, hipStream_t s);
// XCD count of the XCD-local split merge, or 0 for the agent-scope merge
// (probed once per process; environment ESP_ATT_XCD=0 forces 0)
int attn_xcd_mode();
// Switch the XCD-local merge off for the process (a launch found a unit's
// splits on several XCDs).
void attn_xcd_disable();

}  // namespace esp
