// Prefill attention on the matrix cores (k_flash.hip).
#pragma once

#include "common.hpp"

namespace esp {

struct FlashArgs {
    const float *q;    // [M, nq*hd] post-RoPE queries (f32)
    const void *kv;    // layer base of the cache (f16 when kv_f16, else f32)
    int kv_f16;
    long long seq_stride, kv_half_stride, head_stride;
    int seq, p0;       // the rows are positions p0 .. p0+M-1 of sequence `seq`
    int M, nq, nkv, hd, window;
    float *out;        // [M, nq*hd] f32, or the hi plane when out_lo is set
    uint16_t *out_lo;  // nullable: lo plane of a split output
};

bool flash_ok(int hd);
void launch_flash(const FlashArgs &a, hipStream_t s);

}  // namespace esp
