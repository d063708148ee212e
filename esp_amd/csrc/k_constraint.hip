// Grammar mask on the device (decoder/constraint.rs:277-297 `mask`): token
// t is allowed iff its bytes are non-empty and walking them through the
// automaton from the active set leaves a non-empty set.
//
// Two kernels, both exact:
//  - cmask_lane_k: one lane per (row, token). The walk starts from the
//    row's first-byte table (the active set already stepped on each byte,
//    computed by the host) and keeps an unclosed frontier of at most KF
//    positions in registers, deduplicated on insert. A lane whose frontier
//    would exceed KF appends (row, token) to an overflow list instead.
//  - cmask_block_k: one block per overflowing token, frontier in global
//    scratch with two LDS bitmaps that deduplicate at-node entries and
//    freshly opened strings per byte (content positions of one string
//    never collide: equal `used` means equal history).
// A frontier is kept unclosed: an entry at a Split node stands for its
// closure, which is only expanded when the next byte is stepped, using the
// Split's members sorted by accepted byte.
#include "constraint.hpp"

namespace esp {

namespace {

constexpr int KF = 8;  // lane frontier registers (the capacity used is lane_cap <= KF)

__device__ __forceinline__ uint64_t at_entry(uint32_t node) { return node; }

// Successors of one unclosed entry on `b`, passed to emit(u64).
template <class Emit>
__device__ __forceinline__ void cstep(const uint32_t *__restrict__ nodes,
                                      const uint32_t *__restrict__ split_off,
                                      const uint32_t *__restrict__ members, uint64_t e,
                                      uint32_t b, Emit &&emit) {
    const uint32_t lo = (uint32_t)e;
    const uint32_t used = (uint32_t)(e >> 32);
    const uint32_t node = lo & CN_NODE_MASK;
    const uint32_t phase = (lo >> 17) & 7;
    const uint32_t cls = (lo >> 20) & 7;
    const uint32_t w = nodes[node];
    const uint32_t kind = w >> 30;
    if (phase == 0) {
        if (kind == 1) {
            if (((w >> 22) & 0xff) == b) emit(at_entry(w & CN_NODE_MASK));
        } else if (kind == 2) {
            if (b == '"') emit((uint64_t)(node | 1u << 17));
        } else if (kind == 3) {
            const uint32_t s = w & 0x3fffffffu;
            uint32_t l = split_off[s], h = split_off[s + 1];
            const uint32_t key = b << 17;
            while (l < h) {  // first member with accepted byte >= b
                uint32_t mid = (l + h) >> 1;
                if (members[mid] < key) l = mid + 1;
                else h = mid;
            }
            const uint32_t end = split_off[s + 1];
            for (uint32_t i = l; i < end; ++i) {
                const uint32_t mv = members[i];
                if ((mv >> 17) != b) break;
                const uint32_t m = mv & CN_NODE_MASK;
                const uint32_t mw = nodes[m];
                if ((mw >> 30) == 1) emit(at_entry(mw & CN_NODE_MASK));
                else emit((uint64_t)(m | 1u << 17));
            }
        }
        return;
    }
    // content of a String node (constraint.rs:180-243)
    const uint32_t max = (w >> 17) & 0x1fff;
    const uint32_t next = w & CN_NODE_MASK;
    if (phase == 1 && b == '"') {
        if (used > 0) emit(at_entry(next));
        return;
    }
    if (used >= max) return;
    uint32_t np, nc = cls;
    if (phase == 1) {
        if (b == '\\' && used + 2 <= max) {
            np = 2;
        } else if (b >= 0x20 && b <= 0x7f && b != '"' && b != '\\') {
            np = 1;
        } else if (b >= 0xc2 && b <= 0xdf && used + 2 <= max) {
            np = 3;
            nc = 0;
        } else if (b >= 0xe0 && b <= 0xef && used + 3 <= max) {
            np = 4;
            nc = b == 0xe0 ? 1 : b == 0xed ? 2 : 0;
        } else if (b >= 0xf0 && b <= 0xf4 && used + 4 <= max) {
            np = 5;
            nc = b == 0xf0 ? 3 : b == 0xf4 ? 4 : 0;
        } else {
            return;
        }
    } else if (phase == 2) {
        const bool esc = b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' ||
                         b == 'r' || b == 't';
        if (!esc) return;
        np = 1;
    } else {
        // continuation byte in [low, high] of the class
        const uint32_t low = (uint32_t)(0x809080a080ull >> (cls * 8)) & 0xff;
        const uint32_t high = (uint32_t)(0x8fbf9fbfbfull >> (cls * 8)) & 0xff;
        if (b < low || b > high) return;
        np = phase == 3 ? 1 : phase - 1;
        nc = 0;
    }
    emit((uint64_t)node | (uint64_t)np << 17 | (uint64_t)nc << 20 | (uint64_t)(used + 1) << 32);
}

__global__ __launch_bounds__(256) void cmask_lane_k(const CRow *__restrict__ rows,
                                                    uint32_t *__restrict__ status,
                                                    uint64_t *__restrict__ ovf, int lane_cap) {
    const CRow &r = rows[blockIdx.y];
    const int t = blockIdx.x * 256 + threadIdx.x;
    bool ok = false, over = false;
    if (t < r.V) {
        const uint32_t o0 = r.tok_off[t], o1 = r.tok_off[t + 1];
        if (o1 > o0) {
            const uint32_t b0 = r.tok[o0];
            const uint32_t f0 = r.first_off[b0];
            int n = (int)(r.first_off[b0 + 1] - f0);
            if (n > lane_cap) {
                over = true;
            } else if (n > 0) {
                uint64_t cur[KF];
#pragma unroll
                for (int j = 0; j < KF; ++j) cur[j] = j < n ? r.first[f0 + j] : 0;
                for (uint32_t i = o0 + 1; i < o1 && n > 0 && !over; ++i) {
                    const uint32_t b = r.tok[i];
                    uint64_t nxt[KF];
#pragma unroll
                    for (int j = 0; j < KF; ++j) nxt[j] = 0;
                    int nn = 0;
                    auto push = [&](uint64_t s) {
                        bool dup = false;
#pragma unroll
                        for (int j = 0; j < KF; ++j) dup |= j < nn && nxt[j] == s;
                        if (dup) return;
                        if (nn >= lane_cap) {
                            over = true;
                            return;
                        }
#pragma unroll
                        for (int j = 0; j < KF; ++j)
                            if (j == nn) nxt[j] = s;
                        ++nn;
                    };
#pragma unroll
                    for (int j = 0; j < KF; ++j)
                        if (j < n) cstep(r.nodes, r.split_off, r.members, cur[j], b, push);
#pragma unroll
                    for (int j = 0; j < KF; ++j) cur[j] = nxt[j];
                    n = nn;
                }
                ok = n > 0 && !over;
            }
        }
    }
    const uint64_t bal = __ballot(ok);
    const uint64_t ob = __ballot(over);
    const int lane = threadIdx.x & 63;
    const int base = blockIdx.x * 256 + (threadIdx.x & ~63);
    const int words = (r.V + 31) >> 5;
    if (lane == 0 && base < r.V) r.mask[base >> 5] = (uint32_t)bal;
    if (lane == 32 && base + 32 < r.V && (base >> 5) + 1 < words)
        r.mask[(base >> 5) + 1] = (uint32_t)(bal >> 32);
    if (ob) {
        uint32_t slot = 0;
        if (lane == 0) slot = atomicAdd(&status[0], (uint32_t)__popcll(ob));
        slot = __shfl(slot, 0);
        if (over) {
            const uint32_t k = __popcll(ob & ((1ull << lane) - 1));
            ovf[slot + k] = (uint64_t)blockIdx.y << 32 | (uint32_t)t;
        }
    }
}

__global__ __launch_bounds__(256) void cmask_block_k(const CRow *__restrict__ rows,
                                                     uint32_t *__restrict__ status,
                                                     const uint64_t *__restrict__ ovf,
                                                     uint64_t *__restrict__ frontier,
                                                     uint64_t cap_max, int bm_words) {
    extern __shared__ uint32_t bm[];  // [bm_words] at-node | [bm_words] fresh string
    __shared__ uint32_t s_n[2];  // per-byte counters, alternating
    for (int i = threadIdx.x; i < 2 * bm_words; i += 256) bm[i] = 0;
    uint64_t *buf0 = frontier + (size_t)blockIdx.x * 2 * cap_max;
    uint64_t *buf1 = buf0 + cap_max;
    const uint32_t total = __atomic_load_n(&status[0], __ATOMIC_RELAXED);
    __syncthreads();
    for (uint32_t k = blockIdx.x; k < total; k += gridDim.x) {
        const uint64_t item = ovf[k];
        const CRow &r = rows[item >> 32];
        const uint32_t t = (uint32_t)item;
        const uint32_t o0 = r.tok_off[t], o1 = r.tok_off[t + 1];
        const uint64_t cap = r.cap;
        const uint32_t b0 = r.tok[o0];
        const uint32_t f0 = r.first_off[b0];
        uint64_t n = r.first_off[b0 + 1] - f0;
        uint64_t *cur = buf0, *nxt = buf1;
        bool err = n > cap;
        if (err) n = 0;
        for (uint64_t j = threadIdx.x; j < n; j += 256) cur[j] = r.first[f0 + j];
        if (threadIdx.x == 0) s_n[0] = 0;
        int par = 0;
        for (uint32_t i = o0 + 1; i < o1 && n > 0; ++i, par ^= 1) {
            const uint32_t b = r.tok[i];
            __syncthreads();  // cur complete, s_n[par] reset
            auto emit = [&](uint64_t s) {
                const uint32_t lo = (uint32_t)s;
                const uint32_t node = lo & CN_NODE_MASK;
                const uint32_t phase = (lo >> 17) & 7;
                uint32_t *map = phase == 0 ? bm : (phase == 1 && (s >> 32) == 0) ? bm + bm_words
                                                                                : nullptr;
                if (map) {
                    const uint32_t bit = 1u << (node & 31);
                    if (atomicOr(&map[node >> 5], bit) & bit) return;
                }
                const uint32_t slot = atomicAdd(&s_n[par], 1u);
                if (slot < cap) nxt[slot] = s;
            };
            for (uint64_t j = threadIdx.x; j < n; j += 256)
                cstep(r.nodes, r.split_off, r.members, cur[j], b, emit);
            __syncthreads();  // nxt complete
            const uint64_t nn = s_n[par];
            if (threadIdx.x == 0) s_n[par ^ 1] = 0;
            if (nn > cap) {
                err = true;
                n = 0;
                break;
            }
            // clear the bits this byte set: every set bit belongs to an entry of nxt
            for (uint64_t j = threadIdx.x; j < nn; j += 256) {
                const uint64_t s = nxt[j];
                const uint32_t lo = (uint32_t)s;
                const uint32_t node = lo & CN_NODE_MASK;
                const uint32_t phase = (lo >> 17) & 7;
                if (phase == 0) bm[node >> 5] = 0;
                else if (phase == 1 && (s >> 32) == 0) bm[bm_words + (node >> 5)] = 0;
            }
            uint64_t *tmp = cur;
            cur = nxt;
            nxt = tmp;
            n = nn;
        }
        __syncthreads();  // bitmaps clear, s_n free before the next token
        if (threadIdx.x == 0) {
            if (err) {
                for (int w = 0; w < 2 * bm_words; ++w) bm[w] = 0;
                atomicOr(&status[1], 1u);
            } else if (n > 0) {
                atomicOr(&r.mask[t >> 5], 1u << (t & 31));
            }
        }
        __syncthreads();
    }
}

}  // namespace

void launch_cmask(const CMaskLaunch &a, hipStream_t s) {
    dim3 g1((a.v_max + 255) / 256, a.n_rows);
    hipLaunchKernelGGL(cmask_lane_k, g1, dim3(256), 0, s, a.rows, a.status, a.ovf,
                       a.lane_cap < KF ? a.lane_cap : KF);
    const int bm_words = (a.n_nodes_max + 31) / 32;
    hipLaunchKernelGGL(cmask_block_k, dim3(a.blocks), dim3(256), (size_t)2 * bm_words * 4, s,
                       a.rows, a.status, (const uint64_t *)a.ovf, a.frontier, a.cap_max, bm_words);
}

}  // namespace esp
