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
//    When the active set is one JSON-string position, a per-vocabulary
//    table of each token's string class (cstr_class_k) replaces the walk
//    for every token that stays inside the string. Tokens whose frontier
//    outgrows a lane are then walked by their whole wave, one entry per
//    lane; only frontiers above 64 entries are left to the block kernel.
//  - cmask_block_k: one block per token left over, frontier in global
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

constexpr uint64_t NO_ENTRY = ~0ull;

// The successor of one unclosed entry on `b` when the entry is not at a
// Split node (at most one: constraint.rs:172-245), or NO_ENTRY. `w` is the
// entry's node word.
__device__ __forceinline__ uint64_t succ1(uint64_t e, uint32_t w, uint32_t b) {
    const uint32_t lo = (uint32_t)e;
    const uint32_t used = (uint32_t)(e >> 32);
    const uint32_t node = lo & CN_NODE_MASK;
    const uint32_t phase = (lo >> 17) & 7;
    const uint32_t cls = (lo >> 20) & 7;
    const uint32_t kind = w >> 30;
    if (phase == 0) {
        if (kind == 1) return ((w >> 22) & 0xff) == b ? at_entry(w & CN_NODE_MASK) : NO_ENTRY;
        if (kind == 2) return b == '"' ? (uint64_t)(node | 1u << 17) : NO_ENTRY;
        return NO_ENTRY;
    }
    // content of a String node (constraint.rs:180-243)
    const uint32_t max = (w >> 17) & 0x1fff;
    if (phase == 1 && b == '"') return used > 0 ? at_entry(w & CN_NODE_MASK) : NO_ENTRY;
    if (used >= max) return NO_ENTRY;
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
            return NO_ENTRY;
        }
    } else if (phase == 2) {
        const bool esc = b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' ||
                         b == 'r' || b == 't';
        if (!esc) return NO_ENTRY;
        np = 1;
    } else {
        // continuation byte in [low, high] of the class
        const uint32_t low = (uint32_t)(0x809080a080ull >> (cls * 8)) & 0xff;
        const uint32_t high = (uint32_t)(0x8fbf9fbfbfull >> (cls * 8)) & 0xff;
        if (b < low || b > high) return NO_ENTRY;
        np = phase == 3 ? 1 : phase - 1;
        nc = 0;
    }
    return (uint64_t)node | (uint64_t)np << 17 | (uint64_t)nc << 20 | (uint64_t)(used + 1) << 32;
}

__device__ __forceinline__ bool is_split_entry(uint64_t e, uint32_t w) {
    return ((uint32_t)e & (7u << 17)) == 0 && (w >> 30) == 3;
}

// Members of Split word `w` that accept `b`: [*l, *h).
__device__ __forceinline__ void split_members(const uint32_t *__restrict__ split_off,
                                              const uint32_t *__restrict__ members, uint32_t w,
                                              uint32_t b, uint32_t *l_out, uint32_t *h_out) {
    const uint32_t s = w & 0x3fffffffu;
    uint32_t l = split_off[s], h = split_off[s + 1];
    const uint32_t end = h;
    const uint32_t key = b << 17;
    while (l < h) {  // first member with accepted byte >= b
        const uint32_t mid = (l + h) >> 1;
        if (members[mid] < key) l = mid + 1;
        else h = mid;
    }
    h = l;
    while (h < end && (members[h] >> 17) == b) ++h;
    *l_out = l;
    *h_out = h;
}

// The successor of Split member `m` (a Byte or String node) on the byte it
// accepts.
__device__ __forceinline__ uint64_t member_succ(const uint32_t *__restrict__ nodes, uint32_t m) {
    const uint32_t mw = nodes[m];
    return (mw >> 30) == 1 ? at_entry(mw & CN_NODE_MASK) : (uint64_t)(m | 1u << 17);
}

// Every successor of one unclosed entry on `b`, passed to emit(u64).
template <class Emit>
__device__ __forceinline__ void cstep(const uint32_t *__restrict__ nodes,
                                      const uint32_t *__restrict__ split_off,
                                      const uint32_t *__restrict__ members, uint64_t e,
                                      uint32_t b, Emit &&emit) {
    const uint32_t w = nodes[(uint32_t)e & CN_NODE_MASK];
    if (is_split_entry(e, w)) {
        uint32_t l, h;
        split_members(split_off, members, w, b, &l, &h);
        for (uint32_t i = l; i < h; ++i) emit(member_succ(nodes, members[i] & CN_NODE_MASK));
    } else {
        const uint64_t s = succ1(e, w, b);
        if (s != NO_ENTRY) emit(s);
    }
}

// String-content class of one token from one start state, for an
// unbounded JSON string automaton (constraint.rs:180-243 without the
// bound). Start states: 0 phase 1; 1 phase 2; 2 phase 3; 3..5 phase 4 with
// continuation class 0..2; 6..8 phase 5 with class 0, 3, 4; 9 before the
// opening quote (phase 0). Result: kind (bits 1:0: 0 dies, 1 stays inside
// the string, 2 closes it at token byte `at`), C (bits 15:2) = the least
// room (max - used) the content bytes need, `at` (bits 29:16).
__device__ uint32_t str_class(const uint8_t *__restrict__ t, uint32_t len, int state) {
    uint32_t phase, cls = 0, i = 0, k = 0, need = 0;
    if (state == 9) {
        if (t[0] != '"') return 0;
        phase = 1;
        i = 1;
    } else {
        phase = state == 0 ? 1 : state == 1 ? 2 : state == 2 ? 3 : state <= 5 ? 4 : 5;
        cls = state <= 2 ? 0 : state == 3 ? 0 : state == 4 ? 1 : state == 5 ? 2
            : state == 6 ? 0 : state == 7 ? 3 : 4;
    }
    for (; i < len; ++i, ++k) {
        const uint32_t b = t[i];
        if (phase == 1 && b == '"') return 2u | need << 2 | i << 16;
        need = max(need, k + 1);
        if (phase == 1) {
            if (b == '\\') {
                need = max(need, k + 2);
                phase = 2;
            } else if (b >= 0x20 && b <= 0x7f && b != '"') {
            } else if (b >= 0xc2 && b <= 0xdf) {
                need = max(need, k + 2);
                phase = 3;
                cls = 0;
            } else if (b >= 0xe0 && b <= 0xef) {
                need = max(need, k + 3);
                phase = 4;
                cls = b == 0xe0 ? 1 : b == 0xed ? 2 : 0;
            } else if (b >= 0xf0 && b <= 0xf4) {
                need = max(need, k + 4);
                phase = 5;
                cls = b == 0xf0 ? 3 : b == 0xf4 ? 4 : 0;
            } else {
                return 0;
            }
        } else if (phase == 2) {
            if (!(b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' ||
                  b == 'r' || b == 't'))
                return 0;
            phase = 1;
        } else {
            const uint32_t low = (uint32_t)(0x809080a080ull >> (cls * 8)) & 0xff;
            const uint32_t high = (uint32_t)(0x8fbf9fbfbfull >> (cls * 8)) & 0xff;
            if (b < low || b > high) return 0;
            phase = phase == 3 ? 1 : phase - 1;
            cls = 0;
        }
    }
    return 1u | need << 2;
}

__global__ __launch_bounds__(256) void cstr_class_k(const uint8_t *__restrict__ tok,
                                                    const uint32_t *__restrict__ off, int V,
                                                    uint32_t *__restrict__ out) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= V) return;
    const uint32_t o0 = off[t], len = off[t + 1] - o0;
#pragma unroll 1
    for (int st = 0; st < CSTR_STATES; ++st)
        out[(size_t)st * V + t] = len ? str_class(tok + o0, len, st) : 0;
}

// Exclusive prefix sum over the wave.
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v) {
    const int lane = threadIdx.x & 63;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x - v;
}

__global__ __launch_bounds__(256) void cmask_lane_k(const CRow *__restrict__ rows,
                                                    uint32_t *__restrict__ status,
                                                    uint64_t *__restrict__ ovf, int lane_cap,
                                                    int wave_cap) {
    __shared__ uint64_t stage_all[4][64];
    uint64_t *stage = stage_all[threadIdx.x >> 6];
    const CRow &r = rows[blockIdx.y];
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int lane = threadIdx.x & 63;
    bool ok = false, over = false;
    uint32_t o0 = 0, o1 = 0;
    if (t < r.V) {
        o0 = r.tok_off[t];
        o1 = r.tok_off[t + 1];
        uint64_t cur[KF];
#pragma unroll
        for (int j = 0; j < KF; ++j) cur[j] = 0;
        int n = 0;
        uint32_t i0 = o1;
        if (r.mode == 1) {
            // single JSON-string position: the token's class decides, and
            // only a token that closes the string walks on from `next`
            const uint32_t w = r.scls[t];
            const uint32_t kind = w & 3, need = (w >> 2) & 0x3fff, at = w >> 16;
            const uint32_t k = at - (r.s_state == 9 ? 1u : 0u);
            if (kind == 1) {
                ok = r.s_used + need <= r.s_max;
            } else if (kind == 2 && r.s_used + need <= r.s_max && r.s_used + k > 0) {
                cur[0] = at_entry(r.s_next);
                n = 1;
                i0 = o0 + at + 1;
                ok = i0 == o1;
            }
        } else if (o1 > o0) {
            const uint32_t b0 = r.tok[o0];
            const uint32_t f0 = r.first_off[b0];
            n = (int)(r.first_off[b0 + 1] - f0);
            if (n > lane_cap) {
                over = true;
                n = 0;
            } else {
#pragma unroll
                for (int j = 0; j < KF; ++j) cur[j] = j < n ? r.first[f0 + j] : 0;
                i0 = o0 + 1;
                ok = n > 0 && i0 == o1;
            }
        }
        if (n > 0 && i0 < o1) {
            for (uint32_t i = i0; i < o1 && n > 0 && !over; ++i) {
                const uint32_t b = r.tok[i];
                uint64_t nxt[KF];
#pragma unroll
                for (int j = 0; j < KF; ++j) nxt[j] = 0;
                int nn = 0;
                // insert at the front unless present; nxt[0..nn) stay distinct
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
                    for (int j = KF - 1; j > 0; --j) nxt[j] = nxt[j - 1];
                    nxt[0] = s;
                    ++nn;
                };
                // entries are taken from cur[0], rotating the rest forward
                for (int j = 0; j < n && !over; ++j) {
                    const uint64_t e = cur[0];
#pragma unroll
                    for (int q = 0; q < KF - 1; ++q) cur[q] = cur[q + 1];
                    const uint32_t w = r.nodes[(uint32_t)e & CN_NODE_MASK];
                    if (is_split_entry(e, w)) {
                        uint32_t l, h;
                        split_members(r.split_off, r.members, w, b, &l, &h);
                        for (uint32_t m = l; m < h && !over; ++m)
                            push(member_succ(r.nodes, r.members[m] & CN_NODE_MASK));
                    } else {
                        const uint64_t sx = succ1(e, w, b);
                        if (sx != NO_ENTRY) push(sx);
                    }
                }
#pragma unroll
                for (int j = 0; j < KF; ++j) cur[j] = nxt[j];
                n = nn;
            }
            ok = n > 0 && !over;
        }
    }
    // Wave tier: the wave walks each overflowing token of its lanes in turn,
    // one frontier entry per lane (up to wave_cap <= 64), successors
    // compacted through LDS by a prefix sum. Larger frontiers go to the
    // block kernel through the overflow list.
    uint64_t pend = __ballot(over);
    while (pend) {
        const int src = __ffsll((unsigned long long)pend) - 1;
        pend &= pend - 1;
        const uint32_t lo0 = __shfl(o0, src), lo1 = __shfl(o1, src);
        const uint32_t b0 = r.tok[lo0];
        const uint32_t f0 = r.first_off[b0];
        uint32_t live = r.first_off[b0 + 1] - f0;
        bool big = live > (uint32_t)wave_cap;
        uint64_t e = NO_ENTRY;
        if (!big && lane < (int)live) e = r.first[f0 + lane];
        for (uint32_t i = lo0 + 1; i < lo1 && live > 0 && !big; ++i) {
            const uint32_t b = r.tok[i];
            uint32_t c = 0, ml = 0;
            uint64_t s1 = NO_ENTRY;
            bool sp = false;
            if (e != NO_ENTRY) {
                const uint32_t w = r.nodes[(uint32_t)e & CN_NODE_MASK];
                if (is_split_entry(e, w)) {
                    uint32_t mh;
                    split_members(r.split_off, r.members, w, b, &ml, &mh);
                    c = mh - ml;
                    sp = true;
                } else {
                    s1 = succ1(e, w, b);
                    c = s1 != NO_ENTRY;
                }
            }
            const uint32_t pre = wave_excl_scan(c);
            const uint32_t tot = __shfl(pre + c, 63);
            if (tot > (uint32_t)wave_cap) {
                big = true;
                break;
            }
            if (sp) {
                for (uint32_t k = 0; k < c; ++k)
                    stage[pre + k] = member_succ(r.nodes, r.members[ml + k] & CN_NODE_MASK);
            } else if (c) {
                stage[pre] = s1;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            e = lane < (int)tot ? stage[lane] : NO_ENTRY;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            live = tot;
        }
        if (lane == src) {
            ok = !big && live > 0;
            over = big;
        }
    }
    const uint64_t bal = __ballot(ok);
    const uint64_t ob = __ballot(over);
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

void launch_str_class(const uint8_t *tok, const uint32_t *off, int V, uint32_t *out,
                      hipStream_t s) {
    hipLaunchKernelGGL(cstr_class_k, dim3((V + 255) / 256), dim3(256), 0, s, tok, off, V, out);
}

void launch_cmask(const CMaskLaunch &a, hipStream_t s) {
    dim3 g1((a.v_max + 255) / 256, a.n_rows);
    hipLaunchKernelGGL(cmask_lane_k, g1, dim3(256), 0, s, a.rows, a.status, a.ovf,
                       a.lane_cap < KF ? a.lane_cap : KF, a.wave_cap < 64 ? a.wave_cap : 64);
    const int bm_words = (a.n_nodes_max + 31) / 32;
    hipLaunchKernelGGL(cmask_block_k, dim3(a.blocks), dim3(256), (size_t)2 * bm_words * 4, s,
                       a.rows, a.status, (const uint64_t *)a.ovf, a.frontier, a.cap_max, bm_words);
}

}  // namespace esp
