// Byte grammar over a byte-level vocabulary (decoder/constraint.rs): the
// host automaton (compile, close, step, accept, complete, forced bytes) and
// the device tables that the batched mask kernels read.
#pragma once

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "runtime.hpp"

namespace esp {

// ---------------------------------------------------------------- host side

// Compiled node (constraint.rs:10-16). Literals become chains of Byte
// nodes, a choice becomes a Split over its alternatives' entry nodes, a
// JSON string is one String node; node 0 is End.
enum GKind : uint8_t { G_END = 0, G_BYTE = 1, G_STRING = 2, G_SPLIT = 3 };
struct GNode {
    GKind kind = G_END;
    uint8_t byte = 0;            // G_BYTE
    uint32_t next = 0;           // G_BYTE, G_STRING
    uint32_t max = 0;            // G_STRING: bound on encoded content bytes
    std::vector<uint32_t> alts;  // G_SPLIT
};

// Automaton position (constraint.rs:17-35). Ordered field by field, as the
// reference derives Ord, so sorted active sets compare equal.
struct Pos {
    uint32_t node = 0, used = 0;
    uint8_t phase = 0, low = 0, high = 0;
    static Pos at(uint32_t n) { return Pos{n, 0, 0, 0, 0}; }
    bool operator<(const Pos &o) const {
        if (node != o.node) return node < o.node;
        if (used != o.used) return used < o.used;
        if (phase != o.phase) return phase < o.phase;
        if (low != o.low) return low < o.low;
        return high < o.high;
    }
    bool operator==(const Pos &o) const {
        return node == o.node && used == o.used && phase == o.phase && low == o.low &&
               high == o.high;
    }
};

// Token byte strings of one tokenizer (the table constraint.rs:119-154
// derives from the ByteLevel alphabet). Empty = never allowed. Shared by
// every constraint built over it; copied to a device once, on first use.
struct Vocab {
    std::vector<uint8_t> bytes;
    std::vector<uint32_t> off;  // [n + 1]
    uint32_t n = 0, max_len = 0;
    std::mutex mu;
    int device = -1;
    DevMem d_bytes, d_off;
    DevMem d_scls;  // [CSTR_STATES][n] string classes (launch_str_class)
    void to_device();  // idempotent; fails if already on another device
};

// Per-call buffers of the batched mask (one set per owner: a KV handle or a
// constraint used on its own).
struct MaskCtx {
    DevMem io;        // row descriptors | first-byte tables
    DevMem status;    // [0] overflow count, [1] error flag
    DevMem ovf;       // (row << 32 | token) of tokens the lane walk could not hold
    DevMem frontier;  // block walk frontiers
    std::vector<uint8_t> stage;
};

struct Constraint {
    std::shared_ptr<Vocab> vocab;
    std::vector<GNode> nodes;
    std::vector<Pos> active;
    uint32_t n_strings = 0;
    // device tables (built on the first mask)
    int device = -1;
    DevMem d_nodes, d_split_off, d_members;
    MaskCtx ctx;

    // constraint.rs:56-157 (grammar given as the serde JSON of OutputGrammar)
    Constraint(std::shared_ptr<Vocab> v, const char *json, size_t len);
    std::vector<Pos> close(std::vector<Pos> ps) const;
    bool step1(const Pos &p, uint8_t byte, Pos &out) const;
    std::vector<Pos> step(const std::vector<Pos> &set, uint8_t byte) const;
    std::vector<Pos> after(const uint8_t *bytes, size_t n) const;
    bool complete() const;
    void accept(uint32_t id);
    std::vector<uint8_t> forced_bytes() const;
    // Successors of the active set for every first byte, unclosed and
    // deduplicated, as device entries: off[257], entries.
    void first_table(std::vector<uint32_t> &off, std::vector<uint64_t> &ent) const;
    void to_device();
    // Frontier bound of the exact block walk for the current active set.
    uint64_t frontier_cap() const;
};

// ---------------------------------------------------------------- device side

// Node word: kind in bits 31:30.
//   Byte:   byte in 29:22, next in 16:0
//   String: max in 29:17, next in 16:0
//   Split:  split index in 29:0 (members[split_off[s] .. split_off[s+1]])
// Split members: the non-Split nodes reachable through nested Splits that
// consume a byte, packed (accepted byte << 17 | node), ascending.
// Entry (a position, u64): node 16:0, phase 19:17, (low, high) class
// 22:20, used in the upper 32 bits. Classes: 0 = 80..bf, 1 = a0..bf,
// 2 = 80..9f, 3 = 90..bf, 4 = 80..8f (only meaningful in phases 3..5).
constexpr uint32_t CN_NODE_BITS = 17;
constexpr uint32_t CN_NODE_MASK = (1u << CN_NODE_BITS) - 1;

// Start states of the string-class table (see cstr_class_k).
constexpr int CSTR_STATES = 10;
// Longest token the string-class table can describe (14-bit fields).
constexpr uint32_t CSTR_MAX_LEN = 16383;

struct CRow {
    const uint32_t *nodes, *split_off, *members;
    const uint32_t *first_off;  // [257]
    const uint64_t *first;
    const uint8_t *tok;         // vocabulary bytes
    const uint32_t *tok_off;    // [V + 1]
    uint32_t *mask;             // [ceil(V / 32)] allowed bits
    int V;
    int row;
    uint64_t cap;               // block-walk frontier capacity
    // mode 1: the active set is the single JSON-string position (node with
    // bound s_max and successor s_next, `used` s_used, start state s_state);
    // scls = that state's row of the vocabulary's string-class table
    int mode;
    uint32_t s_used, s_max, s_next, s_state;
    const uint32_t *scls;
};

struct CMaskLaunch {
    const CRow *rows;   // device [n_rows]
    int n_rows;
    int v_max;          // largest V over rows
    int n_nodes_max;    // largest node count over rows (bitmap size)
    uint32_t *status;   // [0] overflow count, [1] error flag (zeroed by the launcher)
    uint64_t *ovf;      // [sum V]
    uint64_t *frontier; // [blocks][2][cap_max]
    uint64_t cap_max;
    int blocks;         // block-walk grid
    int lane_cap;       // lane frontier capacity (0 sends every live token to the wave walk)
    int wave_cap;       // wave frontier capacity (0 sends those on to the block walk)
};
void launch_cmask(const CMaskLaunch &a, hipStream_t s);
void launch_str_class(const uint8_t *tok, const uint32_t *off, int V, uint32_t *out,
                      hipStream_t s);

// Build the descriptors and first-byte tables of `n` constraints into ctx,
// then launch the mask. masks[i] is the device output of row i. The error
// flag is left in ctx.status[1] (read back by the caller).
void run_cmask(MaskCtx &ctx, Constraint *const *cs, uint32_t *const *masks, int n,
               hipStream_t s);
// Read back the status words after the stream is synchronised; fails on a
// frontier overflow.
void check_cmask(MaskCtx &ctx, hipStream_t s);

}  // namespace esp
