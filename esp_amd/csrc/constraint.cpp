// Host side of the byte-grammar constraint (decoder/constraint.rs) and the
// set-up of the batched device mask.
#include "constraint.hpp"

#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace esp {

namespace {

[[noreturn]] void bad(const std::string &m) { fail(ESP_INVALID_REQUEST, m); }

// ------------------------------------------------------------- grammar JSON
// OutputGrammar (provider.rs:55-75) in its serde form: an object tagged by
// "kind" (literal | json_string | sequence | choice), snake_case, unknown
// fields refused. Parsed straight into a tree; JSON nesting is limited to
// 128 levels like serde_json's default recursion limit.
struct Gram {
    int kind = -1;  // 0 literal, 1 json_string, 2 sequence, 3 choice
    std::string value;
    uint64_t max_bytes = 0;
    std::vector<Gram> kids;
};

struct Json {
    const char *p, *end;
    int depth = 0;

    [[noreturn]] void err(const std::string &m) { bad("invalid output grammar: " + m); }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) err(std::string("expected '") + c + "'");
    }
    static void put_utf8(std::string &s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xc0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            s += (char)(0xe0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        } else {
            s += (char)(0xf0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3f));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (end - p < 4) err("truncated \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else err("invalid \\u escape");
        }
        return v;
    }
    std::string str() {
        ws();
        if (p >= end || *p != '"') err("expected a string");
        ++p;
        std::string s;
        while (true) {
            if (p >= end) err("unterminated string");
            unsigned char c = (unsigned char)*p++;
            if (c == '"') break;
            if (c < 0x20) err("control character in string");
            if (c != '\\') {
                s += (char)c;
                continue;
            }
            if (p >= end) err("unterminated escape");
            char e = *p++;
            switch (e) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t cp = hex4();
                if (cp >= 0xdc00 && cp <= 0xdfff) err("lone trailing surrogate");
                if (cp >= 0xd800 && cp <= 0xdbff) {
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u') err("lone leading surrogate");
                    p += 2;
                    uint32_t lo = hex4();
                    if (lo < 0xdc00 || lo > 0xdfff) err("invalid surrogate pair");
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                }
                put_utf8(s, cp);
                break;
            }
            default: err("invalid escape");
            }
        }
        return s;
    }
    // A non-negative integer that fits u64 (serde's usize on 64-bit hosts).
    uint64_t uint() {
        ws();
        const char *q = p;
        if (p < end && *p == '-') err("invalid value: negative integer, expected usize");
        uint64_t v = 0;
        bool any = false, overflow = false;
        while (p < end && *p >= '0' && *p <= '9') {
            uint64_t d = (uint64_t)(*p - '0');
            if (v > (UINT64_MAX - d) / 10) overflow = true;
            v = v * 10 + d;
            ++p;
            any = true;
        }
        if (!any) err("invalid type: expected usize");
        if (p - q > 1 && *q == '0') err("invalid number");
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E'))
            err("invalid type: floating point, expected usize");
        if (overflow) err("number out of range for usize");
        return v;
    }
    Gram grammar() {
        if (++depth > 128) err("recursion limit exceeded");
        expect('{');
        Gram g;
        bool has_kind = false, has_value = false, has_max = false, has_items = false,
             has_alts = false;
        std::string kind;
        if (!eat('}')) {
            do {
                std::string key = str();
                expect(':');
                auto dup = [&](bool &seen) {
                    if (seen) err("duplicate field `" + key + "`");
                    seen = true;
                };
                if (key == "kind") {
                    dup(has_kind);
                    kind = str();
                } else if (key == "value") {
                    dup(has_value);
                    g.value = str();
                } else if (key == "max_bytes") {
                    dup(has_max);
                    g.max_bytes = uint();
                } else if (key == "items" || key == "alternatives") {
                    dup(key == "items" ? has_items : has_alts);
                    expect('[');
                    if (!eat(']')) {
                        do g.kids.push_back(grammar());
                        while (eat(','));
                        expect(']');
                    }
                } else {
                    err("unknown field `" + key + "`");
                }
            } while (eat(','));
            expect('}');
        }
        if (!has_kind) err("missing field `kind`");
        int fields = has_value + has_max + has_items + has_alts;
        if (kind == "literal") {
            g.kind = 0;
            if (!has_value) err("missing field `value`");
        } else if (kind == "json_string") {
            g.kind = 1;
            if (!has_max) err("missing field `max_bytes`");
        } else if (kind == "sequence") {
            g.kind = 2;
            if (!has_items) err("missing field `items`");
        } else if (kind == "choice") {
            g.kind = 3;
            if (!has_alts) err("missing field `alternatives`");
        } else {
            err("unknown variant `" + kind + "`");
        }
        if (fields != 1) err("unknown field for variant `" + kind + "`");
        --depth;
        return g;
    }
};

bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint8_t lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) len = 2;
        else if (c >= 0xe0 && c <= 0xef) {
            len = 3;
            if (c == 0xe0) lo = 0xa0;
            if (c == 0xed) hi = 0x9f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            len = 4;
            if (c == 0xf0) lo = 0x90;
            if (c == 0xf4) hi = 0x8f;
        } else
            return false;
        if (i + len > n) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (int k = 2; k < len; ++k)
            if (s[i + k] < 0x80 || s[i + k] > 0xbf) return false;
        i += len;
    }
    return true;
}

// (low, high) of a UTF-8 continuation range as the device's 3-bit class.
uint32_t range_class(uint8_t low, uint8_t high) {
    if (low == 0xa0) return 1;
    if (high == 0x9f) return 2;
    if (low == 0x90) return 3;
    if (high == 0x8f) return 4;
    return 0;
}

uint64_t entry_of(const Pos &p) {
    uint32_t cls = p.phase >= 3 ? range_class(p.low, p.high) : 0;
    return (uint64_t)p.node | ((uint64_t)p.phase << 17) | ((uint64_t)cls << 20) |
           ((uint64_t)p.used << 32);
}

constexpr size_t kMembersMax = size_t(1) << 24;      // flattened Split members
constexpr uint64_t kFrontierBudget = 512ull << 20;   // bytes of block-walk scratch

}  // namespace

// ------------------------------------------------------------------ compile
// constraint.rs:63-113: literals become Byte chains built back to front,
// sequences compile right to left, choices become a Split over the
// alternatives' entries; depth, node and literal-byte bounds as there.
Constraint::Constraint(std::shared_ptr<Vocab> v, const char *json, size_t len)
    : vocab(std::move(v)) {
    if (!json) bad("invalid output grammar: null");
    if (!valid_utf8((const uint8_t *)json, len)) bad("invalid output grammar: not UTF-8");
    Json j{json, json + len};
    Gram g = j.grammar();
    j.ws();
    if (j.p != j.end) j.err("trailing characters");

    nodes.clear();
    nodes.push_back(GNode{});  // End
    size_t bytes = 0;
    struct C {
        std::vector<GNode> &nodes;
        size_t &bytes;
        uint32_t run(const Gram &g, uint32_t next, int depth) {
            if (depth > 24 || nodes.size() > 100000 || bytes > 262144)
                bad("output grammar exceeds its bounds");
            switch (g.kind) {
            case 0: {
                bytes += g.value.size();
                if (bytes > 262144) bad("output grammar literals exceed their bound");
                uint32_t at = next;
                for (size_t i = g.value.size(); i-- > 0;) {
                    GNode n;
                    n.kind = G_BYTE;
                    n.byte = (uint8_t)g.value[i];
                    n.next = at;
                    nodes.push_back(n);
                    at = (uint32_t)nodes.size() - 1;
                }
                return at;
            }
            case 1: {
                if (g.max_bytes < 1 || g.max_bytes > 4096) bad("JSON string bound must be 1..4096");
                GNode n;
                n.kind = G_STRING;
                n.max = (uint32_t)g.max_bytes;
                n.next = next;
                nodes.push_back(n);
                return (uint32_t)nodes.size() - 1;
            }
            case 2: {
                uint32_t at = next;
                for (size_t i = g.kids.size(); i-- > 0;) at = run(g.kids[i], at, depth + 1);
                return at;
            }
            default: {
                if (g.kids.empty() || g.kids.size() > 64)
                    bad("grammar choice must have 1..64 alternatives");
                GNode n;
                n.kind = G_SPLIT;
                for (const Gram &k : g.kids) n.alts.push_back(run(k, next, depth + 1));
                nodes.push_back(std::move(n));
                return (uint32_t)nodes.size() - 1;
            }
            }
        }
    } c{nodes, bytes};
    uint32_t start = c.run(g, 0, 0);
    if (nodes.size() > 100000) bad("compiled output grammar exceeds its state bound");
    for (const GNode &n : nodes) n_strings += n.kind == G_STRING;
    active = close({Pos::at(start)});
}

// constraint.rs:158-169: expand Splits, then sort and deduplicate.
std::vector<Pos> Constraint::close(std::vector<Pos> ps) const {
    std::vector<Pos> out;
    while (!ps.empty()) {
        Pos p = ps.back();
        ps.pop_back();
        const GNode &n = nodes[p.node];
        if (n.kind == G_SPLIT) {
            for (uint32_t id : n.alts) ps.push_back(Pos::at(id));
        } else {
            out.push_back(p);
        }
    }
    std::sort(out.begin(), out.end());
    out.erase(std::unique(out.begin(), out.end()), out.end());
    return out;
}

// One position on one byte (constraint.rs:172-245), before closing: at
// most one successor. JSON string phases: 0 before the opening quote, 1
// content, 2 after a backslash, 3..5 expecting 1..3 UTF-8 continuation
// bytes in [low, high]; `used` counts encoded content bytes.
bool Constraint::step1(const Pos &p, uint8_t byte, Pos &out) const {
    const GNode &n = nodes[p.node];
    if (n.kind == G_BYTE) {
        if (n.byte != byte) return false;
        out = Pos::at(n.next);
        return true;
    }
    if (n.kind != G_STRING) return false;
    Pos q = p;
    if (p.phase == 0) {
        if (byte != '"') return false;
        q.phase = 1;
        out = q;
        return true;
    }
    if (p.phase == 1 && byte == '"') {
        if (p.used == 0) return false;
        out = Pos::at(n.next);
        return true;
    }
    if (p.used >= n.max) return false;
    q.used += 1;
    switch (p.phase) {
    case 1:
        if (byte == '\\' && p.used + 2 <= n.max) {
            q.phase = 2;
        } else if (byte >= 0x20 && byte <= 0x7f && byte != '"' && byte != '\\') {
        } else if (byte >= 0xc2 && byte <= 0xdf && p.used + 2 <= n.max) {
            q.phase = 3;
            q.low = 0x80;
            q.high = 0xbf;
        } else if (byte >= 0xe0 && byte <= 0xef && p.used + 3 <= n.max) {
            q.phase = 4;
            q.low = byte == 0xe0 ? 0xa0 : 0x80;
            q.high = byte == 0xed ? 0x9f : 0xbf;
        } else if (byte >= 0xf0 && byte <= 0xf4 && p.used + 4 <= n.max) {
            q.phase = 5;
            q.low = byte == 0xf0 ? 0x90 : 0x80;
            q.high = byte == 0xf4 ? 0x8f : 0xbf;
        } else {
            return false;
        }
        break;
    case 2:
        if (!memchr("\"\\/bfnrt", byte, 8)) return false;
        q.phase = 1;
        break;
    case 3:
    case 4:
    case 5:
        if (byte < p.low || byte > p.high) return false;
        q.phase = p.phase == 3 ? 1 : p.phase - 1;
        q.low = 0x80;
        q.high = 0xbf;
        break;
    default:
        return false;
    }
    out = q;
    return true;
}

std::vector<Pos> Constraint::step(const std::vector<Pos> &set, uint8_t byte) const {
    std::vector<Pos> out;
    Pos q;
    for (const Pos &p : set)
        if (step1(p, byte, q)) out.push_back(q);
    return close(std::move(out));
}

// constraint.rs:246-255
std::vector<Pos> Constraint::after(const uint8_t *bytes, size_t n) const {
    std::vector<Pos> state = active;
    for (size_t i = 0; i < n; ++i) {
        state = step(state, bytes[i]);
        if (state.empty()) break;
    }
    return state;
}

// constraint.rs:256-260
bool Constraint::complete() const {
    for (const Pos &p : active)
        if (nodes[p.node].kind == G_END) return true;
    return false;
}

// constraint.rs:261-273
void Constraint::accept(uint32_t id) {
    const Vocab &v = *vocab;
    if (id >= v.n || v.off[id + 1] == v.off[id]) bad("constraint encountered an unsupported token");
    std::vector<Pos> state = after(v.bytes.data() + v.off[id], v.off[id + 1] - v.off[id]);
    if (state.empty()) bad("token violates output grammar");
    active = std::move(state);
}

// constraint.rs:296-318: the unique-byte continuation (at most 4096 bytes,
// stopping at End or at the first byte choice), cut back to valid UTF-8.
std::vector<uint8_t> Constraint::forced_bytes() const {
    std::vector<Pos> state = active;
    std::vector<uint8_t> bytes;
    for (int it = 0; it < 4096; ++it) {
        bool end = false;
        for (const Pos &p : state) end |= nodes[p.node].kind == G_END;
        if (end) break;
        // The live bytes are those some position steps on (a closed set's
        // successors always close to a non-empty set); stop at the second.
        int found = -1;
        bool many = false;
        Pos q;
        for (size_t i = 0; i < state.size() && !many; ++i) {
            const Pos &p = state[i];
            const GNode &n = nodes[p.node];
            auto live = [&](int b) {
                if (found >= 0 && found != b) many = true;
                found = b;
            };
            if (n.kind == G_BYTE) live(n.byte);
            else if (n.kind == G_STRING && p.phase == 0) live('"');
            else if (n.kind == G_STRING)
                for (int b = 0; b < 256 && !many; ++b)
                    if (step1(p, (uint8_t)b, q)) live(b);
        }
        if (found < 0 || many) break;
        bytes.push_back((uint8_t)found);
        state = step(state, (uint8_t)found);
    }
    while (!valid_utf8(bytes.data(), bytes.size())) bytes.pop_back();
    return bytes;
}

void Constraint::first_table(std::vector<uint32_t> &off, std::vector<uint64_t> &ent) const {
    std::vector<uint64_t> pairs;  // byte << 56 | entry (entries fit 45 bits)
    Pos q;
    for (const Pos &p : active) {
        const GNode &n = nodes[p.node];
        if (n.kind == G_BYTE) {
            if (step1(p, n.byte, q)) pairs.push_back((uint64_t)n.byte << 56 | entry_of(q));
        } else if (n.kind == G_STRING && p.phase == 0) {
            if (step1(p, '"', q)) pairs.push_back((uint64_t)'"' << 56 | entry_of(q));
        } else if (n.kind == G_STRING) {
            for (int b = 0; b < 256; ++b)
                if (step1(p, (uint8_t)b, q)) pairs.push_back((uint64_t)b << 56 | entry_of(q));
        }
    }
    std::sort(pairs.begin(), pairs.end());
    pairs.erase(std::unique(pairs.begin(), pairs.end()), pairs.end());
    off.assign(257, 0);
    ent.resize(pairs.size());
    for (size_t i = 0; i < pairs.size(); ++i) {
        off[(pairs[i] >> 56) + 1]++;
        ent[i] = pairs[i] & ((1ull << 56) - 1);
    }
    for (int b = 0; b < 256; ++b) off[b + 1] += off[b];
}

uint64_t Constraint::frontier_cap() const {
    // At most one unclosed at-node entry per node, one freshly opened
    // string per String node, and one content position per (String node,
    // used) pair, where `used` spans the bound or the longest token plus
    // the positions already active in that string.
    std::vector<uint32_t> act(nodes.size(), 0);
    for (const Pos &p : active)
        if (p.phase > 0) act[p.node]++;
    uint64_t cap = nodes.size();
    for (size_t i = 0; i < nodes.size(); ++i)
        if (nodes[i].kind == G_STRING)
            cap += 1 + std::min<uint64_t>(nodes[i].max, (uint64_t)vocab->max_len + act[i]);
    return cap;
}

void Vocab::to_device() {
    std::lock_guard<std::mutex> lock(mu);
    int dev = 0;
    ESP_HIP(hipGetDevice(&dev));
    if (device == dev) return;
    if (device >= 0) fail(ESP_INVALID_REQUEST, "vocabulary already resides on another device");
    d_bytes.alloc(std::max<size_t>(bytes.size(), 4));
    d_off.alloc(off.size() * 4);
    if (!bytes.empty())
        ESP_HIP(hipMemcpy(d_bytes.p, bytes.data(), bytes.size(), hipMemcpyHostToDevice));
    ESP_HIP(hipMemcpy(d_off.p, off.data(), off.size() * 4, hipMemcpyHostToDevice));
    if (max_len <= CSTR_MAX_LEN) {
        d_scls.alloc((size_t)CSTR_STATES * n * 4);
        launch_str_class(d_bytes.as<uint8_t>(), d_off.as<uint32_t>(), (int)n,
                         d_scls.as<uint32_t>(), nullptr);
        ESP_HIP(hipGetLastError());
        ESP_HIP(hipStreamSynchronize(nullptr));
    }
    device = dev;
}

void Constraint::to_device() {
    vocab->to_device();
    int dev = 0;
    ESP_HIP(hipGetDevice(&dev));
    if (device == dev) return;
    if (device >= 0) fail(ESP_INVALID_REQUEST, "constraint already resides on another device");
    std::vector<uint32_t> words(nodes.size()), split_off(1, 0), members;
    // Split closures in id order: alternatives always have smaller ids.
    std::vector<int> split_of(nodes.size(), -1);
    std::vector<std::vector<uint32_t>> closure;
    for (size_t i = 0; i < nodes.size(); ++i) {
        const GNode &n = nodes[i];
        switch (n.kind) {
        case G_END: words[i] = 0; break;
        case G_BYTE: words[i] = 1u << 30 | (uint32_t)n.byte << 22 | n.next; break;
        case G_STRING: words[i] = 2u << 30 | n.max << 17 | n.next; break;
        case G_SPLIT: {
            std::vector<uint32_t> cl;
            for (uint32_t a : n.alts) {
                if (nodes[a].kind == G_SPLIT) {
                    const auto &sub = closure[split_of[a]];
                    cl.insert(cl.end(), sub.begin(), sub.end());
                } else {
                    cl.push_back(a);
                }
            }
            std::sort(cl.begin(), cl.end());
            cl.erase(std::unique(cl.begin(), cl.end()), cl.end());
            split_of[i] = (int)closure.size();
            words[i] = 3u << 30 | (uint32_t)closure.size();
            std::vector<uint32_t> packed;
            for (uint32_t m : cl) {
                if (nodes[m].kind == G_BYTE) packed.push_back((uint32_t)nodes[m].byte << 17 | m);
                else if (nodes[m].kind == G_STRING) packed.push_back((uint32_t)'"' << 17 | m);
            }
            std::sort(packed.begin(), packed.end());
            members.insert(members.end(), packed.begin(), packed.end());
            split_off.push_back((uint32_t)members.size());
            if (members.size() > kMembersMax)
                fail(ESP_UNSUPPORTED,
                     "constrained decoding: grammar choice closures exceed the device table bound");
            closure.push_back(std::move(cl));
            break;
        }
        }
    }
    d_nodes.alloc(words.size() * 4);
    d_split_off.alloc(split_off.size() * 4);
    d_members.alloc(std::max<size_t>(members.size(), 1) * 4);
    ESP_HIP(hipMemcpy(d_nodes.p, words.data(), words.size() * 4, hipMemcpyHostToDevice));
    ESP_HIP(hipMemcpy(d_split_off.p, split_off.data(), split_off.size() * 4,
                      hipMemcpyHostToDevice));
    if (!members.empty())
        ESP_HIP(hipMemcpy(d_members.p, members.data(), members.size() * 4, hipMemcpyHostToDevice));
    device = dev;
}

// ---------------------------------------------------------------- batched mask

void run_cmask(MaskCtx &ctx, Constraint *const *cs, uint32_t *const *masks, int n,
               hipStream_t s) {
    if (n <= 0) return;
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    std::vector<std::vector<uint32_t>> offs(n);
    std::vector<std::vector<uint64_t>> ents(n);
    size_t bytes = al(sizeof(CRow) * n);
    std::vector<size_t> at(n);
    int v_max = 0, nodes_max = 1;
    uint64_t cap_max = 1, v_sum = 0;
    std::vector<uint64_t> caps(n);
    for (int i = 0; i < n; ++i) {
        Constraint &c = *cs[i];
        c.to_device();
        c.first_table(offs[i], ents[i]);
        at[i] = bytes;
        bytes += al(257 * 4 + 4) + al(ents[i].size() * 8);
        caps[i] = c.frontier_cap();
        cap_max = std::max(cap_max, caps[i]);
        v_max = std::max<int>(v_max, (int)c.vocab->n);
        v_sum += c.vocab->n;
        nodes_max = std::max<int>(nodes_max, (int)c.nodes.size());
    }
    if (cap_max * 16 > kFrontierBudget)
        fail(ESP_UNSUPPORTED, "constrained decoding: grammar frontier exceeds the device bound");
    // ESP_CMASK_STRCLASS=0 walks string states byte by byte (tests compare both).
    const char *sc = getenv("ESP_CMASK_STRCLASS");
    const bool strclass = !(sc && sc[0] == '0');
    ctx.stage.assign(bytes, 0);
    ctx.io.ensure(bytes);
    char *dev = (char *)ctx.io.p;
    CRow *rows = (CRow *)ctx.stage.data();
    for (int i = 0; i < n; ++i) {
        Constraint &c = *cs[i];
        char *h = (char *)ctx.stage.data() + at[i];
        memcpy(h, offs[i].data(), 257 * 4);
        size_t eo = al(257 * 4 + 4);
        if (!ents[i].empty()) memcpy(h + eo, ents[i].data(), ents[i].size() * 8);
        CRow r{};
        r.nodes = c.d_nodes.as<uint32_t>();
        r.split_off = c.d_split_off.as<uint32_t>();
        r.members = c.d_members.as<uint32_t>();
        r.first_off = (const uint32_t *)(dev + at[i]);
        r.first = (const uint64_t *)(dev + at[i] + eo);
        r.tok = c.vocab->d_bytes.as<uint8_t>();
        r.tok_off = c.vocab->d_off.as<uint32_t>();
        r.mask = masks[i];
        r.V = (int)c.vocab->n;
        r.row = i;
        r.cap = caps[i];
        if (strclass && c.active.size() == 1 && c.nodes[c.active[0].node].kind == G_STRING &&
            c.vocab->d_scls.p) {
            const Pos &p = c.active[0];
            const GNode &g = c.nodes[p.node];
            static const uint8_t st4[3] = {3, 4, 5}, st5[5] = {6, 0, 0, 7, 8};
            uint32_t cls = range_class(p.low, p.high);
            r.mode = 1;
            r.s_used = p.used;
            r.s_max = g.max;
            r.s_next = g.next;
            r.s_state = p.phase == 0 ? 9 : p.phase == 1 ? 0 : p.phase == 2 ? 1 : p.phase == 3 ? 2
                      : p.phase == 4 ? st4[cls] : st5[cls];
            r.scls = c.vocab->d_scls.as<uint32_t>() + (size_t)r.s_state * c.vocab->n;
        }
        rows[i] = r;
    }
    int blocks = (int)std::min<uint64_t>(256, kFrontierBudget / (cap_max * 16));
    ctx.status.ensure(64);
    ctx.ovf.ensure(std::max<uint64_t>(v_sum, 1) * 8);
    ctx.frontier.ensure((size_t)blocks * 2 * cap_max * 8);
    ESP_HIP(hipMemcpyAsync(ctx.io.p, ctx.stage.data(), bytes, hipMemcpyHostToDevice, s));
    ESP_HIP(hipMemsetAsync(ctx.status.p, 0, 8, s));
    CMaskLaunch a{};
    a.rows = (const CRow *)ctx.io.p;
    a.n_rows = n;
    a.v_max = v_max;
    a.n_nodes_max = nodes_max;
    a.status = ctx.status.as<uint32_t>();
    a.ovf = ctx.ovf.as<uint64_t>();
    a.frontier = ctx.frontier.as<uint64_t>();
    a.cap_max = cap_max;
    a.blocks = blocks;
    // ESP_CMASK_LANE_CAP (0..8, default 8) and ESP_CMASK_WAVE_CAP (0..64,
    // default 64) lower the lane and wave frontiers so that tests can drive
    // tokens through the wave and block walks.
    const char *lc = getenv("ESP_CMASK_LANE_CAP");
    const char *wc = getenv("ESP_CMASK_WAVE_CAP");
    a.lane_cap = lc ? std::max(0, std::min(8, atoi(lc))) : 8;
    a.wave_cap = wc ? std::max(0, std::min(64, atoi(wc))) : 64;
    launch_cmask(a, s);
}

void check_cmask(MaskCtx &ctx, hipStream_t s) {
    uint32_t st[2] = {0, 0};
    ESP_HIP(hipMemcpyAsync(st, ctx.status.p, 8, hipMemcpyDeviceToHost, s));
    ESP_HIP(hipStreamSynchronize(s));
    if (st[1]) fail(ESP_BACKEND, "constraint mask frontier exceeded its bound");
}

}  // namespace esp
