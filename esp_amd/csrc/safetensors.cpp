#include "safetensors.hpp"

#include <string.h>

#include "common.hpp"

namespace esp {

namespace {

// A small JSON reader covering what a safetensors header contains.
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    uint64_t u = 0;
    bool is_uint = false;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
};

struct Parser {
    const char *p, *end;
    [[noreturn]] void bad(const char *why) {
        fail(ESP_INVALID_WEIGHTS, std::string("safetensors parse: ") + why);
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    std::string str() {
        if (p >= end || *p != '"') bad("expected string");
        ++p;
        std::string out;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) bad("bad escape");
                char c = *p++;
                switch (c) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (end - p < 4) bad("bad unicode escape");
                        unsigned cp = 0;
                        for (int i = 0; i < 4; ++i) {
                            char h = *p++;
                            cp <<= 4;
                            if (h >= '0' && h <= '9') cp |= h - '0';
                            else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                            else bad("bad unicode escape");
                        }
                        if (cp < 0x80) out += (char)cp;
                        else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: bad("bad escape");
                }
            } else {
                out += *p++;
            }
        }
        if (p >= end) bad("unterminated string");
        ++p;
        return out;
    }
    Json value(int depth) {
        if (depth > 16) bad("nesting too deep");
        ws();
        if (p >= end) bad("unexpected end");
        Json j;
        char c = *p;
        if (c == '{') {
            j.kind = Json::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return j;
            }
            while (true) {
                ws();
                std::string k = str();
                ws();
                if (p >= end || *p != ':') bad("expected ':'");
                ++p;
                j.obj.emplace_back(k, value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return j;
                }
                bad("expected ',' or '}'");
            }
        }
        if (c == '[') {
            j.kind = Json::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return j;
            }
            while (true) {
                j.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return j;
                }
                bad("expected ',' or ']'");
            }
        }
        if (c == '"') {
            j.kind = Json::STR;
            j.s = str();
            return j;
        }
        if (end - p >= 4 && !strncmp(p, "true", 4)) {
            p += 4;
            j.kind = Json::BOOL;
            j.b = true;
            return j;
        }
        if (end - p >= 5 && !strncmp(p, "false", 5)) {
            p += 5;
            j.kind = Json::BOOL;
            return j;
        }
        if (end - p >= 4 && !strncmp(p, "null", 4)) {
            p += 4;
            return j;
        }
        if (c == '-' || (c >= '0' && c <= '9')) {
            const char *s = p;
            bool integral = true;
            if (*p == '-') {
                integral = false;
                ++p;
            }
            while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                               *p == '+' || *p == '-')) {
                if (!(*p >= '0' && *p <= '9')) integral = false;
                ++p;
            }
            j.kind = Json::NUM;
            std::string t(s, p);
            j.num = strtod(t.c_str(), nullptr);
            if (integral && t.size() <= 19) {
                j.is_uint = true;
                j.u = strtoull(t.c_str(), nullptr, 10);
            }
            return j;
        }
        bad("unexpected character");
    }
};

}  // namespace

std::map<std::string, StTensor> parse_safetensors(const uint8_t *buf, size_t len) {
    if (!buf || len < 8) fail(ESP_INVALID_WEIGHTS, "safetensors parse: buffer too small");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | buf[i];
    if (n > len - 8 || n > (100u << 20))
        fail(ESP_INVALID_WEIGHTS, "safetensors parse: header length out of range");
    Parser ps{(const char *)buf + 8, (const char *)buf + 8 + n};
    Json root = ps.value(0);
    if (root.kind != Json::OBJ) fail(ESP_INVALID_WEIGHTS, "safetensors parse: header not an object");
    const uint8_t *data = buf + 8 + n;
    const size_t data_len = len - 8 - n;
    std::map<std::string, StTensor> out;
    for (auto &kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json &t = kv.second;
        if (t.kind != Json::OBJ) fail(ESP_INVALID_WEIGHTS, "safetensors parse: bad entry " + kv.first);
        StTensor st;
        const Json *offs = nullptr;
        for (auto &f : t.obj) {
            if (f.first == "dtype" && f.second.kind == Json::STR) st.dtype = f.second.s;
            else if (f.first == "shape" && f.second.kind == Json::ARR) {
                for (auto &d : f.second.arr) {
                    if (d.kind != Json::NUM || !d.is_uint)
                        fail(ESP_INVALID_WEIGHTS, "safetensors parse: bad shape for " + kv.first);
                    st.shape.push_back(d.u);
                }
            } else if (f.first == "data_offsets" && f.second.kind == Json::ARR) {
                offs = &f.second;
            }
        }
        if (st.dtype.empty() || !offs || offs->arr.size() != 2 || !offs->arr[0].is_uint ||
            !offs->arr[1].is_uint)
            fail(ESP_INVALID_WEIGHTS, "safetensors parse: incomplete entry " + kv.first);
        uint64_t a = offs->arr[0].u, b = offs->arr[1].u;
        if (a > b || b > data_len)
            fail(ESP_INVALID_WEIGHTS, "safetensors parse: offsets out of range for " + kv.first);
        size_t esz = st.dtype == "F32" || st.dtype == "I32" || st.dtype == "U32" ? 4
                     : st.dtype == "BF16" || st.dtype == "F16" || st.dtype == "I16" ? 2
                     : st.dtype == "F64" || st.dtype == "I64" || st.dtype == "U64" ? 8
                     : 1;
        uint64_t count = 1;
        for (auto d : st.shape) count *= d;
        if (count * esz != b - a)
            fail(ESP_INVALID_WEIGHTS, "safetensors parse: byte count disagrees with shape for " + kv.first);
        st.data = data + a;
        st.bytes = b - a;
        out[kv.first] = st;
    }
    return out;
}

}  // namespace esp
