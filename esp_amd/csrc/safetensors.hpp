// Minimal safetensors header reader (host). The format is an 8-byte
// little-endian header length, a JSON object mapping tensor names to
// {dtype, shape, data_offsets}, then the raw little-endian buffer.
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace esp {

struct StTensor {
    std::string dtype;  // "F32", "BF16", "F16", ...
    std::vector<uint64_t> shape;
    const uint8_t *data = nullptr;
    size_t bytes = 0;
};

// Parses `buf`; throws esp::Error{ESP_INVALID_WEIGHTS} on malformed input.
std::map<std::string, StTensor> parse_safetensors(const uint8_t *buf, size_t len);

}  // namespace esp
