// SPDX-License-Identifier: MIT
// File I/O shared by the command-line runners: raw little-endian FP32 tensors, as the
// reference's probes read and write them (probes/block_runner.cpp:28-39,
// probes/denoise_runner.cpp:13-40), and the reduction of a dense [S][S] attention mask
// to the one-row form the device path takes.
#pragma once
#include <cstddef>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace ernie_runner {

namespace fs = std::filesystem;

// Exactly `count` FP32 values, or std::runtime_error (the probes' byte-count check).
inline std::vector<float> read_f32(const fs::path& path, size_t count)
{
    std::error_code ec;
    const auto size = fs::file_size(path, ec);
    if (ec || size != count * sizeof(float))
        throw std::runtime_error("Tensor byte count mismatch: " + path.string());
    std::vector<float> v(count);
    std::ifstream file(path, std::ios::binary);
    if (!file.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(count * sizeof(float))))
        throw std::runtime_error("Cannot read " + path.string());
    return v;
}

// Writes a new file; an existing one is never overwritten.
inline void write_f32(const fs::path& path, const float* data, size_t count)
{
    if (fs::exists(path)) throw std::runtime_error("Refusing to overwrite " + path.string());
    if (path.has_parent_path()) fs::create_directories(path.parent_path());
    std::ofstream file(path, std::ios::binary);
    file.write(reinterpret_cast<const char*>(data), (std::streamsize)(count * sizeof(float)));
    if (!file) throw std::runtime_error("Cannot write " + path.string());
}

// The block graph's attention mask in9 is the one-row mask of src/conditioning.cpp:41-42
// broadcast over the queries (src/ernie_attention.cpp:201-219 expands it so). The device
// path takes that row: `valid_keys` > 0 when it is canonical (zeros, then -1e30 or lower
// from valid_keys on), else the row itself as an additive mask. A mask whose rows differ
// is refused.
struct MaskRow {
    std::vector<float> row;
    int valid_keys = 0;
};

inline MaskRow mask_row(const std::vector<float>& dense, int tokens)
{
    const size_t n = (size_t)tokens;
    if (dense.size() != n * n) throw std::runtime_error("Mask must be [tokens][tokens]");
    for (size_t r = 1; r < n; ++r)
        if (std::memcmp(dense.data() + r * n, dense.data(), n * sizeof(float)) != 0)
            throw std::runtime_error("The block path takes one mask row for every query; mask row " +
                                     std::to_string(r) + " differs from row 0");
    MaskRow m;
    m.row.assign(dense.begin(), dense.begin() + (long)n);
    size_t prefix = 0;
    while (prefix < n && m.row[prefix] == 0.f) ++prefix;
    bool canonical = prefix > 0;
    for (size_t k = prefix; k < n && canonical; ++k) canonical = m.row[k] <= -1e30f;
    if (canonical) m.valid_keys = (int)prefix;
    return m;
}

inline int parse_int(const std::string& flag, const std::string& value)
{
    size_t used = 0;
    int v = 0;
    try {
        v = std::stoi(value, &used);
    } catch (const std::exception&) {
        used = 0;
    }
    if (used != value.size() || value.empty()) throw std::invalid_argument("Invalid integer for " + flag);
    return v;
}

}  // namespace ernie_runner
