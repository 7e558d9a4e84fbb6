// SPDX-License-Identifier: MIT
// SHA-256 (FIPS 180-4), used to check graph-topology contracts and weight files
// (the reference hashes both: tools/build_dit_weights.py:18,34-50,
// src/shape_graph.cpp:12-21).
#pragma once
#include <array>
#include <cstddef>
#include <cstdint>
#include <string>

namespace ernie {

class Sha256 {
public:
    Sha256();
    void update(const void* data, size_t size);
    std::array<unsigned char, 32> finish();
    std::string finish_hex();

private:
    void block(const unsigned char* p);
    uint32_t h_[8];
    unsigned char buf_[64];
    size_t used_ = 0;
    uint64_t total_ = 0;
};

std::string sha256_hex(const void* data, size_t size);

}  // namespace ernie
