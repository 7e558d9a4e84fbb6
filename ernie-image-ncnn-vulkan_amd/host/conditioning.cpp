// SPDX-License-Identifier: MIT
// Compiled with -ffp-contract=off: each product and sum rounds separately.
#include "ernie/conditioning.h"

#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <stdexcept>

namespace ernie {

std::vector<float> rope_frequencies()
{
    std::vector<float> table;
    table.reserve(64);
    for (int dim : {32, 48, 48})
        for (int e = 0; e < dim; e += 2) table.push_back(1.f / std::pow(256.f, float(e) / float(dim)));
    return table;
}

DitConstantsHost dit_constants(const std::vector<float>& frequencies, int w, int h, int valid, int text,
                               int token_limit)
{
    if (w < 1 || w > 256 || h < 1 || h > 256 || valid < 1 || text < valid || text > 2048 ||
        w * h + text > token_limit || frequencies.size() != 64)
        throw std::invalid_argument("Invalid DiT position dimensions or frequency file");
    for (float f : frequencies)
        if (!std::isfinite(f) || f <= 0.f) throw std::runtime_error("Invalid DiT frequency");
    const int image = w * h, length = image + text;
    DitConstantsHost out;
    out.length = length;
    out.valid_keys = image + valid;
    out.cos.resize(size_t(length) * 128);
    out.sin.resize(size_t(length) * 128);
    out.mask.resize(length);
    for (int i = 0; i < length; ++i) {
        // Image token i: (valid, row, column); text token j: (j, 0, 0).
        const int positions[3] = {i < image ? valid : i - image, i < image ? i / w : 0, i < image ? i % w : 0};
        float* c = out.cos.data() + size_t(i) * 128;
        float* s = out.sin.data() + size_t(i) * 128;
        for (int j = 0; j < 64; ++j) {
            const int axis = j < 16 ? 0 : (j < 40 ? 1 : 2);
            const float phase = float(positions[axis]) * frequencies[j];
            // ERNIE's full-width angles: both columns of a pair carry angle j.
            c[2 * j] = c[2 * j + 1] = std::cos(phase);
            s[2 * j] = s[2 * j + 1] = std::sin(phase);
        }
    }
    for (int k = 0; k < length; ++k) out.mask[k] = k >= image + valid ? -1e30f : 0.f;
    return out;
}

DitConstantsHost dit_constants(const std::string& frequency_path, int w, int h, int valid, int text)
{
    constexpr int kPathTokenLimit = 6144;  // src/conditioning.cpp:46-49
    std::error_code ec;
    const auto bytes = std::filesystem::file_size(std::filesystem::u8path(frequency_path), ec);
    if (w < 1 || w > 256 || h < 1 || h > 256 || valid < 1 || text < valid || text > 2048 ||
        w * h + text > kPathTokenLimit || ec || bytes != 64 * sizeof(float))
        throw std::invalid_argument("Invalid DiT position dimensions or frequency file");
    std::vector<float> frequencies(64);
    std::ifstream file(std::filesystem::u8path(frequency_path), std::ios::binary);
    if (!file.read(reinterpret_cast<char*>(frequencies.data()), 64 * sizeof(float)))
        throw std::runtime_error("Cannot read DiT frequencies");
    return dit_constants(frequencies, w, h, valid, text, kPathTokenLimit);
}

std::vector<DeviceMat> upload_constants(const Device& device, const DitConstantsHost& k)
{
    DeviceMat cos = DeviceMat::create(device, 128, k.length);
    DeviceMat sin = DeviceMat::create(device, 128, k.length);
    DeviceMat mask = DeviceMat::create(device, k.length, 1, 1, 1);
    cos.upload(device, k.cos.data(), k.cos.size());
    sin.upload(device, k.sin.data(), k.sin.size());
    mask.upload(device, k.mask.data(), k.mask.size());
    mask.valid_prefix = k.valid_keys;
    return {cos, sin, mask};
}

std::vector<float> pad_text(const std::vector<float>& embeddings, int tokens, int bucket)
{
    if (tokens < 1 || tokens > bucket || bucket > 2048 || embeddings.size() != size_t(tokens) * 3072)
        throw std::invalid_argument("Invalid text embeddings or padding bucket");
    std::vector<float> out(size_t(bucket) * 3072, 0.f);
    std::memcpy(out.data(), embeddings.data(), embeddings.size() * sizeof(float));
    return out;
}

}  // namespace ernie
