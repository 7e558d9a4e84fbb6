// SPDX-License-Identifier: MIT
#include "ernie/text_encoder.h"

#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <stdexcept>

namespace ernie {
namespace {

void bucket_check(int bucket)
{
    if (bucket < 1 || bucket > kTextMaxBucket) throw std::invalid_argument("Text bucket must be in [1,2048]");
}

float bf16_to_float(std::uint16_t bits)
{
    const std::uint32_t word = std::uint32_t(bits) << 16;
    float f;
    std::memcpy(&f, &word, 4);
    return f;
}

}  // namespace

std::vector<float> text_embeddings(const std::uint16_t* table, std::size_t vocabulary, int width,
                                   const std::vector<std::uint32_t>& ids, int bucket)
{
    bucket_check(bucket);
    if (!table || width < 1 || ids.empty() || ids.size() > std::size_t(bucket))
        throw std::invalid_argument("Invalid token IDs or embedding table");
    std::vector<float> out(std::size_t(bucket) * width, 0.f);
    for (std::size_t i = 0; i < ids.size(); ++i) {
        if (ids[i] >= vocabulary) throw std::invalid_argument("Token ID outside vocabulary");
        const std::uint16_t* row = table + std::size_t(ids[i]) * width;
        for (int j = 0; j < width; ++j) out[i * width + j] = bf16_to_float(row[j]);
    }
    return out;
}

std::vector<float> text_embeddings(const std::string& path, const std::vector<std::uint32_t>& ids, int bucket)
{
    bucket_check(bucket);
    const auto file_path = std::filesystem::u8path(path);
    if (ids.empty() || ids.size() > std::size_t(bucket) ||
        std::filesystem::file_size(file_path) != std::uintmax_t(kTextVocabulary) * kTextWidth * 2)
        throw std::invalid_argument("Invalid token IDs or BF16 embedding table size");
    std::ifstream file(file_path, std::ios::binary);
    std::vector<std::uint16_t> row(kTextWidth);
    std::vector<float> out(std::size_t(bucket) * kTextWidth, 0.f);
    for (std::size_t i = 0; i < ids.size(); ++i) {
        if (ids[i] >= std::uint32_t(kTextVocabulary)) throw std::invalid_argument("Token ID outside vocabulary");
        file.seekg(std::streamoff(ids[i]) * kTextWidth * 2);
        if (!file.read(reinterpret_cast<char*>(row.data()), kTextWidth * 2))
            throw std::runtime_error("Embedding row read failed");
        for (int j = 0; j < kTextWidth; ++j) out[i * kTextWidth + j] = bf16_to_float(row[j]);
    }
    return out;
}

TextConstantsHost text_constants(const std::vector<float>& f, int bucket)
{
    bucket_check(bucket);
    if (f.size() != 64) throw std::invalid_argument("Invalid YaRN frequency table size");
    for (float v : f)
        if (!std::isfinite(v) || v <= 0.f) throw std::runtime_error("Invalid YaRN frequency");
    TextConstantsHost k;
    k.bucket = bucket;
    k.cos.resize(std::size_t(bucket) * 128);
    k.sin.resize(std::size_t(bucket) * 128);
    k.mask.resize(std::size_t(bucket) * bucket);
    for (int t = 0; t < bucket; ++t) {
        float* c = &k.cos[std::size_t(t) * 128];
        float* s = &k.sin[std::size_t(t) * 128];
        for (int j = 0; j < 64; ++j) {
            const float phase = float(t) * f[j];
            c[j] = c[j + 64] = std::cos(phase);
            s[j] = s[j + 64] = std::sin(phase);
        }
        float* m = &k.mask[std::size_t(t) * bucket];
        for (int key = 0; key < bucket; ++key) m[key] = key > t ? -std::numeric_limits<float>::max() : 0.f;
    }
    return k;
}

TextConstantsHost text_constants(const std::string& path, int bucket)
{
    bucket_check(bucket);
    const auto file_path = std::filesystem::u8path(path);
    if (std::filesystem::file_size(file_path) != 64 * 4) throw std::invalid_argument("Invalid YaRN frequency table size");
    std::vector<float> f(64);
    std::ifstream file(file_path, std::ios::binary);
    if (!file.read(reinterpret_cast<char*>(f.data()), 64 * 4)) throw std::runtime_error("Cannot read YaRN frequencies");
    return text_constants(f, bucket);
}

std::vector<DeviceMat> upload_text_constants(const Device& device, const TextConstantsHost& k)
{
    DeviceMat cos = DeviceMat::create(device, 128, k.bucket, 1, 2);
    DeviceMat sin = DeviceMat::create(device, 128, k.bucket, 1, 2);
    DeviceMat mask = DeviceMat::create(device, k.bucket, k.bucket, 1, 2);
    cos.upload(device, k.cos.data(), k.cos.size());
    sin.upload(device, k.sin.data(), k.sin.size());
    mask.upload(device, k.mask.data(), k.mask.size());
    mask.causal = true;
    return {cos, sin, mask};
}

DeviceMat run_text_blocks(const std::vector<BlockModel>& models, const DeviceMat& input,
                          const std::vector<DeviceMat>& constants, const Option& option, BlockSequenceStats& stats)
{
    // src/text_encoder.cpp:41-45.
    if (models.size() < 1 || models.size() > 25 || constants.size() != 3)
        throw std::invalid_argument("Text path requires 1..25 blocks and cos/sin/causal mask");
    if (!option.device) throw std::invalid_argument("Text path requires a device");
    option.dtype();
    const Device& device = *option.device;
    ernie_hip_ctx* ctx = device.ctx();
    if (input.empty() || input.dims > 2) throw std::invalid_argument("Text input must be a [tokens][width] FP32 tensor");
    const int S = input.h, width = input.w;
    if (S > kTextMaxBucket) throw std::invalid_argument("Text bucket must be in [1,2048]");
    const DeviceMat &cos = constants[0], &sin = constants[1], &mask = constants[2];
    if (cos.total() != std::size_t(S) * 128 || sin.total() != std::size_t(S) * 128)
        throw std::invalid_argument("Text RoPE tables must be [tokens][128]");
    if (!mask.empty() && mask.total() != std::size_t(S) * S)
        throw std::invalid_argument("Text attention mask must be [tokens][tokens]");
    const bool collect_details = stats.collect_details;
    stats = {};
    stats.collect_details = collect_details;
    stats.peak_loaded_nets = int(models.size());
    DeviceMat current = DeviceMat::create(device, width, S, 1, 2);
    const float* in = input.data;
    for (std::size_t i = 0; i < models.size(); ++i) {
        double seconds = 0;
        const int index = models[i].index;
        const float* m = mask.empty() || mask.causal ? nullptr : mask.data;
        check_status(ernie_hip_text_block_sequence(ctx, &index, 1, in, current.data, cos.data, sin.data, m,
                                                   mask.causal ? 1 : 0, S, &seconds),
                     ctx, "text block");
        in = current.data;
        stats.load_seconds.push_back(0.0);
        stats.compute_seconds.push_back(seconds);
        stats.compute_submissions += 1;
        if (stats.collect_details) stats.details.push_back({int(i), "text_block_compute", "complete", seconds});
    }
    return current;
}

}  // namespace ernie
