// SPDX-License-Identifier: MIT
// Mistral text path (src/text_encoder.h:1-33): embedding rows, the RoPE / causal
// mask constants and the text block sequence, with the reference's argument
// order, counts and exceptions. Blocks are resident text block slots of the
// device context.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ernie/block_sequence.h"
#include "ernie/runtime.h"

namespace ernie {

constexpr int kTextVocabulary = 131072, kTextWidth = 3072, kTextMaxBucket = 2048;

// src/text_encoder.cpp:68-90: rows of a raw BF16 [vocabulary][width] table for
// `ids`, widened to FP32, into [bucket][width]; rows past ids stay zero. Throws
// std::invalid_argument for an empty or oversized id list, an id outside the
// vocabulary or a bucket outside [1,2048].
std::vector<float> text_embeddings(const std::uint16_t* table, std::size_t vocabulary, int width,
                                   const std::vector<std::uint32_t>& ids, int bucket);
// The file form: the table is the reference's converted embedding file
// (131072 x 3072 BF16); only the requested rows are read.
std::vector<float> text_embeddings(const std::string& path, const std::vector<std::uint32_t>& ids, int bucket);

struct TextConstantsHost {
    int bucket = 0;
    std::vector<float> cos, sin, mask;  // [bucket][128], [bucket][128], [bucket][bucket]
};
// src/text_encoder.cpp:92-118: cos/sin with c[j] = c[j+64] = cos(t f_j) from the 64
// YaRN inverse frequencies, and the causal mask (-FLT_MAX above the diagonal).
TextConstantsHost text_constants(const std::vector<float>& inverse_frequencies, int bucket);
// The file form: 64 FP32 values (256 bytes).
TextConstantsHost text_constants(const std::string& inverse_frequency_path, int bucket);
// Uploads: cosine, sine, causal mask (marked causal: the device applies it by position).
std::vector<DeviceMat> upload_text_constants(const Device& device, const TextConstantsHost& constants);

// src/text_encoder.cpp:119-180: blocks in order on input [S][hidden] FP32 with the
// three constants (cos, sin, mask). Throws std::invalid_argument unless 1..25
// blocks and exactly 3 constants (src/text_encoder.cpp:41-45).
DeviceMat run_text_blocks(const std::vector<BlockModel>& models, const DeviceMat& input,
                          const std::vector<DeviceMat>& constants, const Option& option, BlockSequenceStats& stats);

}  // namespace ernie
