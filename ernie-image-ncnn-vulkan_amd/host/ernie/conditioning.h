// SPDX-License-Identifier: MIT
// Shared DiT constants: RoPE tables and the one-row attention mask
// (src/conditioning.h; src/conditioning.cpp:10-67).
#pragma once
#include <string>
#include <vector>

#include "ernie/runtime.h"

namespace ernie {

struct DitConstantsHost {
    int length = 0, valid_keys = 0;
    std::vector<float> cos, sin, mask;  // [length][128], [length][128], [length]
};

// Official 3-axis frequency table, 64 FP32 values (16 + 24 + 24) =
// cat_{dim in 32,48,48} 1/256^(arange(0,dim,2)/dim) (tools/prepare_pipeline.py:63).
std::vector<float> rope_frequencies();
// src/conditioning.cpp:10-43. token_limit 10240 (the ShapePlan overload's bound).
// Throws std::invalid_argument for invalid dimensions or frequencies.
DitConstantsHost dit_constants(const std::vector<float>& frequencies, int width, int height, int valid_text,
                               int text_bucket, int token_limit = 10240);
// src/conditioning.cpp:10-23,46-49: the same from the frequency file the reference
// ships (exactly 64 FP32 values, 256 bytes), read and checked, with that overload's
// token limit of 6144. Dimension or file-size errors throw std::invalid_argument; an
// unreadable file or a non-finite / non-positive frequency std::runtime_error.
DitConstantsHost dit_constants(const std::string& frequency_path, int width, int height, int valid_text,
                               int text_bucket);
// Uploads: cosine, sine, attention mask (mask carries valid_prefix).
std::vector<DeviceMat> upload_constants(const Device& device, const DitConstantsHost& constants);
// src/conditioning.cpp:56-67: zero-pad [tokens][3072] text embeddings to `bucket` rows.
std::vector<float> pad_text(const std::vector<float>& embeddings, int tokens, int bucket);

}  // namespace ernie
