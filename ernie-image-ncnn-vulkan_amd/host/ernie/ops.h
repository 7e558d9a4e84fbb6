// SPDX-License-Identifier: MIT
// Operator registry: the plugin surface the reference registers into ncnn::Net
// (register_layers, src/ernie_gelu.cpp:108-116; register_rmsnorm/layernorm
// src/ernie_rmsnorm.cpp:150-157; register_residual src/ernie_residual.cpp:95-98;
// register_attention src/ernie_attention.cpp:239-244). ncnn is not part of this
// build, so the registry maps the same op names to device launchers.
#pragma once
#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "ernie/runtime.h"

namespace ernie {

// A device tensor argument for an op: pointer, dtype and ncnn-style dims.
struct OpTensor {
    void* data = nullptr;
    int dtype = ERNIE_DTYPE_FP32;
    int w = 0, h = 1, c = 1;
    size_t total() const { return size_t(w) * h * c; }
};

// Layer parameters in ncnn ParamDict spirit: integer/float by id.
struct OpParams {
    std::map<int, int> ints;
    std::map<int, float> floats;
    std::vector<float> weights;  // e.g. the RMSNorm gamma (FP32), uploaded by the op
    int get(int id, int fallback) const;
    float get(int id, float fallback) const;
    // "0=4096 1=1.000000e-6 2=1": the id=value list of a .param layer line; a value
    // with '.', 'e' or 'E' is a float, else an int. Throws std::invalid_argument.
    static OpParams parse(const std::string& text);
};

// Returns 0 / -1 / -100 like ncnn::Layer::forward.
using OpForward = std::function<int(const Device&, const std::vector<OpTensor>& inputs,
                                    std::vector<OpTensor>& outputs, const OpParams& params, const Option& option)>;

class OpRegistry {
public:
    int register_custom_layer(const std::string& type, OpForward forward);
    bool has(const std::string& type) const { return ops_.count(type) != 0; }
    int forward(const std::string& type, const Device& device, const std::vector<OpTensor>& inputs,
                std::vector<OpTensor>& outputs, const OpParams& params, const Option& option) const;
    std::vector<std::string> types() const;

private:
    std::map<std::string, OpForward> ops_;
};

// Registers "ErnieGELU", "RMSNorm", "LayerNorm", "ErnieResidualAdd", "SDPA"
// and "Gemm". Returns 0, or non-zero when a name is already registered.
int register_layers(OpRegistry& registry);
int register_attention(OpRegistry& registry, bool bounded_workspace = true);
// Accepted for compatibility; the flash kernel needs no query chunking.
void set_attention_query_rows(const Device& device, int rows);
uint64_t attention_internal_submissions(const Device& device);

}  // namespace ernie
