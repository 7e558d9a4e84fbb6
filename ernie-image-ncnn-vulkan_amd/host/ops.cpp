// SPDX-License-Identifier: MIT
// Operator registry: the op names the reference registers into ncnn::Net, with
// the parameter checks its custom layers make, forwarding to ernie_hip.
#include "ernie/ops.h"

#include <cmath>
#include <memory>
#include <stdexcept>

namespace ernie {

int OpParams::get(int id, int fallback) const
{
    auto it = ints.find(id);
    return it == ints.end() ? fallback : it->second;
}
float OpParams::get(int id, float fallback) const
{
    auto it = floats.find(id);
    return it == floats.end() ? fallback : it->second;
}

int OpRegistry::register_custom_layer(const std::string& type, OpForward forward)
{
    if (type.empty() || !forward || ops_.count(type)) return -1;
    ops_[type] = std::move(forward);
    return 0;
}

int OpRegistry::forward(const std::string& type, const Device& device, const std::vector<OpTensor>& inputs,
                        std::vector<OpTensor>& outputs, const OpParams& params, const Option& option) const
{
    auto it = ops_.find(type);
    if (it == ops_.end()) return -1;
    return it->second(device, inputs, outputs, params, option);
}

std::vector<std::string> OpRegistry::types() const
{
    std::vector<std::string> out;
    for (const auto& kv : ops_) out.push_back(kv.first);
    return out;
}

namespace {

// Temporary FP32 device copy of host data (layer weights).
struct Scratch {
    ernie_hip_ctx* ctx;
    void* ptr = nullptr;
    Scratch(ernie_hip_ctx* c, const float* host, size_t n) : ctx(c)
    {
        if (ernie_hip_malloc(ctx, (n ? n : 1) * sizeof(float), &ptr) == ERNIE_OK && n)
            if (ernie_hip_memcpy_h2d(ctx, ptr, host, n * sizeof(float)) != ERNIE_OK) {
                ernie_hip_free(ctx, ptr);
                ptr = nullptr;
            }
    }
    ~Scratch()
    {
        if (ptr) {
            ernie_hip_synchronize(ctx);
            ernie_hip_free(ctx, ptr);
        }
    }
    float* f() const { return static_cast<float*>(ptr); }
};

OpTensor& output_like(const std::vector<OpTensor>& inputs, std::vector<OpTensor>& outputs)
{
    if (outputs.empty()) outputs.push_back(inputs[0]);  // in place
    return outputs[0];
}

// ErnieGELU (src/ernie_gelu.cpp:36-61): one blob, in place.
int gelu_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams&,
                 const Option&)
{
    if (in.size() != 1 || !in[0].data) return -1;
    OpTensor& o = output_like(in, out);
    if (o.data != in[0].data) {
        if (ernie_hip_convert(d.ctx(), in[0].data, in[0].dtype, o.data, o.dtype, in[0].total())) return -1;
    }
    return ernie_hip_gelu(d.ctx(), o.data, o.dtype, o.total());
}

// ErnieRMSNorm (src/ernie_rmsnorm.cpp:34-46): affine sizes 128/3072/4096, 2=1.
int rmsnorm_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                    const Option&)
{
    const int width = p.get(0, 0);
    if (in.size() != 1 || (width != 128 && width != 3072 && width != 4096) || p.get(2, 1) != 1) return -1;
    if (p.weights.size() != size_t(width) || in[0].total() % width) return -1;
    OpTensor& o = output_like(in, out);
    Scratch gamma(d.ctx(), p.weights.data(), p.weights.size());
    if (!gamma.ptr) return -100;
    return ernie_hip_rmsnorm(d.ctx(), in[0].data, in[0].dtype, gamma.f(), nullptr, nullptr, int(in[0].total() / width),
                             width, p.get(1, 1e-6f), o.data, o.dtype);
}

// ErnieLayerNorm: non-affine LayerNorm of width 4096 (2=0), FP32 arithmetic.
int layernorm_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                      const Option&)
{
    const int width = p.get(0, 0);
    if (in.size() != 1 || width != 4096 || p.get(2, 1) != 0 || in[0].dtype != ERNIE_DTYPE_FP32) return -1;
    if (in[0].total() % width) return -1;
    OpTensor& o = output_like(in, out);
    const std::vector<float> zeros(width, 0.f);
    Scratch z(d.ctx(), zeros.data(), zeros.size());
    if (!z.ptr) return -100;
    return ernie_hip_layernorm_modulate(d.ctx(), static_cast<const float*>(in[0].data), z.f(), z.f(),
                                        int(in[0].total() / width), width, p.get(1, 1e-6f), o.data, o.dtype);
}

// ErnieResidualAdd (src/ernie_residual.cpp:31-88): BinaryOp add only, FP32 result.
int residual_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                     const Option&)
{
    if (in.size() != 2 || p.get(0, -1) != 0 || p.get(1, 0) != 0 || in[0].total() != in[1].total()) return -1;
    if (out.empty() || out[0].dtype != ERNIE_DTYPE_FP32 || !out[0].data) return -1;
    return ernie_hip_residual_add(d.ctx(), in[0].data, in[0].dtype, in[1].data, in[1].dtype,
                                  static_cast<float*>(out[0].data), in[0].total());
}

// ErnieSDPA (src/ernie_attention.cpp:153-233): q [heads][sq][d], k/v [kv_heads][sk][d],
// optional additive mask [mask_heads][1 or sq][sk] (5=1).
int sdpa_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                 const Option&)
{
    const bool has_mask = p.get(5, 0) != 0;
    if (in.size() < (has_mask ? 4u : 3u) || out.empty() || !out[0].data) return -1;
    const OpTensor &q = in[0], &k = in[1], &v = in[2];
    if (k.w != q.w || v.w != q.w || k.h != v.h || k.c != v.c || q.dtype != k.dtype || q.dtype != v.dtype) return -1;
    const float* mask = nullptr;
    int mask_heads = 1, mask_rows = 1;
    if (has_mask) {
        const OpTensor& m = in[3];
        if (m.dtype != ERNIE_DTYPE_FP32 || m.w != k.h || (m.h != 1 && m.h != q.h)) return -1;
        mask = static_cast<const float*>(m.data);
        mask_heads = m.c;
        mask_rows = m.h;
    }
    const float scale = p.get(6, 0.f);
    return ernie_hip_sdpa(d.ctx(), q.data, k.data, v.data, out[0].data, q.dtype, q.c, k.c, q.h, k.h, q.w,
                          long(q.h) * q.w, q.w, long(k.h) * k.w, k.w, long(v.h) * v.w, v.w, long(q.h) * q.w, q.w,
                          mask, mask_heads, mask_rows, 0, scale);
}

// Gemm with constant transposed B (3=1, 5=1), 7=M 8=N 9=K, 10 = -1 (no C) or
// 4 (per-column bias stored after B): block.ncnn.param lines 19-74.
int gemm_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                 const Option&)
{
    if (in.size() != 1 || p.get(3, 0) != 1 || p.get(5, 0) != 1 || p.get(2, 0) != 0) return -1;
    const int N = p.get(8, 0), K = p.get(9, 0), bias = p.get(10, -1);
    const int M = in[0].total() / (K ? K : 1);
    if (N < 1 || K < 1 || in[0].w != K || (bias != -1 && bias != 4)) return -1;
    const size_t wn = size_t(N) * K + (bias == 4 ? N : 0);
    if (p.weights.size() != wn || out.empty() || !out[0].data) return -1;
    ernie_hip_ctx* ctx = d.ctx();
    // Weights arrive as FP32 and are stored in the operand precision.
    Scratch w32(ctx, p.weights.data(), p.weights.size());
    if (!w32.ptr) return -100;
    void* wdt = w32.ptr;
    void* converted = nullptr;
    if (in[0].dtype != ERNIE_DTYPE_FP32) {
        if (ernie_hip_malloc(ctx, size_t(N) * K * 2, &converted)) return -100;
        if (ernie_hip_convert(ctx, w32.ptr, ERNIE_DTYPE_FP32, converted, in[0].dtype, size_t(N) * K)) return -1;
        wdt = converted;
    }
    const int rc = ernie_hip_gemm(ctx, in[0].data, K, wdt, K, bias == 4 ? w32.f() + size_t(N) * K : nullptr,
                                  out[0].data, N, M, N, K, in[0].dtype, out[0].dtype);
    if (converted) {
        ernie_hip_synchronize(ctx);
        ernie_hip_free(ctx, converted);
    }
    return rc;
}

}  // namespace

int register_attention(OpRegistry& registry, bool) { return registry.register_custom_layer("SDPA", sdpa_forward); }

int register_layers(OpRegistry& registry)
{
    int rc = registry.register_custom_layer("ErnieGELU", gelu_forward);
    if (!rc) rc = registry.register_custom_layer("RMSNorm", rmsnorm_forward);
    if (!rc) rc = registry.register_custom_layer("LayerNorm", layernorm_forward);
    if (!rc) rc = registry.register_custom_layer("ErnieResidualAdd", residual_forward);
    if (!rc) rc = register_attention(registry);
    if (!rc) rc = registry.register_custom_layer("Gemm", gemm_forward);
    return rc;
}

void set_attention_query_rows(const Device& device, int rows)
{
    if (ernie_hip_set_attention_query_rows(device.ctx(), rows) != ERNIE_OK)
        throw std::invalid_argument("Attention query rows must be 128, 64, 32 or 16");
}

uint64_t attention_internal_submissions(const Device& device)
{
    return ernie_hip_attention_internal_submissions(device.ctx());
}

}  // namespace ernie
