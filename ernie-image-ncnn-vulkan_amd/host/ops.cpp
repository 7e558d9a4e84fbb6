// SPDX-License-Identifier: MIT
// Operator registry: the op names the reference registers into ncnn::Net, with
// the parameter checks its custom layers make, forwarding to ernie_hip.
#include "ernie/ops.h"

#include <cmath>
#include <cstdlib>
#include <memory>
#include <sstream>
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

OpParams OpParams::parse(const std::string& text)
{
    // ncnn ParamDict text form: "id=value" pairs; a value with a decimal point or an
    // exponent is a float, any other an int (the distinction ncnn makes when it reads a
    // .param line; tests/test_bf16_gemm.cpp:58-60 relies on it).
    OpParams p;
    std::istringstream in(text);
    std::string token;
    while (in >> token) {
        const size_t eq = token.find('=');
        if (eq == std::string::npos || eq == 0 || eq + 1 == token.size())
            throw std::invalid_argument("Malformed op parameter: " + token);
        char* end = nullptr;
        const long id = std::strtol(token.c_str(), &end, 10);
        if (end != token.c_str() + eq || id < 0 || id > 31)
            throw std::invalid_argument("Op parameter id out of range: " + token);
        const std::string value = token.substr(eq + 1);
        if (value.find_first_of(".eE") != std::string::npos) {
            const float v = std::strtof(value.c_str(), &end);
            if (*end) throw std::invalid_argument("Malformed float op parameter: " + token);
            p.floats[int(id)] = v;
        } else {
            const long v = std::strtol(value.c_str(), &end, 10);
            if (*end) throw std::invalid_argument("Malformed int op parameter: " + token);
            p.ints[int(id)] = int(v);
        }
    }
    return p;
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

// Device scratch owned by one op call. Released to the context's block cache when the
// call returns, without a wait: reuse of a cached block is ordered by the context
// stream, after the work queued here.
class Scratch {
public:
    Scratch(ernie_hip_ctx* ctx, size_t bytes) : ctx_(ctx)
    {
        if (ernie_hip_malloc(ctx_, bytes ? bytes : 1, &ptr_) != ERNIE_OK) ptr_ = nullptr;
    }
    // FP32 copy of host values (layer weights).
    Scratch(ernie_hip_ctx* ctx, const float* host, size_t n) : Scratch(ctx, n * sizeof(float))
    {
        if (ptr_ && n && ernie_hip_memcpy_h2d(ctx_, ptr_, host, n * sizeof(float)) != ERNIE_OK) release();
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    ~Scratch() { release(); }
    explicit operator bool() const { return ptr_ != nullptr; }
    void* get() const { return ptr_; }
    float* f() const { return static_cast<float*>(ptr_); }

private:
    void release()
    {
        if (ptr_) ernie_hip_free(ctx_, ptr_);
        ptr_ = nullptr;
    }
    ernie_hip_ctx* ctx_;
    void* ptr_ = nullptr;
};

size_t esize(int dtype) { return dtype == ERNIE_DTYPE_FP32 ? 4 : 2; }

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
    if (!o.data || o.total() != in[0].total()) return -1;
    if (o.data != in[0].data && ernie_hip_convert(d.ctx(), in[0].data, in[0].dtype, o.data, o.dtype, in[0].total()))
        return -1;
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
    if (!o.data || o.total() != in[0].total()) return -1;
    Scratch gamma(d.ctx(), p.weights.data(), p.weights.size());
    if (!gamma) return -100;
    // The reference layer runs in place (forward_inplace); the kernel reads and writes
    // distinct buffers, so an in-place call goes through a scratch copy.
    const bool inplace = o.data == in[0].data;
    Scratch tmp(d.ctx(), inplace ? o.total() * esize(o.dtype) : 0);
    if (inplace && !tmp) return -100;
    void* dst = inplace ? tmp.get() : o.data;
    const int rc = ernie_hip_rmsnorm(d.ctx(), in[0].data, in[0].dtype, gamma.f(), nullptr, nullptr,
                                     int(in[0].total() / width), width, p.get(1, 1e-6f), dst, o.dtype);
    if (rc || !inplace) return rc;
    return ernie_hip_convert(d.ctx(), dst, o.dtype, o.data, o.dtype, o.total());
}

// ErnieLayerNorm: non-affine LayerNorm of width 4096 (2=0), FP32 arithmetic.
int layernorm_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                      const Option&)
{
    const int width = p.get(0, 0);
    if (in.size() != 1 || width != 4096 || p.get(2, 1) != 0 || in[0].dtype != ERNIE_DTYPE_FP32) return -1;
    if (in[0].total() % width) return -1;
    OpTensor& o = output_like(in, out);
    if (!o.data || o.total() != in[0].total()) return -1;
    const std::vector<float> zeros(width, 0.f);
    Scratch z(d.ctx(), zeros.data(), zeros.size());
    if (!z) return -100;
    const bool inplace = o.data == in[0].data;
    Scratch tmp(d.ctx(), inplace ? o.total() * esize(o.dtype) : 0);
    if (inplace && !tmp) return -100;
    void* dst = inplace ? tmp.get() : o.data;
    const int rc = ernie_hip_layernorm_modulate(d.ctx(), static_cast<const float*>(in[0].data), z.f(), z.f(),
                                                int(in[0].total() / width), width, p.get(1, 1e-6f), dst, o.dtype);
    if (rc || !inplace) return rc;
    return ernie_hip_convert(d.ctx(), dst, o.dtype, o.data, o.dtype, o.total());
}

// ErnieResidualAdd (src/ernie_residual.cpp:31-88): BinaryOp add only, FP32 result.
int residual_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                     const Option&)
{
    if (in.size() != 2 || p.get(0, -1) != 0 || p.get(1, 0) != 0 || in[0].total() != in[1].total()) return -1;
    if (out.empty() || out[0].dtype != ERNIE_DTYPE_FP32 || !out[0].data || out[0].total() != in[0].total()) return -1;
    return ernie_hip_residual_add(d.ctx(), in[0].data, in[0].dtype, in[1].data, in[1].dtype,
                                  static_cast<float*>(out[0].data), in[0].total());
}

// ErnieSDPA (src/ernie_attention.cpp:153-233): q [heads][sq][d], k/v [kv_heads][sk][d],
// optional additive mask [mask_heads][1 or sq][sk] (5=1); 6 = scale (0: 1/sqrt(d)).
int sdpa_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                 const Option&)
{
    const bool has_mask = p.get(5, 0) != 0;
    if (in.size() != (has_mask ? 4u : 3u) || out.empty() || !out[0].data) return -1;
    const OpTensor &q = in[0], &k = in[1], &v = in[2];
    if (k.w != q.w || v.w != q.w || k.h != v.h || k.c != v.c || q.dtype != k.dtype || q.dtype != v.dtype) return -1;
    if (out[0].total() != q.total() || out[0].dtype != q.dtype) return -1;
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

// ncnn Gemm with a constant B (5=1): 0 = alpha, 1 = beta (both 1), 2 = transA,
// 3 = transB, 7/8/9 = M/N/K, 10 = constant C broadcast (-1 none, 3 = [M][N],
// 4 = [N]), 11 = output N1M (a [M][1][N] blob), 14 = output transpose. Weights are
// B ([N][K] with 3=1, else [K][N]), then C. The block graph uses 3=1 5=1 10=-1
// (block.ncnn.param lines 19-74); tests/test_bf16_gemm.cpp:58-70 covers the rest.
// The product runs as the NT kernel; transA and the output transpose are device
// transposes around it, transB=0 a host transpose of the constant weights.
int gemm_forward(const Device& d, const std::vector<OpTensor>& in, std::vector<OpTensor>& out, const OpParams& p,
                 const Option&)
{
    if (in.size() != 1 || !in[0].data || out.empty() || !out[0].data) return -1;
    if (p.get(0, 1.f) != 1.f || p.get(1, 1.f) != 1.f || p.get(4, 0) != 0 || p.get(5, 0) != 1) return -1;
    const int trans_a = p.get(2, 0), trans_b = p.get(3, 0), bias = p.get(10, -1), trans_out = p.get(14, 0);
    const int N = p.get(8, 0), K = p.get(9, 0);
    const OpTensor& a = in[0];
    if (a.c != 1 || (trans_a != 0 && trans_a != 1) || (trans_b != 0 && trans_b != 1) ||
        (trans_out != 0 && trans_out != 1))
        return -1;
    const int M = trans_a ? a.w : a.h;
    if (N < 1 || K < 1 || (trans_a ? a.h : a.w) != K || (p.get(7, 0) && p.get(7, 0) != M)) return -1;
    if (bias != -1 && bias != 3 && bias != 4) return -1;
    const size_t nb = size_t(N) * K, nc = bias == 4 ? size_t(N) : bias == 3 ? size_t(M) * N : 0;
    if (p.weights.size() != nb + nc) return -1;
    OpTensor& o = out[0];
    const int out_w = trans_out ? M : N, out_rows = trans_out ? N : M;
    const bool n1m = p.get(11, 0) != 0;
    if (o.w != out_w || (n1m ? (o.h != 1 || o.c != out_rows) : (o.h != out_rows || o.c != 1))) return -1;
    if (o.dtype != ERNIE_DTYPE_FP32 && o.dtype != a.dtype) return -1;
    ernie_hip_ctx* ctx = d.ctx();
    const int dt = a.dtype;
    const size_t e = esize(dt);

    // W as [N][K] in the operand precision.
    std::vector<float> wt;
    const float* w_host = p.weights.data();
    if (!trans_b) {
        wt.resize(nb);
        for (int k = 0; k < K; ++k)
            for (int n = 0; n < N; ++n) wt[size_t(n) * K + k] = p.weights[size_t(k) * N + n];
        w_host = wt.data();
    }
    Scratch w32(ctx, w_host, nb);
    Scratch c_dev(ctx, p.weights.data() + nb, nc);
    if (!w32 || (nc && !c_dev)) return -100;
    const void* w_op = w32.get();
    Scratch w16(ctx, dt == ERNIE_DTYPE_FP32 ? 0 : nb * e);
    if (dt != ERNIE_DTYPE_FP32) {
        if (!w16) return -100;
        if (ernie_hip_convert(ctx, w32.get(), ERNIE_DTYPE_FP32, w16.get(), dt, nb)) return -1;
        w_op = w16.get();
    }
    // A as [M][K].
    const void* a_op = a.data;
    Scratch at(ctx, trans_a ? size_t(M) * K * e : 0);
    if (trans_a) {
        if (!at) return -100;
        if (ernie_hip_transpose(ctx, a.data, dt, K, M, at.get())) return -1;
        a_op = at.get();
    }
    // [M][N] result: straight into the output unless it is transposed afterwards or a
    // matrix C is added in FP32 before the one rounding to the output precision.
    const int prod_dt = bias == 3 ? ERNIE_DTYPE_FP32 : o.dtype;
    const bool direct = !trans_out && prod_dt == o.dtype;
    Scratch prod(ctx, direct ? 0 : size_t(M) * N * esize(prod_dt));
    if (!direct && !prod) return -100;
    void* c_out = direct ? o.data : prod.get();
    if (ernie_hip_gemm(ctx, a_op, K, w_op, K, bias == 4 ? c_dev.f() : nullptr, c_out, N, M, N, K, dt, prod_dt))
        return -1;
    if (bias == 3) {
        float* sum = static_cast<float*>(c_out);
        if (ernie_hip_residual_add(ctx, sum, ERNIE_DTYPE_FP32, c_dev.get(), ERNIE_DTYPE_FP32, sum, size_t(M) * N))
            return -1;
        if (direct) return 0;  // FP32 output in place
        if (o.dtype == ERNIE_DTYPE_FP32) return ernie_hip_transpose(ctx, sum, o.dtype, M, N, o.data) ? -1 : 0;
        if (!trans_out) return ernie_hip_convert(ctx, sum, ERNIE_DTYPE_FP32, o.data, o.dtype, size_t(M) * N) ? -1 : 0;
        // Round once to the output precision, then move the rounded values.
        Scratch r(ctx, size_t(M) * N * e);
        if (!r) return -100;
        if (ernie_hip_convert(ctx, sum, ERNIE_DTYPE_FP32, r.get(), o.dtype, size_t(M) * N)) return -1;
        return ernie_hip_transpose(ctx, r.get(), o.dtype, M, N, o.data) ? -1 : 0;
    }
    if (trans_out) return ernie_hip_transpose(ctx, c_out, o.dtype, M, N, o.data) ? -1 : 0;
    return 0;
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
