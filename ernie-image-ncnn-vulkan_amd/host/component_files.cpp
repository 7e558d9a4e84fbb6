// SPDX-License-Identifier: MIT
// DiT head and text block readers (declared in ernie/component_files.h).
#include "ernie/component_files.h"

#include <cerrno>
#include <cstdlib>
#include <set>
#include <stdexcept>

#include "ernie/runtime.h"

namespace ernie {
namespace {

// Normalised-graph hashes of the reviewed runtime contracts, src/shape_graph.cpp:31.
const char* const kInputHeadContract = "3710a502802138e8605ca54a9132fb9a9a1888841586c1d7067f7043769bbecb";
const char* const kOutputHeadContract = "98bf1afc154dd05cf419aafad4aa383af311e44658e644d0c322ffb50431533c";
const char* const kTextContract = "dda8db13b6e20a00c1133485c3be2ef37db56b1db058e42a405b51d24fc64b0e";

[[noreturn]] void bad(const std::string& what) { throw std::invalid_argument(what); }

long to_long(const std::string& v, const std::string& what)
{
    char* end = nullptr;
    errno = 0;
    const long x = std::strtol(v.c_str(), &end, 10);
    if (v.empty() || errno || *end) bad("invalid integer '" + v + "' in " + what);
    return x;
}

long iparam(const GraphLayer& l, const char* key, long dflt)
{
    const std::string* v = l.param(key);
    return v ? to_long(*v, "parameter " + std::string(key) + " of " + l.name) : dflt;
}

double fparam(const GraphLayer& l, const char* key, double dflt)
{
    const std::string* v = l.param(key);
    if (!v) return dflt;
    char* end = nullptr;
    const double x = std::strtod(v->c_str(), &end);
    if (v->empty() || *end) bad("invalid number '" + *v + "' in parameter " + key + " of " + l.name);
    return x;
}

const GraphLayer& layer(const Graph& g, const std::string& name, const std::string& type)
{
    for (const GraphLayer& l : g.layers)
        if (l.name == name) {
            if (l.type != type) bad("layer " + name + " is " + l.type + ", expected " + type);
            return l;
        }
    bad("graph lacks layer " + type + " " + name);
}

void check_types(const Graph& g, const std::set<std::string>& known, const char* what)
{
    for (const GraphLayer& l : g.layers)
        if (!known.count(l.type)) bad("layer " + l.name + " has a type outside the " + what + ": " + l.type);
}

void check_io(const Graph& g, int inputs, int outputs, const char* what)
{
    std::set<std::string> in, out;
    for (const GraphLayer& l : g.layers) {
        if (l.type == "Input") in.insert(l.name);
        for (const std::string& o : l.outputs) out.insert(o);
    }
    for (int i = 0; i < inputs; ++i)
        if (!in.count("in" + std::to_string(i))) bad(std::string(what) + " graph lacks input in" + std::to_string(i));
    if ((int)in.size() != inputs) bad(std::string(what) + " graph must have exactly " + std::to_string(inputs) + " inputs");
    for (int i = 0; i < outputs; ++i)
        if (!out.count("out" + std::to_string(i))) bad(std::string(what) + " graph lacks output out" + std::to_string(i));
}

// Weighted layers in graph (= .bin) order.
std::vector<const GraphLayer*> weighted(const Graph& g, const std::set<std::string>& types)
{
    std::vector<const GraphLayer*> w;
    for (const GraphLayer& l : g.layers)
        if (types.count(l.type)) w.push_back(&l);
    return w;
}

// Constant-B Gemm A.B^T with alpha 1 and no operand or output transposes
// (2=0 3=1 4=0 5=1 14=0); `bias` selects 10=4 (per-column C) instead of 10=-1.
void check_gemm(const GraphLayer& l, bool bias)
{
    if (iparam(l, "2", 0) != 0 || iparam(l, "3", 0) != 1 || iparam(l, "4", 0) != 0 || iparam(l, "5", 0) != 1 ||
        iparam(l, "14", 0) != 0 || iparam(l, "10", -1) != (bias ? 4 : -1) || fparam(l, "0", 1.0) != 1.0 ||
        (bias && (iparam(l, "6", 0) != 1 || fparam(l, "1", 1.0) != 1.0)))
        bad(l.name + std::string(" is not the constant-B Gemm A.B^T") + (bias ? " + bias" : ""));
}

// InnerProduct with a bias and no activation; returns num_output, checks the weight size.
long check_inner_product(const GraphLayer& l, long k)
{
    const long n = iparam(l, "0", 0);
    if (n < 1 || iparam(l, "1", 0) != 1 || iparam(l, "2", 0) != n * k || iparam(l, "9", 0) != 0 ||
        iparam(l, "8", 0) != 0)
        bad(l.name + " is not a biased FP InnerProduct of " + std::to_string(k) + " inputs");
    return n;
}

}  // namespace

// ---- heads ------------------------------------------------------------------------------
HeadGraph inspect_head_graph(const std::string& text, bool allow_unreviewed)
{
    HeadGraph h;
    h.graph = parse_graph(text);
    const Graph& g = h.graph;
    const std::vector<const GraphLayer*> w = weighted(g, {"Convolution", "InnerProduct", "Gemm"});
    const bool input = !w.empty() && w[0]->type == "Convolution";
    h.kind = input ? HeadKind::Input : HeadKind::Output;
    if (input) {
        // heads/input head.ncnn.param: conv_1 -> reshape_7 -> transpose_9 ++ gemm_0 -> cat_0 (out0);
        // linear_2 -> silu_5 -> linear_3 (out1) -> silu_6 -> linear_4 -> reshape_8 -> out2..out7.
        check_types(g, {"Input", "Convolution", "Reshape", "Permute", "Gemm", "Concat", "InnerProduct", "Swish",
                        "Split", "Slice"}, "DiT input head");
        check_io(g, 3, 8, "input head");
        if (w.size() != 5 || w[0]->name != "conv_1" || w[1]->name != "gemm_0" || w[1]->type != "Gemm" ||
            w[2]->name != "linear_2" || w[3]->name != "linear_3" || w[4]->name != "linear_4" ||
            w[2]->type != "InnerProduct" || w[3]->type != "InnerProduct" || w[4]->type != "InnerProduct")
            bad("input head must hold conv_1, gemm_0, linear_2, linear_3 and linear_4 in that order");
        const GraphLayer& conv = *w[0];
        const long dim = iparam(conv, "0", 0);
        const long size = iparam(conv, "6", 0);
        // A 1x1, stride 1, unpadded, biased convolution without activation.
        if (dim < 1 || iparam(conv, "1", 0) != 1 || iparam(conv, "11", 1) != 1 || iparam(conv, "2", 1) != 1 ||
            iparam(conv, "12", 1) != 1 || iparam(conv, "3", 1) != 1 || iparam(conv, "13", 1) != 1 ||
            iparam(conv, "4", 0) != 0 || iparam(conv, "14", 0) != 0 || iparam(conv, "5", 0) != 1 ||
            iparam(conv, "9", 0) != 0 || size < dim || size % dim)
            bad("conv_1 is not the 1x1 x_embedder convolution with a bias");
        const GraphLayer& text_proj = *w[1];
        check_gemm(text_proj, false);
        if (iparam(text_proj, "8", 0) != dim) bad("gemm_0 must project the text rows to the conv_1 width");
        if (check_inner_product(*w[2], dim) != dim || check_inner_product(*w[3], dim) != dim ||
            check_inner_product(*w[4], dim) != 6 * dim)
            bad("the time MLP must be dim -> dim -> dim and the adaLN projection dim -> 6 dim");
        const GraphLayer& reshape = layer(g, "reshape_7", "Reshape");
        h.dim = (int)dim;
        h.latent_ch = (int)(size / dim);
        h.text_dim = (int)iparam(text_proj, "9", 0);
        h.text_tokens = (int)iparam(text_proj, "7", 0);
        h.image_tokens = (int)iparam(reshape, "0", 0);
        h.tokens = h.image_tokens + h.text_tokens;
        if (h.text_dim < 1 || h.text_tokens < 1 || h.image_tokens < 1 || iparam(reshape, "1", 0) != dim)
            bad("input head shapes are inconsistent");
        h.contract_sha256 = shape_contract_sha256(
            text, {{"reshape_7", "0", "IMAGE_TOKENS", std::to_string(h.image_tokens)},
                   {"gemm_0", "7", "DIT_TEXT_TOKENS", std::to_string(h.text_tokens)}});
        h.reviewed = h.contract_sha256 == kInputHeadContract;
    } else {
        // heads/output head.ncnn.param: linear_2 -> chunk_0 (scale, shift); ln_1 -> modulate ->
        // gemm_0 (+ bias) -> slice_0 (image rows) -> transpose_6 -> reshape_5 (out0).
        check_types(g, {"Input", "InnerProduct", "Slice", "LayerNorm", "Reshape", "BinaryOp", "Gemm", "Crop",
                        "Permute"}, "DiT output head");
        check_io(g, 2, 1, "output head");
        if (w.size() != 2 || w[0]->name != "linear_2" || w[0]->type != "InnerProduct" || w[1]->name != "gemm_0" ||
            w[1]->type != "Gemm")
            bad("output head must hold linear_2 and gemm_0 in that order");
        const GraphLayer& ln = layer(g, "ln_1", "LayerNorm");
        const long dim = iparam(ln, "0", 0);
        if (dim < 1 || iparam(ln, "2", 1) != 0 || (float)fparam(ln, "1", 0) != 1e-6f)
            bad("ln_1 must be the non-affine LayerNorm with eps 1e-6");
        if (check_inner_product(*w[0], dim) != 2 * dim) bad("linear_2 must map dim -> 2 dim (scale, shift)");
        const GraphLayer& proj = *w[1];
        check_gemm(proj, true);
        if (iparam(proj, "9", 0) != dim) bad("gemm_0 must project dim-wide rows");
        const GraphLayer& crop = layer(g, "slice_0", "Crop");
        const GraphLayer& shape = layer(g, "reshape_5", "Reshape");
        const std::string* ends = crop.param("-23310");
        if (!ends || ends->compare(0, 2, "1,") != 0) bad("slice_0 must keep the first image rows");
        h.dim = (int)dim;
        h.latent_ch = (int)iparam(proj, "8", 0);
        h.tokens = (int)iparam(proj, "7", 0);
        h.image_tokens = (int)to_long(ends->substr(2), "slice_0");
        h.width = (int)iparam(shape, "0", 0);
        h.height = (int)iparam(shape, "1", 0);
        if (h.latent_ch < 1 || h.width < 1 || h.height < 1 || h.image_tokens != h.width * h.height ||
            h.tokens < h.image_tokens || iparam(shape, "2", 0) != h.latent_ch)
            bad("output head shapes are inconsistent");
        h.text_tokens = h.tokens - h.image_tokens;
        h.contract_sha256 = shape_contract_sha256(
            text, {{"gemm_0", "7", "TOTAL_TOKENS", std::to_string(h.tokens)},
                   {"slice_0", "-23310", "IMAGE_TOKENS_ARRAY", "1," + std::to_string(h.image_tokens)},
                   {"reshape_5", "0", "PACKED_WIDTH", std::to_string(h.width)},
                   {"reshape_5", "1", "PACKED_HEIGHT", std::to_string(h.height)}});
        h.reviewed = h.contract_sha256 == kOutputHeadContract;
    }
    if (!h.reviewed && !allow_unreviewed)
        bad(std::string("graph differs from the reviewed ERNIE ") + (input ? "input" : "output") +
            " head topology (normalised sha256 " + (h.contract_sha256.empty() ? "n/a" : h.contract_sha256) + ")");
    return h;
}

std::vector<WeightSection> head_sections(const HeadGraph& g, const unsigned char* bin, size_t size)
{
    std::vector<WeightSection> out;
    const size_t D = g.dim;
    auto tagged = [&](const char* name, size_t n) {
        out.push_back(tagged_section(name, bin, size, out.empty() ? 0 : out.back().end, n));
    };
    auto raw = [&](const char* name, size_t n) {
        out.push_back(raw_section(name, size, out.empty() ? 0 : out.back().end, n));
    };
    if (g.kind == HeadKind::Input) {
        tagged("conv_1", D * g.latent_ch);
        raw("conv_1.bias", D);
        tagged("gemm_0", D * g.text_dim);
        tagged("linear_2", D * D);
        raw("linear_2.bias", D);
        tagged("linear_3", D * D);
        raw("linear_3.bias", D);
        tagged("linear_4", 6 * D * D);
        raw("linear_4.bias", 6 * D);
    } else {
        tagged("linear_2", 2 * D * D);
        raw("linear_2.bias", 2 * D);
        tagged("gemm_0", (size_t)g.latent_ch * D);
        raw("gemm_0.bias", g.latent_ch);
    }
    check_sections_end(out, size);
    return out;
}

namespace {

HeadFile inspect_head_bytes(const std::string& param_path, const unsigned char* bin, size_t size,
                            bool allow_unreviewed, const std::string& expected_bin_sha256)
{
    HeadFile f;
    f.graph = inspect_head_graph(read_graph_text(param_path), allow_unreviewed);
    if (!bin) {
        if (!expected_bin_sha256.empty()) bad("a weight checksum was given without a weight file");
        return f;
    }
    f.bin_bytes = size;
    check_bin_sha256(bin, size, expected_bin_sha256, &f.bin_sha256);
    f.sections = head_sections(f.graph, bin, size);
    return f;
}

TextBlockFile inspect_text_bytes(const std::string& param_path, const unsigned char* bin, size_t size,
                                 bool allow_unreviewed, const std::string& expected_bin_sha256)
{
    TextBlockFile f;
    f.graph = inspect_text_block_graph(read_graph_text(param_path), allow_unreviewed);
    if (!bin) {
        if (!expected_bin_sha256.empty()) bad("a weight checksum was given without a weight file");
        return f;
    }
    f.bin_bytes = size;
    check_bin_sha256(bin, size, expected_bin_sha256, &f.bin_sha256);
    f.sections = text_block_sections(f.graph, bin, size);
    return f;
}

}  // namespace

HeadFile inspect_head_files(const std::string& param_path, const std::string& bin_path, bool allow_unreviewed,
                            const std::string& expected_bin_sha256)
{
    if (bin_path.empty()) return inspect_head_bytes(param_path, nullptr, 0, allow_unreviewed, expected_bin_sha256);
    const MappedFile bin(bin_path);
    return inspect_head_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
}

HeadModel load_head_files(const Device& device, const std::string& param_path, const std::string& bin_path,
                          int storage_dtype, bool allow_unreviewed, const std::string& expected_bin_sha256,
                          HeadFile* info)
{
    if (storage_dtype != ERNIE_DTYPE_FP32 && storage_dtype != ERNIE_DTYPE_FP16 && storage_dtype != ERNIE_DTYPE_BF16)
        throw std::invalid_argument("invalid storage dtype");
    if (bin_path.empty()) throw std::invalid_argument("a weight file is required to load a head");
    const MappedFile bin(bin_path);
    HeadFile f = inspect_head_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
    auto t = [&](size_t i) { return ernie_host_tensor{bin.data() + f.sections[i].data, f.sections[i].dtype}; };
    ernie_heads_host_tensors w{};
    const int part = static_cast<int>(f.graph.kind);
    if (f.graph.kind == HeadKind::Input) {
        w.x_w = t(0); w.x_b = t(1); w.text_w = t(2); w.t1_w = t(3); w.t1_b = t(4);
        w.t2_w = t(5); w.t2_b = t(6); w.mod_w = t(7); w.mod_b = t(8);
    } else {
        w.out_mod_w = t(0); w.out_mod_b = t(1); w.proj_w = t(2); w.proj_b = t(3);
    }
    check_status(ernie_hip_heads_upload_tensors(device.ctx(), &w, f.graph.dim, f.graph.latent_ch, f.graph.text_dim,
                                                storage_dtype, part),
                 device.ctx(), "head upload");
    if (info) *info = std::move(f);
    return HeadModel{part};
}

HeadModel resident_head(const Device& device, int part)
{
    if (part != ERNIE_HEAD_INPUT && part != ERNIE_HEAD_OUTPUT) throw std::invalid_argument("unknown head part");
    if (!(ernie_hip_heads_loaded(device.ctx()) & part))
        throw std::invalid_argument(std::string("the ") + (part == ERNIE_HEAD_INPUT ? "input" : "output") +
                                    " head is not loaded");
    return HeadModel{part};
}

// ---- text blocks --------------------------------------------------------------------------
TextBlockGraph inspect_text_block_graph(const std::string& text, bool allow_unreviewed)
{
    TextBlockGraph t;
    t.graph = parse_graph(text);
    const Graph& g = t.graph;
    check_types(g, {"Input", "Split", "RMSNorm", "Gemm", "Reshape", "Permute", "Slice", "BinaryOp", "Concat", "SDPA",
                    "Swish"}, "text block");
    check_io(g, 4, 1, "text block");
    static const char* const kNames[9] = {"rmsn_8", "gemm_0", "gemm_1", "gemm_2", "gemm_3",
                                          "rmsn_9", "gemm_4", "gemm_5", "gemm_6"};
    const std::vector<const GraphLayer*> w = weighted(g, {"RMSNorm", "Gemm"});
    if (w.size() != 9) bad("text block graph must hold 2 RMSNorm and 7 Gemm layers");
    long tokens = -1;
    long n[9] = {}, k[9] = {};
    for (int i = 0; i < 9; ++i) {
        const GraphLayer& l = *w[i];
        const bool norm = i == 0 || i == 5;
        if (l.name != kNames[i] || (l.type == "RMSNorm") != norm)
            bad("weighted layer " + std::to_string(i) + " is " + l.type + " " + l.name + ", expected " + kNames[i]);
        if (norm) {
            // Mistral RMSNorm: affine, eps 1e-5 (text-s64.ncnn.param lines 8, 53).
            n[i] = iparam(l, "0", 0);
            if (n[i] < 1 || iparam(l, "2", 0) != 1 || (float)fparam(l, "1", 0) != 1e-5f)
                bad(l.name + " must be an affine RMSNorm with eps 1e-5");
        } else {
            check_gemm(l, false);
            const long m = iparam(l, "7", 0);
            if (m < 1 || (tokens >= 0 && m != tokens)) bad("Gemm token counts differ or are missing");
            tokens = m;
            n[i] = iparam(l, "8", 0);
            k[i] = iparam(l, "9", 0);
            if (n[i] < 1 || k[i] < 1) bad(l.name + " lacks its weight shape");
        }
    }
    const long hidden = n[0], q = n[1], kv = n[2], ffn = n[6];
    const bool shapes = k[1] == hidden && k[2] == hidden && n[3] == kv && k[3] == hidden && n[4] == hidden &&
                        k[4] == q && n[5] == hidden && k[6] == hidden && n[7] == ffn && k[7] == hidden &&
                        n[8] == hidden && k[8] == ffn && q % 128 == 0 && kv % 128 == 0 && (q / 128) % (kv / 128) == 0;
    if (!shapes) bad("text block weight shapes are inconsistent (head_dim must be 128)");
    t.tokens = (int)tokens;
    t.hidden = (int)hidden;
    t.heads = (int)(q / 128);
    t.kv_heads = (int)(kv / 128);
    t.ffn = (int)ffn;
    const std::string b = std::to_string(tokens);
    std::vector<ShapeField> fields;
    for (const char* node : {"gemm_0", "gemm_1", "gemm_2", "gemm_3", "gemm_4", "gemm_5", "gemm_6"})
        fields.push_back({node, "7", "TEXT_BUCKET", b});
    for (const char* node : {"reshape_10", "reshape_11", "reshape_12"}) fields.push_back({node, "2", "TEXT_BUCKET", b});
    for (const char* node : {"reshape_13", "unsqueeze_18", "unsqueeze_19"}) fields.push_back({node, "1", "TEXT_BUCKET", b});
    t.contract_sha256 = shape_contract_sha256(text, fields);
    t.reviewed = t.contract_sha256 == kTextContract;
    if (!t.reviewed && !allow_unreviewed)
        bad("graph differs from the reviewed Mistral text block topology (normalised sha256 " +
            (t.contract_sha256.empty() ? std::string("n/a") : t.contract_sha256) + ")");
    return t;
}

std::vector<WeightSection> text_block_sections(const TextBlockGraph& g, const unsigned char* bin, size_t size)
{
    std::vector<WeightSection> out;
    for (const GraphLayer& l : g.graph.layers) {
        const size_t off = out.empty() ? 0 : out.back().end;
        if (l.type == "RMSNorm")
            out.push_back(raw_section(l.name, size, off, (size_t)iparam(l, "0", 0)));
        else if (l.type == "Gemm")
            out.push_back(tagged_section(l.name, bin, size, off, (size_t)iparam(l, "8", 0) * (size_t)iparam(l, "9", 0)));
    }
    check_sections_end(out, size);
    return out;
}

TextBlockFile inspect_text_block_files(const std::string& param_path, const std::string& bin_path,
                                       bool allow_unreviewed, const std::string& expected_bin_sha256)
{
    if (bin_path.empty()) return inspect_text_bytes(param_path, nullptr, 0, allow_unreviewed, expected_bin_sha256);
    const MappedFile bin(bin_path);
    return inspect_text_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
}

TextBlockFile load_text_block_files(const Device& device, int index, const std::string& param_path,
                                    const std::string& bin_path, int storage_dtype, bool allow_unreviewed,
                                    const std::string& expected_bin_sha256)
{
    if (storage_dtype != ERNIE_DTYPE_FP32 && storage_dtype != ERNIE_DTYPE_FP16 && storage_dtype != ERNIE_DTYPE_BF16)
        throw std::invalid_argument("invalid storage dtype");
    if (bin_path.empty()) throw std::invalid_argument("a weight file is required to load a text block");
    const MappedFile bin(bin_path);
    TextBlockFile f = inspect_text_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
    ernie_host_tensor t[9];
    for (int i = 0; i < 9; ++i) t[i] = {bin.data() + f.sections[i].data, f.sections[i].dtype};
    // Section order is the field order of ernie_text_block_host_tensors.
    const ernie_text_block_host_tensors w = {t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8]};
    check_status(ernie_hip_text_block_upload_tensors(device.ctx(), index, &w, f.graph.hidden, f.graph.heads,
                                                     f.graph.kv_heads, f.graph.ffn, storage_dtype),
                 device.ctx(), "text block upload");
    return f;
}

}  // namespace ernie
