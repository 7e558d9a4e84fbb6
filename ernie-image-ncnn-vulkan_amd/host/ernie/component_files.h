// SPDX-License-Identifier: MIT
// On-disk DiT heads (heads/input and heads/output head.ncnn.{param,bin}) and Mistral
// text blocks (text.ncnn.{param,bin}), read without ncnn and uploaded into the device
// context: the head and text-block halves of component_files / load_component
// (src/component_files.cpp:10-60) as src/dit.cpp:22-45 and src/text_encoder.cpp:30-40
// use them. Graph checks follow the reference's runtime shape contracts
// (src/shape_graph.cpp:23-31); the weight layout is ncnn's ModelBin as pnnx writes it
// (tools/export_dit_heads.py) and as tools/build_text_weights.py:52-74 packs it.
#pragma once
#include <string>
#include <vector>

#include "ernie/block_files.h"
#include "ernie_hip.h"

namespace ernie {

// ---- DiT heads ------------------------------------------------------------------------
enum class HeadKind { Input = ERNIE_HEAD_INPUT, Output = ERNIE_HEAD_OUTPUT };

struct HeadGraph {
    Graph graph;
    HeadKind kind = HeadKind::Input;
    int dim = 0, latent_ch = 0;
    int text_dim = 0, text_tokens = 0;  // input head: text_proj width and the graph's text slots
    int width = 0, height = 0;          // output head: the packed latent grid (0 for the input head)
    int image_tokens = 0, tokens = 0;   // image tokens; image + text tokens (output head)
    bool reviewed = false;              // matches the reviewed runtime contract hash
    std::string contract_sha256;        // the normalised graph's hash, "" when a field is missing
};

// Recognises a head graph: the input head (Convolution x_embedder, Gemm text_proj,
// InnerProduct time MLP and adaLN, outputs out0..out7) or the output head (InnerProduct
// shift/scale, non-affine LayerNorm, Gemm projection with a per-column bias, crop and
// reshape to [latent_ch][h][w]), with consistent shapes, plus the reference's runtime
// contract for "input" / "output" (src/shape_graph.cpp:27-31). An unreviewed topology is
// rejected unless `allow_unreviewed` (synthetic widths in tests). Throws std::invalid_argument.
HeadGraph inspect_head_graph(const std::string& text, bool allow_unreviewed);

// Walks a head's weight bytes in graph order: each weighted layer's weight as a tagged
// section, then its bias as raw FP32 (Convolution, InnerProduct: ncnn load types 0 and 1;
// Gemm: constant B tagged, its per-column C raw when 10=4). Input head: conv_1 w, b;
// gemm_0 w; linear_2 w, b; linear_3 w, b; linear_4 w, b. Output head: linear_2 w, b;
// gemm_0 w, b. Truncation and trailing bytes are rejected.
std::vector<WeightSection> head_sections(const HeadGraph& g, const unsigned char* bin, size_t size);

struct HeadFile {
    HeadGraph graph;
    std::vector<WeightSection> sections;  // empty when no weight file was read
    size_t bin_bytes = 0;
    std::string bin_sha256;               // set when a checksum was requested
};

// Reads and checks the files without a device; an empty bin_path checks the graph only.
HeadFile inspect_head_files(const std::string& param_path, const std::string& bin_path, bool allow_unreviewed,
                            const std::string& expected_bin_sha256 = "");

// A DiT head resident in the device context: the role the input_head / output_head
// ComponentFiles play in src/dit.h:17-40 and src/denoiser.h:13-17.
struct HeadModel {
    int part = 0;  // ERNIE_HEAD_INPUT or ERNIE_HEAD_OUTPUT; 0 = none
    bool empty() const { return part == 0; }
};

// inspect_head_files, then uploads the head's weights into the context at storage_dtype
// (biases stay FP32). The other head stays resident when its widths and dtype agree; the
// upload is rejected otherwise. `info` (nullable) receives the file record.
HeadModel load_head_files(const Device& device, const std::string& param_path, const std::string& bin_path,
                          int storage_dtype, bool allow_unreviewed, const std::string& expected_bin_sha256 = "",
                          HeadFile* info = nullptr);

// The head of kind `part` already resident in the context (uploaded through the C ABI);
// throws std::invalid_argument when it is not.
HeadModel resident_head(const Device& device, int part);

// ---- Mistral text blocks ---------------------------------------------------------------
struct TextBlockGraph {
    Graph graph;
    int tokens = 0, hidden = 0, heads = 0, kv_heads = 0, ffn = 0;
    bool reviewed = false;        // matches the reviewed runtime contract hash for "text"
    std::string contract_sha256;  // the normalised graph's hash, "" when a field is missing
};

// Recognises a text decoder block: rmsn_8, gemm_0..2 (q, k, v), gemm_3 (o), rmsn_9,
// gemm_4 (gate), gemm_5 (up), gemm_6 (down) in .bin order (tools/build_text_weights.py:15-25),
// head_dim 128, RMSNorm eps 1e-5, plus the runtime contract (src/shape_graph.cpp:25,31).
TextBlockGraph inspect_text_block_graph(const std::string& text, bool allow_unreviewed);

// RMSNorm gammas raw FP32, each Gemm a tagged section (tools/build_text_weights.py:60-74).
std::vector<WeightSection> text_block_sections(const TextBlockGraph& g, const unsigned char* bin, size_t size);

struct TextBlockFile {
    TextBlockGraph graph;
    std::vector<WeightSection> sections;
    size_t bin_bytes = 0;
    std::string bin_sha256;
};

TextBlockFile inspect_text_block_files(const std::string& param_path, const std::string& bin_path,
                                       bool allow_unreviewed, const std::string& expected_bin_sha256 = "");

// inspect_text_block_files, then uploads the weights into resident text block slot
// `index` (ernie_hip_text_block_upload_tensors).
TextBlockFile load_text_block_files(const Device& device, int index, const std::string& param_path,
                                    const std::string& bin_path, int storage_dtype, bool allow_unreviewed,
                                    const std::string& expected_bin_sha256 = "");

}  // namespace ernie
