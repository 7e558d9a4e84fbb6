// SPDX-License-Identifier: MIT
// On-disk DiT block: the ncnn graph text (block.ncnn.param) and its ModelBin
// weights (block.ncnn.bin), read without ncnn and uploaded into a resident
// block slot. Replaces component_files/load_component (src/component_files.cpp:10-60)
// for the block path; the weight layout is the one tools/build_dit_weights.py:88-121
// and tools/pack_block_weights.py:26-69 write.
#pragma once
#include <cstddef>
#include <string>
#include <utility>
#include <vector>

namespace ernie {

class Device;

// One layer line of an ncnn .param graph: "Type name n_in n_out inputs.. outputs.. key=value..".
struct GraphLayer {
    std::string type, name;
    std::vector<std::string> inputs, outputs;
    std::vector<std::pair<std::string, std::string>> params;
    // Value of `key`, or nullptr when the layer does not set it.
    const std::string* param(const std::string& key) const;
};

struct Graph {
    int layer_count = 0, blob_count = 0;
    std::vector<GraphLayer> layers;
};

// Parses an ncnn .param text (magic 7767517, "layers blobs", one layer per line)
// and checks its structure: counts, unique layer names, each blob produced once
// and consumed only after it is produced. Throws std::invalid_argument.
Graph parse_graph(const std::string& text);

// One field of the reference's runtime shape contract (src/shape_graph.cpp:23-31): in
// the layer named `node`, the one parameter with key `key` must read key=value (this
// graph's dimension) and becomes key=name (the dimension's upper-case name) in the
// normalised text.
struct ShapeField {
    const char* node;
    const char* key;
    const char* name;
    std::string value;
};
// SHA-256 of the graph text normalised by `fields` as src/shape_graph.cpp:52-95 does
// (whitespace-separated fields joined by one space, one '\n' per line), or "" when a
// field is missing, repeated or holds another value. A node may carry several fields.
std::string shape_contract_sha256(const std::string& text, const std::vector<ShapeField>& fields);

// Which reviewed topology a block graph matches once its token count is
// normalised: the component export checked by tools/build_dit_weights.py:18,34-50
// (BinaryOp residual adds) or the runtime package checked by
// src/shape_graph.cpp:23-27,37-95 (ErnieResidualAdd).
enum class GraphContract { Unreviewed = 0, Component = 1, Runtime = 2 };

struct BlockGraph {
    Graph graph;
    int tokens = 0, dim = 0, ffn = 0;
    GraphContract contract = GraphContract::Unreviewed;
    std::string component_sha256, runtime_sha256;  // hashes of the two normalised forms
};

// Recognises the DiT block in a graph: the eleven weighted layers in .bin order
// (tools/build_dit_weights.py:19-31) with their shapes and the bias-free,
// constant-B Gemm form, plus the topology contract. An unreviewed topology is
// rejected unless `allow_unreviewed` (synthetic widths in tests).
BlockGraph inspect_block_graph(const std::string& text, bool allow_unreviewed);

// One ModelBin section, in bytes from the start of the weight file.
struct WeightSection {
    std::string layer;
    int dtype = 0;        // ERNIE_DTYPE_FP32 / FP16 / BF16 of the stored elements
    size_t count = 0;     // elements
    size_t begin = 0;     // first byte of the section (the tag, for a Gemm)
    size_t data = 0;      // first element
    size_t end = 0;       // one past the section, padding included
};

// A ModelBin section read with load type 0 (ncnn's tagged form: Gemm, InnerProduct and
// Convolution weights): a 4-byte tag, 0 = FP32, 0x01348B83 = BF16 or 0x01306B47 = FP16
// (halves padded to 4 bytes), then `count` elements, starting at byte `offset`. Other tags
// (quantized sections) and truncation throw std::invalid_argument.
WeightSection tagged_section(const std::string& layer, const unsigned char* bin, size_t size, size_t offset,
                             size_t count);
// A section read with load type 1: `count` raw FP32 values (RMSNorm gammas, biases).
WeightSection raw_section(const std::string& layer, size_t size, size_t offset, size_t count);
// Throws unless the last section ends exactly at `size` (no trailing bytes).
void check_sections_end(const std::vector<WeightSection>& sections, size_t size);
// Compares the SHA-256 of the bytes with a non-empty `expected` (hex, any case) and
// throws std::invalid_argument on a mismatch; `digest` (nullable) receives the hash.
void check_bin_sha256(const unsigned char* bin, size_t size, const std::string& expected, std::string* digest);

// Walks a block's weight bytes in graph order. RMSNorm gammas are raw FP32;
// each Gemm section starts with a 4-byte tag: 0 = FP32, 0x01348B83 = BF16 and
// 0x01306B47 = FP16 (halves padded to 4 bytes). Other tags (quantized
// sections), truncation and trailing bytes are rejected.
std::vector<WeightSection> block_sections(const BlockGraph& g, const unsigned char* bin, size_t size);

struct BlockFile {
    BlockGraph graph;
    std::vector<WeightSection> sections;  // empty when no weight file was read
    size_t bin_bytes = 0;
    std::string bin_sha256;               // set when a checksum was requested
};

// Read-only memory mapping of a weight file (a regular, non-empty file).
class MappedFile {
public:
    explicit MappedFile(const std::string& path);
    ~MappedFile();
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    const unsigned char* data() const { return data_; }
    size_t size() const { return size_; }

private:
    const unsigned char* data_ = nullptr;
    size_t size_ = 0;
};

// Graph text of at most 1 MiB without NUL bytes (src/component_files.cpp:14-23).
std::string read_graph_text(const std::string& param_path);

// Reads and checks the files without a device; an empty bin_path checks the graph only.
BlockFile inspect_block_files(const std::string& param_path, const std::string& bin_path, bool allow_unreviewed,
                              const std::string& expected_bin_sha256 = "");

// inspect_block_files over weight bytes already in memory; a null `bin` checks the graph only.
BlockFile inspect_block_bytes(const std::string& param_path, const unsigned char* bin, size_t size,
                              bool allow_unreviewed, const std::string& expected_bin_sha256 = "");

// inspect_block_files, then uploads the weights into resident block slot
// `index` at `storage_dtype` (gammas stay FP32). The weight file is memory
// mapped and converted on the device. A non-empty expected_bin_sha256 is
// compared with the file's SHA-256 before anything is uploaded.
BlockFile load_block_files(const Device& device, int index, const std::string& param_path,
                           const std::string& bin_path, int storage_dtype, bool allow_unreviewed,
                           const std::string& expected_bin_sha256 = "");

}  // namespace ernie
