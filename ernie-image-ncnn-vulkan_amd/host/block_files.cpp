// SPDX-License-Identifier: MIT
// Block graph + ModelBin reader (declared in ernie/block_files.h).
#include "ernie/block_files.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <stdexcept>

#include "ernie/sha256.h"
#include "ernie_hip.h"

namespace ernie {
namespace {

// Normalised-graph hashes of the two reviewed block topologies.
// tools/build_dit_weights.py:18 (component export, token fields -> TOKENS).
const char* const kComponentGraphSha256 = "88206e024759e4f8981fa1cb04636e644c3c7a3c7e08b2658a1f9bcce52ea50c";
// src/shape_graph.cpp:27, kind "dit" (runtime package, token fields -> TOTAL_TOKENS).
const char* const kRuntimeGraphSha256 = "51db4065837c28e235784fd0dd196f109ca86822143c025a44ee9372240e4132";

constexpr unsigned kTagFp32 = 0u, kTagBf16 = 0x01348B83u, kTagFp16 = 0x01306B47u;
constexpr size_t kMaxGraphBytes = 1024 * 1024;

// The weighted layers of one block in graph (and .bin) order: tools/build_dit_weights.py:19-31.
struct Weighted { const char* name; bool norm; };
const Weighted kWeighted[11] = {{"rmsn_8", true},  {"gemm_0", false}, {"gemm_1", false}, {"gemm_2", false},
                                {"rmsn_9", true},  {"rmsn_10", true}, {"gemm_3", false}, {"rmsn_11", true},
                                {"gemm_4", false}, {"gemm_5", false}, {"gemm_6", false}};

// Layer types of the block graph; none but RMSNorm and Gemm carries weights.
const std::set<std::string> kKnownTypes = {"Input",   "Split",  "RMSNorm", "BinaryOp",  "Gemm",
                                           "Reshape", "Permute", "Slice",  "Concat",    "SDPA",
                                           "ErnieGELU", "ErnieResidualAdd"};

[[noreturn]] void bad(const std::string& what) { throw std::invalid_argument(what); }

std::vector<std::string> split_fields(const std::string& line)
{
    std::vector<std::string> f;
    size_t i = 0;
    while (i < line.size()) {
        while (i < line.size() && std::isspace((unsigned char)line[i])) ++i;
        size_t j = i;
        while (j < line.size() && !std::isspace((unsigned char)line[j])) ++j;
        if (j > i) f.push_back(line.substr(i, j - i));
        i = j;
    }
    return f;
}

// Lines as Python's str.splitlines() yields them for '\n'-separated text.
std::vector<std::string> split_lines(const std::string& text)
{
    std::vector<std::string> lines;
    size_t start = 0;
    while (start < text.size()) {
        size_t nl = text.find('\n', start);
        if (nl == std::string::npos) nl = text.size();
        lines.push_back(text.substr(start, nl - start));
        start = nl + 1;
    }
    return lines;
}

std::string join(const std::vector<std::string>& f)
{
    std::string s;
    for (size_t i = 0; i < f.size(); ++i) {
        if (i) s += ' ';
        s += f[i];
    }
    return s;
}

long parse_int(const std::string& s, long lo, long hi, const std::string& what)
{
    if (s.empty()) bad("empty integer in " + what);
    char* end = nullptr;
    errno = 0;
    const long v = std::strtol(s.c_str(), &end, 10);
    if (errno || *end || v < lo || v > hi) bad("invalid integer '" + s + "' in " + what);
    return v;
}

std::string lower(std::string s)
{
    for (char& c : s) c = (char)std::tolower((unsigned char)c);
    return s;
}

// Component form (tools/build_dit_weights.py:34-50): in Gemm lines the field
// 7=<tokens>, in reshape_12..14 the field 2=<tokens>, in reshape_15 and
// unsqueeze_20/21 the field 1=<tokens> become <key>=TOKENS. Empty when a
// required field is missing.
std::string component_hash(const std::string& text, int tokens)
{
    const std::string t = std::to_string(tokens);
    std::string canon;
    for (const std::string& line : split_lines(text)) {
        std::vector<std::string> f = split_fields(line);
        const char* key = nullptr;
        if (!f.empty() && f[0] == "Gemm") key = "7";
        else if (f.size() > 1 && (f[1] == "reshape_12" || f[1] == "reshape_13" || f[1] == "reshape_14")) key = "2";
        else if (f.size() > 1 && (f[1] == "reshape_15" || f[1] == "unsqueeze_20" || f[1] == "unsqueeze_21")) key = "1";
        if (key) {
            const std::string target = std::string(key) + "=" + t;
            bool found = false;
            for (std::string& item : f)
                if (item == target) {
                    item = std::string(key) + "=TOKENS";
                    found = true;
                }
            if (!found) return "";
        }
        canon += join(f) + "\n";
    }
    return sha256_hex(canon.data(), canon.size());
}

// Runtime form (src/shape_graph.cpp:23-27,64-95, kind "dit"): the token field of the
// seven Gemms and six reshapes becomes TOTAL_TOKENS.
std::string runtime_hash(const std::string& text, int tokens)
{
    const std::string t = std::to_string(tokens);
    std::vector<ShapeField> fields;
    for (const char* node : {"gemm_0", "gemm_1", "gemm_2", "gemm_3", "gemm_4", "gemm_5", "gemm_6"})
        fields.push_back({node, "7", "TOTAL_TOKENS", t});
    for (const char* node : {"reshape_12", "reshape_13", "reshape_14"}) fields.push_back({node, "2", "TOTAL_TOKENS", t});
    for (const char* node : {"reshape_15", "unsqueeze_20", "unsqueeze_21"})
        fields.push_back({node, "1", "TOTAL_TOKENS", t});
    return shape_contract_sha256(text, fields);
}

}  // namespace

std::string shape_contract_sha256(const std::string& text, const std::vector<ShapeField>& fields)
{
    std::string canon;
    size_t seen = 0;
    for (const std::string& line : split_lines(text)) {
        std::vector<std::string> f = split_fields(line);
        if (f.size() > 1) {
            for (const ShapeField& field : fields) {
                if (f[1] != field.node) continue;
                if (f.size() < 6) return "";
                const size_t start = 4 + (size_t)std::atol(f[2].c_str()) + (size_t)std::atol(f[3].c_str());
                size_t index = 0, count = 0;
                for (size_t i = start; i < f.size(); ++i)
                    if (f[i].substr(0, f[i].find('=')) == field.key) {
                        index = i;
                        ++count;
                    }
                if (count != 1 || f[index] != std::string(field.key) + "=" + field.value) return "";
                f[index] = std::string(field.key) + "=" + field.name;
                ++seen;
            }
        }
        canon += join(f) + "\n";
    }
    if (seen != fields.size()) return "";
    return sha256_hex(canon.data(), canon.size());
}

const std::string* GraphLayer::param(const std::string& key) const
{
    for (const auto& kv : params)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

Graph parse_graph(const std::string& text)
{
    if (text.empty() || text.size() > kMaxGraphBytes) bad("graph text must contain 1..1048576 bytes");
    if (text.find('\0') != std::string::npos) bad("graph text contains NUL");
    const std::vector<std::string> lines = split_lines(text);
    size_t li = 0;
    auto next_fields = [&]() {
        while (li < lines.size()) {
            std::vector<std::string> f = split_fields(lines[li++]);
            if (!f.empty()) return f;
        }
        return std::vector<std::string>{};
    };
    std::vector<std::string> f = next_fields();
    if (f.size() != 1 || f[0] != "7767517") bad("graph text does not start with the ncnn magic 7767517");
    f = next_fields();
    if (f.size() != 2) bad("graph header must hold the layer and blob counts");
    Graph g;
    g.layer_count = (int)parse_int(f[0], 1, 1 << 20, "layer count");
    g.blob_count = (int)parse_int(f[1], 1, 1 << 20, "blob count");
    std::set<std::string> names, produced;
    for (f = next_fields(); !f.empty(); f = next_fields()) {
        if (f.size() < 4) bad("malformed layer line: " + join(f));
        GraphLayer l;
        l.type = f[0];
        l.name = f[1];
        const long n_in = parse_int(f[2], 0, 10000, "layer " + l.name);
        const long n_out = parse_int(f[3], 0, 10000, "layer " + l.name);
        if ((size_t)(4 + n_in + n_out) > f.size()) bad("missing blob names in layer " + l.name);
        if (!names.insert(l.name).second) bad("duplicate layer name " + l.name);
        for (long i = 0; i < n_in; ++i) {
            const std::string& b = f[4 + i];
            if (!produced.count(b)) bad("layer " + l.name + " reads blob " + b + " before it is produced");
            l.inputs.push_back(b);
        }
        for (long i = 0; i < n_out; ++i) {
            const std::string& b = f[4 + n_in + i];
            if (!produced.insert(b).second) bad("blob " + b + " is produced twice");
            l.outputs.push_back(b);
        }
        for (size_t i = 4 + n_in + n_out; i < f.size(); ++i) {
            const size_t eq = f[i].find('=');
            if (eq == std::string::npos || eq == 0) bad("malformed parameter '" + f[i] + "' in layer " + l.name);
            parse_int(f[i].substr(0, eq), -1000000, 1000000, "parameter key of layer " + l.name);
            l.params.emplace_back(f[i].substr(0, eq), f[i].substr(eq + 1));
        }
        g.layers.push_back(std::move(l));
    }
    if ((int)g.layers.size() != g.layer_count) bad("graph declares " + std::to_string(g.layer_count) +
                                                   " layers but holds " + std::to_string(g.layers.size()));
    if ((int)produced.size() != g.blob_count) bad("graph declares " + std::to_string(g.blob_count) +
                                                  " blobs but produces " + std::to_string(produced.size()));
    return g;
}

BlockGraph inspect_block_graph(const std::string& text, bool allow_unreviewed)
{
    BlockGraph bg;
    bg.graph = parse_graph(text);
    const Graph& g = bg.graph;
    std::vector<const GraphLayer*> weighted;
    std::set<std::string> inputs;
    bool has_out0 = false;
    for (const GraphLayer& l : g.layers) {
        if (!kKnownTypes.count(l.type)) bad("layer " + l.name + " has a type outside the DiT block: " + l.type);
        if (l.type == "RMSNorm" || l.type == "Gemm") weighted.push_back(&l);
        if (l.type == "Input") inputs.insert(l.name);
        for (const std::string& o : l.outputs) has_out0 |= o == "out0";
    }
    for (int i = 0; i <= 9; ++i)
        if (!inputs.count("in" + std::to_string(i))) bad("block graph lacks input in" + std::to_string(i));
    if (inputs.size() != 10 || !has_out0) bad("block graph must have inputs in0..in9 and output out0");
    if (weighted.size() != 11) bad("block graph must hold 4 RMSNorm and 7 Gemm layers");
    auto int_param = [](const GraphLayer& l, const char* key, long dflt) {
        const std::string* v = l.param(key);
        return v ? parse_int(*v, -1000000000L, 1000000000L, "parameter " + std::string(key) + " of " + l.name) : dflt;
    };
    long tokens = -1;
    std::vector<long> count(11), n(11), k(11);
    for (int i = 0; i < 11; ++i) {
        const GraphLayer& l = *weighted[i];
        if (l.name != kWeighted[i].name || (l.type == "RMSNorm") != kWeighted[i].norm)
            bad("weighted layer " + std::to_string(i) + " is " + l.type + " " + l.name + ", expected " +
                kWeighted[i].name);
        if (kWeighted[i].norm) {
            // ErnieRMSNorm: affine, eps 1e-6 (src/ernie_rmsnorm.cpp:21-35).
            count[i] = int_param(l, "0", 0);
            const std::string* eps = l.param("1");
            if (count[i] < 1 || int_param(l, "2", 0) != 1) bad(l.name + " must be an affine RMSNorm");
            if (!eps || (float)std::strtod(eps->c_str(), nullptr) != 1e-6f) bad(l.name + " must use eps 1e-6");
        } else {
            // Constant-B, bias-free A.B^T (tools/pack_block_weights.py:44-47).
            if (int_param(l, "2", 0) != 0 || int_param(l, "3", 0) != 1 || int_param(l, "4", 0) != 0 ||
                int_param(l, "5", 0) != 1 || int_param(l, "10", 0) != -1 || int_param(l, "18", 0) != 0 ||
                int_param(l, "14", 0) != 0)
                bad(l.name + " is not the bias-free constant-B Gemm A.B^T");
            const std::string* alpha = l.param("0");
            if (alpha && std::strtod(alpha->c_str(), nullptr) != 1.0) bad(l.name + " must have alpha 1");
            const long t = int_param(l, "7", 0);
            if (t < 1 || (tokens >= 0 && t != tokens)) bad("Gemm token counts differ or are missing");
            tokens = t;
            n[i] = int_param(l, "8", 0);
            k[i] = int_param(l, "9", 0);
            if (n[i] < 1 || k[i] < 1) bad(l.name + " lacks its weight shape");
        }
    }
    const long dim = count[0], ffn = n[8];
    const bool shapes = n[1] == dim && k[1] == dim && n[2] == dim && k[2] == dim && n[3] == dim && k[3] == dim &&
                        count[4] == 128 && count[5] == 128 && n[6] == dim && k[6] == dim && count[7] == dim &&
                        k[8] == dim && n[9] == ffn && k[9] == dim && n[10] == dim && k[10] == ffn;
    if (!shapes) bad("block weight shapes are inconsistent (head_dim must be 128)");
    if (dim > 1 << 20 || ffn > 1 << 20) bad("block width out of range");
    bg.tokens = (int)tokens;
    bg.dim = (int)dim;
    bg.ffn = (int)ffn;
    bg.component_sha256 = component_hash(text, bg.tokens);
    bg.runtime_sha256 = runtime_hash(text, bg.tokens);
    if (bg.component_sha256 == kComponentGraphSha256) bg.contract = GraphContract::Component;
    else if (bg.runtime_sha256 == kRuntimeGraphSha256) bg.contract = GraphContract::Runtime;
    if (bg.contract == GraphContract::Unreviewed && !allow_unreviewed)
        bad("graph differs from the reviewed ERNIE block topology (normalised sha256 " +
            (bg.component_sha256.empty() ? std::string("n/a") : bg.component_sha256) + " / " +
            (bg.runtime_sha256.empty() ? std::string("n/a") : bg.runtime_sha256) + ")");
    return bg;
}

WeightSection tagged_section(const std::string& layer, const unsigned char* bin, size_t size, size_t offset,
                             size_t count)
{
    WeightSection s;
    s.layer = layer;
    s.count = count;
    s.begin = offset;
    if (offset > size || size - offset < 4) bad("weight file ends inside the tag of " + layer);
    const unsigned tag = (unsigned)bin[offset] | (unsigned)bin[offset + 1] << 8 | (unsigned)bin[offset + 2] << 16 |
                         (unsigned)bin[offset + 3] << 24;
    s.data = offset + 4;
    if (tag == kTagFp32) {
        s.dtype = ERNIE_DTYPE_FP32;
        s.end = s.data + 4 * count;
    } else if (tag == kTagBf16 || tag == kTagFp16) {
        s.dtype = tag == kTagBf16 ? ERNIE_DTYPE_BF16 : ERNIE_DTYPE_FP16;
        s.end = s.data + (2 * count + 3) / 4 * 4;
    } else {
        char buf[96];
        std::snprintf(buf, sizeof(buf), "unsupported ModelBin storage tag 0x%08x in %s", tag, layer.c_str());
        bad(buf);
    }
    if (s.end > size) bad("weight file is truncated inside " + layer);
    return s;
}

WeightSection raw_section(const std::string& layer, size_t size, size_t offset, size_t count)
{
    WeightSection s;
    s.layer = layer;
    s.count = count;
    s.dtype = ERNIE_DTYPE_FP32;
    s.begin = s.data = offset;
    s.end = offset + 4 * count;
    if (offset > size || s.end > size) bad("weight file is truncated inside " + layer);
    return s;
}

void check_sections_end(const std::vector<WeightSection>& sections, size_t size)
{
    const size_t off = sections.empty() ? 0 : sections.back().end;
    if (off != size) bad("weight file holds " + std::to_string(size - off) + " bytes beyond the component's sections");
}

void check_bin_sha256(const unsigned char* bin, size_t size, const std::string& expected, std::string* digest)
{
    if (expected.empty()) return;
    const std::string got = sha256_hex(bin, size);
    if (digest) *digest = got;
    if (got != lower(expected)) bad("weight file checksum mismatch: " + got);
}

std::vector<WeightSection> block_sections(const BlockGraph& g, const unsigned char* bin, size_t size)
{
    std::vector<WeightSection> out;
    size_t off = 0;
    for (const GraphLayer& l : g.graph.layers) {
        if (l.type != "RMSNorm" && l.type != "Gemm") continue;
        if (l.type == "RMSNorm")
            out.push_back(raw_section(l.name, size, off, (size_t)std::atol(l.param("0")->c_str())));
        else
            out.push_back(tagged_section(l.name, bin, size, off,
                                         (size_t)std::atol(l.param("8")->c_str()) *
                                             (size_t)std::atol(l.param("9")->c_str())));
        off = out.back().end;
    }
    check_sections_end(out, size);
    return out;
}

std::string read_graph_text(const std::string& param_path)
{
    std::ifstream in(param_path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("cannot open graph file " + param_path);
    const std::streamoff size = in.tellg();
    if (size <= 0 || (size_t)size > kMaxGraphBytes) bad("graph text must contain 1..1048576 bytes");
    std::string text((size_t)size, '\0');
    in.seekg(0);
    if (!in.read(&text[0], size)) throw std::runtime_error("cannot read the complete graph text");
    if (text.find('\0') != std::string::npos) bad("graph text contains NUL");
    return text;
}

MappedFile::MappedFile(const std::string& path)
{
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw std::runtime_error("cannot open weight file " + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        throw std::runtime_error("weight file is not a regular file: " + path);
    }
    size_ = (size_t)st.st_size;
    if (!size_) {
        ::close(fd);
        bad("empty weight file: " + path);
    }
    void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw std::runtime_error("cannot map weight file " + path + ": " + std::strerror(errno));
    (void)::madvise(p, size_, MADV_SEQUENTIAL);
    data_ = static_cast<const unsigned char*>(p);
}

MappedFile::~MappedFile()
{
    if (data_) ::munmap(const_cast<unsigned char*>(data_), size_);
}

BlockFile inspect_block_bytes(const std::string& param_path, const unsigned char* bin, size_t size,
                              bool allow_unreviewed, const std::string& expected_bin_sha256)
{
    BlockFile f;
    f.graph = inspect_block_graph(read_graph_text(param_path), allow_unreviewed);
    if (!bin) {
        if (!expected_bin_sha256.empty()) bad("a weight checksum was given without a weight file");
        return f;
    }
    f.bin_bytes = size;
    check_bin_sha256(bin, size, expected_bin_sha256, &f.bin_sha256);
    f.sections = block_sections(f.graph, bin, size);
    return f;
}

BlockFile inspect_block_files(const std::string& param_path, const std::string& bin_path, bool allow_unreviewed,
                              const std::string& expected_bin_sha256)
{
    if (bin_path.empty()) return inspect_block_bytes(param_path, nullptr, 0, allow_unreviewed, expected_bin_sha256);
    const MappedFile bin(bin_path);
    return inspect_block_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
}

}  // namespace ernie
