// SPDX-License-Identifier: MIT
// Deterministic fuzz driver for the host-side parsers and helpers that take caller
// data: the ncnn .param graph checks (DiT blocks, DiT heads, text blocks), the ModelBin
// section walks, the file readers, SHA-256 and the text padding / RoPE-table helpers. Built by
// tests/test_host_sanitizers.py with AddressSanitizer and UndefinedBehaviorSanitizer
// on the CPU; every input either passes the checks or is rejected with a C++
// exception, and the sanitizers abort the run on any memory or UB error.
//
// usage: host_fuzz <golden dir> <scratch dir> <iterations> <seed>
#include <sys/stat.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "ernie/block_files.h"
#include "ernie/component_files.h"
#include "ernie/conditioning.h"
#include "ernie/latent_ops.h"
#include "ernie/sha256.h"

namespace {

struct Rng {
    uint64_t s;
    uint64_t next()
    {
        s += 0x9e3779b97f4a7c15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    size_t below(size_t n) { return n ? (size_t)(next() % n) : 0; }
};

std::string read_file(const std::string& path)
{
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot read " + path);
    std::stringstream ss;
    ss << in.rdbuf();
    return ss.str();
}

void write_file(const std::string& path, const std::string& bytes)
{
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    out.write(bytes.data(), (std::streamsize)bytes.size());
}

std::vector<std::string> tokens_of(const std::string& line)
{
    std::vector<std::string> f;
    std::istringstream in(line);
    std::string t;
    while (in >> t) f.push_back(t);
    return f;
}

// The reviewed component graph with its widths replaced (an unreviewed topology the
// parser accepts when asked to), as the Python tests build it.
std::string synthetic_graph(const std::string& component, int dim, int ffn, int tokens)
{
    std::istringstream in(component);
    std::string line, out;
    while (std::getline(in, line)) {
        std::vector<std::string> f = tokens_of(line);
        if (f.size() > 1 && (f[1].rfind("gemm_", 0) == 0 || f[1].rfind("rmsn_", 0) == 0 ||
                             f[1].rfind("reshape_", 0) == 0 || f[1].rfind("unsqueeze_", 0) == 0)) {
            for (std::string& x : f) {
                if (x == "7=288" || x == "2=288" || x == "1=288") x = x.substr(0, 2) + std::to_string(tokens);
                else if (x == "8=4096" || x == "9=4096" || x == "0=4096") x = x.substr(0, 2) + std::to_string(dim);
                else if (x == "8=12288" || x == "9=12288") x = x.substr(0, 2) + std::to_string(ffn);
                else if (x == "1=32") x = "1=" + std::to_string(dim / 128);
            }
        }
        for (size_t i = 0; i < f.size(); ++i) out += (i ? " " : "") + f[i];
        out += "\n";
    }
    return out;
}

// A well-formed weight file for `g`: gammas as FP32, each Gemm with a random tag.
std::string weight_bytes(const ernie::BlockGraph& g, Rng& rng)
{
    std::string bin;
    auto put32 = [&](uint32_t v) { bin.append(reinterpret_cast<const char*>(&v), 4); };
    for (const ernie::GraphLayer& l : g.graph.layers) {
        if (l.type == "RMSNorm") {
            const long n = std::atol(l.param("0")->c_str());
            for (long i = 0; i < n; ++i) put32(0x3f800000u);
        } else if (l.type == "Gemm") {
            const size_t n = (size_t)std::atol(l.param("8")->c_str()) * (size_t)std::atol(l.param("9")->c_str());
            const int kind = (int)rng.below(3);
            if (kind == 0) {
                put32(0);
                bin.append(4 * n, '\0');
            } else {
                put32(kind == 1 ? 0x01348B83u : 0x01306B47u);
                bin.append((2 * n + 3) / 4 * 4, '\0');
            }
        }
    }
    return bin;
}

// A reference graph with every parameter value found in `values` replaced (lines whose
// layer name is in `only`, or every line when `only` is empty).
std::string rewrite_values(const std::string& graph, const std::vector<std::pair<std::string, std::string>>& values,
                           const std::vector<std::string>& only = {})
{
    std::istringstream in(graph);
    std::string line, out;
    while (std::getline(in, line)) {
        std::vector<std::string> f = tokens_of(line);
        bool pick = only.empty();
        for (const std::string& n : only) pick |= f.size() > 1 && f[1] == n;
        if (pick)
            for (size_t i = 4; i < f.size(); ++i) {
                const size_t eq = f[i].find('=');
                if (eq == std::string::npos) continue;
                for (const auto& kv : values)
                    if (f[i].substr(eq + 1) == kv.first) {
                        f[i] = f[i].substr(0, eq + 1) + kv.second;
                        break;
                    }
            }
        for (size_t i = 0; i < f.size(); ++i) out += (i ? " " : "") + f[i];
        out += "\n";
    }
    return out;
}

// Weight bytes for a list of (elements, tagged) sections: tagged ones get a random tag.
std::string section_bytes(const std::vector<std::pair<size_t, bool>>& sections, Rng& rng)
{
    std::string bin;
    auto put32 = [&](uint32_t v) { bin.append(reinterpret_cast<const char*>(&v), 4); };
    for (const auto& sec : sections) {
        if (!sec.second) {
            bin.append(4 * sec.first, '\0');
            continue;
        }
        const int kind = (int)rng.below(3);
        put32(kind == 0 ? 0u : kind == 1 ? 0x01348B83u : 0x01306B47u);
        bin.append(kind == 0 ? 4 * sec.first : (2 * sec.first + 3) / 4 * 4, '\0');
    }
    return bin;
}

std::vector<std::pair<size_t, bool>> head_layout(const ernie::HeadGraph& h)
{
    const size_t D = h.dim;
    if (h.kind == ernie::HeadKind::Input)
        return {{D * h.latent_ch, true}, {D, false}, {D * h.text_dim, true}, {D * D, true}, {D, false},
                {D * D, true}, {D, false}, {6 * D * D, true}, {6 * D, false}};
    return {{2 * D * D, true}, {2 * D, false}, {(size_t)h.latent_ch * D, true}, {(size_t)h.latent_ch, false}};
}

std::vector<std::pair<size_t, bool>> text_layout(const ernie::TextBlockGraph& t)
{
    const size_t H = t.hidden, Q = 128 * (size_t)t.heads, KV = 128 * (size_t)t.kv_heads, F = t.ffn;
    return {{H, false}, {Q * H, true}, {KV * H, true}, {KV * H, true}, {H * Q, true},
            {H, false}, {F * H, true}, {F * H, true}, {H * F, true}};
}

const char* const kNumbers[] = {"0", "-1", "1", "7", "128", "4096", "2147483647", "-2147483648",
                                "99999999999999999999", "1e30", "nan", "0x10", "", "=", "12288"};

std::string mutate_text(const std::string& base, Rng& rng)
{
    std::string s = base;
    const int edits = 1 + (int)rng.below(4);
    for (int e = 0; e < edits && !s.empty(); ++e) {
        const size_t pos = rng.below(s.size());
        switch (rng.below(8)) {
        case 0: s[pos] = (char)(rng.next() & 0xff); break;                     // random byte
        case 1: s.erase(pos, 1 + rng.below(16)); break;                          // deletion
        case 2: s.insert(pos, kNumbers[rng.below(15)]); break;                   // inserted number
        case 3: s.resize(pos); break;                                            // truncation
        case 4: {                                                                // duplicated line
            const size_t a = s.rfind('\n', pos), b = s.find('\n', pos);
            if (a != std::string::npos && b != std::string::npos) s.insert(b, s.substr(a, b - a));
            break;
        }
        case 5: {                                                                // numeric value replaced
            const size_t eq = s.find('=', pos);
            if (eq != std::string::npos) {
                size_t end = eq + 1;
                while (end < s.size() && s[end] != ' ' && s[end] != '\n') ++end;
                s.replace(eq + 1, end - eq - 1, kNumbers[rng.below(15)]);
            }
            break;
        }
        case 6: s.insert(pos, 1, ' '); break;
        default: {                                                               // swapped lines
            const size_t a = s.find('\n', pos);
            const size_t b = a == std::string::npos ? a : s.find('\n', a + 1);
            const size_t c = b == std::string::npos ? b : s.find('\n', b + 1);
            if (c != std::string::npos) {
                const std::string l1 = s.substr(a + 1, b - a), l2 = s.substr(b + 1, c - b);
                s.replace(a + 1, c - a, l2 + l1);
            }
            break;
        }
        }
    }
    return s;
}

std::string mutate_bytes(const std::string& base, Rng& rng)
{
    std::string s = base;
    switch (rng.below(5)) {
    case 0:
        for (int i = 0; i < 4 && !s.empty(); ++i) s[rng.below(s.size())] = (char)(rng.next() & 0xff);
        break;
    case 1: s.resize(rng.below(s.size() + 1)); break;
    case 2: s.append(1 + rng.below(64), (char)(rng.next() & 0xff)); break;
    case 3:
        if (s.size() >= 4) {  // overwrite an aligned word with a tag-like value
            const size_t at = rng.below(s.size() / 4) * 4;
            const uint32_t tags[] = {0u, 0x01348B83u, 0x01306B47u, 0x000D4B38u, 0xffffffffu};
            const uint32_t v = tags[rng.below(5)];
            s.replace(at, 4, reinterpret_cast<const char*>(&v), 4);
        }
        break;
    default: s.clear(); break;
    }
    return s;
}

long g_accepted = 0, g_rejected = 0;

template <typename F>
void expect_clean(F&& f)
{
    try {
        f();
        ++g_accepted;
    } catch (const std::exception&) {
        ++g_rejected;
    }
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <golden dir> <scratch dir> <iterations> <seed>\n", argv[0]);
        return 2;
    }
    const std::string golden = argv[1], scratch = argv[2];
    const long iters = std::atol(argv[3]);
    Rng rng{(uint64_t)std::strtoull(argv[4], nullptr, 10)};
    const std::string component = read_file(golden + "/block_component_s288.ncnn.param");
    const std::string runtime = read_file(golden + "/block_runtime_s4160.ncnn.param");

    // The fixtures themselves pass.
    const ernie::BlockGraph comp = ernie::inspect_block_graph(component, false);
    const ernie::BlockGraph rt = ernie::inspect_block_graph(runtime, false);
    if (comp.contract != ernie::GraphContract::Component || rt.contract != ernie::GraphContract::Runtime) {
        std::fprintf(stderr, "reference graphs not recognised\n");
        return 1;
    }
    const std::string small = synthetic_graph(component, 256, 512, 40);
    const ernie::BlockGraph small_g = ernie::inspect_block_graph(small, true);

    // The reference's head and text graphs pass; narrow copies give small weight files.
    std::vector<std::string> heads;
    for (const char* name : {"head_input_s288", "head_input_s4160", "head_output_s288", "head_output_s4160"}) {
        heads.push_back(read_file(golden + "/" + name + ".ncnn.param"));
        if (!ernie::inspect_head_graph(heads.back(), false).reviewed) {
            std::fprintf(stderr, "reference head graph %s not recognised\n", name);
            return 1;
        }
    }
    const std::string text64 = read_file(golden + "/text_s64.ncnn.param");
    if (!ernie::inspect_text_block_graph(text64, false).reviewed) {
        std::fprintf(stderr, "reference text graph not recognised\n");
        return 1;
    }
    const std::vector<std::pair<std::string, std::string>> narrow_head = {
        {"4096", "256"}, {"524288", "8192"}, {"3072", "64"}, {"16777216", "65536"}, {"24576", "1536"},
        {"100663296", "393216"}, {"8192", "512"}, {"33554432", "131072"}};
    const std::string small_in = rewrite_values(heads[0], narrow_head);
    const std::string small_out = rewrite_values(heads[2], narrow_head);
    const ernie::HeadGraph small_in_g = ernie::inspect_head_graph(small_in, true);
    const ernie::HeadGraph small_out_g = ernie::inspect_head_graph(small_out, true);
    const std::string small_text = rewrite_values(
        rewrite_values(text64, {{"3072", "256"}, {"4096", "512"}, {"1024", "256"}, {"9216", "512"}}),
        {{"32", "4"}, {"8", "2"}}, {"reshape_10", "reshape_11", "reshape_12"});
    const ernie::TextBlockGraph small_text_g = ernie::inspect_text_block_graph(small_text, true);

    for (long it = 0; it < iters; ++it) {
        // 1. Graph text: parse and inspect mutated graphs, with and without the contract.
        const std::string& base = (it % 3 == 0) ? runtime : (it % 3 == 1 ? component : small);
        const std::string text = mutate_text(base, rng);
        expect_clean([&] { ernie::parse_graph(text); });
        expect_clean([&] { ernie::inspect_block_graph(text, (it & 1) != 0); });

        // 2. Section walk over mutated weight bytes of the small synthetic block.
        std::string bin = weight_bytes(small_g, rng);
        if (it % 4) bin = mutate_bytes(bin, rng);
        expect_clean([&] {
            const std::vector<ernie::WeightSection> secs =
                ernie::block_sections(small_g, reinterpret_cast<const unsigned char*>(bin.data()), bin.size());
            for (const ernie::WeightSection& s : secs)
                if (s.end > bin.size() || s.data < s.begin || s.end < s.data) throw std::logic_error("bad section");
        });

        // 2b. Head and text block graphs and section walks.
        {
            const std::string& hbase = (it % 5 < 4) ? heads[it % 4] : (it & 1 ? small_in : small_out);
            const std::string htext = mutate_text(hbase, rng);
            expect_clean([&] { ernie::inspect_head_graph(htext, (it & 2) != 0); });
            const std::string ttext = mutate_text(it & 1 ? text64 : small_text, rng);
            expect_clean([&] { ernie::inspect_text_block_graph(ttext, (it & 2) != 0); });
            const ernie::HeadGraph& hg = (it & 1) ? small_in_g : small_out_g;
            std::string hbin = section_bytes(head_layout(hg), rng);
            if (it % 3) hbin = mutate_bytes(hbin, rng);
            expect_clean([&] {
                for (const ernie::WeightSection& sec :
                     ernie::head_sections(hg, reinterpret_cast<const unsigned char*>(hbin.data()), hbin.size()))
                    if (sec.end > hbin.size() || sec.data < sec.begin || sec.end < sec.data)
                        throw std::logic_error("bad head section");
            });
            std::string tbin = section_bytes(text_layout(small_text_g), rng);
            if (it % 3) tbin = mutate_bytes(tbin, rng);
            expect_clean([&] {
                for (const ernie::WeightSection& sec : ernie::text_block_sections(
                         small_text_g, reinterpret_cast<const unsigned char*>(tbin.data()), tbin.size()))
                    if (sec.end > tbin.size() || sec.data < sec.begin || sec.end < sec.data)
                        throw std::logic_error("bad text section");
            });
        }

        // 3. The file readers on mutated files (every 16th iteration: file system work).
        if (it % 16 == 0) {
            const std::string gp = scratch + "/g.param", bp = scratch + "/w.bin";
            write_file(gp, (it % 32 == 0) ? mutate_text(small, rng) : small);
            write_file(bp, mutate_bytes(weight_bytes(small_g, rng), rng));
            expect_clean([&] { ernie::inspect_block_files(gp, bp, true); });
            expect_clean([&] { ernie::inspect_block_files(gp, "", true, "00"); });
            expect_clean([&] { ernie::inspect_block_files(gp, bp, true, std::string(64, 'a')); });
            expect_clean([&] { ernie::inspect_block_files(scratch, bp, true); });   // a directory
            expect_clean([&] { ernie::inspect_block_files(gp, scratch, true); });   // a directory
            expect_clean([&] { ernie::read_graph_text(scratch + "/missing"); });
            write_file(gp, (it % 32 == 0) ? mutate_text(small_in, rng) : small_in);
            write_file(bp, mutate_bytes(section_bytes(head_layout(small_in_g), rng), rng));
            expect_clean([&] { ernie::inspect_head_files(gp, bp, true); });
            expect_clean([&] { ernie::inspect_head_files(gp, bp, true, std::string(64, 'b')); });
            write_file(gp, (it % 32 == 0) ? mutate_text(small_text, rng) : small_text);
            write_file(bp, mutate_bytes(section_bytes(text_layout(small_text_g), rng), rng));
            expect_clean([&] { ernie::inspect_text_block_files(gp, bp, true); });
        }

        // 4. SHA-256: one-shot against random split points.
        {
            std::string data(rng.below(300), '\0');
            for (char& c : data) c = (char)(rng.next() & 0xff);
            ernie::Sha256 h;
            size_t at = 0;
            while (at < data.size()) {
                const size_t n = 1 + rng.below(data.size() - at);
                h.update(data.data() + at, n);
                at += n;
            }
            if (h.finish_hex() != ernie::sha256_hex(data.data(), data.size())) {
                std::fprintf(stderr, "sha256 split mismatch at iteration %ld\n", it);
                return 1;
            }
        }

        // 5. Helpers with arbitrary arguments.
        const int tokens = (int)rng.below(70) - 3, bucket = (int)rng.below(70) - 3;
        std::vector<float> emb(rng.below(4) ? (size_t)std::max(tokens, 0) * 3072 : rng.below(5000));
        expect_clean([&] {
            const std::vector<float> out = ernie::pad_text(emb, tokens, bucket);
            if (out.size() != (size_t)bucket * 3072) throw std::logic_error("pad_text size");
        });
        std::vector<float> freqs = ernie::rope_frequencies();
        if (rng.below(4) == 0) freqs.resize(rng.below(80));
        if (rng.below(8) == 0 && !freqs.empty()) freqs[rng.below(freqs.size())] = -1.f;
        const int w = (int)rng.below(40) - 2, hh = (int)rng.below(40) - 2;
        const int valid = (int)rng.below(80) - 2, text_bucket = (int)rng.below(80) - 2;
        expect_clean([&] {
            const ernie::DitConstantsHost k = ernie::dit_constants(freqs, w, hh, valid, text_bucket, 4096);
            if (k.cos.size() != (size_t)k.length * 128 || k.mask.size() != (size_t)k.length)
                throw std::logic_error("constant sizes");
        });
        expect_clean([&] { ernie::FlowSchedule::turbo((int)rng.below(40) - 4); });
    }
    std::printf("host_fuzz: %ld iterations, %ld accepted, %ld rejected\n", iters, g_accepted, g_rejected);
    return 0;
}
