// SPDX-License-Identifier: MIT
// ernie-denoise-runner: the turbo denoise from the DiT's component files on the MI355X
// path, with the command line, inputs, outputs and progress lines of the reference's
// denoise probe (probes/denoise_runner.cpp:42-238).
//
//   --model DIR (1..36 times)   block.ncnn.param + block.ncnn.bin, in block order
//   --input-head DIR, --output-head DIR   head.ncnn.param + head.ncnn.bin
//   --fixture DIR    in0.f32 latent [128][height][width], in1.f32 text [text][3072],
//                    in3/in4.f32 cos/sin [tokens][128], in5.f32 mask [tokens][tokens]
//   --width W --height H --text-tokens T   packed latent grid and text slots
//   --steps N        turbo schedule length (default 8)
//   --output DIR     a new directory: final.f32, and with --trace prediction-i.f32,
//                    step-i.f32 and features-i.f32 for every step
//   --backend hip|vulkan, --precision fp32|fp16|bf16   as ernie-block-runner
//   --timestep T     only write features.f32 = timestep_features(T) (no device)
//   --allow-unreviewed   accept graphs outside the reviewed topologies
// One JSON line per step, then a closing line. Exit status: 0 ok, 1 failure.
#include <chrono>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <string>
#include <vector>

#include "ernie/block_files.h"
#include "ernie/component_files.h"
#include "ernie/denoiser.h"
#include "runner_io.hpp"

namespace fs = std::filesystem;
using namespace ernie_runner;

namespace {

double sum(const std::vector<double>& xs) { return std::accumulate(xs.begin(), xs.end(), 0.0); }

void write_mat(const fs::path& path, const ernie::Device& device, const ernie::DeviceMat& m)
{
    const std::vector<float> host = m.download(device);
    write_f32(path, host.data(), host.size());
}

}  // namespace

int main(int argc, char** argv)
{
    std::vector<std::string> blocks;
    std::string input_head, output_head;
    fs::path fixture, output;
    std::string backend = "hip", precision = "fp32";
    int w = 0, h = 0, text = 0, steps = 8;
    float only_timestep = -1.f;
    bool trace = false, features_only = false, allow_unreviewed = false;
    try {
        for (int i = 1; i < argc; ++i) {
            const std::string flag = argv[i];
            if (flag == "--trace") { trace = true; continue; }
            if (flag == "--allow-unreviewed") { allow_unreviewed = true; continue; }
            if (i + 1 == argc) throw std::invalid_argument("Missing value for " + flag);
            const std::string value = argv[++i];
            if (flag == "--model") blocks.push_back(value);
            else if (flag == "--input-head") input_head = value;
            else if (flag == "--output-head") output_head = value;
            else if (flag == "--fixture") fixture = value;
            else if (flag == "--output") output = value;
            else if (flag == "--backend") backend = value;
            else if (flag == "--precision") precision = value;
            else if (flag == "--timestep") {
                size_t used = 0;
                only_timestep = std::stof(value, &used);
                if (used != value.size()) throw std::invalid_argument("Invalid timestep");
                features_only = true;
            } else if (flag == "--width") w = parse_int(flag, value);
            else if (flag == "--height") h = parse_int(flag, value);
            else if (flag == "--text-tokens") text = parse_int(flag, value);
            else if (flag == "--steps") steps = parse_int(flag, value);
            else throw std::invalid_argument("Unknown argument: " + flag);
        }
        if (output.empty() || fs::exists(output)) throw std::invalid_argument("Use a new --output directory");
        if (features_only) {
            const std::vector<float> features = ernie::timestep_features(only_timestep);
            fs::create_directories(output);
            write_f32(output / "features.f32", features.data(), features.size());
            return 0;
        }
        if (fixture.empty() || w < 1 || w > 256 || h < 1 || h > 256 || text < 1 || text > 2048 ||
            w * h + text > 10240 || blocks.empty() || blocks.size() > 36 || input_head.empty() ||
            output_head.empty() || steps < 1 || steps > 1000 || (backend != "hip" && backend != "vulkan") ||
            (precision != "fp32" && precision != "fp16" && precision != "bf16"))
            throw std::invalid_argument(backend == "cpu"
                                            ? "This build runs the denoise on the device only (--backend hip)"
                                            : "Require heads, blocks, fixture, dimensions and hip precision");
        const int dtype =
            precision == "fp32" ? ERNIE_DTYPE_FP32 : precision == "fp16" ? ERNIE_DTYPE_FP16 : ERNIE_DTYPE_BF16;
        const int tokens = w * h + text;
        const size_t S = (size_t)tokens;
        const std::vector<float> latent = read_f32(fixture / "in0.f32", (size_t)128 * h * w);
        const std::vector<float> text_rows = read_f32(fixture / "in1.f32", (size_t)text * 3072);
        const std::vector<float> cos_t = read_f32(fixture / "in3.f32", S * 128);
        const std::vector<float> sin_t = read_f32(fixture / "in4.f32", S * 128);
        const MaskRow mask = mask_row(read_f32(fixture / "in5.f32", S * S), tokens);

        ernie::Device device(0);
        ernie::DenoiseModel model;
        model.input_head = ernie::load_head_files(device, (fs::path(input_head) / "head.ncnn.param").string(),
                                                  (fs::path(input_head) / "head.ncnn.bin").string(), dtype,
                                                  allow_unreviewed);
        model.output_head = ernie::load_head_files(device, (fs::path(output_head) / "head.ncnn.param").string(),
                                                   (fs::path(output_head) / "head.ncnn.bin").string(), dtype,
                                                   allow_unreviewed);
        if (model.input_head.part != ERNIE_HEAD_INPUT || model.output_head.part != ERNIE_HEAD_OUTPUT)
            throw std::invalid_argument("--input-head and --output-head must hold the input and output heads");
        for (size_t i = 0; i < blocks.size(); ++i) {
            ernie::load_block_files(device, (int)i, (fs::path(blocks[i]) / "block.ncnn.param").string(),
                                    (fs::path(blocks[i]) / "block.ncnn.bin").string(), dtype, allow_unreviewed);
            model.blocks.push_back({(int)i});
        }

        ernie::DeviceMat initial = ernie::DeviceMat::create(device, w, h, 128, 3);
        initial.upload(device, latent.data(), latent.size());
        ernie::DeviceMat dtext = ernie::DeviceMat::create(device, 3072, text, 1, 2);
        dtext.upload(device, text_rows.data(), text_rows.size());
        ernie::DeviceMat dcos = ernie::DeviceMat::create(device, 128, tokens, 1, 2);
        dcos.upload(device, cos_t.data(), cos_t.size());
        ernie::DeviceMat dsin = ernie::DeviceMat::create(device, 128, tokens, 1, 2);
        dsin.upload(device, sin_t.data(), sin_t.size());
        ernie::DeviceMat dmask = ernie::DeviceMat::create(device, tokens);
        dmask.upload(device, mask.row.data(), mask.row.size());
        dmask.valid_prefix = mask.valid_keys;  // 0: the row is applied as an additive mask
        fs::create_directories(output);

        ernie::Option option;
        option.device = &device;
        option.use_fp16_storage = dtype == ERNIE_DTYPE_FP16;
        option.use_bf16_storage = dtype == ERNIE_DTYPE_BF16;
        std::vector<ernie::DenoiseStepStats> stats;
        auto observer = [&](size_t index, const ernie::DeviceMat& prediction, const ernie::DeviceMat& sample) {
            const auto& step = stats.at(index);
            std::cout << std::setprecision(12) << "{\"step\":" << index << ",\"timestep\":" << step.timestep
                      << ",\"delta\":" << step.delta << ",\"elapsed_seconds\":" << step.elapsed_seconds
                      << ",\"block_load_seconds\":" << sum(step.dit.blocks.load_seconds)
                      << ",\"block_compute_seconds\":" << sum(step.dit.blocks.compute_seconds)
                      << ",\"input_head_seconds\":" << step.dit.input_head_seconds
                      << ",\"output_head_seconds\":" << step.dit.output_head_seconds << "}" << std::endl;
            if (trace) {
                device.synchronize();
                write_mat(output / ("prediction-" + std::to_string(index) + ".f32"), device, prediction);
                write_mat(output / ("step-" + std::to_string(index) + ".f32"), device, sample);
                const std::vector<float> f = ernie::timestep_features(step.timestep);
                write_f32(output / ("features-" + std::to_string(index) + ".f32"), f.data(), f.size());
            }
        };
        const ernie::DeviceMat result = ernie::denoise(model, initial, {dtext, dcos, dsin, dmask}, steps, option, stats,
                                                       observer, 0, /*collect_details=*/true);
        write_mat(output / "final.f32", device, result);
        std::cout << "{\"complete\":true,\"steps\":" << stats.size() << ",\"blocks\":" << blocks.size()
                  << ",\"backend\":\"" << backend << "\",\"device_path\":\"hip\",\"dit_storage\":\"" << precision
                  << "\",\"scheduler_storage\":\"fp32\",\"trace_downloads\":" << (trace ? "true" : "false") << "}\n";
    } catch (const std::exception& e) {
        std::cerr << e.what() << '\n';
        return 1;
    }
    return 0;
}
