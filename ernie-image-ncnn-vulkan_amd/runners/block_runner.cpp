// SPDX-License-Identifier: MIT
// ernie-block-runner: one DiT block from block.ncnn.{param,bin} on the MI355X path, with
// the command line, inputs, output file and result line of the reference's block probe
// (probes/block_runner.cpp:41-245), so that tools/validate_dit_block.py and
// tools/run_block_matrix.py can drive it unchanged.
//
//   --model DIR      block.ncnn.param + block.ncnn.bin (a reviewed block graph)
//   --fixture DIR    in0.f32 [tokens][dim], in1..in6.f32 [dim], in7/in8.f32 [tokens][128],
//                    in9.f32 [tokens][tokens] (the dense broadcast mask)
//   --tokens N       the graph's static token count
//   --output FILE    out0 [tokens][dim] FP32 (a new file)
//   --backend hip|vulkan   the device path ("vulkan" is accepted so the reference's
//                    tools, which pass it, run this path; there is no CPU path here)
//   --precision fp32|fp16|bf16   storage precision (FP32 accumulation)
//   --repeat N       1..20 runs on the same inputs; every run must equal the first bitwise
//   --threads N, --host-weights, --device-io: accepted; weights are always resident in
//                    device memory and inputs are always uploaded once before the runs.
//   --trace-attention   reports the attention launches (one flash launch per run).
//   --output-blob out0 (the only blob the fused block exposes)
//   --allow-unreviewed   accept a block graph outside the reviewed topologies
// Exit status: 0 ok, 1 failure (message on stderr), 2 usage.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <iostream>
#include <string>
#include <vector>

#include "ernie/block_files.h"
#include "ernie/runtime.h"
#include "runner_io.hpp"

namespace fs = std::filesystem;
using Clock = std::chrono::steady_clock;
using namespace ernie_runner;

namespace {

double seconds_since(Clock::time_point t) { return std::chrono::duration<double>(Clock::now() - t).count(); }

int usage(const std::string& why)
{
    std::cerr << why << "\nUsage: ernie-block-runner --model DIR --fixture DIR --tokens N --output FILE "
                        "[--backend hip|vulkan] [--precision fp32|fp16|bf16] [--threads N] [--host-weights] "
                        "[--device-io] [--repeat N] [--trace-attention] [--output-blob out0] [--allow-unreviewed]\n";
    return 2;
}

}  // namespace

int main(int argc, char** argv)
{
    fs::path model, fixture, output;
    std::string backend = "hip", precision = "fp32", output_blob = "out0";
    int tokens = 0, threads = 4, repeat = 1;
    bool host_weights = false, device_io = false, trace_attention = false, allow_unreviewed = false;
    try {
        for (int i = 1; i < argc; ++i) {
            const std::string flag = argv[i];
            if (flag == "--host-weights") { host_weights = true; continue; }
            if (flag == "--device-io") { device_io = true; continue; }
            if (flag == "--trace-attention") { trace_attention = true; continue; }
            if (flag == "--allow-unreviewed") { allow_unreviewed = true; continue; }
            if (i + 1 >= argc) return usage("Missing value for " + flag);
            const std::string value = argv[++i];
            if (flag == "--model") model = value;
            else if (flag == "--fixture") fixture = value;
            else if (flag == "--output") output = value;
            else if (flag == "--output-blob") output_blob = value;
            else if (flag == "--backend") backend = value;
            else if (flag == "--precision") precision = value;
            else if (flag == "--tokens") tokens = parse_int(flag, value);
            else if (flag == "--threads") threads = parse_int(flag, value);
            else if (flag == "--repeat") repeat = parse_int(flag, value);
            else return usage("Unknown option " + flag);
        }
    } catch (const std::invalid_argument& e) {
        return usage(e.what());
    }
    if (model.empty() || fixture.empty() || output.empty() || tokens < 1 || tokens > 10240 || threads < 1 ||
        repeat < 1 || repeat > 20 || (backend != "hip" && backend != "vulkan") ||
        (precision != "fp32" && precision != "fp16" && precision != "bf16"))
        return usage(backend == "cpu" ? "This build runs the block on the device only (--backend hip)"
                                      : "Invalid or missing arguments");
    if (output_blob != "out0") return usage("Only out0 is produced: the block's intermediate blobs are fused");
    const int dtype = precision == "fp32" ? ERNIE_DTYPE_FP32 : precision == "fp16" ? ERNIE_DTYPE_FP16 : ERNIE_DTYPE_BF16;
    try {
        if (fs::exists(output)) throw std::runtime_error("Output exists; use a new path");
        // Graph first: it fixes the block width the inputs are read at.
        const ernie::BlockFile graph =
            ernie::inspect_block_files((model / "block.ncnn.param").string(), "", allow_unreviewed);
        if (graph.graph.tokens != tokens)
            throw std::runtime_error("The graph is static at " + std::to_string(graph.graph.tokens) + " tokens, not " +
                                     std::to_string(tokens));
        const int dim = graph.graph.dim;
        const size_t S = (size_t)tokens;
        const std::vector<float> x = read_f32(fixture / "in0.f32", S * dim);
        std::vector<float> mods;
        for (int i = 1; i <= 6; ++i) {
            const std::vector<float> m = read_f32(fixture / ("in" + std::to_string(i) + ".f32"), (size_t)dim);
            mods.insert(mods.end(), m.begin(), m.end());
        }
        const std::vector<float> cos_t = read_f32(fixture / "in7.f32", S * 128);
        const std::vector<float> sin_t = read_f32(fixture / "in8.f32", S * 128);
        const MaskRow mask = mask_row(read_f32(fixture / "in9.f32", S * S), tokens);

        ernie::Device device(0);
        ernie_hip_ctx* ctx = device.ctx();
        auto t = Clock::now();
        const ernie::BlockFile loaded =
            ernie::load_block_files(device, 0, (model / "block.ncnn.param").string(),
                                    (model / "block.ncnn.bin").string(), dtype, allow_unreviewed);
        device.synchronize();
        const double load_seconds = seconds_since(t);

        t = Clock::now();
        ernie::DeviceMat dx = ernie::DeviceMat::create(device, dim, tokens, 1, 2);
        ernie::DeviceMat dm = ernie::DeviceMat::create(device, dim, 6, 1, 2);
        ernie::DeviceMat dc = ernie::DeviceMat::create(device, 128, tokens, 1, 2);
        ernie::DeviceMat ds = ernie::DeviceMat::create(device, 128, tokens, 1, 2);
        ernie::DeviceMat dmask = ernie::DeviceMat::create(device, tokens);
        ernie::DeviceMat dout = ernie::DeviceMat::create(device, dim, tokens, 1, 2);
        dx.upload(device, x.data(), x.size());
        dm.upload(device, mods.data(), mods.size());
        dc.upload(device, cos_t.data(), cos_t.size());
        ds.upload(device, sin_t.data(), sin_t.size());
        dmask.upload(device, mask.row.data(), mask.row.size());
        device.synchronize();
        const double upload_seconds = seconds_since(t);

        std::vector<double> run_seconds;
        std::vector<float> first, result;
        double repeat_max_abs = 0;
        for (int it = 0; it < repeat; ++it) {
            t = Clock::now();
            ernie::check_status(ernie_hip_block_forward(ctx, 0, dx.data, dout.data, dm.data, dc.data, ds.data,
                                                        mask.valid_keys ? nullptr : dmask.data, mask.valid_keys,
                                                        tokens),
                                ctx, "run block");
            device.synchronize();
            run_seconds.push_back(seconds_since(t));
            result = dout.download(device);
            if (it == 0) first = result;
            else
                for (size_t i = 0; i < result.size(); ++i)
                    repeat_max_abs = std::max(repeat_max_abs, std::abs((double)result[i] - (double)first[i]));
        }
        if (repeat_max_abs != 0) throw std::runtime_error("Repeated same-input execution changed output");
        write_f32(output, result.data(), result.size());
        std::cout.precision(9);
        std::cout << "{\"backend\":\"" << backend << "\",\"device_path\":\"hip\",\"precision\":\"" << precision
                  << "\",\"output_blob\":\"out0\",\"output_shape_whdc\":[" << dim << ',' << tokens << ",1,1]"
                  << ",\"tokens\":" << tokens << ",\"dim\":" << dim << ",\"ffn\":" << loaded.graph.ffn
                  << ",\"load_seconds\":" << load_seconds << ",\"first_run_seconds\":" << run_seconds[0]
                  << ",\"run_seconds\":[";
        for (size_t i = 0; i < run_seconds.size(); ++i) std::cout << (i ? "," : "") << run_seconds[i];
        std::cout << "],\"host_weights\":" << (host_weights ? "true" : "false")
                  << ",\"device_io\":" << (device_io ? "true" : "false") << ",\"upload_seconds\":" << upload_seconds
                  << ",\"repeat_max_abs\":" << repeat_max_abs << ",\"valid_keys\":" << mask.valid_keys
                  << ",\"non_vulkan_compute_layers\":[],\"attention_diagnostic\":";
        // One flash attention launch per block run, over every token and 128-wide heads.
        if (trace_attention)
            std::cout << "{\"calls\":" << repeat << ",\"flash_calls\":" << repeat
                      << ",\"cooperative_calls\":0,\"tokens\":" << tokens << ",\"head_dim\":128}";
        else
            std::cout << "null";
        std::cout << "}\n";
    } catch (const std::exception& e) {
        std::cerr << e.what() << '\n';
        return 1;
    }
    return 0;
}
