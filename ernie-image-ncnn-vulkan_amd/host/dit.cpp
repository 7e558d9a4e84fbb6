// SPDX-License-Identifier: MIT
// run_dit (src/dit.cpp:104-131): input head -> x, c and six modulations; the
// blocks; output head -> prediction. Heads and blocks stay resident, so nothing
// is loaded or released between stages.
//
// Without an observer or collect_details the whole DiT is queued on the context
// stream and nothing waits for it. An observer sees every block output, as the
// reference's does (it passes the observer into run_block_sequence,
// src/dit.cpp:126 -> src/block_sequence.cpp:89): the blocks then run one call
// each. collect_details times the heads and every block with device events and
// waits once, at the end.
#include "ernie/dit.h"

#include <stdexcept>

namespace ernie {
namespace {

// Stream markers of a timed DiT, from the facade's reserved range (the denoise loop has
// the first three): before the input head, after it, after the blocks, after the output head.
enum {
    kMarkStart = ERNIE_MARKERS + 3,
    kMarkHead = ERNIE_MARKERS + 4,
    kMarkBlocks = ERNIE_MARKERS + 5,
    kMarkEnd = ERNIE_MARKERS + 6
};

double marker_seconds(ernie_hip_ctx* ctx, int from, int to)
{
    double s = 0;
    check_status(ernie_hip_marker_elapsed(ctx, from, to, &s), ctx, "DiT timing");
    return s;
}

}  // namespace

DeviceMat run_dit(const DitModel& model, const std::vector<DeviceMat>& inputs, const Option& option, DitStats& stats,
                  const StageObserver& observer)
{
    if (inputs.size() != 6 || !option.device) throw std::invalid_argument("Require six device DiT inputs and a device");
    if (model.input_head.part != ERNIE_HEAD_INPUT || model.output_head.part != ERNIE_HEAD_OUTPUT)
        throw std::invalid_argument("Require the input and output heads");
    if (model.blocks.empty() || model.blocks.size() > 36)
        throw std::invalid_argument("Expected 1..36 blocks and nine shared constants");
    option.dtype();
    const Device& device = *option.device;
    ernie_hip_ctx* ctx = device.ctx();
    const DeviceMat &latent = inputs[0], &text = inputs[1], &features = inputs[2];
    const DeviceMat &cos = inputs[3], &sin = inputs[4], &mask = inputs[5];
    if (latent.empty() || latent.dims != 3) throw std::invalid_argument("Latent must be [channels][H][W]");
    const int hw = latent.w * latent.h, T = text.empty() ? 0 : text.h;
    const int S = hw + T;
    if (features.empty() || cos.total() != size_t(S) * 128 || sin.total() != size_t(S) * 128 ||
        (!mask.empty() && mask.total() != size_t(S)))
        throw std::invalid_argument("DiT constants do not match the token count");
    const int dim = int(features.total());

    const bool collect_details = stats.collect_details;
    stats = {};
    stats.collect_details = collect_details;
    stats.blocks.collect_details = collect_details;

    DeviceMat x = DeviceMat::create(device, dim, S, 1, 2);
    DeviceMat cm = DeviceMat::create(device, dim, 7, 1, 2);  // c, then mods [6][dim]
    DeviceMat c = cm.view(0, dim), mods = cm.view(dim, dim, 6, 1, 2);
    DeviceMat prediction = DeviceMat::create(device, latent.w, latent.h, latent.c, 3);

    if (collect_details) check_status(ernie_hip_marker_record(ctx, kMarkStart), ctx, "DiT timing");
    check_status(ernie_hip_input_head(ctx, latent.data, hw, T ? text.data : nullptr, T, features.data, x.data, c.data,
                                      mods.data),
                 ctx, "input head");
    if (collect_details) check_status(ernie_hip_marker_record(ctx, kMarkHead), ctx, "DiT timing");
    if (observer) {
        device.synchronize();  // the observer may read the tensors by any route
        observer("head-0", x);
        observer("head-1", c);
        for (int i = 0; i < 6; ++i) observer("head-" + std::to_string(i + 2), mods.view(size_t(i) * dim, dim));
    }

    std::vector<int> indices;
    for (const auto& b : model.blocks) indices.push_back(b.index);
    const int count = int(indices.size());
    std::vector<double> seconds(indices.size(), 0.0);
    double* timing = collect_details ? seconds.data() : nullptr;
    if (observer) {
        // One block per call, the observer after each ("block-i").
        for (int i = 0; i < count; ++i) {
            check_status(ernie_hip_block_sequence(ctx, &indices[i], 1, x.data, x.data, mods.data, cos.data, sin.data,
                                                  mask_arg(mask), mask.valid_prefix, S, timing ? timing + i : nullptr),
                         ctx, "extract block output");
            device.synchronize();
            observer("block-" + std::to_string(i), x);
        }
    } else {
        check_status(ernie_hip_block_sequence(ctx, indices.data(), count, x.data, x.data, mods.data, cos.data, sin.data,
                                              mask_arg(mask), mask.valid_prefix, S, timing),
                     ctx, "extract block output");
    }
    if (collect_details) check_status(ernie_hip_marker_record(ctx, kMarkBlocks), ctx, "DiT timing");
    stats.blocks.peak_loaded_nets = count;
    stats.blocks.compute_submissions = count;
    // One load and one compute entry per block, as the reference records them
    // (src/block_sequence.cpp:87,252). Blocks are resident, so nothing is loaded; per-block
    // device time is measured only when details are collected (every block is otherwise
    // queued without a wait) and reads 0 when it was not.
    for (int i = 0; i < count; ++i) {
        stats.blocks.load_seconds.push_back(0.0);
        stats.blocks.compute_seconds.push_back(seconds[i]);
        if (collect_details) stats.blocks.details.push_back({i, "extract_compute_composite", "complete", seconds[i]});
    }

    check_status(ernie_hip_output_head(ctx, x.data, S, hw, c.data, prediction.data), ctx, "output head");
    if (collect_details) {
        check_status(ernie_hip_marker_record(ctx, kMarkEnd), ctx, "DiT timing");
        stats.input_head_seconds = marker_seconds(ctx, kMarkStart, kMarkHead);
        stats.output_head_seconds = marker_seconds(ctx, kMarkBlocks, kMarkEnd);
        stats.details.push_back({"input-head", "compute", "complete", stats.input_head_seconds});
        stats.details.push_back({"output-head", "compute", "complete", stats.output_head_seconds});
    }
    return prediction;
}

}  // namespace ernie
