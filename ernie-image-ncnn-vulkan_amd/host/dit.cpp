// SPDX-License-Identifier: MIT
// run_dit (src/dit.cpp:104-131): input head -> x, c and six modulations; the
// blocks; output head -> prediction. Heads and blocks stay resident, so nothing
// is loaded or released between stages.
#include "ernie/dit.h"

#include <chrono>
#include <stdexcept>

namespace ernie {
namespace {
using Clock = std::chrono::steady_clock;
}

DeviceMat run_dit(const DitModel& model, const std::vector<DeviceMat>& inputs, const Option& option, DitStats& stats,
                  const StageObserver& observer)
{
    if (inputs.size() != 6 || !option.device) throw std::invalid_argument("Require six device DiT inputs and a device");
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

    auto start = Clock::now();
    check_status(ernie_hip_input_head(ctx, latent.data, hw, T ? text.data : nullptr, T, features.data, x.data, c.data,
                                      mods.data),
                 ctx, "input head");
    if (observer) {
        device.synchronize();
        observer("head-0", x);
        observer("head-1", c);
        for (int i = 0; i < 6; ++i) observer("head-" + std::to_string(i + 2), mods.view(size_t(i) * dim, dim));
    }
    stats.input_head_seconds = std::chrono::duration<double>(Clock::now() - start).count();

    std::vector<int> indices;
    for (const auto& b : model.blocks) indices.push_back(b.index);
    std::vector<double> seconds(indices.size(), 0.0);
    check_status(ernie_hip_block_sequence(ctx, indices.data(), int(indices.size()), x.data, x.data, mods.data, cos.data,
                                          sin.data, mask_arg(mask), mask.valid_prefix, S,
                                          seconds.data()),
                 ctx, "extract block output");
    stats.blocks.peak_loaded_nets = int(indices.size());
    for (size_t i = 0; i < seconds.size(); ++i) {
        stats.blocks.load_seconds.push_back(0.0);
        stats.blocks.compute_seconds.push_back(seconds[i]);
        stats.blocks.compute_submissions += 1;
        if (collect_details) stats.blocks.details.push_back({int(i), "extract_compute_composite", "complete", seconds[i]});
    }
    if (observer) observer("block-" + std::to_string(indices.size() - 1), x);

    start = Clock::now();
    check_status(ernie_hip_output_head(ctx, x.data, S, hw, c.data, prediction.data), ctx, "output head");
    stats.output_head_seconds = std::chrono::duration<double>(Clock::now() - start).count();
    return prediction;
}

}  // namespace ernie
