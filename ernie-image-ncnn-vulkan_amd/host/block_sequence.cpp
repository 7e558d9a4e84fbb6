// SPDX-License-Identifier: MIT
#include "ernie/block_sequence.h"

#include <chrono>
#include <stdexcept>
#include <vector>

namespace ernie {
namespace {

using Clock = std::chrono::steady_clock;

// src/block_sequence.cpp:47-53.
void check_request(size_t models, size_t constants, WeightPolicy policy)
{
    if (models < 1 || models > 36 || constants != 9)
        throw std::invalid_argument("Expected 1..36 blocks and nine shared constants");
    if (policy == WeightPolicy::Resident && models > 36)
        throw std::invalid_argument("Resident policy holds at most 36 blocks");
}

}  // namespace

DeviceMat run_block_sequence(const std::vector<BlockModel>& models, const DeviceMat& input,
                             const std::vector<DeviceMat>& constants, const Option& option, WeightPolicy policy,
                             BlockSequenceStats& stats, const StageObserver& observer)
{
    check_request(models.size(), constants.size(), policy);
    if (!option.device) throw std::invalid_argument("Block sequence requires a device");
    option.dtype();  // validates the precision flags
    const Device& device = *option.device;
    ernie_hip_ctx* ctx = device.ctx();
    if (input.empty() || input.dims > 2) throw std::invalid_argument("Block input must be a [S][dim] FP32 tensor");
    const int S = input.h, dim = input.w;
    for (int i = 0; i < 6; ++i)
        if (constants[i].empty() || int(constants[i].total()) != dim)
            throw std::invalid_argument("Modulation constants must have the block width");
    const DeviceMat &cos = constants[6], &sin = constants[7], &mask = constants[8];
    if (cos.total() != size_t(S) * 128 || sin.total() != size_t(S) * 128)
        throw std::invalid_argument("RoPE tables must be [tokens][128]");
    if (!mask.empty() && mask.total() != size_t(S))
        throw std::invalid_argument("Attention mask must be one row of [tokens]");

    const bool collect_details = stats.collect_details;
    stats = {};
    stats.collect_details = collect_details;
    stats.peak_loaded_nets = int(models.size());

    // Modulations as one contiguous [6][dim] buffer (a view when already packed).
    DeviceMat mods;
    bool packed = true;
    for (int i = 1; i < 6; ++i) packed = packed && constants[i].data == constants[0].data + size_t(i) * dim;
    if (packed) {
        mods = constants[0];
    } else {
        mods = DeviceMat::create(device, dim, 6);
        for (int i = 0; i < 6; ++i) {
            const std::vector<float> host = constants[i].download(device);
            check_status(ernie_hip_memcpy_h2d(ctx, mods.data + size_t(i) * dim, host.data(), host.size() * 4), ctx,
                         "pack modulations");
        }
    }
    DeviceMat current = DeviceMat::create(device, dim, S, 1, 2);
    std::vector<int> indices;
    for (const auto& m : models) indices.push_back(m.index);
    const int count = int(indices.size());
    std::vector<double> seconds(indices.size(), 0.0);
    // Without an observer every block is queued in one call and timed with device events
    // (one wait at the end); an observer sees each block's output as it completes, so the
    // blocks then run one call each (the reference's per-block extract,
    // src/block_sequence.cpp:73-89).
    const auto start = Clock::now();
    const int batch = observer ? 1 : count;
    for (int first = 0; first < count; first += batch) {
        const int rc = ernie_hip_block_sequence(ctx, &indices[first], batch, first ? current.data : input.data,
                                                current.data, mods.data, cos.data, sin.data, mask_arg(mask),
                                                mask.valid_prefix, S, &seconds[first]);
        if (rc) {
            if (stats.collect_details)
                stats.details.push_back({first, "extract_compute_composite", "failed",
                                         std::chrono::duration<double>(Clock::now() - start).count()});
            check_status(rc, ctx, "extract block output");
        }
        for (int i = first; i < first + batch; ++i) {
            stats.load_seconds.push_back(0.0);
            stats.compute_seconds.push_back(seconds[i]);
            stats.compute_submissions += 1;
            if (stats.collect_details)
                stats.details.push_back({i, "extract_compute_composite", "complete", seconds[i]});
        }
        if (observer) observer("block-" + std::to_string(first), current);
    }
    return current;
}

}  // namespace ernie
