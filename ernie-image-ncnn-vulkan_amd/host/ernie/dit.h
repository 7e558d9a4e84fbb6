// SPDX-License-Identifier: MIT
// DiT = input head + blocks + output head (src/dit.h:6-40).
#pragma once
#include "ernie/block_sequence.h"

namespace ernie {

struct DitStats {
    struct Detail { std::string component, boundary, status; double seconds = 0; };
    BlockSequenceStats blocks;
    double input_head_seconds = 0;
    double output_head_seconds = 0;
    bool collect_details = false;
    std::vector<Detail> details;
};

// Heads are resident in the device context next to the blocks.
struct DitModel {
    std::vector<BlockModel> blocks;
};

// inputs: packed latent [128][H][W], text [T][3072], time features [4096],
// cosine, sine, mask. Returns the prediction [128][H][W].
DeviceMat run_dit(const DitModel& model, const std::vector<DeviceMat>& inputs, const Option& option, DitStats& stats,
                  const StageObserver& observer = {});

}  // namespace ernie
