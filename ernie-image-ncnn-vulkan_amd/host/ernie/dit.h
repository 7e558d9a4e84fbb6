// SPDX-License-Identifier: MIT
// DiT = input head + blocks + output head (src/dit.h:6-40).
#pragma once
#include "ernie/block_sequence.h"
#include "ernie/component_files.h"

namespace ernie {

struct DitStats {
    struct Detail { std::string component, boundary, status; double seconds = 0; };
    BlockSequenceStats blocks;
    double input_head_seconds = 0;
    double output_head_seconds = 0;
    bool collect_details = false;
    std::vector<Detail> details;
};

// The argument triple of run_dit (src/dit.h:17-19): input head, blocks, output head,
// each resident in the device context (load_head_files / resident_head, load_block_files).
struct DitModel {
    HeadModel input_head;
    std::vector<BlockModel> blocks;
    HeadModel output_head;
};

// inputs: packed latent [128][H][W], text [T][3072], time features [4096],
// cosine, sine, mask. Returns the prediction [128][H][W]. Throws std::invalid_argument
// without both heads, 1..36 blocks and six inputs.
DeviceMat run_dit(const DitModel& model, const std::vector<DeviceMat>& inputs, const Option& option, DitStats& stats,
                  const StageObserver& observer = {});

}  // namespace ernie
