// SPDX-License-Identifier: MIT
// Block sequence runner (src/block_sequence.h:19-60). Blocks are resident in
// the device context (all 36 fit in HBM), so a "model" is a loaded block index
// rather than a param/bin file pair; Stream and Resident policies run the same
// resident path.
#pragma once
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "ernie/runtime.h"

namespace ernie {

using StageObserver = std::function<void(const std::string&, const DeviceMat&)>;
enum class WeightPolicy { Stream, Resident };

struct BlockModel {
    int index = -1;  // resident block slot in the device context
};

struct BlockSequenceStats {
    struct Detail { int block = -1; std::string boundary, status; double seconds = 0; };
    std::vector<double> load_seconds;
    std::vector<double> compute_seconds;  // device time per block (HIP events; 0 when run_dit does not collect details)
    int peak_loaded_nets = 0;
    int compute_submissions = 0;
    bool collect_details = false;
    std::vector<Detail> details;
    std::uint64_t prefetch_started = 0, prefetch_used = 0, prefetch_skipped = 0;
    std::uint64_t prefetch_peak_charged_bytes = 0;
    double prefetch_overlap_seconds = 0;
};

// Nine shared constants: shift_sa, scale_sa, gate_sa, shift_mlp, scale_mlp,
// gate_mlp ([dim] each), cosine, sine ([S][128]) and the one-row mask ([S]).
// Throws std::invalid_argument unless 1..36 blocks and exactly 9 constants
// (src/block_sequence.cpp:47-53). The observer sees "block-i" after each block.
DeviceMat run_block_sequence(const std::vector<BlockModel>& models, const DeviceMat& input,
                             const std::vector<DeviceMat>& constants, const Option& option, WeightPolicy policy,
                             BlockSequenceStats& stats, const StageObserver& observer = {});

}  // namespace ernie
