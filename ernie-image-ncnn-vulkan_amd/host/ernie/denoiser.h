// SPDX-License-Identifier: MIT
// Denoise loop (src/denoiser.h:1-52).
#pragma once
#include <functional>

#include "ernie/dit.h"
#include "ernie/latent_ops.h"

namespace ernie {

// ERNIE Timesteps(4096, flip_sin_to_cos=false, downscale_freq_shift=0),
// src/denoiser.cpp:22-39. Throws std::invalid_argument outside [0,1000].
std::vector<float> timestep_features(float timestep);

// src/denoiser.h:13-17: the two head components and the blocks, here resident in the
// device context.
struct DenoiseModel {
    HeadModel input_head, output_head;
    std::vector<BlockModel> blocks;
};

struct DenoiseStepStats {
    float timestep = 0, delta = 0;
    DitStats dit;
    // Device time from the end of the previous step (or the loop start) to the end of
    // this one; steps are queued without waiting, so host time would not measure them.
    double elapsed_seconds = 0;
    bool complete = false;
};

using StepObserver = std::function<void(size_t, const DeviceMat&, const DeviceMat&)>;

// Constants: text embeddings, cosine, sine, attention mask. start_step keeps the
// absolute schedule and observer step indices; stats holds executed steps only;
// start_step == steps performs no model work (src/denoiser.h:26-33).
DeviceMat denoise(const DenoiseModel& model, const DeviceMat& initial, const std::vector<DeviceMat>& constants,
                  int steps, const Option& option, std::vector<DenoiseStepStats>& stats,
                  const StepObserver& observer = {}, int start_step = 0, bool collect_details = false);

}  // namespace ernie
