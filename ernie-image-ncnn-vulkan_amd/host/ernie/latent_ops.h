// SPDX-License-Identifier: MIT
// Batch-one, deterministic FlowMatch Euler with the Turbo shift 4
// (src/latent_ops.h; src/latent_ops.cpp:31-92). Latent storage and arithmetic are FP32.
#pragma once
#include <cstddef>
#include <vector>

#include "ernie/runtime.h"

namespace ernie {

struct FlowSchedule {
    std::vector<float> sigmas;     // steps + 1 entries, last = 0
    std::vector<float> timesteps;  // 1000 * sigma
    static FlowSchedule turbo(int steps = 8);
    float delta(size_t step) const;
};

// Device Euler x + (delta * v) without FMA; `next` may be `sample` itself
// (alias-safe consume-and-replace, tests/test_latent_contract.cpp:41-45).
void euler_step(const Device& device, const DeviceMat& sample, const DeviceMat& prediction, float delta,
                DeviceMat& next);
bool finite_latent(const Device& device, const DeviceMat& value);

}  // namespace ernie
