// SPDX-License-Identifier: MIT
// Compiled with -ffp-contract=off, as the reference compiles denoiser.cpp.
#include "ernie/denoiser.h"

#include <chrono>
#include <cmath>
#include <stdexcept>

namespace ernie {
namespace {

using Clock = std::chrono::steady_clock;

// src/denoiser.cpp:12-19.
void check_request(const DenoiseModel& model, const DeviceMat& initial, size_t constants)
{
    if (model.blocks.empty() || model.blocks.size() > 36 || constants != 4 || initial.empty() || initial.dims != 3 ||
        initial.c != 128 || initial.w < 1 || initial.h < 1 || initial.w > 256 || initial.h > 256)
        throw std::invalid_argument("Require heads, 1..36 blocks, four constants and a pack1 FP32 latent");
}

}  // namespace

std::vector<float> timestep_features(float timestep)
{
    if (!std::isfinite(timestep) || timestep < 0.f || timestep > 1000.f)
        throw std::invalid_argument("Timestep must be finite and in [0,1000]");
    std::vector<float> out(4096);
    const float factor = -float(std::log(10000.0));
    for (int i = 0; i < 2048; ++i) {
        const float product = factor * float(i);
        const float exponent = product / 2048.f;
        const float phase = timestep * std::exp(exponent);
        out[i] = std::sin(phase);
        out[2048 + i] = std::cos(phase);
    }
    return out;
}

DeviceMat denoise(const DenoiseModel& model, const DeviceMat& initial, const std::vector<DeviceMat>& constants,
                  int steps, const Option& option, std::vector<DenoiseStepStats>& stats, const StepObserver& observer,
                  int start_step, bool collect_details)
{
    check_request(model, initial, constants.size());
    if (start_step < 0 || start_step > steps) throw std::invalid_argument("Denoising start step must be in [0,steps]");
    if (!option.device) throw std::invalid_argument("Device denoiser requires a device");
    const Device& device = *option.device;
    const auto schedule = FlowSchedule::turbo(steps);
    stats.clear();
    DeviceMat sample = DeviceMat::create(device, initial.w, initial.h, initial.c, 3);
    check_status(ernie_hip_convert(device.ctx(), initial.data, ERNIE_DTYPE_FP32, sample.data, ERNIE_DTYPE_FP32,
                                   initial.total()),
                 device.ctx(), "copy initial latent");
    if (!finite_latent(device, sample)) throw std::invalid_argument("Initial latent is not finite");
    DeviceMat features = DeviceMat::create(device, 4096);
    DitModel dit{model.blocks};
    for (int i = start_step; i < steps; ++i) {
        const auto start = Clock::now();
        DenoiseStepStats step;
        step.dit.collect_details = collect_details;
        step.timestep = schedule.timesteps[i];
        step.delta = schedule.delta(i);
        DeviceMat prediction;
        try {
            const auto host_features = timestep_features(step.timestep);
            features.upload(device, host_features.data(), host_features.size());
            const std::vector<DeviceMat> inputs{sample, constants[0], features, constants[1], constants[2], constants[3]};
            prediction = run_dit(dit, inputs, option, step.dit);
            euler_step(device, sample, prediction, step.delta, sample);
            if (!finite_latent(device, sample))
                throw std::runtime_error("Non-finite latent after denoise step " + std::to_string(i + 1));
        } catch (...) {
            step.elapsed_seconds = std::chrono::duration<double>(Clock::now() - start).count();
            stats.push_back(step);
            throw;
        }
        step.elapsed_seconds = std::chrono::duration<double>(Clock::now() - start).count();
        step.complete = true;
        stats.push_back(step);
        if (observer) observer(size_t(i), prediction, sample);
    }
    return sample;
}

}  // namespace ernie
