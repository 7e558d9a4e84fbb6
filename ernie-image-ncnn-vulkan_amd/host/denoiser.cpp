// SPDX-License-Identifier: MIT
// Compiled with -ffp-contract=off, as the reference compiles denoiser.cpp.
#include "ernie/denoiser.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <exception>
#include <stdexcept>

namespace ernie {
namespace {

using Clock = std::chrono::steady_clock;

// A latent found non-finite by the step-behind check: the error the reference raises
// before it starts the next step (src/denoiser.cpp:56-57, 84-86). Kept apart from device
// failures so the error path below can tell them apart; callers see the base types.
struct NonFiniteInitial : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct NonFiniteStep : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// The facade's own finite-check slots and stream markers (reserved in ernie_hip.h).
constexpr int kStepSlot = ERNIE_FINITE_SLOTS;           // two, alternating by step
constexpr int kInitialSlot = ERNIE_FINITE_SLOTS + 2;
constexpr int kStepMarker = ERNIE_MARKERS;              // three, rotating by step

// src/denoiser.cpp:12-19.
void check_request(const DenoiseModel& model, const DeviceMat& initial, size_t constants)
{
    if (model.input_head.part != ERNIE_HEAD_INPUT || model.output_head.part != ERNIE_HEAD_OUTPUT ||
        model.blocks.empty() || model.blocks.size() > 36 || constants != 4 || initial.empty() || initial.dims != 3 ||
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
    ernie_hip_ctx* ctx = device.ctx();
    const auto schedule = FlowSchedule::turbo(steps);
    stats.clear();
    DeviceMat sample = DeviceMat::create(device, initial.w, initial.h, initial.c, 3);
    check_status(ernie_hip_convert(ctx, initial.data, ERNIE_DTYPE_FP32, sample.data, ERNIE_DTYPE_FP32, initial.total()),
                 ctx, "copy initial latent");
    const int executed = steps - start_step;
    if (!executed) {
        if (!finite_latent(device, sample)) throw std::invalid_argument("Initial latent is not finite");
        return sample;
    }

    // Time features (computed on the host in the reference's FP32 order,
    // src/denoiser.cpp:22-39) go to the device through pinned staging without a wait:
    // step 0's before its DiT, every later step's while the previous step runs.
    DeviceMat features = DeviceMat::create(device, 4096, executed, 1, 2);
    auto upload_features = [&](int k) {
        const auto f = timestep_features(schedule.timesteps[start_step + k]);
        check_status(ernie_hip_upload_async(ctx, features.data + size_t(k) * 4096, f.data(), f.size() * sizeof(float)),
                     ctx, "Upload time features");
    };
    upload_features(0);
    // The initial latent's check is read once step 0's DiT is queued (the reference
    // rejects a non-finite initial latent before any step, src/denoiser.cpp:56-57; here
    // the queued work of that step is simply dropped).
    check_status(ernie_hip_finite_begin(ctx, sample.data, sample.total(), kInitialSlot), ctx, "Latent finite check");
    auto check_initial = [&]() {
        int finite = 0;
        check_status(ernie_hip_finite_end(ctx, kInitialSlot, &finite), ctx, "Latent finite check");
        if (!finite) throw NonFiniteInitial("Initial latent is not finite");
    };

    // Each step is queued without a wait. Its finiteness flag is read one step behind:
    // step i's check is awaited after step i + 1's DiT has been queued, so the device
    // never runs dry; a non-finite step is still reported as that step, and the
    // observer still sees its prediction and sample (step i + 1's Euler update, which
    // replaces the sample, is queued after the check). elapsed_seconds is the device
    // time from the end of the previous step (or the loop start) to the end of this one,
    // from the facade's three step markers.
    struct Pending {
        size_t stat;
        int step, slot, mark_from, mark_to;
        DeviceMat prediction;
    };
    std::vector<Pending> pending;
    bool in_observer = false;  // set while the observer runs inside resolve()
    auto resolve = [&]() {
        Pending p = pending.back();
        pending.clear();
        int finite = 0;
        check_status(ernie_hip_finite_end(ctx, p.slot, &finite), ctx, "Latent finite check");
        double seconds = 0;
        check_status(ernie_hip_marker_elapsed(ctx, p.mark_from, p.mark_to, &seconds), ctx, "Step timing");
        DenoiseStepStats& st = stats[p.stat];
        st.elapsed_seconds = seconds;
        if (!finite) throw NonFiniteStep("Non-finite latent after denoise step " + std::to_string(p.step + 1));
        st.complete = true;
        if (observer) {
            in_observer = true;
            observer(size_t(p.step), p.prediction, sample);
            in_observer = false;
        }
    };

    check_status(ernie_hip_marker_record(ctx, kStepMarker), ctx, "Step timing");
    DitModel dit{model.input_head, model.blocks, model.output_head};
    for (int i = start_step; i < steps; ++i) {
        const int k = i - start_step;
        const auto start = Clock::now();
        DenoiseStepStats step;
        step.dit.collect_details = collect_details;
        step.timestep = schedule.timesteps[i];
        step.delta = schedule.delta(i);
        DeviceMat prediction;
        try {
            const std::vector<DeviceMat> inputs{sample,         constants[0], features.view(size_t(k) * 4096, 4096),
                                                constants[1], constants[2], constants[3]};
            prediction = run_dit(dit, inputs, option, step.dit);
        } catch (...) {
            // The reference finishes each step (finite check, observer) before it starts the
            // next, so what that would have raised first wins: a non-finite earlier latent,
            // or the observer's own exception. A device error met while reading the earlier
            // check gives way to this step's failure, which is rethrown as it was raised.
            const std::exception_ptr failure = std::current_exception();
            try {
                if (k == 0) check_initial();
                if (!pending.empty()) resolve();
            } catch (const NonFiniteInitial&) {
                throw;
            } catch (const NonFiniteStep&) {
                throw;
            } catch (...) {
                if (in_observer) throw;
            }
            step.elapsed_seconds = std::chrono::duration<double>(Clock::now() - start).count();
            stats.push_back(step);
            std::rethrow_exception(failure);
        }
        if (k == 0) check_initial();
        if (!pending.empty()) resolve();
        euler_step(device, sample, prediction, step.delta, sample);
        const int slot = kStepSlot + k % 2;
        check_status(ernie_hip_finite_begin(ctx, sample.data, sample.total(), slot), ctx, "Latent finite check");
        check_status(ernie_hip_marker_record(ctx, kStepMarker + (k + 1) % 3), ctx, "Step timing");
        stats.push_back(step);
        pending.push_back({stats.size() - 1, i, slot, kStepMarker + k % 3, kStepMarker + (k + 1) % 3, prediction});
        if (k + 1 < executed) upload_features(k + 1);
    }
    resolve();
    return sample;
}

}  // namespace ernie
