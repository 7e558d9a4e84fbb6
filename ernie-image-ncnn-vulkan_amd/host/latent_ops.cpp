// SPDX-License-Identifier: MIT
// Compiled with -ffp-contract=off (the reference builds latent_ops.cpp so).
#include "ernie/latent_ops.h"

#include <cmath>
#include <stdexcept>

namespace ernie {

FlowSchedule FlowSchedule::turbo(int steps)
{
    if (steps < 1 || steps > 1000) throw std::invalid_argument("Steps must be in [1,1000]");
    FlowSchedule result;
    result.sigmas.resize(steps + 1);
    result.timesteps.resize(steps);
    const float increment = -1.f / float(steps);
    for (int i = 0; i < steps; ++i) {
        // FP32 linspace(1, 0) from the nearer endpoint (the rule PyTorch's CPU
        // linspace follows; the fma belongs to that rule), then shift 4.
        const float raw = i < (steps + 1) / 2 ? std::fma(increment, float(i), 1.f) : -increment * float(steps - i);
        const float scaled = 4.f * raw;
        const float denominator = 1.f + 3.f * raw;
        result.sigmas[i] = scaled / denominator;
        result.timesteps[i] = 1000.f * result.sigmas[i];
    }
    result.sigmas[steps] = 0.f;
    return result;
}

float FlowSchedule::delta(size_t step) const
{
    if (step >= timesteps.size() || sigmas.size() != timesteps.size() + 1)
        throw std::out_of_range("Euler schedule exhausted or malformed");
    return sigmas[step + 1] - sigmas[step];
}

namespace {
void check_latent(const DeviceMat& value)
{
    if (value.empty() || value.dims != 3 || value.c != 128 || value.w < 1 || value.h < 1 || value.w > 256 ||
        value.h > 256)
        throw std::invalid_argument("Expected FP32 [128,H,W] latent with 1 <= H,W <= 256");
}
}  // namespace

void euler_step(const Device& device, const DeviceMat& sample, const DeviceMat& prediction, float delta,
                DeviceMat& next)
{
    check_latent(sample);
    check_latent(prediction);
    if (sample.w != prediction.w || sample.h != prediction.h || !std::isfinite(delta) || delta >= 0.f || delta < -1.f)
        throw std::invalid_argument("Incompatible Euler shapes or delta outside [-1,0)");
    if (next.data != sample.data && (next.empty() || next.total() != sample.total()))
        next = DeviceMat::create(device, sample.w, sample.h, sample.c, 3);
    next.w = sample.w; next.h = sample.h; next.c = sample.c; next.dims = 3;
    check_status(ernie_hip_euler_step(device.ctx(), sample.data, prediction.data, delta, sample.total(), next.data),
                 device.ctx(), "Euler step");
}

bool finite_latent(const Device& device, const DeviceMat& value)
{
    check_latent(value);
    int finite = 0;
    check_status(ernie_hip_finite(device.ctx(), value.data, value.total(), &finite), device.ctx(), "Latent finite check");
    return finite != 0;
}

}  // namespace ernie
