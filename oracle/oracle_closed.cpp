// SPDX-License-Identifier: MIT
// Closed-form host helpers of the oracle (test infrastructure only).
// Built with -ffp-contract=off, as the reference builds latent_ops.cpp and
// denoiser.cpp (src/CMakeLists.txt:11-13), so every float operation below is
// rounded exactly where the reference rounds it.
#include "oracle.h"

#include <cmath>
#include <limits>
#include <cstdint>

namespace {
inline uint64_t mix64(uint64_t z)
{
    // splitmix64 finaliser (Steele, Lea, Flood 2014).
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
}  // namespace

extern "C" void orc_normal_fill(float* out, size_t n, uint64_t seed, uint64_t offset, float mean, float std_dev)
{
    const uint64_t key = mix64(seed ^ 0x5851F42D4C957F2Dull);
    const double two_pi = 6.283185307179586476925286766559;
    const double unit = 1.0 / 9007199254740992.0;  // 2^-53
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) {
        const uint64_t c = 2ull * (offset + (uint64_t)i);
        const uint64_t a = mix64(key + c), b = mix64(key + c + 1ull);
        const double u1 = double((a >> 11) + 1ull) * unit;  // (0, 1]
        const double u2 = double(b >> 11) * unit;            // [0, 1)
        const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
        out[i] = float(double(mean) + double(std_dev) * z);
    }
}

// src/denoiser.cpp:22-39 (ERNIE Timesteps(4096, flip_sin_to_cos=false, shift 0)).
extern "C" int orc_timestep_features(float timestep, float* out)
{
    if (!std::isfinite(timestep) || timestep < 0.f || timestep > 1000.f) return -1;
    const float factor = -float(std::log(10000.0));
    for (int i = 0; i < 2048; ++i) {
        const float product = factor * float(i);
        const float exponent = product / 2048.f;
        const float phase = timestep * std::exp(exponent);
        out[i] = std::sin(phase);
        out[2048 + i] = std::cos(phase);
    }
    return 0;
}

// src/latent_ops.cpp:31-51 (FlowSchedule::turbo, shift 4).
extern "C" int orc_flow_schedule_turbo(int steps, float* sigmas, float* timesteps)
{
    if (steps < 1 || steps > 1000) return -1;
    const float increment = -1.f / float(steps);
    for (int i = 0; i < steps; ++i) {
        // linspace(1, 0) evaluated from the nearer endpoint, as PyTorch's CPU
        // FP32 linspace does; the fma on the first half is part of that rule.
        const float raw = i < (steps + 1) / 2 ? std::fma(increment, float(i), 1.f)
                                              : -increment * float(steps - i);
        const float scaled = 4.f * raw;
        const float denominator = 1.f + 3.f * raw;
        sigmas[i] = scaled / denominator;
        timesteps[i] = 1000.f * sigmas[i];
    }
    sigmas[steps] = 0.f;
    return 0;
}

// src/latent_ops.cpp:72-92: change = delta * v, then x + change, two roundings.
extern "C" void orc_euler_step(const float* x, const float* v, float delta, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i) {
        const float change = delta * v[i];
        out[i] = x[i] + change;
    }
}

// tools/prepare_pipeline.py:63 evaluated in FP32 element by element.
extern "C" void orc_rope_frequencies(float* out)
{
    const int dims[3] = {32, 48, 48};
    int j = 0;
    for (int a = 0; a < 3; ++a)
        for (int e = 0; e < dims[a]; e += 2) {
            const float exponent = float(e) / float(dims[a]);
            out[j++] = 1.f / std::pow(256.f, exponent);
        }
}

// src/conditioning.cpp:10-43. Image token i has positions (valid, i / w, i % w),
// text token j has (j, 0, 0); angle j uses axis 0 for j < 16, 1 for j < 40, else 2,
// and is written to both columns 2j and 2j+1.
extern "C" int orc_dit_constants(const float* freqs, int w, int h, int valid, int text,
                                 float* cos_out, float* sin_out, float* mask_out)
{
    if (w < 1 || w > 256 || h < 1 || h > 256 || valid < 1 || text < valid || text > 2048) return -1;
    for (int j = 0; j < 64; ++j)
        if (!std::isfinite(freqs[j]) || freqs[j] <= 0.f) return -1;
    const int image = w * h, length = image + text;
    for (int i = 0; i < length; ++i) {
        const int pos[3] = {i < image ? valid : i - image, i < image ? i / w : 0, i < image ? i % w : 0};
        float* c = cos_out + (size_t)i * 128;
        float* s = sin_out + (size_t)i * 128;
        for (int j = 0; j < 64; ++j) {
            const int axis = j < 16 ? 0 : (j < 40 ? 1 : 2);
            const float phase = float(pos[axis]) * freqs[j];
            c[2 * j] = c[2 * j + 1] = std::cos(phase);
            s[2 * j] = s[2 * j + 1] = std::sin(phase);
        }
    }
    for (int k = 0; k < length; ++k) mask_out[k] = k >= image + valid ? -1e30f : 0.f;
    return 0;
}

// block.ncnn.param lines 15-17: add_0 (scale + 1.0), mul_1, add_2 (+ shift).
extern "C" void orc_modulate(float* h, const float* shift, const float* scale, int rows, int width)
{
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float* row = h + (size_t)r * width;
        for (int i = 0; i < width; ++i) {
            const float one_plus = scale[i] + 1.0f;
            const float scaled = row[i] * one_plus;
            row[i] = scaled + shift[i];
        }
    }
}

// src/text_encoder.cpp:92-118 (float phase = t * f_j; std::cos / std::sin in FP32).
extern "C" int orc_text_constants(const float* freqs64, int bucket, float* cos_out, float* sin_out, float* mask_out)
{
    if (bucket < 1 || bucket > 2048) return -1;
    for (int j = 0; j < 64; ++j)
        if (!std::isfinite(freqs64[j]) || freqs64[j] <= 0.f) return -1;
    for (int t = 0; t < bucket; ++t) {
        float* c = cos_out + (size_t)t * 128;
        float* s = sin_out + (size_t)t * 128;
        for (int j = 0; j < 64; ++j) {
            const float phase = float(t) * freqs64[j];
            c[j] = c[j + 64] = std::cos(phase);
            s[j] = s[j + 64] = std::sin(phase);
        }
        float* m = mask_out + (size_t)t * bucket;
        for (int k = 0; k < bucket; ++k) m[k] = k > t ? -std::numeric_limits<float>::max() : 0.f;
    }
    return 0;
}
