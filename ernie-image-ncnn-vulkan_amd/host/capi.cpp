// SPDX-License-Identifier: MIT
// C entry points over the C++ facade (declared in include/ernie.h).
#include "ernie.h"

#include <algorithm>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

#include "ernie/block_files.h"
#include "ernie/component_files.h"
#include "ernie/conditioning.h"
#include "ernie/denoiser.h"
#include "ernie/dit.h"
#include "ernie/ops.h"
#include "ernie/sha256.h"
#include "ernie/text_encoder.h"

struct ernie_device {
    ernie::Device device;
    explicit ernie_device(int index) : device(index) {}
};

namespace {

void set_err(char* err, size_t len, const char* msg)
{
    if (!err || !len) return;
    std::strncpy(err, msg, len - 1);
    err[len - 1] = '\0';
}

template <class F>
int guarded(char* err, size_t len, F&& body)
{
    try {
        return body();
    } catch (const ernie::GpuAllocationError& e) {
        set_err(err, len, e.what());
        return ERNIE_ALLOCATION_FAILED;
    } catch (const std::invalid_argument& e) {
        set_err(err, len, e.what());
        return ERNIE_INVALID_REQUEST;
    } catch (const std::out_of_range& e) {
        set_err(err, len, e.what());
        return ERNIE_INVALID_REQUEST;
    } catch (const std::exception& e) {
        set_err(err, len, e.what());
        return ERNIE_ERROR;
    }
}

// Non-owning device view of caller memory.
ernie::DeviceMat wrap(const float* p, int w, int h = 1, int c = 1, int dims = 0)
{
    ernie::DeviceMat m;
    m.data = const_cast<float*>(p);
    m.w = w;
    m.h = h;
    m.c = c;
    m.dims = dims ? dims : (c > 1 ? 3 : (h > 1 ? 2 : 1));
    return m;
}

void fill_info(ernie_block_file_info* info, const ernie::BlockFile& f)
{
    if (!info) return;
    std::memset(info, 0, sizeof(*info));
    info->tokens = f.graph.tokens;
    info->dim = f.graph.dim;
    info->ffn = f.graph.ffn;
    info->contract = static_cast<int>(f.graph.contract);
    std::strncpy(info->component_sha256, f.graph.component_sha256.c_str(), 64);
    std::strncpy(info->runtime_sha256, f.graph.runtime_sha256.c_str(), 64);
    info->bin_bytes = f.bin_bytes;
    info->section_count = static_cast<int>(f.sections.size());
    for (size_t i = 0; i < f.sections.size() && i < 11; ++i) {
        info->section_dtype[i] = f.sections[i].dtype;
        info->section_begin[i] = f.sections[i].begin;
        info->section_data[i] = f.sections[i].data;
        info->section_end[i] = f.sections[i].end;
    }
}

template <class Info, class File>
void fill_sections(Info* info, const File& f, size_t max)
{
    info->bin_bytes = f.bin_bytes;
    info->section_count = static_cast<int>(std::min(f.sections.size(), max));
    for (size_t i = 0; i < f.sections.size() && i < max; ++i) {
        info->section_dtype[i] = f.sections[i].dtype;
        info->section_begin[i] = f.sections[i].begin;
        info->section_data[i] = f.sections[i].data;
        info->section_end[i] = f.sections[i].end;
    }
}

void fill_head_info(ernie_head_file_info* info, const ernie::HeadFile& f)
{
    if (!info) return;
    std::memset(info, 0, sizeof(*info));
    const auto& g = f.graph;
    info->part = static_cast<int>(g.kind);
    info->dim = g.dim;
    info->latent_ch = g.latent_ch;
    info->text_dim = g.text_dim;
    info->text_tokens = g.text_tokens;
    info->image_tokens = g.image_tokens;
    info->tokens = g.tokens;
    info->width = g.width;
    info->height = g.height;
    info->reviewed = g.reviewed;
    std::strncpy(info->contract_sha256, g.contract_sha256.c_str(), 64);
    fill_sections(info, f, 9);
}

void fill_text_info(ernie_text_block_file_info* info, const ernie::TextBlockFile& f)
{
    if (!info) return;
    std::memset(info, 0, sizeof(*info));
    const auto& g = f.graph;
    info->tokens = g.tokens;
    info->hidden = g.hidden;
    info->heads = g.heads;
    info->kv_heads = g.kv_heads;
    info->ffn = g.ffn;
    info->reviewed = g.reviewed;
    std::strncpy(info->contract_sha256, g.contract_sha256.c_str(), 64);
    fill_sections(info, f, 9);
}

ernie::Option option_for(const ernie::Device& d, int dtype)
{
    ernie::Option o;
    o.device = &d;
    o.use_fp16_storage = dtype == ERNIE_DTYPE_FP16;
    o.use_bf16_storage = dtype == ERNIE_DTYPE_BF16;
    return o;
}

}  // namespace

extern "C" {

int ernie_device_create(int index, ernie_device** out)
{
    if (!out) return ERNIE_INVALID_REQUEST;
    *out = nullptr;
    return guarded(nullptr, 0, [&] {
        *out = new ernie_device(index);
        return ERNIE_OK;
    });
}

void ernie_device_destroy(ernie_device* device) { delete device; }

ernie_hip_ctx* ernie_device_ctx(ernie_device* device) { return device ? device->device.ctx() : nullptr; }

int ernie_timestep_features(float timestep, float* out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        const auto f = ernie::timestep_features(timestep);
        std::memcpy(out, f.data(), f.size() * sizeof(float));
        return ERNIE_OK;
    });
}

int ernie_flow_schedule_turbo(int steps, float* sigmas, float* timesteps, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        const auto s = ernie::FlowSchedule::turbo(steps);
        std::memcpy(sigmas, s.sigmas.data(), s.sigmas.size() * sizeof(float));
        std::memcpy(timesteps, s.timesteps.data(), s.timesteps.size() * sizeof(float));
        return ERNIE_OK;
    });
}

int ernie_rope_frequencies(float* out)
{
    const auto f = ernie::rope_frequencies();
    std::memcpy(out, f.data(), f.size() * sizeof(float));
    return ERNIE_OK;
}

int ernie_dit_constants(const float* frequencies, int width, int height, int valid_text, int text_bucket,
                        float* cos_out, float* sin_out, float* mask_out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        const auto k = ernie::dit_constants(std::vector<float>(frequencies, frequencies + 64), width, height,
                                            valid_text, text_bucket);
        std::memcpy(cos_out, k.cos.data(), k.cos.size() * sizeof(float));
        std::memcpy(sin_out, k.sin.data(), k.sin.size() * sizeof(float));
        std::memcpy(mask_out, k.mask.data(), k.mask.size() * sizeof(float));
        return k.valid_keys;
    });
}

int ernie_dit_constants_file(const char* frequency_path, int width, int height, int valid_text, int text_bucket,
                             float* cos_out, float* sin_out, float* mask_out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        if (!frequency_path || !cos_out || !sin_out || !mask_out) throw std::invalid_argument("null argument");
        const auto k = ernie::dit_constants(std::string(frequency_path), width, height, valid_text, text_bucket);
        std::memcpy(cos_out, k.cos.data(), k.cos.size() * sizeof(float));
        std::memcpy(sin_out, k.sin.data(), k.sin.size() * sizeof(float));
        std::memcpy(mask_out, k.mask.data(), k.mask.size() * sizeof(float));
        return k.valid_keys;
    });
}

int ernie_pad_text(const float* embeddings, int tokens, int bucket, float* out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        if (!embeddings || !out) throw std::invalid_argument("null argument");
        if (tokens < 1 || tokens > 2048) throw std::invalid_argument("Invalid text embeddings or padding bucket");
        const std::vector<float> in(embeddings, embeddings + size_t(tokens) * 3072);
        const auto padded = ernie::pad_text(in, tokens, bucket);
        std::memcpy(out, padded.data(), padded.size() * sizeof(float));
        return ERNIE_OK;
    });
}

int ernie_run_block_sequence(ernie_device* device, const int* blocks, int count, const float* x, int S, int dim,
                             const float* const* mods, const float* cos_t, const float* sin_t, const float* mask,
                             int valid_prefix, int storage_dtype, float* out, double* compute_seconds, char* err,
                             size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !blocks || !mods || count < 0) throw std::invalid_argument("null block sequence argument");
        std::vector<ernie::BlockModel> models;
        for (int i = 0; i < count; ++i) models.push_back({blocks[i]});
        std::vector<ernie::DeviceMat> constants;
        for (int i = 0; i < 6; ++i) constants.push_back(wrap(mods[i], dim));
        constants.push_back(wrap(cos_t, 128, S));
        constants.push_back(wrap(sin_t, 128, S));
        ernie::DeviceMat m = mask ? wrap(mask, S) : ernie::DeviceMat{};
        m.valid_prefix = valid_prefix;
        constants.push_back(m);
        ernie::BlockSequenceStats stats;
        const auto& d = device->device;
        const auto result = ernie::run_block_sequence(models, wrap(x, dim, S, 1, 2), constants,
                                                      option_for(d, storage_dtype), ernie::WeightPolicy::Stream, stats);
        ernie::check_status(ernie_hip_convert(d.ctx(), result.data, ERNIE_DTYPE_FP32, out, ERNIE_DTYPE_FP32,
                                              result.total()),
                            d.ctx(), "copy block output");
        d.synchronize();
        if (compute_seconds)
            for (size_t i = 0; i < stats.compute_seconds.size(); ++i) compute_seconds[i] = stats.compute_seconds[i];
        return ERNIE_OK;
    });
}

int ernie_op_forward(ernie_device* device, const char* type, const char* params, const float* weights,
                     size_t weight_count, const ernie_op_blob* inputs, int input_count, ernie_op_blob* outputs,
                     int output_count, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !type || input_count < 0 || output_count < 0 || (input_count && !inputs) ||
            (output_count && !outputs) || (weight_count && !weights))
            throw std::invalid_argument("null op argument");
        ernie::OpRegistry registry;
        if (ernie::register_layers(registry)) throw std::runtime_error("op registration failed");
        ernie::OpParams p = ernie::OpParams::parse(params ? params : "");
        p.weights.assign(weights, weights + weight_count);
        auto tensor = [](const ernie_op_blob& b) {
            ernie::OpTensor t;
            t.data = b.data;
            t.dtype = b.dtype;
            t.w = b.w;
            t.h = b.h;
            t.c = b.c;
            return t;
        };
        std::vector<ernie::OpTensor> in, out;
        for (int i = 0; i < input_count; ++i) in.push_back(tensor(inputs[i]));
        for (int i = 0; i < output_count; ++i) out.push_back(tensor(outputs[i]));
        ernie::Option option = option_for(device->device, ERNIE_DTYPE_FP32);
        if (!registry.has(type)) {
            set_err(err, errlen, (std::string("no registered op ") + type).c_str());
            return ERNIE_ERROR;
        }
        const int rc = registry.forward(type, device->device, in, out, p, option);
        if (rc) set_err(err, errlen, (std::string(type) + " rejected the call or failed").c_str());
        return rc;
    });
}

int ernie_text_constants(const float* inverse_frequencies, int bucket, float* cos_out, float* sin_out,
                         float* mask_out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        if (!inverse_frequencies || !cos_out || !sin_out || !mask_out) throw std::invalid_argument("null text constant");
        const auto k = ernie::text_constants(std::vector<float>(inverse_frequencies, inverse_frequencies + 64), bucket);
        std::memcpy(cos_out, k.cos.data(), k.cos.size() * sizeof(float));
        std::memcpy(sin_out, k.sin.data(), k.sin.size() * sizeof(float));
        std::memcpy(mask_out, k.mask.data(), k.mask.size() * sizeof(float));
        return ERNIE_OK;
    });
}

int ernie_text_embeddings(const uint16_t* table, size_t vocabulary, int width, const uint32_t* ids, int count,
                          int bucket, float* out, char* err, size_t errlen)
{
    return guarded(err, errlen, [&] {
        if (!ids || !out || count < 0) throw std::invalid_argument("null text embedding argument");
        const auto rows = ernie::text_embeddings(table, vocabulary, width, std::vector<uint32_t>(ids, ids + count),
                                                 bucket);
        std::memcpy(out, rows.data(), rows.size() * sizeof(float));
        return ERNIE_OK;
    });
}

int ernie_run_text_blocks(ernie_device* device, const int* blocks, int count, const float* x, int S, int width,
                          const float* cos_t, const float* sin_t, const float* mask, int causal, int storage_dtype,
                          float* out, double* compute_seconds, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !blocks || count < 0) throw std::invalid_argument("null text block argument");
        std::vector<ernie::BlockModel> models;
        for (int i = 0; i < count; ++i) models.push_back({blocks[i]});
        std::vector<ernie::DeviceMat> constants = {wrap(cos_t, 128, S), wrap(sin_t, 128, S),
                                                   mask ? wrap(mask, S, S) : ernie::DeviceMat{}};
        constants[2].causal = causal != 0;
        if (causal && !mask) throw std::invalid_argument("A causal text mask needs its [S][S] tensor");
        ernie::BlockSequenceStats stats;
        const auto& d = device->device;
        const auto result =
            ernie::run_text_blocks(models, wrap(x, width, S, 1, 2), constants, option_for(d, storage_dtype), stats);
        ernie::check_status(ernie_hip_convert(d.ctx(), result.data, ERNIE_DTYPE_FP32, out, ERNIE_DTYPE_FP32,
                                              result.total()),
                            d.ctx(), "copy text block output");
        d.synchronize();
        if (compute_seconds)
            for (size_t i = 0; i < stats.compute_seconds.size(); ++i) compute_seconds[i] = stats.compute_seconds[i];
        return ERNIE_OK;
    });
}

int ernie_denoise_observed(ernie_device* device, const int* blocks, int count, float* latent, int height, int width,
                           const float* text, int text_tokens, const float* cos_t, const float* sin_t,
                           const float* mask, int valid_prefix, int steps, int start_step, int storage_dtype,
                           int collect_details, double* step_seconds, float* step_timesteps,
                           ernie_step_observer observer, void* user, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !blocks || count < 0) throw std::invalid_argument("null denoise argument");
        const auto& d = device->device;
        ernie::DenoiseModel model;
        model.input_head = ernie::resident_head(d, ERNIE_HEAD_INPUT);
        model.output_head = ernie::resident_head(d, ERNIE_HEAD_OUTPUT);
        for (int i = 0; i < count; ++i) model.blocks.push_back({blocks[i]});
        const int S = height * width + text_tokens;
        ernie::DeviceMat m = mask ? wrap(mask, S) : ernie::DeviceMat{};
        m.valid_prefix = valid_prefix;
        const std::vector<ernie::DeviceMat> constants{
            text_tokens ? wrap(text, 3072, text_tokens, 1, 2) : ernie::DeviceMat{}, wrap(cos_t, 128, S),
            wrap(sin_t, 128, S), m};
        std::vector<ernie::DenoiseStepStats> stats;
        ernie::StepObserver step_observer;
        if (observer)
            step_observer = [&](size_t step, const ernie::DeviceMat& prediction, const ernie::DeviceMat& sample) {
                d.synchronize();
                observer(int(step), prediction.data, sample.data, sample.total(), user);
            };
        const auto result = ernie::denoise(model, wrap(latent, width, height, 128, 3), constants, steps,
                                           option_for(d, storage_dtype), stats, step_observer, start_step,
                                           collect_details != 0);
        ernie::check_status(ernie_hip_convert(d.ctx(), result.data, ERNIE_DTYPE_FP32, latent, ERNIE_DTYPE_FP32,
                                              result.total()),
                            d.ctx(), "copy denoised latent");
        d.synchronize();
        for (size_t i = 0; i < stats.size(); ++i) {
            if (step_seconds) step_seconds[i] = stats[i].elapsed_seconds;
            if (step_timesteps) step_timesteps[i] = stats[i].timestep;
        }
        return ERNIE_OK;
    });
}

int ernie_denoise(ernie_device* device, const int* blocks, int count, float* latent, int height, int width,
                  const float* text, int text_tokens, const float* cos_t, const float* sin_t, const float* mask,
                  int valid_prefix, int steps, int start_step, int storage_dtype, double* step_seconds,
                  float* step_timesteps, char* err, size_t errlen)
{
    return ernie_denoise_observed(device, blocks, count, latent, height, width, text, text_tokens, cos_t, sin_t,
                                  mask, valid_prefix, steps, start_step, storage_dtype, 0, step_seconds,
                                  step_timesteps, nullptr, nullptr, err, errlen);
}

int ernie_run_dit(ernie_device* device, const int* blocks, int count, const float* latent, int height, int width,
                  const float* text, int text_tokens, const float* time_features, int dim, const float* cos_t,
                  const float* sin_t, const float* mask, int valid_prefix, int storage_dtype, float* prediction,
                  double* block_seconds, ernie_stage_observer observer, void* user, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !blocks || count < 0 || !latent || !time_features || !prediction || dim < 1)
            throw std::invalid_argument("null run_dit argument");
        const auto& d = device->device;
        ernie::DitModel model;
        model.input_head = ernie::resident_head(d, ERNIE_HEAD_INPUT);
        model.output_head = ernie::resident_head(d, ERNIE_HEAD_OUTPUT);
        for (int i = 0; i < count; ++i) model.blocks.push_back({blocks[i]});
        const int S = height * width + text_tokens;
        ernie::DeviceMat m = mask ? wrap(mask, S) : ernie::DeviceMat{};
        m.valid_prefix = valid_prefix;
        const std::vector<ernie::DeviceMat> inputs{
            wrap(latent, width, height, 128, 3), text_tokens ? wrap(text, 3072, text_tokens, 1, 2) : ernie::DeviceMat{},
            wrap(time_features, dim), wrap(cos_t, 128, S), wrap(sin_t, 128, S), m};
        ernie::DitStats stats;
        stats.collect_details = block_seconds != nullptr;
        ernie::StageObserver stage_observer;
        if (observer)
            stage_observer = [&](const std::string& stage, const ernie::DeviceMat& t) {
                observer(stage.c_str(), t.data, t.w, t.h, t.c, user);
            };
        const auto result = ernie::run_dit(model, inputs, option_for(d, storage_dtype), stats, stage_observer);
        ernie::check_status(ernie_hip_convert(d.ctx(), result.data, ERNIE_DTYPE_FP32, prediction, ERNIE_DTYPE_FP32,
                                              result.total()),
                            d.ctx(), "copy prediction");
        d.synchronize();
        if (block_seconds)
            for (size_t i = 0; i < stats.blocks.compute_seconds.size(); ++i)
                block_seconds[i] = stats.blocks.compute_seconds[i];
        return ERNIE_OK;
    });
}

int ernie_sha256_hex(const void* data, size_t size, char* hex65)
{
    if (!hex65 || (!data && size)) return ERNIE_INVALID_REQUEST;
    const std::string h = ernie::sha256_hex(data, size);
    std::memcpy(hex65, h.c_str(), 65);
    return ERNIE_OK;
}

int ernie_block_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                             const char* expected_bin_sha256, ernie_block_file_info* info, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!param_path) throw std::invalid_argument("null graph path");
        const auto f = ernie::inspect_block_files(param_path, bin_path ? bin_path : "", allow_unreviewed != 0,
                                                  expected_bin_sha256 ? expected_bin_sha256 : "");
        fill_info(info, f);
        return ERNIE_OK;
    });
}

int ernie_block_load(ernie_device* device, int index, const char* param_path, const char* bin_path,
                     int storage_dtype, int allow_unreviewed, const char* expected_bin_sha256,
                     ernie_block_file_info* info, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !param_path || !bin_path) throw std::invalid_argument("null block load argument");
        const auto f = ernie::load_block_files(device->device, index, param_path, bin_path, storage_dtype,
                                               allow_unreviewed != 0, expected_bin_sha256 ? expected_bin_sha256 : "");
        fill_info(info, f);
        return ERNIE_OK;
    });
}

int ernie_head_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                            const char* expected_bin_sha256, ernie_head_file_info* info, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!param_path) throw std::invalid_argument("null graph path");
        const auto f = ernie::inspect_head_files(param_path, bin_path ? bin_path : "", allow_unreviewed != 0,
                                                 expected_bin_sha256 ? expected_bin_sha256 : "");
        fill_head_info(info, f);
        return ERNIE_OK;
    });
}

int ernie_head_load(ernie_device* device, const char* param_path, const char* bin_path, int storage_dtype,
                    int allow_unreviewed, const char* expected_bin_sha256, ernie_head_file_info* info, char* err,
                    size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !param_path || !bin_path) throw std::invalid_argument("null head load argument");
        ernie::HeadFile f;
        ernie::load_head_files(device->device, param_path, bin_path, storage_dtype, allow_unreviewed != 0,
                               expected_bin_sha256 ? expected_bin_sha256 : "", &f);
        fill_head_info(info, f);
        return ERNIE_OK;
    });
}

int ernie_text_block_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                                  const char* expected_bin_sha256, ernie_text_block_file_info* info, char* err,
                                  size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!param_path) throw std::invalid_argument("null graph path");
        const auto f = ernie::inspect_text_block_files(param_path, bin_path ? bin_path : "", allow_unreviewed != 0,
                                                       expected_bin_sha256 ? expected_bin_sha256 : "");
        fill_text_info(info, f);
        return ERNIE_OK;
    });
}

int ernie_text_block_load(ernie_device* device, int index, const char* param_path, const char* bin_path,
                          int storage_dtype, int allow_unreviewed, const char* expected_bin_sha256,
                          ernie_text_block_file_info* info, char* err, size_t errlen)
{
    return guarded(err, errlen, [&]() -> int {
        if (!device || !param_path || !bin_path) throw std::invalid_argument("null text block load argument");
        const auto f = ernie::load_text_block_files(device->device, index, param_path, bin_path, storage_dtype,
                                                    allow_unreviewed != 0,
                                                    expected_bin_sha256 ? expected_bin_sha256 : "");
        fill_text_info(info, f);
        return ERNIE_OK;
    });
}

}  // extern "C"
