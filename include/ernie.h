/* SPDX-License-Identifier: MIT
 *
 * C entry points of the ernie C++ facade (libernie.so). They drive the same
 * host code a C++ caller reaches through ernie/denoiser.h, ernie/dit.h and
 * ernie/block_sequence.h, for bindings that cannot call C++ (ctypes, cgo...).
 *
 * Status: 0 ok, -1 runtime/device error, -100 GpuAllocationError,
 * -22 std::invalid_argument / std::out_of_range (request rejected before any
 * device work, like the reference's argument checks). `err` (nullable) receives
 * the exception message.
 */
#ifndef ERNIE_H
#define ERNIE_H

#include <stddef.h>
#include <stdint.h>

#include "ernie_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ERNIE_INVALID_REQUEST (-22)

typedef struct ernie_device ernie_device;

/* ernie::Device (the device context standing in for the Vulkan device). */
int ernie_device_create(int index, ernie_device** out);
void ernie_device_destroy(ernie_device* device);
ernie_hip_ctx* ernie_device_ctx(ernie_device* device);

/* timestep_features (src/denoiser.cpp:22-39) -> out[4096]. */
int ernie_timestep_features(float timestep, float* out, char* err, size_t errlen);
/* FlowSchedule::turbo (src/latent_ops.cpp:31-51): sigmas[steps+1], timesteps[steps]. */
int ernie_flow_schedule_turbo(int steps, float* sigmas, float* timesteps, char* err, size_t errlen);
/* rope frequency table (tools/prepare_pipeline.py:63) -> out[64]. */
int ernie_rope_frequencies(float* out);
/* dit_constants (src/conditioning.cpp:10-43) on the host: cos/sin [S][128], mask [S];
 * returns the valid key count (> 0) or a negative status. */
int ernie_dit_constants(const float* frequencies, int width, int height, int valid_text, int text_bucket,
                        float* cos_out, float* sin_out, float* mask_out, char* err, size_t errlen);

/* dit_constants(path, ...) (src/conditioning.cpp:10-23,46-49): the frequency file of
 * exactly 64 FP32 values is read and checked, token limit 6144; outputs as above. */
int ernie_dit_constants_file(const char* frequency_path, int width, int height, int valid_text, int text_bucket,
                             float* cos_out, float* sin_out, float* mask_out, char* err, size_t errlen);
/* pad_text (src/conditioning.cpp:56-67): [tokens][3072] host embeddings zero-padded
 * to out [bucket][3072]; tokens <= bucket <= 2048. */
int ernie_pad_text(const float* embeddings, int tokens, int bucket, float* out, char* err, size_t errlen);

/* run_block_sequence (src/block_sequence.h:38-41): x [S][dim] device FP32,
 * mods = six [dim] device vectors, cos/sin [S][128], mask [S]. valid_prefix > 0
 * declares the mask canonical (0 below it, -1e30 from it, as dit_constants
 * builds it): the key count then replaces the mask, whose contents are not
 * read; 0 applies the mask as given. out [S][dim] device FP32.
 * compute_seconds (nullable) gets per-block device time. */
int ernie_run_block_sequence(ernie_device* device, const int* blocks, int count, const float* x, int S, int dim,
                             const float* const* mods, const float* cos_t, const float* sin_t, const float* mask,
                             int valid_prefix, int storage_dtype, float* out, double* compute_seconds, char* err,
                             size_t errlen);

/* denoise (src/denoiser.h:30-33): latent [128][height][width] device FP32 is
 * replaced by the denoised latent. Constants: text [text_tokens][3072], cos,
 * sin, mask (device). step_seconds / step_timesteps (nullable) get one entry
 * per executed step. */
int ernie_denoise(ernie_device* device, const int* blocks, int count, float* latent, int height, int width,
                  const float* text, int text_tokens, const float* cos_t, const float* sin_t, const float* mask,
                  int valid_prefix, int steps, int start_step, int storage_dtype, double* step_seconds,
                  float* step_timesteps, char* err, size_t errlen);

/* Observer of run_dit's stages (the StageObserver of src/dit.h:17-40): "head-0"
 * (x [S][dim]), "head-1" (c [dim]) and "head-2".."head-7" (the six modulations) after the
 * input head, then "block-i" after block i (x). `data` is device FP32 memory of w*h*c
 * values, readable during the callback only (the device has finished writing it). */
typedef void (*ernie_stage_observer)(const char* stage, const float* data, int w, int h, int c, void* user);
/* run_dit (src/dit.h:17-40; src/dit.cpp:104-131): latent [128][height][width], text
 * [text_tokens][3072], time features [dim] (4096 for the ERNIE model), cos/sin [S][128],
 * mask [S] (all device FP32) -> prediction [128][height][width] (device FP32).
 * block_seconds (nullable, `count` entries) requests per-block device timing
 * (DitStats::collect_details). */
int ernie_run_dit(ernie_device* device, const int* blocks, int count, const float* latent, int height, int width,
                  const float* text, int text_tokens, const float* time_features, int dim, const float* cos_t,
                  const float* sin_t, const float* mask, int valid_prefix, int storage_dtype, float* prediction,
                  double* block_seconds, ernie_stage_observer observer, void* user, char* err, size_t errlen);
/* Observer of denoise steps (src/denoiser.h:26-33): absolute step index, the step's
 * prediction and the sample after its Euler update (device FP32, `count` values each),
 * readable during the callback only. */
typedef void (*ernie_step_observer)(int step, const float* prediction, const float* sample, size_t count,
                                    void* user);
/* ernie_denoise with a step observer (nullable) and DitStats::collect_details. */
int ernie_denoise_observed(ernie_device* device, const int* blocks, int count, float* latent, int height, int width,
                           const float* text, int text_tokens, const float* cos_t, const float* sin_t,
                           const float* mask, int valid_prefix, int steps, int start_step, int storage_dtype,
                           int collect_details, double* step_seconds, float* step_timesteps,
                           ernie_step_observer observer, void* user, char* err, size_t errlen);

/* ---- the op registry (register_layers, src/ernie_gelu.cpp:108-116) -------------- */
/* One blob of an op call: device data, element type (ERNIE_DTYPE_*), ncnn dims w/h/c
 * with w fastest and no channel padding. */
typedef struct {
    void* data;
    int dtype;
    int w, h, c;
} ernie_op_blob;
/* Registers the reference's custom layers ("ErnieGELU", "RMSNorm", "LayerNorm",
 * "ErnieResidualAdd", "SDPA") plus "Gemm" into an OpRegistry and runs one forward of
 * `type`, as a one-layer ncnn graph of that op would (probes/rmsnorm_probe.cpp:44-53,
 * tests/test_bf16_gemm.cpp:64-75): `params` is the layer line's parameter list
 * ("0=4096 1=1.000000e-6 2=1"; a value with '.', 'e' or 'E' is a float), `weights` its
 * FP32 model data in .bin order without section tags. output_count 0 runs an in-place
 * op on inputs[0]. Returns the layer's status (0, -1 rejected, -100 allocation) or -22
 * for malformed parameter text; queued on the device stream. */
int ernie_op_forward(ernie_device* device, const char* type, const char* params, const float* weights,
                     size_t weight_count, const ernie_op_blob* inputs, int input_count, ernie_op_blob* outputs,
                     int output_count, char* err, size_t errlen);

/* ---- Mistral text path (src/text_encoder.h) ------------------------------------ */
/* text_constants (src/text_encoder.cpp:92-118) on the host from the 64 YaRN inverse
 * frequencies: cos/sin [bucket][128], causal mask [bucket][bucket]. */
int ernie_text_constants(const float* inverse_frequencies, int bucket, float* cos_out, float* sin_out,
                         float* mask_out, char* err, size_t errlen);
/* text_embeddings (src/text_encoder.cpp:68-90) from an in-memory BF16 table
 * [vocabulary][width] -> out [bucket][width] FP32 (rows past `count` zero). */
int ernie_text_embeddings(const uint16_t* table, size_t vocabulary, int width, const uint32_t* ids, int count,
                          int bucket, float* out, char* err, size_t errlen);
/* run_text_blocks (src/text_encoder.h:17-19): x [S][width] device FP32, cos/sin
 * [S][128], mask [S][S] (device; NULL = none), blocks = resident text block slots.
 * causal = 1 declares the mask the causal one text_constants builds: it is then
 * applied by position and not read. out [S][width] device FP32. compute_seconds
 * (nullable) gets per-block time. */
int ernie_run_text_blocks(ernie_device* device, const int* blocks, int count, const float* x, int S, int width,
                          const float* cos_t, const float* sin_t, const float* mask, int causal, int storage_dtype,
                          float* out, double* compute_seconds, char* err, size_t errlen);

/* ---- on-disk blocks (block.ncnn.param + block.ncnn.bin) ----------------------- */
typedef struct {
    int tokens, dim, ffn;         /* static token count of the graph, block widths */
    int contract;                 /* 0 unreviewed, 1 component export, 2 runtime package graph */
    char component_sha256[65];    /* the two normalised graph hashes, "" where a form does not apply */
    char runtime_sha256[65];
    size_t bin_bytes;             /* 0 when no weight file was read */
    int section_count;            /* 11, or 0 without a weight file */
    int section_dtype[11];        /* ERNIE_DTYPE_* stored in each section, .bin order */
    size_t section_begin[11], section_data[11], section_end[11];
} ernie_block_file_info;

/* SHA-256 of a byte string as 64 lower-case hex digits + NUL (hex65). */
int ernie_sha256_hex(const void* data, size_t size, char* hex65);
/* Checks a block graph and, when bin_path is non-NULL, walks its ModelBin
 * sections (and compares the file's SHA-256 when expected_bin_sha256 is
 * non-NULL). Replaces the graph checks of src/shape_graph.cpp:37-95 and
 * tools/build_dit_weights.py:34-50 plus ModelBin parsing for the block. An
 * unreviewed topology is rejected (-22) unless allow_unreviewed. No device. */
int ernie_block_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                             const char* expected_bin_sha256, ernie_block_file_info* info, char* err, size_t errlen);
/* ernie_block_file_inspect, then uploads the weights into resident block slot
 * `index` at storage_dtype: replaces load_component (src/component_files.cpp:37-60)
 * for a block Net. `info` is nullable. */
int ernie_block_load(ernie_device* device, int index, const char* param_path, const char* bin_path,
                     int storage_dtype, int allow_unreviewed, const char* expected_bin_sha256,
                     ernie_block_file_info* info, char* err, size_t errlen);

/* ---- on-disk DiT heads (heads/input, heads/output head.ncnn.{param,bin}) ----------- */
typedef struct {
    int part;                     /* ERNIE_HEAD_INPUT or ERNIE_HEAD_OUTPUT */
    int dim, latent_ch;
    int text_dim, text_tokens;    /* input head: text_proj width and the graph's text slots */
    int image_tokens, tokens;     /* image tokens; image + text tokens (output head) */
    int width, height;            /* output head: packed latent grid */
    int reviewed;                 /* 1 when the graph matches the reviewed runtime contract */
    char contract_sha256[65];     /* the normalised graph's hash, "" when a contract field is missing */
    size_t bin_bytes;             /* 0 when no weight file was read */
    int section_count;            /* 9 (input) or 4 (output) weights and biases, or 0 without a weight file */
    int section_dtype[9];
    size_t section_begin[9], section_data[9], section_end[9];
} ernie_head_file_info;
/* Checks a head graph (the input or output head of src/dit.cpp:22-45; the reference's
 * runtime contract of src/shape_graph.cpp:27-31) and, when bin_path is non-NULL, walks its
 * ModelBin sections: each weight tagged (FP32 0, BF16 0x01348B83, FP16 0x01306B47), each
 * bias raw FP32. An unreviewed topology is rejected (-22) unless allow_unreviewed. No device. */
int ernie_head_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                            const char* expected_bin_sha256, ernie_head_file_info* info, char* err, size_t errlen);
/* ernie_head_file_inspect, then uploads the head into the context at storage_dtype
 * (ernie_hip_heads_upload_tensors with the part the graph declares): replaces the head
 * Net's load_component (src/dit.cpp:22-45, src/component_files.cpp:37-60). */
int ernie_head_load(ernie_device* device, const char* param_path, const char* bin_path, int storage_dtype,
                    int allow_unreviewed, const char* expected_bin_sha256, ernie_head_file_info* info, char* err,
                    size_t errlen);

/* ---- on-disk Mistral text blocks (text.ncnn.{param,bin}) ------------------------- */
typedef struct {
    int tokens, hidden, heads, kv_heads, ffn;
    int reviewed;                 /* 1 when the graph matches the reviewed runtime contract */
    char contract_sha256[65];
    size_t bin_bytes;
    int section_count;            /* 9, or 0 without a weight file */
    int section_dtype[9];
    size_t section_begin[9], section_data[9], section_end[9];
} ernie_text_block_file_info;
/* Checks a text block graph (tests/fixtures/text-s64.ncnn.param form; the runtime contract
 * of src/shape_graph.cpp:25,31) and walks its ModelBin sections (RMSNorm gammas raw FP32,
 * Gemms tagged, tools/build_text_weights.py:52-74). No device. */
int ernie_text_block_file_inspect(const char* param_path, const char* bin_path, int allow_unreviewed,
                                  const char* expected_bin_sha256, ernie_text_block_file_info* info, char* err,
                                  size_t errlen);
/* ernie_text_block_file_inspect, then uploads the block into resident text slot `index`:
 * replaces load_component of a text block Net (src/text_encoder.cpp:30-40). */
int ernie_text_block_load(ernie_device* device, int index, const char* param_path, const char* bin_path,
                          int storage_dtype, int allow_unreviewed, const char* expected_bin_sha256,
                          ernie_text_block_file_info* info, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif /* ERNIE_H */
