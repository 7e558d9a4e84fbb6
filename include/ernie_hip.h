/* SPDX-License-Identifier: MIT
 *
 * ernie_hip: C ABI of the MI355X (gfx950) implementation of the ERNIE-Image
 * DiT denoiser block path. Plain pointers and sizes only; every pointer named
 * "device" is HIP device memory owned by the caller unless stated otherwise.
 *
 * Status codes follow the ncnn::Layer convention the reference's custom layers
 * return (src/ernie_attention.cpp:116,122; src/vulkan_memory.h:14-21):
 *   0 = success, -1 = invalid argument or device error, -100 = allocation failure.
 * The message of the last failure is available from ernie_hip_last_error().
 *
 * Threading: a context owns one HIP stream; calls on one context are not
 * thread-safe (the reference serialises generate calls the same way,
 * include/ernie/pipeline.h:143-146). All launches are asynchronous on the
 * context stream unless a function says it synchronises.
 */
#ifndef ERNIE_HIP_H
#define ERNIE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ERNIE_OK 0
#define ERNIE_ERROR (-1)
#define ERNIE_ALLOCATION_FAILED (-100)

/* Storage precision: FP32, FP16 or BF16 storage with FP32 accumulation and FP32
 * norm / softmax statistics and residual stream (ncnn Option use_fp16_storage /
 * use_bf16_storage with use_fp16_arithmetic=false, probes/block_runner.cpp:102-109). */
enum { ERNIE_DTYPE_FP32 = 0, ERNIE_DTYPE_FP16 = 1, ERNIE_DTYPE_BF16 = 2 };

typedef struct ernie_hip_ctx ernie_hip_ctx;

/* ---- context ---------------------------------------------------------------- */
/* Replaces the Vulkan device/session setup around the block runner
 * (src/gpu_context.cpp; src/block_sequence.cpp:119-140). */
int ernie_hip_create(int device, ernie_hip_ctx** out);
void ernie_hip_destroy(ernie_hip_ctx* ctx);
const char* ernie_hip_last_error(const ernie_hip_ctx* ctx);
/* Launch on `hip_stream` (a hipStream_t; NULL = the default null stream, which
 * orders with every blocking stream). ernie_hip_own_stream returns the
 * non-blocking stream the context created, which is its initial stream. */
int ernie_hip_set_stream(ernie_hip_ctx* ctx, void* hip_stream);
void* ernie_hip_own_stream(ernie_hip_ctx* ctx);
void* ernie_hip_get_stream(ernie_hip_ctx* ctx);
int ernie_hip_synchronize(ernie_hip_ctx* ctx);
/* Device memory owned by the context's caller-facing allocator. Freed blocks (up to
 * 8 GiB) are kept for reuse by later allocations of the same rounded size and released
 * by ernie_hip_trim or ernie_hip_destroy: hipFree synchronises the device. Reuse is
 * ordered by the context stream, so memory freed here must not be in use on another
 * stream. Blocks still allocated are freed by ernie_hip_destroy, which must therefore
 * come after the last ernie_hip_free of the context. */
int ernie_hip_malloc(ernie_hip_ctx* ctx, size_t bytes, void** out);
int ernie_hip_free(ernie_hip_ctx* ctx, void* ptr);
/* Waits for the context stream and returns every cached freed block to the driver;
 * returns the bytes released. An allocation that finds the device out of memory does
 * the same once before it fails. */
size_t ernie_hip_trim(ernie_hip_ctx* ctx);
int ernie_hip_memcpy_h2d(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int ernie_hip_memcpy_d2h(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Queues a host-to-device copy without waiting: src is first copied into pinned
 * staging memory owned by the context, so the caller may reuse it on return. The
 * reference records such uploads into the step's command buffer
 * (command.record_upload, src/denoiser.cpp:120-125). */
int ernie_hip_upload_async(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ---- operators: the custom layers the reference registers --------------------
 * register_layers (src/ernie_gelu.cpp:108-116) maps op names to these. */

/* "RMSNorm" -> ErnieRMSNorm::forward_inplace (src/ernie_rmsnorm.cpp:93-129): FP32
 * statistics over `width`, affine gamma (NULL = 1), result cast to out_dtype.
 * Optional fused adaLN modulate n*(1+scale)+shift (block.ncnn.param lines 15-17);
 * pass shift = scale = NULL for the plain op. width % 4 == 0, width <= 4096. */
int ernie_hip_rmsnorm(ernie_hip_ctx* ctx, const void* x, int x_dtype, const float* gamma, const float* shift,
                      const float* scale, int rows, int width, float eps, void* out, int out_dtype);
/* "LayerNorm" (non-affine, output head ln_1) fused with modulate. x FP32. */
int ernie_hip_layernorm_modulate(ernie_hip_ctx* ctx, const float* x, const float* shift, const float* scale,
                                 int rows, int width, float eps, void* out, int out_dtype);
/* "ErnieGELU" -> ErnieGELU::forward_inplace (src/ernie_gelu.cpp:49-61). */
int ernie_hip_gelu(ernie_hip_ctx* ctx, void* data, int dtype, size_t count);
/* "ErnieResidualAdd" -> ErnieResidualAdd::forward (src/ernie_residual.cpp:62-88): FP32 a + b. */
int ernie_hip_residual_add(ernie_hip_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype,
                           float* out, size_t count);
/* "Gemm" with 3=1 (transB), 5=1 (constant B), 10=-1 or 4 (no C / per-column bias)
 * (block.ncnn.param line 19 etc.): C[m][n] = sum_k A[m][k] W[n][k] (+ bias[n]).
 * A, W row strides lda / ldw (elements, multiples of 8 for 16-bit, 4 for FP32;
 * 16-byte aligned bases); K % 32 == 0 (16-bit) or K % 16 == 0 (FP32).
 * out_dtype: FP32 or equal to dtype. */
int ernie_hip_gemm(ernie_hip_ctx* ctx, const void* a, long lda, const void* w, long ldw, const float* bias,
                   void* c, long ldc, int m, int n, int k, int dtype, int out_dtype);
/* "SDPA" with 5=1 (attn mask) -> ErnieSDPA::forward (src/ernie_attention.cpp:201-230):
 * out = softmax(q k^T * scale + mask) v per head; kv head = h / (heads / kv_heads).
 * Strides in elements (head stride, row stride). mask: NULL or additive FP32
 * [mask_heads][mask_rows][sk] with mask_rows 1 (one row broadcast over queries)
 * or sq, mask_heads 1 or heads. valid_keys > 0 excludes keys >= valid_keys
 * (equivalent to the reference's -1e30 padded-text mask). scale <= 0 -> 1/sqrt(d).
 * 16-bit calls with d = 128 and a partial last 128-query tile split that tile along
 * the keys in the context's split workspace (allocated on first use and kept), as
 * the block does. */
int ernie_hip_sdpa(ernie_hip_ctx* ctx, const void* q, const void* k, const void* v, void* out, int dtype,
                   int heads, int kv_heads, int sq, int sk, int d, long q_head_stride, long q_row_stride,
                   long k_head_stride, long k_row_stride, long v_head_stride, long v_row_stride,
                   long o_head_stride, long o_row_stride, const float* mask, int mask_heads, int mask_rows,
                   int valid_keys, float scale);
/* Causal prefill attention (the text encoder's mask, src/text_encoder.cpp:115-116,
 * applied without a mask tensor): key k is visible to query q iff k <= q + (sk - sq);
 * sq <= sk. Otherwise as ernie_hip_sdpa. */
int ernie_hip_sdpa_causal(ernie_hip_ctx* ctx, const void* q, const void* k, const void* v, void* out, int dtype,
                          int heads, int kv_heads, int sq, int sk, int d, long q_head_stride, long q_row_stride,
                          long k_head_stride, long k_row_stride, long v_head_stride, long v_row_stride,
                          long o_head_stride, long o_row_stride, float scale);
/* set_attention_query_rows (src/ernie_attention.cpp:245-255): accepted for
 * compatibility (rows in {128,64,32,16}, else -1); flash attention needs no chunks. */
int ernie_hip_set_attention_query_rows(ernie_hip_ctx* ctx, int rows);
/* attention_internal_submissions (src/ernie_attention.cpp:256-265): always 0 here. */
uint64_t ernie_hip_attention_internal_submissions(const ernie_hip_ctx* ctx);
/* Rounding order of the Q/K RMSNorm (rmsn_9 / rmsn_10) in 16-bit DiT blocks. The reference
 * graph rounds the gemm_0 / gemm_1 outputs to the storage dtype and normalises and rotates
 * those (block.ncnn.param lines 19-57): ERNIE_QK_ROUND_STORAGE does the same, with a
 * separate pass after the QKV GEMM. ERNIE_QK_ROUND_FUSED (the default) normalises and
 * rotates Q and K from the GEMM's FP32 accumulators in its epilogue and rounds once, after
 * the rotation: one rounding fewer and no extra pass. FP32 blocks are the same either way.
 * The mode applies to block forwards issued after the call. */
#define ERNIE_QK_ROUND_FUSED 0
#define ERNIE_QK_ROUND_STORAGE 1
int ernie_hip_set_qk_rounding(ernie_hip_ctx* ctx, int mode);
/* rmsn_9/rmsn_10 + rotary (block.ncnn.param lines 28-57) in place on `heads`
 * heads of 128 values per token at x + t*row_stride + h*128; cos/sin [rows][128].
 * gamma NULL: rotary only (the text block's q/k path, text-s64.ncnn.param lines 18-44). */
int ernie_hip_qk_norm_rope(ernie_hip_ctx* ctx, void* x, int dtype, int rows, int heads, long row_stride,
                           const float* gamma, const float* cos_t, const float* sin_t);

/* ---- denoise-loop helpers (src/latent_ops.cpp) ---------------------------------- */
/* euler_step (src/latent_ops.cpp:72-92): out = x + (delta * v), no FMA; out may alias x. */
int ernie_hip_euler_step(ernie_hip_ctx* ctx, const float* x, const float* v, float delta, size_t count,
                         float* out);
/* finite_latent (src/latent_ops.cpp:60-70): synchronises; *finite = 1 if all finite. */
int ernie_hip_finite(ernie_hip_ctx* ctx, const float* x, size_t count, int* finite);
/* The same check split in two so a denoise step needs no queue drain. The reference
 * submits its finite shader and waits (VulkanLatentOps::finite_latent,
 * src/latent_ops.cpp:160-183); here _begin queues the check of x and the copy of its
 * flag to pinned host memory in `slot`, and _end waits for that copy only (work queued
 * after _begin keeps the device busy meanwhile). One check may be pending per slot. */
#define ERNIE_FINITE_SLOTS 4
/* Slots ERNIE_FINITE_SLOTS .. ERNIE_FINITE_SLOTS + 2 belong to the C++ facade (its denoise
 * loop, ernie/denoiser.h); they are accepted here but a caller that keeps to slots
 * 0 .. ERNIE_FINITE_SLOTS - 1 never shares a slot with a facade call on the same context. */
#define ERNIE_FINITE_SLOTS_RESERVED 3
int ernie_hip_finite_begin(ernie_hip_ctx* ctx, const float* x, size_t count, int slot);
int ernie_hip_finite_end(ernie_hip_ctx* ctx, int slot, int* finite);
/* Stream markers: pooled HIP events recorded on the context stream without a wait;
 * _elapsed waits for marker `to` and returns the device time from `from` to `to`. They
 * stand in for the host clock the reference reads around each synchronous submission
 * (src/denoiser.cpp:104-146, src/block_sequence.cpp:241-253). */
#define ERNIE_MARKERS 64
/* Markers ERNIE_MARKERS .. ERNIE_MARKERS + 7 belong to the C++ facade (denoise steps use
 * the first three, run_dit's stage timing the next four); callers keep to 0 .. 63. */
#define ERNIE_MARKERS_RESERVED 8
int ernie_hip_marker_record(ernie_hip_ctx* ctx, int marker);
int ernie_hip_marker_elapsed(ernie_hip_ctx* ctx, int from, int to, double* seconds);
/* Counter-based N(mean, std) synthetic data directly in device memory. */
int ernie_hip_fill_normal(ernie_hip_ctx* ctx, void* out, int dtype, size_t count, uint64_t seed,
                          uint64_t offset, float mean, float std_dev);
int ernie_hip_convert(ernie_hip_ctx* ctx, const void* in, int in_dtype, void* out, int out_dtype, size_t count);
/* out [cols][rows] = in [rows][cols] (element type dtype; separate buffers): the operand
 * and result transposes of ncnn's Gemm (2=transA, 14=output_transpose), which the
 * registry's "Gemm" applies around the NT kernel. */
int ernie_hip_transpose(ernie_hip_ctx* ctx, const void* in, int dtype, int rows, int cols, void* out);

/* ---- resident block weights (replaces per-block Net load/destroy,
 *      src/block_sequence.cpp:137-142, 241-261; all 36 blocks fit in HBM) ------- */
/* Host FP32 weights in the .bin order of tools/build_dit_weights.py:19-31;
 * matrices are [out][in] row-major. */
typedef struct {
    const float* norm1;            /* adaLN_sa_ln.weight [dim] */
    const float* wq;               /* self_attention.to_q.weight [dim][dim] */
    const float* wk;               /* to_k [dim][dim] */
    const float* wv;               /* to_v [dim][dim] */
    const float* norm_q;           /* norm_q [128] */
    const float* norm_k;           /* norm_k [128] */
    const float* wo;               /* to_out.0 [dim][dim] */
    const float* norm2;            /* adaLN_mlp_ln.weight [dim] */
    const float* w_up;             /* mlp.up_proj [ffn][dim] */
    const float* w_gate;           /* mlp.gate_proj [ffn][dim] */
    const float* w_down;           /* mlp.linear_fc2 [dim][ffn] */
} ernie_block_host_weights;

int ernie_hip_block_upload(ernie_hip_ctx* ctx, int index, const ernie_block_host_weights* w, int dim, int ffn,
                           int dtype);

/* One host tensor with its own element type (ERNIE_DTYPE_FP32/FP16/BF16). */
typedef struct {
    const void* data;
    int dtype;
} ernie_host_tensor;
/* The same eleven tensors, each in the element type it is stored in on disk:
 * the reference's ModelBin keeps RMSNorm gammas as raw FP32 and tags each Gemm
 * weight section FP32 or BF16 (tools/pack_block_weights.py:34-69,
 * tools/build_dit_weights.py:88-121). */
typedef struct {
    ernie_host_tensor norm1, wq, wk, wv, norm_q, norm_k, wo, norm2, w_up, w_gate, w_down;
} ernie_block_host_tensors;
/* Replaces ModelBin loading of one block Net's weights (load_model of the
 * RMSNorm and Gemm layers, src/component_files.cpp:55-60): each tensor is
 * converted on the device to the storage dtype (gammas to FP32). The host
 * memory may be released when the call returns. */
int ernie_hip_block_upload_tensors(ernie_hip_ctx* ctx, int index, const ernie_block_host_tensors* w, int dim,
                                   int ffn, int dtype);
/* Synthetic block: matrices N(0, std), norm gammas 1 + N(0, std), from `seed`. */
int ernie_hip_block_init_random(ernie_hip_ctx* ctx, int index, int dim, int ffn, int dtype, uint64_t seed,
                                float std_dev);
int ernie_hip_block_release(ernie_hip_ctx* ctx, int index);
int ernie_hip_block_count(const ernie_hip_ctx* ctx);

/* One DiT block = block.ncnn.param: in0 = x [S][dim] FP32 (device), mods =
 * in1..in6 as 6 x dim FP32 (shift_sa, scale_sa, gate_sa, shift_mlp, scale_mlp,
 * gate_mlp), cos/sin = in7/in8 [S][128] FP32, mask = in9 one-row additive [S]
 * (NULL allowed) and/or valid_keys (0 = all). out0 [S][dim] FP32; out may alias x.
 * cos/sin hold each rotary angle in two adjacent columns (2k, 2k + 1), as the
 * reference's tables do (src/conditioning.cpp:34-37): 16-bit blocks of a width that is a
 * multiple of 256 read the angles once per pair, and a row whose pair columns differ gets
 * NaN Q/K values there (a table of another layout shows as a non-finite output, never as
 * a silently different one). */
int ernie_hip_block_forward(ernie_hip_ctx* ctx, int index, const float* x, float* out, const float* mods,
                            const float* cos_t, const float* sin_t, const float* mask, int valid_keys, int S);
/* run_block_sequence core (src/block_sequence.cpp:56-94): blocks[0..count) in order.
 * seconds (nullable, count entries) receives per-block device time from HIP
 * events (one wait after the last block). */
int ernie_hip_block_sequence(ernie_hip_ctx* ctx, const int* blocks, int count, const float* x, float* out,
                             const float* mods, const float* cos_t, const float* sin_t, const float* mask,
                             int valid_keys, int S, double* seconds);

/* ---- Mistral text blocks (src/text_encoder.h:14-33, tests/fixtures/text-s64.ncnn.param) ----
 * One decoder block: RMSNorm (eps 1e-5) -> q/k/v projections -> rotary on q and k ->
 * SDPA with grouped K/V heads and an additive mask -> o_proj + residual -> RMSNorm ->
 * down(silu(gate) * up) + residual, head_dim 128, FP32 residual stream. */
/* Host tensors in the .bin order of tools/build_text_weights.py:15-25 (matrices [out][in]). */
typedef struct {
    ernie_host_tensor norm1;   /* input_layernorm.weight [hidden] */
    ernie_host_tensor wq;      /* self_attn.q_proj [heads*128][hidden] */
    ernie_host_tensor wk;      /* self_attn.k_proj [kv_heads*128][hidden] */
    ernie_host_tensor wv;      /* self_attn.v_proj [kv_heads*128][hidden] */
    ernie_host_tensor wo;      /* self_attn.o_proj [hidden][heads*128] */
    ernie_host_tensor norm2;   /* post_attention_layernorm.weight [hidden] */
    ernie_host_tensor w_gate;  /* mlp.gate_proj [ffn][hidden] */
    ernie_host_tensor w_up;    /* mlp.up_proj [ffn][hidden] */
    ernie_host_tensor w_down;  /* mlp.down_proj [hidden][ffn] */
} ernie_text_block_host_tensors;
/* Replaces load_component of one text block Net (src/text_encoder.cpp:30-40); the
 * reference's path is hidden 3072, 32 heads, 8 K/V heads, ffn 9216. */
int ernie_hip_text_block_upload_tensors(ernie_hip_ctx* ctx, int index, const ernie_text_block_host_tensors* w,
                                        int hidden, int heads, int kv_heads, int ffn, int dtype);
/* Synthetic text block: matrices N(0, std), norm gammas 1 + N(0, std), from `seed`. */
int ernie_hip_text_block_init_random(ernie_hip_ctx* ctx, int index, int hidden, int heads, int kv_heads, int ffn,
                                     int dtype, uint64_t seed, float std_dev);
int ernie_hip_text_block_release(ernie_hip_ctx* ctx, int index);
/* in0 = x [S][hidden] FP32, in1/in2 = cos/sin [S][128] FP32 (text_constants),
 * in3 = additive mask [S][S] FP32 (NULL = none); causal = 1 applies the causal mask
 * text_constants builds without reading a tensor (pass mask = NULL then). out0
 * [S][hidden] FP32; out may alias x. */
int ernie_hip_text_block_forward(ernie_hip_ctx* ctx, int index, const float* x, float* out, const float* cos_t,
                                 const float* sin_t, const float* mask, int causal, int S);
/* ernie_hip_text_block_forward that allocates nothing, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops). It has no counterpart
 * in the reference. Its workspace is a fixed 24 MiB device array of the library (one per
 * GPU, held until the process ends), so it takes at most ERNIE_NOALLOC_TEXT_TOKENS
 * tokens (the reference's 32- and 64-token text buckets) and rejects larger calls with
 * an error. Calls that overlap on one GPU share that array and race; calls on one
 * context stream are ordered. Results are bitwise those of ernie_hip_text_block_forward. */
#define ERNIE_NOALLOC_TEXT_TOKENS 64
int ernie_hip_text_block_forward_noalloc(ernie_hip_ctx* ctx, int index, const float* x, float* out,
                                         const float* cos_t, const float* sin_t, const float* mask, int causal, int S);
/* run_text_blocks core (src/text_encoder.cpp:124-180): blocks[0..count), 1..25.
 * seconds (nullable) receives per-block device time. */
int ernie_hip_text_block_sequence(ernie_hip_ctx* ctx, const int* blocks, int count, const float* x, float* out,
                                  const float* cos_t, const float* sin_t, const float* mask, int causal, int S,
                                  double* seconds);

/* ---- DiT heads (heads/input, heads/output head.ncnn.param) ----------------------- */
typedef struct {
    const float* x_w; const float* x_b;     /* x_embedder [dim][latent_ch], [dim] */
    const float* text_w;                     /* text_proj [dim][text_dim] */
    const float* t1_w; const float* t1_b;   /* time MLP [dim][dim], [dim] */
    const float* t2_w; const float* t2_b;   /* [dim][dim], [dim] */
    const float* mod_w; const float* mod_b; /* adaLN [6*dim][dim], [6*dim] */
    const float* out_mod_w; const float* out_mod_b;  /* output head [2*dim][dim], [2*dim] */
    const float* proj_w; const float* proj_b;        /* output proj [latent_ch][dim], [latent_ch] */
} ernie_heads_host_weights;

int ernie_hip_heads_upload(ernie_hip_ctx* ctx, const ernie_heads_host_weights* w, int dim, int latent_ch,
                           int text_dim, int dtype);
/* The two head components (src/denoiser.h:13-17 holds them as separate input_head and
 * output_head ComponentFiles); each can be loaded on its own. */
#define ERNIE_HEAD_INPUT 1
#define ERNIE_HEAD_OUTPUT 2
/* The head tensors, each in the element type it is stored in: the ModelBin sections of
 * heads/input and heads/output head.ncnn.bin keep Convolution, InnerProduct and Gemm
 * weights tagged FP32 (BF16 / FP16 also accepted) and their biases raw FP32. */
typedef struct {
    ernie_host_tensor x_w, x_b, text_w, t1_w, t1_b, t2_w, t2_b, mod_w, mod_b; /* input head */
    ernie_host_tensor out_mod_w, out_mod_b, proj_w, proj_b;                   /* output head */
} ernie_heads_host_tensors;
/* Replaces load_model of the head Nets (src/dit.cpp:22-45): uploads the parts in `parts`
 * (ERNIE_HEAD_INPUT and/or ERNIE_HEAD_OUTPUT), converting each matrix on the device to the
 * storage dtype (biases stay FP32); the fields of a part not uploaded are not read, and
 * text_dim is read only for the input head. A resident part of the same kind is replaced.
 * The other part stays resident and must have the same dim, latent_ch and dtype, else the
 * call is rejected. The host memory may be released when the call returns. */
int ernie_hip_heads_upload_tensors(ernie_hip_ctx* ctx, const ernie_heads_host_tensors* w, int dim, int latent_ch,
                                   int text_dim, int dtype, int parts);
/* ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT bits of the head parts resident in the context. */
int ernie_hip_heads_loaded(const ernie_hip_ctx* ctx);
int ernie_hip_heads_init_random(ernie_hip_ctx* ctx, int dim, int latent_ch, int text_dim, int dtype,
                                uint64_t seed, float std_dev);
/* Input head: latent [latent_ch][hw], text [text_tokens][text_dim], time features
 * [dim] (all FP32 device) -> x [hw+text_tokens][dim], c [dim], mods [6][dim] (FP32). */
int ernie_hip_input_head(ernie_hip_ctx* ctx, const float* latent, int hw, const float* text, int text_tokens,
                         const float* time_features, float* x, float* c, float* mods);
/* Output head: x [S][dim], c [dim] -> prediction [latent_ch][hw] (FP32). */
int ernie_hip_output_head(ernie_hip_ctx* ctx, const float* x, int S, int hw, const float* c, float* prediction);
/* run_dit (src/dit.cpp:104-131): input head, blocks[0..count), output head. */
int ernie_hip_dit_forward(ernie_hip_ctx* ctx, const float* latent, int hw, const float* text, int text_tokens,
                          const float* time_features, const float* cos_t, const float* sin_t, const float* mask,
                          int valid_keys, const int* blocks, int count, float* prediction);

/* ---- per-kernel device timing (HIP events on the context stream) ------------------ */
/* Kernel classes: 0 gemm_qkv, 1 sdpa, 2 gemm_out, 3 gemm_up_gate, 4 gemm_down,
 * 5 rmsnorm_modulate, 6 qk_norm_rope, 7 heads. */
#define ERNIE_PROFILE_CLASSES 8
int ernie_hip_profile_enable(ernie_hip_ctx* ctx, int enable);
/* Restricts event recording to the classes whose bit is set (default: all), so a
 * timed run brackets only the kernel it measures. No reference counterpart: the
 * reference times whole blocks on the host clock (src/block_sequence.cpp:83-88, 247-253). */
int ernie_hip_profile_classes(ernie_hip_ctx* ctx, unsigned class_mask);
/* Brackets only every `stride`-th launch of each recorded class (default 1: every one).
 * Each event record leaves a few-microsecond hole in the queue, so a timed run samples
 * a kernel's launches instead of bracketing all of them. No reference counterpart. */
int ernie_hip_profile_stride(ernie_hip_ctx* ctx, int stride);
/* Synchronises and folds recorded launches into the totals. */
int ernie_hip_profile_collect(ernie_hip_ctx* ctx);
int ernie_hip_profile_reset(ernie_hip_ctx* ctx);
/* launches, total milliseconds, algorithmic FLOP and HBM bytes summed over launches. */
int ernie_hip_profile_query(const ernie_hip_ctx* ctx, int cls, long* launches, double* ms, double* flop,
                            double* bytes);

/* ---- matrix-core ceiling of the device (no reference counterpart) ----------------
 * The reference publishes no device ceiling; this measures the one the FP16 roofline
 * fractions are read against. `launches` back-to-back launches (after one untimed
 * launch) of a kernel in which every wave of one 512-thread workgroup per CU (two
 * waves per SIMD) issues `iters` x 8 independent v_mfma_f32_16x16x32_f16 from
 * registers, with operand bits toggling between consecutive MFMAs. Synchronises.
 * Returns the dense FP16 FLOP/s over the timed launches (HIP events), their seconds,
 * and the shader clock in Hz the chip held during the last launch (median over its
 * waves of s_memtime ticks per s_memrealtime tick, times the constant counter rate). */
int ernie_hip_mfma_rate(ernie_hip_ctx* ctx, int iters, int launches, double* flop_per_s, double* clock_hz,
                        double* seconds);

#ifdef __cplusplus
}
#endif
#endif /* ERNIE_HIP_H */
