// SPDX-License-Identifier: MIT
//
// CPU oracle for the ERNIE-Image DiT block path.
//
// TEST INFRASTRUCTURE ONLY. The HIP implementation is compared against this
// library: only the test suite, the smoke check and the CPU-baseline
// leg of the benchmark may load it. The product library never links it and
// never falls back to it.
//
// It restates, in plain C++ (FP32 storage, FP64 reductions where noted), the
// semantics of the reference block graph and its host-side helpers:
//   block graph ........ artifacts/2026-09-05/pipeline/models/dit-s4160-residual-v1/
//                        block-04/block.ncnn.param:1-76 (layer order and wiring)
//   block equations .... tools/export_dit_block.py:39-68
//   RMSNorm (FP32) ..... src/ernie_rmsnorm.cpp:21-135
//   erf GELU ........... src/ernie_gelu.cpp:49-61
//   FP32 residual ...... src/ernie_residual.cpp:62-88
//   SDPA + row mask .... src/ernie_attention.cpp:201-221
//   RoPE / mask tables . src/conditioning.cpp:10-43, tools/prepare_pipeline.py:63
//   time features ...... src/denoiser.cpp:22-39
//   schedule / Euler ... src/latent_ops.cpp:31-92
//   DiT heads .......... artifacts/2026-09-05/components/heads/{input,output}/head.ncnn.param
//   text block ......... tests/fixtures/text-s64.ncnn.param, tools/export_text_block.py:56-67
//   text constants ..... src/text_encoder.cpp:92-118
//
// Every function is pinned by a check in tests/ (known-answer tests ported
// from the reference probes, closed forms, invariants, or a brute-force FP64
// evaluation); the pinning for each function is listed next to it below.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- synthetic inputs -------------------------------------------------------
// Counter-based N(mean, std) stream: element i of stream `seed` is a
// Box-Muller transform of splitmix64(seed, offset + i). Order-independent, so
// any slice can be regenerated alone. Pinned: moments / slice consistency test.
void orc_normal_fill(float* out, size_t n, uint64_t seed, uint64_t offset, float mean, float std_dev);

// ---- closed-form host helpers (compiled with -ffp-contract=off) -------------
// src/denoiser.cpp:22-39. Returns 0, or -1 for t outside [0,1000].
// Pinned: FP64 closed form, t=0 gives sin=0/cos=1.
int orc_timestep_features(float timestep, float* out4096);
// src/latent_ops.cpp:31-51 (FlowSchedule::turbo). sigmas has steps+1 entries.
// Pinned: endpoints/monotonicity (tests/test_latent_contract.cpp:19-28), FP64 closed form.
int orc_flow_schedule_turbo(int steps, float* sigmas, float* timesteps);
// src/latent_ops.cpp:72-92, no FMA. Pinned: independent recurrence (test_memory_execution.cpp:323-330).
void orc_euler_step(const float* x, const float* v, float delta, size_t n, float* out);
// tools/prepare_pipeline.py:63: cat_{dim in 32,48,48} 1/256^(arange(0,dim,2)/dim).
// Pinned: torch-generated fixture tests/golden/rope_inv_freq.f32.
void orc_rope_frequencies(float* out64);
// src/conditioning.cpp:10-43. cos/sin [w*h+text][128], mask [w*h+text].
// Pinned: brute-force FP64 table, duplicated-angle and position structure.
int orc_dit_constants(const float* freqs64, int w, int h, int valid, int text,
                      float* cos_out, float* sin_out, float* mask_out);

// ---- operators ---------------------------------------------------------------
// RMSNorm with affine gamma; FP64 sum of squares. Pinned: probes/rmsnorm_probe.cpp KAT.
void orc_rmsnorm(const float* x, const float* gamma, int rows, int width, float eps, float* out);
// Non-affine LayerNorm (output head ln_1). Pinned: rmsnorm_probe --layernorm KAT form.
void orc_layernorm(const float* x, int rows, int width, float eps, float* out);
// h = h * (1 + scale) + shift, broadcast over rows (param lines 15-17, 66-68).
void orc_modulate(float* h, const float* shift, const float* scale, int rows, int width);
// C[M,N] = A[M,K] * W[N,K]^T (+ bias[N]); FP32 arithmetic, blocked/OpenMP.
// Pinned: tests/test_bf16_gemm.cpp exact-product KAT, FP64 brute force.
void orc_gemm_nt(const float* A, const float* W, const float* bias, int M, int N, int K,
                 float* C, int threads);
// 0.5*x*erfc(-x/sqrt2) in FP32 (src/ernie_gelu.cpp:49-61). Pinned: probes/gelu_probe.cpp KAT.
void orc_gelu(const float* x, size_t n, float* out);
// ERNIE rotary on one [rows][128] slab with full-width cos/sin tables.
// Pinned: FP64 restatement of tools/export_dit_block.py:39-47 in tests.
void orc_rope_rows(float* x, const float* cos_t, const float* sin_t, int rows, long row_stride,
                   long table_stride);
// softmax(q k^T * scale + mask) v, FP64 accumulation when precise != 0.
// Strides in elements. kv head = h / (heads / kv_heads). mask: additive FP32,
// [mask_heads][mask_rows][sk] with mask_rows 1 (row broadcast) or sq; NULL = none.
// Only query rows [q_begin, q_end) are computed.
// Pinned: tests/test_attention_mask.cpp and probes/attention_accuracy_probe.cpp KATs.
void orc_sdpa(const float* q, const float* k, const float* v, float* out,
              int heads, int kv_heads, int sq, int sk, int d,
              long q_head_stride, long q_row_stride, long kv_head_stride, long kv_row_stride,
              long o_head_stride, long o_row_stride,
              const float* mask, int mask_heads, int mask_rows, float scale,
              int q_begin, int q_end, int precise, int threads);

// ---- DiT block (block.ncnn.param) ----------------------------------------------
// Weight layout matches the .bin order of tools/build_dit_weights.py:19-31.
typedef struct {
    const float* norm1;              // adaLN_sa_ln.weight [dim]
    const float* wq, *wk, *wv;       // [dim][dim]
    const float* norm_q, *norm_k;    // [128]
    const float* wo;                 // [dim][dim]
    const float* norm2;              // adaLN_mlp_ln.weight [dim]
    const float* w_up, *w_gate;      // [ffn][dim]
    const float* w_down;             // [dim][ffn]
} orc_block_weights;

// mods: 6 x dim (shift_sa, scale_sa, gate_sa, shift_mlp, scale_mlp, gate_mlp)
// = in1..in6. cos/sin [S][128] = in7/in8, mask [S] row mask = in9.
// out may alias x. Pinned: composition of pinned operators + invariants
// (zero gates are identity, zero-weight branches, head permutation symmetry).
int orc_block_forward(const orc_block_weights* w, int dim, int ffn, const float* x,
                      const float* mods, const float* cos_t, const float* sin_t, const float* mask,
                      int S, float* out, int precise_attention, int threads);

// ---- DiT heads (heads/input, heads/output head.ncnn.param) -------------------
typedef struct {
    const float* x_w; const float* x_b;        // x_embedder 1x1 conv [dim][latent_ch], [dim]
    const float* text_w;                        // text_proj [dim][text_dim], no bias
    const float* t1_w; const float* t1_b;      // time MLP linear_2 [dim][dim], [dim]
    const float* t2_w; const float* t2_b;      // linear_3 [dim][dim], [dim]
    const float* mod_w; const float* mod_b;    // linear_4 [6*dim][dim], [6*dim]
} orc_input_head_weights;
typedef struct {
    const float* mod_w; const float* mod_b;    // linear_2 [2*dim][dim], [2*dim]
    const float* proj_w; const float* proj_b;  // gemm_0 [latent_ch][dim], [latent_ch]
} orc_output_head_weights;

// latent [latent_ch][h*w], text [text_tokens][text_dim], time features [dim]
// -> x [h*w + text_tokens][dim], c [dim], mods [6][dim].
int orc_input_head(const orc_input_head_weights* w, int dim, int latent_ch, int text_dim,
                   const float* latent, int hw, const float* text, int text_tokens,
                   const float* time_features, float* x, float* c, float* mods, int threads);
// x [S][dim], c [dim] -> prediction [latent_ch][hw] (first hw tokens).
int orc_output_head(const orc_output_head_weights* w, int dim, int latent_ch,
                    const float* x, int S, int hw, const float* c, float* pred, int threads);

// ---- Mistral text block (tests/fixtures/text-s64.ncnn.param; tools/export_text_block.py:56-67) ----
// x * sigmoid(x) in FP32 as x / (1 + exp(-x)) (the graph's Swish layer silu_7).
// Pinned: FP64 closed form and torch.nn.functional.silu in tests.
void orc_silu(const float* x, size_t n, float* out);
// src/text_encoder.cpp:92-118: cos/sin [bucket][128] with c[j] = c[j+64] = cos(t * f_j)
// from the 64 YaRN inverse frequencies, and the causal mask [bucket][bucket]
// (-FLT_MAX above the diagonal, 0 elsewhere). Returns -1 for a bucket outside
// [1,2048] or a non-finite / non-positive frequency.
// Pinned: FP64 closed form and the mask's exact structure in tests.
int orc_text_constants(const float* freqs64, int bucket, float* cos_out, float* sin_out, float* mask_out);
// Weight layout of tools/build_text_weights.py:15-25 (.bin order); matrices [out][in].
typedef struct {
    const float* norm1;          // input_layernorm.weight [hidden]
    const float* wq;             // q_proj [heads*128][hidden]
    const float* wk, *wv;        // k_proj / v_proj [kv_heads*128][hidden]
    const float* wo;             // o_proj [hidden][heads*128]
    const float* norm2;          // post_attention_layernorm.weight [hidden]
    const float* w_gate, *w_up;  // gate_proj / up_proj [ffn][hidden]
    const float* w_down;         // down_proj [hidden][ffn]
} orc_text_block_weights;
// One decoder block: RMSNorm (eps 1e-5) -> q/k/v -> rotary on q and k -> SDPA with
// GQA and the additive mask [S][S] (NULL = none) -> o_proj + residual -> RMSNorm ->
// down(silu(gate) * up) + residual. out may alias x.
// Pinned: composition of pinned operators + a PyTorch FP64 restatement of
// tools/export_text_block.py:56-67 in tests.
int orc_text_block_forward(const orc_text_block_weights* w, int hidden, int heads, int kv_heads, int ffn,
                           const float* x, const float* cos_t, const float* sin_t, const float* mask, int S,
                           float* out, int precise_attention, int threads);

#ifdef __cplusplus
}
#endif
