// SPDX-License-Identifier: MIT
// Host-side launch interface of the HIP kernels. Every launcher validates the
// shapes its kernel assumes and returns 0 or a negative status (-1 invalid
// argument, or a hipError_t negated) without launching when they do not hold.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ehip {

// ---- GEMM: C[M,N] = A[M,K] * W[N,K]^T with a fused epilogue -----------------
enum Epilogue : int {
    EPI_STORE = 0,       // C = acc (+ bias[n]), C dtype = c_dtype
    EPI_GATE_RESID = 1,  // C(f32) = resid(f32) + gate[n] * acc
    EPI_GEGLU = 2,       // W rows interleaved in 32-row [up | gate] pairs; C[m][n/2] = up * gelu(gate)
    EPI_SWIGLU = 4,      // as EPI_GEGLU with SiLU on the gate: C[m][n/2] = up * silu(gate) (the text MLP)
    // C = acc in the output precision; the columns below qk_cols are 128-column Q / K heads
    // whose W rows are stored permuted (tile_k32 head_rows): each head is RMS-normalised
    // (gamma gq, or gk from column k_col on, eps qk_eps) and rotated with the cos / sin
    // rows of its token, and written in natural order (rmsn_9 / rmsn_10 and the rotary
    // BinaryOps of block.ncnn.param lines 28-57, fused). 16-bit operands only.
    EPI_QKROPE = 5,
};
// Gated epilogues: W rows interleaved in 32-row [up | gate] pairs, N/2 outputs.
constexpr bool epi_glu(int e) { return e == EPI_GEGLU || e == EPI_SWIGLU; }

struct GemmArgs {
    const void* A = nullptr;  // [M][lda], dtype
    long lda = 0;
    const void* W = nullptr;  // [N][ldw], dtype
    long ldw = 0;
    int M = 0, N = 0, K = 0;
    int dtype = 0;            // operand dtype (F32 / F16 / BF16)
    int epilogue = EPI_STORE;
    void* C = nullptr;
    long ldc = 0;
    int c_dtype = 0;
    const float* bias = nullptr;   // [N] (EPI_STORE only)
    const float* resid = nullptr;  // [M][ld_resid] f32 (EPI_GATE_RESID; may alias C)
    long ld_resid = 0;
    const float* gate = nullptr;   // [N]
    // W stored K-tiled as [K/32][N][32] (16-bit operands, N a multiple of 256,
    // ldw = K): the layout tile_k32 writes. Row-major [N][ldw] otherwise.
    bool w_k32 = false;
    // A stored K-tiled as [K/32][a_k32_rows][32] (16-bit operands, lda = K), with
    // a_k32_rows >= M rounded up to 256 so a tail tile's rows stay inside each
    // 32-column slab (rows past M are read but never stored). 0 = row-major [M][lda].
    int a_k32_rows = 0;
    // EPI_GEGLU only: C stored K-tiled as [(N/2)/32][c_k32_rows][32], c_k32_rows >= M,
    // i.e. in the layout a following GEMM reads through a_k32_rows. 0 = row-major.
    int c_k32_rows = 0;
    // Optional split-K scratch for the tail row of tiles (M % 256 rows): FP32 partial
    // sums, summed by a second launch on the same stream. Calls on one stream may
    // share it; calls that run concurrently must not.
    void* split_ws = nullptr;
    size_t split_ws_bytes = 0;
    // EPI_QKROPE: Q / K columns [0, qk_cols) (K heads from k_col), their gammas [128],
    // and each row's rotary angles as rope_pack writes them, [M][64] (cos, sin) pairs.
    int qk_cols = 0;
    long k_col = 0;
    const float* gq = nullptr;
    const float* gk = nullptr;
    const float* cs_t = nullptr;
    float qk_eps = 1e-6f;
};
int gemm(const GemmArgs& a, hipStream_t stream);
// The ping-pong 16-bit kernel (gemm16_pp.hip); returns 1 without launching when
// the shape needs the register-staged kernel instead (operands of 2 GiB or more).
int gemm16_pingpong(const GemmArgs& a, hipStream_t stream);

// ---- flash SDPA ---------------------------------------------------------------
struct SdpaArgs {
    const void* q = nullptr; const void* k = nullptr; const void* v = nullptr; void* o = nullptr;
    int dtype = 0;
    int heads = 0, kv_heads = 0, sq = 0, sk = 0, d = 0;
    long q_hs = 0, q_rs = 0, k_hs = 0, k_rs = 0, v_hs = 0, v_rs = 0, o_hs = 0, o_rs = 0;  // strides (elements)
    // Element distance between consecutive 32-value groups of one output row of a
    // head (0 = 32: contiguous). With o_rs = 32, o_ds = rows * 32 and o_hs = 4 * o_ds
    // the output is K-tiled for the next GEMM (head_dim 128, 16-bit kernel only).
    long o_ds = 0;
    const float* mask = nullptr;  // additive [mask_heads][mask_rows][sk]; mask_rows 1 or sq
    int mask_heads = 1, mask_rows = 1;
    int valid_keys = 0;           // keys >= valid_keys are excluded (0 = sk)
    // Causal: key k is visible to query q only if k <= q + (sk - sq) (the text encoder's
    // prefill mask, src/text_encoder.cpp:115-116, without reading a mask tensor). Key
    // tiles wholly above the diagonal are skipped by the head_dim-128 16-bit kernel.
    int causal = 0;
    float scale = 0.f;
    // Optional FP32 scratch for splitting a partial last query tile along the keys
    // (merged by a second launch on the same stream); calls that run concurrently
    // must not share it.
    void* split_ws = nullptr;
    size_t split_ws_bytes = 0;
};
int sdpa(const SdpaArgs& a, hipStream_t stream);
// The head_dim-128 16-bit kernel (sdpa16_dl.hip); returns 1 without launching for
// problems the general kernel in sdpa.hip has to take.
int sdpa16_d128(const SdpaArgs& a, hipStream_t stream);

// ---- bandwidth-bound kernels ------------------------------------------------------
// out = RMSNorm(x) * gamma [* (1 + scale) + shift]; FP32 statistics.
// out_k32_rows > 0 (16-bit out, width a multiple of 32): out is K-tiled as
// [width/32][out_k32_rows][32] for a GEMM that reads A through a_k32_rows.
int rmsnorm_modulate(const void* x, int x_dtype, const float* gamma, const float* shift, const float* scale,
                     int rows, int width, float eps, void* out, int out_dtype, hipStream_t s, int out_k32_rows = 0);
// out = LayerNorm(x) (non-affine) * (1 + scale) + shift.
int layernorm_modulate(const float* x, const float* shift, const float* scale, int rows, int width, float eps,
                       void* out, int out_dtype, hipStream_t s);
// Per-head RMSNorm over 128 values followed by ERNIE rotary, in place, for
// `nheads` heads of `rows` tokens at x + t*row_stride + h*128.
int qk_norm_rope(void* x, int dtype, int rows, int nheads, long row_stride, const float* gamma,
                 const float* cos_t, const float* sin_t, hipStream_t s);
// The same for the q heads (nq, gamma gq, at the row start) and the k heads (nk,
// gamma gk, at k_offset) of each row in one launch.
int qk_norm_rope_qk(void* x, int dtype, int rows, int nq, int nk, long row_stride, long k_offset, const float* gq,
                    const float* gk, const float* cos_t, const float* sin_t, hipStream_t s);
// The same in place on rows [r0, r1) whose Q / K head values are stored permuted
// (qk_stored_column order, as a QKV GEMM over permuted weights writes them): each head
// is normalised and rotated and written back in natural order. cs_t: the rows' rotary
// angles as rope_pack writes them, [rows][64] (cos, sin).
int qk_norm_rope_permuted(void* x, int dtype, int r0, int r1, int nq, int nk, long row_stride, long k_offset,
                          const float* gq, const float* gk, const float* cs_t, float eps, hipStream_t s);
// ERNIE rotary tables [rows][128] whose columns 2k and 2k + 1 repeat angle k (the layout
// src/conditioning.cpp:34-37 builds) -> out [rows][64][2] = (cos, sin) of each angle, the
// form the fused Q/K epilogue reads. Where the two columns of a pair differ (another
// table layout), both values of the pair are NaN, so such a table cannot pass unnoticed.
int rope_pack(const float* cos_t, const float* sin_t, int rows, float* out, hipStream_t s);
int gelu_inplace(void* x, int dtype, size_t n, hipStream_t s);
int residual_add(const void* a, int a_dtype, const void* b, int b_dtype, float* out, size_t n, hipStream_t s);
int euler_step(const float* x, const float* v, float delta, size_t n, float* out, hipStream_t s);
int finite_flags(const float* x, size_t n, int* flag, hipStream_t s);
// out [cols][rows] = in [rows][cols] transposed (element type dt; in and out must not overlap).
int transpose2d(const void* in, int dt, int rows, int cols, void* out, hipStream_t s);
// p[0..n) = value by a kernel (no memset node, so the clear may be captured in a graph).
int fill_int(int* p, int value, size_t n, hipStream_t s);
int convert(const void* in, int in_dtype, void* out, int out_dtype, size_t n, hipStream_t s);
int fill_normal(void* out, int dtype, size_t n, uint64_t seed, uint64_t offset, float mean, float std_dev,
                hipStream_t s);
// y[n] = act(x)[k] . W[n][k] + b[n] in FP32 accumulation (matrix-vector).
int gemv(const void* W, int w_dtype, const float* b, const float* x, int N, int K, int silu_input, float* y,
         hipStream_t s);
// latent [ch][hw] f32 -> tokens [hw][ch] in dtype.
int transpose_to_tokens(const float* latent, int ch, int hw, void* out, int dtype, hipStream_t s);
// proj [hw][ch] (f32, bias applied) -> pred [ch][hw] f32.
int tokens_to_latent(const float* proj, int hw, int ch, float* pred, hipStream_t s);

// Row-major [rows][cols] 16-bit matrix -> K-tiled [cols/32][rows][32] (the
// layout GemmArgs::w_k32 reads); in and out must not overlap. The first head_rows rows
// (a multiple of 128: the Q and K projections) are stored permuted within each 128-row
// head, row d at qk_stored_column(d) (common.hpp), the layout EPI_QKROPE reads.
int tile_k32(const void* in, void* out, int rows, int cols, hipStream_t s, int head_rows = 0);

// Up or gate matrix [rows][cols] (dtype in_dt) -> its rows of the interleaved W_ug (parity 0 = up).
int interleave_up_gate(const void* in, int in_dt, void* out, int dt, int rows, int cols, int parity, hipStream_t s);

// Matrix-core issue-rate probe (mfma_rate.hip): `workgroups` of 512 threads, each wave
// `iters` iterations of 8 independent v_mfma_f32_16x16x32_f16 from registers. sink holds
// workgroups * 512 floats; stamps 4 u64 per wave (s_memtime start / end, s_memrealtime
// start / end).
size_t mfma_rate_waves(int workgroups);
double mfma_rate_flop(int workgroups, int iters);
int launch_mfma_rate(int workgroups, int iters, float* sink, unsigned long long* stamps, hipStream_t stream);

}  // namespace ehip
