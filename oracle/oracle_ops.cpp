// SPDX-License-Identifier: MIT
// Operators, block and heads of the oracle (test infrastructure only).
// Semantics follow the reference files cited in oracle.h; the arithmetic is
// FP32 storage with FP64 reductions (norm statistics, attention when precise).
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {
int pick_threads(int threads)
{
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

typedef float v8 __attribute__((vector_size(32)));

inline v8 load8(const float* p)
{
    v8 v;
    std::memcpy(&v, p, sizeof(v));
    return v;
}
inline void store8(float* p, v8 v) { std::memcpy(p, &v, sizeof(v)); }

// R x 16 register tile: C[R][16] += A[R][kc] * Bp[kc][16].
template <int R>
inline void micro(int kc, const float* A, long lda, const float* Bp, float* C, long ldc)
{
    v8 acc[R][2];
    for (int r = 0; r < R; ++r) {
        acc[r][0] = load8(C + r * ldc);
        acc[r][1] = load8(C + r * ldc + 8);
    }
    for (int k = 0; k < kc; ++k) {
        const v8 b0 = load8(Bp + k * 16), b1 = load8(Bp + k * 16 + 8);
        for (int r = 0; r < R; ++r) {
            const float a = A[r * lda + k];
            const v8 av = {a, a, a, a, a, a, a, a};
            acc[r][0] += av * b0;
            acc[r][1] += av * b1;
        }
    }
    for (int r = 0; r < R; ++r) {
        store8(C + r * ldc, acc[r][0]);
        store8(C + r * ldc + 8, acc[r][1]);
    }
}

void micro_rows(int rows, int kc, const float* A, long lda, const float* Bp, float* C, long ldc)
{
    switch (rows) {
        case 6: micro<6>(kc, A, lda, Bp, C, ldc); break;
        case 5: micro<5>(kc, A, lda, Bp, C, ldc); break;
        case 4: micro<4>(kc, A, lda, Bp, C, ldc); break;
        case 3: micro<3>(kc, A, lda, Bp, C, ldc); break;
        case 2: micro<2>(kc, A, lda, Bp, C, ldc); break;
        case 1: micro<1>(kc, A, lda, Bp, C, ldc); break;
        default: break;
    }
}

double silu(double x) { return x / (1.0 + std::exp(-x)); }

void linear_vec(const float* W, const float* b, const float* x, int N, int K, float* y, bool silu_input, int threads)
{
    std::vector<float> in(x, x + K);
    if (silu_input)
        for (int k = 0; k < K; ++k) in[k] = float(silu(in[k]));
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static)
    for (int n = 0; n < N; ++n) {
        double acc = 0.0;
        const float* w = W + (size_t)n * K;
        for (int k = 0; k < K; ++k) acc += double(w[k]) * in[k];
        y[n] = float(acc + (b ? double(b[n]) : 0.0));
    }
}
}  // namespace

extern "C" void orc_rmsnorm(const float* x, const float* gamma, int rows, int width, float eps, float* out)
{
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* in = x + (size_t)r * width;
        double ss = 0.0;
        for (int i = 0; i < width; ++i) ss += double(in[i]) * in[i];
        const double inv = 1.0 / std::sqrt(ss / width + double(eps));
        float* o = out + (size_t)r * width;
        for (int i = 0; i < width; ++i) o[i] = float(double(in[i]) * inv * (gamma ? double(gamma[i]) : 1.0));
    }
}

extern "C" void orc_layernorm(const float* x, int rows, int width, float eps, float* out)
{
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* in = x + (size_t)r * width;
        double mean = 0.0;
        for (int i = 0; i < width; ++i) mean += in[i];
        mean /= width;
        double var = 0.0;
        for (int i = 0; i < width; ++i) var += (in[i] - mean) * (in[i] - mean);
        const double inv = 1.0 / std::sqrt(var / width + double(eps));
        float* o = out + (size_t)r * width;
        for (int i = 0; i < width; ++i) o[i] = float((in[i] - mean) * inv);
    }
}

extern "C" void orc_gemm_nt(const float* A, const float* W, const float* bias, int M, int N, int K, float* C,
                            int threads)
{
    const int KC = 256, MC = 96, NC = 128;
    const int n16 = N / 16 * 16;
    const int mblocks = (M + MC - 1) / MC, nblocks = (n16 + NC - 1) / NC;
#pragma omp parallel num_threads(pick_threads(threads))
    {
        std::vector<float> packed((size_t)NC * KC), cblk((size_t)MC * NC);
#pragma omp for collapse(2) schedule(dynamic)
        for (int jb = 0; jb < nblocks; ++jb)
            for (int ib = 0; ib < mblocks; ++ib) {
                const int j0 = jb * NC, nc = std::min(NC, n16 - j0);
                const int i0 = ib * MC, mc = std::min(MC, M - i0);
                for (int i = 0; i < mc; ++i)
                    for (int j = 0; j < nc; ++j) cblk[(size_t)i * NC + j] = bias ? bias[j0 + j] : 0.f;
                for (int p0 = 0; p0 < K; p0 += KC) {
                    const int kc = std::min(KC, K - p0);
                    // Pack W[j0 .. j0+nc][p0 .. p0+kc] into 16-column panels [kc][16].
                    for (int panel = 0; panel < nc / 16; ++panel)
                        for (int jj = 0; jj < 16; ++jj) {
                            const float* src = W + (size_t)(j0 + panel * 16 + jj) * K + p0;
                            float* dst = packed.data() + (size_t)panel * kc * 16 + jj;
                            for (int k = 0; k < kc; ++k) dst[k * 16] = src[k];
                        }
                    for (int ir = 0; ir < mc; ir += 6) {
                        const int rows = std::min(6, mc - ir);
                        for (int panel = 0; panel < nc / 16; ++panel)
                            micro_rows(rows, kc, A + (size_t)(i0 + ir) * K + p0, K,
                                       packed.data() + (size_t)panel * kc * 16, cblk.data() + (size_t)ir * NC + panel * 16,
                                       NC);
                    }
                }
                for (int i = 0; i < mc; ++i)
                    std::memcpy(C + (size_t)(i0 + i) * N + j0, cblk.data() + (size_t)i * NC, sizeof(float) * nc);
            }
        // Columns beyond the last full 16-column panel.
        if (n16 < N) {
#pragma omp for schedule(static)
            for (int i = 0; i < M; ++i)
                for (int j = n16; j < N; ++j) {
                    float acc = bias ? bias[j] : 0.f;
                    const float* a = A + (size_t)i * K;
                    const float* w = W + (size_t)j * K;
                    for (int k = 0; k < K; ++k) acc += a[k] * w[k];
                    C[(size_t)i * N + j] = acc;
                }
        }
    }
}

extern "C" void orc_gelu(const float* x, size_t n, float* out)
{
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        out[i] = 0.5f * x[i] * std::erfc(-0.7071067811865475f * x[i]);
}

// block.ncnn.param lines 29-46: first/second halves of 64, full-width tables.
extern "C" void orc_rope_rows(float* x, const float* cos_t, const float* sin_t, int rows, long row_stride,
                              long table_stride)
{
    for (int r = 0; r < rows; ++r) {
        float* v = x + (size_t)r * row_stride;
        const float* c = cos_t + (size_t)r * table_stride;
        const float* s = sin_t + (size_t)r * table_stride;
        float tmp[128];
        for (int d = 0; d < 64; ++d) {
            const float first = v[d], second = v[d + 64];
            tmp[d] = first * c[d] - second * s[d];
            tmp[d + 64] = second * c[d + 64] + first * s[d + 64];
        }
        std::memcpy(v, tmp, sizeof(tmp));
    }
}

extern "C" void orc_sdpa(const float* q, const float* k, const float* v, float* out, int heads, int kv_heads, int sq,
                         int sk, int d, long q_hs, long q_rs, long kv_hs, long kv_rs, long o_hs, long o_rs,
                         const float* mask, int mask_heads, int mask_rows, float scale, int q_begin, int q_end,
                         int precise, int threads)
{
    (void)sq;
    const int group = heads / kv_heads;
    const int rows = q_end - q_begin;
#pragma omp parallel num_threads(pick_threads(threads))
    {
        std::vector<double> pd(sk);
        std::vector<float> pf(sk);
        std::vector<double> accd(d);
        std::vector<float> accf(d);
#pragma omp for collapse(2) schedule(dynamic, 4)
        for (int h = 0; h < heads; ++h)
            for (int r = 0; r < rows; ++r) {
                const int i = q_begin + r;
                const int kh = h / group;
                const float* qi = q + h * q_hs + (long)i * q_rs;
                const float* mrow = mask ? mask + (size_t)(mask_heads == 1 ? 0 : h) * mask_rows * sk +
                                               (size_t)(mask_rows == 1 ? 0 : i) * sk
                                         : nullptr;
                float* oi = out + h * o_hs + (long)i * o_rs;
                if (precise) {
                    double m = -INFINITY;
                    for (int j = 0; j < sk; ++j) {
                        const float* kj = k + kh * kv_hs + (long)j * kv_rs;
                        double dot = 0.0;
                        for (int x = 0; x < d; ++x) dot += double(qi[x]) * kj[x];
                        double s = dot * double(scale) + (mrow ? double(mrow[j]) : 0.0);
                        pd[j] = s;
                        m = std::max(m, s);
                    }
                    double total = 0.0;
                    for (int j = 0; j < sk; ++j) {
                        pd[j] = std::exp(pd[j] - m);
                        total += pd[j];
                    }
                    std::fill(accd.begin(), accd.end(), 0.0);
                    for (int j = 0; j < sk; ++j) {
                        const float* vj = v + kh * kv_hs + (long)j * kv_rs;
                        const double p = pd[j];
                        for (int x = 0; x < d; ++x) accd[x] += p * vj[x];
                    }
                    for (int x = 0; x < d; ++x) oi[x] = float(accd[x] / total);
                } else {
                    float m = -INFINITY;
                    for (int j = 0; j < sk; ++j) {
                        const float* kj = k + kh * kv_hs + (long)j * kv_rs;
                        float dot = 0.f;
                        for (int x = 0; x < d; ++x) dot += qi[x] * kj[x];
                        const float s = dot * scale + (mrow ? mrow[j] : 0.f);
                        pf[j] = s;
                        m = std::max(m, s);
                    }
                    float total = 0.f;
                    for (int j = 0; j < sk; ++j) {
                        pf[j] = std::exp(pf[j] - m);
                        total += pf[j];
                    }
                    std::fill(accf.begin(), accf.end(), 0.f);
                    for (int j = 0; j < sk; ++j) {
                        const float* vj = v + kh * kv_hs + (long)j * kv_rs;
                        const float p = pf[j];
                        for (int x = 0; x < d; ++x) accf[x] += p * vj[x];
                    }
                    for (int x = 0; x < d; ++x) oi[x] = accf[x] / total;
                }
            }
    }
}

// block.ncnn.param (whole graph); equations tools/export_dit_block.py:49-68.
extern "C" int orc_block_forward(const orc_block_weights* w, int dim, int ffn, const float* x, const float* mods,
                                 const float* cos_t, const float* sin_t, const float* mask, int S, float* out,
                                 int precise_attention, int threads)
{
    if (!w || dim % 128 || dim <= 0 || ffn <= 0 || S < 1) return -1;
    const int heads = dim / 128;
    const size_t SD = (size_t)S * dim, SF = (size_t)S * ffn;
    const float *shift_sa = mods, *scale_sa = mods + dim, *gate_sa = mods + 2 * dim;
    const float *shift_mlp = mods + 3 * dim, *scale_mlp = mods + 4 * dim, *gate_mlp = mods + 5 * dim;
    std::vector<float> h(SD), q(SD), k(SD), vv(SD), attn(SD), x1(SD);
    // rmsn_8, add_0/mul_1/add_2
    orc_rmsnorm(x, w->norm1, S, dim, 1e-6f, h.data());
    orc_modulate(h.data(), shift_sa, scale_sa, S, dim);
    // gemm_0/1/2 (transB, no bias)
    orc_gemm_nt(h.data(), w->wq, nullptr, S, dim, dim, q.data(), threads);
    orc_gemm_nt(h.data(), w->wk, nullptr, S, dim, dim, k.data(), threads);
    orc_gemm_nt(h.data(), w->wv, nullptr, S, dim, dim, vv.data(), threads);
    // rmsn_9 / rmsn_10 over each head's 128 values, then rotary (lines 29-57).
    orc_rmsnorm(q.data(), w->norm_q, S * heads, 128, 1e-6f, q.data());
    orc_rmsnorm(k.data(), w->norm_k, S * heads, 128, 1e-6f, k.data());
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static)
    for (int hh = 0; hh < heads; ++hh) {
        orc_rope_rows(q.data() + hh * 128, cos_t, sin_t, S, dim, 128);
        orc_rope_rows(k.data() + hh * 128, cos_t, sin_t, S, dim, 128);
    }
    // sdpa_22 with the one-row additive mask broadcast over queries.
    orc_sdpa(q.data(), k.data(), vv.data(), attn.data(), heads, heads, S, S, 128, 128, dim, 128, dim, 128, dim, mask,
             1, 1, 1.0f / std::sqrt(128.0f), 0, S, precise_attention, threads);
    // gemm_3, mul_15 (gate * branch), ErnieResidualAdd add_16 in FP32.
    orc_gemm_nt(attn.data(), w->wo, nullptr, S, dim, dim, q.data(), threads);
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static)
    for (long long i = 0; i < (long long)SD; ++i) {
        const float gated = gate_sa[i % dim] * q[i];
        x1[i] = x[i] + gated;
    }
    // rmsn_11, add_17/mul_18/add_19
    orc_rmsnorm(x1.data(), w->norm2, S, dim, 1e-6f, h.data());
    orc_modulate(h.data(), shift_mlp, scale_mlp, S, dim);
    q.clear(); k.clear(); vv.clear(); attn.clear();
    q.shrink_to_fit(); k.shrink_to_fit(); vv.shrink_to_fit(); attn.shrink_to_fit();
    // gemm_4 (up), gemm_5 (gate), ErnieGELU on gate, mul_20, gemm_6 (down)
    std::vector<float> up(SF), gate(SF);
    orc_gemm_nt(h.data(), w->w_up, nullptr, S, ffn, dim, up.data(), threads);
    orc_gemm_nt(h.data(), w->w_gate, nullptr, S, ffn, dim, gate.data(), threads);
    orc_gelu(gate.data(), SF, gate.data());
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static)
    for (long long i = 0; i < (long long)SF; ++i) up[i] = up[i] * gate[i];
    gate.clear();
    gate.shrink_to_fit();
    orc_gemm_nt(up.data(), w->w_down, nullptr, S, dim, ffn, h.data(), threads);
    // mul_21, ErnieResidualAdd add_22
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static)
    for (long long i = 0; i < (long long)SD; ++i) {
        const float gated = gate_mlp[i % dim] * h[i];
        out[i] = x1[i] + gated;
    }
    return 0;
}

// heads/input/head.ncnn.param: conv_1 (1x1, bias) + transpose, gemm_0 (text, no
// bias), cat_0 (image tokens first); linear_2 -> silu_5 -> linear_3 = out1;
// silu_6 -> linear_4 -> six [dim] slices out2..out7.
extern "C" int orc_input_head(const orc_input_head_weights* w, int dim, int latent_ch, int text_dim,
                              const float* latent, int hw, const float* text, int text_tokens,
                              const float* time_features, float* x, float* c, float* mods, int threads)
{
    if (!w || dim <= 0 || hw < 1 || text_tokens < 0) return -1;
    std::vector<float> tokens((size_t)hw * latent_ch);
    for (int ch = 0; ch < latent_ch; ++ch)
        for (int t = 0; t < hw; ++t) tokens[(size_t)t * latent_ch + ch] = latent[(size_t)ch * hw + t];
    orc_gemm_nt(tokens.data(), w->x_w, w->x_b, hw, dim, latent_ch, x, threads);
    if (text_tokens > 0)
        orc_gemm_nt(text, w->text_w, nullptr, text_tokens, dim, text_dim, x + (size_t)hw * dim, threads);
    std::vector<float> t1(dim);
    linear_vec(w->t1_w, w->t1_b, time_features, dim, dim, t1.data(), false, threads);
    linear_vec(w->t2_w, w->t2_b, t1.data(), dim, dim, c, true, threads);
    linear_vec(w->mod_w, w->mod_b, c, 6 * dim, dim, mods, true, threads);
    return 0;
}

// heads/output/head.ncnn.param: linear_2 on c -> [scale | shift] (chunk_0),
// ln_1 non-affine LayerNorm, add_0/mul_1/add_2, gemm_0 (bias), crop image
// tokens, transpose to [latent_ch][hw].
extern "C" int orc_output_head(const orc_output_head_weights* w, int dim, int latent_ch, const float* x, int S,
                               int hw, const float* c, float* pred, int threads)
{
    if (!w || hw > S || hw < 1) return -1;
    std::vector<float> mm(2 * (size_t)dim);
    linear_vec(w->mod_w, w->mod_b, c, 2 * dim, dim, mm.data(), false, threads);
    std::vector<float> y((size_t)hw * dim);
    orc_layernorm(x, hw, dim, 1e-6f, y.data());
    orc_modulate(y.data(), mm.data() + dim, mm.data(), hw, dim);
    std::vector<float> proj((size_t)hw * latent_ch);
    orc_gemm_nt(y.data(), w->proj_w, w->proj_b, hw, latent_ch, dim, proj.data(), threads);
    for (int t = 0; t < hw; ++t)
        for (int ch = 0; ch < latent_ch; ++ch) pred[(size_t)ch * hw + t] = proj[(size_t)t * latent_ch + ch];
    return 0;
}

extern "C" void orc_silu(const float* x, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + std::exp(-x[i]));
}

// tests/fixtures/text-s64.ncnn.param: rmsn_8 -> gemm_0/1/2 -> rotary (Slice/BinaryOp
// lines 18-44) -> sdpa_20 (GQA, mask in3) -> gemm_3 -> add_12 -> rmsn_9 -> gemm_4
// (gate) -> silu_7, gemm_5 (up), mul_13 -> gemm_6 -> add_14.
extern "C" int orc_text_block_forward(const orc_text_block_weights* w, int hidden, int heads, int kv_heads, int ffn,
                                      const float* x, const float* cos_t, const float* sin_t, const float* mask,
                                      int S, float* out, int precise_attention, int threads)
{
    if (!w || hidden <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || ffn <= 0 || S < 1) return -1;
    const int qd = heads * 128, kvd = kv_heads * 128;
    const size_t SH = (size_t)S * hidden, SF = (size_t)S * ffn;
    std::vector<float> h(SH), q((size_t)S * qd), k((size_t)S * kvd), v((size_t)S * kvd), attn((size_t)S * qd),
        x1(SH);
    orc_rmsnorm(x, w->norm1, S, hidden, 1e-5f, h.data());
    orc_gemm_nt(h.data(), w->wq, nullptr, S, qd, hidden, q.data(), threads);
    orc_gemm_nt(h.data(), w->wk, nullptr, S, kvd, hidden, k.data(), threads);
    orc_gemm_nt(h.data(), w->wv, nullptr, S, kvd, hidden, v.data(), threads);
    for (int hh = 0; hh < heads; ++hh) orc_rope_rows(q.data() + hh * 128, cos_t, sin_t, S, qd, 128);
    for (int hh = 0; hh < kv_heads; ++hh) orc_rope_rows(k.data() + hh * 128, cos_t, sin_t, S, kvd, 128);
    orc_sdpa(q.data(), k.data(), v.data(), attn.data(), heads, kv_heads, S, S, 128, 128, qd, 128, kvd, 128, qd, mask,
             1, mask ? S : 1, 1.0f / std::sqrt(128.0f), 0, S, precise_attention, threads);
    orc_gemm_nt(attn.data(), w->wo, nullptr, S, hidden, qd, h.data(), threads);
    for (size_t i = 0; i < SH; ++i) x1[i] = x[i] + h[i];
    orc_rmsnorm(x1.data(), w->norm2, S, hidden, 1e-5f, h.data());
    std::vector<float> gate(SF), up(SF);
    orc_gemm_nt(h.data(), w->w_gate, nullptr, S, ffn, hidden, gate.data(), threads);
    orc_gemm_nt(h.data(), w->w_up, nullptr, S, ffn, hidden, up.data(), threads);
    orc_silu(gate.data(), SF, gate.data());
    for (size_t i = 0; i < SF; ++i) up[i] = gate[i] * up[i];
    orc_gemm_nt(up.data(), w->w_down, nullptr, S, hidden, ffn, h.data(), threads);
    for (size_t i = 0; i < SH; ++i) out[i] = x1[i] + h[i];
    return 0;
}
