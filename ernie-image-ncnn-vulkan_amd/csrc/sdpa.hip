// SPDX-License-Identifier: MIT
// Fused masked SDPA, O = softmax(Q K^T * scale + mask) V, for gfx950.
// Replaces ErnieSDPA / AccurateSDPA (src/ernie_attention.cpp:35-233), including
// the one-row additive mask broadcast over queries (src/ernie_attention.cpp:201-221)
// and GQA (kv head = h / (heads / kv_heads)). No score matrix is materialised, so
// the reference's query-row chunking (set_attention_query_rows) is unnecessary.
//
// 16-bit problems with head_dim 128 and no per-query mask go to sdpa16_dl.hip; the
// kernels below take the rest (FP32, other head sizes, per-query masks).
// Work split: one workgroup = 4 waves = 128 queries of one head; K/V tiles of 64
// keys are staged in double-buffered LDS. Each wave computes S^T = K Q^T for its
// 32 queries (MFMA M = keys, N = queries), so every lane ends up owning one query
// column: the softmax statistics need one cross-lane exchange (lanes l, l^32),
// and the probabilities are already in the B-operand layout of O^T = V^T P^T.
// V is stored transposed in LDS ([d][key]) so the A operand of that product is two
// ds_read_b64 per MFMA.
//
// FP32 kernel: v_mfma_f32_32x32x2_f32; each 64-key tile is reduced in a fresh FP32
// accumulator and added to FP64 running sums, which keeps long (4k+ key) softmax
// sums and P.V products accurate (the reference compensates the same two sums
// with Kahan accumulation, cmake/ErnieAttentionShader.cmake:14-55).
#include "common.hpp"
#include "kernels.hpp"

namespace ehip {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int BQ = 128, BKV = 64;
constexpr int KS_STRIDE = 128 + 8;  // halves, K tile row (one key)
constexpr int VT_STRIDE = BKV + 8;  // halves, transposed V row (one d)

struct SdpaParams {
    const void* q; const void* k; const void* v; void* o;
    int heads, group, sq, sk, d, kv_end;
    int causal, qk_off;  // causal: keys > query + qk_off (= sk - sq) excluded
    long q_hs, q_rs, k_hs, k_rs, v_hs, v_rs, o_hs, o_rs;
    const float* mask; long mask_hs; long mask_rs;
    float scale_log2;
    int vec_ok;
};

template <typename T> struct Mfma16;
template <> struct Mfma16<f16> {
    typedef f16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma16<bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// 8 consecutive elements starting at column c8*8 of a row of length d (zero past d).
// FAST: d == 128 and every row / head stride and base is 16-byte aligned.
template <typename T, bool FAST>
__device__ __forceinline__ u32x4 load_row8(const T* row, int c8, int d)
{
    if constexpr (FAST) {
        return *reinterpret_cast<const u32x4*>(row + c8 * 8);
    } else {
        const int c = c8 * 8;
        union { u32x4 u; T e[8]; } r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.e[i] = (c + i < d) ? row[c + i] : T(0.f);
        return r.u;
    }
}

// Keys of one 64-key tile owned by lane (lrow, g) in register r of S^T subtile t.
__device__ __forceinline__ int tile_key(int t, int r, int g) { return 32 * t + 8 * (r >> 2) + 4 * g + (r & 3); }

// Rescale threshold (log2 units): the running maximum used for exp2 is only
// raised when a tile's maximum exceeds it by more than this, so P <= 2^8 and the
// O / l rescale is skipped for almost every tile. Exact: O and l share the offset.
constexpr float kRescaleSlack = 8.0f;

// Mask modes: none, one additive row broadcast over queries (staged in LDS per
// tile), or one additive row per query (read by each lane).
enum MaskMode : int { MASK_NONE = 0, MASK_ROW = 1, MASK_PER_QUERY = 2 };

template <typename T, bool FAST, int MM>
__global__ void __launch_bounds__(256, 2) sdpa16_kernel(SdpaParams p)
{
    typedef typename Mfma16<T>::vec vec8;
    __shared__ __attribute__((aligned(16))) T Ks[2][BKV * KS_STRIDE];
    __shared__ __attribute__((aligned(16))) T Vt[2][128 * VT_STRIDE];
    __shared__ float Ms[2][BKV];

    // XCD-aware placement: the 8 XCDs each take a contiguous range of (head,
    // query tile) pairs, so a head's K/V stream from HBM into one XCD's L2.
    const int qtiles = (p.sq + BQ - 1) / BQ;
    const int total = qtiles * p.heads;
    int logical = blockIdx.x;
    if ((total & 7) == 0) logical = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int h = logical / qtiles;
    const int q_base = (logical - h * qtiles) * BQ;
    const int kvh = h / p.group;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lrow = lane & 31, g = lane >> 5;
    const int my_q = q_base + wave * 32 + lrow;

    const T* Q = static_cast<const T*>(p.q) + (size_t)h * p.q_hs;
    const T* K = static_cast<const T*>(p.k) + (size_t)kvh * p.k_hs;
    const T* V = static_cast<const T*>(p.v) + (size_t)kvh * p.v_hs;

    // Q fragments: B operand of S^T = K Q^T (k = d): lane holds query lrow, d 16s+8g..+7.
    vec8 qf[8];
    {
        const T* qrow = Q + (size_t)min(my_q, p.sq - 1) * p.q_rs;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(vec8, load_row8<T, FAST>(qrow, 2 * s + g, p.d));
    }

    // Tile loaders. K: thread -> (key = tid/16 + 16*pass, chunk = tid%16).
    // V: thread -> (key pair kp = tid/16 + 16*pass, chunk = tid%16), stored transposed.
    const int ld_chunk = tid & 15, ld_key = tid >> 4;
    u32x4 kreg[4], vreg[2][2];
    float mreg = 0.f;
    auto load_global = [&](int kv0) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int key = min(kv0 + ld_key + 16 * s, p.sk - 1);
            kreg[s] = load_row8<T, FAST>(K + (size_t)key * p.k_rs, ld_chunk, p.d);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int key = min(kv0 + 2 * (ld_key + 16 * s) + e, p.sk - 1);
                vreg[s][e] = load_row8<T, FAST>(V + (size_t)key * p.v_rs, ld_chunk, p.d);
            }
        if constexpr (MM == MASK_ROW) {
            if (tid < BKV) {
                const int key = kv0 + tid;
                mreg = key < p.sk ? p.mask[(size_t)h * p.mask_hs + key] : 0.f;
            }
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            *reinterpret_cast<u32x4*>(&Ks[buf][(ld_key + 16 * s) * KS_STRIDE + ld_chunk * 8]) = kreg[s];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kp = ld_key + 16 * s;
#pragma unroll
            for (int ii = 0; ii < 8; ++ii) {
                // Rotate the d order by chunk to spread the transposed stores over banks.
                const int i = (ii + ld_chunk) & 7;
                const uint32_t a = vreg[s][0][i >> 1], b = vreg[s][1][i >> 1];
                const uint32_t packed = __builtin_amdgcn_perm(b, a, (i & 1) ? 0x07060302u : 0x05040100u);
                *reinterpret_cast<uint32_t*>(&Vt[buf][(ld_chunk * 8 + i) * VT_STRIDE + 2 * kp]) = packed;
            }
        }
        if constexpr (MM == MASK_ROW) {
            if (tid < BKV) Ms[buf][tid] = mreg * kLog2e;
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float c = p.scale_log2;
    const float* qmask = MM == MASK_PER_QUERY
                             ? p.mask + (size_t)h * p.mask_hs + (size_t)min(my_q, p.sq - 1) * p.mask_rs
                             : nullptr;
    constexpr bool MASK = MM != MASK_NONE;
    // Keys at or past lim are excluded: the valid-key bound, and the diagonal when causal.
    const int lim = p.causal ? min(p.kv_end, my_q + 1 + p.qk_off) : p.kv_end;

    const int ntiles = (p.kv_end + BKV - 1) / BKV;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int buf = it & 1;
        const int kv0 = it * BKV;
        if (it + 1 < ntiles) load_global(kv0 + BKV);

        // S^T tile: 64 keys x 32 queries as two 32x32 MFMA outputs.
        f32x16 sacc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[t][r] = 0.f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const vec8 kf =
                    *reinterpret_cast<const vec8*>(&Ks[buf][(t * 32 + lrow) * KS_STRIDE + s * 16 + g * 8]);
                sacc[t] = Mfma16<T>::run(kf, qf[s], sacc[t]);
            }
        }
        // Scores in log2 units: s * c (+ mask * log2 e); keys >= kv_end excluded.
        const bool partial = kv0 + BKV > p.kv_end || p.causal;
        if (MASK || partial) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kk = tile_key(t, r, g);
                    float v = sacc[t][r] * c;
                    if constexpr (MM == MASK_ROW) v += Ms[buf][kk];
                    if constexpr (MM == MASK_PER_QUERY) v += (kv0 + kk < p.sk ? qmask[kv0 + kk] : 0.f) * kLog2e;
                    sacc[t][r] = kv0 + kk < lim ? v : -INFINITY;
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; r += 2) tmax = fmaxf(tmax, fmaxf(sacc[t][r], sacc[t][r + 1]));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        if (!(MASK || partial)) tmax *= c;  // unscaled scores: c > 0 preserves the order
        // Raise the running offset only past the slack (wave-uniform decision).
        const bool raise = tmax > m_run + kRescaleSlack;
        if (__any(raise)) {
            const float m_new = raise ? tmax : m_run;
            const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
            m_run = m_new;
        }
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float psum = 0.f;
        vec8 pf[2][2];
        if (MASK || partial) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = exp2f(sacc[t][r] - m_use);
                    psum += pv;
                    pf[t][r >> 3][r & 7] = T(pv);
                }
        } else {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = exp2f(__builtin_fmaf(sacc[t][r], c, -m_use));
                    psum += pv;
                    pf[t][r >> 3][r & 7] = T(pv);
                }
        }
        psum += __shfl_xor(psum, 32, 64);
        l_run += psum;

        // O^T += V^T P^T: A operand = V^T[d][keys], keys matching pf's layout.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int kk = 32 * t + 16 * hh + 4 * g;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const T* vrow = &Vt[buf][(dt * 32 + lrow) * VT_STRIDE];
                    const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + kk);
                    const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + kk + 8);
                    const u32x4 packed = {lo[0], lo[1], hi[0], hi[1]};
                    oacc[dt] = Mfma16<T>::run(__builtin_bit_cast(vec8, packed), pf[t][hh], oacc[dt]);
                }
            }
        if (it + 1 < ntiles) store_lds(buf ^ 1);
        __syncthreads();
    }

    if (my_q >= p.sq) return;
    const float inv = 1.f / l_run;
    T* orow = static_cast<T*>(p.o) + (size_t)h * p.o_hs + (size_t)my_q * p.o_rs;
    // O^T accumulator: register r of subtile dt holds d = 32dt + 8(r/4) + 4g + r%4.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const int d0 = 32 * dt + 8 * rq + 4 * g;
            if constexpr (FAST) {
                union { u32x2 u; T e[4]; } pk;
#pragma unroll
                for (int e = 0; e < 4; ++e) pk.e[e] = T(oacc[dt][4 * rq + e] * inv);
                *reinterpret_cast<u32x2*>(orow + d0) = pk.u;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < p.d) orow[d0 + e] = T(oacc[dt][4 * rq + e] * inv);
            }
        }
}

// ---------------------------------------------------------------------------------
// FP32
// ---------------------------------------------------------------------------------
constexpr int KS32 = 128 + 4;  // floats per staged K / V row

__device__ __forceinline__ f32x4 load_row4(const float* row, int c4, int d, int vec_ok)
{
    const int c = c4 * 4;
    if (vec_ok && c + 4 <= d) return *reinterpret_cast<const f32x4*>(row + c);
    f32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (c + i < d) ? row[c + i] : 0.f;
    return r;
}

__global__ void __launch_bounds__(256) sdpa32_kernel(SdpaParams p)
{
    __shared__ __attribute__((aligned(16))) float Ks[BKV * KS32];
    __shared__ __attribute__((aligned(16))) float Vs[BKV * KS32];

    const int h = blockIdx.y;
    const int kvh = h / p.group;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lrow = lane & 31, g = lane >> 5;
    const int my_q = blockIdx.x * BQ + wave * 32 + lrow;

    const float* Q = static_cast<const float*>(p.q) + (size_t)h * p.q_hs;
    const float* K = static_cast<const float*>(p.k) + (size_t)kvh * p.k_hs;
    const float* V = static_cast<const float*>(p.v) + (size_t)kvh * p.v_hs;

    // Q fragments: chunk c of 8 d values; lane group g supplies d = 8c + 4g + j to MFMA j.
    f32x4 qf[16];
    {
        const float* qrow = Q + (size_t)min(my_q, p.sq - 1) * p.q_rs;
#pragma unroll
        for (int c = 0; c < 16; ++c) qf[c] = load_row4(qrow, 2 * c + g, p.d, p.vec_ok);
    }
    // Loader: thread -> (key = tid/32 + 8*pass, chunk = tid%32 of 4 floats).
    const int ld_chunk = tid & 31, ld_key = tid >> 5;
    f32x4 kreg[8], vreg[8];
    auto load_global = [&](int kv0) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int key = min(kv0 + ld_key + 8 * s, p.sk - 1);
            kreg[s] = load_row4(K + (size_t)key * p.k_rs, ld_chunk, p.d, p.vec_ok);
            vreg[s] = load_row4(V + (size_t)key * p.v_rs, ld_chunk, p.d, p.vec_ok);
        }
    };
    auto store_lds = [&]() {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            *reinterpret_cast<f32x4*>(&Ks[(ld_key + 8 * s) * KS32 + ld_chunk * 4]) = kreg[s];
            *reinterpret_cast<f32x4*>(&Vs[(ld_key + 8 * s) * KS32 + ld_chunk * 4]) = vreg[s];
        }
    };

    double o_run[4][16];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_run[t][r] = 0.0;
    float m_run = -INFINITY;
    double l_run = 0.0;
    const float* mrow = p.mask ? p.mask + (size_t)h * p.mask_hs + (size_t)min(my_q, p.sq - 1) * p.mask_rs : nullptr;
    const int lim = p.causal ? min(p.kv_end, my_q + 1 + p.qk_off) : p.kv_end;

    const int ntiles = (p.kv_end + BKV - 1) / BKV;
    load_global(0);
    for (int it = 0; it < ntiles; ++it) {
        const int kv0 = it * BKV;
        __syncthreads();  // previous tile fully consumed
        store_lds();
        __syncthreads();
        if (it + 1 < ntiles) load_global(kv0 + BKV);

        f32x16 sacc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[t][r] = 0.f;
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const f32x4 kf = *reinterpret_cast<const f32x4*>(&Ks[(t * 32 + lrow) * KS32 + c * 8 + g * 4]);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    sacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j], qf[c][j], sacc[t], 0, 0, 0);
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kv0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
                float s = sacc[t][r] * p.scale_log2;
                if (mrow) s += (key < p.sk ? mrow[key] : 0.f) * kLog2e;
                s = key < lim ? s : -INFINITY;
                sacc[t][r] = s;
                tmax = fmaxf(tmax, s);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const double alpha = (double)exp2f(m_run - m_use);
        float psum = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sacc[t][r] = exp2f(sacc[t][r] - m_use);
                psum += sacc[t][r];
            }
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + (double)psum;
        m_run = m_new;
        // Tile partial O^T in FP32, then folded into the FP64 running sum.
        f32x16 part[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) part[dt][r] = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const float vv = Vs[key * KS32 + dt * 32 + lrow];
                    part[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, sacc[t][r], part[dt], 0, 0, 0);
                }
            }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o_run[dt][r] = o_run[dt][r] * alpha + (double)part[dt][r];
    }
    if (my_q >= p.sq) return;
    float* orow = static_cast<float*>(p.o) + (size_t)h * p.o_hs + (size_t)my_q * p.o_rs;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dd = 32 * dt + 8 * (r >> 2) + 4 * g + (r & 3);
            if (dd < p.d) orow[dd] = float(o_run[dt][r] / l_run);
        }
}

}  // namespace

int sdpa(const SdpaArgs& a, hipStream_t s)
{
    if (!a.q || !a.k || !a.v || !a.o) return -1;
    if (a.heads < 1 || a.kv_heads < 1 || a.heads % a.kv_heads || a.sq < 1 || a.sk < 1) return -1;
    if (a.d < 1 || a.d > 128) return -1;
    if (a.dtype != DT_F32 && a.dtype != DT_F16 && a.dtype != DT_BF16) return -1;
    if (a.mask && (a.mask_rows != 1 && a.mask_rows != a.sq)) return -1;
    if (a.mask && a.mask_heads != 1 && a.mask_heads != a.heads) return -1;
    const int kv_end = a.valid_keys > 0 ? a.valid_keys : a.sk;
    if (kv_end > a.sk) return -1;
    if (a.causal && a.sq > a.sk) return -1;  // every query must see at least key 0
    if (a.o_ds != 0 && a.o_ds != 32 && (a.dtype == DT_F32 || a.d != 128 || a.o_ds % 8)) return -1;
    SdpaParams p{};
    p.q = a.q; p.k = a.k; p.v = a.v; p.o = a.o;
    p.heads = a.heads; p.group = a.heads / a.kv_heads; p.sq = a.sq; p.sk = a.sk; p.d = a.d; p.kv_end = kv_end;
    p.causal = a.causal ? 1 : 0; p.qk_off = a.sk - a.sq;
    p.q_hs = a.q_hs; p.q_rs = a.q_rs; p.k_hs = a.k_hs; p.k_rs = a.k_rs;
    p.v_hs = a.v_hs; p.v_rs = a.v_rs; p.o_hs = a.o_hs; p.o_rs = a.o_rs;
    p.mask = a.mask;
    p.mask_hs = a.mask && a.mask_heads > 1 ? (long)a.mask_rows * a.sk : 0;
    p.mask_rs = a.mask && a.mask_rows > 1 ? a.sk : 0;
    const float scale = a.scale > 0.f ? a.scale : 1.f / sqrtf((float)a.d);
    p.scale_log2 = scale * kLog2e;
    const long vec = a.dtype == DT_F32 ? 4 : 8;
    const uintptr_t bases = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                            reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.o);
    p.vec_ok = (bases % 16 == 0) && a.q_hs % vec == 0 && a.q_rs % vec == 0 && a.k_hs % vec == 0 &&
               a.k_rs % vec == 0 && a.v_hs % vec == 0 && a.v_rs % vec == 0 && a.o_hs % vec == 0 &&
               a.o_rs % vec == 0;
    const dim3 block(256);
    if (a.dtype == DT_F32) {
        hipLaunchKernelGGL(sdpa32_kernel, dim3((a.sq + BQ - 1) / BQ, a.heads), block, 0, s, p);
    } else if (const int rc = sdpa16_d128(a, s); rc != 1) {
        return rc;
    } else if (a.o_ds != 0 && a.o_ds != 32) {
        return -1;  // only the head_dim-128 kernel writes grouped (K-tiled) output rows
    } else {
        const bool fast = p.vec_ok && a.d == 128;
        const int mm = !a.mask ? MASK_NONE : (a.mask_rows > 1 ? MASK_PER_QUERY : MASK_ROW);
        const dim3 grid(((a.sq + BQ - 1) / BQ) * a.heads);
#define EHIP_SDPA16(T)                                                                                     \
    do {                                                                                                   \
        if (fast) {                                                                                        \
            if (mm == MASK_NONE) hipLaunchKernelGGL((sdpa16_kernel<T, true, MASK_NONE>), grid, block, 0, s, p); \
            else if (mm == MASK_ROW) hipLaunchKernelGGL((sdpa16_kernel<T, true, MASK_ROW>), grid, block, 0, s, p); \
            else hipLaunchKernelGGL((sdpa16_kernel<T, true, MASK_PER_QUERY>), grid, block, 0, s, p);      \
        } else {                                                                                           \
            if (mm == MASK_NONE) hipLaunchKernelGGL((sdpa16_kernel<T, false, MASK_NONE>), grid, block, 0, s, p); \
            else if (mm == MASK_ROW) hipLaunchKernelGGL((sdpa16_kernel<T, false, MASK_ROW>), grid, block, 0, s, p); \
            else hipLaunchKernelGGL((sdpa16_kernel<T, false, MASK_PER_QUERY>), grid, block, 0, s, p);     \
        }                                                                                                  \
    } while (0)
        if (a.dtype == DT_F16) EHIP_SDPA16(f16);
        else EHIP_SDPA16(bf16);
#undef EHIP_SDPA16
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -int(e);
}

}  // namespace ehip
