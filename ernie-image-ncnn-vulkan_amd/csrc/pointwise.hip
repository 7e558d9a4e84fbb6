// SPDX-License-Identifier: MIT
// Bandwidth-bound kernels of the DiT block and denoise loop (gfx950).
//   rmsnorm_modulate ... ErnieRMSNorm (src/ernie_rmsnorm.cpp:21-135, FP32 statistics)
//                        fused with the adaLN BinaryOps add_0/mul_1/add_2 (param 15-17)
//   layernorm_modulate . output head ln_1 + add_0/mul_1/add_2 (heads/output head.ncnn.param)
//   qk_norm_rope ....... rmsn_9/rmsn_10 + the rotary BinaryOps (param 28-57), in place
//   gelu_inplace ....... ErnieGELU (src/ernie_gelu.cpp:49-61)
//   residual_add ....... ErnieResidualAdd (src/ernie_residual.cpp:62-88), FP32 result
//   euler_step ......... Euler x + delta*v with two roundings (src/latent_ops.cpp:72-92)
//   finite_flags ....... finite_latent (src/latent_ops.cpp:60-70)
#include "common.hpp"
#include "kernels.hpp"

namespace ehip {
namespace {

template <typename T> struct Vec4;
template <> struct Vec4<float> {
    static __device__ __forceinline__ f32x4 load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
    // Streaming load (nontemporal): the value is read once, so it should not displace
    // what the caches hold.
    static __device__ __forceinline__ f32x4 load_stream(const float* p)
    {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    }
    static __device__ __forceinline__ void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <typename T> struct Vec4 {
    typedef T t4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 load(const T* p)
    {
        const t4 v = *reinterpret_cast<const t4*>(p);
        return f32x4{float(v[0]), float(v[1]), float(v[2]), float(v[3])};
    }
    static __device__ __forceinline__ f32x4 load_stream(const T* p)
    {
        const t4 v = __builtin_nontemporal_load(reinterpret_cast<const t4*>(p));
        return f32x4{float(v[0]), float(v[1]), float(v[2]), float(v[3])};
    }
    static __device__ __forceinline__ void store(T* p, f32x4 v)
    {
        t4 o;
        o[0] = T(v[0]); o[1] = T(v[1]); o[2] = T(v[2]); o[3] = T(v[3]);
        *reinterpret_cast<t4*>(p) = o;
    }
};

__device__ __forceinline__ float block_sum(float v, float* red)
{
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
    return t;
}

// One 256-thread block per row; width % 4 == 0 and width <= 4 * 256 * kMaxPer
// (the layernorm kernel below keeps this shape).
constexpr int kMaxPer = 4;  // float4 groups per thread -> width up to 4096

// RMSNorm + modulate over rows of `width` values, one wave per row. Each
// workgroup first folds gamma * (1 + scale) and shift into LDS, so every row
// reads only its own values from memory (the per-column vectors are read once
// per workgroup instead of once per row); no workgroup barrier inside the row
// loop, the statistics are a single wave reduction.
constexpr int kRowWaves = 4, kRowMaxWidth = 4096;
// Element (r, c) of a [rows][width] output: row-major, or K-tiled as
// [width/32][out_rows][32] when out_rows > 0 (four-value groups never straddle a
// 32-column slab).
__device__ __forceinline__ size_t out_index(int r, int c, int width, int out_rows)
{
    return out_rows ? ((size_t)(c >> 5) * out_rows + r) * 32 + (c & 31) : (size_t)r * width + c;
}
template <typename TIn, typename TOut>
__global__ void __launch_bounds__(256) rmsnorm_rows_kernel(const TIn* __restrict__ x, const float* __restrict__ gamma,
                                                           const float* __restrict__ shift,
                                                           const float* __restrict__ scale, int rows, int width,
                                                           int rows_per_block, float eps, TOut* __restrict__ out,
                                                           int out_rows)
{
    __shared__ f32x4 mul4[kRowMaxWidth / 4], add4[kRowMaxWidth / 4];
    const int w4 = width >> 2;
    for (int c4 = threadIdx.x; c4 < w4; c4 += blockDim.x) {
        f32x4 m, a;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = 4 * c4 + e;
            const float g = gamma ? gamma[c] : 1.0f;
            m[e] = scale ? g * (scale[c] + 1.0f) : g;
            a[e] = shift ? shift[c] : 0.0f;
        }
        mul4[c4] = m;
        add4[c4] = a;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r_end = min((blockIdx.x + 1) * rows_per_block, rows);
    for (int r = blockIdx.x * rows_per_block + wave; r < r_end; r += kRowWaves) {
        const TIn* xr = x + (size_t)r * width;
        f32x4 v[kRowMaxWidth / 256];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kRowMaxWidth / 256; ++i) {
            const int c4 = lane + 64 * i;
            if (c4 < w4) {
                v[i] = Vec4<TIn>::load(xr + 4 * c4);
                ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
            }
        }
        const float inv = 1.0f / sqrtf(wave_sum(ss) / float(width) + eps);
#pragma unroll
        for (int i = 0; i < kRowMaxWidth / 256; ++i) {
            const int c4 = lane + 64 * i;
            if (c4 < w4) {
                const f32x4 m = mul4[c4], a = add4[c4];
                f32x4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = (v[i][e] * inv) * m[e] + a[e];
                Vec4<TOut>::store(out + out_index(r, 4 * c4, width, out_rows), y);
            }
        }
    }
}

// Same operation for widths of PER x 1024 (the block width 4096 has PER = 4):
// persistent 256-thread workgroups striding over the rows. Thread t owns the
// four-column groups t + 256 i, so its factors gamma (1 + scale) and shift stay
// in registers for every row it touches, and the next row's load is in flight
// while this row is reduced (wave sums, then the four wave partials through a
// double-buffered LDS slot: one barrier per row) and stored.
template <typename TIn, typename TOut, int PER>
__global__ void __launch_bounds__(256) rmsnorm_persist_kernel(const TIn* __restrict__ x,
                                                              const float* __restrict__ gamma,
                                                              const float* __restrict__ shift,
                                                              const float* __restrict__ scale, int rows, float eps,
                                                              TOut* __restrict__ out, int out_rows)
{
    constexpr int width = PER * 1024;
    __shared__ float red[2][4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    f32x4 m[PER], a[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int c = 4 * (tid + 256 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float g = gamma ? gamma[c + e] : 1.0f;
            m[i][e] = scale ? g * (scale[c + e] + 1.0f) : g;
            a[i][e] = shift ? shift[c + e] : 0.0f;
        }
    }
    int r = blockIdx.x;
    f32x4 v[PER];
    if (r < rows) {
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = Vec4<TIn>::load(x + (size_t)r * width + 4 * (tid + 256 * i));
    }
    for (int it = 0; r < rows; r += gridDim.x, ++it) {
        const int rn = r + gridDim.x;
        f32x4 vn[PER];
        if (rn < rows) {
#pragma unroll
            for (int i = 0; i < PER; ++i) vn[i] = Vec4<TIn>::load(x + (size_t)rn * width + 4 * (tid + 256 * i));
        }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        ss = wave_sum(ss);
        if (lane == 0) red[it & 1][wave] = ss;
        __syncthreads();
        const float tot = (red[it & 1][0] + red[it & 1][1]) + (red[it & 1][2] + red[it & 1][3]);
        const float inv = 1.0f / sqrtf(tot / float(width) + eps);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = (v[i][e] * inv) * m[i][e] + a[i][e];
            Vec4<TOut>::store(out + out_index(r, 4 * (tid + 256 * i), width, out_rows), y);
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = vn[i];
    }
}

// The same operation writing K-tiled output ([width/32][out_rows][32]) for widths
// of NI x 512: persistent workgroups take rows in pairs (r0 even, r0 + 1), so each
// store instruction covers, per 32-column slab, both rows' 64 bytes, which are
// adjacent in the tiled layout: four whole 128-byte lines per instruction. Lane l of
// wave w holds row r0 + (l / 8 % 2) and columns 32 s + 4 (l % 8) .. + 3 of slabs
// s = 4 (w + 4 i) + l / 16, i < NI. The per-column factors gamma (1 + scale) and
// shift are folded into LDS once per workgroup rather than held in registers: at
// 116 VGPRs four workgroups share a CU, which keeps enough row loads in flight to
// stream at close to copy bandwidth (holding them in registers, 178 VGPRs, halved
// the workgroups per CU and the achieved bandwidth). The rows are read with streaming
// (nontemporal) loads, issued before the factors are staged: with the rows not
// resident in the caches, as after the GEMM that wrote them, that measured 23-24 us
// against 31-32 us for ordinary loads at 4160 x 4096.
template <typename TIn, typename TOut, int NI>
__global__ void __launch_bounds__(256) rmsnorm_pair_k32_kernel(const TIn* __restrict__ x,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ shift,
                                                               const float* __restrict__ scale, int rows, float eps,
                                                               TOut* __restrict__ out, int out_rows)
{
    constexpr int width = NI * 512;
    __shared__ f32x4 mul_l[width / 4], add_l[width / 4];
    __shared__ float red[2][4][2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, b = (lane >> 3) & 1;
    int col[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) col[i] = 32 * (4 * (wave + 4 * i) + (lane >> 4)) + 4 * (lane & 7);
    const int pairs = (rows + 1) >> 1;
    int pr = blockIdx.x;
    f32x4 v[NI];
    auto load = [&](int pair) {
        const int r = 2 * pair + b;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            v[i] = r < rows ? Vec4<TIn>::load_stream(x + (size_t)r * width + col[i]) : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    if (pr < pairs) load(pr);  // in flight while the factors are staged
    for (int j = tid; j < width / 4; j += 256) {
        f32x4 m, a;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = 4 * j + e;
            const float g = gamma ? gamma[c] : 1.0f;
            m[e] = scale ? g * (scale[c] + 1.0f) : g;
            a[e] = shift ? shift[c] : 0.0f;
        }
        mul_l[j] = m;
        add_l[j] = a;
    }
    __syncthreads();  // the LDS factors are in place
    for (int it = 0; pr < pairs; pr += gridDim.x, ++it) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        // Sum over the 32 lanes of this wave that hold the same row (lane bit 3 fixed).
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        ss += __shfl_xor(ss, 4, 64);
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if ((lane & ~8) == 0) red[it & 1][wave][b] = ss;
        __syncthreads();
        const float tot = (red[it & 1][0][b] + red[it & 1][1][b]) + (red[it & 1][2][b] + red[it & 1][3][b]);
        const float inv = 1.0f / sqrtf(tot / float(width) + eps);
        const int r = 2 * pr + b;
        if (r < rows) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const f32x4 m = mul_l[col[i] >> 2], a = add_l[col[i] >> 2];
                f32x4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = (v[i][e] * inv) * m[e] + a[e];
                Vec4<TOut>::store(out + ((size_t)(col[i] >> 5) * out_rows + r) * 32 + (col[i] & 31), y);
            }
        }
        if (pr + (int)gridDim.x < pairs) load(pr + gridDim.x);
    }
}

template <typename TOut>
__global__ void __launch_bounds__(256) layernorm_mod_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ shift,
                                                            const float* __restrict__ scale, int width, float eps,
                                                            TOut* __restrict__ out)
{
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const float* xr = x + row * width;
    f32x4 v[kMaxPer];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = (threadIdx.x + i * 256) * 4;
        if (c < width) {
            v[i] = Vec4<float>::load(xr + c);
            s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
        }
    }
    const float mean = block_sum(s, red) / float(width);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = (threadIdx.x + i * 256) * 4;
        if (c < width)
#pragma unroll
            for (int e = 0; e < 4; ++e) q += (v[i][e] - mean) * (v[i][e] - mean);
    }
    const float inv = 1.0f / sqrtf(block_sum(q, red) / float(width) + eps);
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = (threadIdx.x + i * 256) * 4;
        if (c < width) {
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = (v[i][e] - mean) * inv * (scale[c + e] + 1.0f) + shift[c + e];
            Vec4<TOut>::store(out + row * width + c, y);
        }
    }
}

// Per-head RMSNorm over 128 values + ERNIE rotary, in place, for one token row
// per workgroup: the q heads (gamma gq, at the row start) and then the k heads
// (gamma gk, at k_offset). A head is handled by 16 lanes, lane l owning values
// [4l, 4l+4) and [64+4l, 64+4l+4), the rotary pairs (d, d+64); the token's cos /
// sin and the two gammas are loaded once per lane and reused for every head. A NULL
// gamma skips the norm of its heads: rotary only (the text block has no Q/K norm).
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(T* __restrict__ x, int nq, int nk, long row_stride,
                                                           long k_offset, const float* __restrict__ gq,
                                                           const float* __restrict__ gk,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t)
{
    const size_t t = blockIdx.x;
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int slot = threadIdx.x >> 4;  // 16 heads in flight per workgroup
    const int d = 4 * l;
    const f32x4 c_lo = Vec4<float>::load(cos_t + t * 128 + d), c_hi = Vec4<float>::load(cos_t + t * 128 + 64 + d);
    const f32x4 s_lo = Vec4<float>::load(sin_t + t * 128 + d), s_hi = Vec4<float>::load(sin_t + t * 128 + 64 + d);
    T* row = x + t * row_stride;
    for (int h = slot; h < nq + nk; h += 16) {
        const bool is_k = h >= nq;
        T* v = row + (is_k ? k_offset + (long)(h - nq) * 128 : (long)h * 128);
        const float* g = is_k ? gk : gq;
        const f32x4 a = Vec4<T>::load(v + d), b = Vec4<T>::load(v + 64 + d);
        float inv = 1.0f;
        f32x4 ga = {1.f, 1.f, 1.f, 1.f}, gb = {1.f, 1.f, 1.f, 1.f};
        if (g) {  // NULL gamma: rotary only (the text block has no Q/K norm)
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += a[e] * a[e] + b[e] * b[e];
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
            inv = 1.0f / sqrtf(ss / 128.f + 1e-6f);
            ga = Vec4<float>::load(g + d);
            gb = Vec4<float>::load(g + 64 + d);
        }
        f32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float na = a[e] * inv * ga[e], nb = b[e] * inv * gb[e];
            lo[e] = na * c_lo[e] - nb * s_lo[e];
            hi[e] = nb * c_hi[e] + na * s_hi[e];
        }
        Vec4<T>::store(v + d, lo);
        Vec4<T>::store(v + 64 + d, hi);
    }
}

template <typename T>
__global__ void gelu_kernel(T* __restrict__ x, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = T(gelu_erf(float(x[i])));
}

__global__ void residual_kernel(const void* a, int adt, const void* b, int bdt, float* out, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = __fadd_rn(load_any(a, i, adt), load_any(b, i, bdt));
}

// Element-wise read-then-write, so out may alias x (in-place latent update).
__global__ void euler_kernel(const float* x, const float* v, float delta, size_t n, float* out)
{
    // The reference compiles its Euler update without contraction (-ffp-contract=off,
    // src/CMakeLists.txt:12-13): the product is rounded before the sum. hipcc contracts
    // by default, and __fmul_rn / __fadd_rn alone do not stop it from fusing the two into
    // one v_fmac_f32, so contraction is switched off for this function.
#pragma clang fp contract(off)
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float change = delta * v[i];
        out[i] = x[i] + change;
    }
}

__global__ void finite_kernel(const float* __restrict__ x, size_t n, int* __restrict__ flag)
{
    int bad = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        bad |= !isfinite(x[i]);
    if (bad) atomicOr(flag, 1);
}

// out[c][r] = in[r][c] for one element size (2 or 4 bytes), 32 x 32 tiles through LDS
// so both the reads and the writes are row-contiguous. Grid (ceil(cols/32),
// ceil(rows/32)), block 32 x 8.
template <typename E>
__global__ void __launch_bounds__(256) transpose_kernel(const E* __restrict__ in, E* __restrict__ out, int rows, int cols)
{
    __shared__ E tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x, ty = threadIdx.y;
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = in[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) out[(size_t)c * rows + r] = tile[tx][i];
    }
}

// One wave per (row, head) of rows [r0, r1): lane l takes head dimensions l and l + 64
// from their permuted columns, and writes the normalised, rotated pair back to columns
// l and l + 64. Every load of a head precedes its stores (the stores depend on the
// wave-wide sum), so rewriting the head in place is safe. The angles come packed
// (rope_pack): dimension d rotates by angle d / 2, whose (cos, sin) pair is at 2 (d / 2).
template <typename T>
__global__ void __launch_bounds__(256) qk_rope_permuted_kernel(T* __restrict__ x, int r0, int r1, int nq, int nk,
                                                               long row_stride, long k_offset,
                                                               const float* __restrict__ gq,
                                                               const float* __restrict__ gk,
                                                               const float* __restrict__ cs_t, float eps)
{
    const int lane = threadIdx.x & 63;
    const long w = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int heads = nq + nk;
    if (w >= (long)(r1 - r0) * heads) return;
    const int m = r0 + (int)(w / heads), h = (int)(w % heads);
    const bool is_k = h >= nq;
    T* v = x + (size_t)m * row_stride + (is_k ? k_offset + (long)(h - nq) * 128 : (long)h * 128);
    const float* g = is_k ? gk : gq;
    const int d0 = lane, d1 = lane + 64;
    const float a = float(v[qk_stored_column(d0)]), b = float(v[qk_stored_column(d1)]);
    const float ss = wave_sum(a * a + b * b);
    const float inv = 1.0f / sqrtf(ss / 128.f + eps);
    const float na = a * inv * g[d0], nb = b * inv * g[d1];
    const f32x2 c0 = *reinterpret_cast<const f32x2*>(cs_t + (size_t)m * 128 + 2 * (d0 >> 1));
    const f32x2 c1 = *reinterpret_cast<const f32x2*>(cs_t + (size_t)m * 128 + 2 * (d1 >> 1));
    const float lo = na * c0[0] - nb * c0[1], hi = nb * c1[0] + na * c1[1];
    v[d0] = T(lo);
    v[d1] = T(hi);
}

// Angle i = (row, k) of the flattened [rows][64]: columns 2k and 2k + 1 of the cos and sin rows must
// hold the same bits; their value goes to out[r][k] as a (cos, sin) pair, else NaN.
__global__ void rope_pack_kernel(const float* __restrict__ cos_t, const float* __restrict__ sin_t, size_t n,
                                 float* __restrict__ out)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const f32x2 c = *reinterpret_cast<const f32x2*>(cos_t + 2 * i);
        const f32x2 sn = *reinterpret_cast<const f32x2*>(sin_t + 2 * i);
        const bool same =
            __float_as_uint(c[0]) == __float_as_uint(c[1]) && __float_as_uint(sn[0]) == __float_as_uint(sn[1]);
        *reinterpret_cast<f32x2*>(out + 2 * i) =
            same ? f32x2{c[0], sn[0]} : f32x2{__builtin_nanf(""), __builtin_nanf("")};
    }
}

__global__ void fill_int_kernel(int* __restrict__ p, int value, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = value;
}

__global__ void convert_kernel(const void* __restrict__ in, int idt, void* __restrict__ out, int odt, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        store_any(out, i, odt, load_any(in, i, idt));
}

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Counter-based N(mean, std): Box-Muller of splitmix64(seed, offset + i).
__global__ void normal_kernel(void* __restrict__ out, int dt, size_t n, uint64_t seed, uint64_t offset, float mean,
                              float std_dev)
{
    const uint64_t key = mix64(seed ^ 0x5851F42D4C957F2Dull);
    const double unit = 1.0 / 9007199254740992.0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t c = 2ull * (offset + i);
        const uint64_t a = mix64(key + c), b = mix64(key + c + 1ull);
        const double u1 = double((a >> 11) + 1ull) * unit;
        const double u2 = double(b >> 11) * unit;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
        store_any(out, i, dt, float(double(mean) + double(std_dev) * z));
    }
}

// One wave per output; x (optionally SiLU'd) staged in LDS once per block.
template <typename T>
__global__ void __launch_bounds__(256) gemv_kernel(const T* __restrict__ W, const float* __restrict__ b,
                                                   const float* __restrict__ x, int N, int K, int silu,
                                                   float* __restrict__ y)
{
    extern __shared__ float xs[];
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = x[k];
        xs[k] = silu ? v / (1.0f + expf(-v)) : v;
    }
    __syncthreads();
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const int lane = threadIdx.x & 63;
    const T* w = W + (size_t)n * K;
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) acc += float(w[k]) * xs[k];
    acc = wave_sum(acc);
    if (lane == 0) y[n] = acc + (b ? b[n] : 0.f);
}

// Four outputs per wave, 16 per workgroup, for K a multiple of 8 with 16-bit W: each
// lane reads 16 bytes of each of its wave's four W rows per step (one 1-KiB request
// per row and wave) and the matching eight x values (SiLU'd on the fly), which stay
// in L1 / L2 across the waves; no LDS staging of x per workgroup.
template <typename T>
__global__ void __launch_bounds__(256) gemv4_kernel(const T* __restrict__ W, const float* __restrict__ b,
                                                    const float* __restrict__ x, int N, int K, int silu,
                                                    float* __restrict__ y)
{
    typedef T t8 __attribute__((ext_vector_type(8)));
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
    if (n0 >= N) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = lane * 8; k < K; k += 512) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(x + k), x1 = *reinterpret_cast<const f32x4*>(x + k + 4);
        float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        if (silu) {
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[e] = xv[e] / (1.0f + expf(-xv[e]));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (n0 + r < N) {
                const t8 w = *reinterpret_cast<const t8*>(W + (size_t)(n0 + r) * K + k);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r] += float(w[e]) * xv[e];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && n0 + r < N) y[n0 + r] = v + (b ? b[n0 + r] : 0.f);
    }
}

template <typename T>
__global__ void transpose_tokens_kernel(const float* __restrict__ latent, int ch, int hw, T* __restrict__ out)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)ch * hw) return;
    const int t = (int)(i / ch), c = (int)(i % ch);
    out[i] = T(latent[(size_t)c * hw + t]);
}

__global__ void tokens_latent_kernel(const float* __restrict__ proj, int hw, int ch, float* __restrict__ pred)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)ch * hw) return;
    const int c = (int)(i / hw), t = (int)(i % hw);
    pred[i] = proj[(size_t)t * ch + c];
}


// W_ug row layout: rows [64c, 64c+32) = up rows [32c, 32c+32), rows [64c+32, 64c+64)
// = gate rows [32c, 32c+32); lets one 64-column MFMA tile hold matching up/gate columns.
__global__ void interleave_kernel(const void* __restrict__ in, int idt, void* __restrict__ out, int dt, int rows,
                                  int cols, int parity)
{
    const size_t n = (size_t)rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        const size_t orow = 64 * (size_t)(r / 32) + 32 * parity + (r % 32);
        store_any(out, orow * cols + c, dt, load_any(in, i, idt));
    }
}

// Row-major [rows][cols] -> K-tiled [cols/32][rows][32], 16 bytes (8 values) per
// thread: chunk q = (r, c8) of the source lands at ((c8/4)*rows + r)*32 + (c8%4)*8.
__global__ void tile_k32_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, int rows, int cols,
                                int head_rows)
{
    const int c8n = cols / 8;
    const size_t n = (size_t)rows * c8n;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / c8n), c8 = (int)(i % c8n);
        const int o = r < head_rows ? (r & ~127) + qk_stored_column(r & 127) : r;
        out[((size_t)(c8 / 4) * rows + o) * 4 + (c8 % 4)] = in[i];
    }
}

inline int launch_status()
{
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -int(e);
}

inline unsigned grid_for(size_t n, unsigned block = 256)
{
    const size_t g = (n + block - 1) / block;
    return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}

bool valid_dt(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16; }

template <typename TIn>
int rms_dispatch_out(const TIn* x, const float* gamma, const float* shift, const float* scale, int rows, int width,
                     float eps, void* out, int odt, hipStream_t s, int out_rows)
{
    if (out_rows && width % 512 == 0 && width <= 4096 && odt != DT_F32) {
        // Persistent workgroups of about six row pairs each, at least one per CU of an
        // MI355X (256) and never more than the row pairs or four per CU. Each workgroup
        // stages the per-column factors (32 KiB at width 4096) once, so fewer, longer
        // workgroups move fewer bytes: at 4160 x 4096 after the output projection, 347
        // workgroups took 26.5 us where 1024 (two pairs each) took 30.6 and 694 / 520 /
        // 260 took 27.9 / 29.5 / 28.3 (bench A/B, two runs each on one box).
        const int pairs = (rows + 1) / 2;
        const dim3 grid((unsigned)std::min(std::max(std::min(pairs, 256), (pairs + 5) / 6), 1024)), block(256);
#define EHIP_RMS_PAIR(NI)                                                                                        \
        do {                                                                                                     \
            if (odt == DT_F16)                                                                                   \
                hipLaunchKernelGGL((rmsnorm_pair_k32_kernel<TIn, f16, NI>), grid, block, 0, s, x, gamma, shift,   \
                                   scale, rows, eps, static_cast<f16*>(out), out_rows);                          \
            else                                                                                                 \
                hipLaunchKernelGGL((rmsnorm_pair_k32_kernel<TIn, bf16, NI>), grid, block, 0, s, x, gamma, shift,  \
                                   scale, rows, eps, static_cast<bf16*>(out), out_rows);                         \
        } while (0)
        switch (width / 512) {
        case 1: EHIP_RMS_PAIR(1); break;
        case 2: EHIP_RMS_PAIR(2); break;
        case 3: EHIP_RMS_PAIR(3); break;
        case 4: EHIP_RMS_PAIR(4); break;
        case 5: EHIP_RMS_PAIR(5); break;
        case 6: EHIP_RMS_PAIR(6); break;
        case 7: EHIP_RMS_PAIR(7); break;
        default: EHIP_RMS_PAIR(8); break;
        }
#undef EHIP_RMS_PAIR
        return launch_status();
    }
    if (width % 1024 == 0) {
        // Four persistent workgroups per CU of an MI355X (256 CUs), never more than the rows.
        const dim3 grid((unsigned)std::min(rows, 1024)), block(256);
#define EHIP_RMS_PERSIST(PER)                                                                                    \
        do {                                                                                                     \
            if (odt == DT_F32)                                                                                   \
                hipLaunchKernelGGL((rmsnorm_persist_kernel<TIn, float, PER>), grid, block, 0, s, x, gamma, shift, \
                                   scale, rows, eps, static_cast<float*>(out), out_rows);                                  \
            else if (odt == DT_F16)                                                                              \
                hipLaunchKernelGGL((rmsnorm_persist_kernel<TIn, f16, PER>), grid, block, 0, s, x, gamma, shift,   \
                                   scale, rows, eps, static_cast<f16*>(out), out_rows);                                    \
            else                                                                                                 \
                hipLaunchKernelGGL((rmsnorm_persist_kernel<TIn, bf16, PER>), grid, block, 0, s, x, gamma, shift,  \
                                   scale, rows, eps, static_cast<bf16*>(out), out_rows);                                   \
        } while (0)
        switch (width / 1024) {
        case 1: EHIP_RMS_PERSIST(1); break;
        case 2: EHIP_RMS_PERSIST(2); break;
        case 3: EHIP_RMS_PERSIST(3); break;
        default: EHIP_RMS_PERSIST(4); break;
        }
#undef EHIP_RMS_PERSIST
        return launch_status();
    }
    // Other widths. Rows per workgroup: enough workgroups to cover the CUs several
    // times over, with the per-column vectors staged once per workgroup.
    const int rpb = rows >= 2048 ? 8 : (rows >= 512 ? 4 : 1);
    const dim3 grid((rows + rpb - 1) / rpb), block(64 * kRowWaves);
    if (odt == DT_F32)
        hipLaunchKernelGGL((rmsnorm_rows_kernel<TIn, float>), grid, block, 0, s, x, gamma, shift, scale, rows, width,
                           rpb, eps, static_cast<float*>(out), out_rows);
    else if (odt == DT_F16)
        hipLaunchKernelGGL((rmsnorm_rows_kernel<TIn, f16>), grid, block, 0, s, x, gamma, shift, scale, rows, width,
                           rpb, eps, static_cast<f16*>(out), out_rows);
    else
        hipLaunchKernelGGL((rmsnorm_rows_kernel<TIn, bf16>), grid, block, 0, s, x, gamma, shift, scale, rows, width,
                           rpb, eps, static_cast<bf16*>(out), out_rows);
    return launch_status();
}

}  // namespace

int rmsnorm_modulate(const void* x, int xdt, const float* gamma, const float* shift, const float* scale, int rows,
                     int width, float eps, void* out, int odt, hipStream_t s, int out_rows)
{
    if (!x || !out || rows < 1 || width < 4 || width % 4 || width > kRowMaxWidth) return -1;
    if (!valid_dt(xdt) || !valid_dt(odt) || (!shift) != (!scale)) return -1;
    if (out_rows && (out_rows < rows || width % 32 || odt == DT_F32)) return -1;
    if (xdt == DT_F32)
        return rms_dispatch_out(static_cast<const float*>(x), gamma, shift, scale, rows, width, eps, out, odt, s, out_rows);
    if (xdt == DT_F16)
        return rms_dispatch_out(static_cast<const f16*>(x), gamma, shift, scale, rows, width, eps, out, odt, s, out_rows);
    return rms_dispatch_out(static_cast<const bf16*>(x), gamma, shift, scale, rows, width, eps, out, odt, s, out_rows);
}

int layernorm_modulate(const float* x, const float* shift, const float* scale, int rows, int width, float eps,
                       void* out, int odt, hipStream_t s)
{
    if (!x || !out || !shift || !scale || rows < 1 || width < 4 || width % 4 || width > 1024 * kMaxPer) return -1;
    if (odt == DT_F32)
        hipLaunchKernelGGL(layernorm_mod_kernel<float>, dim3(rows), dim3(256), 0, s, x, shift, scale, width, eps,
                           static_cast<float*>(out));
    else if (odt == DT_F16)
        hipLaunchKernelGGL(layernorm_mod_kernel<f16>, dim3(rows), dim3(256), 0, s, x, shift, scale, width, eps,
                           static_cast<f16*>(out));
    else if (odt == DT_BF16)
        hipLaunchKernelGGL(layernorm_mod_kernel<bf16>, dim3(rows), dim3(256), 0, s, x, shift, scale, width, eps,
                           static_cast<bf16*>(out));
    else return -1;
    return launch_status();
}

int qk_norm_rope_qk(void* x, int dt, int rows, int nq, int nk, long row_stride, long k_offset, const float* gq,
                    const float* gk, const float* cos_t, const float* sin_t, hipStream_t s)
{
    if (!x || !cos_t || !sin_t || rows < 1 || nq < 0 || nk < 0 || nq + nk < 1) return -1;
    if (row_stride < (long)nq * 128 || (nk && (k_offset < (long)nq * 128 || row_stride < k_offset + (long)nk * 128)))
        return -1;
    // Four-value vector accesses: 16-byte (FP32) or 8-byte (16-bit) alignment of every head.
    const uintptr_t align = dt == DT_F32 ? 16 : 8;
    const long vec = dt == DT_F32 ? 4 : 4;
    if ((reinterpret_cast<uintptr_t>(x) % align) || row_stride % vec || k_offset % vec) return -1;
    const dim3 grid((unsigned)rows), block(256);
    if (dt == DT_F32)
        hipLaunchKernelGGL(qk_norm_rope_kernel<float>, grid, block, 0, s, static_cast<float*>(x), nq, nk, row_stride,
                           k_offset, gq, gk, cos_t, sin_t);
    else if (dt == DT_F16)
        hipLaunchKernelGGL(qk_norm_rope_kernel<f16>, grid, block, 0, s, static_cast<f16*>(x), nq, nk, row_stride,
                           k_offset, gq, gk, cos_t, sin_t);
    else if (dt == DT_BF16)
        hipLaunchKernelGGL(qk_norm_rope_kernel<bf16>, grid, block, 0, s, static_cast<bf16*>(x), nq, nk, row_stride,
                           k_offset, gq, gk, cos_t, sin_t);
    else return -1;
    return launch_status();
}

int qk_norm_rope(void* x, int dt, int rows, int nheads, long row_stride, const float* gamma, const float* cos_t,
                 const float* sin_t, hipStream_t s)
{
    return qk_norm_rope_qk(x, dt, rows, nheads, 0, row_stride, 0, gamma, nullptr, cos_t, sin_t, s);
}

int gelu_inplace(void* x, int dt, size_t n, hipStream_t s)
{
    if (!x || !n) return n ? -1 : 0;
    if (dt == DT_F32) hipLaunchKernelGGL(gelu_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s, static_cast<float*>(x), n);
    else if (dt == DT_F16) hipLaunchKernelGGL(gelu_kernel<f16>, dim3(grid_for(n)), dim3(256), 0, s, static_cast<f16*>(x), n);
    else if (dt == DT_BF16) hipLaunchKernelGGL(gelu_kernel<bf16>, dim3(grid_for(n)), dim3(256), 0, s, static_cast<bf16*>(x), n);
    else return -1;
    return launch_status();
}

int residual_add(const void* a, int adt, const void* b, int bdt, float* out, size_t n, hipStream_t s)
{
    if (!a || !b || !out || !valid_dt(adt) || !valid_dt(bdt)) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(residual_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, adt, b, bdt, out, n);
    return launch_status();
}

int euler_step(const float* x, const float* v, float delta, size_t n, float* out, hipStream_t s)
{
    if (!x || !v || !out) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(euler_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, v, delta, n, out);
    return launch_status();
}

int finite_flags(const float* x, size_t n, int* flag, hipStream_t s)
{
    if (!x || !flag) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(finite_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, n, flag);
    return launch_status();
}

int transpose2d(const void* in, int dt, int rows, int cols, void* out, hipStream_t s)
{
    if (!in || !out || !valid_dt(dt) || rows < 0 || cols < 0) return -1;
    if (!rows || !cols) return 0;
    const dim3 grid((cols + 31) / 32, (rows + 31) / 32), block(32, 8);
    if (grid.y > 65535) return -1;
    if (dt == DT_F32)
        hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, block, 0, s, static_cast<const uint32_t*>(in),
                           static_cast<uint32_t*>(out), rows, cols);
    else
        hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, block, 0, s, static_cast<const uint16_t*>(in),
                           static_cast<uint16_t*>(out), rows, cols);
    return launch_status();
}

int qk_norm_rope_permuted(void* x, int dt, int r0, int r1, int nq, int nk, long row_stride, long k_offset,
                          const float* gq, const float* gk, const float* cs_t, float eps, hipStream_t s)
{
    if (!x || !gq || !gk || !cs_t || (uintptr_t)cs_t % 8 || r0 < 0 || r1 < r0 || nq < 0 || nk < 0 ||
        dt == DT_F32 || !valid_dt(dt))
        return -1;
    const long waves = (long)(r1 - r0) * (nq + nk);
    if (!waves) return 0;
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    if (dt == DT_F16)
        hipLaunchKernelGGL(qk_rope_permuted_kernel<f16>, grid, block, 0, s, static_cast<f16*>(x), r0, r1, nq, nk,
                           row_stride, k_offset, gq, gk, cs_t, eps);
    else
        hipLaunchKernelGGL(qk_rope_permuted_kernel<bf16>, grid, block, 0, s, static_cast<bf16*>(x), r0, r1, nq, nk,
                           row_stride, k_offset, gq, gk, cs_t, eps);
    return launch_status();
}

int rope_pack(const float* cos_t, const float* sin_t, int rows, float* out, hipStream_t s)
{
    if (!cos_t || !sin_t || !out || rows < 0 || ((uintptr_t)cos_t | (uintptr_t)sin_t | (uintptr_t)out) % 8) return -1;
    const size_t n = (size_t)rows * 64;
    if (!n) return 0;
    hipLaunchKernelGGL(rope_pack_kernel, dim3(grid_for(n)), dim3(256), 0, s, cos_t, sin_t, n, out);
    return launch_status();
}

int fill_int(int* p, int value, size_t n, hipStream_t s)
{
    if (!p) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(fill_int_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, value, n);
    return launch_status();
}

int convert(const void* in, int idt, void* out, int odt, size_t n, hipStream_t s)
{
    if (!in || !out || !valid_dt(idt) || !valid_dt(odt)) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(convert_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, idt, out, odt, n);
    return launch_status();
}

int fill_normal(void* out, int dt, size_t n, uint64_t seed, uint64_t offset, float mean, float std_dev,
                hipStream_t s)
{
    if (!out || !valid_dt(dt)) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(normal_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, dt, n, seed, offset, mean, std_dev);
    return launch_status();
}

int gemv(const void* W, int wdt, const float* b, const float* x, int N, int K, int silu, float* y, hipStream_t s)
{
    if (!W || !x || !y || N < 1 || K < 1 || K > 16384) return -1;
    if (wdt != DT_F32 && K % 8 == 0 && reinterpret_cast<uintptr_t>(W) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        const dim3 grid4((N + 15) / 16), block4(256);
        if (wdt == DT_F16)
            hipLaunchKernelGGL(gemv4_kernel<f16>, grid4, block4, 0, s, static_cast<const f16*>(W), b, x, N, K, silu, y);
        else if (wdt == DT_BF16)
            hipLaunchKernelGGL(gemv4_kernel<bf16>, grid4, block4, 0, s, static_cast<const bf16*>(W), b, x, N, K, silu, y);
        else return -1;
        return launch_status();
    }
    const dim3 grid((N + 3) / 4), block(256);
    const size_t lds = sizeof(float) * K;
    if (wdt == DT_F32)
        hipLaunchKernelGGL(gemv_kernel<float>, grid, block, lds, s, static_cast<const float*>(W), b, x, N, K, silu, y);
    else if (wdt == DT_F16)
        hipLaunchKernelGGL(gemv_kernel<f16>, grid, block, lds, s, static_cast<const f16*>(W), b, x, N, K, silu, y);
    else if (wdt == DT_BF16)
        hipLaunchKernelGGL(gemv_kernel<bf16>, grid, block, lds, s, static_cast<const bf16*>(W), b, x, N, K, silu, y);
    else return -1;
    return launch_status();
}

int transpose_to_tokens(const float* latent, int ch, int hw, void* out, int dt, hipStream_t s)
{
    if (!latent || !out || ch < 1 || hw < 1) return -1;
    const size_t n = (size_t)ch * hw;
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    if (dt == DT_F32) hipLaunchKernelGGL(transpose_tokens_kernel<float>, grid, block, 0, s, latent, ch, hw, static_cast<float*>(out));
    else if (dt == DT_F16) hipLaunchKernelGGL(transpose_tokens_kernel<f16>, grid, block, 0, s, latent, ch, hw, static_cast<f16*>(out));
    else if (dt == DT_BF16) hipLaunchKernelGGL(transpose_tokens_kernel<bf16>, grid, block, 0, s, latent, ch, hw, static_cast<bf16*>(out));
    else return -1;
    return launch_status();
}

int tokens_to_latent(const float* proj, int hw, int ch, float* pred, hipStream_t s)
{
    if (!proj || !pred || ch < 1 || hw < 1) return -1;
    const size_t n = (size_t)ch * hw;
    hipLaunchKernelGGL(tokens_latent_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, proj, hw, ch, pred);
    return launch_status();
}

int interleave_up_gate(const void* in, int idt, void* out, int dt, int rows, int cols, int parity, hipStream_t s)
{
    if (!in || !out || !valid_dt(idt) || !valid_dt(dt) || rows % 32 || cols < 1 || (parity != 0 && parity != 1))
        return -1;
    const size_t n = (size_t)rows * cols;
    hipLaunchKernelGGL(interleave_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, idt, out, dt, rows, cols, parity);
    return launch_status();
}

int tile_k32(const void* in, void* out, int rows, int cols, hipStream_t s, int head_rows)
{
    if (head_rows < 0 || head_rows % 128 || head_rows > rows) return -1;
    if (!in || !out || rows < 1 || cols < 32 || cols % 32) return -1;
    if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) return -1;
    const size_t n = (size_t)rows * (cols / 8);
    hipLaunchKernelGGL(tile_k32_kernel, dim3(grid_for(n)), dim3(256), 0, s, static_cast<const uint4*>(in),
                       static_cast<uint4*>(out), rows, cols, head_rows);
    return launch_status();
}

}  // namespace ehip
