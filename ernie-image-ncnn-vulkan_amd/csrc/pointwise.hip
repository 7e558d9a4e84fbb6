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
    static __device__ __forceinline__ void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <typename T> struct Vec4 {
    typedef T t4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 load(const T* p)
    {
        const t4 v = *reinterpret_cast<const t4*>(p);
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

// One 256-thread block per row; width % 4 == 0 and width <= 4 * 256 * kMaxPer.
constexpr int kMaxPer = 4;  // float4 groups per thread -> width up to 4096
template <typename TIn, typename TOut>
__global__ void __launch_bounds__(256) rmsnorm_mod_kernel(const TIn* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ shift,
                                                          const float* __restrict__ scale, int width, float eps,
                                                          TOut* __restrict__ out)
{
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const TIn* xr = x + row * width;
    TOut* orow = out + row * width;
    f32x4 v[kMaxPer];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = (threadIdx.x + i * 256) * 4;
        if (c < width) {
            v[i] = Vec4<TIn>::load(xr + c);
            ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        }
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(width) + eps);
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = (threadIdx.x + i * 256) * 4;
        if (c < width) {
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float n = v[i][e] * inv;
                if (gamma) n = n * gamma[c + e];
                if (scale) n = n * (scale[c + e] + 1.0f) + shift[c + e];
                y[e] = n;
            }
            Vec4<TOut>::store(orow + c, y);
        }
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

// One wave per (token, head); lane d holds elements d and d + 64.
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(T* __restrict__ x, int rows, int nheads, long row_stride,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t)
{
    const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (long)rows * nheads) return;
    const int lane = threadIdx.x & 63;
    const long row = item / nheads;
    const int head = (int)(item - row * nheads);
    T* v = x + row * row_stride + head * 128;
    const float a = float(v[lane]), b = float(v[lane + 64]);
    const float inv = 1.0f / sqrtf(wave_sum(a * a + b * b) / 128.f + 1e-6f);
    const float na = a * inv * gamma[lane], nb = b * inv * gamma[lane + 64];
    const float* c = cos_t + row * 128;
    const float* s = sin_t + row * 128;
    v[lane] = T(na * c[lane] - nb * s[lane]);
    v[lane + 64] = T(nb * c[lane + 64] + na * s[lane + 64]);
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
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float change = __fmul_rn(delta, v[i]);
        out[i] = __fadd_rn(x[i], change);
    }
}

__global__ void finite_kernel(const float* __restrict__ x, size_t n, int* __restrict__ flag)
{
    int bad = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        bad |= !isfinite(x[i]);
    if (bad) atomicOr(flag, 1);
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
__global__ void interleave_kernel(const float* __restrict__ in, void* __restrict__ out, int dt, int rows, int cols,
                                  int parity)
{
    const size_t n = (size_t)rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        const size_t orow = 64 * (size_t)(r / 32) + 32 * parity + (r % 32);
        store_any(out, orow * cols + c, dt, in[i]);
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
                     float eps, void* out, int odt, hipStream_t s)
{
    if (odt == DT_F32)
        hipLaunchKernelGGL((rmsnorm_mod_kernel<TIn, float>), dim3(rows), dim3(256), 0, s, x, gamma, shift, scale,
                           width, eps, static_cast<float*>(out));
    else if (odt == DT_F16)
        hipLaunchKernelGGL((rmsnorm_mod_kernel<TIn, f16>), dim3(rows), dim3(256), 0, s, x, gamma, shift, scale, width,
                           eps, static_cast<f16*>(out));
    else
        hipLaunchKernelGGL((rmsnorm_mod_kernel<TIn, bf16>), dim3(rows), dim3(256), 0, s, x, gamma, shift, scale,
                           width, eps, static_cast<bf16*>(out));
    return launch_status();
}

}  // namespace

int rmsnorm_modulate(const void* x, int xdt, const float* gamma, const float* shift, const float* scale, int rows,
                     int width, float eps, void* out, int odt, hipStream_t s)
{
    if (!x || !out || rows < 1 || width < 4 || width % 4 || width > 1024 * kMaxPer) return -1;
    if (!valid_dt(xdt) || !valid_dt(odt) || (!shift) != (!scale)) return -1;
    if (xdt == DT_F32) return rms_dispatch_out(static_cast<const float*>(x), gamma, shift, scale, rows, width, eps, out, odt, s);
    if (xdt == DT_F16) return rms_dispatch_out(static_cast<const f16*>(x), gamma, shift, scale, rows, width, eps, out, odt, s);
    return rms_dispatch_out(static_cast<const bf16*>(x), gamma, shift, scale, rows, width, eps, out, odt, s);
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

int qk_norm_rope(void* x, int dt, int rows, int nheads, long row_stride, const float* gamma, const float* cos_t,
                 const float* sin_t, hipStream_t s)
{
    if (!x || !gamma || !cos_t || !sin_t || rows < 1 || nheads < 1 || row_stride < (long)nheads * 128) return -1;
    const long items = (long)rows * nheads;
    const dim3 grid((unsigned)((items + 3) / 4)), block(256);
    if (dt == DT_F32)
        hipLaunchKernelGGL(qk_norm_rope_kernel<float>, grid, block, 0, s, static_cast<float*>(x), rows, nheads,
                           row_stride, gamma, cos_t, sin_t);
    else if (dt == DT_F16)
        hipLaunchKernelGGL(qk_norm_rope_kernel<f16>, grid, block, 0, s, static_cast<f16*>(x), rows, nheads, row_stride,
                           gamma, cos_t, sin_t);
    else if (dt == DT_BF16)
        hipLaunchKernelGGL(qk_norm_rope_kernel<bf16>, grid, block, 0, s, static_cast<bf16*>(x), rows, nheads,
                           row_stride, gamma, cos_t, sin_t);
    else return -1;
    return launch_status();
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

int interleave_up_gate(const float* in, void* out, int dt, int rows, int cols, int parity, hipStream_t s)
{
    if (!in || !out || !valid_dt(dt) || rows % 32 || cols < 1 || (parity != 0 && parity != 1)) return -1;
    const size_t n = (size_t)rows * cols;
    hipLaunchKernelGGL(interleave_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, dt, rows, cols, parity);
    return launch_status();
}

}  // namespace ehip
