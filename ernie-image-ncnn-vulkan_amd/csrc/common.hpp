// SPDX-License-Identifier: MIT
// Shared device types and helpers for the gfx950 (CDNA4) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ehip {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Q/K projection rows of a 16-bit block are stored permuted within each 128-row head,
// so that the GEMM wave holding head dimension d also holds its rotary partner d + 64,
// in the same lane, 32 columns further on: stored column c (wave half c / 64, position
// l = c % 64) holds head dimension 32 (c / 64) + l % 32 + 64 (l / 32).
__host__ __device__ constexpr int qk_dim_of_column(int c) { return (c >> 6) * 32 + (c & 31) + ((c >> 5) & 1) * 64; }
__host__ __device__ constexpr int qk_stored_column(int d) { return ((d & 63) >> 5) * 64 + (d >> 6) * 32 + (d & 31); }
static_assert(qk_stored_column(qk_dim_of_column(38)) == 38 && qk_dim_of_column(72) == 40 &&
                  qk_dim_of_column(38) == 70 && qk_stored_column(100) == 100,
              "Q/K head permutation");

// Storage dtypes; values match ERNIE_DTYPE_* in the public header.
enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

inline size_t dtype_size(int dt) { return dt == DT_F32 ? 4 : 2; }

template <typename T> __device__ __forceinline__ float to_f32(T v) { return float(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return T(v); }

// Load one element of a buffer whose dtype is only known at run time.
__device__ __forceinline__ float load_any(const void* p, size_t i, int dt)
{
    if (dt == DT_F32) return static_cast<const float*>(p)[i];
    if (dt == DT_F16) return float(static_cast<const f16*>(p)[i]);
    return float(static_cast<const bf16*>(p)[i]);
}
__device__ __forceinline__ void store_any(void* p, size_t i, int dt, float v)
{
    if (dt == DT_F32) static_cast<float*>(p)[i] = v;
    else if (dt == DT_F16) static_cast<f16*>(p)[i] = f16(v);
    else static_cast<bf16*>(p)[i] = bf16(v);
}

// Full-wavefront (64-lane) reductions.
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// erf-form GELU, x * Phi(x) = 0.5 * x * erfc(-x / sqrt(2)), in FP32 through
// Abramowitz & Stegun 7.1.26 (|error in erf| <= 1.5e-7), the approximation the
// reference's GPU layer evaluates (src/ernie_gelu.cpp:12-31): the tail
// erfc(z) ~= t P(t) exp(-z^2), t = 1 / (1 + 0.3275911 z), z = |x| / sqrt(2), is
// computed directly, so the negative side keeps its small values. One
// reciprocal, one exp2 and five FMAs instead of the library erfc's branches.
__device__ __forceinline__ float gelu_erf(float x)
{
    const float z = fabsf(x) * 0.7071067811865475f;
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, z, 1.0f));
    float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
    p = __builtin_fmaf(p, t, 1.421413741f);
    p = __builtin_fmaf(p, t, -0.284496736f);
    p = __builtin_fmaf(p, t, 0.254829592f);
    const float tail = p * t * __builtin_amdgcn_exp2f(-1.4426950408889634f * z * z);
    return x * (x >= 0.f ? __builtin_fmaf(-0.5f, tail, 1.0f) : 0.5f * tail);
}

// x * sigmoid(x) = x / (1 + exp(-x)) (ncnn Swish, the text MLP's silu_7), with bare
// v_exp_f32 / v_rcp_f32: exp(-x) overflows to +inf for x < -88, giving -0.
__device__ __forceinline__ float silu(float x)
{
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// Activation on the gate half of a gated-MLP epilogue: SiLU or erf GELU.
template <bool kSilu> __device__ __forceinline__ float glu_act(float g) { return kSilu ? silu(g) : gelu_erf(g); }

}  // namespace ehip
