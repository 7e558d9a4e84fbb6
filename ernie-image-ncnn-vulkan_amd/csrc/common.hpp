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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

// erf-form GELU, 0.5 * x * erfc(-x / sqrt(2)), FP32 arithmetic.
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * erfcf(-0.7071067811865475f * x); }

}  // namespace ehip
