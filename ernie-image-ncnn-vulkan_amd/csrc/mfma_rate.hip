// SPDX-License-Identifier: MIT
// Matrix-core issue-rate probe: the box's own dense FP16 MFMA ceiling and the clock
// it holds under that load, measured beside every benchmark run so that a slow box
// and a slow kernel can be told apart.
//
// Every wave issues back-to-back v_mfma_f32_16x16x32_f16 into eight independent
// accumulators, straight from registers (no memory traffic inside the loop). The two
// operand sets alternate between consecutive MFMAs, so the operand bits toggle as
// they do with real data (constant operands let the chip hold a higher clock). Two
// waves share each SIMD (512-thread workgroups, one per CU). Each wave reads the
// shader-clock counter (s_memtime) and the constant-rate counter (s_memrealtime) at
// its start and end; the host turns those into the clock the chip ran at.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "kernels.hpp"

namespace ehip {
namespace {

constexpr int kRateAcc = 8;

__global__ __launch_bounds__(512) void mfma_rate_kernel(int iters, float* __restrict__ sink,
                                                        unsigned long long* __restrict__ stamps)
{
    const int lane = threadIdx.x & 63;
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    f16x8 a0, a1, b0, b1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // Values in [-0.75, 0.75] with mixed mantissa bits; a1/b1 differ from a0/b0 in
        // most bits, so alternating them toggles the operand lines.
        const int v = (lane * 8 + i) * 37;
        a0[i] = (_Float16)((float)(v % 97 - 48) * (1.0f / 64.0f));
        a1[i] = (_Float16)((float)((v + 41) % 89 - 44) * (-1.0f / 59.0f));
        b0[i] = (_Float16)((float)((v + 7) % 83 - 41) * (1.0f / 55.0f));
        b1[i] = (_Float16)((float)((v + 23) % 79 - 39) * (-1.0f / 53.0f));
    }
    f32x4 acc[kRateAcc];
#pragma unroll
    for (int j = 0; j < kRateAcc; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < kRateAcc; j += 2) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc[j], 0, 0, 0);
            acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc[j + 1], 0, 0, 0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kRateAcc; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (lane == 0) {
        const size_t w = (size_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
        stamps[4 * w + 0] = c0;
        stamps[4 * w + 1] = c1;
        stamps[4 * w + 2] = r0;
        stamps[4 * w + 3] = r1;
    }
}

}  // namespace

size_t mfma_rate_waves(int workgroups) { return (size_t)workgroups * 8; }

double mfma_rate_flop(int workgroups, int iters)
{
    // 16 x 16 x 32 multiply-adds per MFMA, kRateAcc MFMAs per iteration, 8 waves per workgroup.
    return 2.0 * 16 * 16 * 32 * kRateAcc * (double)iters * (double)mfma_rate_waves(workgroups);
}

int launch_mfma_rate(int workgroups, int iters, float* sink, unsigned long long* stamps, hipStream_t stream)
{
    if (workgroups < 1 || workgroups > 65536 || iters < 1 || !sink || !stamps) return -1;
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(workgroups), dim3(512), 0, stream, iters, sink, stamps);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -(int)e;
}

}  // namespace ehip
