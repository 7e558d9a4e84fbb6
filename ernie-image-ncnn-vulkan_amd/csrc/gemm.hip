// SPDX-License-Identifier: MIT
// MFMA GEMMs for gfx950: C[M,N] = A[M,K] * W[N,K]^T, both operands K-contiguous
// (the reference's Gemm layers use transB=1 with constant B, block.ncnn.param
// lines 19/22/25/61/70/71/74), FP32 accumulation and fused epilogues.
//
// 16-bit operands go to the ping-pong kernel (gemm16_pp.hip); the register-staged
// kernel below serves operands of 2 GiB or more, which need 64-bit addressing.
// 16-bit kernel (FP16 / BF16 operands, v_mfma_f32_32x32x16_{f16,bf16}):
//   * 512 threads = 8 waves arranged 2 (M) x 4 (N); N tile 256, K step 32.
//   * M tiles have a variable height of 1..10 subtiles of 32 rows, chosen on
//     the host so that (M tiles x N tiles) fills the 256 CUs in whole rounds
//     (M = 4160 = 130 subtiles does not divide into 256-row tiles).
//   * Each wave owns subtiles wm, wm+2, ... of its tile (up to 5) and 2 N
//     subtiles of 32 columns -> up to 10 f32x16 accumulators.
//   * LDS is double-buffered (one barrier per K step); rows are padded to 80 B
//     so ds_read_b128 of 16 lanes covers all 64 banks without conflict.
//   * Tile ids are remapped so that consecutive tiles land on one XCD (each of
//     the 8 XCDs has its own L2) and walk 4 M tiles per N sweep.
// FP32 kernel (v_mfma_f32_32x32x2_f32): 256 threads, 128 x 128 tiles, K step 16;
//   one ds_read_b128 feeds four MFMAs (lane group g supplies k = 4g + j).
#include "common.hpp"
#include "kernels.hpp"

namespace ehip {
namespace {

constexpr int kNumCU = 256;

struct GemmParams {
    const void* A; long lda;
    const void* W; long ldw;
    int M, N, K;
    int m_tiles, n_tiles, m_sub;
    void* C; long ldc;
    const float* bias;
    const float* resid; long ld_resid;
    const float* gate;
};

__device__ __forceinline__ void tile_coords(int bid, int m_tiles, int n_tiles, int& mt, int& nt)
{
    const int total = m_tiles * n_tiles;
    int logical = bid;
    if ((total & 7) == 0) logical = (bid & 7) * (total >> 3) + (bid >> 3);
    constexpr int GM = 4;
    const int group_size = GM * n_tiles;
    const int group = logical / group_size;
    const int first_m = group * GM;
    const int gm = min(m_tiles - first_m, GM);
    const int in_group = logical - group * group_size;
    mt = first_m + in_group % gm;
    nt = in_group / gm;
}

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

template <typename OutT, int EPI>
__device__ __forceinline__ void epilogue_store(const GemmParams& p, int m, int n, float v)
{
    if (EPI == EPI_STORE) {
        if (p.bias) v += p.bias[n];
        static_cast<OutT*>(p.C)[(size_t)m * p.ldc + n] = OutT(v);
    } else if (EPI == EPI_GATE_RESID) {
        const float r = p.resid[(size_t)m * p.ld_resid + n];
        static_cast<float*>(p.C)[(size_t)m * p.ldc + n] = r + p.gate[n] * v;
    }
}

// ------------------------------------------------------------------------------
// 16-bit operands
// ------------------------------------------------------------------------------
constexpr int G16_BN = 256, G16_BK = 32, G16_LDSK = G16_BK + 8, G16_TMX = 5, G16_MAX_SUB = 10;
constexpr int G16_BM_MAX = G16_MAX_SUB * 32;

template <typename T, typename OutT, int EPI>
__global__ void __launch_bounds__(512) gemm16_kernel(GemmParams p)
{
    typedef typename Mfma16<T>::vec vec8;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][G16_BM_MAX * G16_LDSK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][G16_BN * G16_LDSK];

    int mt, nt;
    tile_coords(blockIdx.x, p.m_tiles, p.n_tiles, mt, nt);
    const int base = p.m_sub / p.m_tiles, extra = p.m_sub % p.m_tiles;
    const int sub_cnt = base + (mt < extra ? 1 : 0);
    const int sub0 = mt * base + min(mt, extra);
    const int row0 = sub0 * 32;
    const int tile_rows = sub_cnt * 32;
    const int n0 = nt * G16_BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int lrow = lane & 31, lgrp = lane >> 5;

    // Global -> LDS copy assignment: 4 x 16 B chunks per 64 B row segment.
    const int ld_chunk = tid & 3, ld_row = tid >> 2;  // 128 rows per pass
    const T* A = static_cast<const T*>(p.A);
    const T* W = static_cast<const T*>(p.W);
    const T* a_src[3];
    const T* b_src[2];
#pragma unroll
    for (int s = 0; s < 3; ++s) {
        const int r = min(row0 + ld_row + 128 * s, p.M - 1);
        a_src[s] = A + (size_t)r * p.lda + ld_chunk * 8;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int r = min(n0 + ld_row + 128 * s, p.N - 1);
        b_src[s] = W + (size_t)r * p.ldw + ld_chunk * 8;
    }
    u32x4 a_reg[3], b_reg[2];

    auto load_global = [&](int kt) {
        const int koff = kt * G16_BK;
#pragma unroll
        for (int s = 0; s < 3; ++s)
            if (ld_row + 128 * s < tile_rows) a_reg[s] = *reinterpret_cast<const u32x4*>(a_src[s] + koff);
#pragma unroll
        for (int s = 0; s < 2; ++s) b_reg[s] = *reinterpret_cast<const u32x4*>(b_src[s] + koff);
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 3; ++s)
            if (ld_row + 128 * s < tile_rows)
                *reinterpret_cast<u32x4*>(&As[buf][(ld_row + 128 * s) * G16_LDSK + ld_chunk * 8]) = a_reg[s];
#pragma unroll
        for (int s = 0; s < 2; ++s)
            *reinterpret_cast<u32x4*>(&Bs[buf][(ld_row + 128 * s) * G16_LDSK + ld_chunk * 8]) = b_reg[s];
    };

    f32x16 acc[G16_TMX][2];
#pragma unroll
    for (int i = 0; i < G16_TMX; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = p.K / G16_BK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_global(kt + 1);
#pragma unroll
        for (int ks = 0; ks < G16_BK / 16; ++ks) {
            const int kcol = ks * 16 + lgrp * 8;
            vec8 bfrag[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfrag[j] = *reinterpret_cast<const vec8*>(&Bs[cur][(wn * 64 + j * 32 + lrow) * G16_LDSK + kcol]);
#pragma unroll
            for (int i = 0; i < G16_TMX; ++i) {
                const int sub = wm + 2 * i;
                if (sub < sub_cnt) {
                    const vec8 afrag =
                        *reinterpret_cast<const vec8*>(&As[cur][(sub * 32 + lrow) * G16_LDSK + kcol]);
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[i][j] = Mfma16<T>::run(afrag, bfrag[j], acc[i][j]);
                }
            }
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }

    // Accumulator layout (32x32 f32): lane -> column lane%32, register r -> row
    // 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
    for (int i = 0; i < G16_TMX; ++i) {
        const int sub = wm + 2 * i;
        if (sub >= sub_cnt) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = row0 + sub * 32 + 8 * (r >> 2) + 4 * lgrp + (r & 3);
            if (m >= p.M) continue;
            if (epi_glu(EPI)) {
                const int nout = (n0 + wn * 64) / 2 + lrow;
                if (2 * nout < p.N) {
                    const float up = acc[i][0][r], g = acc[i][1][r];
                    static_cast<OutT*>(p.C)[(size_t)m * p.ldc + nout] = OutT(up * glu_act<EPI == EPI_SWIGLU>(g));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = n0 + wn * 64 + j * 32 + lrow;
                    if (n < p.N) epilogue_store<OutT, EPI>(p, m, n, acc[i][j][r]);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------
// FP32 operands
// ------------------------------------------------------------------------------
constexpr int G32_BM = 128, G32_BN = 128, G32_BK = 16, G32_LDSK = G32_BK + 4;

template <int EPI>
__global__ void __launch_bounds__(256) gemm32_kernel(GemmParams p)
{
    __shared__ __attribute__((aligned(16))) float As[2][G32_BM * G32_LDSK];
    __shared__ __attribute__((aligned(16))) float Bs[2][G32_BN * G32_LDSK];
    int mt, nt;
    tile_coords(blockIdx.x, p.m_tiles, p.n_tiles, mt, nt);
    const int m0 = mt * G32_BM, n0 = nt * G32_BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int lrow = lane & 31, lgrp = lane >> 5;
    const int ld_chunk = tid & 3, ld_row = tid >> 2;  // 64 rows per pass
    const float* A = static_cast<const float*>(p.A);
    const float* W = static_cast<const float*>(p.W);
    const float* a_src[2];
    const float* b_src[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        a_src[s] = A + (size_t)min(m0 + ld_row + 64 * s, p.M - 1) * p.lda + ld_chunk * 4;
        b_src[s] = W + (size_t)min(n0 + ld_row + 64 * s, p.N - 1) * p.ldw + ld_chunk * 4;
    }
    f32x4 a_reg[2], b_reg[2];
    auto load_global = [&](int kt) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            a_reg[s] = *reinterpret_cast<const f32x4*>(a_src[s] + kt * G32_BK);
            b_reg[s] = *reinterpret_cast<const f32x4*>(b_src[s] + kt * G32_BK);
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            *reinterpret_cast<f32x4*>(&As[buf][(ld_row + 64 * s) * G32_LDSK + ld_chunk * 4]) = a_reg[s];
            *reinterpret_cast<f32x4*>(&Bs[buf][(ld_row + 64 * s) * G32_LDSK + ld_chunk * 4]) = b_reg[s];
        }
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = p.K / G32_BK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_global(kt + 1);
#pragma unroll
        for (int kq = 0; kq < G32_BK / 8; ++kq) {
            const int kcol = kq * 8 + lgrp * 4;
            f32x4 af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const f32x4*>(&As[cur][(wm * 64 + i * 32 + lrow) * G32_LDSK + kcol]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = *reinterpret_cast<const f32x4*>(&Bs[cur][(wn * 64 + j * 32 + lrow) * G32_LDSK + kcol]);
#pragma unroll
            for (int x = 0; x < 4; ++x)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][x], bfr[j][x], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lgrp + (r & 3);
            if (m >= p.M) continue;
            if (epi_glu(EPI)) {
                const int nout = (n0 + wn * 64) / 2 + lrow;
                if (2 * nout < p.N)
                    static_cast<float*>(p.C)[(size_t)m * p.ldc + nout] =
                        acc[i][0][r] * glu_act<EPI == EPI_SWIGLU>(acc[i][1][r]);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = n0 + wn * 64 + j * 32 + lrow;
                    if (n < p.N) epilogue_store<float, EPI>(p, m, n, acc[i][j][r]);
                }
            }
        }
}

// Pick the number of variable-height M tiles: fewest whole rounds over the CUs,
// weighted by the tallest tile (+1 subtile for the per-tile B traffic).
int choose_m_tiles(int m_sub, int n_tiles)
{
    const int min_mt = (m_sub + G16_MAX_SUB - 1) / G16_MAX_SUB;
    int best = min_mt;
    long best_cost = -1;
    for (int mt = min_mt; mt <= m_sub; ++mt) {
        const long rounds = ((long)mt * n_tiles + kNumCU - 1) / kNumCU;
        const long tallest = (m_sub + mt - 1) / mt;
        const long cost = rounds * (tallest + 1);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = mt;
        }
    }
    return best;
}

template <typename T>
int launch16(const GemmArgs& a, GemmParams& p, hipStream_t s)
{
    p.m_sub = (a.M + 31) / 32;
    p.n_tiles = (a.N + G16_BN - 1) / G16_BN;
    p.m_tiles = choose_m_tiles(p.m_sub, p.n_tiles);
    const dim3 grid(p.m_tiles * p.n_tiles), block(512);
    if (a.epilogue == EPI_STORE) {
        if (a.c_dtype == DT_F32) hipLaunchKernelGGL((gemm16_kernel<T, float, EPI_STORE>), grid, block, 0, s, p);
        else if (a.c_dtype == a.dtype) hipLaunchKernelGGL((gemm16_kernel<T, T, EPI_STORE>), grid, block, 0, s, p);
        else return -1;
    } else if (a.epilogue == EPI_GATE_RESID) {
        hipLaunchKernelGGL((gemm16_kernel<T, float, EPI_GATE_RESID>), grid, block, 0, s, p);
    } else if (a.epilogue == EPI_SWIGLU) {
        if (a.c_dtype != a.dtype) return -1;
        hipLaunchKernelGGL((gemm16_kernel<T, T, EPI_SWIGLU>), grid, block, 0, s, p);
    } else if (a.epilogue == EPI_GEGLU) {
        if (a.c_dtype != a.dtype) return -1;
        hipLaunchKernelGGL((gemm16_kernel<T, T, EPI_GEGLU>), grid, block, 0, s, p);
    } else {
        return -1;
    }
    return 0;
}

}  // namespace

int gemm(const GemmArgs& a, hipStream_t s)
{
    if (!a.A || !a.W || !a.C || a.M < 1 || a.N < 1 || a.K < 1) return -1;
    if (a.dtype != DT_F32 && a.dtype != DT_F16 && a.dtype != DT_BF16) return -1;
    const int kstep = a.dtype == DT_F32 ? G32_BK : G16_BK;
    if (a.K % kstep) return -1;
    const size_t align = a.dtype == DT_F32 ? 4 : 8;  // 16-byte vector loads along K
    if (a.lda < a.K || a.ldw < a.K || a.lda % align || a.ldw % align) return -1;
    if ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W)) & 15) return -1;
    if (a.epilogue == EPI_GATE_RESID && (!a.resid || !a.gate || a.c_dtype != DT_F32)) return -1;
    if (epi_glu(a.epilogue) && (a.N % 64 || a.ldc < a.N / 2)) return -1;
    if (!epi_glu(a.epilogue) && a.ldc < a.N) return -1;
    if (a.epilogue < 0 || (a.epilogue > EPI_GEGLU && a.epilogue != EPI_SWIGLU && a.epilogue != EPI_QKROPE)) return -1;
    if (a.epilogue == EPI_QKROPE && a.dtype == DT_F32) return -1;  // the fused Q/K path is the 16-bit kernel's
    // Only the 16-bit kernel reads or writes K-tiled operands.
    if ((a.w_k32 || a.a_k32_rows || a.c_k32_rows) && a.dtype == DT_F32) return -1;
    GemmParams p{};
    p.A = a.A; p.lda = a.lda; p.W = a.W; p.ldw = a.ldw;
    p.M = a.M; p.N = a.N; p.K = a.K;
    p.C = a.C; p.ldc = a.ldc; p.bias = a.bias; p.resid = a.resid; p.ld_resid = a.ld_resid; p.gate = a.gate;
    int rc = 0;
    if (a.dtype == DT_F32) {
        if (a.c_dtype != DT_F32) return -1;
        p.m_tiles = (a.M + G32_BM - 1) / G32_BM;
        p.n_tiles = (a.N + G32_BN - 1) / G32_BN;
        p.m_sub = 0;
        const dim3 grid(p.m_tiles * p.n_tiles), block(256);
        if (a.epilogue == EPI_STORE) hipLaunchKernelGGL((gemm32_kernel<EPI_STORE>), grid, block, 0, s, p);
        else if (a.epilogue == EPI_GATE_RESID) hipLaunchKernelGGL((gemm32_kernel<EPI_GATE_RESID>), grid, block, 0, s, p);
        else if (a.epilogue == EPI_SWIGLU) hipLaunchKernelGGL((gemm32_kernel<EPI_SWIGLU>), grid, block, 0, s, p);
        else if (a.epilogue == EPI_GEGLU) hipLaunchKernelGGL((gemm32_kernel<EPI_GEGLU>), grid, block, 0, s, p);
        else return -1;
    } else if ((rc = gemm16_pingpong(a, s)) != 1) {
        return rc;
    } else if (a.dtype == DT_F16) {
        rc = launch16<f16>(a, p, s);
    } else {
        rc = launch16<bf16>(a, p, s);
    }
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -int(e);
}

}  // namespace ehip
