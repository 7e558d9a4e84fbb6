// SPDX-License-Identifier: MIT
// 16-bit GEMM for gfx950, C[M,N] = A[M,K] * W[N,K]^T with FP32 accumulation and the
// fused epilogues of the DiT block (the reference's Gemm layers, transB with
// constant B: block.ncnn.param lines 19/22/25/61/70/71/74).
//
// Design (256 x 256 output tile per 512-thread workgroup, K step 32):
//   * Operands reach LDS through direct global->LDS buffer loads (16 bytes per lane,
//     1 KiB per instruction), so no VGPR staging and no ds_write is involved. A ring
//     of 4 stages (128 KiB) keeps three K steps in flight.
//   * Staged rows are 64 bytes; their four 16-byte chunks are XOR-swizzled by row
//     bits 2-3, so the 16 rows one fragment read touches at one chunk fall on 16
//     distinct 16-byte bank groups.
//   * The 8 waves form two groups with one wave of each per SIMD. The groups run half
//     a K step apart: while one executes a cluster of 32 v_mfma_f32_16x16x32 from
//     registers, the other reads its next fragments from LDS and issues its share of
//     the next stage's loads; they swap at each workgroup barrier (ping-pong), so the
//     matrix cores are fed while LDS latency is taken by the other group.
//   * Each wave owns a 128 x 64 sub-tile (8 x 4 accumulators of 16 x 16). The
//     16x16x32 form does the same work per cycle as 32x32x16 from the same LDS
//     fragments but draws less power: under this load the chip is power-limited, and
//     the clock it holds gave 5-7% more throughput on every projection shape.
//     Rows past M and columns past N read as zero through the buffer range checks;
//     tail tiles (M % 256) compute only their 64-row multiples.
//   * W and A may be stored K-tiled, [K/32][rows][32] (GemmArgs::w_k32,
//     a_k32_rows): then every 1-KiB load of a stage reads 1 KiB of contiguous
//     memory instead of 16 half cache lines, which lowers the power the loads draw
//     and lets the clock run higher. The block weights and the activations the
//     block's GEMMs read (RMSNorm, attention and GEGLU outputs) are stored this way.
//   * Workgroup b runs on XCD b % 8: each XCD gets a contiguous range of tiles
//     (4 M tiles per N sweep, sharing its own L2), and the tail row of tiles last.
//   * A tail row (M % 256 rows) is computed one of four ways. Split: its tiles are
//     cut along K into parts that fill the CUs and a reduction launch adds them.
//     Heavy (Params::heavy): the last row of full tiles is 320 rows tall. Riding
//     (Params::ride): every full tile computes one K range of the tail rows below
//     it. Light (Params::light): a 16- or 32-row chunk of the tail rows rides along
//     all of K in some full tiles, at most one per workgroup. The last three reuse the W rows
//     already in LDS instead of streaming all of W again for at most 64 rows.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace ehip {
namespace {
// Target number of tail-row items: one per CU of an MI355X.
constexpr int kSplitTargetItems = 256;
// Most K parts a split tile is cut into.
constexpr int kMaxSplit = 16;
}
namespace pingpong {

constexpr int BM = 256, BN = 256, BK = 32, NS = 4;
constexpr int ROWB = BK * 2;                // 64 bytes per staged row
// Launch modes: plain; heavy (Params::heavy: the last row of full tiles is 320 rows
// tall); ride (Params::ride: every full tile also computes one K range of the tail
// rows); light (Params::light: some full tiles also compute 16 or 32 of the tail rows
// over all of K). Heavy, ride and light launches keep room for 320 A rows in every stage.
enum { MODE_PLAIN = 0, MODE_HEAVY = 1, MODE_RIDE = 2, MODE_LIGHT = 3 };
// Stage layout: the A rows of the stage, then the W rows.
template <bool HV> struct Ring {
    static constexpr int A_ROWS = HV ? BM + 64 : BM;
    static constexpr int A_REGION = A_ROWS * ROWB;      // 16 or 20 KiB
    static constexpr int STAGE = A_REGION + BN * ROWB;  // 32 or 36 KiB
};
constexpr uint32_t kRsrcFlags = 0x00020000;

struct Params {
    const void* A; long lda;
    const void* W; long ldw;
    int M, N, K;
    int m_full, tail_sub, n_tiles;
    // heavy: the tail rows (M % 256 <= 64) are computed by the last row of full tiles,
    // as 320-row tiles, instead of as split tail items: no tail phase that streams all
    // of W for 64 rows, and no reduction launch. m_main: the M tiles walked by the
    // full-tile order (m_full, or m_full - 1 when the last row is heavy).
    int heavy, m_main;
    // ride: the tail rows (M % 256 <= 64) are computed by the full tiles while they
    // hold the W rows in LDS: full tile (mt, nt) adds tail part mt of tail column block
    // nt, K steps [K/32 * mt / m_full, K/32 * (mt + 1) / m_full), and stores it as
    // partial `mt` of `split` = m_full (the tail-row partial layout below), so there
    // is no tail phase that streams all of W again for 64 rows.
    int ride;
    // light: the tail rows (M % 256 <= 64) are cut into light_c chunks of light_h (16 or
    // 32) rows; for each column block nt, chunk e is computed over all of K by the full
    // tile (light_mt[e][nt], nt), as light_h more rows while it holds W. The host picks
    // those tiles so that no workgroup carries more than ceil(light tiles / grid) of
    // them: the extra MFMAs (a sixteenth or an eighth of a tile each) are spread over
    // the CUs, with no tail phase and no reduction.
    int light, light_c, light_h;
    uint8_t light_mt[4][128];
    void* C; long ldc;
    const float* bias;
    const float* resid; long ld_resid;
    const float* gate;
    uint32_t a_bytes, w_bytes;
    int w_row_bytes;  // byte distance of consecutive W rows within a K step: ldw * 2, or 64 if K-tiled
    int w_kstep;      // byte distance of consecutive K steps of one W row: 64, or N * 64 if K-tiled
    int a_row_bytes;  // the same for A: lda * 2 or 64
    int a_kstep;      // 64, or a_k32_rows * 64
    long c_rs, c_ss;  // EPI_GEGLU output: element distance of rows and of 32-column groups
    int split;        // K parts per tail tile (1 = no split)
    // split_all: every tile (not only the tail row) is split into `split` K parts; used
    // when the GEMM has too few tiles to fill the CUs. Partial layout then
    // [m_tiles][n_tiles][split][BM][BN]; else [n_tiles][split][64 * tail_sub][BN].
    int split_all;
    float* part;
    // Late split: the last `late` full tiles of the tile order (a partial last round
    // of workgroups) are each split into `late_split` K parts, so that round fills
    // the CUs with shorter items. Partials [late][late_split][BM][BN] at late_part.
    int late, late_split;
    float* late_part;
    // vec: every output row, residual row and the gate / bias vectors start 16-byte
    // aligned (8-byte for 16-bit outputs) and N % 4 == 0, so a lane's four consecutive
    // columns move as one vector; else element by element.
    int vec;
    int items;  // work items (tiles and tile parts); workgroup b takes items b, b + grid, ...
    // EPI_QKROPE (GemmArgs fields of the same names).
    int qk_cols;
    long k_col;
    const float* gq;
    const float* gk;
    const float* cs_t;  // [M][64] (cos, sin) pairs of each row's rotary angles (rope_pack)
    float qk_eps;
};

// Full tile f of the tile order -> (mt, nt): GM M tiles per N sweep, so the
// workgroups that run together share A and W panels.
constexpr int GM = 4;
__host__ __device__ __forceinline__ void full_order(const Params& p, int f, int& mt, int& nt)
{
    const int group_size = GM * p.n_tiles;
    const int group = f / group_size;
    const int first_m = group * GM;
    const int gm = p.m_main - first_m < GM ? p.m_main - first_m : GM;
    const int in_group = f - group * group_size;
    mt = first_m + in_group % gm;
    nt = in_group / gm;
}

// Light tiles: the tail chunk (rows m_full * 256 + light_h e .. + light_h - 1) that full
// tile (mt, nt) also computes, or -1.
__host__ __device__ __forceinline__ int light_chunk(const Params& p, int mt, int nt)
{
    if (!p.light) return -1;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (e < p.light_c && p.light_mt[e][nt] == mt) return e;
    return -1;
}

// The epilogue of a reduced element: row m, output column c (GEGLU / SwiGLU: of
// N / 2), tile-grid column n, summed value v (and gate sum g).
template <typename OutT, int EPI>
__device__ __forceinline__ void reduce_store(const Params& p, int m, int c, int n, float v, float g)
{
    if (epi_glu(EPI)) {
        static_cast<OutT*>(p.C)[(size_t)m * p.c_rs + (size_t)(c >> 5) * p.c_ss + (c & 31)] =
            OutT(v * glu_act<EPI == EPI_SWIGLU>(g));
    } else if (EPI == EPI_STORE) {
        if (p.bias) v += p.bias[n];
        static_cast<OutT*>(p.C)[(size_t)m * p.ldc + n] = OutT(v);
    } else {
        static_cast<float*>(p.C)[(size_t)m * p.ldc + n] = p.resid[(size_t)m * p.ld_resid + n] + p.gate[n] * v;
    }
}

// The epilogue of four reduced elements: row m, output columns c .. c + 3 (tile-grid
// columns n .. n + 3), every row, residual and vector 16-byte aligned (Params::vec).
template <typename OutT, int EPI>
__device__ __forceinline__ void reduce_store4(const Params& p, int m, int c, int n, f32x4 v, f32x4 g)
{
    typedef OutT out4 __attribute__((ext_vector_type(4)));
    if (epi_glu(EPI)) {
        out4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = OutT(v[r] * glu_act<EPI == EPI_SWIGLU>(g[r]));
        *reinterpret_cast<out4*>(static_cast<OutT*>(p.C) + (size_t)m * p.c_rs + (size_t)(c >> 5) * p.c_ss + (c & 31)) = o;
    } else if (EPI == EPI_STORE) {
        if (p.bias) v += *reinterpret_cast<const f32x4*>(p.bias + n);
        *reinterpret_cast<out4*>(static_cast<OutT*>(p.C) + (size_t)m * p.ldc + n) =
            out4{OutT(v[0]), OutT(v[1]), OutT(v[2]), OutT(v[3])};
    } else {
        const f32x4 rv = *reinterpret_cast<const f32x4*>(p.resid + (size_t)m * p.ld_resid + n);
        const f32x4 gv = *reinterpret_cast<const f32x4*>(p.gate + n);
        f32x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = rv[r] + gv[r] * v[r];
        *reinterpret_cast<f32x4*>(static_cast<float*>(p.C) + (size_t)m * p.ldc + n) = o;
    }
}

// Sum of `parts` partials `stride` floats apart, in part order, every load issued
// before the first add (at most kMaxSplit parts), so the sum does not wait out one
// load latency per part. V = 4: four consecutive columns per thread, 16-byte loads.
template <int EPI, int V, typename Vec>
__device__ __forceinline__ void sum_parts(const float* base, size_t stride, int parts, Vec& v, Vec& g)
{
    Vec pv[kMaxSplit], pg[kMaxSplit];
#pragma unroll
    for (int q = 0; q < kMaxSplit; ++q) {
        if (q < parts) {
            pv[q] = *reinterpret_cast<const Vec*>(base + (size_t)q * stride);
            if (epi_glu(EPI)) pg[q] = *reinterpret_cast<const Vec*>(base + (size_t)q * stride + 32);
        }
    }
    v = Vec(0.f);
    g = Vec(0.f);
#pragma unroll
    for (int q = 0; q < kMaxSplit; ++q) {
        if (q < parts) {
            v += pv[q];
            if (epi_glu(EPI)) g += pg[q];
        }
    }
}

// Sums the K parts of the split tiles and applies the epilogue: one thread per
// V consecutive output columns (GEGLU: up/gate column pairs) of a row, first over the
// tail row (or every row when split_all), then over the late-split tiles. V = 4 needs
// Params::vec; each element is summed in the same part order either way.
template <typename OutT, int EPI, int V>
__global__ void __launch_bounds__(256) split_reduce_kernel(Params p)
{
    typedef typename std::conditional<V == 4, f32x4, float>::type Vec;
    const int rows = p.split <= 1 ? 0 : (p.split_all ? p.M : 64 * p.tail_sub);
    const int cols = (epi_glu(EPI) ? p.N / 2 : p.N) / V;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    auto store = [&](int m, int c, int n, const Vec& v, const Vec& g) {
        if constexpr (V == 4) reduce_store4<OutT, EPI>(p, m, c, n, v, g);
        else reduce_store<OutT, EPI>(p, m, c, n, v, g);
    };
    if (idx >= (long)rows * cols) {
        // Late-split tile li: BM rows x BN grid columns (BN / 2 output columns for GLU).
        const int cols_t = (epi_glu(EPI) ? BN / 2 : BN) / V;
        const long j = idx - (long)rows * cols;
        if (j >= (long)p.late * BM * cols_t) return;
        const int li = (int)(j / (BM * cols_t));
        const int rem = (int)(j - (long)li * BM * cols_t);
        const int rl = rem / cols_t, cc = (rem - rl * cols_t) * V;
        int mt, nt;
        full_order(p, p.m_main * p.n_tiles - p.late + li, mt, nt);
        const int m = mt * BM + rl;
        const int c = (epi_glu(EPI) ? nt * (BN / 2) : nt * BN) + cc;
        const int n = epi_glu(EPI) ? (c / 32) * 64 + (c % 32) : c;
        Vec v, g;
        sum_parts<EPI, V>(p.late_part + ((size_t)li * p.late_split * BM + rl) * BN + (n - nt * BN), (size_t)BM * BN,
                          p.late_split, v, g);
        store(m, c, n, v, g);
        return;
    }
    const int rl = (int)(idx / cols), c = (int)(idx - (long)rl * cols) * V;
    const int m = p.split_all ? rl : p.m_full * BM + rl;
    if (m >= p.M) return;
    // Column n of the tile grid; GEGLU output column c holds up column (c / 32) * 64 + c % 32
    // and gate column + 32 of the interleaved W rows.
    const int n = epi_glu(EPI) ? (c / 32) * 64 + (c % 32) : c;
    const int nt = n / BN, cl = n - nt * BN;
    const int slot_rows = p.split_all ? BM : rows;
    const float* base = p.split_all
                            ? p.part + ((size_t)((m / BM) * p.n_tiles + nt) * p.split * BM + m % BM) * BN + cl
                            : p.part + (size_t)nt * p.split * rows * BN + (size_t)rl * BN + cl;
    Vec v, g;
    sum_parts<EPI, V>(base, (size_t)slot_rows * BN, p.split, v, g);
    store(m, c, n, v, g);
}

template <typename T> struct Mfma;
// 16 x 16 x 32 MFMA D = X Y^T. Operands: lane l supplies row l % 16 of X or Y,
// k = 8 (l / 16) .. + 7. Result: lane l holds D column l % 16 (a row of Y), register
// r D row 4 (l / 16) + r (a row of X). The tile passes W as X and A as Y, so a lane
// holds one output row and four consecutive output columns: 8- or 16-byte stores.
template <> struct Mfma<f16> {
    typedef f16x8 vec;
    static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c)
    { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <> struct Mfma<bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c)
    { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

// Physical chunk = logical chunk ^ fsw(row). A fragment read has 16 lanes at rows
// r0..r0+15 (r0 a multiple of 16) and one logical chunk. The LDS serves a
// ds_read_b128 eight lanes (128 bytes) at a time, so each group of eight rows
// must cover 8 distinct 16-byte slots mod 128: rows r and r + 1 sit 64 bytes
// apart, and XOR-ing the chunk with row bits 1-2 spreads the four row pairs
// over the four chunks. (Row bits 2-3, conflict-free for 16 lanes over 256
// bytes, leaves two-way conflicts in every group of eight: measured 269 against
// 424 GB/s per CU.)
__device__ __forceinline__ int fsw(int r) { return (r >> 1) & 3; }

// Tile order: workgroup b runs on XCD b % 8. Each XCD gets a contiguous share of
// the full-height tiles (walked 4 M tiles per N sweep), then of the late-split
// items (the last `late` full tiles, each in `late_split` K parts) and then of the
// tail-row items (a tail tile split into `split` K parts), so the short items run
// last and spread over all XCDs; or, with heavy tiles, of the last row of full
// tiles, one per workgroup in the last round. Riding and light launches have no
// tail-row items. li = index of a late-split tile, else -1.
__host__ __device__ __forceinline__ void tile_of(const Params& p, int bid, int& mt, int& nt, int& part, int& li)
{
    li = -1;
    if (p.split_all) {
        // Items (tile, part), a tile's parts adjacent and on one XCD; tiles walk the M
        // tiles of one N column before the next (the W panel shared within an XCD).
        const int m_tiles = p.m_full + (p.tail_sub ? 1 : 0);
        const int items = m_tiles * p.n_tiles * p.split;
        const int u = (items & 7) == 0 ? (bid & 7) * (items >> 3) + (bid >> 3) : bid;
        const int t = u / p.split;
        part = u - t * p.split;
        nt = t / m_tiles;
        mt = t - nt * m_tiles;
        return;
    }
    const int main_full = p.m_main * p.n_tiles - p.late;
    const int late_items = p.late * p.late_split;
    const int tail_items = p.heavy ? p.n_tiles : p.ride || p.light ? 0 : p.tail_sub ? p.n_tiles * p.split : 0;
    part = 0;
    int region, u;
    if ((main_full & 7) == 0 && (late_items & 7) == 0 && (tail_items & 7) == 0) {
        const int x = bid & 7, j = bid >> 3;
        const int a = main_full >> 3, b = late_items >> 3;
        if (j < a) { region = 0; u = x * a + j; }
        else if (j < a + b) { region = 1; u = x * b + (j - a); }
        else { region = 2; u = x * (tail_items >> 3) + (j - a - b); }
    } else {
        if (bid < main_full) { region = 0; u = bid; }
        else if (bid < main_full + late_items) { region = 1; u = bid - main_full; }
        else { region = 2; u = bid - main_full - late_items; }
    }
    if (region == 0) {
        full_order(p, u, mt, nt);
    } else if (region == 1) {
        li = u / p.late_split;
        part = u - li * p.late_split;
        full_order(p, main_full + li, mt, nt);
    } else if (p.heavy) {
        mt = p.m_full - 1;
        nt = u;
    } else {
        mt = p.m_full;
        nt = u / p.split;
        part = u - nt * p.split;
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Phase boundary: LDS reads issued before it have returned, every wave of the
// workgroup has arrived, and neither the compiler's scheduler nor its memory
// model moves instructions across it. No release fence: that would also wait for
// the stages still being loaded.
__device__ __forceinline__ void phase_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt vmcnt(n) for n in {0, 4, 8} (gfx9 encoding, other counters at max).
__device__ __forceinline__ void wait_vm(int n)
{
    if (n >= 8) __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));
    else if (n >= 4) __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8));
    else __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
}

// Wait until at most `stages` stages of LPS loads each are outstanding (more than two
// are waited down to two).
template <int LPS>
__device__ __forceinline__ void wait_stages(int stages)
{
    if (stages >= 2) __builtin_amdgcn_s_waitcnt((2 * LPS) | (7 << 4) | (15 << 8));
    else if (stages == 1) __builtin_amdgcn_s_waitcnt(LPS | (7 << 4) | (15 << 8));
    else __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ int item_parts(const Params& p, int mt, int li)
{
    return (p.split_all || mt == p.m_full) ? p.split : (li >= 0 ? p.late_split : 1);
}

// EPI_QKROPE epilogue of a Q or K tile (n0 < qk_cols). The wave pair (wm, wn) and
// (wm, wn ^ 1) holds one head's 128 columns for the same rows, each lane four rows of 16
// and, through the permuted W rows, head dimensions d_j = 32 (wn & 1) + 4 q16 + 16 j
// (+0..3) in acc[][j] and their rotary partners d_j + 64 in acc[][j + 2]. Each row's sum
// of squares is taken over the lane's 16 values, the four lanes of the row and, through
// `red` in LDS, the partner wave; then each pair is normalised, rotated and stored in
// natural column order. The FP32 accumulators are normalised directly: the only rounding
// is that of the rotated result, where a separate pass would first read back the
// projection rounded to the storage precision.
template <typename OutT, int MSUB>
__device__ __forceinline__ void qk_rope_epilogue(const Params& p, const f32x4 (&acc)[2 * MSUB][4], int n0, int row_w,
                                                 int wave, int wn, int q16, int r16, float* red)
{
    typedef OutT out4 __attribute__((ext_vector_type(4)));
    const int hf = wn & 1;
    const int head_col = n0 + 128 * (wn >> 1);
    const float* g = head_col >= p.k_col ? p.gk : p.gq;
    float ss[2 * MSUB];
#pragma unroll
    for (int i = 0; i < 2 * MSUB; ++i) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a = acc[i][j][r];
                t += a * a;
            }
        t += __shfl_xor(t, 16, 64);
        t += __shfl_xor(t, 32, 64);
        ss[i] = t;
    }
    // Gammas for the whole tile and the first two rows' angles are requested before the
    // partner exchange; each later row's are requested two rows ahead of their use.
    const int d0 = 32 * hf + 4 * q16;
    f32x4 ga[2], gb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        ga[j] = *reinterpret_cast<const f32x4*>(g + d0 + 16 * j);
        gb[j] = *reinterpret_cast<const f32x4*>(g + d0 + 16 * j + 64);
    }
    // Dimensions d .. d + 3 (d = d0 + 16 j, even) use angles d / 2 and d / 2 + 1 (each
    // twice), their partners d + 64 .. angles d / 2 + 32 and + 33. cs[b][j][0] holds
    // (cos, sin, cos, sin) of the first two, cs[b][j][1] of the second two, for buffer
    // b's row (clamped into [0, M)).
    f32x4 cs[3][2][2];
    auto load_row = [&](int i, f32x4 (&dst)[2][2]) {
        const size_t m = (size_t)min(row_w + 16 * i, p.M - 1) * 128;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int k = (d0 + 16 * j) >> 1;
            dst[j][0] = *reinterpret_cast<const f32x4*>(p.cs_t + m + 2 * k);
            dst[j][1] = *reinterpret_cast<const f32x4*>(p.cs_t + m + 2 * (k + 32));
        }
    };
    load_row(0, cs[0]);
    if (2 * MSUB > 1) load_row(1, cs[1]);
    if (q16 == 0)
#pragma unroll
        for (int i = 0; i < 2 * MSUB; ++i) red[(wave * 2 * MSUB + i) * 16 + r16] = ss[i];
    phase_barrier();
#pragma unroll
    for (int i = 0; i < 2 * MSUB; ++i) {
        if (i + 2 < 2 * MSUB) load_row(i + 2, cs[(i + 2) % 3]);
        const int m = row_w + 16 * i;
        const float inv = 1.0f / sqrtf((ss[i] + red[((wave ^ 2) * 2 * MSUB + i) * 16 + r16]) / 128.f + p.qk_eps);
        OutT* crow = static_cast<OutT*>(p.C) + (size_t)m * p.ldc + head_col;
        const f32x4(&c)[2][2] = cs[i % 3];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int d = d0 + 16 * j;
            out4 lo, hi;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float na = acc[i][j][r] * inv * ga[j][r];
                const float nb = acc[i][j + 2][r] * inv * gb[j][r];
                const int a = 2 * (r >> 1);
                lo[r] = OutT(na * c[j][0][a] - nb * c[j][0][a + 1]);
                hi[r] = OutT(nb * c[j][1][a] + na * c[j][1][a + 1]);
            }
            if (m < p.M) {
                *reinterpret_cast<out4*>(crow + d) = lo;
                *reinterpret_cast<out4*>(crow + d + 64) = hi;
            }
        }
        // Three rows' angles in flight at most: hoisting every row's would raise the
        // register peak.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Epilogue of a light tile's tail chunk e. XR = 1 (16-row chunks): output row
// m_full * 256 + 16 e + r16, and the wave holds the chunk's columns 16 j + 4 q16 + r of
// its 64 for j = wm (lacc[0]) and j = wm + 2 (lacc[1]), the pairs that the GLU epilogues
// (up, gate) and the Q/K epilogue (dimension, rotary partner) combine in one lane; a
// Q or K head's 128 columns then lie in the four waves 4 h .. 4 h + 3, and each row's
// sum of squares is added over them through `red` in one fixed order, so all four use
// the same value. XR = 2 (32-row chunks, GLU only): output row
// m_full * 256 + 32 e + 16 wm + r16 and all four column blocks j in lacc[j], as in a
// full tile's row group.
template <typename OutT, int EPI, int XR>
__device__ __forceinline__ void light_epilogue(const Params& p, const f32x4 (&lacc)[2 * XR], int chunk, int n0,
                                               int wave, int wm, int wn, int q16, int r16, float* red)
{
    typedef OutT out4 __attribute__((ext_vector_type(4)));
    const int m = p.m_full * BM + p.light_h * chunk + (XR == 2 ? 16 * wm : 0) + r16;
    if constexpr (EPI == EPI_QKROPE) {
        static_assert(XR == 1, "the Q/K epilogue takes 16-row chunks");
        if (n0 < p.qk_cols) {
            const int head_col = n0 + 128 * (wn >> 1);
            const float* g = head_col >= p.k_col ? p.gk : p.gq;
            float t = 0.f;
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int r = 0; r < 4; ++r) t += lacc[x][r] * lacc[x][r];
            t += __shfl_xor(t, 16, 64);
            t += __shfl_xor(t, 32, 64);
            float* lred = red + 8 * 8 * 16;  // after the full rows' slots
            if (q16 == 0) lred[wave * 16 + r16] = t;
            const int d = 32 * (wn & 1) + 4 * q16 + 16 * wm;
            const f32x4 ga = *reinterpret_cast<const f32x4*>(g + d);
            const f32x4 gb = *reinterpret_cast<const f32x4*>(g + d + 64);
            // (cos, sin) of angles d / 2, d / 2 + 1 and of d / 2 + 32, + 33 (see qk_rope_epilogue).
            const size_t mc = (size_t)min(m, p.M - 1) * 128;
            const f32x4 cl = *reinterpret_cast<const f32x4*>(p.cs_t + mc + d);
            const f32x4 ch = *reinterpret_cast<const f32x4*>(p.cs_t + mc + d + 64);
            phase_barrier();
            const int w0 = wave & ~3;
            const float ss = (lred[w0 * 16 + r16] + lred[(w0 + 1) * 16 + r16]) +
                             (lred[(w0 + 2) * 16 + r16] + lred[(w0 + 3) * 16 + r16]);
            const float inv = 1.0f / sqrtf(ss / 128.f + p.qk_eps);
            out4 lo, hi;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float na = lacc[0][r] * inv * ga[r];
                const float nb = lacc[1][r] * inv * gb[r];
                const int a = 2 * (r >> 1);
                lo[r] = OutT(na * cl[a] - nb * cl[a + 1]);
                hi[r] = OutT(nb * ch[a] + na * ch[a + 1]);
            }
            if (m < p.M) {
                OutT* crow = static_cast<OutT*>(p.C) + (size_t)m * p.ldc + head_col;
                *reinterpret_cast<out4*>(crow + d) = lo;
                *reinterpret_cast<out4*>(crow + d + 64) = hi;
            }
            return;
        }
        // V columns: stored as they are, below.
    }
    if (m >= p.M) return;
    // Column block of lacc[x] (and, for GLU, of its gate partner lacc[x + XR]).
    auto jb = [&](int x) { return XR == 1 ? wm + 2 * x : x; };
    if constexpr (epi_glu(EPI)) {
        if (n0 + wn * 64 >= p.N) return;
        OutT* c = static_cast<OutT*>(p.C) + (size_t)m * p.c_rs + (size_t)((n0 + wn * 64) >> 6) * p.c_ss + 4 * q16;
#pragma unroll
        for (int x = 0; x < XR; ++x) {
            out4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = OutT(lacc[x][r] * glu_act<EPI == EPI_SWIGLU>(lacc[x + XR][r]));
            if (p.vec) *reinterpret_cast<out4*>(c + 16 * jb(x)) = o;
            else
#pragma unroll
                for (int r = 0; r < 4; ++r) c[16 * jb(x) + r] = o[r];
        }
    } else {
        static_assert(EPI != EPI_GATE_RESID, "light tiles take no gate + residual epilogue");
#pragma unroll
        for (int x = 0; x < 2 * XR; ++x) {
            const int n = n0 + wn * 64 + 4 * q16 + 16 * (XR == 1 ? wm + 2 * x : x);
            if (n >= p.N) continue;
            OutT* c = static_cast<OutT*>(p.C) + (size_t)m * p.ldc + n;
            if (p.vec) {
                f32x4 v = lacc[x];
                if (p.bias) v += *reinterpret_cast<const f32x4*>(p.bias + n);
                *reinterpret_cast<out4*>(c) = out4{OutT(v[0]), OutT(v[1]), OutT(v[2]), OutT(v[3])};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (n + r >= p.N) continue;
                    float v = lacc[x][r];
                    if (p.bias) v += p.bias[n + r];
                    c[r] = OutT(v);
                }
            }
        }
    }
}

// One work item. `pre`: its first NS stages were requested by the previous item of this
// workgroup. nmt >= 0 names the next item (nmt, nnt, npart, nli), whose first NS stages
// this one requests once its own ring is drained, before its epilogue. XR: this item is
// a light tile carrying tail chunk xe of 16 (XR = 1) or 32 (XR = 2) rows; nxe: the next
// item's chunk (or -1).
template <typename T, typename OutT, int EPI, int MSUB, int MODE, int XR = 0>
__device__ __forceinline__ void tile(const Params& p, int mt, int nt, int part, int li, uint8_t* smem, bool pre,
                                     int nmt, int nnt, int npart, int nli, float* red, int xe = -1, int nxe = -1)
{
    typedef typename Mfma<T>::vec vec8;
    constexpr bool HV = MODE != MODE_PLAIN;
    typedef Ring<HV> R;
    // A heavy tile (MSUB 5: 320 rows) or a light tile loads one more A instruction per
    // stage and wave.
    constexpr int LPS = MSUB == 5 || XR ? 5 : 4;
    const int m0 = mt * BM, n0 = nt * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = wave >> 2;              // waves 0-3 and 4-7: one of each per SIMD
    const int wm = wave & 1, wn = wave >> 1;  // output sub-tile of this wave

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.A), (short)0, p.a_bytes, kRsrcFlags);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.W), (short)0, p.w_bytes, kRsrcFlags);

    // Direct loads: wave w fills rows [32w, 32w+32) of the A and W halves of a stage
    // with two 1-KiB instructions each; lane l lands at bytes [16l, 16l+16), i.e.
    // row (l >> 2), physical chunk l & 3 = logical chunk (l & 3) ^ fsw(row). The tail
    // rows of a heavy or riding tile (stage rows 256 + 8w .. + 7) come from a third
    // instruction of lanes 0-31; the chunk rows of a light tile (stage rows
    // 256 + h w .. + h - 1, h = light_h / 8) from a third instruction of lanes 0 .. 4h - 1.
    uint32_t a_src[3], w_src[2];
    auto sources = [&](int m_0, int n_0, uint32_t* as, uint32_t* ws, int chunk) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int row = wave * 32 + q * 16 + (lane >> 2);
            const int c = (lane & 3) ^ fsw(row);
            as[q] = (uint32_t)((long)(m_0 + row) * p.a_row_bytes + c * 16);
            ws[q] = (uint32_t)((long)(n_0 + row) * p.w_row_bytes + c * 16);
        }
        if constexpr (MODE == MODE_LIGHT) {
            const int h = p.light_h >> 3;
            const int row = BM + wave * h + (lane >> 2);
            const int src = p.m_full * BM + p.light_h * max(chunk, 0) + wave * h + (lane >> 2);
            as[2] = (uint32_t)((long)src * p.a_row_bytes + (((lane & 3) ^ fsw(row)) << 4));
        } else if constexpr (HV) {
            const int row = BM + wave * 8 + (lane >> 2);
            const int tail0 = MODE == MODE_HEAVY ? m_0 : (p.m_full - 1) * BM;  // + BM: the first tail row
            as[2] = (uint32_t)((long)(tail0 + row) * p.a_row_bytes + (((lane & 3) ^ fsw(row)) << 4));
        }
    };
    sources(m0, n0, a_src, w_src, xe);
    // K steps of this item: all of them, or part `part` of `split` for a tail tile.
    const int nk_all = p.K / BK;
    const int parts = item_parts(p, mt, li);
    const int kt0 = (int)((long)nk_all * part / parts);
    const int nk = (int)((long)nk_all * (part + 1) / parts) - kt0;
    // Stage kt (of the item starting at K step k0) into ring slot kt % NS.
    auto issue_at = [&](const uint32_t* as, const uint32_t* ws, int k0, int kt, bool heavy_item) {
        uint8_t* st = smem + (kt & (NS - 1)) * R::STAGE;
        const int koff = (k0 + kt) * p.a_kstep, koff_w = (k0 + kt) * p.w_kstep;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + (wave * 32 + q * 16) * ROWB), 16, as[q],
                                                     koff, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(st + R::A_REGION + (wave * 32 + q * 16) * ROWB),
                                                     16, ws[q], koff_w, 0, 0);
        }
        if constexpr (MODE == MODE_LIGHT) {
            if (heavy_item && lane < (p.light_h >> 1))
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + (BM + wave * (p.light_h >> 3)) * ROWB), 16,
                                                         as[2], koff, 0, 0);
        } else if constexpr (HV) {
            if (heavy_item && lane < 32)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + (BM + wave * 8) * ROWB), 16, as[2], koff,
                                                         0, 0);
        }
    };
    // Riding: the K steps [rk0, rk1) of this item that also compute its tail part.
    const int rk0 = MODE == MODE_RIDE ? (int)((long)nk_all * mt / p.m_full) - kt0 : 0;
    const int rk1 = MODE == MODE_RIDE ? (int)((long)nk_all * (mt + 1) / p.m_full) - kt0 : 0;
    auto riding = [&](int kt) { return MODE == MODE_RIDE && kt >= rk0 && kt < rk1; };
    auto issue = [&](int kt) { issue_at(a_src, w_src, kt0, kt, MSUB == 5 || XR || riding(kt)); };

    // Fragment of 16 rows x 32 k: lane l reads row l % 16, logical chunk l / 16.
    const int r16 = lane & 15, q16 = lane >> 4;
    const uint32_t frag = r16 * ROWB + ((q16 ^ fsw(r16)) << 4);

    // acc[i][j][r]: row 16i + r16 of this wave's 32 MSUB rows, column 16j + 4 q16 + r
    // of its 64 columns.
    f32x4 acc[2 * MSUB][4];
#pragma unroll
    for (int i = 0; i < 2 * MSUB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

    vec8 af[2 * MSUB], bf[4];
    // Riding: the tail part's accumulators (this wave's 32 of the 64 tail rows) and
    // fragments.
    constexpr int TR = MODE == MODE_RIDE ? 2 : 0;
    f32x4 tacc[TR ? TR : 1][4];
    vec8 tf[TR ? TR : 1];
#pragma unroll
    for (int i = 0; i < TR; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) tacc[i][j][r] = 0.f;
    // Light tile: this wave's chunk fragment (stage rows 256 .. 271, or 256 + 16 wm ..
    // + 15 for 32-row chunks) and its accumulators: column blocks j = wm and wm + 2, or
    // all four.
    f32x4 lacc[XR ? 2 * XR : 1];
    vec8 lf;
#pragma unroll
    for (int x = 0; x < (XR ? 2 * XR : 1); ++x)
#pragma unroll
        for (int r = 0; r < 4; ++r) lacc[x][r] = 0.f;
    // Memory cluster: this wave's fragments of stage kt into registers.
    auto read_frags = [&](int kt) {
        const uint8_t* st = smem + (kt & (NS - 1)) * R::STAGE;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bf[j] = *reinterpret_cast<const vec8*>(st + R::A_REGION + (wn * 64 + j * 16) * ROWB + frag);
#pragma unroll
        for (int i = 0; i < 2 * MSUB; ++i)
            af[i] = *reinterpret_cast<const vec8*>(st + (wm * 32 * MSUB + i * 16) * ROWB + frag);
        if (riding(kt))
#pragma unroll
            for (int i = 0; i < TR; ++i)
                tf[i] = *reinterpret_cast<const vec8*>(st + (BM + wm * 32 + i * 16) * ROWB + frag);
        if constexpr (XR == 1) lf = *reinterpret_cast<const vec8*>(st + BM * ROWB + frag);
        if constexpr (XR == 2) lf = *reinterpret_cast<const vec8*>(st + (BM + 16 * wm) * ROWB + frag);
    };
    // MFMA cluster on the registers of stage kt.
    auto mfma_cluster = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 2 * MSUB; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::run(bf[j], af[i], acc[i][j]);
        if (riding(kt))
#pragma unroll
            for (int i = 0; i < TR; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) tacc[i][j] = Mfma<T>::run(bf[j], tf[i], tacc[i][j]);
        if constexpr (XR == 1) {
            // Column blocks wm and wm + 2, selected without a branch in the cluster.
            const vec8 b0 = wm ? bf[1] : bf[0], b1 = wm ? bf[3] : bf[2];
            lacc[0] = Mfma<T>::run(b0, lf, lacc[0]);
            lacc[1] = Mfma<T>::run(b1, lf, lacc[1]);
        }
        if constexpr (XR == 2)
#pragma unroll
            for (int j = 0; j < 4; ++j) lacc[j] = Mfma<T>::run(bf[j], lf, lacc[j]);
    };
    // Loads requested after stage s, per wave, when s must have landed: LPS x min(NS-2, nk-1-s).
    // A riding item's window stages carry a fifth load; counting four for every stage
    // can only wait for more loads than stage s needs, never fewer.
    auto wait_stage = [&](int s) { wait_stages<LPS>(min(NS - 2, nk - 1 - s)); };

    // Prologue: request stages 0..NS-1 (unless the previous item did), wait for stage 0
    // everywhere. After a previous item, its epilogue's stores are counted too: wait
    // for everything.
    if (!pre) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
            if (s < nk) issue(s);
        wait_stages<LPS>(min(NS - 1, nk - 1));
    } else {
        wait_vm(0);
    }
    phase_barrier();

    // Phase 2t+1: group 0 computes stage t, group 1 reads stage t and requests
    // stage t-1+NS. Phase 2t+2: group 1 computes stage t, group 0 reads stage t+1
    // and requests stage t+NS. Stage s is read in phases 2s and 2s+1, so its slot
    // is refilled from phase 2s+2 on; it must land before phase 2s.
    if (group == 0) {
        read_frags(0);
        phase_barrier();  // end of phase 0
        for (int t = 0; t < nk; ++t) {
            mfma_cluster(t);
            if (t + 1 < nk) wait_stage(t + 1);
            phase_barrier();  // end of phase 2t+1
            if (t + 1 < nk) {
                read_frags(t + 1);
                if (t + NS < nk) issue(t + NS);
            }
            phase_barrier();  // end of phase 2t+2
        }
    } else {
        phase_barrier();  // end of phase 0
        for (int t = 0; t < nk; ++t) {
            read_frags(t);
            if (t >= 1 && t - 1 + NS < nk) issue(t - 1 + NS);
            if (t + 1 < nk) wait_stage(t + 1);
            phase_barrier();  // end of phase 2t+1
            mfma_cluster(t);
            phase_barrier();  // end of phase 2t+2
        }
    }

    // The last barrier above follows every wave's last LDS read: the ring is free for
    // the next item's first stages, which then land during this epilogue.
    if (nmt >= 0) {
        const int nparts = item_parts(p, nmt, nli);
        const int nkt0 = (int)((long)nk_all * npart / nparts);
        const int nnk = (int)((long)nk_all * (npart + 1) / nparts) - nkt0;
        uint32_t na[3], nw[2];
        sources(nmt * BM, nnt * BN, na, nw, nxe);
        const bool nheavy = (MODE == MODE_HEAVY && nmt == p.m_full - 1) || nxe >= 0;
        // Riding: the next item's tail K steps among its first stages.
        const int nrk0 = MODE == MODE_RIDE ? (int)((long)nk_all * nmt / p.m_full) - nkt0 : 0;
        const int nrk1 = MODE == MODE_RIDE ? (int)((long)nk_all * (nmt + 1) / p.m_full) - nkt0 : 0;
#pragma unroll
        for (int s = 0; s < NS; ++s)
            if (s < nnk) issue_at(na, nw, nkt0, s, nheavy || (s >= nrk0 && s < nrk1));
    }
    // A light tile finishes its chunk first: its accumulators are then free before the
    // full rows' epilogue, which sets the register peak.
    if constexpr (XR) light_epilogue<OutT, EPI, XR>(p, lacc, xe, n0, wave, wm, wn, q16, r16, red);
    if constexpr (MODE == MODE_RIDE) {
        // The tail part: partial mt of tail column block nt.
        float* base = p.part + ((size_t)nt * p.split + mt) * 64 * BN;
#pragma unroll
        for (int i = 0; i < TR; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(base + (size_t)(wm * 32 + 16 * i + r16) * BN + wn * 64 + 4 * q16 + 16 * j) =
                    tacc[i][j];
    }

    const int row_w = m0 + wm * 32 * MSUB + r16;  // + 16 i: output row
    const int col_w = n0 + wn * 64 + 4 * q16;      // + 16 j + r: output column (W row)
    if (li >= 0 || (p.split > 1 && (p.split_all || mt == p.m_full))) {
        // Split tile: store this part's FP32 partial; split_reduce_kernel, the next
        // launch on the stream, adds the parts and applies the epilogue.
        const int rows = (li >= 0 || p.split_all) ? BM : 64 * p.tail_sub;
        float* base = li >= 0       ? p.late_part + ((size_t)li * p.late_split + part) * BM * BN
                      : p.split_all ? p.part + (((size_t)mt * p.n_tiles + nt) * p.split + part) * BM * BN
                                    : p.part + ((size_t)nt * p.split + part) * rows * BN;
#pragma unroll
        for (int i = 0; i < 2 * MSUB; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(base + (size_t)(row_w - m0 + 16 * i) * BN + (col_w - n0) + 16 * j) = acc[i][j];
        return;
    }

    if constexpr (EPI == EPI_QKROPE) {
        if (n0 < p.qk_cols) {
            qk_rope_epilogue<OutT, MSUB>(p, acc, n0, row_w, wave, wn, q16, r16, red);
            return;
        }
        // V columns: stored as they are, below.
    }
    if constexpr (EPI == EPI_GATE_RESID) {
        // C = resid + gate * acc, C possibly aliasing resid. Each element is read and
        // written by this lane only, so a 32-row block's residuals (8 loads of 16 bytes
        // per lane) are requested before the previous block's stores. Stores and loads
        // share one in-order counter, so a load requested after a store could only be
        // waited for together with that store's write acknowledgement; requested one
        // block ahead, each block's wait leaves the previous block's stores in flight.
        float* C = static_cast<float*>(p.C);
        if (p.vec) {
            f32x4 gv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = col_w + 16 * j;
                gv[j] = n < p.N ? *reinterpret_cast<const f32x4*>(p.gate + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
            f32x4 rv[2][2][4];
            // Whole tile inside M x N (every tile but the tail row's, N a multiple of 256):
            // no per-element bounds, so no branches, and the wait before each block's
            // stores counts only the loads it needs.
            const bool whole = m0 + 64 * MSUB <= p.M && n0 + BN <= p.N;
            auto load_block = [&](int i2, f32x4 (&dst)[2][4]) {
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int m = row_w + 16 * (2 * i2 + ii), n = col_w + 16 * j;
                        dst[ii][j] = whole || (m < p.M && n < p.N)
                                         ? *reinterpret_cast<const f32x4*>(p.resid + (size_t)m * p.ld_resid + n)
                                         : f32x4{0.f, 0.f, 0.f, 0.f};
                    }
            };
            auto store_block = [&](int i2, const f32x4 (&src)[2][4]) {
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int m = row_w + 16 * (2 * i2 + ii), n = col_w + 16 * j;
                        f32x4 o;
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = __builtin_fmaf(gv[j][r], acc[2 * i2 + ii][j][r], src[ii][j][r]);
                        if (whole || (m < p.M && n < p.N)) *reinterpret_cast<f32x4*>(C + (size_t)m * p.ldc + n) = o;
                    }
            };
            if (whole) {
                load_block(0, rv[0]);
#pragma unroll
                for (int i2 = 0; i2 < MSUB; ++i2) {
                    if (i2 + 1 < MSUB) load_block(i2 + 1, rv[(i2 + 1) & 1]);
                    store_block(i2, rv[i2 & 1]);
                }
            } else {
                load_block(0, rv[0]);
#pragma unroll
                for (int i2 = 0; i2 < MSUB; ++i2) {
                    if (i2 + 1 < MSUB) load_block(i2 + 1, rv[(i2 + 1) & 1]);
                    store_block(i2, rv[i2 & 1]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2 * MSUB; ++i) {
                const int m = row_w + 16 * i;
                if (m >= p.M) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = col_w + 16 * j + r;
                        if (n < p.N)
                            C[(size_t)m * p.ldc + n] = __builtin_fmaf(p.gate[n], acc[i][j][r], p.resid[(size_t)m * p.ld_resid + n]);
                    }
            }
        }
        return;
    }
    typedef OutT out4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < 2 * MSUB; ++i) {
        const int m = row_w + 16 * i;
        if (m >= p.M) continue;
        if (epi_glu(EPI)) {
            // This wave's 64 W rows are 32 up rows then the 32 matching gate rows:
            // output columns 32 g .. 32 g + 31, g = (n0 + 64 wn) / 64.
            if (n0 + wn * 64 >= p.N) continue;
            OutT* c = static_cast<OutT*>(p.C) + (size_t)m * p.c_rs + (size_t)((n0 + wn * 64) >> 6) * p.c_ss + 4 * q16;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                out4 o;
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = OutT(acc[i][j][r] * glu_act<EPI == EPI_SWIGLU>(acc[i][j + 2][r]));
                if (p.vec) *reinterpret_cast<out4*>(c + 16 * j) = o;
                else
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[16 * j + r] = o[r];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = col_w + 16 * j;
                if (n >= p.N) continue;
                OutT* c = static_cast<OutT*>(p.C) + (size_t)m * p.ldc + n;
                if (p.vec) {
                    f32x4 v = acc[i][j];
                    if (p.bias) v += *reinterpret_cast<const f32x4*>(p.bias + n);
                    *reinterpret_cast<out4*>(c) = out4{OutT(v[0]), OutT(v[1]), OutT(v[2]), OutT(v[3])};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (n + r >= p.N) continue;
                        float v = acc[i][j][r];
                        if (p.bias) v += p.bias[n + r];
                        c[r] = OutT(v);
                    }
                }
            }
        }
    }
}

template <typename T, typename OutT, int EPI, int MODE>
__global__ void __launch_bounds__(512, 1) kernel(Params p)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * Ring<MODE != MODE_PLAIN>::STAGE];
    // Per-row partial sums of squares of the EPI_QKROPE epilogue: [wave][row group][16],
    // then a light chunk's [wave][16].
    __shared__ float red[EPI == EPI_QKROPE ? 8 * 8 * 16 + 8 * 16 : 1];
    // Items blockIdx.x, + gridDim.x, ...: with gridDim.x a multiple of 8 every item of
    // a workgroup maps to the XCD its blockIdx.x runs on.
    int bid = blockIdx.x, mt, nt, part, li;
    tile_of(p, bid, mt, nt, part, li);
    bool pre = false;
    for (;;) {
        const int nb = bid + (int)gridDim.x;
        int nmt = -1, nnt = 0, npart = 0, nli = -1;
        if (nb < p.items) tile_of(p, nb, nmt, nnt, npart, nli);
        if constexpr (MODE == MODE_HEAVY) {
            if (mt == p.m_full - 1) tile<T, OutT, EPI, 5, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
            else tile<T, OutT, EPI, 4, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
        } else if constexpr (MODE == MODE_RIDE) {
            tile<T, OutT, EPI, 4, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
        } else if constexpr (MODE == MODE_LIGHT) {
            const int xe = light_chunk(p, mt, nt);
            const int nxe = nmt >= 0 ? light_chunk(p, nmt, nnt) : -1;
            if (xe < 0) {
                tile<T, OutT, EPI, 4, MODE, 0>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red, -1, nxe);
            } else if constexpr (epi_glu(EPI)) {
                if (p.light_h == 32) tile<T, OutT, EPI, 4, MODE, 2>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red, xe, nxe);
                else tile<T, OutT, EPI, 4, MODE, 1>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red, xe, nxe);
            } else {
                tile<T, OutT, EPI, 4, MODE, 1>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red, xe, nxe);
            }
        } else {
            if (mt < p.m_full) tile<T, OutT, EPI, 4, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
            else if (p.tail_sub == 1) tile<T, OutT, EPI, 1, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
            else if (p.tail_sub == 2) tile<T, OutT, EPI, 2, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
            else tile<T, OutT, EPI, 3, MODE>(p, mt, nt, part, li, smem, pre, nmt, nnt, npart, nli, red);
        }
        if (nb >= p.items) break;
        bid = nb; mt = nmt; nt = nnt; part = npart; li = nli;
        pre = true;
    }
}

}  // namespace pingpong

// CUs of the current device, rounded down to a multiple of 8 (one per XCD slot). Every
// extern "C" entry point makes its context's device current first, so this is the CU
// count of the device the launch goes to.
static int cu_count()
{
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cached[dev] = n / 8 * 8;
    }
    return cached[dev];
}

// Q / K heads must not straddle a 256-column tile.
constexpr int BN_QK = 256;

// Chooses the light tiles of a launch with p.light set (p.light_mt), walking the
// kernel's items as the kernel walks them (workgroup b takes items b, b + grid, ...).
// First choice, a fixed pattern: chunk e of column block nt goes to M tile
// 4 e + (nt / 8 + e) mod 4 (M group e of the tile order, the offset turning every 8
// column blocks), taken when no workgroup then carries more than its even share,
// rounded up. Otherwise each (chunk, column block) goes to the tile of that column whose
// workgroup, then whose XCD (b % 8), carries the fewest light tiles so far, then the
// lowest M tile, never to a tile that already carries a chunk. (On the Q/K/V GEMM at
// 4160 tokens the pattern measured 344 us, the greedy choice 348 us, 361 us without
// its XCD term, which filled six XCDs and left two without light tiles; the up/gate
// GEMM's two 32-row chunks cannot be spread by the pattern.) True when no workgroup
// carries more than its share. The last few shapes' tables are remembered per thread.
static bool light_assign(pingpong::Params& p, int grid)
{
    struct Entry { int m_full, n_tiles, light_c, grid; bool ok; uint8_t mt[4][128]; };
    thread_local Entry cache[8];
    thread_local int next = 0;
    for (const Entry& e : cache)
        if (e.grid && e.m_full == p.m_full && e.n_tiles == p.n_tiles && e.light_c == p.light_c && e.grid == grid) {
            std::memcpy(p.light_mt, e.mt, sizeof p.light_mt);
            return e.ok;
        }
    bool ok = p.m_full <= 255 && p.n_tiles <= 128 && p.light_c <= 4;
    std::memset(p.light_mt, 0xff, sizeof p.light_mt);
    const int total = p.light_c * p.n_tiles, share = (total + grid - 1) / grid;
    if (ok) {
        std::vector<int> wg_of((size_t)p.m_full * p.n_tiles, -1), load(grid, 0), xcd_load(8, 0);
        for (int b = 0; b < p.items; ++b) {
            int mt, nt, part, li;
            pingpong::tile_of(p, b, mt, nt, part, li);
            wg_of[(size_t)mt * p.n_tiles + nt] = b % grid;
        }
        bool pattern = p.m_full >= pingpong::GM * p.light_c;
        for (int nt = 0; nt < p.n_tiles && pattern; ++nt)
            for (int e = 0; e < p.light_c && pattern; ++e) {
                const int mt = pingpong::GM * e + (nt / 8 + e) % pingpong::GM;
                const int w = wg_of[(size_t)mt * p.n_tiles + nt];
                pattern = w >= 0 && ++load[w] <= share;
                p.light_mt[e][nt] = (uint8_t)mt;
            }
        if (!pattern) {
            std::fill(load.begin(), load.end(), 0);
            std::memset(p.light_mt, 0xff, sizeof p.light_mt);
            std::vector<char> taken((size_t)p.m_full * p.n_tiles, 0);
            for (int nt = 0; nt < p.n_tiles && ok; ++nt)
                for (int e = 0; e < p.light_c && ok; ++e) {
                    int best = -1;
                    for (int mt = 0; mt < p.m_full; ++mt) {
                        const size_t t = (size_t)mt * p.n_tiles + nt;
                        if (wg_of[t] < 0 || taken[t]) continue;
                        if (best < 0) {
                            best = mt;
                            continue;
                        }
                        const int w = wg_of[t], bw = wg_of[(size_t)best * p.n_tiles + nt];
                        if (load[w] < load[bw] || (load[w] == load[bw] && xcd_load[w % 8] < xcd_load[bw % 8]))
                            best = mt;
                    }
                    ok = best >= 0;
                    if (ok) {
                        const size_t t = (size_t)best * p.n_tiles + nt;
                        taken[t] = 1;
                        ++load[wg_of[t]];
                        ++xcd_load[wg_of[t] % 8];
                        p.light_mt[e][nt] = (uint8_t)best;
                    }
                }
            ok = ok && *std::max_element(load.begin(), load.end()) <= share;
        }
    }
    Entry& slot = cache[next];
    slot = Entry{p.m_full, p.n_tiles, p.light_c, grid, ok, {}};
    std::memcpy(slot.mt, p.light_mt, sizeof p.light_mt);
    next = (next + 1) % 8;
    return ok;
}

int gemm16_pingpong(const GemmArgs& a, hipStream_t s)
{
    // No other kernel takes K-tiled operands or fuses the Q/K epilogue: shapes this one
    // rejects are errors then.
    const bool qk = a.epilogue == EPI_QKROPE;
    const int other = a.w_k32 || a.a_k32_rows || a.c_k32_rows || qk ? -1 : 1;
    if (qk && (a.c_dtype != a.dtype || !a.w_k32 || a.qk_cols <= 0 || a.qk_cols % BN_QK || a.qk_cols > a.N ||
               a.k_col <= 0 || a.k_col % 128 || a.k_col >= a.qk_cols || !a.gq || !a.gk || !a.cs_t ||
               (uintptr_t)a.cs_t % 16 || a.ldc % 4 || (uintptr_t)a.C % 8))
        return -1;
    if (a.dtype == DT_F32 || a.K % pingpong::BK) return other;
    if (a.epilogue == EPI_STORE && a.c_dtype != DT_F32 && a.c_dtype != a.dtype) return -1;
    if (epi_glu(a.epilogue) && a.c_dtype != a.dtype) return -1;
    // Buffer offsets are 32-bit: every staged row of every tile (rounded up to 256)
    // must lie below 2^31 bytes; larger operands take the register-staged kernel.
    const double ab = ((a.M + 255) / 256 * 256.0) * a.lda * 2, wb = ((a.N + 255) / 256 * 256.0) * a.ldw * 2;
    if (ab >= 2147483647.0 || wb >= 2147483647.0) return other;
    // K-tiled W: a stage's rows past N would alias the next K step, so N is whole tiles.
    if (a.w_k32 && (a.N % pingpong::BN || a.ldw != a.K)) return -1;
    // K-tiled A: every tile row, the tail's included, inside each 32-column slab.
    if (a.a_k32_rows && (a.a_k32_rows < (a.M + pingpong::BM - 1) / pingpong::BM * pingpong::BM || a.lda != a.K ||
                         (double)a.a_k32_rows * a.K * 2 >= 2147483647.0))
        return -1;
    if (a.c_k32_rows && (!epi_glu(a.epilogue) || a.c_k32_rows < a.M)) return -1;
    pingpong::Params p{};
    p.A = a.A; p.lda = a.lda; p.W = a.W; p.ldw = a.ldw; p.M = a.M; p.N = a.N; p.K = a.K;
    p.C = a.C; p.ldc = a.ldc; p.bias = a.bias; p.resid = a.resid; p.ld_resid = a.ld_resid; p.gate = a.gate;
    p.a_bytes = (uint32_t)(a.a_k32_rows ? (long)a.a_k32_rows * a.K * 2 : (long)a.M * a.lda * 2);
    p.a_row_bytes = a.a_k32_rows ? pingpong::ROWB : (int)(a.lda * 2);
    p.a_kstep = a.a_k32_rows ? a.a_k32_rows * pingpong::ROWB : pingpong::ROWB;
    p.c_rs = a.c_k32_rows ? 32 : a.ldc;
    p.c_ss = a.c_k32_rows ? 32L * a.c_k32_rows : 32;
    {
        auto aligned = [](const void* q, size_t b) { return (uintptr_t)q % b == 0; };
        const size_t out_bytes = a.epilogue == EPI_GATE_RESID || a.c_dtype == DT_F32 ? 4 : 2;
        bool v = aligned(a.C, 4 * out_bytes) && a.N % 4 == 0 &&
                 (epi_glu(a.epilogue) ? p.c_rs % 4 == 0 && p.c_ss % 4 == 0 : a.ldc % 4 == 0);
        if (a.epilogue == EPI_STORE && a.bias) v = v && aligned(a.bias, 16);
        if (a.epilogue == EPI_GATE_RESID) v = v && aligned(a.resid, 16) && aligned(a.gate, 16) && a.ld_resid % 4 == 0;
        p.vec = v;
    }
    p.qk_cols = a.qk_cols; p.k_col = a.k_col; p.gq = a.gq; p.gk = a.gk; p.cs_t = a.cs_t;
    p.qk_eps = a.qk_eps;
    p.w_bytes = (uint32_t)((long)a.N * a.ldw * 2);
    p.w_row_bytes = a.w_k32 ? pingpong::ROWB : (int)(a.ldw * 2);
    p.w_kstep = a.w_k32 ? a.N * pingpong::ROWB : pingpong::ROWB;
    p.m_full = a.M / pingpong::BM;
    p.tail_sub = (a.M % pingpong::BM + 63) / 64;
    p.n_tiles = (a.N + pingpong::BN - 1) / pingpong::BN;
    // Split the tail row of tiles along K so that its items cover the CUs once
    // (at most 16 parts, at least 4 K steps each), within the caller's workspace.
    // With M < 256 the tail row is the whole GEMM (a short prompt's projections).
    p.split = 1;
    p.split_all = 0;
    p.heavy = 0;
    p.m_main = p.m_full;
    const int m_tiles = p.m_full + (p.tail_sub ? 1 : 0);
    const int full = p.m_full * p.n_tiles;
    // A tail of at most 64 rows under whole rounds of full tiles, with an epilogue that
    // finishes rows within the tile (the block's Q/K/V projection with the Q/K norm and
    // rotary, and its up/gate projection, at 4096 image + 64 text tokens): light tiles
    // (Params::light). Each adds a 16- or 32-row chunk of the tail, a sixteenth or an
    // eighth more MFMAs, and no workgroup gets more than its share of them, so the
    // launch ends that much later per light tile a workgroup carries, with no tail phase
    // streaming all of W for 64 rows and no reduction launch. The Q/K/V GEMM takes
    // 16-row chunks (192 light tiles, at most one per workgroup: 362 -> 347 us against
    // the split tail). A GLU epilogue over two or more rounds takes 32-row chunks: the
    // up/gate GEMM then has 192 light tiles, at most one per workgroup, where 16-row
    // chunks gave 384, two per workgroup on half of them (no faster than the heavy last
    // row).
    p.light = 0;
    p.light_c = 0;
    p.light_h = 16;
    {
        const bool glu_rounds = epi_glu(a.epilogue) && full >= 2 * cu_count();
        const int tail_rows = a.M % pingpong::BM, h = glu_rounds ? 32 : 16, chunks = (tail_rows + h - 1) / h;
        if ((qk || epi_glu(a.epilogue) || a.epilogue == EPI_STORE) && tail_rows > 0 && tail_rows <= 64 &&
            full >= cu_count() && full % cu_count() == 0 && p.m_full >= chunks) {
            p.light = 1;
            p.light_c = chunks;
            p.light_h = h;
            p.items = full;
            if (!light_assign(p, cu_count())) {
                p.light = 0;
                p.light_c = 0;
                p.light_h = 16;
            }
        }
    }
    // A tail of at most 64 rows under at least two rounds of full tiles, when light
    // tiles do not apply: the last row of full tiles takes the tail rows as 320-row
    // tiles, one per workgroup in the last round, which then ends a quarter of a tile
    // later instead of being followed by a tail phase and a reduction launch. (The Q/K
    // epilogue would not fit 320 rows in registers.)
    if (!p.light && a.epilogue == EPI_GEGLU && p.tail_sub == 1 && p.m_full >= 1 &&
        (long)p.m_full * p.n_tiles >= 2L * cu_count()) {
        p.heavy = 1;
        p.m_main = p.m_full - 1;
    }
    if (!p.heavy && !p.light && a.split_ws && p.m_full && m_tiles * p.n_tiles <= kSplitTargetItems / 2) {
        // Too few tiles for the CUs (a short sequence's narrow projections): split
        // every tile along K, at least 4 K steps per part.
        const size_t per_part = (size_t)m_tiles * p.n_tiles * pingpong::BM * pingpong::BN * sizeof(float);
        int sp = std::min(kMaxSplit, kSplitTargetItems / (m_tiles * p.n_tiles));
        sp = std::min(sp, std::max(1, a.K / pingpong::BK / 4));
        while (sp > 1 && (size_t)sp * per_part > a.split_ws_bytes) --sp;
        if (sp > 1) {
            p.split = sp;
            p.split_all = 1;
            p.part = static_cast<float*>(a.split_ws);
        }
    }
    // A tail of at most 64 rows under whole rounds of full tiles (the block's output and
    // down projections): the full tiles compute it while they hold W (Params::ride),
    // m_full K ranges of it, one per row of full tiles. (The Q/K/V projection keeps its
    // 5-part split tail: with 16 parts its reduction would read three times as much.)
    p.ride = 0;
    if (!p.heavy && !p.light && !p.split_all && a.split_ws && a.epilogue == EPI_GATE_RESID &&
        p.tail_sub == 1 && p.m_full >= 2 && p.m_full <= kMaxSplit && a.K / pingpong::BK >= p.m_full &&
        full >= cu_count() && full % cu_count() == 0 &&
        (size_t)p.m_full * p.n_tiles * 64 * pingpong::BN * sizeof(float) <= a.split_ws_bytes) {
        p.ride = 1;
        p.split = p.m_full;
        p.part = static_cast<float*>(a.split_ws);
    }
    if (!p.heavy && !p.ride && !p.light && !p.split_all && p.tail_sub && a.split_ws) {
        const size_t per_part = (size_t)p.n_tiles * 64 * p.tail_sub * pingpong::BN * sizeof(float);
        int sp = std::min(kMaxSplit, std::max(1, kSplitTargetItems / p.n_tiles));
        sp = std::min(sp, std::max(1, a.K / pingpong::BK / 4));
        while (sp > 1 && (size_t)sp * per_part > a.split_ws_bytes) --sp;
        p.split = sp;
        p.part = static_cast<float*>(a.split_ws);
    }
    // A last round of workgroups at most half full (the full tiles modulo one per
    // CU): split those tiles along K so that round fills the CUs with shorter
    // items. Their partials follow the tail row's in the workspace.
    p.late = 0;
    p.late_split = 1;
    p.late_part = nullptr;
    const int last_round = full % kSplitTargetItems;
    // (Not for the fused Q/K epilogue, whose rows are finished per tile.)
    if (!qk && !p.heavy && !p.ride && !p.light && !p.split_all && a.split_ws && full > kSplitTargetItems &&
        last_round <= kSplitTargetItems / 2 && last_round > 0) {
        const size_t tail_bytes =
            p.tail_sub ? ((size_t)p.split * p.n_tiles * 64 * p.tail_sub * pingpong::BN * sizeof(float) + 255) / 256 * 256 : 0;
        const size_t per_part = (size_t)last_round * pingpong::BM * pingpong::BN * sizeof(float);
        int sp = std::min(kMaxSplit, kSplitTargetItems / last_round);
        sp = std::min(sp, std::max(1, a.K / pingpong::BK / 4));
        while (sp > 1 && tail_bytes + (size_t)sp * per_part > a.split_ws_bytes) --sp;
        if (sp > 1) {
            p.late = last_round;
            p.late_split = sp;
            p.late_part = reinterpret_cast<float*>(static_cast<char*>(a.split_ws) + tail_bytes);
        }
    }
    const int tiles = p.split_all ? m_tiles * p.n_tiles * p.split
                      : p.heavy || p.ride || p.light ? full
                                  : full - p.late + p.late * p.late_split + (p.tail_sub ? p.n_tiles * p.split : 0);
    // One workgroup per CU (the LDS ring allows no second), each walking its items.
    p.items = tiles;
    const dim3 grid(std::min(tiles, cu_count())), block(512);
    // Fused Q/K epilogue: tiles whose every part is split (split_all) are stored as they
    // are and the whole GEMM is normalised and rotated afterwards; otherwise the full
    // tiles are finished in the epilogue and only a split tail row needs that pass.
    const int epi = qk && p.split_all ? EPI_STORE : a.epilogue;
#define EHIP_PINGPONG(T)                                                                                            \
    do {                                                                                                      \
        if (p.light) {                                                                                        \
            if (epi == EPI_QKROPE)                                                                            \
                hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_QKROPE, pingpong::MODE_LIGHT>), grid, block, 0, s, p); \
            else if (epi == EPI_STORE && a.c_dtype == DT_F32)                                                 \
                hipLaunchKernelGGL((pingpong::kernel<T, float, EPI_STORE, pingpong::MODE_LIGHT>), grid, block, 0, s, p); \
            else if (epi == EPI_STORE)                                                                        \
                hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_STORE, pingpong::MODE_LIGHT>), grid, block, 0, s, p); \
            else if (epi == EPI_SWIGLU)                                                                       \
                hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_SWIGLU, pingpong::MODE_LIGHT>), grid, block, 0, s, p); \
            else                                                                                              \
                hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_GEGLU, pingpong::MODE_LIGHT>), grid, block, 0, s, p); \
        } else if (p.heavy) {                                                                                 \
            hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_GEGLU, pingpong::MODE_HEAVY>), grid, block, 0, s, p);    \
        } else if (p.ride) {                                                                                  \
            hipLaunchKernelGGL((pingpong::kernel<T, float, EPI_GATE_RESID, pingpong::MODE_RIDE>), grid, block, 0, s, p); \
        } else if (epi == EPI_QKROPE) {                                                                       \
            hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_QKROPE, false>), grid, block, 0, s, p);                  \
        } else if (epi == EPI_STORE) {                                                                        \
            if (a.c_dtype == DT_F32) hipLaunchKernelGGL((pingpong::kernel<T, float, EPI_STORE, false>), grid, block, 0, s, p); \
            else hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_STORE, false>), grid, block, 0, s, p);              \
        } else if (a.epilogue == EPI_GATE_RESID) {                                                            \
            hipLaunchKernelGGL((pingpong::kernel<T, float, EPI_GATE_RESID, false>), grid, block, 0, s, p);          \
        } else if (a.epilogue == EPI_SWIGLU) {                                                                \
            hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_SWIGLU, false>), grid, block, 0, s, p);                  \
        } else {                                                                                              \
            hipLaunchKernelGGL((pingpong::kernel<T, T, EPI_GEGLU, false>), grid, block, 0, s, p);                   \
        }                                                                                                     \
    } while (0)
    if (a.dtype == DT_F16) EHIP_PINGPONG(f16);
    else EHIP_PINGPONG(bf16);
#undef EHIP_PINGPONG
    if (p.split > 1 || p.late) {
        const long cols = epi_glu(a.epilogue) ? a.N / 2 : a.N;
        // Four columns per thread when every row and vector is 16-byte aligned.
        const int V = p.vec && cols % 4 == 0 ? 4 : 1;
        const long items = ((p.split > 1 ? (long)(p.split_all ? a.M : 64 * p.tail_sub) * cols : 0) +
                            (long)p.late * pingpong::BM * (epi_glu(a.epilogue) ? pingpong::BN / 2 : pingpong::BN)) /
                           V;
        const dim3 rgrid((unsigned)((items + 255) / 256)), rblock(256);
#define EHIP_REDUCE(OUT, EPI)                                                                                   \
    do {                                                                                                        \
        if (V == 4) hipLaunchKernelGGL((pingpong::split_reduce_kernel<OUT, EPI, 4>), rgrid, rblock, 0, s, p);   \
        else hipLaunchKernelGGL((pingpong::split_reduce_kernel<OUT, EPI, 1>), rgrid, rblock, 0, s, p);          \
    } while (0)
        if (qk) {
            // Split rows are summed as they are (permuted Q / K columns) ...
            if (a.dtype == DT_F16) EHIP_REDUCE(f16, EPI_STORE);
            else EHIP_REDUCE(bf16, EPI_STORE);
        } else if (a.epilogue == EPI_STORE) {
            if (a.c_dtype == DT_F32) EHIP_REDUCE(float, EPI_STORE);
            else if (a.dtype == DT_F16) EHIP_REDUCE(f16, EPI_STORE);
            else EHIP_REDUCE(bf16, EPI_STORE);
        } else if (a.epilogue == EPI_GATE_RESID) {
            EHIP_REDUCE(float, EPI_GATE_RESID);
        } else if (a.epilogue == EPI_SWIGLU) {
            if (a.dtype == DT_F16) EHIP_REDUCE(f16, EPI_SWIGLU);
            else EHIP_REDUCE(bf16, EPI_SWIGLU);
        } else {
            if (a.dtype == DT_F16) EHIP_REDUCE(f16, EPI_GEGLU);
            else EHIP_REDUCE(bf16, EPI_GEGLU);
        }
#undef EHIP_REDUCE
    }
    if (qk && p.split > 1) {
        // ... and then normalised, rotated and put in natural order: every row when all
        // tiles were split, else the tail rows.
        const int r0 = p.split_all ? 0 : p.m_full * pingpong::BM;
        const int rc = qk_norm_rope_permuted(a.C, a.dtype, r0, a.M, (int)(a.k_col / 128),
                                             (int)((a.qk_cols - a.k_col) / 128), a.ldc, a.k_col, a.gq, a.gk, a.cs_t,
                                             a.qk_eps, s);
        if (rc) return rc;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -int(e);
}

}  // namespace ehip
