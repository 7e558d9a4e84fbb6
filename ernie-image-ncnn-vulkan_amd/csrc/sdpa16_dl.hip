// SPDX-License-Identifier: MIT
// Flash SDPA for 16-bit operands with head_dim 128 on gfx950: the path the DiT
// block takes (ErnieSDPA, src/ernie_attention.cpp:35-233; sdpa_22 in
// block.ncnn.param line 58) with no mask, one additive mask row broadcast over the
// queries or a per-query mask (src/ernie_attention.cpp:201-221), plus a
// valid-key bound. Every mask form goes through the same arithmetic, so a row
// mask and its dense broadcast give bitwise identical results.
//
//   * One workgroup = 4 waves = 128 queries of one head (8 waves = 256 queries when the
//     unmasked problem has whole 256-query tiles); each wave holds its 32 queries' Q
//     fragments in registers and computes S^T = K Q^T with v_mfma_f32_16x16x32 on
//     16-key x 16-query blocks, so each lane owns two query columns (one per 16-query
//     block) and the probabilities are already the Y operand of O^T = V^T P^T. Under
//     this load the 16x16x32 form holds a higher clock than 32x32x16 (a probe of both
//     at equal work: 2.04 against 1.77 GHz). The four lanes l % 16 + 16 g share a
//     query: the tile maximum is exchanged with v_permlane16/32_swap (VALU, no LDS
//     round trip) and the row sums are kept per lane and combined after the last tile.
//   * exp2 is the bare v_exp_f32: results below 2^-126 flush to zero, which cannot
//     move a row sum that is at least 1.
//   * K and V tiles (64 keys) reach LDS through direct global->LDS loads into two
//     two-stage rings, K one tile ahead of V: no VGPR staging, no transpose on the
//     way in. Key rows at or past the valid-key bound lie past the buffer range and
//     load as zeros.
//   * Software pipeline: while the matrix cores compute S of tile i+1, the VALU turns
//     S of tile i into probabilities, in 16 hand-ordered groups (K fragment n + 2
//     read, fragment n awaited, its two MFMAs with a probability after each) that
//     sched_barrier keeps in order; then P_i V_i accumulates and tile i+1's maximum
//     is taken. The LDS reads are inline assembly with explicit lgkmcnt waits (see
//     ds_read_tr).
//   * Row sums use v_dot2_f32_{f16,bf16} on the rounded probabilities the MFMA
//     consumes, so numerator and denominator see the same weights.
//   * V^T fragments come from ds_read_b64_tr_b16: within each 16-lane group, lane
//     i receives the (i % 4)-th 16-bit value at the addresses of lanes 4e + i/4
//     (e = 0..3), so lanes pointing at 4 consecutive key rows deliver 4 keys of
//     one head-dim column per lane. The MFMA sums over its 32 k positions in any
//     order, so P and V^T only have to agree on which key sits at which position:
//     positions 8 g .. 8 g + 7 hold keys 4 g + 0..3 and 16 + 4 g + 0..3 of the
//     32-key chunk, the keys a lane's S^T accumulators already hold.
//   * K rows are chunk-swizzled by (key & 15), V rows by 2 (key & 7) (32-byte
//     pairs kept together for the transposing reads): both measured conflict-free
//     for these read patterns.
//   * Causal mode (key k visible to query q iff k <= q + sk - sq): a workgroup's
//     key loop ends at the tile holding its last query's diagonal, and only tiles
//     that cross a wave's diagonal are masked, per lane, without a mask tensor.
//   * Online softmax in the log2 domain; the running offset is raised only when a
//     tile's maximum exceeds it by more than 8, so the O / l rescale is almost
//     always skipped (exact: O and l share the offset).
#include "common.hpp"
#include "kernels.hpp"

namespace ehip {
namespace {
// Key-range parts of a partial last query tile, summed over the heads: 192, i.e. 6
// parts per head at 32 heads. The parts run in the slots the last full tiles leave
// free as they finish unevenly; at 4096 image + 64 text tokens, 4, 6 and 8 parts per
// head measured 290-291 us against 293-294 us for 16 (one per slot of the 256 CUs x 2),
// whose shorter parts cost more in the merge and in per-part start-up than they save
// at the end of the launch.
constexpr int kSdpaSlots = 192;
}
namespace sdl {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int BKV = 64, D = 128;
constexpr int ROWB = D * 2;                 // 256 bytes per staged key row
constexpr int KV_BYTES = BKV * ROWB;        // 16 KiB
constexpr int KSTAGE = KV_BYTES + BKV * 4;  // K tile + its mask row
constexpr int V_BASE = 2 * KSTAGE;           // the V ring follows the two K stages
constexpr int LDS_BYTES = V_BASE + 2 * KV_BYTES;
constexpr uint32_t kRsrcFlags = 0x00020000;
constexpr float kRescaleSlack = 8.0f;
// A tile whose maximum was not taken before its softmax (see step) has it taken after
// all when its probabilities sum to at least this much: below it every probability is
// below 2^6, so the tile maximum is below offset + 6 and could not raise the offset.
constexpr float kLazyCheck = 64.0f;
constexpr int kMaxParts = 16;  // most key-range parts of the split query tile

struct Params {
    const void* q; const void* k; const void* v; void* o;
    int heads, group, sq, sk, kv_end;
    long q_hs, q_rs, k_hs, k_rs, v_hs, v_rs, o_hs, o_rs;
    long o_ds;  // element distance between the four 32-value groups of an output row
    const float* mask; long mask_hs;  // additive FP32 mask: one row [sk] or per query [sq][sk] per head
    float scale_log2;
    int causal, qk_off;  // causal: keys > query + qk_off (= sk - sq) excluded
    // Split of the last, partial query tile (sq % part_rows queries, part_rows = the
    // workgroup's queries) along the keys: tail_parts > 0 parts per head write
    // unnormalised FP32 O and their (m, l) to part_o [heads * tail_parts][part_rows][128]
    // / part_ml [heads * tail_parts][part_rows][2].
    int full_qt, tail_parts, part_rows;
    float* part_o;
    float* part_ml;
};

// Merges the key-range parts of the split query tile: O = sum_p O_p 2^(m_p - M) /
// sum_p l_p 2^(m_p - M) with M = max_p m_p (log2 domain). One wave per (head, query):
// the query's (m, l) of every part are wave-uniform loads, and lane l merges values
// 2l and 2l + 1 with one 8-byte load per part.
template <typename T>
__global__ void __launch_bounds__(256) combine_kernel(Params p, int tail_q)
{
    const int wq = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
    if (wq >= p.heads * tail_q) return;
    const int lane = threadIdx.x & 63;
    const int h = wq / tail_q, ql = wq - h * tail_q;
    const float* ml = p.part_ml + ((size_t)h * p.tail_parts * p.part_rows + ql) * 2;
    const float* po = p.part_o + ((size_t)h * p.tail_parts * p.part_rows + ql) * D + 2 * lane;
    // Every part's loads are issued before the first use (at most kMaxParts parts);
    // the merge then runs in part order.
    float mv[kMaxParts], lv[kMaxParts];
    f32x2 ov[kMaxParts];
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
        if (q < p.tail_parts) {
            mv[q] = ml[(size_t)q * p.part_rows * 2];
            lv[q] = ml[(size_t)q * p.part_rows * 2 + 1];
            ov[q] = *reinterpret_cast<const f32x2*>(po + (size_t)q * p.part_rows * D);
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
        if (q < p.tail_parts) M = fmaxf(M, mv[q]);
    float L = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
        if (q < p.tail_parts) {
            const float w = mv[q] == -INFINITY ? 0.f : exp2f(mv[q] - M);
            L += lv[q] * w;
            O0 += ov[q][0] * w;
            O1 += ov[q][1] * w;
        }
    }
    const int qi = p.full_qt * p.part_rows + ql, d = 2 * lane;
    typedef T t2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<t2*>(static_cast<T*>(p.o) + (size_t)h * p.o_hs + (size_t)qi * p.o_rs + (size_t)(d >> 5) * p.o_ds +
                           (d & 31)) = t2{T(O0 / L), T(O1 / L)};
}

template <typename T> struct Mfma;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <> struct Mfma<f16> {
    typedef f16x8 vec;
    // acc + the sum of the 8 probabilities, as stored for the MFMA (v_dot2_f32_f16 against 1).
    static __device__ __forceinline__ float rowsum(vec p, float acc)
    {
        const f16x2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
        for (int i = 0; i < 8; i += 2) acc = __builtin_amdgcn_fdot2(f16x2{p[i], p[i + 1]}, one, acc, false);
        return acc;
    }
    // D = X Y^T on 16 x 16 blocks with k = 32: lane l supplies row l % 16 of X and of Y
    // at k = 8 (l / 16) .. + 7 and receives D[4 (l / 16) + r][l % 16], r = 0..3.
    static __device__ __forceinline__ f32x4 run(vec x, vec y, f32x4 c)
    { return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c, 0, 0, 0); }
};
template <> struct Mfma<bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ float rowsum(vec p, float acc)
    {
        const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
        for (int i = 0; i < 8; i += 2) acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p[i], p[i + 1]}, one, acc, false);
        return acc;
    }
    static __device__ __forceinline__ f32x4 run(vec x, vec y, f32x4 c)
    { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c, 0, 0, 0); }
};

// K rows: 16-byte chunk c of key row r at physical chunk c ^ (r & 15).
// V rows: chunk c at c ^ 2(r & 7), which keeps each 32-byte pair together for the
// transposing reads (4 keys x 32 bytes per 16-lane group).
__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int r) { return 2 * (r & 7); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// max(a, b, c) in one v_max3_f32. Written out because the compiler otherwise
// canonicalises every MFMA result before a two-input v_max (NaN-quieting that
// scores never need), tripling the instruction count of the tile maximum.
__device__ __forceinline__ float max3(float a, float b, float c)
{
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// max / sum over lanes l, l ^ 16, l ^ 32 and l ^ 48, the four lanes that hold one
// query's scores: v_permlane16_swap exchanges 16-lane rows 0 <-> 1 and 2 <-> 3,
// v_permlane32_swap the two halves (VALU, no LDS round trip). All four lanes get the
// same bits: the sum is (r0 + r1) + (r2 + r3) in every one of them.
__device__ __forceinline__ float quad_max(float x)
{
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float quad_sum(float x)
{
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16 (see the V^T fragments below) as inline assembly. Through the
// builtin, the compiler treats the read as possibly aliasing the K / V tiles still
// in flight from the direct global->LDS loads and waits for all of them (vmcnt(0))
// before the first read, which would expose the prefetch latency in every step.
// The tile read here always landed before the step's barrier, so only the LDS
// counter matters: lgkm_wait_for waits until at most `after` LDS operations are
// outstanding and names the destination registers, so no consumer of them can be
// scheduled above the wait. LDS operations complete in order, so counting only the
// reads issued here after the awaited one is enough (anything else in flight only
// makes the wait stricter).
__device__ __forceinline__ u32x2 ds_read_tr(uint32_t addr, int offset)
{
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(offset));
    return r;
}
__device__ __forceinline__ void lgkm_wait_for(u32x2& a, u32x2& b, int after)
{
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(after));
}
// ds_read_b128 of a K fragment the same way (with the builtin load the compiler
// could not keep a second fragment in flight at this register pressure).
__device__ __forceinline__ u32x4 ds_read_b128(uint32_t addr, int offset)
{
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(offset));
    return r;
}
__device__ __forceinline__ void lgkm_wait_for(u32x4& a, int after)
{
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(after));
}

// a ^ imm in one VALU instruction that the compiler keeps where it is written
// (hoisted out of the key loop it would hold one register per immediate).
__device__ __forceinline__ uint32_t xor_imm(uint32_t a, int imm)
{
    uint32_t r;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "i"(imm), "v"(a));
    return r;
}

// Workgroup barrier without the release fence of __syncthreads() (that fence would
// also wait for the tile still being loaded): LDS reads issued before it have
// returned and the memory clobber keeps LDS accesses on their side.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A workgroup of NW waves: BQW queries, and RPW key rows of each tile loaded per wave
// by IPW 1-KiB instructions.
template <int NW> struct Waves {
    static constexpr int BQW = 32 * NW, RPW = BKV / NW, IPW = RPW / 4;
};

// Mask modes: none, one row broadcast over the queries, one row per query.
enum { MASK_NONE = 0, MASK_ROW = 1, MASK_DENSE = 2 };

template <typename T, int MM, int NW>
__global__ void __launch_bounds__(64 * NW, 8 / NW) kernel(Params p)
{
    typedef typename Mfma<T>::vec vec8;
    constexpr int BQW = Waves<NW>::BQW, RPW = Waves<NW>::RPW, IPW = Waves<NW>::IPW;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];

    // Workgroup -> (head, query tile[, key range]). Workgroup b runs on XCD b % 8:
    // each XCD takes a contiguous range of full query tiles (so a head's K / V stream
    // into one L2) and then its share of the key-range parts of the split tail tile,
    // which therefore run last and fill the CUs.
    const int ntiles = (p.kv_end + BKV - 1) / BKV;
    int h, q_base, it0 = 0, it1 = ntiles, part = -1;
    {
        const int full = p.tail_parts ? p.full_qt * p.heads : ((p.sq + BQW - 1) / BQW) * p.heads;
        const int tail = p.tail_parts * p.heads;
        const int qt = p.tail_parts ? p.full_qt : (p.sq + BQW - 1) / BQW;
        const int bid = blockIdx.x;
        int f = -1, u = -1;
        if ((full & 7) == 0 && (tail & 7) == 0) {
            const int x = bid & 7, j = bid >> 3, per = full >> 3;
            if (j < per) f = x * per + j;
            else u = x * (tail >> 3) + (j - per);
        } else {
            if (bid < full) f = bid;
            else u = bid - full;
        }
        if (f >= 0) {
            h = f / qt;
            q_base = (f - h * qt) * BQW;
        } else {
            h = u / p.tail_parts;
            part = u - h * p.tail_parts;
            q_base = p.full_qt * BQW;
        }
        // Causal: no key tile past the one holding the last query's diagonal.
        const int nt = p.causal ? min(ntiles, (min(q_base + BQW, p.sq) - 1 + p.qk_off) / BKV + 1) : ntiles;
        it1 = nt;
        if (part >= 0) {
            it0 = (int)((long)nt * part / p.tail_parts);
            it1 = (int)((long)nt * (part + 1) / p.tail_parts);
        }
    }
    const int kvh = h / p.group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    // Each lane holds two queries, one of each 16-query block qb of its wave's 32.
    auto my_q = [&](int qb) { return q_base + wave * 32 + 16 * qb + l16; };
    // Keys at or past key_lim are excluded: the valid-key bound, and the diagonal when causal.
    auto key_lim = [&](int qb) { return p.causal ? min(p.kv_end, my_q(qb) + 1 + p.qk_off) : p.kv_end; };
    // A wave whose 32 queries all lie past sq (in a partial last query tile) only loads
    // its share of the K / V tiles and keeps the barriers.
    const bool active = q_base + wave * 32 < p.sq;

    // Q fragments (Y of S^T = K Q^T): query block qb, head-dim chunk dc: row my_q[qb],
    // values 32 dc + 8 g .. + 7.
    const T* Q = static_cast<const T*>(p.q) + (size_t)h * p.q_hs;
    vec8 qf[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const T* qrow = Q + (size_t)min(my_q(qb), p.sq - 1) * p.q_rs;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) qf[qb][dc] = *reinterpret_cast<const vec8*>(qrow + 32 * dc + 8 * g);
    }

    // Key rows past kv_end lie past the buffer range and load as zeros.
    const T* Kh = static_cast<const T*>(p.k) + (size_t)kvh * p.k_hs;
    const T* Vh = static_cast<const T*>(p.v) + (size_t)kvh * p.v_hs;
    const uint32_t k_bytes = (uint32_t)(((long)(p.kv_end - 1) * p.k_rs + D) * 2);
    const uint32_t v_bytes = (uint32_t)(((long)(p.kv_end - 1) * p.v_rs + D) * 2);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(Kh), (short)0, k_bytes, kRsrcFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(Vh), (short)0, v_bytes, kRsrcFlags);
    constexpr bool MASKROW = MM == MASK_ROW, DENSE = MM == MASK_DENSE;
    __amdgpu_buffer_rsrc_t rm;
    if constexpr (DENSE)
        rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.mask + (size_t)h * p.mask_hs), (short)0,
                                               (uint32_t)((size_t)p.sq * p.sk * 4), kRsrcFlags);
    else if constexpr (MASKROW)
        rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.mask + (size_t)h * p.mask_hs), (short)0,
                                               (uint32_t)(p.sk * 4), kRsrcFlags);

    // Direct loads: wave w fills key rows [RPW w, RPW (w + 1)) of the K and V tiles with
    // IPW 1-KiB instructions each (4 rows x 256 bytes); lane l lands at row l >> 4,
    // physical chunk l & 15. K (with its mask row) and V have rings of their own
    // because K runs one tile ahead of V.
    uint32_t k_src[4], v_src[4];  // IPW <= 4 used
#pragma unroll
    for (int q = 0; q < IPW; ++q) {
        const int row = wave * RPW + q * 4 + (lane >> 4);
        k_src[q] = (uint32_t)(((long)row * p.k_rs * 2) + (((lane & 15) ^ kswz(row)) << 4));
        v_src[q] = (uint32_t)(((long)row * p.v_rs * 2) + (((lane & 15) ^ vswz(row)) << 4));
    }
    const uint32_t k_tile = (uint32_t)(BKV * p.k_rs * 2), v_tile = (uint32_t)(BKV * p.v_rs * 2);
    auto kstage = [&](int slot) { return smem + slot * KSTAGE; };
    auto vstage = [&](int slot) { return smem + V_BASE + slot * KV_BYTES; };
    auto issue_k = [&](int it, int slot) {
        uint8_t* st = kstage(slot);
#pragma unroll
        for (int q = 0; q < IPW; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(st + (wave * RPW + q * 4) * ROWB), 16, k_src[q],
                                                     it * k_tile, 0, 0);
        if constexpr (MASKROW) {
            if (wave == 0)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr_t)(st + KV_BYTES), 4, lane * 4, it * BKV * 4, 0, 0);
        }
    };
    auto issue_v = [&](int it, int slot) {
        uint8_t* st = vstage(slot);
#pragma unroll
        for (int q = 0; q < IPW; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(st + (wave * RPW + q * 4) * ROWB), 16, v_src[q],
                                                     it * v_tile, 0, 0);
    };

    // K fragment (X of S^T = K Q^T) of key block kb (16 keys) and head-dim chunk dc: key
    // 16 kb + l16, logical chunk 4 dc + g. The swizzle depends on l16 only, so the
    // per-lane LDS addresses (of stage 0) are fixed per dc and the key-block and stage
    // offsets fold into the reads' immediate offsets.
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
    uint32_t k_addr[4];
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) k_addr[dc] = lds0 + l16 * ROWB + (((4 * dc + g) ^ kswz(l16)) << 4);
    // V^T fragment (X of O^T = V^T P^T) of head-dim block db (16 values) and key chunk kc
    // (32 keys) by two transposing reads: lane j = l16 of 16-lane group g points at key
    // 32 kc + 4 g + j / 4 (lo) or that + 16 (hi), values 16 db + 4 (j % 4) .. + 3, and
    // receives value 16 db + j of keys 32 kc + 4 g + 0..3 (lo) and 32 kc + 16 + 4 g + 0..3
    // (hi): the MFMA's k positions 8 g .. 8 g + 7 in that order. The swizzle 2 (key & 7)
    // is fixed per lane: db's 32-byte pair lands at pair db ^ (key & 7), so the address
    // of db is v_base ^ 32 db (v_base's bits 5-7 hold the lane's pair, the rest of the
    // address has none there); the XOR is issued with the read, which keeps one
    // register per lane instead of eight.
    const int v_key = 4 * g + (l16 >> 2);
    const uint32_t v_base = lds0 + V_BASE + v_key * ROWB + ((v_key & 7) << 5) + (((l16 & 3) >> 1) << 4) +
                            (((4 * (l16 & 3)) & 7) << 1);

    // O^T accumulators: oacc[db][qb][r] = value 16 db + 4 g + r of query my_q[qb].
    f32x4 oacc[8][2];
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) oacc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    const float c = p.scale_log2;

    // S^T of one key tile: sacc[qb][kb][r] = score of key 16 kb + 4 g + r for query
    // my_q[qb]. With a mask the accumulators start at mask / scale, so the scaled score
    // is s c + mask log2(e) without holding the mask in registers. A row mask comes
    // from LDS; a per-query mask row is read straight from memory (its keys past sk
    // read as zero through the buffer range, and fall past kv_end anyway).
    const float inv_scale = kLog2e / c;
    auto dense_row = [&](int qb) { return (uint32_t)(min(my_q(qb), p.sq - 1) * p.sk) * 4u; };
    auto qk_init = [&](const uint8_t* ks, int kv0, f32x4 (&sacc)[2][4]) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kk = 16 * kb + 4 * g + r;
                if constexpr (MASKROW) {
                    const float mv = reinterpret_cast<const float*>(ks + KV_BYTES)[kk] * inv_scale;
                    sacc[0][kb][r] = mv;
                    sacc[1][kb][r] = mv;
                } else if constexpr (DENSE) {
#pragma unroll
                    for (int qb = 0; qb < 2; ++qb) {
                        const float mv = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rm, dense_row(qb) + (uint32_t)(kv0 + kk) * 4u, 0, 0));
                        sacc[qb][kb][r] = mv * inv_scale;
                    }
                } else {
                    sacc[0][kb][r] = 0.f;
                    sacc[1][kb][r] = 0.f;
                }
            }
    };
    // K fragment n of the tile in stage `slot` (a compile-time constant at every call):
    // head-dim chunk n / 4, key block n % 4. Each feeds the MFMAs of both query blocks,
    // and an accumulator is used again only four fragments (eight MFMAs) later.
    auto kfrag = [&](int slot, int n) { return ds_read_b128(k_addr[n >> 2], slot * KSTAGE + (n & 3) * 16 * ROWB); };
    // Wait for K fragment n when fragments up to n + 2 have been issued.
    auto kwait = [&](u32x4& f, int n) { lgkm_wait_for(f, n + 2 < 16 ? 2 : 15 - n); };
    auto qk = [&](int slot, int kv0, f32x4 (&sacc)[2][4]) {
        qk_init(kstage(slot), kv0, sacc);
        u32x4 kf[16];
        kf[0] = kfrag(slot, 0);
        kf[1] = kfrag(slot, 1);
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            if (n + 2 < 16) kf[n + 2] = kfrag(slot, n + 2);
            kwait(kf[n], n);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                sacc[qb][n & 3] = Mfma<T>::run(__builtin_bit_cast(vec8, kf[n]), qf[qb][n >> 2], sacc[qb][n & 3]);
        }
    };
    // Tiles whose scores are masked per lane here: past the valid keys, or (causal)
    // across this wave's diagonal, or any tile under a mask tensor.
    auto needs_prep = [&](int it) {
        const int kv0 = it * BKV;
        return MM != MASK_NONE || kv0 + BKV > p.kv_end || (p.causal && kv0 + BKV - 1 > q_base + wave * 32 + p.qk_off);
    };
    // Tile maximum of query block qb in the log2 domain (scores already scaled by c
    // when `scaled`).
    auto tile_max = [&](const f32x4 (&sacc)[2][4], int qb, bool scaled) {
        float tmax = max3(sacc[qb][0][0], sacc[qb][0][1], sacc[qb][0][2]);
#pragma unroll
        for (int i = 3; i < 15; i += 2)
            tmax = max3(tmax, sacc[qb][i >> 2][i & 3], sacc[qb][(i + 1) >> 2][(i + 1) & 3]);
        tmax = quad_max(fmaxf(tmax, sacc[qb][3][3]));
        return scaled ? tmax : tmax * c;
    };
    // O and l of query block qb rescaled to the offset m_new.
    auto rescale = [&](int qb, float m_new, float l_base) {
        const float alpha = m_run[qb] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
        l_run[qb] = l_base * alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r) oacc[db][qb][r] *= alpha;
        m_run[qb] = m_new;
    };
    // Mask, bound and tile maximum (log2 domain) of tile `it`; raises the running
    // offset when the maximum passes it by more than the slack. Returns the factor
    // the softmax applies to the scores: 1 when they were scaled here, else c.
    auto prep = [&](f32x4 (&sacc)[2][4], int it) -> float {
        const int kv0 = it * BKV;
        const bool scaled = needs_prep(it);
        if (scaled) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int kk = 16 * kb + 4 * g + r;
                        sacc[qb][kb][r] = kv0 + kk < key_lim(qb) ? sacc[qb][kb][r] * c : -INFINITY;
                    }
        }
        float tmax[2];
        bool raise[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            tmax[qb] = tile_max(sacc, qb, scaled);
            raise[qb] = tmax[qb] > m_run[qb] + kRescaleSlack;
        }
        if (__any(raise[0] || raise[1])) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) rescale(qb, raise[qb] ? tmax[qb] : m_run[qb], l_run[qb]);
        }
        return scaled ? 1.f : c;
    };
    // Probabilities of a prepared tile as MFMA Y operands, and their row sums:
    // pf[qb][kc] = keys 32 kc + 4 g + 0..3 and 32 kc + 16 + 4 g + 0..3 of query my_q[qb],
    // the order of the V^T fragments' k positions.
    auto softmax = [&](const f32x4 (&sacc)[2][4], float cs, vec8 (&pf)[2][2]) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const float m_use = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    pf[qb][kb >> 1][4 * (kb & 1) + r] = T(__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][kb][r], cs, -m_use)));
        }
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) l_run[qb] = Mfma<T>::rowsum(pf[qb][kc], l_run[qb]);
    };
    // The offset check of an unmasked tile whose maximum was not taken before its
    // softmax: its probabilities were computed with the running offset, adding to l_run
    // from l_before. When each query's probabilities sum to less than kLazyCheck no score
    // passed the offset by the slack, which is the common case after the first tiles,
    // and they stand. Else the tile maxima decide as prep would have: if one raises its
    // query's offset, O and l_before are rescaled and the probabilities recomputed, so
    // the outcome is exactly prep's, in the same order of operations.
    auto settle = [&](const f32x4 (&cur)[2][4], const float (&l_before)[2], vec8 (&pf)[2][2]) {
        const bool big0 = quad_sum(l_run[0] - l_before[0]) >= kLazyCheck;
        const bool big1 = quad_sum(l_run[1] - l_before[1]) >= kLazyCheck;
        if (!__any(big0 || big1)) return;
        float tmax[2];
        bool raise[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            tmax[qb] = tile_max(cur, qb, false);
            raise[qb] = tmax[qb] > m_run[qb] + kRescaleSlack;
        }
        if (!__any(raise[0] || raise[1])) return;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) rescale(qb, raise[qb] ? tmax[qb] : m_run[qb], l_before[qb]);
        softmax(cur, c, pf);
    };
    // O^T += V^T P^T. V^T fragment n = 8 kc + db (two transposing reads, issued two
    // fragments ahead of their use) feeds the MFMAs of both query blocks; an accumulator
    // is used again eight fragments (sixteen MFMAs) later.
    auto pv = [&](int slot, const vec8 (&pf)[2][2]) {
        u32x2 lo[16], hi[16];
        auto issue = [&](int n) {
            const int kc = n >> 3, db = n & 7;
            const uint32_t a = xor_imm(v_base, 32 * db);
            lo[n] = ds_read_tr(a, slot * KV_BYTES + 32 * kc * ROWB);
            hi[n] = ds_read_tr(a, slot * KV_BYTES + (32 * kc + 16) * ROWB);
        };
        issue(0);
        issue(1);
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            if (n + 2 < 16) issue(n + 2);
            // Reads issued after fragment n's two: those of fragments n+1 and n+2 (if any).
            lgkm_wait_for(lo[n], hi[n], 2 * ((n + 2 < 16 ? n + 2 : 15) - n));
            const u32x4 packed = {lo[n][0], lo[n][1], hi[n][0], hi[n][1]};
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                oacc[n & 7][qb] = Mfma<T>::run(__builtin_bit_cast(vec8, packed), pf[qb][n >> 3], oacc[n & 7][qb]);
        }
    };

    // Software pipeline over the key tiles i = 0 .. n-1 of [it0, it1): step i computes
    // S of tile i+1 on the matrix cores while the VALU turns the S of tile i into
    // probabilities, then accumulates P_i V_i. K_{i+1} and V_i are in LDS at the top of
    // step i; it loads K_{i+2} and V_{i+1} into the stages tiles i and i-1 left.
    // Masked tiles and the first one are prepared (bound, maximum, offset) before their
    // softmax; the others take the running offset as it stands and are settled after
    // it, which almost never has to take their maximum.
    const int n = it1 - it0;
    f32x4 sa[2][4], sb[2][4];
    vec8 pf[2][2];
    float cs_cur = c, cs_nxt = c;
    bool lazy_cur = false, lazy_nxt = false;  // the tile's maximum was not taken before its softmax
    // P = i % 2 as a compile-time constant: K_{i+1} sits in stage 1 - P, V_i in stage P.
    auto step = [&](int i, f32x4 (&cur)[2][4], f32x4 (&nxt)[2][4], auto has_next, auto parity) {
        constexpr int P = decltype(parity)::value;
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // this wave's loads of K_{i+1}, V_i landed
        lds_barrier();                                         // ... every wave's; tile i-1 fully consumed
        const float l_before[2] = {l_run[0], l_run[1]};
        if constexpr (decltype(has_next)::value) {
            if (i + 2 < n) issue_k(it0 + i + 2, P);
            issue_v(it0 + i + 1, 1 - P);
            // S of the next tile on the matrix cores, interleaved by hand with the
            // softmax of this one: each group issues K fragment n + 2, waits for
            // fragment n, issues its two MFMAs (one per query block) and turns one score
            // of this tile into a probability after each (plus a row-sum term when a
            // probability vector is complete); sched_barrier keeps the groups in order.
            qk_init(kstage(1 - P), (it0 + i + 1) * BKV, nxt);
            const float m_use[2] = {m_run[0] == -INFINITY ? 0.f : m_run[0], m_run[1] == -INFINITY ? 0.f : m_run[1]};
            u32x4 kf[16];
            kf[0] = kfrag(1 - P, 0);
            kf[1] = kfrag(1 - P, 1);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (k + 2 < 16) kf[k + 2] = kfrag(1 - P, k + 2);
                kwait(kf[k], k);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    nxt[qb][k & 3] = Mfma<T>::run(__builtin_bit_cast(vec8, kf[k]), qf[qb][k >> 2], nxt[qb][k & 3]);
                    // Score e = 2 k + qb of this tile: query block e / 16, key block e / 4 % 4, r = e % 4.
                    const int e = 2 * k + qb, eq = e >> 4, kb = (e >> 2) & 3, r = e & 3;
                    pf[eq][kb >> 1][4 * (kb & 1) + r] =
                        T(__builtin_amdgcn_exp2f(__builtin_fmaf(cur[eq][kb][r], cs_cur, -m_use[eq])));
                    // The two MFMAs of a fragment stay apart: an MFMA issued while the
                    // previous one still occupies the matrix unit holds up the wave's
                    // independent VALU work behind it.
                    if (qb == 0) __builtin_amdgcn_sched_barrier(0);
                }
                // Probability vector (k / 8, k / 4 % 2) complete after score 2 k + 1.
                if ((k & 3) == 3) l_run[k >> 3] = Mfma<T>::rowsum(pf[k >> 3][(k >> 2) & 1], l_run[k >> 3]);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (lazy_cur) settle(cur, l_before, pf);
            pv(P, pf);
            lazy_nxt = !needs_prep(it0 + i + 1);
            cs_nxt = lazy_nxt ? c : prep(nxt, it0 + i + 1);
        } else {
            softmax(cur, cs_cur, pf);
            if (lazy_cur) settle(cur, l_before, pf);
            pv(P, pf);
        }
    };
    typedef std::integral_constant<bool, true> more;
    typedef std::integral_constant<bool, false> last;
    typedef std::integral_constant<int, 0> even;
    typedef std::integral_constant<int, 1> odd;
    if (n > 0) {
        issue_k(it0, 0);
        issue_v(it0, 0);
        if (n > 1) issue_k(it0 + 1, 1);
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
        lds_barrier();
        if (!active) {
            // Loads and barriers only, step for step as below.
            for (int i = 0; i < n; ++i) {
                __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
                lds_barrier();
                if (i + 1 < n) {
                    if (i + 2 < n) issue_k(it0 + i + 2, i & 1);
                    issue_v(it0 + i + 1, 1 - (i & 1));
                }
            }
            return;
        }
        qk(0, it0 * BKV, sa);
        cs_cur = prep(sa, it0);
        int i = 0;  // always even at the top of the loop
        for (; i + 2 < n; i += 2) {
            step(i, sa, sb, more(), even());
            cs_cur = cs_nxt;
            lazy_cur = lazy_nxt;
            step(i + 1, sb, sa, more(), odd());
            cs_cur = cs_nxt;
            lazy_cur = lazy_nxt;
        }
        if (n - i == 2) {
            step(i, sa, sb, more(), even());
            cs_cur = cs_nxt;
            lazy_cur = lazy_nxt;
            step(i + 1, sb, sa, last(), odd());
        } else {
            step(i, sa, sb, last(), even());
        }
    }

    if (!active) return;  // n == 0
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) l_run[qb] = quad_sum(l_run[qb]);
    if (part >= 0) {
        // Key-range part of the split tail tile: unnormalised O and (m, l) for combine_kernel.
        const size_t slot = (size_t)h * p.tail_parts + part;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int ql = wave * 32 + 16 * qb + l16;
            float* po = p.part_o + (slot * p.part_rows + ql) * D;
#pragma unroll
            for (int db = 0; db < 8; ++db) *reinterpret_cast<f32x4*>(po + 16 * db + 4 * g) = oacc[db][qb];
            if (g == 0) {
                p.part_ml[(slot * p.part_rows + ql) * 2] = m_run[qb];
                p.part_ml[(slot * p.part_rows + ql) * 2 + 1] = l_run[qb];
            }
        }
        return;
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        if (my_q(qb) >= p.sq) continue;
        const float inv = 1.f / l_run[qb];
        T* orow = static_cast<T*>(p.o) + (size_t)h * p.o_hs + (size_t)my_q(qb) * p.o_rs;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            // Values 16 db + 4 g .. + 3: offset 16 (db % 2) + 4 g in the (db / 2)-th group of 32.
            union { u32x2 u; T e[4]; } pk;
#pragma unroll
            for (int e = 0; e < 4; ++e) pk.e[e] = T(oacc[db][qb][e] * inv);
            *reinterpret_cast<u32x2*>(orow + (size_t)(db >> 1) * p.o_ds + 16 * (db & 1) + 4 * g) = pk.u;
        }
    }
}

}  // namespace sdl

// Returns 1 without launching when the problem is not one this kernel takes
// (FP32, head_dim != 128, unaligned strides, >= 2 GiB K/V spans or per-query masks).
int sdpa16_d128(const SdpaArgs& a, hipStream_t s)
{
    if (a.dtype == DT_F32 || a.d != 128) return 1;
    if (a.mask && a.mask_rows != 1 && (size_t)a.sq * a.sk * 4 >= 2147483648ull) return 1;
    const long vec = 8;
    const uintptr_t bases = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                            reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.o);
    if (bases % 16 || a.q_hs % vec || a.q_rs % vec || a.k_hs % vec || a.k_rs % vec || a.v_hs % vec || a.v_rs % vec ||
        a.o_hs % vec || a.o_rs % vec || a.o_ds % vec)
        return a.o_ds != 0 && a.o_ds != 32 ? -1 : 1;
    const int kv_end = a.valid_keys > 0 ? a.valid_keys : a.sk;
    const int ntiles = (kv_end + sdl::BKV - 1) / sdl::BKV;
    if ((double)ntiles * sdl::BKV * (double)std::max(a.k_rs, a.v_rs) * 2 >= 2147483647.0) return 1;
    sdl::Params p{};
    p.q = a.q; p.k = a.k; p.v = a.v; p.o = a.o;
    p.heads = a.heads; p.group = a.heads / a.kv_heads; p.sq = a.sq; p.sk = a.sk; p.kv_end = kv_end;
    p.q_hs = a.q_hs; p.q_rs = a.q_rs; p.k_hs = a.k_hs; p.k_rs = a.k_rs;
    p.v_hs = a.v_hs; p.v_rs = a.v_rs; p.o_hs = a.o_hs; p.o_rs = a.o_rs;
    p.causal = a.causal ? 1 : 0; p.qk_off = a.sk - a.sq;
    p.o_ds = a.o_ds ? a.o_ds : 32;
    p.mask = a.mask;
    const bool dense = a.mask && a.mask_rows > 1;
    p.mask_hs = a.mask && a.mask_heads > 1 ? (long)a.sk * (dense ? a.sq : 1) : 0;
    const float scale = a.scale > 0.f ? a.scale : 1.f / sqrtf(128.f);
    p.scale_log2 = scale * sdl::kLog2e;
    // Workgroups of 8 waves (256 queries, one per CU) when the unmasked, non-causal
    // problem has whole 256-query tiles, else 4 waves (128 queries, two per CU). At 4096
    // queries x 4160 keys the 8-wave form took 273 against 280 us, bitwise the same; with a
    // partial last tile its key-range parts run on two of a CU's four SIMDs after the full
    // tiles and cost more than that (4160 queries: 295-299 against 285 us).
    const bool nw8 = !a.mask && !a.causal && a.sq % 256 == 0;
    const int bqw = nw8 ? 256 : 128;
    // A partial last query tile is split along the keys when a workspace is given:
    // kSdpaSlots parts over all heads, at most 16 and at least 1 per head.
    p.part_rows = bqw;
    p.full_qt = a.sq / bqw;
    const int tail_q = a.sq - p.full_qt * bqw;
    if (tail_q && p.full_qt && a.split_ws) {
        int parts = std::min(std::min(sdl::kMaxParts, ntiles), std::max(1, kSdpaSlots / a.heads));
        const size_t per_part = (size_t)a.heads * bqw * (sdl::D + 2) * sizeof(float);
        while (parts > 1 && (size_t)parts * per_part > a.split_ws_bytes) --parts;
        if (parts > 1) {
            p.tail_parts = parts;
            p.part_o = static_cast<float*>(a.split_ws);
            p.part_ml = p.part_o + (size_t)a.heads * parts * bqw * sdl::D;
        }
    }
    const int wgs = p.tail_parts ? (p.full_qt + p.tail_parts) * a.heads : ((a.sq + bqw - 1) / bqw) * a.heads;
    const dim3 grid(wgs), block(256);
    if (nw8) {
        const dim3 block8(512);
        if (a.dtype == DT_F16) hipLaunchKernelGGL((sdl::kernel<f16, sdl::MASK_NONE, 8>), grid, block8, 0, s, p);
        else hipLaunchKernelGGL((sdl::kernel<bf16, sdl::MASK_NONE, 8>), grid, block8, 0, s, p);
    } else if (a.dtype == DT_F16) {
        if (dense) hipLaunchKernelGGL((sdl::kernel<f16, sdl::MASK_DENSE, 4>), grid, block, 0, s, p);
        else if (a.mask) hipLaunchKernelGGL((sdl::kernel<f16, sdl::MASK_ROW, 4>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((sdl::kernel<f16, sdl::MASK_NONE, 4>), grid, block, 0, s, p);
    } else {
        if (dense) hipLaunchKernelGGL((sdl::kernel<bf16, sdl::MASK_DENSE, 4>), grid, block, 0, s, p);
        else if (a.mask) hipLaunchKernelGGL((sdl::kernel<bf16, sdl::MASK_ROW, 4>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((sdl::kernel<bf16, sdl::MASK_NONE, 4>), grid, block, 0, s, p);
    }
    if (p.tail_parts) {
        const long n = (long)a.heads * tail_q;  // one wave per (head, query), four per workgroup
        const dim3 cgrid((unsigned)((n + 3) / 4));
        if (a.dtype == DT_F16) hipLaunchKernelGGL((sdl::combine_kernel<f16>), cgrid, block, 0, s, p, tail_q);
        else hipLaunchKernelGGL((sdl::combine_kernel<bf16>), cgrid, block, 0, s, p, tail_q);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -int(e);
}

}  // namespace ehip
