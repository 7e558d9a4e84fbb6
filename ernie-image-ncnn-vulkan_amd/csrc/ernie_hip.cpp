// SPDX-License-Identifier: MIT
// extern "C" layer of ernie_hip (declarations and reference citations in
// include/ernie_hip.h). Owns the HIP stream, the resident block / head weights,
// the activation workspace and the optional per-kernel event timing.
#include "ernie_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <unordered_map>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "noalloc.hpp"

using namespace ehip;

namespace {

constexpr int kHeadDim = 128;
// Callers' finite-check slots and markers, then the ranges the C++ facade reserves.
constexpr int kFiniteSlots = ERNIE_FINITE_SLOTS + ERNIE_FINITE_SLOTS_RESERVED;
constexpr int kMarkers = ERNIE_MARKERS + ERNIE_MARKERS_RESERVED;

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct BlockWeights {
    bool loaded = false;
    int dim = 0, ffn = 0, dtype = 0;
    DeviceBuffer norm1, norm_q, norm_k, norm2;  // FP32
    DeviceBuffer wqkv;                          // [3*dim][dim]
    DeviceBuffer wo;                            // [dim][dim]
    DeviceBuffer w_ug;                          // [2*ffn][dim], 32-row up/gate interleave
    DeviceBuffer w_down;                        // [dim][ffn]
    // 16-bit projections whose output count is a multiple of 256 are stored K-tiled,
    // [K/32][N][32] (GemmArgs::w_k32); flags for wqkv, wo, w_ug, w_down.
    bool k32[4] = {false, false, false, false};
    // K-tiled wqkv whose Q and K rows are stored permuted within each head
    // (qk_stored_column), so the QKV GEMM finishes Q/K norm and rotary in its epilogue.
    bool qk_fused = false;
};

// One Mistral text decoder block (tests/fixtures/text-s64.ncnn.param), head_dim 128.
struct TextBlockWeights {
    bool loaded = false;
    int hidden = 0, heads = 0, kv_heads = 0, ffn = 0, dtype = 0;
    DeviceBuffer norm1, norm2;  // FP32 [hidden]
    DeviceBuffer wqkv;          // [(heads + 2 kv_heads) * 128][hidden]: q, k, v rows (gemm_0/1/2)
    DeviceBuffer wo;            // [hidden][heads * 128]
    DeviceBuffer w_ug;          // [2 ffn][hidden]: up / gate rows interleaved in 32-row groups
    DeviceBuffer w_down;        // [hidden][ffn]
    bool k32[4] = {false, false, false, false};  // K-tiled wqkv, wo, w_ug, w_down (16-bit)
};

// The two DiT heads (heads/input and heads/output head.ncnn.param); each part is loaded
// and released on its own, sharing dim, latent_ch and dtype.
struct HeadWeights {
    int parts = 0;  // ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT
    int dim = 0, latent_ch = 0, text_dim = 0, dtype = 0;
    DeviceBuffer x_w, x_b, text_w, t1_w, t1_b, t2_w, t2_b, mod_w, mod_b;  // input head
    DeviceBuffer out_mod_w, out_mod_b, proj_w, proj_b;                    // output head
};

struct Launch {
    int cls;
    hipEvent_t start, stop;
    double flop, bytes;
};

}  // namespace

struct ernie_hip_ctx {
    int device = 0;
    // This device's copy of the fixed scratch (noalloc.hip), looked up at creation;
    // nullptr when the lookup failed (the no-allocation entry point then refuses).
    void* scratch = nullptr;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string error;
    int query_rows = 128;
    // ERNIE_QK_ROUND_STORAGE: 16-bit blocks round the Q/K projections before their RMSNorm.
    bool qk_storage_rounding = false;
    std::vector<BlockWeights> blocks;
    std::vector<TextBlockWeights> text_blocks;
    HeadWeights heads;
    // Activation workspace, grown on demand.
    DeviceBuffer ws;
    DeviceBuffer staging;  // FP32 upload staging
    DeviceBuffer head_ws;  // head intermediates
    DeviceBuffer dit_act;  // run_dit activations: x [S][dim], c, mods
    DeviceBuffer split_ws;   // GEMM tail-row split-K partial sums
    DeviceBuffer rope_pack;  // [S][64] (cos, sin) pairs of the rotary angles, per call
    DeviceBuffer text_ws;    // text block activations
    DeviceBuffer ones;       // FP32 ones: unit gates of the text block's residual epilogues
    // Event timing.
    bool profiling = false;
    unsigned profile_mask = ~0u;  // classes that record events while profiling
    int profile_stride = 1;       // record every profile_stride-th launch of a class
    long class_seen[32] = {};     // launches of each class since the last reset
    std::vector<hipEvent_t> event_pool;
    // Freed device blocks kept for reuse, by size: hipFree synchronises the whole device,
    // which drained the queue several times per denoise step. A reused block's earlier
    // work was enqueued on this context's stream before any new work on it.
    std::multimap<size_t, void*> free_cache;
    std::unordered_map<void*, size_t> live;
    size_t cached_bytes = 0;
    std::mutex alloc_mu;
    // Finiteness flags: kFiniteSlots for the asynchronous check (the callers' slots, then
    // the facade's) plus one for ernie_hip_finite, on the device; their pinned host copies
    // and completion events.
    int* finite_flag = nullptr;
    int* finite_host = nullptr;
    hipEvent_t finite_event[kFiniteSlots] = {};
    bool finite_pending[kFiniteSlots] = {};
    // Stream markers (ernie_hip_marker_*: the callers', then the facade's) and the
    // per-block events of a timed block sequence: created once, reused by every call.
    hipEvent_t marker[kMarkers] = {};
    bool marker_recorded[kMarkers] = {};
    std::vector<hipEvent_t> seq_events;
    // Pinned staging blocks of ernie_hip_upload_async, each with the event of its last
    // copy: a block is reused once that copy has finished.
    struct Staging { void* host; size_t bytes; hipEvent_t done; };
    std::vector<Staging> upload_staging;
    size_t event_next = 0;
    std::vector<Launch> pending;
    long launches[ERNIE_PROFILE_CLASSES] = {};
    double ms[ERNIE_PROFILE_CLASSES] = {};
    double flop[ERNIE_PROFILE_CLASSES] = {};
    double bytes[ERNIE_PROFILE_CLASSES] = {};
};

namespace {

int fail(ernie_hip_ctx* ctx, int code, const std::string& msg)
{
    if (ctx) ctx->error = msg;
    return code;
}

int hip_status(ernie_hip_ctx* ctx, hipError_t e, const char* what)
{
    if (e == hipSuccess) return ERNIE_OK;
    const int code = e == hipErrorOutOfMemory ? ERNIE_ALLOCATION_FAILED : ERNIE_ERROR;
    return fail(ctx, code, std::string(what) + ": " + hipGetErrorString(e));
}

// Kernel launcher statuses: -1 = rejected shape, -k = hipError k.
int kernel_status(ernie_hip_ctx* ctx, int rc, const char* what)
{
    if (rc == 0) return ERNIE_OK;
    if (rc == -1) return fail(ctx, ERNIE_ERROR, std::string(what) + ": invalid arguments");
    return hip_status(ctx, hipError_t(-rc), what);
}

bool valid_dtype(int dt) { return dt == ERNIE_DTYPE_FP32 || dt == ERNIE_DTYPE_FP16 || dt == ERNIE_DTYPE_BF16; }
size_t esize(int dt) { return dt == ERNIE_DTYPE_FP32 ? 4 : 2; }

// Returns the freed blocks kept for reuse to the driver. hipFree synchronises the device,
// so this runs only when an allocation failed or the caller asks (ernie_hip_trim).
size_t release_cache(ernie_hip_ctx* ctx)
{
    std::lock_guard<std::mutex> lock(ctx->alloc_mu);
    const size_t released = ctx->cached_bytes;
    for (auto& kv : ctx->free_cache) (void)hipFree(kv.second);
    ctx->free_cache.clear();
    ctx->cached_bytes = 0;
    return released;
}

// hipMalloc; when the device is out of memory while freed blocks of other sizes are
// cached, they are released (after the stream's work that may still use them) and the
// allocation is tried once more.
hipError_t device_malloc(ernie_hip_ctx* ctx, void** out, size_t bytes)
{
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipErrorOutOfMemory) return e;
    (void)hipGetLastError();
    size_t cached = 0;
    {
        std::lock_guard<std::mutex> lock(ctx->alloc_mu);
        cached = ctx->cached_bytes;
    }
    if (!cached) return e;
    (void)hipStreamSynchronize(ctx->stream);
    release_cache(ctx);
    e = hipMalloc(out, bytes);
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

int dev_alloc(ernie_hip_ctx* ctx, DeviceBuffer& b, size_t bytes, const char* what)
{
    if (b.ptr && b.bytes >= bytes) return ERNIE_OK;
    if (b.ptr) {
        // Work queued on the stream may still read the old buffer.
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
    }
    if (!bytes) return ERNIE_OK;
    const hipError_t e = device_malloc(ctx, &b.ptr, bytes);
    if (e != hipSuccess) {
        b.ptr = nullptr;
        return hip_status(ctx, e, what);
    }
    b.bytes = bytes;
    return ERNIE_OK;
}

void dev_free(DeviceBuffer& b)
{
    if (b.ptr) (void)hipFree(b.ptr);
    b = DeviceBuffer{};
}

void free_block(BlockWeights& w)
{
    for (DeviceBuffer* b : {&w.norm1, &w.norm_q, &w.norm_k, &w.norm2, &w.wqkv, &w.wo, &w.w_ug, &w.w_down}) dev_free(*b);
    w = BlockWeights{};
}

void free_text_block(TextBlockWeights& w)
{
    for (DeviceBuffer* b : {&w.norm1, &w.norm2, &w.wqkv, &w.wo, &w.w_ug, &w.w_down}) dev_free(*b);
    w = TextBlockWeights{};
}

// Releases the head parts in `parts`; the dimensions go with the last part.
void free_heads(HeadWeights& h, int parts = ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT)
{
    if (parts & ERNIE_HEAD_INPUT)
        for (DeviceBuffer* b : {&h.x_w, &h.x_b, &h.text_w, &h.t1_w, &h.t1_b, &h.t2_w, &h.t2_b, &h.mod_w, &h.mod_b})
            dev_free(*b);
    if (parts & ERNIE_HEAD_OUTPUT)
        for (DeviceBuffer* b : {&h.out_mod_w, &h.out_mod_b, &h.proj_w, &h.proj_b}) dev_free(*b);
    h.parts &= ~parts;
    if (!h.parts) h = HeadWeights{};
}

// ---- event timing ------------------------------------------------------------------
hipEvent_t next_event(ernie_hip_ctx* ctx)
{
    if (ctx->event_next == ctx->event_pool.size()) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        ctx->event_pool.push_back(e);
    }
    return ctx->event_pool[ctx->event_next++];
}

struct Timed {
    ernie_hip_ctx* ctx;
    int cls;
    double flop, bytes;
    hipEvent_t start = nullptr;
    Timed(ernie_hip_ctx* c, int k, double f, double b) : ctx(c), cls(k), flop(f), bytes(b)
    {
        if (ctx->profiling && (ctx->profile_mask >> cls & 1u) && ctx->class_seen[cls]++ % ctx->profile_stride == 0) {
            start = next_event(ctx);
            if (start) (void)hipEventRecord(start, ctx->stream);
        }
    }
    ~Timed()
    {
        if (!start) return;
        hipEvent_t stop = next_event(ctx);
        if (!stop) return;
        (void)hipEventRecord(stop, ctx->stream);
        ctx->pending.push_back(Launch{cls, start, stop, flop, bytes});
    }
};

int collect(ernie_hip_ctx* ctx)
{
    if (ctx->pending.empty()) {
        ctx->event_next = 0;
        return ERNIE_OK;
    }
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_status(ctx, e, "profile synchronize");
    for (const Launch& l : ctx->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, l.start, l.stop) == hipSuccess) {
            ctx->launches[l.cls] += 1;
            ctx->ms[l.cls] += ms;
            ctx->flop[l.cls] += l.flop;
            ctx->bytes[l.cls] += l.bytes;
        }
    }
    ctx->pending.clear();
    ctx->event_next = 0;
    return ERNIE_OK;
}

enum { P_QKV = 0, P_SDPA = 1, P_OUT = 2, P_UG = 3, P_DOWN = 4, P_NORM = 5, P_ROPE = 6, P_HEADS = 7 };

double gemm_bytes(double M, double N, double K, double e, double eo) { return (M * K + N * K) * e + M * N * eo; }

// ---- uploads ------------------------------------------------------------------------
// Host tensor (FP32, FP16 or BF16) -> device dtype at `dst` (+ element offset) through the
// staging buffer; the conversion runs on the device. An FP32 -> FP32 upload copies directly.
int upload_tensor(ernie_hip_ctx* ctx, void* dst, size_t dst_offset, int dtype, const void* src, int src_dtype,
                  size_t count, const char* what)
{
    if (!valid_dtype(src_dtype)) return fail(ctx, ERNIE_ERROR, "invalid source dtype");
    char* base = static_cast<char*>(dst) + dst_offset * esize(dtype);
    if (src_dtype == dtype)
        return hip_status(ctx, hipMemcpyAsync(base, src, count * esize(dtype), hipMemcpyHostToDevice, ctx->stream), what);
    int rc = dev_alloc(ctx, ctx->staging, count * esize(src_dtype), "staging buffer");
    if (rc) return rc;
    rc = hip_status(ctx, hipMemcpyAsync(ctx->staging.ptr, src, count * esize(src_dtype), hipMemcpyHostToDevice,
                                        ctx->stream), what);
    if (rc) return rc;
    rc = kernel_status(ctx, convert(ctx->staging.ptr, src_dtype, base, dtype, count, ctx->stream), what);
    if (rc) return rc;
    // The staging buffer is reused by the next upload: finish this one first.
    return hip_status(ctx, hipStreamSynchronize(ctx->stream), what);
}

int alloc_block(ernie_hip_ctx* ctx, BlockWeights& w, int dim, int ffn, int dtype)
{
    const size_t e = esize(dtype);
    int rc = 0;
    rc = rc ? rc : dev_alloc(ctx, w.norm1, (size_t)dim * 4, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.norm2, (size_t)dim * 4, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.norm_q, kHeadDim * 4, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.norm_k, kHeadDim * 4, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.wqkv, 3 * (size_t)dim * dim * e, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.wo, (size_t)dim * dim * e, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.w_ug, 2 * (size_t)ffn * dim * e, "block weights");
    rc = rc ? rc : dev_alloc(ctx, w.w_down, (size_t)dim * ffn * e, "block weights");
    if (rc) {
        free_block(w);
        return rc;
    }
    w.dim = dim;
    w.ffn = ffn;
    w.dtype = dtype;
    return ERNIE_OK;
}

// Rewrites the 16-bit projection matrices of a freshly written block K-tiled,
// through the staging buffer, and records which ones were.
// head_rows: leading rows stored permuted within 128-row heads (tile_k32).
struct TiledMat { DeviceBuffer* b; int rows, cols, head_rows; };

int tile_matrices(ernie_hip_ctx* ctx, int dtype, const TiledMat (&mats)[4], bool (&k32)[4])
{
    if (dtype == ERNIE_DTYPE_FP32) return ERNIE_OK;
    size_t most = 0;
    for (const TiledMat& m : mats) most = std::max(most, (size_t)m.rows * m.cols * 2);
    int rc = dev_alloc(ctx, ctx->staging, most, "staging buffer");
    for (int i = 0; i < 4 && !rc; ++i) {
        const TiledMat& m = mats[i];
        const size_t bytes = (size_t)m.rows * m.cols * 2;
        if (m.rows % 256 || m.cols % 32 || bytes >= (1ull << 31)) continue;
        rc = hip_status(ctx, hipMemcpyAsync(ctx->staging.ptr, m.b->ptr, bytes, hipMemcpyDeviceToDevice, ctx->stream),
                        "tile weights");
        if (!rc)
            rc = kernel_status(ctx, tile_k32(ctx->staging.ptr, m.b->ptr, m.rows, m.cols, ctx->stream, m.head_rows),
                               "tile weights");
        if (!rc) k32[i] = true;
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "tile weights");
    return rc;
}

int tile_block_weights(ernie_hip_ctx* ctx, BlockWeights& w)
{
    const int D = w.dim, F = w.ffn;
    const TiledMat mats[4] = {{&w.wqkv, 3 * D, D, 2 * D}, {&w.wo, D, D, 0}, {&w.w_ug, 2 * F, D, 0}, {&w.w_down, D, F, 0}};
    const int rc = tile_matrices(ctx, w.dtype, mats, w.k32);
    w.qk_fused = !rc && w.k32[0];
    return rc;
}

int tile_text_weights(ernie_hip_ctx* ctx, TextBlockWeights& w)
{
    const int H = w.hidden, F = w.ffn, QD = w.heads * 128, QKV = (w.heads + 2 * w.kv_heads) * 128;
    const TiledMat mats[4] = {{&w.wqkv, QKV, H, 0}, {&w.wo, H, QD, 0}, {&w.w_ug, 2 * F, H, 0}, {&w.w_down, H, F, 0}};
    return tile_matrices(ctx, w.dtype, mats, w.k32);
}

int check_block_dims(ernie_hip_ctx* ctx, int dim, int ffn, int dtype)
{
    if (!valid_dtype(dtype)) return fail(ctx, ERNIE_ERROR, "invalid dtype");
    if (dim < 128 || dim % 128 || dim > 4096) return fail(ctx, ERNIE_ERROR, "dim must be a multiple of 128 in [128,4096]");
    if (ffn < 32 || ffn % 32) return fail(ctx, ERNIE_ERROR, "ffn must be a positive multiple of 32");
    return ERNIE_OK;
}

BlockWeights* block_slot(ernie_hip_ctx* ctx, int index)
{
    if (index < 0 || index > 4096) return nullptr;
    if ((size_t)index >= ctx->blocks.size()) ctx->blocks.resize(index + 1);
    return &ctx->blocks[index];
}

// ---- workspace -------------------------------------------------------------------------
// The GEMM operands h, attn and p are K-tiled, [cols/32][rows][32] with rows = S
// rounded up to 256, at 16-bit storage (rows past S are read by a tail tile but never
// stored); row-major [S][cols] at FP32.
struct BlockWs {
    void* h;      // dim columns, dtype
    void* qkv;    // [S][3dim] dtype
    void* attn;   // dim columns, dtype
    float* x1;    // [S][dim] f32
    void* p;      // ffn columns, dtype
    int rows;     // K-tiled row count (0: row-major)
};

int block_workspace(ernie_hip_ctx* ctx, int S, int dim, int ffn, int dtype, BlockWs& ws)
{
    const size_t e = esize(dtype);
    ws.rows = dtype == ERNIE_DTYPE_FP32 ? 0 : (S + 255) / 256 * 256;
    const size_t R = ws.rows ? ws.rows : S;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t h = up(R * dim * e), qkv = up(3 * (size_t)S * dim * e), x1 = up((size_t)S * dim * 4),
                 p = up(R * ffn * e);
    const int rc = dev_alloc(ctx, ctx->ws, h + qkv + h + x1 + p, "block workspace");
    if (rc) return rc;
    char* b = static_cast<char*>(ctx->ws.ptr);
    ws.h = b;
    ws.qkv = b + h;
    ws.attn = b + h + qkv;
    ws.x1 = reinterpret_cast<float*>(b + h + qkv + h);
    ws.p = b + h + qkv + h + x1;
    return ERNIE_OK;
}

// Split-K scratch of the block GEMMs: the tail row of tiles (S % 256 rows) or, for a
// GEMM with too few tiles for the CUs, every tile: at most 256 items of up to 256 x 256
// FP32 partials.
constexpr int kSplitItems = 256;

// The same buffer also holds the attention key-range parts of a partial last query
// tile: up to 16 parts per head of 128 queries x (128 values + m, l) FP32.
size_t split_bytes(int S, int heads)
{
    const size_t gemm = 2 * (size_t)kSplitItems * 256 * 256 * sizeof(float);
    const size_t attn = S % 128 ? (size_t)heads * 16 * 128 * (128 + 2) * sizeof(float) : 0;
    return std::max(gemm, attn);
}

int split_workspace(ernie_hip_ctx* ctx, int S, int heads, void** ws, size_t* bytes)
{
    const size_t need = split_bytes(S, heads);
    if (!need) return ERNIE_OK;
    const int rc = dev_alloc(ctx, ctx->split_ws, need, "split workspace");
    if (rc) return rc;
    *ws = ctx->split_ws.ptr;
    *bytes = ctx->split_ws.bytes;
    return ERNIE_OK;
}

// The rotary angles (cos, sin) packed once per call (rope_pack) for the blocks in
// `blocks` whose Q/K weights have the fused layout: into the context's buffer, or nullptr
// when no block has it.
int pack_rope(ernie_hip_ctx* ctx, const int* blocks, int count, const float* cos_t, const float* sin_t, int S,
              const float** cs)
{
    *cs = nullptr;
    bool fused = false;
    for (int i = 0; i < count; ++i) fused |= ctx->blocks[blocks[i]].qk_fused;
    if (!fused) return ERNIE_OK;
    int rc = dev_alloc(ctx, ctx->rope_pack, (size_t)S * 128 * sizeof(float), "rotary angle pairs");
    if (rc) return rc;
    rc = kernel_status(ctx, rope_pack(cos_t, sin_t, S, static_cast<float*>(ctx->rope_pack.ptr), ctx->stream),
                       "rotary angle pairs");
    if (!rc) *cs = static_cast<const float*>(ctx->rope_pack.ptr);
    return rc;
}

int block_forward(ernie_hip_ctx* ctx, const BlockWeights& w, const float* x, float* out, const float* mods,
                  const float* cos_t, const float* sin_t, const float* cs_t, const float* mask, int valid_keys, int S)
{
    const int D = w.dim, F = w.ffn, dt = w.dtype, H = D / kHeadDim;
    const double e = (double)esize(dt), dS = S;
    BlockWs ws{};
    int rc = block_workspace(ctx, S, D, F, dt, ws);
    if (rc) return rc;
    hipStream_t s = ctx->stream;
    const float *shift_sa = mods, *scale_sa = mods + D, *gate_sa = mods + 2 * D;
    const float *shift_mlp = mods + 3 * D, *scale_mlp = mods + 4 * D, *gate_mlp = mods + 5 * D;
    // rmsn_8 + add_0/mul_1/add_2
    {
        Timed t(ctx, P_NORM, 0, dS * D * (4 + e));
        rc = kernel_status(ctx, rmsnorm_modulate(x, ERNIE_DTYPE_FP32, static_cast<const float*>(w.norm1.ptr), shift_sa, scale_sa,
                                                 S, D, 1e-6f, ws.h, dt, s, ws.rows), "rmsnorm_modulate");
        if (rc) return rc;
    }
    // gemm_0/1/2 as one [3D][D] projection; with permuted Q/K weight rows, rmsn_9 /
    // rmsn_10 and the rotary BinaryOps run in its epilogue.
    {
        GemmArgs g;
        g.A = ws.h; g.lda = D; g.W = w.wqkv.ptr; g.ldw = D; g.M = S; g.N = 3 * D; g.K = D; g.dtype = dt;
        g.w_k32 = w.k32[0];
        g.a_k32_rows = ws.rows;
        g.epilogue = EPI_STORE; g.C = ws.qkv; g.ldc = 3 * D; g.c_dtype = dt;
        if (w.qk_fused && !ctx->qk_storage_rounding) {
            g.epilogue = EPI_QKROPE;
            g.cs_t = cs_t;
            g.qk_cols = 2 * D; g.k_col = D;
            g.gq = static_cast<const float*>(w.norm_q.ptr); g.gk = static_cast<const float*>(w.norm_k.ptr);
            g.qk_eps = 1e-6f;
        }
        rc = split_workspace(ctx, S, H, &g.split_ws, &g.split_ws_bytes);
        if (rc) return rc;
        Timed t(ctx, P_QKV, 2.0 * dS * 3 * D * D, gemm_bytes(dS, 3.0 * D, D, e, e));
        rc = kernel_status(ctx, gemm(g, s), "gemm qkv");
        if (rc) return rc;
    }
    // rmsn_9 / rmsn_10 + rotary on the Q and K columns the GEMM rounded to the storage
    // dtype: in place and in natural order, or from the permuted order of fused-layout weights.
    if (w.qk_fused && ctx->qk_storage_rounding) {
        Timed t(ctx, P_ROPE, 0, dS * 2 * D * e * 2 + dS * 128 * 8);
        rc = kernel_status(ctx, qk_norm_rope_permuted(ws.qkv, dt, 0, S, H, H, 3L * D, D,
                                                      static_cast<const float*>(w.norm_q.ptr),
                                                      static_cast<const float*>(w.norm_k.ptr), cs_t, 1e-6f, s),
                           "qk_norm_rope");
        if (rc) return rc;
    } else if (!w.qk_fused) {
        Timed t(ctx, P_ROPE, 0, dS * 2 * D * e * 2 + dS * 128 * 8);
        rc = kernel_status(ctx, qk_norm_rope_qk(ws.qkv, dt, S, H, H, 3L * D, D, static_cast<const float*>(w.norm_q.ptr),
                                                static_cast<const float*>(w.norm_k.ptr), cos_t, sin_t, s),
                           "qk_norm_rope");
        if (rc) return rc;
    }
    // sdpa_22
    {
        SdpaArgs a;
        const size_t eb = esize(dt);
        a.q = ws.qkv; a.k = static_cast<char*>(ws.qkv) + (size_t)D * eb; a.v = static_cast<char*>(ws.qkv) + 2 * (size_t)D * eb;
        a.o = ws.attn; a.dtype = dt; a.heads = H; a.kv_heads = H; a.sq = S; a.sk = S; a.d = kHeadDim;
        a.q_hs = a.k_hs = a.v_hs = kHeadDim; a.q_rs = a.k_rs = a.v_rs = 3L * D;
        if (ws.rows) {
            a.o_rs = 32; a.o_ds = 32L * ws.rows; a.o_hs = 4 * a.o_ds;  // K-tiled for the out projection
        } else {
            a.o_hs = kHeadDim; a.o_rs = D;
        }
        a.mask = mask; a.mask_heads = 1; a.mask_rows = 1; a.valid_keys = valid_keys;
        rc = split_workspace(ctx, S, H, &a.split_ws, &a.split_ws_bytes);
        if (rc) return rc;
        Timed t(ctx, P_SDPA, 4.0 * dS * dS * kHeadDim * H, 4.0 * dS * D * e);
        rc = kernel_status(ctx, sdpa(a, s), "sdpa");
        if (rc) return rc;
    }
    // gemm_3 + mul_15 + ErnieResidualAdd add_16 (FP32)
    {
        GemmArgs g;
        g.A = ws.attn; g.lda = D; g.W = w.wo.ptr; g.ldw = D; g.M = S; g.N = D; g.K = D; g.dtype = dt;
        g.w_k32 = w.k32[1];
        g.a_k32_rows = ws.rows;
        g.epilogue = EPI_GATE_RESID; g.C = ws.x1; g.ldc = D; g.c_dtype = ERNIE_DTYPE_FP32; g.resid = x; g.ld_resid = D;
        g.gate = gate_sa;
        rc = split_workspace(ctx, S, H, &g.split_ws, &g.split_ws_bytes);
        if (rc) return rc;
        Timed t(ctx, P_OUT, 2.0 * dS * D * D, gemm_bytes(dS, D, D, e, 8));
        rc = kernel_status(ctx, gemm(g, s), "gemm out");
        if (rc) return rc;
    }
    // rmsn_11 + add_17/mul_18/add_19
    {
        Timed t(ctx, P_NORM, 0, dS * D * (4 + e));
        rc = kernel_status(ctx, rmsnorm_modulate(ws.x1, ERNIE_DTYPE_FP32, static_cast<const float*>(w.norm2.ptr), shift_mlp,
                                                 scale_mlp, S, D, 1e-6f, ws.h, dt, s, ws.rows), "rmsnorm_modulate 2");
        if (rc) return rc;
    }
    // gemm_4 (up) + gemm_5 (gate) + ErnieGELU + mul_20 in one GEMM epilogue
    {
        GemmArgs g;
        g.A = ws.h; g.lda = D; g.W = w.w_ug.ptr; g.ldw = D; g.M = S; g.N = 2 * F; g.K = D; g.dtype = dt;
        g.w_k32 = w.k32[2];
        g.a_k32_rows = ws.rows;
        g.c_k32_rows = ws.rows;
        g.epilogue = EPI_GEGLU; g.C = ws.p; g.ldc = F; g.c_dtype = dt;
        rc = split_workspace(ctx, S, H, &g.split_ws, &g.split_ws_bytes);
        if (rc) return rc;
        Timed t(ctx, P_UG, 2.0 * dS * 2 * F * D, gemm_bytes(dS, 2.0 * F, D, e, 0) + dS * F * e);
        rc = kernel_status(ctx, gemm(g, s), "gemm up/gate");
        if (rc) return rc;
    }
    // gemm_6 + mul_21 + ErnieResidualAdd add_22
    {
        GemmArgs g;
        g.A = ws.p; g.lda = F; g.W = w.w_down.ptr; g.ldw = F; g.M = S; g.N = D; g.K = F; g.dtype = dt;
        g.w_k32 = w.k32[3];
        g.a_k32_rows = ws.rows;
        g.epilogue = EPI_GATE_RESID; g.C = out; g.ldc = D; g.c_dtype = ERNIE_DTYPE_FP32; g.resid = ws.x1; g.ld_resid = D;
        g.gate = gate_mlp;
        rc = split_workspace(ctx, S, H, &g.split_ws, &g.split_ws_bytes);
        if (rc) return rc;
        Timed t(ctx, P_DOWN, 2.0 * dS * D * F, gemm_bytes(dS, D, F, e, 8));
        rc = kernel_status(ctx, gemm(g, s), "gemm down");
        if (rc) return rc;
    }
    return ERNIE_OK;
}

// ---- Mistral text block (tests/fixtures/text-s64.ncnn.param) ------------------------------
int ones_buffer(ernie_hip_ctx* ctx, int n, const float** out)
{
    const size_t bytes = (size_t)n * 4;
    if (ctx->ones.bytes < bytes) {
        int rc = dev_alloc(ctx, ctx->ones, bytes, "ones");
        if (rc) return rc;
        rc = hip_status(ctx, hipMemsetD32Async(static_cast<hipDeviceptr_t>(ctx->ones.ptr), 0x3f800000u, n, ctx->stream),
                        "ones");
        if (rc) return rc;
    }
    *out = static_cast<const float*>(ctx->ones.ptr);
    return ERNIE_OK;
}

// Device buffers one text block forward works in: activations, the unit gate of the
// residual epilogues, and the GEMM split-K partials.
struct TextWs {
    void *h, *qkv, *attn, *p;
    float* x1;
    const float* ones;
    void* split_ws;
    size_t split_ws_bytes;
};

// Activation bytes of one text block forward: h, qkv, attention output, x1 and p, each
// 256-byte aligned; `at` (nullable) receives their offsets in that order.
size_t text_activation_bytes(const TextBlockWeights& w, int S, size_t* at = nullptr)
{
    const size_t e = esize(w.dtype), QD = (size_t)w.heads * 128, QKV = QD + 2 * (size_t)w.kv_heads * 128;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t sizes[5] = {up((size_t)S * w.hidden * e), up((size_t)S * QKV * e), up((size_t)S * QD * e),
                             up((size_t)S * w.hidden * 4), up((size_t)S * w.ffn * e)};
    size_t total = 0;
    for (int i = 0; i < 5; ++i) {
        if (at) at[i] = total;
        total += sizes[i];
    }
    return total;
}

TextWs text_ws_at(const TextBlockWeights& w, int S, void* activations)
{
    size_t at[5];
    text_activation_bytes(w, S, at);
    char* b = static_cast<char*>(activations);
    TextWs ws{};
    ws.h = b + at[0];
    ws.qkv = b + at[1];
    ws.attn = b + at[2];
    ws.x1 = reinterpret_cast<float*>(b + at[3]);
    ws.p = b + at[4];
    return ws;
}

int text_block_run(ernie_hip_ctx* ctx, const TextBlockWeights& w, const float* x, float* out, const float* cos_t,
                   const float* sin_t, const float* mask, int causal, int S, const TextWs& ws);

// rmsn_8 -> gemm_0/1/2 -> rotary (lines 18-44) -> sdpa_20 (GQA, additive mask in3) ->
// gemm_3 + add_12 -> rmsn_9 -> gemm_4 (gate) silu_7, gemm_5 (up), mul_13 -> gemm_6 + add_14.
// The residual adds are the GEMM epilogues with a unit gate; the gated MLP is one GEMM
// over the interleaved up/gate rows with a SiLU epilogue. out may alias x. The
// workspace comes from the context (grown on demand).
int text_block_forward(ernie_hip_ctx* ctx, const TextBlockWeights& w, const float* x, float* out, const float* cos_t,
                       const float* sin_t, const float* mask, int causal, int S)
{
    int rc = dev_alloc(ctx, ctx->text_ws, text_activation_bytes(w, S), "text workspace");
    if (rc) return rc;
    TextWs ws = text_ws_at(w, S, ctx->text_ws.ptr);
    rc = ones_buffer(ctx, w.hidden, &ws.ones);
    if (rc) return rc;
    rc = split_workspace(ctx, S, w.heads, &ws.split_ws, &ws.split_ws_bytes);
    if (rc) return rc;
    return text_block_run(ctx, w, x, out, cos_t, sin_t, mask, causal, S, ws);
}

int text_block_run(ernie_hip_ctx* ctx, const TextBlockWeights& w, const float* x, float* out, const float* cos_t,
                   const float* sin_t, const float* mask, int causal, int S, const TextWs& ws)
{
    const int H = w.hidden, F = w.ffn, nq = w.heads, nk = w.kv_heads, dt = w.dtype;
    const int QD = nq * 128, KVD = nk * 128, QKV = QD + 2 * KVD;
    const size_t e = esize(dt);
    const double dS = S;
    void *h = ws.h, *qkv = ws.qkv, *attn = ws.attn, *p = ws.p;
    float* x1 = ws.x1;
    const float* ones = ws.ones;
    void* split_ws = ws.split_ws;
    const size_t split_ws_bytes = ws.split_ws_bytes;
    hipStream_t s = ctx->stream;
    int rc = 0;
    {
        Timed t(ctx, P_NORM, 0, dS * H * (4 + e));
        rc = kernel_status(ctx, rmsnorm_modulate(x, ERNIE_DTYPE_FP32, static_cast<const float*>(w.norm1.ptr), nullptr,
                                                 nullptr, S, H, 1e-5f, h, dt, s), "text rmsnorm");
        if (rc) return rc;
    }
    {
        GemmArgs g;
        g.A = h; g.lda = H; g.W = w.wqkv.ptr; g.ldw = H; g.M = S; g.N = QKV; g.K = H; g.dtype = dt;
        g.w_k32 = w.k32[0];
        g.epilogue = EPI_STORE; g.C = qkv; g.ldc = QKV; g.c_dtype = dt;
        g.split_ws = split_ws; g.split_ws_bytes = split_ws_bytes;
        Timed t(ctx, P_QKV, 2.0 * dS * QKV * H, gemm_bytes(dS, QKV, H, e, e));
        rc = kernel_status(ctx, gemm(g, s), "text gemm qkv");
        if (rc) return rc;
    }
    {
        Timed t(ctx, P_ROPE, 0, dS * (QD + KVD) * e * 2 + dS * 128 * 8);
        rc = kernel_status(ctx, qk_norm_rope_qk(qkv, dt, S, nq, nk, QKV, QD, nullptr, nullptr, cos_t, sin_t, s),
                           "text rotary");
        if (rc) return rc;
    }
    {
        SdpaArgs a;
        a.q = qkv; a.k = static_cast<char*>(qkv) + (size_t)QD * e; a.v = static_cast<char*>(qkv) + (size_t)(QD + KVD) * e;
        a.o = attn; a.dtype = dt; a.heads = nq; a.kv_heads = nk; a.sq = S; a.sk = S; a.d = kHeadDim;
        a.q_hs = a.k_hs = a.v_hs = kHeadDim; a.q_rs = a.k_rs = a.v_rs = QKV;
        a.o_hs = kHeadDim; a.o_rs = QD;
        a.mask = mask; a.mask_heads = 1; a.mask_rows = mask ? S : 1; a.causal = causal;
        a.split_ws = split_ws; a.split_ws_bytes = split_ws_bytes;
        // All-key FLOP (the causal launch skips about half of them).
        Timed t(ctx, P_SDPA, 4.0 * dS * dS * kHeadDim * nq, dS * (2 * QD + 2 * KVD) * e);
        rc = kernel_status(ctx, sdpa(a, s), "text sdpa");
        if (rc) return rc;
    }
    {
        GemmArgs g;
        g.A = attn; g.lda = QD; g.W = w.wo.ptr; g.ldw = QD; g.M = S; g.N = H; g.K = QD; g.dtype = dt;
        g.w_k32 = w.k32[1];
        g.epilogue = EPI_GATE_RESID; g.C = x1; g.ldc = H; g.c_dtype = ERNIE_DTYPE_FP32; g.resid = x; g.ld_resid = H;
        g.gate = ones;
        g.split_ws = split_ws; g.split_ws_bytes = split_ws_bytes;
        Timed t(ctx, P_OUT, 2.0 * dS * H * QD, gemm_bytes(dS, H, QD, e, 8));
        rc = kernel_status(ctx, gemm(g, s), "text gemm o");
        if (rc) return rc;
    }
    {
        Timed t(ctx, P_NORM, 0, dS * H * (4 + e));
        rc = kernel_status(ctx, rmsnorm_modulate(x1, ERNIE_DTYPE_FP32, static_cast<const float*>(w.norm2.ptr), nullptr,
                                                 nullptr, S, H, 1e-5f, h, dt, s), "text rmsnorm 2");
        if (rc) return rc;
    }
    {
        GemmArgs g;
        g.A = h; g.lda = H; g.W = w.w_ug.ptr; g.ldw = H; g.M = S; g.N = 2 * F; g.K = H; g.dtype = dt;
        g.w_k32 = w.k32[2];
        g.epilogue = EPI_SWIGLU; g.C = p; g.ldc = F; g.c_dtype = dt;
        g.split_ws = split_ws; g.split_ws_bytes = split_ws_bytes;
        Timed t(ctx, P_UG, 2.0 * dS * 2 * F * H, gemm_bytes(dS, 2.0 * F, H, e, 0) + dS * F * e);
        rc = kernel_status(ctx, gemm(g, s), "text gemm gate/up");
        if (rc) return rc;
    }
    {
        GemmArgs g;
        g.A = p; g.lda = F; g.W = w.w_down.ptr; g.ldw = F; g.M = S; g.N = H; g.K = F; g.dtype = dt;
        g.w_k32 = w.k32[3];
        g.epilogue = EPI_GATE_RESID; g.C = out; g.ldc = H; g.c_dtype = ERNIE_DTYPE_FP32; g.resid = x1; g.ld_resid = H;
        g.gate = ones;
        g.split_ws = split_ws; g.split_ws_bytes = split_ws_bytes;
        Timed t(ctx, P_DOWN, 2.0 * dS * H * F, gemm_bytes(dS, H, F, e, 8));
        rc = kernel_status(ctx, gemm(g, s), "text gemm down");
        if (rc) return rc;
    }
    return ERNIE_OK;
}

int check_text_dims(ernie_hip_ctx* ctx, int hidden, int heads, int kv_heads, int ffn, int dtype)
{
    if (!valid_dtype(dtype)) return fail(ctx, ERNIE_ERROR, "invalid dtype");
    if (hidden < 128 || hidden % 128 || hidden > 4096) return fail(ctx, ERNIE_ERROR, "hidden must be a multiple of 128 in [128,4096]");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || heads * 128 > 8192)
        return fail(ctx, ERNIE_ERROR, "heads must be a positive multiple of kv_heads, at most 64");
    if (ffn < 32 || ffn % 32) return fail(ctx, ERNIE_ERROR, "ffn must be a positive multiple of 32");
    return ERNIE_OK;
}

int alloc_text_block(ernie_hip_ctx* ctx, TextBlockWeights& w, int hidden, int heads, int kv_heads, int ffn, int dtype)
{
    const size_t e = esize(dtype), QKV = (size_t)(heads + 2 * kv_heads) * 128;
    int rc = 0;
    rc = rc ? rc : dev_alloc(ctx, w.norm1, (size_t)hidden * 4, "text block weights");
    rc = rc ? rc : dev_alloc(ctx, w.norm2, (size_t)hidden * 4, "text block weights");
    rc = rc ? rc : dev_alloc(ctx, w.wqkv, QKV * hidden * e, "text block weights");
    rc = rc ? rc : dev_alloc(ctx, w.wo, (size_t)hidden * heads * 128 * e, "text block weights");
    rc = rc ? rc : dev_alloc(ctx, w.w_ug, 2 * (size_t)ffn * hidden * e, "text block weights");
    rc = rc ? rc : dev_alloc(ctx, w.w_down, (size_t)hidden * ffn * e, "text block weights");
    if (rc) {
        free_text_block(w);
        return rc;
    }
    w.hidden = hidden; w.heads = heads; w.kv_heads = kv_heads; w.ffn = ffn; w.dtype = dtype;
    return ERNIE_OK;
}

TextBlockWeights* text_slot(ernie_hip_ctx* ctx, int index)
{
    if (index < 0 || index > 4096) return nullptr;
    if ((size_t)index >= ctx->text_blocks.size()) ctx->text_blocks.resize(index + 1);
    return &ctx->text_blocks[index];
}

int check_text_call(ernie_hip_ctx* ctx, int index, int S, const void* x, const void* out, const void* cos_t,
                    const void* sin_t)
{
    if (index < 0 || (size_t)index >= ctx->text_blocks.size() || !ctx->text_blocks[index].loaded)
        return fail(ctx, ERNIE_ERROR, "text block " + std::to_string(index) + " is not loaded");
    if (S < 1 || S > 65536) return fail(ctx, ERNIE_ERROR, "token count out of range");
    if (!x || !out || !cos_t || !sin_t) return fail(ctx, ERNIE_ERROR, "null text block tensor");
    return ERNIE_OK;
}

// ---- heads ------------------------------------------------------------------------
int head_gemm(ernie_hip_ctx* ctx, const void* a, const void* w, const float* bias, float* c, int M, int N, int K, int dt)
{
    GemmArgs g;
    g.A = a; g.lda = K; g.W = w; g.ldw = K; g.M = M; g.N = N; g.K = K; g.dtype = dt;
    g.epilogue = EPI_STORE; g.C = c; g.ldc = N; g.c_dtype = ERNIE_DTYPE_FP32; g.bias = bias;
    // The split-K scratch lets the narrow projections (4096 -> 128 output channels: 16
    // tiles; the text rows: one partial row of tiles) spread over the CUs.
    int rc = split_workspace(ctx, M, 1, &g.split_ws, &g.split_ws_bytes);
    if (rc) return rc;
    Timed t(ctx, P_HEADS, 2.0 * M * N * K, gemm_bytes(M, N, K, (double)esize(dt), 4));
    return kernel_status(ctx, gemm(g, ctx->stream), "head gemm");
}

int input_head(ernie_hip_ctx* ctx, const float* latent, int hw, const float* text, int T, const float* feat, float* x,
               float* c, float* mods)
{
    const HeadWeights& h = ctx->heads;
    const int D = h.dim, dt = h.dtype;
    const size_t e = esize(dt);
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t tok = up((size_t)hw * h.latent_ch * e), txt = up((size_t)T * h.text_dim * e), t1 = up((size_t)D * 4);
    int rc = dev_alloc(ctx, ctx->head_ws, tok + txt + t1, "head workspace");
    if (rc) return rc;
    char* b = static_cast<char*>(ctx->head_ws.ptr);
    void* tokens = b;
    void* text_d = b + tok;
    float* t1v = reinterpret_cast<float*>(b + tok + txt);
    hipStream_t s = ctx->stream;
    rc = kernel_status(ctx, transpose_to_tokens(latent, h.latent_ch, hw, tokens, dt, s), "latent tokens");
    if (rc) return rc;
    rc = head_gemm(ctx, tokens, h.x_w.ptr, static_cast<const float*>(h.x_b.ptr), x, hw, D, h.latent_ch, dt);
    if (rc) return rc;
    if (T > 0) {
        rc = kernel_status(ctx, convert(text, ERNIE_DTYPE_FP32, text_d, dt, (size_t)T * h.text_dim, s), "text convert");
        if (rc) return rc;
        rc = head_gemm(ctx, text_d, h.text_w.ptr, nullptr, x + (size_t)hw * D, T, D, h.text_dim, dt);
        if (rc) return rc;
    }
    Timed t(ctx, P_HEADS, 2.0 * D * (8.0 * D), (double)D * 8 * D * e);
    rc = kernel_status(ctx, gemv(h.t1_w.ptr, dt, static_cast<const float*>(h.t1_b.ptr), feat, D, D, 0, t1v, s), "time mlp 1");
    if (rc) return rc;
    rc = kernel_status(ctx, gemv(h.t2_w.ptr, dt, static_cast<const float*>(h.t2_b.ptr), t1v, D, D, 1, c, s), "time mlp 2");
    if (rc) return rc;
    return kernel_status(ctx, gemv(h.mod_w.ptr, dt, static_cast<const float*>(h.mod_b.ptr), c, 6 * D, D, 1, mods, s),
                         "adaLN");
}

int output_head(ernie_hip_ctx* ctx, const float* x, int hw, const float* c, float* pred)
{
    const HeadWeights& h = ctx->heads;
    const int D = h.dim, dt = h.dtype;
    const size_t e = esize(dt);
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t mm = up(2 * (size_t)D * 4), y = up((size_t)hw * D * e), proj = up((size_t)hw * h.latent_ch * 4);
    int rc = dev_alloc(ctx, ctx->head_ws, mm + y + proj, "head workspace");
    if (rc) return rc;
    char* b = static_cast<char*>(ctx->head_ws.ptr);
    float* mmv = reinterpret_cast<float*>(b);
    void* yv = b + mm;
    float* projv = reinterpret_cast<float*>(b + mm + y);
    hipStream_t s = ctx->stream;
    {
        Timed t(ctx, P_HEADS, 2.0 * D * 2 * D, 2.0 * D * D * e);
        rc = kernel_status(ctx, gemv(h.out_mod_w.ptr, dt, static_cast<const float*>(h.out_mod_b.ptr), c, 2 * D, D, 0,
                                     mmv, s), "output adaLN");
        if (rc) return rc;
    }
    rc = kernel_status(ctx, layernorm_modulate(x, mmv + D, mmv, hw, D, 1e-6f, yv, dt, s), "output layernorm");
    if (rc) return rc;
    rc = head_gemm(ctx, yv, h.proj_w.ptr, static_cast<const float*>(h.proj_b.ptr), projv, hw, h.latent_ch, D, dt);
    if (rc) return rc;
    return kernel_status(ctx, tokens_to_latent(projv, hw, h.latent_ch, pred, s), "output unpatchify");
}

// At least n timing events in the context's pool (created once, reused by later calls).
int sequence_events(ernie_hip_ctx* ctx, int n)
{
    while ((int)ctx->seq_events.size() < n) {
        hipEvent_t e = nullptr;
        const int rc = hip_status(ctx, hipEventCreate(&e), "event create");
        if (rc) return rc;
        ctx->seq_events.push_back(e);
    }
    return ERNIE_OK;
}

// Records the closing event after `count` timed items, waits for it once and writes the
// device time between consecutive events.
int sequence_seconds(ernie_hip_ctx* ctx, int count, double* seconds)
{
    int rc = hip_status(ctx, hipEventRecord(ctx->seq_events[count], ctx->stream), "block timing");
    if (!rc) rc = hip_status(ctx, hipEventSynchronize(ctx->seq_events[count]), "block timing");
    for (int i = 0; i < count && !rc; ++i) {
        float ms = 0.f;
        rc = hip_status(ctx, hipEventElapsedTime(&ms, ctx->seq_events[i], ctx->seq_events[i + 1]), "block timing");
        seconds[i] = ms * 1e-3;
    }
    return rc;
}

int check_block_call(ernie_hip_ctx* ctx, int index, int S, const void* x, const void* out, const void* mods,
                     const void* cos_t, const void* sin_t, int valid_keys)
{
    if (index < 0 || (size_t)index >= ctx->blocks.size() || !ctx->blocks[index].loaded)
        return fail(ctx, ERNIE_ERROR, "block " + std::to_string(index) + " is not loaded");
    if (S < 1 || S > 65536) return fail(ctx, ERNIE_ERROR, "token count out of range");
    if (!x || !out || !mods || !cos_t || !sin_t) return fail(ctx, ERNIE_ERROR, "null block tensor");
    if (valid_keys < 0 || valid_keys > S) return fail(ctx, ERNIE_ERROR, "valid_keys out of range");
    return ERNIE_OK;
}

// Makes a context's device current for the duration of one entry point and gives the
// calling thread its own selection back afterwards. Allocations (hipMalloc), device
// queries (the GEMM launcher's CU count) and launches then all refer to the context's
// device, whichever device the calling thread had selected before the call.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int device)
    {
        if (device < 0) return;
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev == device) {
            prev = -1;
            return;
        }
        ok = hipSetDevice(device) == hipSuccess;
        if (!ok) (void)hipGetLastError();
    }
    explicit DeviceGuard(const ernie_hip_ctx* ctx) : DeviceGuard(ctx ? ctx->device : -1) {}
    ~DeviceGuard()
    {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;
};

}  // namespace

// =====================================================================================
extern "C" {

int ernie_hip_create(int device, ernie_hip_ctx** out)
{
    if (!out) return ERNIE_ERROR;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return ERNIE_ERROR;
    DeviceGuard guard(device);
    if (!guard.ok) return ERNIE_ERROR;
    auto* ctx = new (std::nothrow) ernie_hip_ctx();
    if (!ctx) return ERNIE_ALLOCATION_FAILED;
    ctx->device = device;
    if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return ERNIE_ERROR;
    }
    ctx->stream = ctx->own_stream;
    if (scratch_init(device) == 0) ctx->scratch = scratch_address(device);
    *out = ctx;
    return ERNIE_OK;
}

void ernie_hip_destroy(ernie_hip_ctx* ctx)
{
    DeviceGuard guard(ctx);
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& b : ctx->blocks) free_block(b);
    for (auto& b : ctx->text_blocks) free_text_block(b);
    free_heads(ctx->heads);
    dev_free(ctx->text_ws);
    dev_free(ctx->ones);
    dev_free(ctx->ws);
    dev_free(ctx->staging);
    dev_free(ctx->head_ws);
    dev_free(ctx->dit_act);
    dev_free(ctx->split_ws);
    dev_free(ctx->rope_pack);
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->seq_events) (void)hipEventDestroy(e);
    for (auto& st : ctx->upload_staging) {
        (void)hipEventDestroy(st.done);
        (void)hipHostFree(st.host);
    }
    for (hipEvent_t e : ctx->marker)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->finite_event)
        if (e) (void)hipEventDestroy(e);
    release_cache(ctx);
    for (auto& kv : ctx->live) (void)hipFree(kv.first);
    if (ctx->finite_flag) (void)hipFree(ctx->finite_flag);
    if (ctx->finite_host) (void)hipHostFree(ctx->finite_host);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

const char* ernie_hip_last_error(const ernie_hip_ctx* ctx) { return ctx ? ctx->error.c_str() : "null context"; }

int ernie_hip_set_stream(ernie_hip_ctx* ctx, void* stream)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    // Cached blocks may still be in use by work on the old stream: let it finish first.
    if (ctx->stream != static_cast<hipStream_t>(stream) && ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    ctx->stream = static_cast<hipStream_t>(stream);
    return ERNIE_OK;
}

void* ernie_hip_own_stream(ernie_hip_ctx* ctx) { return ctx ? ctx->own_stream : nullptr; }

void* ernie_hip_get_stream(ernie_hip_ctx* ctx) { return ctx ? ctx->stream : nullptr; }

int ernie_hip_synchronize(ernie_hip_ctx* ctx)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return hip_status(ctx, hipStreamSynchronize(ctx->stream), "synchronize");
}

// Freed blocks the cache keeps at most (larger frees go back to the driver).
constexpr size_t kCacheCapBytes = size_t(8) << 30;

int ernie_hip_malloc(ernie_hip_ctx* ctx, size_t bytes, void** out)
{
    DeviceGuard guard(ctx);
    if (!ctx || !out) return ERNIE_ERROR;
    *out = nullptr;
    const size_t b = ((bytes ? bytes : 1) + 255) / 256 * 256;
    {
        std::lock_guard<std::mutex> lock(ctx->alloc_mu);
        auto it = ctx->free_cache.find(b);
        if (it != ctx->free_cache.end()) {
            *out = it->second;
            ctx->free_cache.erase(it);
            ctx->cached_bytes -= b;
            ctx->live[*out] = b;
            return ERNIE_OK;
        }
    }
    const int rc = hip_status(ctx, device_malloc(ctx, out, b), "malloc");
    if (!rc) {
        std::lock_guard<std::mutex> lock(ctx->alloc_mu);
        ctx->live[*out] = b;
    }
    return rc;
}

int ernie_hip_free(ernie_hip_ctx* ctx, void* ptr)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!ptr) return ERNIE_OK;
    {
        std::lock_guard<std::mutex> lock(ctx->alloc_mu);
        auto it = ctx->live.find(ptr);
        if (it != ctx->live.end()) {
            const size_t b = it->second;
            ctx->live.erase(it);
            if (ctx->cached_bytes + b <= kCacheCapBytes) {
                ctx->free_cache.emplace(b, ptr);
                ctx->cached_bytes += b;
                return ERNIE_OK;
            }
        }
    }
    return hip_status(ctx, hipFree(ptr), "free");
}

size_t ernie_hip_trim(ernie_hip_ctx* ctx)
{
    DeviceGuard guard(ctx);
    if (!ctx) return 0;
    (void)hipStreamSynchronize(ctx->stream);
    return release_cache(ctx);
}

int ernie_hip_memcpy_h2d(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = hip_status(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "h2d");
    return rc ? rc : hip_status(ctx, hipStreamSynchronize(ctx->stream), "h2d");
}

int ernie_hip_upload_async(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    DeviceGuard guard(ctx);
    if (!ctx || (!src && bytes) || (!dst && bytes)) return ERNIE_ERROR;
    if (!bytes) return ERNIE_OK;
    // A staging block whose previous copy has finished and that is large enough.
    ernie_hip_ctx::Staging* st = nullptr;
    for (auto& b : ctx->upload_staging)
        if (b.bytes >= bytes && hipEventQuery(b.done) == hipSuccess) {
            st = &b;
            break;
        }
    if (!st) {
        if (ctx->upload_staging.size() >= 64) return fail(ctx, ERNIE_ERROR, "too many uploads in flight");
        ernie_hip_ctx::Staging b{nullptr, std::max<size_t>(bytes, size_t(64) << 10), nullptr};
        int rc = hip_status(ctx, hipHostMalloc(&b.host, b.bytes, 0), "upload staging");
        if (!rc) rc = hip_status(ctx, hipEventCreateWithFlags(&b.done, hipEventDisableTiming), "upload staging");
        if (rc) {
            if (b.host) (void)hipHostFree(b.host);
            return rc;
        }
        ctx->upload_staging.push_back(b);
        st = &ctx->upload_staging.back();
    }
    std::memcpy(st->host, src, bytes);
    int rc = hip_status(ctx, hipMemcpyAsync(dst, st->host, bytes, hipMemcpyHostToDevice, ctx->stream), "upload");
    if (!rc) rc = hip_status(ctx, hipEventRecord(st->done, ctx->stream), "upload");
    return rc;
}

int ernie_hip_memcpy_d2h(ernie_hip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = hip_status(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "d2h");
    return rc ? rc : hip_status(ctx, hipStreamSynchronize(ctx->stream), "d2h");
}

// ---- operators ----------------------------------------------------------------------
int ernie_hip_rmsnorm(ernie_hip_ctx* ctx, const void* x, int x_dtype, const float* gamma, const float* shift,
                      const float* scale, int rows, int width, float eps, void* out, int out_dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, rmsnorm_modulate(x, x_dtype, gamma, shift, scale, rows, width, eps, out, out_dtype,
                                               ctx->stream), "rmsnorm");
}

int ernie_hip_layernorm_modulate(ernie_hip_ctx* ctx, const float* x, const float* shift, const float* scale, int rows,
                                 int width, float eps, void* out, int out_dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, layernorm_modulate(x, shift, scale, rows, width, eps, out, out_dtype, ctx->stream),
                         "layernorm");
}

int ernie_hip_gelu(ernie_hip_ctx* ctx, void* data, int dtype, size_t count)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, gelu_inplace(data, dtype, count, ctx->stream), "gelu");
}

int ernie_hip_residual_add(ernie_hip_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, float* out,
                           size_t count)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, residual_add(a, a_dtype, b, b_dtype, out, count, ctx->stream), "residual_add");
}

int ernie_hip_gemm(ernie_hip_ctx* ctx, const void* a, long lda, const void* w, long ldw, const float* bias, void* c,
                   long ldc, int m, int n, int k, int dtype, int out_dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    GemmArgs g;
    g.A = a; g.lda = lda; g.W = w; g.ldw = ldw; g.M = m; g.N = n; g.K = k; g.dtype = dtype;
    g.epilogue = EPI_STORE; g.C = c; g.ldc = ldc; g.c_dtype = out_dtype; g.bias = bias;
    return kernel_status(ctx, gemm(g, ctx->stream), "gemm");
}

// The standalone attention takes the same key-range split of a partial last 128-query
// tile as the block does (16-bit, head_dim 128), with the context's split workspace.
static int attention_workspace(ernie_hip_ctx* ctx, SdpaArgs& a)
{
    if (a.d != 128 || a.dtype == ERNIE_DTYPE_FP32 || a.sq % 128 == 0 || a.sq < 128) return ERNIE_OK;
    return split_workspace(ctx, a.sq, a.heads, &a.split_ws, &a.split_ws_bytes);
}

int ernie_hip_sdpa(ernie_hip_ctx* ctx, const void* q, const void* k, const void* v, void* out, int dtype, int heads,
                   int kv_heads, int sq, int sk, int d, long q_hs, long q_rs, long k_hs, long k_rs, long v_hs,
                   long v_rs, long o_hs, long o_rs, const float* mask, int mask_heads, int mask_rows, int valid_keys,
                   float scale)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    SdpaArgs a;
    a.q = q; a.k = k; a.v = v; a.o = out; a.dtype = dtype; a.heads = heads; a.kv_heads = kv_heads;
    a.sq = sq; a.sk = sk; a.d = d; a.q_hs = q_hs; a.q_rs = q_rs; a.k_hs = k_hs; a.k_rs = k_rs;
    a.v_hs = v_hs; a.v_rs = v_rs; a.o_hs = o_hs; a.o_rs = o_rs; a.mask = mask; a.mask_heads = mask_heads;
    a.mask_rows = mask_rows; a.valid_keys = valid_keys; a.scale = scale;
    const int rc = attention_workspace(ctx, a);
    if (rc) return rc;
    return kernel_status(ctx, sdpa(a, ctx->stream), "sdpa");
}

int ernie_hip_sdpa_causal(ernie_hip_ctx* ctx, const void* q, const void* k, const void* v, void* out, int dtype,
                          int heads, int kv_heads, int sq, int sk, int d, long q_hs, long q_rs, long k_hs, long k_rs,
                          long v_hs, long v_rs, long o_hs, long o_rs, float scale)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    SdpaArgs a;
    a.q = q; a.k = k; a.v = v; a.o = out; a.dtype = dtype; a.heads = heads; a.kv_heads = kv_heads;
    a.sq = sq; a.sk = sk; a.d = d; a.q_hs = q_hs; a.q_rs = q_rs; a.k_hs = k_hs; a.k_rs = k_rs;
    a.v_hs = v_hs; a.v_rs = v_rs; a.o_hs = o_hs; a.o_rs = o_rs; a.causal = 1; a.scale = scale;
    const int rc = attention_workspace(ctx, a);
    if (rc) return rc;
    return kernel_status(ctx, sdpa(a, ctx->stream), "sdpa causal");
}

int ernie_hip_set_attention_query_rows(ernie_hip_ctx* ctx, int rows)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (rows != 128 && rows != 64 && rows != 32 && rows != 16)
        return fail(ctx, ERNIE_ERROR, "Attention query rows must be 128, 64, 32 or 16");
    ctx->query_rows = rows;
    return ERNIE_OK;
}

uint64_t ernie_hip_attention_internal_submissions(const ernie_hip_ctx*) { return 0; }

int ernie_hip_set_qk_rounding(ernie_hip_ctx* ctx, int mode)
{
    if (!ctx) return ERNIE_ERROR;
    if (mode != ERNIE_QK_ROUND_FUSED && mode != ERNIE_QK_ROUND_STORAGE)
        return fail(ctx, ERNIE_ERROR, "Q/K rounding mode must be ERNIE_QK_ROUND_FUSED or ERNIE_QK_ROUND_STORAGE");
    ctx->qk_storage_rounding = mode == ERNIE_QK_ROUND_STORAGE;
    return ERNIE_OK;
}

int ernie_hip_qk_norm_rope(ernie_hip_ctx* ctx, void* x, int dtype, int rows, int heads, long row_stride,
                           const float* gamma, const float* cos_t, const float* sin_t)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, qk_norm_rope(x, dtype, rows, heads, row_stride, gamma, cos_t, sin_t, ctx->stream),
                         "qk_norm_rope");
}

int ernie_hip_euler_step(ernie_hip_ctx* ctx, const float* x, const float* v, float delta, size_t count, float* out)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!std::isfinite(delta) || delta >= 0.f || delta < -1.f)
        return fail(ctx, ERNIE_ERROR, "Incompatible Euler shapes or delta outside [-1,0)");
    return kernel_status(ctx, euler_step(x, v, delta, count, out, ctx->stream), "euler");
}

// Lazily creates the finiteness flags (device), their pinned host copies and events.
static int finite_setup(ernie_hip_ctx* ctx)
{
    if (ctx->finite_flag) return ERNIE_OK;
    constexpr int n = kFiniteSlots + 1;
    int rc = hip_status(ctx, device_malloc(ctx, reinterpret_cast<void**>(&ctx->finite_flag), n * sizeof(int)),
                        "finite flags");
    if (!rc) rc = hip_status(ctx, hipHostMalloc(reinterpret_cast<void**>(&ctx->finite_host), n * sizeof(int), 0),
                             "finite flags");
    for (int i = 0; i < kFiniteSlots && !rc; ++i)
        rc = hip_status(ctx, hipEventCreateWithFlags(&ctx->finite_event[i], hipEventDisableTiming), "finite event");
    if (rc) {
        for (hipEvent_t& e : ctx->finite_event)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        if (ctx->finite_host) (void)hipHostFree(ctx->finite_host);
        if (ctx->finite_flag) (void)hipFree(ctx->finite_flag);
        ctx->finite_host = nullptr;
        ctx->finite_flag = nullptr;
    }
    return rc;
}

// Clears flag `index`, checks x into it and queues its copy to the pinned host slot.
static int finite_enqueue(ernie_hip_ctx* ctx, const float* x, size_t count, int index)
{
    int rc = finite_setup(ctx);
    int* flag = ctx ? ctx->finite_flag + index : nullptr;
    if (!rc) rc = kernel_status(ctx, fill_int(flag, 0, 1, ctx->stream), "finite flag");
    if (!rc) rc = kernel_status(ctx, finite_flags(x, count, flag, ctx->stream), "finite");
    if (!rc) rc = hip_status(ctx, hipMemcpyAsync(ctx->finite_host + index, flag, sizeof(int), hipMemcpyDeviceToHost,
                                                 ctx->stream), "finite");
    return rc;
}

int ernie_hip_finite(ernie_hip_ctx* ctx, const float* x, size_t count, int* finite)
{
    DeviceGuard guard(ctx);
    if (!ctx || !finite || (!x && count)) return ERNIE_ERROR;
    int rc = finite_enqueue(ctx, x, count, kFiniteSlots);
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "finite");
    if (!rc) *finite = ctx->finite_host[kFiniteSlots] ? 0 : 1;
    return rc;
}

int ernie_hip_finite_begin(ernie_hip_ctx* ctx, const float* x, size_t count, int slot)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (slot < 0 || slot >= kFiniteSlots) return fail(ctx, ERNIE_ERROR, "finite slot out of range");
    if (!x && count) return fail(ctx, ERNIE_ERROR, "null finite input");
    int rc = finite_enqueue(ctx, x, count, slot);
    if (!rc) rc = hip_status(ctx, hipEventRecord(ctx->finite_event[slot], ctx->stream), "finite event");
    ctx->finite_pending[slot] = rc == ERNIE_OK;
    return rc;
}

int ernie_hip_finite_end(ernie_hip_ctx* ctx, int slot, int* finite)
{
    DeviceGuard guard(ctx);
    if (!ctx || !finite) return ERNIE_ERROR;
    if (slot < 0 || slot >= kFiniteSlots || !ctx->finite_pending[slot])
        return fail(ctx, ERNIE_ERROR, "no finite check pending in this slot");
    ctx->finite_pending[slot] = false;
    const int rc = hip_status(ctx, hipEventSynchronize(ctx->finite_event[slot]), "finite wait");
    if (!rc) *finite = ctx->finite_host[slot] ? 0 : 1;
    return rc;
}

int ernie_hip_marker_record(ernie_hip_ctx* ctx, int marker)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (marker < 0 || marker >= kMarkers) return fail(ctx, ERNIE_ERROR, "marker out of range");
    if (!ctx->marker[marker]) {
        const int rc = hip_status(ctx, hipEventCreate(&ctx->marker[marker]), "marker");
        if (rc) return rc;
    }
    const int rc = hip_status(ctx, hipEventRecord(ctx->marker[marker], ctx->stream), "marker");
    ctx->marker_recorded[marker] = rc == ERNIE_OK;
    return rc;
}

int ernie_hip_marker_elapsed(ernie_hip_ctx* ctx, int from, int to, double* seconds)
{
    DeviceGuard guard(ctx);
    if (!ctx || !seconds) return ERNIE_ERROR;
    if (from < 0 || to < 0 || from >= kMarkers || to >= kMarkers || !ctx->marker_recorded[from] ||
        !ctx->marker_recorded[to])
        return fail(ctx, ERNIE_ERROR, "marker not recorded");
    int rc = hip_status(ctx, hipEventSynchronize(ctx->marker[to]), "marker wait");
    float ms = 0.f;
    if (!rc) rc = hip_status(ctx, hipEventElapsedTime(&ms, ctx->marker[from], ctx->marker[to]), "marker elapsed");
    if (!rc) *seconds = ms * 1e-3;
    return rc;
}

int ernie_hip_transpose(ernie_hip_ctx* ctx, const void* in, int dtype, int rows, int cols, void* out)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (in == out && rows > 1 && cols > 1) return fail(ctx, ERNIE_ERROR, "transpose cannot run in place");
    return kernel_status(ctx, transpose2d(in, dtype, rows, cols, out, ctx->stream), "transpose");
}

int ernie_hip_fill_normal(ernie_hip_ctx* ctx, void* out, int dtype, size_t count, uint64_t seed, uint64_t offset,
                          float mean, float std_dev)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, fill_normal(out, dtype, count, seed, offset, mean, std_dev, ctx->stream), "fill_normal");
}

int ernie_hip_convert(ernie_hip_ctx* ctx, const void* in, int in_dtype, void* out, int out_dtype, size_t count)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    return kernel_status(ctx, convert(in, in_dtype, out, out_dtype, count, ctx->stream), "convert");
}

// ---- blocks -----------------------------------------------------------------------------
int ernie_hip_block_upload_tensors(ernie_hip_ctx* ctx, int index, const ernie_block_host_tensors* w, int dim, int ffn,
                                   int dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx || !w) return ERNIE_ERROR;
    int rc = check_block_dims(ctx, dim, ffn, dtype);
    if (rc) return rc;
    const ernie_host_tensor* parts[] = {&w->norm1, &w->wq, &w->wk, &w->wv, &w->norm_q, &w->norm_k,
                                        &w->wo, &w->norm2, &w->w_up, &w->w_gate, &w->w_down};
    for (const ernie_host_tensor* t : parts) {
        if (!t->data) return fail(ctx, ERNIE_ERROR, "null block weight");
        if (!valid_dtype(t->dtype)) return fail(ctx, ERNIE_ERROR, "invalid block weight dtype");
    }
    BlockWeights* slot = block_slot(ctx, index);
    if (!slot) return fail(ctx, ERNIE_ERROR, "block index out of range");
    free_block(*slot);
    BlockWeights bw;
    rc = alloc_block(ctx, bw, dim, ffn, dtype);
    if (rc) return rc;
    const size_t DD = (size_t)dim * dim, DF = (size_t)dim * ffn;
    constexpr int F32 = ERNIE_DTYPE_FP32;
    // RMSNorm gammas stay FP32 whatever the storage precision (src/ernie_rmsnorm.cpp:11-17).
    rc = rc ? rc : upload_tensor(ctx, bw.norm1.ptr, 0, F32, w->norm1.data, w->norm1.dtype, dim, "norm1");
    rc = rc ? rc : upload_tensor(ctx, bw.norm2.ptr, 0, F32, w->norm2.data, w->norm2.dtype, dim, "norm2");
    rc = rc ? rc : upload_tensor(ctx, bw.norm_q.ptr, 0, F32, w->norm_q.data, w->norm_q.dtype, kHeadDim, "norm_q");
    rc = rc ? rc : upload_tensor(ctx, bw.norm_k.ptr, 0, F32, w->norm_k.data, w->norm_k.dtype, kHeadDim, "norm_k");
    rc = rc ? rc : upload_tensor(ctx, bw.wqkv.ptr, 0, dtype, w->wq.data, w->wq.dtype, DD, "wq");
    rc = rc ? rc : upload_tensor(ctx, bw.wqkv.ptr, DD, dtype, w->wk.data, w->wk.dtype, DD, "wk");
    rc = rc ? rc : upload_tensor(ctx, bw.wqkv.ptr, 2 * DD, dtype, w->wv.data, w->wv.dtype, DD, "wv");
    rc = rc ? rc : upload_tensor(ctx, bw.wo.ptr, 0, dtype, w->wo.data, w->wo.dtype, DD, "wo");
    rc = rc ? rc : upload_tensor(ctx, bw.w_down.ptr, 0, dtype, w->w_down.data, w->w_down.dtype, DF, "w_down");
    for (int parity = 0; parity < 2 && !rc; ++parity) {
        const ernie_host_tensor& src = parity ? w->w_gate : w->w_up;
        const size_t bytes = DF * esize(src.dtype);
        rc = dev_alloc(ctx, ctx->staging, bytes, "staging buffer");
        if (!rc) rc = hip_status(ctx, hipMemcpyAsync(ctx->staging.ptr, src.data, bytes, hipMemcpyHostToDevice, ctx->stream), "w_ug");
        if (!rc) rc = kernel_status(ctx, interleave_up_gate(ctx->staging.ptr, src.dtype, bw.w_ug.ptr, dtype, ffn, dim,
                                                            parity, ctx->stream), "w_ug");
        if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "w_ug");
    }
    // Host memory may be released once this returns: every copy out of it has finished.
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "block upload");
    if (!rc) rc = tile_block_weights(ctx, bw);
    if (rc) {
        free_block(bw);
        return rc;
    }
    bw.loaded = true;
    *slot = bw;
    return ERNIE_OK;
}

int ernie_hip_block_upload(ernie_hip_ctx* ctx, int index, const ernie_block_host_weights* w, int dim, int ffn,
                           int dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx || !w) return ERNIE_ERROR;
    auto f32 = [](const float* p) { return ernie_host_tensor{p, ERNIE_DTYPE_FP32}; };
    const ernie_block_host_tensors t = {f32(w->norm1), f32(w->wq),     f32(w->wk),     f32(w->wv),
                                        f32(w->norm_q), f32(w->norm_k), f32(w->wo),     f32(w->norm2),
                                        f32(w->w_up),  f32(w->w_gate), f32(w->w_down)};
    return ernie_hip_block_upload_tensors(ctx, index, &t, dim, ffn, dtype);
}

int ernie_hip_block_init_random(ernie_hip_ctx* ctx, int index, int dim, int ffn, int dtype, uint64_t seed,
                                float std_dev)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = check_block_dims(ctx, dim, ffn, dtype);
    if (rc) return rc;
    BlockWeights* slot = block_slot(ctx, index);
    if (!slot) return fail(ctx, ERNIE_ERROR, "block index out of range");
    free_block(*slot);
    BlockWeights bw;
    rc = alloc_block(ctx, bw, dim, ffn, dtype);
    if (rc) return rc;
    const uint64_t stride = 1ull << 40;  // independent sub-stream per tensor
    hipStream_t s = ctx->stream;
    struct Item { void* p; int dt; size_t n; float mean; };
    const Item items[] = {
        {bw.norm1.ptr, ERNIE_DTYPE_FP32, (size_t)dim, 1.f}, {bw.wqkv.ptr, dtype, 3 * (size_t)dim * dim, 0.f},
        {bw.norm_q.ptr, ERNIE_DTYPE_FP32, kHeadDim, 1.f},   {bw.norm_k.ptr, ERNIE_DTYPE_FP32, kHeadDim, 1.f},
        {bw.wo.ptr, dtype, (size_t)dim * dim, 0.f}, {bw.norm2.ptr, ERNIE_DTYPE_FP32, (size_t)dim, 1.f},
        {bw.w_ug.ptr, dtype, 2 * (size_t)ffn * dim, 0.f}, {bw.w_down.ptr, dtype, (size_t)dim * ffn, 0.f}};
    uint64_t k = 0;
    for (const Item& it : items) {
        rc = kernel_status(ctx, fill_normal(it.p, it.dt, it.n, seed, (k++) * stride, it.mean, std_dev, s), "init");
        if (rc) break;
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(s), "init");
    if (!rc) rc = tile_block_weights(ctx, bw);
    if (rc) {
        free_block(bw);
        return rc;
    }
    bw.loaded = true;
    *slot = bw;
    return ERNIE_OK;
}

int ernie_hip_block_release(ernie_hip_ctx* ctx, int index)
{
    DeviceGuard guard(ctx);
    if (!ctx || index < 0 || (size_t)index >= ctx->blocks.size()) return ERNIE_ERROR;
    (void)hipStreamSynchronize(ctx->stream);
    free_block(ctx->blocks[index]);
    return ERNIE_OK;
}

int ernie_hip_block_count(const ernie_hip_ctx* ctx)
{
    if (!ctx) return 0;
    int n = 0;
    for (const auto& b : ctx->blocks) n += b.loaded ? 1 : 0;
    return n;
}

int ernie_hip_block_forward(ernie_hip_ctx* ctx, int index, const float* x, float* out, const float* mods,
                            const float* cos_t, const float* sin_t, const float* mask, int valid_keys, int S)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = check_block_call(ctx, index, S, x, out, mods, cos_t, sin_t, valid_keys);
    const float* cs = nullptr;
    if (!rc) rc = pack_rope(ctx, &index, 1, cos_t, sin_t, S, &cs);
    if (rc) return rc;
    return block_forward(ctx, ctx->blocks[index], x, out, mods, cos_t, sin_t, cs, mask, valid_keys, S);
}

int ernie_hip_block_sequence(ernie_hip_ctx* ctx, const int* blocks, int count, const float* x, float* out,
                             const float* mods, const float* cos_t, const float* sin_t, const float* mask,
                             int valid_keys, int S, double* seconds)
{
    DeviceGuard guard(ctx);
    if (!ctx || !blocks) return ERNIE_ERROR;
    if (count < 1 || count > 36) return fail(ctx, ERNIE_ERROR, "Expected 1..36 blocks");
    for (int i = 0; i < count; ++i) {
        int rc = check_block_call(ctx, blocks[i], S, x, out, mods, cos_t, sin_t, valid_keys);
        if (rc) return rc;
        if (ctx->blocks[blocks[i]].dim != ctx->blocks[blocks[0]].dim)
            return fail(ctx, ERNIE_ERROR, "blocks differ in width");
    }
    // One event before each block and one after the last; a single wait at the end.
    int rc = seconds ? sequence_events(ctx, count + 1) : ERNIE_OK;
    const float* cs = nullptr;
    if (!rc) rc = pack_rope(ctx, blocks, count, cos_t, sin_t, S, &cs);
    for (int i = 0; i < count && !rc; ++i) {
        if (seconds) (void)hipEventRecord(ctx->seq_events[i], ctx->stream);
        rc = block_forward(ctx, ctx->blocks[blocks[i]], i == 0 ? x : out, out, mods, cos_t, sin_t, cs, mask,
                           valid_keys, S);
    }
    if (seconds && !rc) rc = sequence_seconds(ctx, count, seconds);
    return rc;
}

// ---- Mistral text blocks -----------------------------------------------------------------
int ernie_hip_text_block_upload_tensors(ernie_hip_ctx* ctx, int index, const ernie_text_block_host_tensors* w,
                                        int hidden, int heads, int kv_heads, int ffn, int dtype)
{
    DeviceGuard guard(ctx);
    if (!ctx || !w) return ERNIE_ERROR;
    int rc = check_text_dims(ctx, hidden, heads, kv_heads, ffn, dtype);
    if (rc) return rc;
    const ernie_host_tensor* parts[] = {&w->norm1, &w->wq, &w->wk, &w->wv, &w->wo,
                                        &w->norm2, &w->w_gate, &w->w_up, &w->w_down};
    for (const ernie_host_tensor* t : parts) {
        if (!t->data) return fail(ctx, ERNIE_ERROR, "null text block weight");
        if (!valid_dtype(t->dtype)) return fail(ctx, ERNIE_ERROR, "invalid text block weight dtype");
    }
    TextBlockWeights* slot = text_slot(ctx, index);
    if (!slot) return fail(ctx, ERNIE_ERROR, "text block index out of range");
    free_text_block(*slot);
    TextBlockWeights tw;
    rc = alloc_text_block(ctx, tw, hidden, heads, kv_heads, ffn, dtype);
    if (rc) return rc;
    const size_t QD = (size_t)heads * 128 * hidden, KVD = (size_t)kv_heads * 128 * hidden;
    constexpr int F32 = ERNIE_DTYPE_FP32;
    rc = rc ? rc : upload_tensor(ctx, tw.norm1.ptr, 0, F32, w->norm1.data, w->norm1.dtype, hidden, "norm1");
    rc = rc ? rc : upload_tensor(ctx, tw.norm2.ptr, 0, F32, w->norm2.data, w->norm2.dtype, hidden, "norm2");
    rc = rc ? rc : upload_tensor(ctx, tw.wqkv.ptr, 0, dtype, w->wq.data, w->wq.dtype, QD, "wq");
    rc = rc ? rc : upload_tensor(ctx, tw.wqkv.ptr, QD, dtype, w->wk.data, w->wk.dtype, KVD, "wk");
    rc = rc ? rc : upload_tensor(ctx, tw.wqkv.ptr, QD + KVD, dtype, w->wv.data, w->wv.dtype, KVD, "wv");
    rc = rc ? rc : upload_tensor(ctx, tw.wo.ptr, 0, dtype, w->wo.data, w->wo.dtype, QD, "wo");
    rc = rc ? rc : upload_tensor(ctx, tw.w_down.ptr, 0, dtype, w->w_down.data, w->w_down.dtype,
                                 (size_t)hidden * ffn, "w_down");
    for (int parity = 0; parity < 2 && !rc; ++parity) {
        const ernie_host_tensor& src = parity ? w->w_gate : w->w_up;
        const size_t bytes = (size_t)ffn * hidden * esize(src.dtype);
        rc = dev_alloc(ctx, ctx->staging, bytes, "staging buffer");
        if (!rc) rc = hip_status(ctx, hipMemcpyAsync(ctx->staging.ptr, src.data, bytes, hipMemcpyHostToDevice, ctx->stream), "w_ug");
        if (!rc) rc = kernel_status(ctx, interleave_up_gate(ctx->staging.ptr, src.dtype, tw.w_ug.ptr, dtype, ffn, hidden,
                                                            parity, ctx->stream), "w_ug");
        if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "w_ug");
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "text block upload");
    if (!rc) rc = tile_text_weights(ctx, tw);
    if (rc) {
        free_text_block(tw);
        return rc;
    }
    tw.loaded = true;
    *slot = tw;
    return ERNIE_OK;
}

int ernie_hip_text_block_init_random(ernie_hip_ctx* ctx, int index, int hidden, int heads, int kv_heads, int ffn,
                                     int dtype, uint64_t seed, float std_dev)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = check_text_dims(ctx, hidden, heads, kv_heads, ffn, dtype);
    if (rc) return rc;
    TextBlockWeights* slot = text_slot(ctx, index);
    if (!slot) return fail(ctx, ERNIE_ERROR, "text block index out of range");
    free_text_block(*slot);
    TextBlockWeights tw;
    rc = alloc_text_block(ctx, tw, hidden, heads, kv_heads, ffn, dtype);
    if (rc) return rc;
    const uint64_t stride = 1ull << 40;
    struct Item { void* p; int dt; size_t n; float mean; };
    const size_t QKV = (size_t)(heads + 2 * kv_heads) * 128;
    const Item items[] = {{tw.norm1.ptr, ERNIE_DTYPE_FP32, (size_t)hidden, 1.f},
                          {tw.wqkv.ptr, dtype, QKV * hidden, 0.f},
                          {tw.wo.ptr, dtype, (size_t)hidden * heads * 128, 0.f},
                          {tw.norm2.ptr, ERNIE_DTYPE_FP32, (size_t)hidden, 1.f},
                          {tw.w_ug.ptr, dtype, 2 * (size_t)ffn * hidden, 0.f},
                          {tw.w_down.ptr, dtype, (size_t)hidden * ffn, 0.f}};
    uint64_t k = 0;
    for (const Item& it : items) {
        rc = kernel_status(ctx, fill_normal(it.p, it.dt, it.n, seed, (k++) * stride, it.mean, std_dev, ctx->stream),
                           "text init");
        if (rc) break;
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "text init");
    if (!rc) rc = tile_text_weights(ctx, tw);
    if (rc) {
        free_text_block(tw);
        return rc;
    }
    tw.loaded = true;
    *slot = tw;
    return ERNIE_OK;
}

int ernie_hip_text_block_release(ernie_hip_ctx* ctx, int index)
{
    DeviceGuard guard(ctx);
    if (!ctx || index < 0 || (size_t)index >= ctx->text_blocks.size()) return ERNIE_ERROR;
    (void)hipStreamSynchronize(ctx->stream);
    free_text_block(ctx->text_blocks[index]);
    return ERNIE_OK;
}

int ernie_hip_text_block_forward(ernie_hip_ctx* ctx, int index, const float* x, float* out, const float* cos_t,
                                 const float* sin_t, const float* mask, int causal, int S)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    const int rc = check_text_call(ctx, index, S, x, out, cos_t, sin_t);
    if (rc) return rc;
    return text_block_forward(ctx, ctx->text_blocks[index], x, out, cos_t, sin_t, mask, causal, S);
}

int ernie_hip_text_block_forward_noalloc(ernie_hip_ctx* ctx, int index, const float* x, float* out,
                                         const float* cos_t, const float* sin_t, const float* mask, int causal, int S)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = check_text_call(ctx, index, S, x, out, cos_t, sin_t);
    if (rc) return rc;
    if (!ctx->scratch) return fail(ctx, ERNIE_ERROR, "fixed scratch unavailable on this device");
    const TextBlockWeights& w = ctx->text_blocks[index];
    // With at most 64 tokens every GEMM is one partial row of tiles, whose split-K
    // partials (at most 256 parts of 64 x 256 FP32) fit the 16 MiB split region, and the
    // attention has no query tile to split.
    if (S > ERNIE_NOALLOC_TEXT_TOKENS)
        return fail(ctx, ERNIE_ERROR, "no-allocation text block: at most " +
                                          std::to_string(ERNIE_NOALLOC_TEXT_TOKENS) + " tokens");
    const size_t act = text_activation_bytes(w, S), ones = ((size_t)w.hidden * 4 + 255) / 256 * 256;
    if (act + ones > kScratchBytes - kScratchSplitBytes)
        return fail(ctx, ERNIE_ERROR, "no-allocation text block: activations exceed the " +
                                          std::to_string((kScratchBytes - kScratchSplitBytes) >> 20) +
                                          " MiB scratch");
    char* base = static_cast<char*>(ctx->scratch);
    TextWs ws = text_ws_at(w, S, base + kScratchSplitBytes);
    float* ones_ptr = reinterpret_cast<float*>(base + kScratchSplitBytes + act);
    // The scratch keeps the previous call's contents: the unit gate is rewritten (by a
    // kernel, no memset node) every call; everything else is written before it is read.
    rc = kernel_status(ctx, fill_int(reinterpret_cast<int*>(ones_ptr), 0x3f800000, w.hidden, ctx->stream), "ones");
    if (rc) return rc;
    ws.ones = ones_ptr;
    ws.split_ws = base;
    ws.split_ws_bytes = kScratchSplitBytes;
    return text_block_run(ctx, w, x, out, cos_t, sin_t, mask, causal, S, ws);
}

int ernie_hip_text_block_sequence(ernie_hip_ctx* ctx, const int* blocks, int count, const float* x, float* out,
                                  const float* cos_t, const float* sin_t, const float* mask, int causal, int S,
                                  double* seconds)
{
    DeviceGuard guard(ctx);
    if (!ctx || !blocks) return ERNIE_ERROR;
    if (count < 1 || count > 25) return fail(ctx, ERNIE_ERROR, "Text path requires 1..25 blocks");
    for (int i = 0; i < count; ++i) {
        const int rc = check_text_call(ctx, blocks[i], S, x, out, cos_t, sin_t);
        if (rc) return rc;
        if (ctx->text_blocks[blocks[i]].hidden != ctx->text_blocks[blocks[0]].hidden)
            return fail(ctx, ERNIE_ERROR, "text blocks differ in width");
    }
    int rc = seconds ? sequence_events(ctx, count + 1) : ERNIE_OK;
    for (int i = 0; i < count && !rc; ++i) {
        if (seconds) (void)hipEventRecord(ctx->seq_events[i], ctx->stream);
        rc = text_block_forward(ctx, ctx->text_blocks[blocks[i]], i == 0 ? x : out, out, cos_t, sin_t, mask, causal,
                                S);
    }
    if (seconds && !rc) rc = sequence_seconds(ctx, count, seconds);
    return rc;
}

// ---- heads --------------------------------------------------------------------------------
int ernie_hip_heads_upload_tensors(ernie_hip_ctx* ctx, const ernie_heads_host_tensors* w, int dim, int latent_ch,
                                   int text_dim, int dtype, int parts)
{
    DeviceGuard guard(ctx);
    if (!ctx || !w) return ERNIE_ERROR;
    const int all = ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT;
    if (parts < 1 || parts > all) return fail(ctx, ERNIE_ERROR, "head parts must be ERNIE_HEAD_INPUT and/or _OUTPUT");
    const bool in = parts & ERNIE_HEAD_INPUT, out = parts & ERNIE_HEAD_OUTPUT;
    if (!valid_dtype(dtype) || dim < 128 || dim % 128 || latent_ch < 1 || (in && text_dim < 1))
        return fail(ctx, ERNIE_ERROR, "invalid head dimensions");
    if (latent_ch % 32 || (in && text_dim % 32)) return fail(ctx, ERNIE_ERROR, "head widths must be multiples of 32");
    HeadWeights& h = ctx->heads;
    const int kept = h.parts & ~parts;
    if (kept && (h.dim != dim || h.latent_ch != latent_ch || h.dtype != dtype))
        return fail(ctx, ERNIE_ERROR, std::string("the resident ") + (kept == ERNIE_HEAD_INPUT ? "input" : "output") +
                                          " head has another width, channel count or storage dtype");
    free_heads(h, parts);
    const size_t e = esize(dtype), D = dim;
    int rc = 0;
    auto mat = [&](DeviceBuffer& b, const ernie_host_tensor& t, size_t n, const char* what) {
        if (rc) return;
        if (!t.data) { rc = fail(ctx, ERNIE_ERROR, std::string("null ") + what); return; }
        rc = dev_alloc(ctx, b, n * e, what);
        if (!rc) rc = upload_tensor(ctx, b.ptr, 0, dtype, t.data, t.dtype, n, what);
    };
    auto vec = [&](DeviceBuffer& b, const ernie_host_tensor& t, size_t n, const char* what) {
        if (rc) return;
        if (!t.data) { rc = fail(ctx, ERNIE_ERROR, std::string("null ") + what); return; }
        rc = dev_alloc(ctx, b, n * 4, what);
        if (!rc) rc = upload_tensor(ctx, b.ptr, 0, ERNIE_DTYPE_FP32, t.data, t.dtype, n, what);
    };
    if (in) {
        mat(h.x_w, w->x_w, D * latent_ch, "x_w");
        vec(h.x_b, w->x_b, D, "x_b");
        mat(h.text_w, w->text_w, D * text_dim, "text_w");
        mat(h.t1_w, w->t1_w, D * D, "t1_w");
        vec(h.t1_b, w->t1_b, D, "t1_b");
        mat(h.t2_w, w->t2_w, D * D, "t2_w");
        vec(h.t2_b, w->t2_b, D, "t2_b");
        mat(h.mod_w, w->mod_w, 6 * D * D, "mod_w");
        vec(h.mod_b, w->mod_b, 6 * D, "mod_b");
    }
    if (out) {
        mat(h.out_mod_w, w->out_mod_w, 2 * D * D, "out_mod_w");
        vec(h.out_mod_b, w->out_mod_b, 2 * D, "out_mod_b");
        mat(h.proj_w, w->proj_w, (size_t)latent_ch * D, "proj_w");
        vec(h.proj_b, w->proj_b, latent_ch, "proj_b");
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "heads upload");
    if (rc) {
        free_heads(h, parts);
        return rc;
    }
    h.dim = dim;
    h.latent_ch = latent_ch;
    h.dtype = dtype;
    if (in) h.text_dim = text_dim;
    h.parts |= parts;
    return ERNIE_OK;
}

int ernie_hip_heads_upload(ernie_hip_ctx* ctx, const ernie_heads_host_weights* w, int dim, int latent_ch, int text_dim,
                           int dtype)
{
    if (!ctx || !w) return ERNIE_ERROR;
    const int F32 = ERNIE_DTYPE_FP32;
    const ernie_heads_host_tensors t = {{w->x_w, F32},     {w->x_b, F32},  {w->text_w, F32},   {w->t1_w, F32},
                                        {w->t1_b, F32},    {w->t2_w, F32}, {w->t2_b, F32},     {w->mod_w, F32},
                                        {w->mod_b, F32},   {w->out_mod_w, F32}, {w->out_mod_b, F32},
                                        {w->proj_w, F32},  {w->proj_b, F32}};
    return ernie_hip_heads_upload_tensors(ctx, &t, dim, latent_ch, text_dim, dtype,
                                          ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT);
}

int ernie_hip_heads_loaded(const ernie_hip_ctx* ctx) { return ctx ? ctx->heads.parts : 0; }

int ernie_hip_heads_init_random(ernie_hip_ctx* ctx, int dim, int latent_ch, int text_dim, int dtype, uint64_t seed,
                                float std_dev)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!valid_dtype(dtype) || dim < 128 || dim % 128 || latent_ch < 32 || latent_ch % 32 || text_dim < 32 ||
        text_dim % 32)
        return fail(ctx, ERNIE_ERROR, "invalid head dimensions");
    free_heads(ctx->heads);
    HeadWeights& h = ctx->heads;
    const size_t D = dim;
    struct Item { DeviceBuffer* b; bool matrix; size_t n; };
    const Item items[] = {{&h.x_w, true, D * latent_ch}, {&h.x_b, false, D}, {&h.text_w, true, D * text_dim},
                          {&h.t1_w, true, D * D}, {&h.t1_b, false, D}, {&h.t2_w, true, D * D}, {&h.t2_b, false, D},
                          {&h.mod_w, true, 6 * D * D}, {&h.mod_b, false, 6 * D}, {&h.out_mod_w, true, 2 * D * D},
                          {&h.out_mod_b, false, 2 * D}, {&h.proj_w, true, (size_t)latent_ch * D},
                          {&h.proj_b, false, (size_t)latent_ch}};
    int rc = 0;
    uint64_t k = 0;
    for (const Item& it : items) {
        const int dt = it.matrix ? dtype : ERNIE_DTYPE_FP32;
        rc = dev_alloc(ctx, *it.b, it.n * esize(dt), "heads");
        if (!rc) rc = kernel_status(ctx, fill_normal(it.b->ptr, dt, it.n, seed, (k++) << 40, 0.f, std_dev, ctx->stream), "heads init");
        if (rc) break;
    }
    if (!rc) rc = hip_status(ctx, hipStreamSynchronize(ctx->stream), "heads init");
    if (rc) {
        free_heads(h);
        return rc;
    }
    h.dim = dim; h.latent_ch = latent_ch; h.text_dim = text_dim; h.dtype = dtype;
    h.parts = ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT;
    return ERNIE_OK;
}

int ernie_hip_input_head(ernie_hip_ctx* ctx, const float* latent, int hw, const float* text, int text_tokens,
                         const float* time_features, float* x, float* c, float* mods)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!(ctx->heads.parts & ERNIE_HEAD_INPUT)) return fail(ctx, ERNIE_ERROR, "the input head is not loaded");
    if (!latent || !time_features || !x || !c || !mods || hw < 1 || text_tokens < 0 || (text_tokens && !text))
        return fail(ctx, ERNIE_ERROR, "invalid input head arguments");
    return input_head(ctx, latent, hw, text, text_tokens, time_features, x, c, mods);
}

int ernie_hip_output_head(ernie_hip_ctx* ctx, const float* x, int S, int hw, const float* c, float* prediction)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!(ctx->heads.parts & ERNIE_HEAD_OUTPUT)) return fail(ctx, ERNIE_ERROR, "the output head is not loaded");
    if (!x || !c || !prediction || hw < 1 || hw > S) return fail(ctx, ERNIE_ERROR, "invalid output head arguments");
    return output_head(ctx, x, hw, c, prediction);
}

int ernie_hip_dit_forward(ernie_hip_ctx* ctx, const float* latent, int hw, const float* text, int text_tokens,
                          const float* time_features, const float* cos_t, const float* sin_t, const float* mask,
                          int valid_keys, const int* blocks, int count, float* prediction)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (ctx->heads.parts != (ERNIE_HEAD_INPUT | ERNIE_HEAD_OUTPUT))
        return fail(ctx, ERNIE_ERROR, "the input and output heads are not both loaded");
    const int D = ctx->heads.dim, S = hw + text_tokens;
    if (!blocks || count < 1 || count > 36) return fail(ctx, ERNIE_ERROR, "Expected 1..36 blocks");
    for (int i = 0; i < count; ++i) {
        int rc = check_block_call(ctx, blocks[i], S, latent, prediction, prediction, cos_t, sin_t, valid_keys);
        if (rc) return rc;
        if (ctx->blocks[blocks[i]].dim != D) return fail(ctx, ERNIE_ERROR, "block and head widths differ");
    }
    // x [S][D], c [D], mods [6][D], all FP32, in a context-owned buffer.
    const size_t bytes = ((size_t)S * D + 7 * (size_t)D) * 4;
    int rc = dev_alloc(ctx, ctx->dit_act, bytes, "dit activations");
    if (rc) return rc;
    float* x = static_cast<float*>(ctx->dit_act.ptr);
    float* c = x + (size_t)S * D;
    float* mods = c + D;
    rc = input_head(ctx, latent, hw, text, text_tokens, time_features, x, c, mods);
    const float* cs = nullptr;
    if (!rc) rc = pack_rope(ctx, blocks, count, cos_t, sin_t, S, &cs);
    for (int i = 0; i < count && !rc; ++i)
        rc = block_forward(ctx, ctx->blocks[blocks[i]], x, x, mods, cos_t, sin_t, cs, mask, valid_keys, S);
    if (!rc) rc = output_head(ctx, x, hw, c, prediction);
    return rc;
}

// ---- profiling ------------------------------------------------------------------------------
int ernie_hip_profile_enable(ernie_hip_ctx* ctx, int enable)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    if (!enable) {
        int rc = collect(ctx);
        ctx->profiling = false;
        return rc;
    }
    ctx->profiling = true;
    return ERNIE_OK;
}

int ernie_hip_profile_classes(ernie_hip_ctx* ctx, unsigned class_mask)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    ctx->profile_mask = class_mask;
    return ERNIE_OK;
}

int ernie_hip_profile_stride(ernie_hip_ctx* ctx, int stride)
{
    DeviceGuard guard(ctx);
    if (!ctx || stride < 1) return ERNIE_ERROR;
    ctx->profile_stride = stride;
    for (long& n : ctx->class_seen) n = 0;
    return ERNIE_OK;
}

int ernie_hip_profile_collect(ernie_hip_ctx* ctx) { return ctx ? collect(ctx) : ERNIE_ERROR; }

int ernie_hip_profile_reset(ernie_hip_ctx* ctx)
{
    DeviceGuard guard(ctx);
    if (!ctx) return ERNIE_ERROR;
    int rc = collect(ctx);
    for (int i = 0; i < ERNIE_PROFILE_CLASSES; ++i) {
        ctx->launches[i] = 0;
        ctx->ms[i] = ctx->flop[i] = ctx->bytes[i] = 0;
    }
    return rc;
}

int ernie_hip_profile_query(const ernie_hip_ctx* ctx, int cls, long* launches, double* ms, double* flop, double* bytes)
{
    if (!ctx || cls < 0 || cls >= ERNIE_PROFILE_CLASSES) return ERNIE_ERROR;
    if (launches) *launches = ctx->launches[cls];
    if (ms) *ms = ctx->ms[cls];
    if (flop) *flop = ctx->flop[cls];
    if (bytes) *bytes = ctx->bytes[cls];
    return ERNIE_OK;
}

int ernie_hip_mfma_rate(ernie_hip_ctx* ctx, int iters, int launches, double* flop_per_s, double* clock_hz,
                        double* seconds)
{
    DeviceGuard guard(ctx);
    if (!ctx || iters < 1 || iters > (1 << 24) || launches < 1 || launches > 1000)
        return fail(ctx, ERNIE_ERROR, "mfma_rate: iters in [1, 2^24] and launches in [1, 1000]");
    int cus = 0, rtc_khz = 0;
    int rc = hip_status(ctx, hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device),
                        "mfma_rate: CU count");
    if (!rc)
        rc = hip_status(ctx, hipDeviceGetAttribute(&rtc_khz, hipDeviceAttributeWallClockRate, ctx->device),
                        "mfma_rate: constant counter rate");
    if (rc) return rc;
    if (cus < 1 || rtc_khz < 1) return fail(ctx, ERNIE_ERROR, "mfma_rate: device reports no CUs or counter rate");
    const size_t waves = mfma_rate_waves(cus);
    DeviceBuffer sink, stamps;
    rc = dev_alloc(ctx, sink, (size_t)cus * 512 * sizeof(float), "mfma_rate sink");
    if (!rc) rc = dev_alloc(ctx, stamps, waves * 4 * sizeof(unsigned long long), "mfma_rate stamps");
    hipEvent_t ev[2] = {nullptr, nullptr};
    if (!rc) rc = hip_status(ctx, hipEventCreate(&ev[0]), "mfma_rate event");
    if (!rc) rc = hip_status(ctx, hipEventCreate(&ev[1]), "mfma_rate event");
    auto* sk = static_cast<float*>(sink.ptr);
    auto* st = static_cast<unsigned long long*>(stamps.ptr);
    // One untimed launch first (clocks ramp, code object loaded).
    if (!rc) rc = kernel_status(ctx, launch_mfma_rate(cus, iters, sk, st, ctx->stream), "mfma_rate");
    if (!rc) rc = hip_status(ctx, hipEventRecord(ev[0], ctx->stream), "mfma_rate event");
    for (int i = 0; i < launches && !rc; ++i)
        rc = kernel_status(ctx, launch_mfma_rate(cus, iters, sk, st, ctx->stream), "mfma_rate");
    if (!rc) rc = hip_status(ctx, hipEventRecord(ev[1], ctx->stream), "mfma_rate event");
    if (!rc) rc = hip_status(ctx, hipEventSynchronize(ev[1]), "mfma_rate");
    float ms = 0.f;
    if (!rc) rc = hip_status(ctx, hipEventElapsedTime(&ms, ev[0], ev[1]), "mfma_rate elapsed");
    std::vector<unsigned long long> h(waves * 4);
    if (!rc)
        rc = hip_status(ctx, hipMemcpy(h.data(), st, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost),
                        "mfma_rate stamps");
    if (!rc) {
        // Median over the last launch's waves of shader cycles per constant-counter tick.
        std::vector<double> hz;
        hz.reserve(waves);
        for (size_t w = 0; w < waves; ++w) {
            const unsigned long long dc = h[4 * w + 1] - h[4 * w + 0], dr = h[4 * w + 3] - h[4 * w + 2];
            if (dr > 0) hz.push_back((double)dc / (double)dr * rtc_khz * 1e3);
        }
        if (hz.empty()) {
            rc = fail(ctx, ERNIE_ERROR, "mfma_rate: no wave recorded a time span");
        } else {
            std::nth_element(hz.begin(), hz.begin() + hz.size() / 2, hz.end());
            if (clock_hz) *clock_hz = hz[hz.size() / 2];
            const double s = ms * 1e-3;
            if (seconds) *seconds = s;
            if (flop_per_s) *flop_per_s = s > 0 ? mfma_rate_flop(cus, iters) * launches / s : 0.0;
        }
    }
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    dev_free(sink);
    dev_free(stamps);
    return rc;
}

}  // extern "C"
