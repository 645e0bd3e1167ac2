// aih_runtime.hip -- device, buffers, transfers, queue and timing of
// libaihost_hip.so.  This is the HIP device that replaces the reference's ROCm
// backend (AIHost/AIHost/ICompute/ROCm/*.cs) for the quantized-matmul path.
#include "aih_internal.h"
#include "aih_operand.h"

#include <cstring>
#include <cstdio>
#include <mutex>
#include <new>

namespace {

// Staging memory of aih_matmul_weights_q_noalloc: one copy per GPU, created
// with the code object.  Host code never uses this name as an address: each
// device's copy is looked up once (hipGetSymbolAddress, with that device
// current, in aih_init) and that pointer is passed to the kernels.
static __device__ __align__(256) unsigned char scratch[AIH_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (the current device).
int scratch_address(int device, void **out)
{
    if (device < 0 || device >= kMaxDevices) return AIH_E_LIMIT;
    std::lock_guard<std::mutex> g(g_scratch_lock);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        AIH_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return AIH_E_INVALID;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return AIH_OK;
}

int select_device(aih_ctx *ctx)
{
    int cur = -1;
    AIH_TRY(hipGetDevice(&cur));
    if (cur != ctx->device) AIH_TRY(hipSetDevice(ctx->device));
    return AIH_OK;
}

int release(aih_ctx *ctx)
{
    // Dispose never fails (ROCmComputeBuffer.cs:81-93): errors are ignored here.
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->allocs) (void)hipFree(kv.first);
    ctx->allocs.clear();
    ctx->tracked_bytes = 0;
    for (int i = 0; i < aih_ctx::kStageSlots; ++i) {
        if (ctx->stage_done[i]) (void)hipEventDestroy(ctx->stage_done[i]);
        if (ctx->stage[i]) (void)hipHostFree(ctx->stage[i]);
    }
    for (int i = 0; i < aih_ctx::kEvents; ++i)
        if (ctx->ev[i]) (void)hipEventDestroy(ctx->ev[i]);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->work2) (void)hipFree(ctx->work2);
    for (void *p : ctx->work_retired) (void)hipFree(p);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return AIH_OK;
}

}  // namespace

namespace {

int grow_workspace(aih_ctx *ctx, void *&work, size_t &work_bytes, size_t bytes, void **out)
{
    if (bytes <= work_bytes) {
        *out = work;
        return AIH_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    AIH_TRY(hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone) return AIH_E_LIMIT;
    // whole MiB, at least double the current size (the retired ones then
    // add up to less than the current one)
    size_t sz = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
    if (sz < 2 * work_bytes) sz = 2 * work_bytes;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return (int)e;
    }
    if (work) {
        // kept until aih_destroy (graphs captured earlier hold its address);
        // the list may allocate on the host: nothing may throw across the C ABI
        try {
            ctx->work_retired.push_back(work);
        } catch (...) {
            (void)hipFree(p);
            return (int)hipErrorOutOfMemory;
        }
    }
    work = p;
    work_bytes = sz;
    *out = work;
    return AIH_OK;
}

}  // namespace

int aih_workspace(aih_ctx *ctx, size_t bytes, void **out)
{
    return grow_workspace(ctx, ctx->work, ctx->work_bytes, bytes, out);
}

int aih_workspace2(aih_ctx *ctx, size_t bytes, void **out)
{
    return grow_workspace(ctx, ctx->work2, ctx->work2_bytes, bytes, out);
}

aih_copy_pool::~aih_copy_pool()
{
    {
        std::lock_guard<std::mutex> g(mu);
        stopping = true;
    }
    start_cv.notify_all();
    for (auto &t : workers) t.join();
}

// Part `part` of `parts` of the current job, on 4 KiB boundaries.
static void copy_part(char *dst, const char *src, size_t bytes, int part, int parts)
{
    const size_t per = ((bytes + parts - 1) / parts + 4095) & ~(size_t)4095;
    const size_t a = std::min(bytes, per * (size_t)part), b = std::min(bytes, a + per);
    if (b > a) std::memcpy(dst + a, src + a, b - a);
}

void aih_copy_pool::worker(int index)
{
    unsigned long long seen = 0;
    for (;;) {
        char *d;
        const char *s;
        size_t n;
        int parts;
        {
            std::unique_lock<std::mutex> g(mu);
            start_cv.wait(g, [&] { return stopping || generation != seen; });
            if (stopping) return;
            seen = generation;
            d = job_dst, s = job_src, n = job_bytes, parts = job_parts;
        }
        if (index + 1 < parts) copy_part(d, s, n, index + 1, parts);
        {
            std::lock_guard<std::mutex> g(mu);
            if (--pending == 0) done_cv.notify_one();
        }
    }
}

bool aih_copy_pool::copy(void *dst, const void *src, size_t bytes, int threads)
{
    try {
        while ((int)workers.size() < threads - 1) workers.emplace_back(&aih_copy_pool::worker, this,
                                                                      (int)workers.size());
    } catch (...) {
        if (workers.empty()) return false;
    }
    const int parts = (int)workers.size() + 1;
    {
        std::lock_guard<std::mutex> g(mu);
        job_dst = static_cast<char *>(dst);
        job_src = static_cast<const char *>(src);
        job_bytes = bytes;
        job_parts = parts;
        pending = (int)workers.size();
        ++generation;
    }
    start_cv.notify_all();
    copy_part(static_cast<char *>(dst), static_cast<const char *>(src), bytes, 0, parts);
    std::unique_lock<std::mutex> g(mu);
    done_cv.wait(g, [&] { return pending == 0; });
    return true;
}

int aih_stage(aih_ctx *ctx, const aih_scratch *ext, size_t bytes, void **out)
{
    if (!ext) return aih_workspace(ctx, bytes, out);
    if (bytes > ext->bytes || !ext->ptr) return AIH_E_SCRATCH;
    *out = ext->ptr;
    return AIH_OK;
}

extern "C" {

int aih_abi_version(void) { return AIH_ABI_VERSION; }

int aih_init(int device_index, aih_ctx **out)
{
    if (!out) return AIH_E_INVALID;
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) return AIH_E_NO_DEVICE;
    if (device_index < 0 || device_index >= count) return AIH_E_NO_DEVICE;
    hipDeviceProp_t prop;
    AIH_TRY(hipGetDeviceProperties(&prop, device_index));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return AIH_E_NOT_GFX950;
    AIH_TRY(hipSetDevice(device_index));

    aih_ctx *ctx = new (std::nothrow) aih_ctx();
    if (!ctx) return (int)hipErrorOutOfMemory;
    ctx->device = device_index;
    ctx->cu_count = prop.multiProcessorCount;
    const int src = scratch_address(device_index, &ctx->noalloc_scratch);
    if (src != AIH_OK) {
        delete ctx;
        return src;
    }
    hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    for (int i = 0; err == hipSuccess && i < aih_ctx::kStageSlots; ++i) {
        err = hipHostMalloc(&ctx->stage[i], aih_ctx::kStageBytes, hipHostMallocDefault);
        if (err == hipSuccess) err = hipEventCreateWithFlags(&ctx->stage_done[i], hipEventDisableTiming);
    }
    for (int i = 0; err == hipSuccess && i < aih_ctx::kEvents; ++i)
        err = hipEventCreate(&ctx->ev[i]);
    if (err != hipSuccess) {
        release(ctx);
        return (int)err;
    }
    *out = ctx;
    return AIH_OK;
}

int aih_destroy(aih_ctx *ctx)
{
    if (!ctx) return AIH_E_INVALID;
    (void)select_device(ctx);
    return release(ctx);
}

int aih_device_info_get(aih_ctx *ctx, aih_device_info *out)
{
    if (!ctx || !out) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    hipDeviceProp_t prop;
    AIH_TRY(hipGetDeviceProperties(&prop, ctx->device));
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    out->device_index = ctx->device;
    out->compute_units = prop.multiProcessorCount;
    out->wavefront_size = prop.warpSize;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width = prop.memoryBusWidth;
    size_t free_b = 0, total_b = 0;
    AIH_TRY(hipMemGetInfo(&free_b, &total_b));
    out->total_bytes = total_b;
    out->free_bytes = free_b;
    std::lock_guard<std::mutex> g(ctx->lock);
    out->tracked_bytes = ctx->tracked_bytes;
    out->tracked_buffers = (int64_t)ctx->allocs.size();
    return AIH_OK;
}

int aih_malloc(aih_ctx *ctx, size_t bytes, void **dptr)
{
    if (!ctx || !dptr) return AIH_E_INVALID;
    *dptr = nullptr;
    if (bytes == 0) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky error so later calls are unaffected
        return (int)e;
    }
    // the table insert may allocate on the host: nothing may throw across the C ABI
    try {
        std::lock_guard<std::mutex> g(ctx->lock);
        ctx->allocs[p] = bytes;
        ctx->tracked_bytes += bytes;
    } catch (...) {
        (void)hipFree(p);
        return (int)hipErrorOutOfMemory;
    }
    *dptr = p;
    return AIH_OK;
}

int aih_free(aih_ctx *ctx, void *dptr)
{
    if (!ctx || !dptr) return AIH_E_INVALID;
    size_t bytes = 0;
    {
        std::lock_guard<std::mutex> g(ctx->lock);
        auto it = ctx->allocs.find(dptr);
        if (it == ctx->allocs.end()) return AIH_E_NOT_ALLOCATED;
        bytes = it->second;
        ctx->allocs.erase(it);
        ctx->tracked_bytes -= bytes;
    }
    int rc = select_device(ctx);
    if (rc) return rc;
    // hipFree synchronises with outstanding work that may still read the buffer.
    AIH_TRY(hipFree(dptr));
    return AIH_OK;
}

int aih_memset(aih_ctx *ctx, void *dptr, int value, size_t bytes)
{
    if (!ctx || (!dptr && bytes)) return AIH_E_INVALID;
    if (!bytes) return AIH_OK;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipMemsetAsync(dptr, value, bytes, ctx->stream));
    return AIH_OK;
}

// Staging fills of at least this many bytes are split over kCopyThreads host
// threads.
constexpr size_t kParallelCopyBytes = 2u << 20;
constexpr int kCopyThreads = 4;

int aih_memcpy_h2d(aih_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    if (!ctx || ((!dst || !src) && bytes)) return AIH_E_INVALID;
    if (!bytes) return AIH_OK;
    int rc = select_device(ctx);
    if (rc) return rc;
    const char *s = static_cast<const char *>(src);
    char *d = static_cast<char *>(dst);
    size_t off = 0;
    int slot = 0;
    // Double-buffered: the CPU fills one pinned slot while the DMA engine
    // drains the other.
    while (off < bytes) {
        size_t len = bytes - off < aih_ctx::kStageBytes ? bytes - off : aih_ctx::kStageBytes;
        if (ctx->stage_pending[slot]) {
            AIH_TRY(hipEventSynchronize(ctx->stage_done[slot]));
            ctx->stage_pending[slot] = false;
        }
        // large fills are split over host threads; a pool that cannot start
        // leaves the copy to this thread
        bool done = false;
        if (len >= kParallelCopyBytes) {
            if (!ctx->copier) ctx->copier.reset(new (std::nothrow) aih_copy_pool());
            try {
                if (ctx->copier) done = ctx->copier->copy(ctx->stage[slot], s + off, len, kCopyThreads);
            } catch (...) {
                done = false;   // the same bytes are copied again below
            }
        }
        if (!done) std::memcpy(ctx->stage[slot], s + off, len);
        AIH_TRY(hipMemcpyAsync(d + off, ctx->stage[slot], len, hipMemcpyHostToDevice, ctx->stream));
        AIH_TRY(hipEventRecord(ctx->stage_done[slot], ctx->stream));
        ctx->stage_pending[slot] = true;
        off += len;
        slot ^= 1;
    }
    return AIH_OK;
}

int aih_upload_tensor(aih_ctx *ctx, void *dst, const void *host_src, size_t bytes)
{
    return aih_memcpy_h2d(ctx, dst, host_src, bytes);
}

int aih_memcpy_d2h(aih_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    if (!ctx || ((!dst || !src) && bytes)) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    if (bytes) AIH_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    AIH_TRY(hipStreamSynchronize(ctx->stream));
    return AIH_OK;
}

int aih_memcpy_d2d(aih_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    if (!ctx || ((!dst || !src) && bytes)) return AIH_E_INVALID;
    if (!bytes) return AIH_OK;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return AIH_OK;
}

int aih_sync(aih_ctx *ctx)
{
    if (!ctx) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipStreamSynchronize(ctx->stream));
    return AIH_OK;
}

void *aih_stream(aih_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

struct aih_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int aih_capture_begin(aih_ctx *ctx)
{
    if (!ctx) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return AIH_OK;
}

int aih_capture_end(aih_ctx *ctx, aih_graph **out)
{
    if (!ctx || !out) return AIH_E_INVALID;
    *out = nullptr;
    int rc = select_device(ctx);
    if (rc) return rc;
    hipGraph_t g = nullptr;
    AIH_TRY(hipStreamEndCapture(ctx->stream, &g));
    aih_graph *ag = new (std::nothrow) aih_graph();
    if (!ag) {
        (void)hipGraphDestroy(g);
        return (int)hipErrorOutOfMemory;
    }
    ag->graph = g;
    hipError_t e = hipGraphInstantiate(&ag->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete ag;
        return (int)e;
    }
    *out = ag;
    return AIH_OK;
}

int aih_graph_launch(aih_ctx *ctx, aih_graph *graph)
{
    if (!ctx || !graph) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipGraphLaunch(graph->exec, ctx->stream));
    return AIH_OK;
}

int aih_graph_destroy(aih_graph *graph)
{
    if (!graph) return AIH_E_INVALID;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
    return AIH_OK;
}

int aih_event_record(aih_ctx *ctx, int slot)
{
    if (!ctx || slot < 0 || slot >= aih_ctx::kEvents) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipEventRecord(ctx->ev[slot], ctx->stream));
    return AIH_OK;
}

int aih_event_elapsed(aih_ctx *ctx, int a, int b, float *ms)
{
    if (!ctx || !ms || a < 0 || b < 0 || a >= aih_ctx::kEvents || b >= aih_ctx::kEvents)
        return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    AIH_TRY(hipEventSynchronize(ctx->ev[b]));
    AIH_TRY(hipEventElapsedTime(ms, ctx->ev[a], ctx->ev[b]));
    return AIH_OK;
}

const char *aih_strerror(int status)
{
    switch (status) {
    case AIH_OK: return "success";
    case AIH_E_INVALID: return "invalid argument (null pointer, size or shape)";
    case AIH_E_UNSUPPORTED: return "ggml tensor type not supported on this path";
    case AIH_E_NOT_GFX950: return "device is not a gfx950 (MI355X) part";
    case AIH_E_NOT_ALLOCATED: return "pointer not allocated by this context (double free?)";
    case AIH_E_LIMIT: return "shape exceeds the kernel limits";
    case AIH_E_NO_DEVICE: return "no HIP device at that index";
    case AIH_E_SCRATCH:
        return "the operation needs more staging memory than the allocation-free entry point's static buffer "
               "(AIH_NOALLOC_SCRATCH_BYTES): use aih_matmul_weights_q, or fewer rows per call";
    default: break;
    }
    if (status > 0) return hipGetErrorString((hipError_t)status);
    return "unknown aihost_hip status";
}

// GGUFTensorType -> DataType as TransformerBase.MapType does
// (TransformerBase.cs:558-575); the DataType ordinals are the declaration
// order of IComputeBuffer.cs:57-75.
namespace {
struct TypePair { int ggml, dt; };
constexpr TypePair kTypeMap[] = {
    {0, AIH_DT_F32},   {1, AIH_DT_F16},   {2, AIH_DT_Q4_0},  {3, AIH_DT_Q4_1},  {6, AIH_DT_Q5_0},
    {7, AIH_DT_Q5_1},  {8, AIH_DT_Q8_0},  {9, AIH_DT_Q8_1},  {10, AIH_DT_Q2_K}, {11, AIH_DT_Q3_K},
    {12, AIH_DT_Q4_K}, {13, AIH_DT_Q5_K}, {14, AIH_DT_Q6_K}, {15, AIH_DT_Q8_K},
};
}  // namespace

int aih_datatype_from_type(int ggml_type)
{
    for (const TypePair &p : kTypeMap)
        if (p.ggml == ggml_type) return p.dt;
    return AIH_E_UNSUPPORTED;
}

int aih_type_from_datatype(int datatype)
{
    for (const TypePair &p : kTypeMap)
        if (p.dt == datatype) return p.ggml;
    return AIH_E_UNSUPPORTED;
}

int64_t aih_row_bytes(int type, int64_t k)
{
    aih_block_geom g = aih_geom(type);
    if (g.elems == 0) return AIH_E_UNSUPPORTED;
    if (k < 0 || k % g.elems) return AIH_E_INVALID;
    return (k / g.elems) * g.bytes;
}

int aih_dequantize(aih_ctx *ctx, int type, const void *q, float *out,
                   uint64_t n_elems, int f16_mode)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    if (f16_mode != AIH_F16_IEEE && f16_mode != AIH_F16_REFCPU) return AIH_E_INVALID;
    aih_block_geom g = aih_geom(type);
    if (n_elems % (uint64_t)g.elems) return AIH_E_INVALID;
    if (!n_elems) return AIH_OK;
    if (!q || !out) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    return aih_launch_dequant(ctx, type, q, out, n_elems / (uint64_t)g.elems, f16_mode);
}

int aih_qmatvec_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                      const float *X2, float eps, int pre, int post, float *Y)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    aih_block_geom g = aih_geom(type);
    if (N < 0 || K <= 0 || K % g.elems) return AIH_E_INVALID;
    if (pre < AIH_PRE_NONE || pre > AIH_PRE_SILU_MUL) return AIH_E_INVALID;
    if (post < AIH_POST_STORE || post > AIH_POST_SILU_PAIRS) return AIH_E_INVALID;
    if (post == AIH_POST_SILU_PAIRS && N % 2) return AIH_E_INVALID;
    if (pre != AIH_PRE_NONE && !X2) return AIH_E_INVALID;
    if (!N) return AIH_OK;
    if (!W || !X || !Y) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    return aih_launch_qmatvec_fused(ctx, type, W, N, K, X, X2, eps, pre, post, Y);
}

}  // extern "C"

namespace {

int qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X, int64_t ldx, float *Y,
            int64_t ldy, int batch, const aih_scratch *ext)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    aih_block_geom g = aih_geom(type);
    if (N < 0 || K <= 0 || K % g.elems || batch < 1 || batch > 8) return AIH_E_INVALID;
    if (ldx < K || ldy < N) return AIH_E_INVALID;
    if (!N) return AIH_OK;
    if (!W || !X || !Y) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    return aih_launch_qmatvec(ctx, type, W, N, K, X, ldx, Y, ldy, batch, ext);
}

int qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X, int64_t M, float *Y,
          const aih_scratch *ext, bool may_split)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    aih_block_geom g = aih_geom(type);
    if (N < 0 || M < 0 || K <= 0 || K % g.elems) return AIH_E_INVALID;
    if (!N || !M) return AIH_OK;
    if (!W || !X || !Y) return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    return aih_launch_qgemm(ctx, type, W, N, K, X, M, Y, ext, may_split);
}

int matmul_weights_q(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X, int64_t M,
                     float *Y, const aih_scratch *ext)
{
    if (M >= 1 && M <= 8) return qmatvec(ctx, type, W, N, K, X, K, Y, N, (int)M, ext);
    // never split over K: the allocation-free variant, which shares this
    // path, has no room for partial sums, and both return the same bits
    return qgemm(ctx, type, W, N, K, X, M, Y, ext, false);
}

}  // namespace

extern "C" {

int aih_qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    return qmatvec(ctx, type, W, N, K, X, ldx, Y, ldy, batch, nullptr);
}

int aih_qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
              const float *X, int64_t M, float *Y)
{
    return qgemm(ctx, type, W, N, K, X, M, Y, nullptr, true);
}

int aih_matmul_weights_q(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                         const float *X, int64_t M, float *Y)
{
    return matmul_weights_q(ctx, type, W, N, K, X, M, Y, nullptr);
}

int aih_qgemm_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                    const float *X2, float eps, int64_t M, int pre, int post, float *Y)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    aih_block_geom g = aih_geom(type);
    if (N < 0 || M < 0 || K <= 0 || K % g.elems) return AIH_E_INVALID;
    if (pre < AIH_PRE_NONE || pre > AIH_PRE_F16_OPERAND) return AIH_E_INVALID;
    if (post != AIH_POST_STORE && post != AIH_POST_ACCUMULATE && post != AIH_POST_SILU_PAIRS_F16)
        return AIH_E_INVALID;
    if (post == AIH_POST_SILU_PAIRS_F16 && N % 128) return AIH_E_INVALID;
    const bool uses_x2 = pre == AIH_PRE_RMSNORM || pre == AIH_PRE_SILU_MUL;
    if (uses_x2 && !X2) return AIH_E_INVALID;
    if (!N || !M) return AIH_OK;
    if (!W || !X || !Y) return AIH_E_INVALID;
    if (K % 64 != 0) return AIH_E_LIMIT;
    if (reinterpret_cast<uintptr_t>(X) % 16 || (uses_x2 && reinterpret_cast<uintptr_t>(X2) % 16) ||
        (post == AIH_POST_SILU_PAIRS_F16 && reinterpret_cast<uintptr_t>(Y) % 16))
        return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int epi = post == AIH_POST_ACCUMULATE ? 1 : post == AIH_POST_SILU_PAIRS_F16 ? 2 : 0;
    if (pre == AIH_PRE_F16_OPERAND) {
        // an image written in 32-column blocks: one exponent per row first
        void *img = const_cast<float *>(X);
        rc = aih_launch_operand_fixup(ctx, img, M, K);
        if (rc) return rc;
        return aih_launch_qgemm_tiled(ctx, type, W, N, K, img, M, Y, epi, true);
    }
    void *work = nullptr;
    rc = aih_stage(ctx, nullptr, (size_t)aih_operand::image_bytes(aih_operand::mpad_of(M), K, false), &work);
    if (rc) return rc;
    rc = pre == AIH_PRE_NONE ? aih_launch_x_tile(ctx, X, M, K, work)
                             : aih_launch_x_tile_pre(ctx, pre, X, X2, eps, M, K, work);
    if (rc) return rc;
    return aih_launch_qgemm_tiled(ctx, type, W, N, K, work, M, Y, epi, true);
}

int aih_qgemm_qkv_rope(aih_ctx *ctx, int type, const void *W, int64_t K, const float *X, const float *X2, float eps,
                       int64_t M, int pre, float *Q, float *Kc, float *Vc, int32_t n_heads, int32_t n_kv_heads,
                       int32_t head_dim, int32_t start, const int32_t *pos, const float *table, int32_t table_rows,
                       int64_t cache_rows)
{
    if (!ctx) return AIH_E_INVALID;
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    aih_block_geom g = aih_geom(type);
    if (M < 0 || K <= 0 || K % g.elems) return AIH_E_INVALID;
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2) return AIH_E_INVALID;
    if (pre != AIH_PRE_NONE && pre != AIH_PRE_RMSNORM) return AIH_E_INVALID;
    if (pre == AIH_PRE_RMSNORM && !X2) return AIH_E_INVALID;
    // a 32-column block of the product is all queries, all keys or all values
    if (head_dim % 32) return AIH_E_UNSUPPORTED;
    const int64_t qd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_kv_heads * head_dim;
    if (qd + 2 * kvd > 0x7FFFFFFF) return AIH_E_LIMIT;
    if (!M) return AIH_OK;
    if (!W || !X || !Q || !Kc || !Vc || !table) return AIH_E_INVALID;
    if (!pos && (start < 0 || start + M > table_rows || start + M > cache_rows)) return AIH_E_LIMIT;
    if (K % 64 != 0) return AIH_E_LIMIT;
    if (reinterpret_cast<uintptr_t>(X) % 16 || (X2 && reinterpret_cast<uintptr_t>(X2) % 16) ||
        reinterpret_cast<uintptr_t>(table) % 8)
        return AIH_E_INVALID;
    int rc = select_device(ctx);
    if (rc) return rc;
    void *work = nullptr;
    rc = aih_stage(ctx, nullptr, (size_t)aih_operand::image_bytes(aih_operand::mpad_of(M), K, false), &work);
    if (rc) return rc;
    rc = pre == AIH_PRE_NONE ? aih_launch_x_tile(ctx, X, M, K, work)
                             : aih_launch_x_tile_pre(ctx, pre, X, X2, eps, M, K, work);
    if (rc) return rc;
    aih_rope_qkv_args ra;
    ra.Kc = Kc;
    ra.Vc = Vc;
    ra.table = table;
    ra.pos = pos;
    ra.cache_rows = cache_rows;
    ra.start = start;
    ra.qd = (int32_t)qd;
    ra.kvd = (int32_t)kvd;
    ra.head_dim = head_dim;
    ra.table_rows = table_rows;
    return aih_launch_qgemm_tiled(ctx, type, W, qd + 2 * kvd, K, work, M, Q, 3, false, &ra);
}

int64_t aih_operand_bytes(int64_t M, int64_t K)
{
    if (M < 0 || K <= 0 || K % 64) return AIH_E_INVALID;
    const int64_t mpad = aih_operand::mpad_of(M);
    if (mpad > (INT64_MAX / 4) / (K + 2)) return AIH_E_LIMIT;
    return aih_operand::image_bytes(mpad, K, true);
}

int aih_matmul_weights_q_noalloc(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                                 const float *X, int64_t M, float *Y)
{
    if (!ctx) return AIH_E_INVALID;
    // the device address of this GPU's static buffer, looked up in aih_init
    const aih_scratch ext = {ctx->noalloc_scratch, AIH_NOALLOC_SCRATCH_BYTES};
    return matmul_weights_q(ctx, type, W, N, K, X, M, Y, &ext);
}

}  // extern "C"
