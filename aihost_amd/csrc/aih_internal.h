// aih_internal.h -- shared definitions of libaihost_hip.so (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

// Host threads that split a large host memcpy (the fill of a pinned staging
// slot) into parts, so that the copy into pinned memory keeps up with the DMA
// engine.  Workers start on first use and stop when the pool is destroyed.
class aih_copy_pool {
public:
    ~aih_copy_pool();
    // memcpy(dst, src, bytes) by up to `threads` threads (this one included);
    // false when no worker could be started (the caller then copies alone).
    bool copy(void *dst, const void *src, size_t bytes, int threads);

private:
    void worker(int index);
    std::mutex mu;
    std::condition_variable start_cv, done_cv;
    std::vector<std::thread> workers;
    char *job_dst = nullptr;
    const char *job_src = nullptr;
    size_t job_bytes = 0;
    int job_parts = 0;
    unsigned long long generation = 0;
    int pending = 0;
    bool stopping = false;
};

#include "../../include/aihost_hip.h"

// GGUF block geometry (AIHost/AIHost/GGUF/GGUFTensorInfo.cs:60-71,
// AIHost/AIHost/Compute/QuantizationFormats.cs:6-12).
struct aih_block_geom { int elems; int bytes; };

static inline aih_block_geom aih_geom(int type)
{
    switch (type) {
    case AIH_TYPE_Q8_0: return {32, 34};
    case AIH_TYPE_Q4_0: return {32, 18};
    case AIH_TYPE_Q4_K: return {256, 144};
    case AIH_TYPE_Q6_K: return {256, 210};
    case AIH_TYPE_F32:  return {1, 4};
    default:            return {0, 0};
    }
}

static inline bool aih_is_quant(int type)
{
    return type == AIH_TYPE_Q8_0 || type == AIH_TYPE_Q4_0 ||
           type == AIH_TYPE_Q4_K || type == AIH_TYPE_Q6_K;
}

// One device + one in-order stream + a pinned staging ring for uploads.
struct aih_ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    static constexpr int kStageSlots = 2;
    static constexpr size_t kStageBytes = 16u << 20;   // 16 MiB per slot
    void *stage[kStageSlots] = {nullptr, nullptr};
    hipEvent_t stage_done[kStageSlots] = {nullptr, nullptr};
    bool stage_pending[kStageSlots] = {false, false};
    static constexpr int kEvents = 16;
    hipEvent_t ev[kEvents] = {};
    std::mutex lock;                                    // guards `allocs`
    std::unordered_map<void *, size_t> allocs;
    size_t tracked_bytes = 0;
    int cu_count = 0;
    // Grow-only device workspace for kernels that stage data (the GEMM's fp16
    // copy of X, the small-batch matvec's partial sums).  Not counted in
    // tracked_bytes.  A smaller one that a larger replaced stays allocated
    // (graphs captured earlier still point at it); all are freed by aih_destroy.
    void *work = nullptr;
    size_t work_bytes = 0;
    // A second one, for the partial sums of a GEMM split over K (its operand
    // may sit in the first).
    void *work2 = nullptr;
    size_t work2_bytes = 0;
    std::vector<void *> work_retired;
    // Device address of this GPU's static staging buffer (the allocation-free
    // entry point's), set by aih_init.
    void *noalloc_scratch = nullptr;
    // Host threads for filling the staging slots (aih_memcpy_h2d).
    std::unique_ptr<aih_copy_pool> copier;
};

// Device workspace of at least `bytes` on the context's device.  Growing it
// allocates, which is refused while the stream is being captured into a graph
// (AIH_E_LIMIT): run the operation once outside the capture first.  Returns
// AIH_OK or a status.
int aih_workspace(aih_ctx *ctx, size_t bytes, void **out);
// The second workspace (split-K partial sums), same rules.
int aih_workspace2(aih_ctx *ctx, size_t bytes, void **out);

// Staging memory a caller supplies in place of the context workspace (the
// allocation-free entry point passes its static device buffer).
struct aih_scratch {
    void *ptr;
    size_t bytes;
};

// Staging memory of at least `bytes`: `ext` when given (AIH_E_SCRATCH when it
// is smaller; nothing is allocated), else the context workspace.
int aih_stage(aih_ctx *ctx, const aih_scratch *ext, size_t bytes, void **out);

#define AIH_TRY(expr)                                  \
    do {                                               \
        hipError_t aih_e_ = (expr);                    \
        if (aih_e_ != hipSuccess) return (int)aih_e_;  \
    } while (0)

// Status of the most recent launch on this thread.
static inline int aih_launch_status()
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? AIH_OK : (int)e;
}

// Kernel launch entry points implemented per source file.
int aih_launch_dequant(aih_ctx *ctx, int type, const void *q, float *out,
                       uint64_t n_blocks, int f16_mode);
// `ext`: staging memory to use instead of the context workspace (may be null).
int aih_launch_qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                       const float *X, int64_t ldx, float *Y, int64_t ldy, int batch,
                       const aih_scratch *ext = nullptr);
int aih_launch_qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                     const float *X, int64_t M, float *Y, const aih_scratch *ext = nullptr,
                     bool may_split = false);
// The prefill GEMM in parts: X (M x K fp32) -> the fp16 fragment-order
// operand image Xt with its row exponents (aih_operand.h; mpad = M rounded up
// to 32); the same operand computed by a fused element-wise step
// (AIH_PRE_RMSNORM / SILU_MUL / SILU_PAIRS, aih_decoder.hip); the pass that
// gives every row of an image written in 32-column blocks one exponent; the
// GEMM from Xt with epilogue `epi`: 0 stores Y, 1 adds into Y, 2 writes SiLU
// of its gate/up column pairs into Y as the fp16 operand image of a GEMM over
// N/2 columns.
int aih_launch_x_tile(aih_ctx *ctx, const float *X, int64_t M, int64_t K, void *Xt);
int aih_launch_x_tile_pre(aih_ctx *ctx, int pre, const float *X, const float *X2, float eps, int64_t M, int64_t K,
                          void *Xt);
int aih_launch_operand_fixup(aih_ctx *ctx, void *Xt, int64_t M, int64_t K);
// The Q|K|V epilogue (epi 3): for output columns [0, qd) the rotated queries
// into Y, for [qd, qd + kvd) the rotated keys and for [qd + kvd, qd + 2 kvd)
// the values into the caches at row p = start (+ *pos) + m, with the
// arithmetic and the row conditions of aih_rope_qkv.
struct aih_rope_qkv_args {
    float *Kc = nullptr, *Vc = nullptr;
    const float *table = nullptr;
    const int32_t *pos = nullptr;
    int64_t cache_rows = 0;
    int32_t start = 0, qd = 0, kvd = 0, head_dim = 0, table_rows = 0;
};

// may_split: the GEMM may split K over workgroups, with partial sums in the
// second workspace and a reduction (never with caller-provided staging).
// rope: the epilogue's arguments for epi 3 (else unused).
int aih_launch_qgemm_tiled(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const void *Xt,
                           int64_t M, float *Y, int epi, bool may_split = false,
                           const aih_rope_qkv_args *rope = nullptr);
int aih_launch_qmatvec_mfma(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                            const float *X, int64_t ldx, float *Y, int64_t ldy, int batch,
                            const aih_scratch *ext = nullptr);
int aih_launch_qmatvec_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                             const float *X2, float eps, int pre, int post, float *Y);
int aih_launch_embed(aih_ctx *ctx, int type, const void *table, int64_t vocab, int64_t dim,
                     const int32_t *ids, int64_t n, float *out);
