/*
 * aihost_hip.h -- C ABI of libaihost_hip.so, the gfx950 (MI355X) backend for
 * AIHost's GGUF block-quantized matrix-product path.
 *
 * The library replaces, for this path, the reference's ROCm compute device and
 * the two-pass "dequantize into an F32 scratch, then F32 SIMT matmul" sequence
 * with fused HIP kernels compiled offline for gfx950.  Paths below are relative
 * to the reference repository (Timka654/AIHost).
 *
 * Conventions (all entry points):
 *   - return int status: AIH_OK (0); > 0 is a hipError_t value; < 0 is one of
 *     the AIH_E_* codes.  Nothing throws or aborts.
 *     (Replaces HipApi.CheckError, AIHost/AIHost/ICompute/ROCm/HipApi.cs:43-47,
 *     which throws InvalidOperationException on the managed side.)
 *   - one aih_ctx = one device + one in-order HIP stream.  A context is not
 *     thread-safe; callers serialise, as InferenceEngine._gpuLock does today
 *     (AIHost/AIHost/Inference/InferenceEngine.cs:70,251).
 *   - device pointers are plain `void*` from aih_malloc.  Pointers passed in
 *     stay owned by the caller; the library keeps no reference after a call.
 *   - everything except aih_memcpy_d2h, aih_sync, aih_event_elapsed and the
 *     aih_host_* utilities is asynchronous on the context stream.
 *   - ggml type ids are GGUFTensorType values
 *     (AIHost/AIHost/GGUF/GGUFValueType.cs:26-56).
 *   - weights are GGUF tensors with dims [ne0 = K, ne1 = N]: row n is K/QK
 *     consecutive packed blocks, exactly the on-disk byte order.
 */
#ifndef AIHOST_HIP_H
#define AIHOST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIH_ABI_VERSION 1

/* ---- status codes ------------------------------------------------------ */
#define AIH_OK               0
#define AIH_E_INVALID       -1  /* null pointer, bad size or shape            */
#define AIH_E_UNSUPPORTED   -2  /* ggml type not handled by this path         */
#define AIH_E_NOT_GFX950    -3  /* device is not a gfx950 part                */
#define AIH_E_NOT_ALLOCATED -4  /* pointer not owned by this context (double free) */
#define AIH_E_LIMIT         -5  /* shape beyond what the kernels support      */
#define AIH_E_NO_DEVICE     -6  /* no HIP device at that index                */
#define AIH_E_SCRATCH       -7  /* needs more staging memory than the static
                                   buffer of aih_matmul_weights_q_noalloc  */

/* ---- ggml tensor types handled on this path ---------------------------- */
/* The operators take GGUFTensorType / ggml ids (GGUFValueType.cs:26-56), the
 * numbering of the file's tensor infos. */
#define AIH_TYPE_F32   0
#define AIH_TYPE_Q4_0  2
#define AIH_TYPE_Q8_0  8
#define AIH_TYPE_Q4_K 12
#define AIH_TYPE_Q6_K 14

/* ---- the reference's operator-level type: DataType --------------------- */
/* A reference Tensor carries DataType (Tensor.cs:12), whose ordinals
 * (AIHost/AIHost/ICompute/IComputeBuffer.cs:57-75) are NOT the ggml ids:
 * DataType.Q8_0 = 6, Q4_K = 10, Q6_K = 12 while the ggml ids 8, 10, 12 are
 * Q8_0, Q2_K, Q4_K.  Translate with aih_type_from_datatype before calling an
 * operator; passing a DataType ordinal as a type would read Q6_K blocks as
 * Q4_K. */
#define AIH_DT_F32   0
#define AIH_DT_F16   1
#define AIH_DT_Q4_0  2
#define AIH_DT_Q4_1  3
#define AIH_DT_Q5_0  4
#define AIH_DT_Q5_1  5
#define AIH_DT_Q8_0  6
#define AIH_DT_Q8_1  7
#define AIH_DT_Q2_K  8
#define AIH_DT_Q3_K  9
#define AIH_DT_Q4_K 10
#define AIH_DT_Q5_K 11
#define AIH_DT_Q6_K 12
#define AIH_DT_Q8_K 13
#define AIH_DT_I8   14
#define AIH_DT_I16  15
#define AIH_DT_I32  16

/* ---- fp16 scale decoding modes for aih_dequantize ---------------------- */
/* IEEE: the reference's GPU decoder, QuantizationFormats.cs:147-152
 *       (-0 decodes to +0, every NaN to 0x7FC00000).
 * REFCPU: the reference's CPU decoder ComputeOps.F16ToF32,
 *       AIHost/AIHost/Compute/ComputeOps.cs:1497-1522, bit for bit, including
 *       its wrong exponent for fp16 subnormals. */
#define AIH_F16_IEEE   0
#define AIH_F16_REFCPU 1

typedef struct aih_ctx aih_ctx;

typedef struct aih_device_info {
    char     name[256];
    char     arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t  device_index;
    int32_t  compute_units;
    int32_t  wavefront_size;
    int32_t  clock_khz;
    int32_t  memory_clock_khz;
    int32_t  memory_bus_width;
    uint64_t total_bytes;       /* HBM capacity                               */
    uint64_t free_bytes;        /* hipMemGetInfo at the time of the call      */
    uint64_t tracked_bytes;     /* bytes currently held through aih_malloc    */
    int64_t  tracked_buffers;   /* live aih_malloc allocations                */
} aih_device_info;

/* ---- device / context (IComputeDevice, AIHost/AIHost/ICompute/IComputeDevice.cs:27-72) */

/* Open device `device_index`, create its stream and the pinned staging ring.
 * Fails with AIH_E_NOT_GFX950 on any other architecture.
 * Replaces ROCmComputeDevice's constructor (AIHost/AIHost/ICompute/ROCm/ROCmComputeDevice.cs:15-50). */
int aih_init(int device_index, aih_ctx **out);

/* Free every allocation still owned by the context, then the context.
 * Replaces ROCmComputeDevice.Dispose. Never fails on a valid context. */
int aih_destroy(aih_ctx *ctx);

/* Fixed-size device description; replaces the truncated HipDeviceProp
 * marshalling (HipApi.cs:71-99) and IComputeDevice.GetMemoryInfo (IComputeDevice.cs:71). */
int aih_device_info_get(aih_ctx *ctx, aih_device_info *out);

/* ---- buffers (IComputeBuffer, AIHost/AIHost/ICompute/IComputeBuffer.cs:6-42) */

/* Device allocation.  Out of memory returns hipErrorOutOfMemory (2), which the
 * managed side maps to InsufficientVramException
 * (AIHost/AIHost/ICompute/InsufficientVramException.cs:10-29).
 * Replaces IComputeDevice.CreateBuffer (IComputeDevice.cs:46) /
 * ROCmComputeBuffer's constructor (ROCmComputeBuffer.cs:15-24). */
int aih_malloc(aih_ctx *ctx, size_t bytes, void **dptr);

/* Free an aih_malloc pointer; AIH_E_NOT_ALLOCATED for anything else, including
 * a second free.  Replaces ROCmComputeBuffer.Dispose (ROCmComputeBuffer.cs:81-93). */
int aih_free(aih_ctx *ctx, void *dptr);

/* Asynchronous byte fill. */
int aih_memset(aih_ctx *ctx, void *dptr, int value, size_t bytes);

/* Host -> device through the pinned double-buffered staging ring; returns as
 * soon as `src` may be reused.  Replaces IComputeBuffer.Write /
 * IComputeCommandQueue.WriteBuffer (IComputeCommandQueue.cs:11). */
int aih_memcpy_h2d(aih_ctx *ctx, void *dst, const void *src, size_t bytes);

/* Device -> host, synchronous (waits for prior work on the stream).
 * Replaces IComputeBuffer.Read / ReadRange (IComputeBuffer.cs:26-41). */
int aih_memcpy_d2h(aih_ctx *ctx, void *dst, const void *src, size_t bytes);

/* Device -> device, asynchronous. */
int aih_memcpy_d2d(aih_ctx *ctx, void *dst, const void *src, size_t bytes);

/* Upload one GGUF tensor's packed blocks verbatim (on-disk layout) from host
 * memory (typically an mmap view of the file).  Same transfer as
 * aih_memcpy_h2d; named separately because it replaces the host memcpy into
 * a device pointer in LazyGGUFModel.LoadTensor
 * (AIHost/AIHost/GGUF/LazyGGUFModel.cs:140-177) and GGUFModel.LoadTensor
 * (AIHost/AIHost/GGUF/GGUFModel.cs:30-63). */
int aih_upload_tensor(aih_ctx *ctx, void *dst, const void *host_src, size_t bytes);

/* ---- operators (ComputeOps, AIHost/AIHost/Compute/ComputeOps.cs) ------- */

/* TransformerBase.MapType (AIHost/AIHost/Compute/TransformerBase.cs:558-575):
 * the DataType ordinal of a GGUF tensor type, for the fourteen types MapType
 * maps (F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K .. Q8_K);
 * AIH_E_UNSUPPORTED for any other value (where MapType throws
 * NotSupportedException).  Needs no context and no device. */
int aih_datatype_from_type(int ggml_type);

/* The inverse: the ggml id that the operators take for a reference DataType
 * ordinal; AIH_E_UNSUPPORTED for I8/I16/I32 and out-of-range values.  The
 * operators themselves then reject the types this path does not compute on.
 * Needs no context and no device. */
int aih_type_from_datatype(int datatype);

/* Bytes of one row of k elements of `type`, or a negative status.
 * (GGUFTensorInfo.SizeInBytes, AIHost/AIHost/GGUF/GGUFTensorInfo.cs:51-78.) */
int64_t aih_row_bytes(int type, int64_t k);

/* out[0..n_elems) = dequantized blocks of `q` (n_elems a whole number of
 * blocks), bit-exact to the reference decoders for f16_mode.
 * Replaces ComputeOps.Dequantize / DequantizeInto (ComputeOps.cs:733-745,
 * 761-861) and their shaders (QuantizationFormats.cs:140-196, 269-321);
 * adds Q8_0 and Q4_0, which the reference rejects (ComputeOps.cs:743,774). */
int aih_dequantize(aih_ctx *ctx, int type, const void *q, float *out,
                   uint64_t n_elems, int f16_mode);

/* Decode matvec, dequantization fused:
 *   Y[b*ldy + n] = sum_k X[b*ldx + k] * W[n, k],   b < batch (1..8), n < N.
 * K must be a multiple of 64 (a whole number of blocks; the kernels read
 * 64-element units) and at most 65536, else AIH_E_LIMIT.  fp32
 * accumulation.  For batch 3..8, K
 * is split over workgroups and the partial sums (splits x batch x N floats)
 * go through the context workspace (see aih_qgemm); a call captured into a
 * graph before the workspace is large enough runs with one split instead.
 * Replaces TempF32 + ComputeOps.MatMulWeights for M = batch <= 8
 * (TransformerBase.cs:254-271, ComputeOps.cs:275-309, ComputeShaders.cs:93-129). */
int aih_qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                const float *X, int64_t ldx, float *Y, int64_t ldy, int batch);

/* Decode matvec (one column) with the neighbouring element-wise steps of a
 * Llama layer fused in, so that a decode step needs no separate kernels for
 * them.  y[n] = sum_k x[k] W[n, k] with
 *   pre = AIH_PRE_NONE       x = X
 *   pre = AIH_PRE_RMSNORM    x = (X / sqrt(mean(X^2) + eps)) * X2   (X2: norm weights)
 *   pre = AIH_PRE_SILU_MUL   x = SiLU(X) * X2                        (X2: the up projection)
 * and
 *   post = AIH_POST_STORE       Y[n] = y[n]
 *   post = AIH_POST_ACCUMULATE  Y[n] += y[n]                 (the residual add)
 *   post = AIH_POST_SILU_PAIRS  Y[i] = SiLU(y[2i]) * y[2i+1], i < N/2 (W holds
 *                               gate and up rows interleaved; K <= 16384)
 * with the formulas of aih_rmsnorm, aih_silu_mul and aih_add.  X, X2 16-byte
 * aligned; Y must not alias X or X2.  Replaces, for a decode step, the
 * LayerNorm / SiLU+Multiply / Add around MatMulWeights in
 * ComputeOps.TransformerLayer (ComputeOps.cs:1250-1356) and FeedForward
 * (ComputeOps.cs:1218-1241). */
#define AIH_PRE_NONE        0
#define AIH_PRE_RMSNORM     1
#define AIH_PRE_SILU_MUL    2
#define AIH_POST_STORE      0
#define AIH_POST_ACCUMULATE 1
#define AIH_POST_SILU_PAIRS 2
/* aih_qgemm_fused only:  x[k] = SiLU(X[2k]) * X[2k+1]  (X rows of 2K floats:
 * the output of a GEMM over gate/up rows interleaved; X2 unused). */
#define AIH_PRE_SILU_PAIRS  3
/* aih_qgemm_fused only: X is a GEMM operand image of M rows and K columns
 * (aih_operand_bytes(M, K) bytes), as AIH_POST_SILU_PAIRS_F16 or
 * aih_attention_operand writes it (X2 unused).  The call first gives every
 * row of the image one power-of-two exponent, rewriting it in place; the
 * values it holds do not change. */
#define AIH_PRE_F16_OPERAND 4
/* aih_qgemm_fused only: SiLU(y[m, 2i]) * y[m, 2i+1] (W holds gate and up rows
 * interleaved, N a multiple of 128), stored in Y as the operand image of a
 * GEMM over those N/2 columns (aih_operand_bytes(M, N/2) bytes), for a
 * following aih_qgemm_fused with pre = AIH_PRE_F16_OPERAND and K = N/2. */
#define AIH_POST_SILU_PAIRS_F16 3
int aih_qmatvec_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                      const float *X2, float eps, int pre, int post, float *Y);

/* Prefill GEMM, dequantization fused:  Y[m*N + n] = sum_k X[m*K + k] * W[n, k].
 * X is converted once to fp16 in a context workspace (about M*K*2 bytes,
 * grown on demand and kept until aih_destroy), each row scaled by a power of
 * two that keeps its largest value within fp16's range (rows whose largest
 * magnitude lies in [2^-12, 2^15) are not scaled; the power of two is undone
 * exactly in the fp32 result, so any finite fp32 row keeps 11 significant
 * bits per value); tiles of W are dequantized into LDS as fp16 and contracted
 * on MFMA with fp32 accumulation.  K must be a multiple
 * of 64 (else AIH_E_LIMIT) and X 16-byte aligned.  The workspace cannot grow
 * while the stream is being captured (AIH_E_LIMIT): run the largest GEMM once
 * before capturing.  A workspace replaced by a larger one stays allocated
 * until aih_destroy, so graphs captured earlier stay valid.  A product of
 * more than 256 rows whose tiles would leave CUs idle splits K over
 * workgroups (aih_qgemm_plan): its partial sums (splits * M * N floats) go
 * to a second context workspace under the same rules and are added in a
 * fixed order, so a result depends only on the shape (and the device's CU
 * count), not on the call; where that workspace cannot grow (during a
 * capture, out of memory), the call fails like the X workspace's.  Replaces
 * TempF32 + ComputeOps.MatMulWeights for M > 8. */
int aih_qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
              const float *X, int64_t M, float *Y);

/* The tiling aih_qgemm and aih_qgemm_fused choose for an M x K by N product
 * on this context's device: rows per workgroup tile (128, 256 or 512) and
 * the number of K splits (1 = none), for a call that may split
 * (may_split != 0: aih_qgemm, aih_qgemm_fused with AIH_POST_STORE or
 * AIH_POST_ACCUMULATE) or may not (aih_matmul_weights_q and its
 * allocation-free twin).  K a multiple of 64.  No counterpart in the
 * reference: it lets tests and tools see which kernel a shape reaches. */
int aih_qgemm_plan(aih_ctx *ctx, int64_t N, int64_t K, int64_t M, int may_split, int32_t *tile_rows,
                   int32_t *splits);

/* ComputeOps.MatMulWeights semantics for a quantized weight: routes M <= 8 to
 * aih_qmatvec and larger M to aih_qgemm, never split over K (the results of
 * aih_matmul_weights_q_noalloc, which has no room for partial sums). */
int aih_matmul_weights_q(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                         const float *X, int64_t M, float *Y);

/* Prefill GEMM with the neighbouring element-wise steps of a Llama layer
 * fused in:  y[m, n] = sum_k x[m, k] W[n, k] for M rows, with
 *   pre = AIH_PRE_NONE        x = X
 *   pre = AIH_PRE_RMSNORM     x[m] = (X[m] / sqrt(mean(X[m]^2) + eps)) * X2   (X2: K norm weights)
 *   pre = AIH_PRE_SILU_MUL    x = SiLU(X) * X2                               (X2: M x K)
 *   pre = AIH_PRE_SILU_PAIRS  x[m, k] = SiLU(X[m, 2k]) * X[m, 2k+1]           (X: M x 2K)
 * and
 *   pre = AIH_PRE_F16_OPERAND x: the fp16 operand image X (see below)
 * and
 *   post = AIH_POST_STORE           Y[m, n] = y[m, n]
 *   post = AIH_POST_ACCUMULATE      Y[m, n] += y[m, n]      (the residual add)
 *   post = AIH_POST_SILU_PAIRS_F16  Y = the fp16 operand image of
 *                                   SiLU(y[m, 2i]) * y[m, 2i+1]
 * The element-wise step writes the GEMM's fp16 operand directly (no fp32
 * intermediate, no separate conversion) with the formulas of aih_rmsnorm,
 * aih_silu_mul, aih_silu_mul_pairs and aih_add, so the result is bit for bit
 * that of the separate operator, then aih_qgemm (and aih_add); likewise the
 * gate|up GEMM with AIH_POST_SILU_PAIRS_F16 followed by the down GEMM with
 * AIH_PRE_F16_OPERAND gives the bits of the gate|up GEMM, aih_silu_mul_pairs
 * and the down GEMM.  Workspace, split over K,
 * K and alignment rules as aih_qgemm; X, X2 16-byte aligned; Y must not
 * alias X or X2.  Replaces, for a prompt, the LayerNorm / SiLU+Multiply /
 * Add around MatMulWeights in ComputeOps.TransformerLayer
 * (ComputeOps.cs:1250-1356) and FeedForward (ComputeOps.cs:1218-1241). */
int aih_qgemm_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                    const float *X2, float eps, int64_t M, int pre, int post, float *Y);

/* The prompt's Q|K|V projection with the position steps in its epilogue:
 * the same results, bit for bit, as aih_qgemm_fused(type, W, N = q_dim +
 * 2 kv_dim, K, X, X2, eps, M, pre, AIH_POST_STORE, Q) followed by
 * aih_rope_qkv(Q, N, Q + q_dim, N, Q + q_dim + kv_dim, N, Kc, Vc, M, n_heads,
 * n_kv_heads, head_dim, start, pos, table, table_rows, cache_rows), with
 * q_dim = n_heads*head_dim and kv_dim = n_kv_heads*head_dim, but one GEMM
 * launch writes the rotated queries into Q (M rows of N floats) and the
 * rotated keys and the values straight into the caches; the key and value
 * columns of Q are not written.  pre is AIH_PRE_NONE or AIH_PRE_RMSNORM;
 * head_dim a multiple of 32 (else AIH_E_UNSUPPORTED); X, X2 16-byte and table
 * 8-byte aligned.  Replaces, for a
 * prompt, the Q/K/V MatMulWeights, ApplyRoPEFull and the KV cache append of
 * ComputeOps.TransformerLayer (ComputeOps.cs:1250-1356, ComputeOps.cs:959-979,
 * InferenceEngine.cs:598-622). */
int aih_qgemm_qkv_rope(aih_ctx *ctx, int type, const void *W, int64_t K, const float *X, const float *X2, float eps,
                       int64_t M, int pre, float *Q, float *Kc, float *Vc, int32_t n_heads, int32_t n_kv_heads,
                       int32_t head_dim, int32_t start, const int32_t *pos, const float *table, int32_t table_rows,
                       int64_t cache_rows);

/* Bytes of the fp16 operand image of an M x K activation matrix (K a
 * multiple of 64) that AIH_POST_SILU_PAIRS_F16 and aih_attention_operand
 * write and AIH_PRE_F16_OPERAND reads: the values in the matrix cores'
 * fragment order, one power-of-two exponent per row and one per 32-column
 * block of a row (the scaling that keeps every finite fp32 value within
 * fp16's range).  A negative status for invalid sizes.  No counterpart in the
 * reference (its activations stay fp32); needs no context and no device. */
int64_t aih_operand_bytes(int64_t M, int64_t K);

/* aih_matmul_weights_q without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * being captured into a HIP graph, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments, routing, kernels and results as
 * aih_matmul_weights_q; the staging memory those kernels need (the partial
 * sums of the 3..8-column matvec, the GEMM's fp16 copy of X: mpad * (2K + 4)
 * bytes, mpad = M rounded up to 32) comes from one static device buffer of
 * AIH_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, instead of
 * the context workspace.  A call that needs more returns AIH_E_SCRATCH
 * before launching anything (at K = 4096 the GEMM takes M up to 2048; at
 * K = 14336, up to 576).  Every call on one GPU shares that buffer: calls
 * that overlap on one GPU (two streams, two contexts, two threads) race and
 * must be serialized by the caller.  Nothing in it has to start at zero. */
#define AIH_NOALLOC_SCRATCH_BYTES ((16u << 20) + (64u << 10))
int aih_matmul_weights_q_noalloc(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                                 const float *X, int64_t M, float *Y);

/* ---- decoder operators (the rest of a Llama layer around the matmuls) --
 *
 * All tensors are fp32 device arrays, row-major.  Position-dependent
 * operators take `start` and an optional device pointer `pos`: row r is at
 * position start + r, plus *pos when pos is not NULL (a decode step captured
 * into a graph reads its position from device memory; aih_argmax advances
 * it).  Bounds that depend on *pos are enforced on the device by skipping
 * rows past the cache; with pos == NULL they are checked here (AIH_E_LIMIT). */

/* Row-wise RMSNorm: Y[r,:] = (X[r,:] / sqrt(mean(X[r,:]^2) + eps)) * W.
 * Y may alias X.  Replaces ComputeOps.LayerNorm (ComputeOps.cs:517-542,
 * shader ComputeShaders.cs:247-278). */
int aih_rmsnorm(aih_ctx *ctx, const float *X, const float *W, float *Y, int64_t rows, int64_t cols, float eps);

/* RoPE table: table[(p*head_dim/2 + i)*2 + {0,1}] = {cos, sin}(p * freq_i),
 * freq_i = 1 / theta^(2i/head_dim), for p < max_pos (the reference's fp32
 * angle; power, cos and sin in double, rounded to float).  Computed once per
 * context length and shared by every layer and head. */
int aih_rope_table(aih_ctx *ctx, float *table, int32_t max_pos, int32_t head_dim, float theta);

/* Interleaved-pair RoPE of n_heads heads of each row: pair (2i, 2i+1) of a
 * head at position p is rotated by the table's angle for (p, i).  Output row
 * r, or row p itself when y_at_pos != 0 (writing rotated keys straight into a
 * KV cache of y_rows rows).  Y may alias X when !y_at_pos.  Replaces
 * ComputeOps.ApplyRoPEFull (ComputeOps.cs:959-979, shader
 * ComputeShaders.cs:517-543). */
int aih_rope(aih_ctx *ctx, const float *X, int64_t ldx, float *Y, int64_t ldy, int64_t rows, int32_t n_heads,
             int32_t head_dim, int32_t start, const int32_t *pos, const float *table, int32_t table_rows,
             int y_at_pos, int64_t y_rows);

/* The three position steps of a layer in one launch: RoPE of the query heads
 * of Q in place, RoPE of the key heads of K into the K cache at their
 * positions, V rows into the V cache (cache rows n_kv_heads*head_dim floats;
 * positions at or past cache_rows are skipped).  Q/K/V row strides ldq/ldk/ldv
 * let them be parts of one fused projection output.  Same results as
 * aih_rope (Q), aih_rope with y_at_pos (K) and aih_store_rows (V). */
int aih_rope_qkv(aih_ctx *ctx, float *Q, int64_t ldq, const float *K, int64_t ldk, const float *V, int64_t ldv,
                 float *Kc, float *Vc, int64_t rows, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                 int32_t start, const int32_t *pos, const float *table, int32_t table_rows, int64_t cache_rows);

/* KV cache append: Y[(p + r)*cols + c] = X[r*cols + c] for positions below
 * y_rows.  Replaces KVCache.Add's O(L^2) concat (InferenceEngine.cs:598-622). */
int aih_store_rows(aih_ctx *ctx, const float *X, int64_t rows, int64_t cols, float *Y, int64_t y_rows, int32_t start,
                   const int32_t *pos);

/* Y = SiLU(G) * U = (G * (1 / (1 + exp(-G)))) * U, element-wise (Y may alias
 * G or U).  Replaces the SiLU + Multiply steps of ComputeOps.FeedForward
 * (ComputeOps.cs:1218-1241). */
int aih_silu_mul(aih_ctx *ctx, const float *G, const float *U, float *Y, int64_t n);

/* Y[r, i] = SiLU(X[r, 2i]) * X[r, 2i+1] for i < n, r < rows: the SiLU * up
 * step over the output of a GEMM with gate/up rows interleaved (row stride 2n
 * in X, n in Y). */
int aih_silu_mul_pairs(aih_ctx *ctx, const float *X, float *Y, int64_t rows, int64_t n);

/* Y = SiLU(X) = X * (1 / (1 + exp(-X))), element-wise (Y may alias X).
 * Replaces ComputeOps.SiLU (ComputeOps.cs:493-510, shader ComputeShaders.cs:280-292),
 * which works in place. */
int aih_silu(aih_ctx *ctx, const float *X, float *Y, int64_t n);

/* Y = A * B, element-wise (Y may alias A or B).  Replaces ComputeOps.Multiply
 * (ComputeOps.cs:360-387, shader ComputeShaders.cs:294-306). */
int aih_mul(aih_ctx *ctx, const float *A, const float *B, float *Y, int64_t n);

/* Y = A + B, element-wise (Y may alias A or B).  Replaces ComputeOps.Add
 * (ComputeOps.cs:389). */
int aih_add(aih_ctx *ctx, const float *A, const float *B, float *Y, int64_t n);

/* Floats of scratch aih_attention needs for single-query rows with a cache of
 * max_len rows (per-split partial results), or a negative status. */
int64_t aih_attention_scratch_floats(int32_t n_heads, int32_t max_len);

/* Causal grouped-query attention over a KV cache.  Query row i (position
 * p_i) of head h attends to cache rows 0..p_i of KV head
 * h / (n_heads / n_kv_heads):  O = softmax(scale * q K^T) V.  Q and O rows
 * hold n_heads*head_dim floats, cache rows n_kv_heads*head_dim; the rows for
 * the query positions must already be in the cache.  head_dim must be 128.
 * One query row uses a split-over-keys kernel and a combine kernel, with
 * `scratch` (aih_attention_scratch_floats floats); more rows use a tiled
 * kernel with an online softmax on the fp16 matrix cores, each fp32 operand
 * split into two fp16 halves (22 significant bits, products exact, sums in
 * fp32; normwise error about 1e-7), one workgroup per 64-query tile whose
 * two halves take the first and last halves of a long key range and merge
 * in LDS (no workspace).  Calls sharing a scratch must not overlap.
 * Replaces ComputeOps.MultiHeadAttention and FusedMHAGenerate
 * (ComputeOps.cs:1015-1102, shaders ComputeShaders.cs:656-733), without the
 * latter's 4096-key limit. */
int aih_attention(aih_ctx *ctx, const float *Q, const float *Kc, const float *Vc, float *O, int64_t n_q,
                  int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start, const int32_t *pos,
                  int32_t max_len, float scale, float *scratch, int64_t scratch_floats);

/* aih_attention with query rows ldq floats apart (ldq >= n_heads*head_dim,
 * a multiple of 4): the query block of a fused Q|K|V projection output read
 * in place.  O rows stay n_heads*head_dim floats apart.  Same results as
 * aih_attention on the same query values. */
int aih_attention_strided(aih_ctx *ctx, const float *Q, int64_t ldq, const float *Kc, const float *Vc, float *O,
                          int64_t n_q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start,
                          const int32_t *pos, int32_t max_len, float scale, float *scratch,
                          int64_t scratch_floats);

/* aih_attention_strided writing its output, instead of as fp32 rows, as the
 * operand image of a GEMM over its n_heads*head_dim columns: the X of
 * aih_qgemm_fused with AIH_PRE_F16_OPERAND (aih_operand_bytes(n_q,
 * n_heads*head_dim) bytes, 16-byte aligned; rows past n_q, up to the next
 * multiple of 32, zero).  For n_q > 1 the values are the ones
 * aih_attention_strided computes, rounded to fp16 with a power of two per
 * 32-column block of a row (the same rounding as aih_qgemm_fused's
 * conversion of an fp32 X wherever both leave a value a normal fp16 number),
 * so the GEMM that follows gives the bits of aih_attention_strided +
 * aih_qgemm_fused (AIH_PRE_NONE) there, without the fp32 rows and their
 * conversion pass.  Every
 * n_q uses the tiled kernel (a single row there takes the decode kernel).
 * Replaces, for a prompt, the
 * attention output that feeds the W_o MatMulWeights in
 * ComputeOps.TransformerLayer (ComputeOps.cs:1250-1356). */
int aih_attention_operand(aih_ctx *ctx, const float *Q, int64_t ldq, const float *Kc, const float *Vc, void *Xt,
                          int64_t n_q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start,
                          const int32_t *pos, int32_t max_len, float scale);

/* One decode step's attention with the position steps before it fused in:
 * for the projection output QKV of one row at position p = start + *pos
 * (q | k | v: n_heads*head_dim, then n_kv_heads*head_dim twice, as one fused
 * Q|K|V matvec writes it), RoPE of q and k from `table`, the k and v rows
 * stored into the caches at row p (when p < max_len), and attention of each
 * query head over cache rows 0..min(p, max_len - 1).  QKV is not modified.
 * Same results, bit for bit, as aih_rope_qkv (one row) followed by
 * aih_attention (one row).  n_heads / n_kv_heads must be 1, 2, 4 or 8
 * (AIH_E_UNSUPPORTED otherwise), table_rows >= max_len; scratch as for
 * aih_attention.  Replaces, for a decode step, ApplyRoPEFull, the KV cache
 * append and FusedMHAGenerate (ComputeOps.cs:959-979, 1015-1043,
 * InferenceEngine.cs:598-622, shader ComputeShaders.cs:656-733). */
int aih_attention_decode_qkv(aih_ctx *ctx, const float *QKV, float *Kc, float *Vc, float *O, int32_t n_heads,
                             int32_t n_kv_heads, int32_t head_dim, int32_t start, const int32_t *pos,
                             const float *table, int32_t table_rows, int32_t max_len, float scale, float *scratch,
                             int64_t scratch_floats);

/* Quantized embedding gather: Y[i,:] = dequantized row ids[i] of a [vocab,
 * dim] table of `type` blocks (ids from device memory; an id outside
 * [0, vocab) gives zeros).  Bit-exact to aih_dequantize (IEEE fp16 scales).
 * Replaces ComputeOps.EmbeddingLookupFromQuantized (ComputeOps.cs:1399-1454),
 * which dequantizes the whole table below 512 MiB.  type = AIH_TYPE_F32
 * gathers rows of an fp32 table: ComputeOps.EmbeddingLookup
 * (ComputeOps.cs:1780-1800, shader ComputeShaders.cs:499-515; there a
 * negative id leaves its row unwritten and one past the table reads beyond
 * it). */
int aih_embed_q(aih_ctx *ctx, int type, const void *table, int64_t vocab, int64_t dim, const int32_t *ids, int64_t n,
                float *Y);

/* Greedy sampling step: *token = first index of the maximum of X[0..n) (NaN
 * never wins).  When pos is not NULL, also history[*pos - hist_offset] = token
 * (if inside [0, hist_len)) and *pos += 1.  Replaces the sampling of
 * InferenceEngine.RunGenerationLoop (InferenceEngine.cs:213-390) for a
 * greedy configuration. */
int aih_argmax(aih_ctx *ctx, const float *X, int64_t n, int32_t *token, int32_t *pos, int32_t *history,
               int64_t hist_len, int32_t hist_offset);

/* ---- queue (IComputeCommandQueue, IComputeCommandQueue.cs:6-33) -------- */

/* Wait for all work on the context stream.  Replaces Flush
 * (ROCmComputeCommandQueue.cs:73-80); InsertMemoryBarrier needs no
 * counterpart because the stream is in order. */
int aih_sync(aih_ctx *ctx);

/* The context's hipStream_t, for callers that interoperate with other HIP code. */
void *aih_stream(aih_ctx *ctx);

/* HIP graphs on the context stream: aih_capture_begin starts stream capture,
 * every asynchronous aih_* call until aih_capture_end is recorded instead of
 * run, and aih_graph_launch replays the recorded work (e.g. a whole decode
 * step) with one launch.  Captured work must not include aih_memset, which
 * records a memset node. */
typedef struct aih_graph aih_graph;
int aih_capture_begin(aih_ctx *ctx);
int aih_capture_end(aih_ctx *ctx, aih_graph **out);
int aih_graph_launch(aih_ctx *ctx, aih_graph *graph);
int aih_graph_destroy(aih_graph *graph);

/* GPU timestamps on the context stream (slots 0..15), replacing the host
 * stopwatch of GlobalProfiler (AIHost/Compute/ComputeProfiler.cs:16-93). */
int aih_event_record(aih_ctx *ctx, int slot);
/* Milliseconds between two recorded slots; waits for the later one. */
int aih_event_elapsed(aih_ctx *ctx, int slot_start, int slot_end, float *ms);

/* ---- measurement (no reference counterpart) ---------------------------
 * The ceiling the matvec's HBM throughput is judged against: streams `bytes`
 * (a multiple of 16, 16-byte aligned) from src with 16-byte loads, one
 * workgroup of 512 threads per CU, and nothing else; nontemporal != 0 adds
 * the non-temporal hint to the loads.  bytes == 0 launches the same grid
 * with nothing to read (the fixed cost of a launch).  `out` is a device
 * buffer of 8192 uint32 that receives an XOR of the data (one word per
 * wave).  Asynchronous on the context's stream, like the operators. */
int aih_probe_stream_read(aih_ctx *ctx, const void *src, uint64_t bytes, int nontemporal, uint32_t *out);

/* Human-readable text for any status code.  Never returns NULL. */
const char *aih_strerror(int status);

/* ABI version of the loaded library (AIH_ABI_VERSION). */
int aih_abi_version(void);

/* ---- host utilities (no reference counterpart: the reference has no
 *      quantizer; these create synthetic GGUF tensors for tests/benchmarks) */

/* out[i] = mean + std * z_i, z ~ N(0,1) from splitmix64 + Box-Muller in
 * double, cast to float.  Deterministic for a seed; multithreaded. */
int aih_host_fill_normal(uint64_t seed, float mean, float std, float *out, uint64_t n);

/* Quantize n_rows rows of k floats to `type` blocks following the GGUF rules
 * (Q8_0: d = absmax/127; Q4_0: d = signed max / -8; Q4_K: 6-bit sub-block
 * scales and mins; Q6_K: int8 sub-block scales).  dst holds
 * n_rows * aih_row_bytes(type, k) bytes.  Multithreaded. */
int aih_host_quantize(int type, const float *src, void *dst, int64_t n_rows, int64_t k);

#ifdef __cplusplus
}
#endif
#endif /* AIHOST_HIP_H */
