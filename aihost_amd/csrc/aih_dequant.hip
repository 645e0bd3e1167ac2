// aih_dequant.hip -- standalone GGUF block dequantization, bit-exact to the
// reference decoders.
//
// Element order and arithmetic follow the code that actually runs in the
// reference: the inline GLSL shaders and their CPU twins
//   Q4_K  AIHost/AIHost/Compute/QuantizationFormats.cs:140-196, ComputeOps.cs:1629-1678
//   Q6_K  AIHost/AIHost/Compute/QuantizationFormats.cs:269-321, ComputeOps.cs:1735-1774
// and, for the two formats the reference rejects (ComputeOps.cs:743), the GGUF
// definitions of Q8_0 (y = q*d) and Q4_0 (y = (q-8)*d).
//
// Each lane produces 4 consecutive outputs (one 16-byte store), so a wave
// writes 1 KiB contiguous: one K-quant super-block, or eight Q8_0/Q4_0 blocks.
// The fp32 expressions are evaluated exactly as the C# source writes them,
// left to right with one rounding per operation (contraction is disabled for
// the whole file), which makes the result bit-identical to the CPU decoder.
#include "aih_internal.h"

#pragma clang fp contract(off)

namespace {

// QuantizationFormats.cs:147-152 (the reference GPU decoder): IEEE decoding
// with -0 -> +0 and every NaN -> 0x7FC00000.
__device__ __forceinline__ float f16_ieee_glsl(uint32_t h)
{
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0u) {
        if (m == 0u) return 0.0f;
        float v = (float)m * 5.9604644775390625e-8f;   // m * 2^-24, exact
        return s ? -v : v;
    }
    if (e == 31u) return m ? __uint_as_float(0x7FC00000u) : __uint_as_float(s ? 0xFF800000u : 0x7F800000u);
    return __uint_as_float((s << 31) | ((e + 112u) << 23) | (m << 13));
}

// ComputeOps.cs:1497-1522 (the reference CPU decoder), reproduced bit for bit:
// for subnormals it normalises the mantissa but sets the exponent to
// 1 - shift + 127 (shift = index of the leading mantissa bit), NaN payloads
// and the sign of zero are kept.
__device__ __forceinline__ float f16_refcpu(uint32_t h)
{
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    if (exp == 0u) {
        if (mant == 0u) return __uint_as_float(sign << 31);
        int shift = 31 - __clz((int)mant);            // leading bit position, 0..9
        exp = (uint32_t)(1 - shift + 127);
        mant = ((mant << (10 - shift)) & 0x3FFu) << 13;
    } else if (exp == 0x1Fu) {
        exp = 0xFFu;
        mant <<= 13;
    } else {
        exp = exp - 15u + 127u;
        mant <<= 13;
    }
    return __uint_as_float((sign << 31) | (exp << 23) | (mant & 0x7FFFFFu));
}

template <int MODE>
__device__ __forceinline__ float f16_decode(uint32_t h)
{
    return MODE == AIH_F16_REFCPU ? f16_refcpu(h) : f16_ieee_glsl(h);
}

__device__ __forceinline__ uint32_t ld_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p)
{
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p)
{
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

typedef float f4 __attribute__((ext_vector_type(4)));

// Q4_K: 64 lanes per 144-byte block (QuantizationFormats.cs:167-195).
template <int MODE>
__device__ __forceinline__ f4 deq4_q4_k(const uint8_t *b, int lane)
{
    int e0 = lane * 4;
    int group = e0 / 64, within = e0 % 64;
    int is_upper = within >= 32 ? 1 : 0;
    int wg_lower = within % 32;
    int j = group * 2 + is_upper;
    const uint8_t *sc_p = b + 4;
    uint32_t sc8, mn8;
    if (j < 4) {
        sc8 = ld_u8(sc_p + j) & 63u;
        mn8 = ld_u8(sc_p + j + 4) & 63u;
    } else {
        sc8 = (ld_u8(sc_p + j + 4) & 0xFu) | ((ld_u8(sc_p + j - 4) >> 6) << 4);
        mn8 = (ld_u8(sc_p + j + 4) >> 4) | ((ld_u8(sc_p + j) >> 6) << 4);
    }
    float d = f16_decode<MODE>(ld_u16(b)), dmin = f16_decode<MODE>(ld_u16(b + 2));
    float sc = (float)sc8, mn = (float)mn8;
    uint32_t q4 = ld_u32(b + 16 + group * 32 + wg_lower) >> (is_upper * 4);
    f4 r;
    // y = d * sc * q - dmin * mn, one rounding per operation
    r.x = d * sc * (float)(q4 & 15u) - dmin * mn;
    r.y = d * sc * (float)((q4 >> 8) & 15u) - dmin * mn;
    r.z = d * sc * (float)((q4 >> 16) & 15u) - dmin * mn;
    r.w = d * sc * (float)((q4 >> 24) & 15u) - dmin * mn;
    return r;
}

// Q6_K: 64 lanes per 210-byte block (QuantizationFormats.cs:286-320).
template <int MODE>
__device__ __forceinline__ f4 deq4_q6_k(const uint8_t *b, int lane)
{
    int e0 = lane * 4;
    int blk_h = e0 / 128, w = e0 % 128, quarter = w / 32, wq = w % 32;
    int ql_extra = (quarter == 1 || quarter == 3) ? 32 : 0;
    int is_upper = (quarter == 2 || quarter == 3) ? 1 : 0;
    uint32_t ql = ld_u32(b + blk_h * 64 + ql_extra + wq) >> (is_upper * 4);
    uint32_t qh = ld_u32(b + 128 + blk_h * 32 + wq) >> (quarter * 2);
    int sc = (int)(int8_t)ld_u8(b + 192 + e0 / 16);
    float d = f16_decode<MODE>(ld_u16(b + 208));
    f4 r;
    // y = d * sc * (q - 32)
    r.x = d * (float)sc * (float)((int)((ql & 15u) | ((qh & 3u) << 4)) - 32);
    r.y = d * (float)sc * (float)((int)(((ql >> 8) & 15u) | (((qh >> 8) & 3u) << 4)) - 32);
    r.z = d * (float)sc * (float)((int)(((ql >> 16) & 15u) | (((qh >> 16) & 3u) << 4)) - 32);
    r.w = d * (float)sc * (float)((int)(((ql >> 24) & 15u) | (((qh >> 24) & 3u) << 4)) - 32);
    return r;
}

// Q8_0: 8 lanes per 34-byte block; y = q * d.
template <int MODE>
__device__ __forceinline__ f4 deq4_q8_0(const uint8_t *b, int lane)
{
    float d = f16_decode<MODE>(ld_u16(b));
    uint32_t q = ld_u32(b + 2 + lane * 4);
    f4 r;
    r.x = (float)(int8_t)(q & 0xFFu) * d;
    r.y = (float)(int8_t)((q >> 8) & 0xFFu) * d;
    r.z = (float)(int8_t)((q >> 16) & 0xFFu) * d;
    r.w = (float)(int8_t)(q >> 24) * d;
    return r;
}

// Q4_0: 8 lanes per 18-byte block; low nibble -> j, high nibble -> j + 16,
// y = (q - 8) * d.
template <int MODE>
__device__ __forceinline__ f4 deq4_q4_0(const uint8_t *b, int lane)
{
    float d = f16_decode<MODE>(ld_u16(b));
    uint32_t q = ld_u32(b + 2 + (lane & 3) * 4) >> ((lane >> 2) * 4);
    f4 r;
    r.x = (float)((int)(q & 15u) - 8) * d;
    r.y = (float)((int)((q >> 8) & 15u) - 8) * d;
    r.z = (float)((int)((q >> 16) & 15u) - 8) * d;
    r.w = (float)((int)((q >> 24) & 15u) - 8) * d;
    return r;
}

template <int TYPE, int MODE>
__global__ void __launch_bounds__(256)
dequant_kernel(const uint8_t *__restrict__ q, f4 *__restrict__ out, uint64_t n_blocks)
{
    constexpr int QK = (TYPE == AIH_TYPE_Q4_K || TYPE == AIH_TYPE_Q6_K) ? 256 : 32;
    constexpr int BB = TYPE == AIH_TYPE_Q4_K ? 144 : TYPE == AIH_TYPE_Q6_K ? 210 : TYPE == AIH_TYPE_Q8_0 ? 34 : 18;
    constexpr int LPB = QK / 4;  // lanes per block
    const uint64_t total = n_blocks * LPB;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
        uint64_t blk = t / LPB;
        int lane = (int)(t % LPB);
        const uint8_t *b = q + blk * BB;
        f4 r;
        if (TYPE == AIH_TYPE_Q4_K) r = deq4_q4_k<MODE>(b, lane);
        else if (TYPE == AIH_TYPE_Q6_K) r = deq4_q6_k<MODE>(b, lane);
        else if (TYPE == AIH_TYPE_Q8_0) r = deq4_q8_0<MODE>(b, lane);
        else r = deq4_q4_0<MODE>(b, lane);
        out[t] = r;
    }
}

// Row gather: out[i, :] = dequantized row ids[i] of a [vocab, dim] table,
// with the same per-lane decoders as dequant_kernel (bit-exact to it).  An
// id outside [0, vocab) yields a row of zeros.
template <int TYPE>
__global__ void __launch_bounds__(256)
embed_kernel(const uint8_t *__restrict__ table, int64_t vocab, int64_t row_bytes, int64_t blocks_per_row,
             const int32_t *__restrict__ ids, int64_t n, f4 *__restrict__ out)
{
    constexpr int QK = (TYPE == AIH_TYPE_Q4_K || TYPE == AIH_TYPE_Q6_K) ? 256 : 32;
    constexpr int BB = TYPE == AIH_TYPE_Q4_K ? 144 : TYPE == AIH_TYPE_Q6_K ? 210 : TYPE == AIH_TYPE_Q8_0 ? 34 : 18;
    constexpr int LPB = QK / 4;
    const uint64_t per_row = (uint64_t)blocks_per_row * LPB;
    const uint64_t total = (uint64_t)n * per_row;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
        const uint64_t i = t / per_row, r = t % per_row;
        const int64_t id = ids[i];
        f4 v = {0.f, 0.f, 0.f, 0.f};
        if (id >= 0 && id < vocab) {
            const uint8_t *b = table + id * row_bytes + (r / LPB) * BB;
            const int lane = (int)(r % LPB);
            if (TYPE == AIH_TYPE_Q4_K) v = deq4_q4_k<AIH_F16_IEEE>(b, lane);
            else if (TYPE == AIH_TYPE_Q6_K) v = deq4_q6_k<AIH_F16_IEEE>(b, lane);
            else if (TYPE == AIH_TYPE_Q8_0) v = deq4_q8_0<AIH_F16_IEEE>(b, lane);
            else v = deq4_q4_0<AIH_F16_IEEE>(b, lane);
        }
        out[t] = v;
    }
}

template <int TYPE>
int launch_embed(aih_ctx *ctx, const void *table, int64_t vocab, int64_t dim, const int32_t *ids, int64_t n,
                 float *out)
{
    constexpr int QK = (TYPE == AIH_TYPE_Q4_K || TYPE == AIH_TYPE_Q6_K) ? 256 : 32;
    constexpr int BB = TYPE == AIH_TYPE_Q4_K ? 144 : TYPE == AIH_TYPE_Q6_K ? 210 : TYPE == AIH_TYPE_Q8_0 ? 34 : 18;
    const int64_t bpr = dim / QK;
    const uint64_t threads = (uint64_t)n * bpr * (QK / 4);
    const uint64_t want = (threads + 255) / 256;
    const uint64_t cap = (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256) * 16;
    const unsigned grid = (unsigned)(want < cap ? want : cap);
    hipLaunchKernelGGL((embed_kernel<TYPE>), dim3(grid), dim3(256), 0, ctx->stream,
                       static_cast<const uint8_t *>(table), vocab, bpr * BB, bpr, ids, n, reinterpret_cast<f4 *>(out));
    return aih_launch_status();
}

template <int TYPE>
int launch_type(aih_ctx *ctx, const void *q, float *out, uint64_t n_blocks, int mode)
{
    constexpr int LPB = (TYPE == AIH_TYPE_Q4_K || TYPE == AIH_TYPE_Q6_K) ? 64 : 8;
    uint64_t threads = n_blocks * LPB;
    uint64_t want = (threads + 255) / 256;
    uint64_t cap = (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256) * 64;
    unsigned grid = (unsigned)(want < cap ? want : cap);
    const uint8_t *qb = static_cast<const uint8_t *>(q);
    f4 *o = reinterpret_cast<f4 *>(out);
    if (mode == AIH_F16_REFCPU)
        hipLaunchKernelGGL((dequant_kernel<TYPE, AIH_F16_REFCPU>), dim3(grid), dim3(256), 0, ctx->stream, qb, o, n_blocks);
    else
        hipLaunchKernelGGL((dequant_kernel<TYPE, AIH_F16_IEEE>), dim3(grid), dim3(256), 0, ctx->stream, qb, o, n_blocks);
    return aih_launch_status();
}

}  // namespace

int aih_launch_embed(aih_ctx *ctx, int type, const void *table, int64_t vocab, int64_t dim,
                     const int32_t *ids, int64_t n, float *out)
{
    if (n == 0) return AIH_OK;
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return AIH_E_INVALID;
    switch (type) {
    case AIH_TYPE_Q4_K: return launch_embed<AIH_TYPE_Q4_K>(ctx, table, vocab, dim, ids, n, out);
    case AIH_TYPE_Q6_K: return launch_embed<AIH_TYPE_Q6_K>(ctx, table, vocab, dim, ids, n, out);
    case AIH_TYPE_Q8_0: return launch_embed<AIH_TYPE_Q8_0>(ctx, table, vocab, dim, ids, n, out);
    case AIH_TYPE_Q4_0: return launch_embed<AIH_TYPE_Q4_0>(ctx, table, vocab, dim, ids, n, out);
    default: return AIH_E_UNSUPPORTED;
    }
}

int aih_launch_dequant(aih_ctx *ctx, int type, const void *q, float *out,
                       uint64_t n_blocks, int f16_mode)
{
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return AIH_E_INVALID;
    switch (type) {
    case AIH_TYPE_Q4_K: return launch_type<AIH_TYPE_Q4_K>(ctx, q, out, n_blocks, f16_mode);
    case AIH_TYPE_Q6_K: return launch_type<AIH_TYPE_Q6_K>(ctx, q, out, n_blocks, f16_mode);
    case AIH_TYPE_Q8_0: return launch_type<AIH_TYPE_Q8_0>(ctx, q, out, n_blocks, f16_mode);
    case AIH_TYPE_Q4_0: return launch_type<AIH_TYPE_Q4_0>(ctx, q, out, n_blocks, f16_mode);
    default: return AIH_E_UNSUPPORTED;
    }
}
