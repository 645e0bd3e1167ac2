/*
 * oracle.c -- CPU restatement of AIHost's GGUF dequantization and weight
 * matmul.  TEST INFRASTRUCTURE ONLY (see oracle.h for the file:line map).
 *
 * Floating-point model: C# `float` arithmetic under RyuJIT is IEEE single with
 * round-to-nearest and no FMA contraction, evaluated left to right.  This file
 * is compiled with -ffp-contract=off so `a * b - c * d` rounds after every
 * operation exactly like the C# expression.
 */
#include "oracle.h"
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ComputeOps.cs:1497-1522.  The subnormal branch computes the exponent as
 * 1 - shift + 127 where shift counts down from 10 while normalising; that is
 * the reference's behaviour (wrong for every fp16 subnormal) and it is kept
 * here on purpose: this is the "refcpu" decoding mode. */
float orc_f16_refcpu(uint16_t h)
{
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return sign == 0 ? 0.0f : -0.0f;
        int shift = 10;
        while ((mant & 0x400u) == 0) { mant <<= 1; shift--; }
        exp = (uint32_t)(1 - shift + 127);
        mant = (mant & 0x3FFu) << 13;
    } else if (exp == 0x1F) {
        exp = 0xFF;
        mant <<= 13;
    } else {
        exp = exp - 15 + 127;
        mant <<= 13;
    }
    uint32_t bits = (sign << 31) | (exp << 23) | (mant & 0x7FFFFFu);
    return bits_to_f32(bits);
}

/* QuantizationFormats.cs:147-152: correct IEEE decoding; every NaN becomes the
 * canonical 0x7FC00000 and infinities keep their sign. */
float orc_f16_glsl(uint16_t h)
{
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0u) {
        if (m == 0u) return 0.0f;          /* GLSL returns +0.0 for both zeros */
        e = 1u;
        while ((m & 1024u) == 0u) { m <<= 1u; e -= 1u; }
        m &= 1023u;
    } else if (e == 31u) {
        return m != 0u ? bits_to_f32(0x7FC00000u) : (s ? bits_to_f32(0xFF800000u) : bits_to_f32(0x7F800000u));
    }
    e = e - 15u + 127u;
    return bits_to_f32((s << 31) | (e << 23) | (m << 13));
}

static inline float f16_decode(uint16_t h, int mode)
{
    return mode == ORC_F16_REFCPU ? orc_f16_refcpu(h) : orc_f16_glsl(h);
}

void orc_f16_decode_array(const uint16_t *h, float *out, int64_t n, int mode)
{
    for (int64_t i = 0; i < n; ++i) out[i] = f16_decode(h[i], mode);
}

/* QuantizationFormats.cs:157-165 / ComputeOps.cs:1653-1666: 6-bit scale and
 * min of sub-block j (0..7) from the 12-byte packed scales. */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

int64_t orc_block_elems(int type)
{
    switch (type) {
    case ORC_Q8_0: case ORC_Q4_0: return 32;
    case ORC_Q4_K: case ORC_Q6_K: return 256;
    case ORC_F32: return 1;
    default: return -1;
    }
}

/* AIHost/AIHost/GGUF/GGUFTensorInfo.cs:60-71 */
int64_t orc_block_bytes(int type)
{
    switch (type) {
    case ORC_Q8_0: return 34;
    case ORC_Q4_0: return 18;
    case ORC_Q4_K: return 144;
    case ORC_Q6_K: return 210;
    case ORC_F32: return 4;
    default: return -1;
    }
}

int64_t orc_row_bytes(int type, int64_t k)
{
    int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (be <= 0 || k < 0 || k % be) return -1;
    return (k / be) * bb;
}

static uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* GGUF Q8_0: d f16 | qs int8[32]; y[j] = qs[j] * d (ggml dequantize_row_q8_0). */
static void deq_q8_0(const uint8_t *b, float *y, int mode)
{
    float d = f16_decode(rd_u16(b), mode);
    const int8_t *qs = (const int8_t *)(b + 2);
    for (int j = 0; j < 32; ++j) y[j] = (float)qs[j] * d;
}

/* GGUF Q4_0: d f16 | qs u8[16]; low nibble -> j, high nibble -> j+16,
 * y = (q - 8) * d (ggml dequantize_row_q4_0). */
static void deq_q4_0(const uint8_t *b, float *y, int mode)
{
    float d = f16_decode(rd_u16(b), mode);
    const uint8_t *qs = b + 2;
    for (int j = 0; j < 16; ++j) {
        int x0 = (qs[j] & 0x0F) - 8;
        int x1 = (qs[j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}

/* ComputeOps.cs:1629-1678 (DequantizeRowQ4K), element by element:
 *   d f16 @0 | dmin f16 @2 | scales[12] @4 | qs[128] @16
 *   group = e/64, upper = (e%64) >= 32, q = (qs[group*32 + e%32] >> 4*upper) & 15,
 *   y = d * sc * q - dmin * mn   with (sc, mn) = get_scale_min_k4(2*group + upper). */
static void deq_q4_k(const uint8_t *b, float *y, int mode)
{
    float d = f16_decode(rd_u16(b), mode);
    float dmin = f16_decode(rd_u16(b + 2), mode);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int e = 0; e < 256; ++e) {
        int group = e / 64;
        int within = e % 64;
        int is_upper = within >= 32 ? 1 : 0;
        int wg_lower = within % 32;
        uint8_t sc8, mn8;
        orc_get_scale_min_k4(group * 2 + is_upper, scales, &sc8, &mn8);
        float sc = (float)sc8, mn = (float)mn8;
        int q = (qs[group * 32 + wg_lower] >> (is_upper * 4)) & 0x0F;
        y[e] = d * sc * (float)q - dmin * mn;
    }
}

/* ComputeOps.cs:1735-1774 (DequantizeRowQ6K):
 *   ql[128] @0 | qh[64] @128 | scales int8[16] @192 | d f16 @208
 *   half = e/128, w = e%128, quarter = w/32, wq = w%32,
 *   lo4 = (ql[half*64 + (quarter odd ? 32 : 0) + wq] >> (quarter >= 2 ? 4 : 0)) & 15,
 *   hi2 = (qh[half*32 + wq] >> 2*quarter) & 3,  q = lo4 | hi2 << 4,
 *   y = d * sc * (q - 32)  with sc = (int8) scales[e/16]. */
static void deq_q6_k(const uint8_t *b, float *y, int mode)
{
    float d = f16_decode(rd_u16(b + 208), mode);
    for (int e = 0; e < 256; ++e) {
        int blk_h = e / 128, w = e % 128, quarter = w / 32, wq = w % 32;
        int ql_extra = (quarter == 1 || quarter == 3) ? 32 : 0;
        int is_upper = (quarter == 2 || quarter == 3) ? 1 : 0;
        int lower4 = (b[blk_h * 64 + ql_extra + wq] >> (is_upper * 4)) & 0x0F;
        int upper2 = (b[128 + blk_h * 32 + wq] >> (quarter * 2)) & 0x03;
        int q = lower4 | (upper2 << 4);
        int sc = (int8_t)b[192 + e / 16];
        y[e] = d * (float)sc * (float)(q - 32);
    }
}

typedef void (*deq_fn)(const uint8_t *, float *, int);

static deq_fn pick(int type)
{
    switch (type) {
    case ORC_Q8_0: return deq_q8_0;
    case ORC_Q4_0: return deq_q4_0;
    case ORC_Q4_K: return deq_q4_k;
    case ORC_Q6_K: return deq_q6_k;
    default: return 0;
    }
}

int orc_dequantize(int type, const void *src, float *dst, int64_t n, int f16_mode)
{
    if (type == ORC_F32) { memcpy(dst, src, (size_t)n * 4); return 0; }
    deq_fn f = pick(type);
    int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (!f || n < 0 || n % be) return -1;
    const uint8_t *s = (const uint8_t *)src;
    for (int64_t i = 0; i < n / be; ++i) f(s + i * bb, dst + i * be, f16_mode);
    return 0;
}

/* One output row: dequantize row n of W, then for each batch column b
 * acc = 0; for k: acc += x[k] * w[k]  (TransformerBase.cs:454-456 order). */
int orc_matvec(int type, const void *w, int64_t n_rows, int64_t k,
               const float *x, int64_t ldx, int64_t batch, float *y, int64_t ldy,
               int f16_mode, int nthreads)
{
    int64_t rb = orc_row_bytes(type, k);
    if (rb < 0 || n_rows < 0 || batch < 1 || ldx < k || ldy < n_rows) return -1;
    if (type != ORC_F32 && !pick(type)) return -1;
    const uint8_t *wb = (const uint8_t *)w;
    int bad = 0;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads) reduction(|:bad)
#endif
    {
        float *row = (float *)malloc((size_t)k * sizeof(float));
        if (!row) bad = 1;
        else {
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t n = 0; n < n_rows; ++n) {
                orc_dequantize(type, wb + n * rb, row, k, f16_mode);
                for (int64_t b = 0; b < batch; ++b) {
                    const float *xb = x + b * ldx;
                    float acc = 0.0f;
                    for (int64_t i = 0; i < k; ++i) acc += xb[i] * row[i];
                    y[b * ldy + n] = acc;
                }
            }
            free(row);
        }
    }
    (void)nthreads;
    return bad ? -1 : 0;
}

int orc_matvec_f64(int type, const void *w, int64_t n_rows, int64_t k,
                   const float *x, int64_t ldx, int64_t batch, double *y, int64_t ldy,
                   int f16_mode, int nthreads)
{
    int64_t rb = orc_row_bytes(type, k);
    if (rb < 0 || n_rows < 0 || batch < 1 || ldx < k || ldy < n_rows) return -1;
    if (type != ORC_F32 && !pick(type)) return -1;
    const uint8_t *wb = (const uint8_t *)w;
    int bad = 0;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads) reduction(|:bad)
#endif
    {
        float *row = (float *)malloc((size_t)k * sizeof(float));
        if (!row) bad = 1;
        else {
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t n = 0; n < n_rows; ++n) {
                orc_dequantize(type, wb + n * rb, row, k, f16_mode);
                for (int64_t b = 0; b < batch; ++b) {
                    const float *xb = x + b * ldx;
                    double acc = 0.0;
                    for (int64_t i = 0; i < k; ++i) acc += (double)xb[i] * (double)row[i];
                    y[b * ldy + n] = acc;
                }
            }
            free(row);
        }
    }
    (void)nthreads;
    return bad ? -1 : 0;
}
