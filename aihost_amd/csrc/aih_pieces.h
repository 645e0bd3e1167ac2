// aih_pieces.h -- per-format weight dequantization in 16-element pieces, shared
// by the MFMA kernels (prefill GEMM and small-batch matvec).
//
// For 64-element chunk c of a row and piece s (elements 16s .. 16s+15 of the
// chunk), each format provides load() of the packed bytes the piece needs
// (raw, unconverted) and piece(), which returns the 16 fp32 weights in natural element order,
// computed with the reference's formulas (ComputeOps.cs:1629-1678 for Q4_K,
// :1735-1774 for Q6_K; the GGUF definitions for Q8_0 and Q4_0).
#pragma once

#include "aih_internal.h"

namespace aih_pieces {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <class T>
__device__ __forceinline__ T ldg(const void *p)
{
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// fp16 bits (low 16 bits of v) -> fp32.  load() keeps scales as raw bits and
// piece() converts them, so that nothing computed from a load sits on the
// load side of the scheduling barrier that keeps prefetches ahead of the math.
__device__ __forceinline__ float f16_bits(uint32_t v)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
}

__device__ __forceinline__ uint32_t byte_of(const u4 &v, int j)
{
    const uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;
    const uint32_t w = (j >> 2) == 0 ? w0 : (j >> 2) == 1 ? w1 : (j >> 2) == 2 ? w2 : w3;
    return (w >> (8 * (j & 3))) & 0xFFu;
}

// fp16 pair (1024 + c0, 1024 + c1) from code bytes 0, 1 (lo) or 2, 3 (hi) of
// c: a code byte under the exponent byte 0x64 is the fp16 value 1024 + code.
__device__ __forceinline__ uint32_t magic_lo(uint32_t c)
{
    return __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u);
}
__device__ __forceinline__ uint32_t magic_hi(uint32_t c)
{
    return __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u);
}

// Two weights (1024 + c) * s - cst from such a pair, computed in fp32 (one
// v_fma_mix_f32 each) and rounded to fp16 as a pair (v_cvt_pk_f16_f32).  The
// empty asm keeps the compiler from fusing them into v_fma_mixlo/mixhi, which
// issue at half rate on gfx950.  Rounding cst = 1024 s + m to fp32 moves a
// weight by at most 2^-24 * 1056 * |s| + 2^-24 |m|, far below its fp16 rounding.
__device__ __forceinline__ uint32_t weights2(uint32_t p, float s, float cst)
{
    typedef float f2 __attribute__((ext_vector_type(2)));
    const h2 h = __builtin_bit_cast(h2, p);
    float a = __builtin_fmaf((float)h.x, s, -cst), b = __builtin_fmaf((float)h.y, s, -cst);
    asm("" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
}

// Eight weights from the code bytes of w0, then w1, in order.
__device__ __forceinline__ h8 weights8(uint32_t w0, uint32_t w1, float s, float cst)
{
    const u4 r = {weights2(magic_lo(w0), s, cst), weights2(magic_hi(w0), s, cst),
                  weights2(magic_lo(w1), s, cst), weights2(magic_hi(w1), s, cst)};
    return __builtin_bit_cast(h8, r);
}

// Q4_K: chunk c is 64-group g = c % 4 of block c / 4; elements 0..31 of the
// group are the low nibbles of qs[32g .. 32g+31] (sub-block 2g), elements
// 32..63 the high nibbles (sub-block 2g+1) (ComputeOps.cs:1642-1675).
struct G4K {
    struct Raw { u4 hdr, qs; };
    __device__ static void load(const uint8_t *row, int c, int s, Raw &r)
    {
        const uint8_t *b = row + (c >> 2) * 144;
        r.hdr = ldg<u4>(b);
        r.qs = ldg<u4>(b + 16 + 32 * (c & 3) + 16 * (s & 1));
    }
    __device__ static void piece(const Raw &r, int c, int s, float *y)
    {
        const int hi = s >> 1;
        const int sb = 2 * (c & 3) + hi;   // sub-block 0..7
        // get_scale_min_k4 (QuantizationFormats.cs:157-165) on scales = hdr bytes 4..15
        uint32_t sc, mn;
        if (sb < 4) {
            sc = byte_of(r.hdr, 4 + sb) & 63u;
            mn = byte_of(r.hdr, 8 + sb) & 63u;
        } else {
            sc = (byte_of(r.hdr, 8 + sb) & 0xFu) | ((byte_of(r.hdr, sb) >> 6) << 4);
            mn = (byte_of(r.hdr, 8 + sb) >> 4) | ((byte_of(r.hdr, 4 + sb) >> 6) << 4);
        }
        const uint32_t h0 = r.hdr.x;
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(h0 & 0xFFFFu));
        const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h0 >> 16));
        const float D = d * (float)sc, Mn = dmin * (float)mn;
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = __builtin_amdgcn_ubfe(w[j >> 2], 8 * (j & 3) + 4 * hi, 4);
            y[j] = D * (float)q - Mn;
        }
    }
    // The same 16 weights as fp16: a nibble under 0x64 is 1024 + q (a high
    // nibble left in place is 1024 + 16q, with the scale divided by 16), and
    // (1024 + q) * D - (1024 D + Mn) = D q - Mn.  The scale and min of
    // sub-block j come from shifted header words (get_scale_min_k4 without
    // per-lane byte selects).
    __device__ static void piece_h(const Raw &r, int c, int s, h8 &lo, h8 &hi8)
    {
        const int hi = s >> 1;
        const int j = 2 * (c & 3) + hi, sh = 8 * (j & 3);
        const uint32_t a = r.hdr.y >> sh, b = r.hdr.z >> sh, w = r.hdr.w >> sh;
        const uint32_t sc = j < 4 ? (a & 63u) : ((w & 0xFu) | ((a >> 2) & 0x30u));
        const uint32_t mn = j < 4 ? (b & 63u) : (((w >> 4) & 0xFu) | ((b >> 2) & 0x30u));
        const float D = f16_bits(r.hdr.x) * (float)sc, Mn = f16_bits(r.hdr.x >> 16) * (float)mn;
        const float Dp = hi ? D * 0.0625f : D;
        const float C = 1024.f * Dp + Mn;
        const uint32_t m = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        lo = weights8(r.qs.x & m, r.qs.y & m, Dp, C);
        hi8 = weights8(r.qs.z & m, r.qs.w & m, Dp, C);
    }
};

// Q4_K in 32-weight pieces: half ph of the 32 code bytes of group g = c % 4
// holds elements 16 ph .. 16 ph + 15 of sub-block 2g (low nibbles, chunk
// columns 16 ph ..) and of sub-block 2g + 1 (high nibbles, columns 32 + 16 ph
// ..).  One header and one 16-byte code load give 32 weights, and the two
// scale/min pairs come from the same shifted header words: for g < 2 they are
// plain 6-bit fields, for g >= 2 (sub-blocks 4..7) the low four bits sit in
// the last header word and the top two in the first two (get_scale_min_k4,
// QuantizationFormats.cs:157-165), selected here by per-lane masks rather
// than branches.
struct G4K32 {
    typedef G4K::Raw Raw;
    __device__ static void load(const uint8_t *row, int c, int ph, Raw &r)
    {
        const uint8_t *b = row + (c >> 2) * 144;
        r.hdr = ldg<u4>(b);
        r.qs = ldg<u4>(b + 16 + 32 * (c & 3) + 16 * ph);
    }
    __device__ static void piece(const Raw &r, int c, int, h8 out[4])
    {
        const int g = c & 3;
        const int sh = 16 * (g & 1);
        const bool upper = g >= 2;
        const uint32_t sA = upper ? 2u : 0u, mA = upper ? 0x30u : 0x3Fu, mW = upper ? 0xFu : 0u;
        const uint32_t a = r.hdr.y >> sh, b = r.hdr.z >> sh, w = r.hdr.w >> sh;
        const uint32_t sc0 = ((a >> sA) & mA) | (w & mW);
        const uint32_t sc1 = ((a >> (8u + sA)) & mA) | ((w >> 8) & mW);
        const uint32_t mn0 = ((b >> sA) & mA) | ((w >> 4) & mW);
        const uint32_t mn1 = ((b >> (8u + sA)) & mA) | ((w >> 12) & mW);
        const float d = f16_bits(r.hdr.x), dmin = f16_bits(r.hdr.x >> 16);
        // high nibbles stay in place (16 q under the exponent byte): scale / 16
        const float D0 = d * (float)sc0, D1 = d * (float)sc1 * 0.0625f;
        const float C0 = 1024.f * D0 + dmin * (float)mn0, C1 = 1024.f * D1 + dmin * (float)mn1;
        const uint32_t lo = 0x0F0F0F0Fu, hi = 0xF0F0F0F0u;
        out[0] = weights8(r.qs.x & lo, r.qs.y & lo, D0, C0);
        out[1] = weights8(r.qs.z & lo, r.qs.w & lo, D0, C0);
        out[2] = weights8(r.qs.x & hi, r.qs.y & hi, D1, C1);
        out[3] = weights8(r.qs.z & hi, r.qs.w & hi, D1, C1);
    }
    // chunk column of out[q] for half ph
    __device__ static constexpr int col(int ph, int q) { return 16 * ph + 8 * (q & 1) + 32 * (q >> 1); }
    // LDS position (in 16-byte granules) of chunk granule g = 8 pc + col / 8:
    // with g = 16a + 8b + 4c + 2d + e, position e + 2d + 4b + 8a + 16c, so
    // that the eight lanes of a row store one piece q to eight positions of
    // one parity, 16 apart from none: with rows 33 granules apart, the 16
    // lanes of two rows then reach 16 different bank groups.
    __device__ static constexpr int swz(int g) { return (g & 3) | (((g >> 3) & 3) << 2) | (((g >> 2) & 1) << 4); }
};

// Q6_K: chunk c covers half h = (c % 4) / 2 of block c / 4, quarters
// Q0 = 2 * (c % 2) and Q0 + 1; piece s is quarter Q = Q0 + s / 2, columns
// 16 * (s % 2) .. +15 (ComputeOps.cs:1748-1771).
struct G6K {
    struct Raw { u4 ql, qh; uint32_t sc, d; };
    __device__ static void load(const uint8_t *row, int c, int s, Raw &r)
    {
        const uint8_t *b = row + (c >> 2) * 210;
        const int h = (c & 3) >> 1, Q = 2 * (c & 1) + (s >> 1), t = s & 1;
        r.ql = ldg<u4>(b + 64 * h + 32 * (Q & 1) + 16 * t);
        r.qh = ldg<u4>(b + 128 + 32 * h + 16 * t);
        r.sc = b[192 + 8 * h + 2 * Q + t];
        r.d = ldg<uint16_t>(b + 208);
    }
    __device__ static void piece(const Raw &r, int c, int s, float *y)
    {
        const int Q = 2 * (c & 1) + (s >> 1);
        const float ds = f16_bits(r.d) * (float)(int)(int8_t)(uint8_t)r.sc;
        const uint32_t l[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
        const uint32_t hb[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t lo = __builtin_amdgcn_ubfe(l[j >> 2], 8 * (j & 3) + 4 * (Q >> 1), 4);
            const uint32_t hi = __builtin_amdgcn_ubfe(hb[j >> 2], 8 * (j & 3) + 2 * Q, 2);
            y[j] = ds * (float)((int)(lo | (hi << 4)) - 32);
        }
    }
    // fp16 path: the 6-bit code (nibble | 2 high bits << 4) under 0x64 is
    // 1024 + q, and (1024 + q) * ds - 1056 * ds = ds * (q - 32).
    __device__ static void piece_h(const Raw &r, int c, int s, h8 &lo, h8 &hi8)
    {
        const int Q = 2 * (c & 1) + (s >> 1);
        const float ds = f16_bits(r.d) * (float)(int)(int8_t)(uint8_t)r.sc;
        const float C = 1056.f * ds;
        const int ls = 4 * (Q >> 1), hs = 2 * Q;
        const uint32_t l[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
        const uint32_t hb[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ((l[i] >> ls) & 0x0F0F0F0Fu) | (((hb[i] >> hs) << 4) & 0x30303030u);
        lo = weights8(q[0], q[1], ds, C);
        hi8 = weights8(q[2], q[3], ds, C);
    }
};

// Q8_0: chunk c is blocks 2c and 2c+1; piece s is elements 16 * (s % 2) ..
// of block 2c + s / 2.  y = d * q.
struct G80 {
    struct Raw { u4 qs; uint32_t d; };
    __device__ static void load(const uint8_t *row, int c, int s, Raw &r)
    {
        const uint8_t *b = row + 34 * (2 * c + (s >> 1));
        r.d = ldg<uint16_t>(b);
        r.qs = ldg<u4>(b + 2 + 16 * (s & 1));
    }
    __device__ static void piece(const Raw &r, int, int, float *y)
    {
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int j = 0; j < 16; ++j)
            y[j] = f16_bits(r.d) * (float)(int)__builtin_amdgcn_sbfe((int)w[j >> 2], 8 * (j & 3), 8);
    }
    // fp16 path: a code byte biased by 128 (xor 0x80) under 0x64 is
    // 1024 + 128 + q, and (1152 + q) * d - 1152 * d = d * q.
    __device__ static void piece_h(const Raw &r, int, int, h8 &lo, h8 &hi8)
    {
        const float d = f16_bits(r.d), C = 1152.f * d;
        lo = weights8(r.qs.x ^ 0x80808080u, r.qs.y ^ 0x80808080u, d, C);
        hi8 = weights8(r.qs.z ^ 0x80808080u, r.qs.w ^ 0x80808080u, d, C);
    }
};

// Q4_0: chunk c is blocks 2c and 2c+1; piece s is block 2c + s / 2, low
// nibbles (elements 0..15) for even s, high nibbles (16..31) for odd s.
// y = d * (q - 8).
struct G40 {
    struct Raw { u4 qs; uint32_t d; };
    __device__ static void load(const uint8_t *row, int c, int s, Raw &r)
    {
        const uint8_t *b = row + 18 * (2 * c + (s >> 1));
        r.d = ldg<uint16_t>(b);
        r.qs = ldg<u4>(b + 2);
    }
    __device__ static void piece(const Raw &r, int, int s, float *y)
    {
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = __builtin_amdgcn_ubfe(w[j >> 2], 8 * (j & 3) + 4 * (s & 1), 4);
            y[j] = f16_bits(r.d) * (float)((int)q - 8);
        }
    }
    // fp16 path as for Q4_K: a nibble under 0x64 is 1024 + q (1024 + 16q for
    // a high nibble left in place, with d' = d / 16), and
    // (1024 + q) * d' - (1024 d' + 8 d) = d' q - 8 d.
    __device__ static void piece_h(const Raw &r, int, int s, h8 &lo, h8 &hi8)
    {
        const float d = f16_bits(r.d);
        const float Dp = (s & 1) ? d * 0.0625f : d;
        const float C = 1024.f * Dp + 8.f * d;
        const uint32_t m = (s & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        lo = weights8(r.qs.x & m, r.qs.y & m, Dp, C);
        hi8 = weights8(r.qs.z & m, r.qs.w & m, Dp, C);
    }
};

__device__ __forceinline__ h8 pack8(const float *v)
{
    h8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)v[i];
    return r;
}

// fp16 weights of a piece for formats without a dedicated fp16 path.
template <class T>
__device__ __forceinline__ void piece_h_of(const typename T::Raw &r, int c, int s, h8 &lo, h8 &hi)
{
    float y[16];
    T::piece(r, c, s, y);
    lo = pack8(y);
    hi = pack8(y + 8);
}

template <class T>
struct HasPieceH {
    template <class U> static auto test(int) -> decltype(&U::piece_h, char());
    template <class U> static int test(...);
    static constexpr bool value = sizeof(test<T>(0)) == 1;
};

// 32-weight pieces for formats without a dedicated form: half ph of chunk c
// is pieces 2 ph and 2 ph + 1, columns 32 ph .. 32 ph + 31.
template <class T>
struct Pair32 {
    struct Raw { typename T::Raw a, b; };
    __device__ static void load(const uint8_t *row, int c, int ph, Raw &r)
    {
        T::load(row, c, 2 * ph, r.a);
        T::load(row, c, 2 * ph + 1, r.b);
    }
    __device__ static void piece(const Raw &r, int c, int ph, h8 out[4]);
    __device__ static constexpr int col(int ph, int q) { return 32 * ph + 8 * q; }
    // LDS position of chunk granule g = 16a + 8b + 4ph + 2q1 + q0 (see
    // G4K32::swz): q0 + 2ph + 4b + 8a + 16q1
    __device__ static constexpr int swz(int g)
    {
        return (g & 1) | (((g >> 2) & 1) << 1) | (((g >> 3) & 3) << 2) | (((g >> 1) & 1) << 4);
    }
};

// The GEMM producers' piece type for format T.
template <class T> struct Piece32 { typedef Pair32<T> type; };
template <> struct Piece32<G4K> { typedef G4K32 type; };

// The 16 weights of piece s of chunk c as two fp16 vectors.
template <class T>
__device__ __forceinline__ void piece16h(const typename T::Raw &r, int c, int s, h8 &lo, h8 &hi)
{
    if constexpr (HasPieceH<T>::value) T::piece_h(r, c, s, lo, hi);
    else piece_h_of<T>(r, c, s, lo, hi);
}

template <class T>
__device__ void Pair32<T>::piece(const Raw &r, int c, int ph, h8 out[4])
{
    piece16h<T>(r.a, c, 2 * ph, out[0], out[1]);
    piece16h<T>(r.b, c, 2 * ph + 1, out[2], out[3]);
}

}  // namespace aih_pieces
