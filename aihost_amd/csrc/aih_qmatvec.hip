// aih_qmatvec.hip -- decode matvec with the GGUF block dequantization fused in.
//
//   Y[b*ldy + n] = sum_k X[b*ldx + k] * W[n, k]        (b < batch, n < N)
//
// This replaces, for small M, the reference's TempF32 -> DequantizeInto ->
// MatMulWeights sequence (AIHost/AIHost/Compute/TransformerBase.cs:254-271,
// ComputeOps.cs:761-861, ComputeOps.cs:275-309, ComputeShaders.cs:93-129),
// which writes and re-reads an F32 copy of every weight per token.  Here each
// packed byte is read from HBM once and never materialised as F32.
//
// Work split.  K is cut into 64-element "units"; lane u of a workgroup owns
// unit u of every row (a Q4_K (block, 64-group), a pair of Q8_0/Q4_0 blocks, or
// a Q6_K (block, half, 16-column) slice).  Because that mapping is the same for
// every row, a lane converts its 64 activations to fp16 pairs once and keeps
// them in registers; each row then costs the lane one to four 16-byte loads of
// packed bytes.  A workgroup is ceil(K/64 / 64) waves and handles R rows at a
// time (all R rows' loads are issued before any arithmetic); partial sums are
// reduced with DPP inside the wave and through LDS across waves.
//
// Arithmetic.  A 4-bit (or 6-bit, or biased 8-bit) code q is turned into the
// fp16 value 1024 + q by OR-ing it into the mantissa of 0x6400, two codes per
// 32-bit register, and contracted against fp16 activations with
// v_dot2_f32_f16, which accumulates in fp32.  The 1024 * sum(x) bias (and the
// format's own offset: -8 for Q4_0, -32 for Q6_K, +128 for biased Q8_0) is
// removed by starting the accumulator at -(1024 + offset) * sum(x).  Codes that
// sit in the high nibble are used in place (value 16*q) and the 1/16 goes into
// the per-sub-block scale.  The sub-block scales/mins are applied once per
// sub-block in fp32:
//   Q4_K: d*sc*S - dmin*mn*X      (S = sum q*x, X = sum x over the sub-block)
//   Q6_K: d*sc*sum((q-32)*x)      Q8_0: d*sum(q*x)      Q4_0: d*sum((q-8)*x)
// The only rounding beyond fp32 accumulation is that of x to fp16 (relative
// 2^-11 per element), which gives a normwise error near 2e-4, inside the 1e-3
// bound this path is held to.
#include "aih_internal.h"

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ float dot2(uint32_t p, h2 x, float acc)
{
    return __builtin_amdgcn_fdot2(as_h2(p), x, acc, false);
}
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t b) { return (a & mask) | b; }
__device__ __forceinline__ float f16lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu)); }
__device__ __forceinline__ float f16hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }
__device__ __forceinline__ h2 pack2(float a, float b)
{
    h2 r;
    r.x = (_Float16)a;  // round to nearest even
    r.y = (_Float16)b;
    return r;
}
__device__ __forceinline__ float hsum(h2 v) { return __builtin_amdgcn_fdot2(v, pack2(1.0f, 1.0f), 0.0f, false); }

template <class T>
__device__ __forceinline__ T ldg(const void *p)
{
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// ---------------------------------------------------------------- Q4_K ----
// Unit u: block u/4, 64-group g = u%4 -> qs bytes 32g..32g+31 of the block,
// low nibbles are sub-block 2g (k0 + 0..31), high nibbles sub-block 2g+1
// (k0 + 32..63), k0 = 64u.  (Element order: ComputeOps.cs:1642-1675.)
struct Q4K {
    static constexpr int kRaw = 12;
    struct X { h2 la[8], lb[8], ha[8], hb[8]; float slo, shi; };
    __device__ static void load(const uint8_t *row, int u, uint32_t *raw)
    {
        const uint8_t *b = row + (u >> 2) * 144;
        u4 h = ldg<u4>(b), qa = ldg<u4>(b + 16 + (u & 3) * 32), qb = ldg<u4>(b + 32 + (u & 3) * 32);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = qa.x; raw[5] = qa.y; raw[6] = qa.z; raw[7] = qa.w;
        raw[8] = qb.x; raw[9] = qb.y; raw[10] = qb.z; raw[11] = qb.w;
    }
    __device__ static void prep(const float *x, int u, X &r)
    {
        const float *p = x + 64 * u;
        float lo[32], hi[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            f4 a = ldg<f4>(p + 4 * i), c = ldg<f4>(p + 32 + 4 * i);
            lo[4 * i] = a.x; lo[4 * i + 1] = a.y; lo[4 * i + 2] = a.z; lo[4 * i + 3] = a.w;
            hi[4 * i] = c.x; hi[4 * i + 1] = c.y; hi[4 * i + 2] = c.z; hi[4 * i + 3] = c.w;
        }
        r.slo = r.shi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            r.la[i] = pack2(lo[4 * i], lo[4 * i + 2]);
            r.lb[i] = pack2(lo[4 * i + 1], lo[4 * i + 3]);
            r.ha[i] = pack2(hi[4 * i], hi[4 * i + 2]);
            r.hb[i] = pack2(hi[4 * i + 1], hi[4 * i + 3]);
            r.slo += hsum(r.la[i]) + hsum(r.lb[i]);
            r.shi += hsum(r.ha[i]) + hsum(r.hb[i]);
        }
    }
    template <int B>
    __device__ static void dot(const uint32_t *raw, const X *xr, int u, float *out)
    {
        // 6-bit (scale, min) of sub-blocks 2g and 2g+1 (get_scale_min_k4,
        // QuantizationFormats.cs:157-165), branch-free per lane.
        const int g = u & 3;
        const bool upper = g >= 2;
        const uint32_t s0 = (g & 1) * 16;
        const uint32_t wlo = upper ? 4u : 6u, whi = upper ? 2u : 0u, moff = upper ? 4u : 0u;
        const uint32_t a_sc = upper ? raw[3] : raw[1], a_mn = upper ? raw[3] : raw[2];
        uint32_t sc0 = __builtin_amdgcn_ubfe(a_sc, s0, wlo) | (__builtin_amdgcn_ubfe(raw[1], s0 + 6, whi) << 4);
        uint32_t sc1 = __builtin_amdgcn_ubfe(a_sc, s0 + 8, wlo) | (__builtin_amdgcn_ubfe(raw[1], s0 + 14, whi) << 4);
        uint32_t mn0 = __builtin_amdgcn_ubfe(a_mn, s0 + moff, wlo) | (__builtin_amdgcn_ubfe(raw[2], s0 + 6, whi) << 4);
        uint32_t mn1 = __builtin_amdgcn_ubfe(a_mn, s0 + 8 + moff, wlo) | (__builtin_amdgcn_ubfe(raw[2], s0 + 14, whi) << 4);
        const float d = f16lo(raw[0]), dmin = f16hi(raw[0]);
        const float c_lo = d * (float)sc0, c_hi = d * (float)sc1 * 0.0625f;
        const float m_lo = dmin * (float)mn0, m_hi = dmin * (float)mn1;
        float alo[B], ahi[B];
#pragma unroll
        for (int b = 0; b < B; ++b) { alo[b] = -1024.f * xr[b].slo; ahi[b] = -1024.f * xr[b].shi; }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t w = raw[4 + i], w8 = w >> 8;
            uint32_t p0 = and_or(w, 0x000F000Fu, kMagic), p1 = and_or(w, 0x00F000F0u, kMagic);
            uint32_t p2 = and_or(w8, 0x000F000Fu, kMagic), p3 = and_or(w8, 0x00F000F0u, kMagic);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                alo[b] = dot2(p0, xr[b].la[i], alo[b]);
                alo[b] = dot2(p2, xr[b].lb[i], alo[b]);
                ahi[b] = dot2(p1, xr[b].ha[i], ahi[b]);
                ahi[b] = dot2(p3, xr[b].hb[i], ahi[b]);
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b)
            out[b] += c_lo * alo[b] + c_hi * ahi[b] - (m_lo * xr[b].slo + m_hi * xr[b].shi);
    }
};

// ---------------------------------------------------------------- Q8_0 ----
// Unit u: blocks 2u and 2u+1 (68 bytes, 4-byte aligned), k0 = 64u.
// Block A: d at byte 0, qs at 2..33 (realigned with alignbyte); block B: d at
// 34..35, qs at 36..67.  Codes are biased by +128 (xor 0x80) to make them
// unsigned before the fp16 trick.
struct Q80 {
    static constexpr int kRaw = 17;
    struct X { h2 a[16], b[16]; float s0, s1; };  // a: (x[4i], x[4i+2]), b: (x[4i+1], x[4i+3]); i<8 block A, 8..15 block B
    __device__ static void load(const uint8_t *row, int u, uint32_t *raw)
    {
        const uint8_t *p = row + 68 * u;
        u4 v0 = ldg<u4>(p), v1 = ldg<u4>(p + 16), v2 = ldg<u4>(p + 32), v3 = ldg<u4>(p + 48);
        raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
        raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
        raw[8] = v2.x; raw[9] = v2.y; raw[10] = v2.z; raw[11] = v2.w;
        raw[12] = v3.x; raw[13] = v3.y; raw[14] = v3.z; raw[15] = v3.w;
        raw[16] = ldg<uint32_t>(p + 64);
    }
    __device__ static void prep(const float *x, int u, X &r)
    {
        const float *p = x + 64 * u;
        r.s0 = r.s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            f4 v = ldg<f4>(p + 4 * i);
            r.a[i] = pack2(v.x, v.z);
            r.b[i] = pack2(v.y, v.w);
            float s = hsum(r.a[i]) + hsum(r.b[i]);
            if (i < 8) r.s0 += s; else r.s1 += s;
        }
    }
    template <int B>
    __device__ static void dot(const uint32_t *raw, const X *xr, int, float *out)
    {
        const float dA = f16lo(raw[0]), dB = f16hi(raw[8]);
        float aA[B], aB[B];
#pragma unroll
        for (int b = 0; b < B; ++b) { aA[b] = -1152.f * xr[b].s0; aB[b] = -1152.f * xr[b].s1; }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            uint32_t w = i < 8 ? __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2) : raw[i + 1];
            uint32_t p0 = (w & 0x00FF00FFu) ^ 0x64806480u;
            uint32_t p1 = ((w >> 8) & 0x00FF00FFu) ^ 0x64806480u;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (i < 8) {
                    aA[b] = dot2(p0, xr[b].a[i], aA[b]);
                    aA[b] = dot2(p1, xr[b].b[i], aA[b]);
                } else {
                    aB[b] = dot2(p0, xr[b].a[i], aB[b]);
                    aB[b] = dot2(p1, xr[b].b[i], aB[b]);
                }
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) out[b] += dA * aA[b] + dB * aB[b];
    }
};

// ---------------------------------------------------------------- Q4_0 ----
// Unit u: blocks 2u and 2u+1 (36 bytes, 4-byte aligned), k0 = 64u.  In each
// block qs[j] holds element j (low nibble) and j+16 (high nibble).
struct Q40 {
    static constexpr int kRaw = 9;
    struct X { h2 la[8], lb[8], ha[8], hb[8]; float slo[2], shi[2]; };  // index 4*blk + i
    __device__ static void load(const uint8_t *row, int u, uint32_t *raw)
    {
        const uint8_t *p = row + 36 * u;
        u4 v0 = ldg<u4>(p), v1 = ldg<u4>(p + 16);
        raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
        raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
        raw[8] = ldg<uint32_t>(p + 32);
    }
    __device__ static void prep(const float *x, int u, X &r)
    {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const float *p = x + 64 * u + 32 * blk;
            r.slo[blk] = r.shi[blk] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f4 lo = ldg<f4>(p + 4 * i), hi = ldg<f4>(p + 16 + 4 * i);
                r.la[4 * blk + i] = pack2(lo.x, lo.z);
                r.lb[4 * blk + i] = pack2(lo.y, lo.w);
                r.ha[4 * blk + i] = pack2(hi.x, hi.z);
                r.hb[4 * blk + i] = pack2(hi.y, hi.w);
                r.slo[blk] += hsum(r.la[4 * blk + i]) + hsum(r.lb[4 * blk + i]);
                r.shi[blk] += hsum(r.ha[4 * blk + i]) + hsum(r.hb[4 * blk + i]);
            }
        }
    }
    template <int B>
    __device__ static void dot(const uint32_t *raw, const X *xr, int, float *out)
    {
        const float d[2] = {f16lo(raw[0]), f16hi(raw[4])};
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            float alo[B], ahi[B];
#pragma unroll
            for (int b = 0; b < B; ++b) { alo[b] = -1032.f * xr[b].slo[blk]; ahi[b] = -1152.f * xr[b].shi[blk]; }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t w = blk == 0 ? __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2) : raw[5 + i];
                uint32_t w8 = w >> 8;
                uint32_t p0 = and_or(w, 0x000F000Fu, kMagic), p1 = and_or(w, 0x00F000F0u, kMagic);
                uint32_t p2 = and_or(w8, 0x000F000Fu, kMagic), p3 = and_or(w8, 0x00F000F0u, kMagic);
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    alo[b] = dot2(p0, xr[b].la[4 * blk + i], alo[b]);
                    alo[b] = dot2(p2, xr[b].lb[4 * blk + i], alo[b]);
                    ahi[b] = dot2(p1, xr[b].ha[4 * blk + i], ahi[b]);
                    ahi[b] = dot2(p3, xr[b].hb[4 * blk + i], ahi[b]);
                }
            }
#pragma unroll
            for (int b = 0; b < B; ++b) out[b] += d[blk] * (alo[b] + 0.0625f * ahi[b]);
        }
    }
};

// ---------------------------------------------------------------- Q6_K ----
// Unit u: block u/4, half h = (u/2)%2, column group t = u%2.  The lane reads
// ql[64h+16t .. +15] (quarters 0 and 2), ql[64h+32+16t .. +15] (quarters 1
// and 3) and qh[32h+16t .. +15] (high 2 bits of all four quarters), i.e.
// elements 128h + 32*quarter + 16t + i, i < 16 (ComputeOps.cs:1748-1771).
// Each quarter's 16 elements form one sub-block with an int8 scale.
struct Q6K {
    static constexpr int kRaw = 15;
    struct X { h2 a[4][8]; float s[4]; };  // per quarter: i-th pair ((x[4m], x[4m+2]) for i=2m, (x[4m+1], x[4m+3]) for i=2m+1)
    __device__ static void load(const uint8_t *row, int u, uint32_t *raw)
    {
        const uint8_t *b = row + (u >> 2) * 210;
        const int h = (u >> 1) & 1, t = u & 1;
        u4 qa = ldg<u4>(b + 64 * h + 16 * t), qb = ldg<u4>(b + 64 * h + 32 + 16 * t);
        u4 qh = ldg<u4>(b + 128 + 32 * h + 16 * t);
        uint64_t sc = ldg<uint64_t>(b + 192 + 8 * h);
        raw[0] = qa.x; raw[1] = qa.y; raw[2] = qa.z; raw[3] = qa.w;
        raw[4] = qb.x; raw[5] = qb.y; raw[6] = qb.z; raw[7] = qb.w;
        raw[8] = qh.x; raw[9] = qh.y; raw[10] = qh.z; raw[11] = qh.w;
        raw[12] = (uint32_t)sc; raw[13] = (uint32_t)(sc >> 32);
        raw[14] = ldg<uint16_t>(b + 208);
    }
    __device__ static void prep(const float *x, int u, X &r)
    {
        const int h = (u >> 1) & 1, t = u & 1;
        const float *p = x + (u >> 2) * 256 + 128 * h + 16 * t;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            r.s[q] = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                f4 v = ldg<f4>(p + 32 * q + 4 * m);
                r.a[q][2 * m] = pack2(v.x, v.z);
                r.a[q][2 * m + 1] = pack2(v.y, v.w);
                r.s[q] += hsum(r.a[q][2 * m]) + hsum(r.a[q][2 * m + 1]);
            }
        }
    }
    template <int B>
    __device__ static void dot(const uint32_t *raw, const X *xr, int u, float *out)
    {
        const uint32_t t8 = (u & 1) * 8;
        const float sc0 = (float)(int)__builtin_amdgcn_sbfe((int)raw[12], t8, 8);
        const float sc1 = (float)(int)__builtin_amdgcn_sbfe((int)raw[12], t8 + 16, 8);
        const float sc2 = (float)(int)__builtin_amdgcn_sbfe((int)raw[13], t8, 8) * 0.0625f;
        const float sc3 = (float)(int)__builtin_amdgcn_sbfe((int)raw[13], t8 + 16, 8) * 0.0625f;
        const float d = f16lo(raw[14]);
        float a0[B], a1[B], a2[B], a3[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            a0[b] = -1056.f * xr[b].s[0]; a1[b] = -1056.f * xr[b].s[1];
            a2[b] = -1536.f * xr[b].s[2]; a3[b] = -1536.f * xr[b].s[3];
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t w = raw[m], v = raw[4 + m], hb = raw[8 + m];
            const uint32_t w8 = w >> 8, v8 = v >> 8, hb4 = hb << 4, hb2 = hb << 2, hr4 = hb >> 4, hr6 = hb >> 6;
            // quarter 0: low nibble of ql[A] + qh bits 0-1; quarter 2: high nibble of ql[A] + bits 4-5 (x16)
            // quarter 1: low nibble of ql[B] + qh bits 2-3; quarter 3: high nibble of ql[B] + bits 6-7 (x16)
            const uint32_t q0e = and_or(hb4, 0x00300030u, and_or(w, 0x000F000Fu, kMagic));
            const uint32_t q2e = and_or(hb4, 0x03000300u, and_or(w, 0x00F000F0u, kMagic));
            const uint32_t q1e = and_or(hb2, 0x00300030u, and_or(v, 0x000F000Fu, kMagic));
            const uint32_t q3e = and_or(hb2, 0x03000300u, and_or(v, 0x00F000F0u, kMagic));
            const uint32_t q0o = and_or(hr4, 0x00300030u, and_or(w8, 0x000F000Fu, kMagic));
            const uint32_t q2o = and_or(hr4, 0x03000300u, and_or(w8, 0x00F000F0u, kMagic));
            const uint32_t q1o = and_or(hr6, 0x00300030u, and_or(v8, 0x000F000Fu, kMagic));
            const uint32_t q3o = and_or(hr6, 0x03000300u, and_or(v8, 0x00F000F0u, kMagic));
#pragma unroll
            for (int b = 0; b < B; ++b) {
                a0[b] = dot2(q0o, xr[b].a[0][2 * m + 1], dot2(q0e, xr[b].a[0][2 * m], a0[b]));
                a1[b] = dot2(q1o, xr[b].a[1][2 * m + 1], dot2(q1e, xr[b].a[1][2 * m], a1[b]));
                a2[b] = dot2(q2o, xr[b].a[2][2 * m + 1], dot2(q2e, xr[b].a[2][2 * m], a2[b]));
                a3[b] = dot2(q3o, xr[b].a[3][2 * m + 1], dot2(q3e, xr[b].a[3][2 * m], a3[b]));
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b)
            out[b] += d * (sc0 * a0[b] + sc1 * a1[b] + (sc2 * a2[b] + sc3 * a3[b]));
    }
};

// Sum over the 64 lanes of a wave; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v)
{
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);  // row_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

template <class T, int B, int R, int MAXT>
__global__ void __launch_bounds__(MAXT)
qmatvec_kernel(const uint8_t *__restrict__ W, int64_t N, int64_t row_bytes, int units,
               const float *__restrict__ X, int64_t ldx, float *__restrict__ Y, int64_t ldy)
{
    __shared__ float red[MAXT / 64][R * B];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const bool active = tid < units;
    const int u = active ? tid : 0;

    typename T::X xr[B];
#pragma unroll
    for (int b = 0; b < B; ++b) T::prep(X + b * ldx, u, xr[b]);

    const int64_t nchunks = (N + R - 1) / R;
    for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const int64_t n0 = c * R;
        uint32_t raw[R][T::kRaw];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int64_t n = n0 + r < N ? n0 + r : N - 1;
            T::load(W + n * row_bytes, u, raw[r]);
        }
        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r][b] = 0.f;
            T::template dot<B>(raw[r], xr, u, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float v = wave_sum_to_lane63(active ? acc[r][b] : 0.f);
                if (nwaves == 1) {
                    if (lane == 63 && n0 + r < N) Y[b * ldy + n0 + r] = v;
                } else if (lane == 63) {
                    red[wave][r * B + b] = v;
                }
            }
        }
        if (nwaves > 1) {
            __syncthreads();
            if (tid < R * B) {
                const int r = tid / B, b = tid % B;
                float s = 0.f;
                for (int w = 0; w < nwaves; ++w) s += red[w][tid];
                if (n0 + r < N) Y[b * ldy + n0 + r] = s;
            }
            __syncthreads();
        }
    }
}

template <class T, int B, int R, int MAXT>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t row_bytes, int units,
           const float *X, int64_t ldx, float *Y, int64_t ldy)
{
    const int threads = ((units + 63) / 64) * 64;
    const int64_t nchunks = (N + R - 1) / R;
    const int64_t cap = (int64_t)1 << 30;
    const unsigned grid = (unsigned)(nchunks < cap ? nchunks : cap);
    hipLaunchKernelGGL((qmatvec_kernel<T, B, R, MAXT>), dim3(grid), dim3(threads), 0, ctx->stream,
                       W, N, row_bytes, units, X, ldx, Y, ldy);
    return aih_launch_status();
}

template <class T>
int launch_type(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
                const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    const int units = (int)(K / 64);
    // Columns are processed in passes of at most two; each pass re-reads W.
    for (int b0 = 0; b0 < batch; b0 += 2) {
        const float *xb = X + b0 * ldx;
        float *yb = Y + b0 * ldy;
        const bool two = batch - b0 >= 2;
        int rc;
        if (units <= 256)
            rc = two ? launch<T, 2, 4, 256>(ctx, W, N, row_bytes, units, xb, ldx, yb, ldy)
                     : launch<T, 1, 4, 256>(ctx, W, N, row_bytes, units, xb, ldx, yb, ldy);
        else  // up to 16 waves per workgroup: fewer rows in flight to stay within 128 VGPRs
            rc = two ? launch<T, 2, 1, 1024>(ctx, W, N, row_bytes, units, xb, ldx, yb, ldy)
                     : launch<T, 1, 1, 1024>(ctx, W, N, row_bytes, units, xb, ldx, yb, ldy);
        if (rc) return rc;
    }
    return AIH_OK;
}

}  // namespace

int aih_launch_qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                       const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    // Every kernel reads 64-element units: K must be a multiple of 64, and the
    // workgroup (one lane per unit) holds at most 1024 lanes.
    if (K % 64 != 0) return AIH_E_LIMIT;
    if (K / 64 > 1024) return AIH_E_LIMIT;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
    if (wa % 16 != 0) return AIH_E_INVALID;
    if (reinterpret_cast<uintptr_t>(X) % 16 != 0 || (ldx % 4) != 0) return AIH_E_INVALID;
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch_type<Q4K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q6_K: return launch_type<Q6K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q8_0: return launch_type<Q80>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q4_0: return launch_type<Q40>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    default: return AIH_E_UNSUPPORTED;
    }
}
