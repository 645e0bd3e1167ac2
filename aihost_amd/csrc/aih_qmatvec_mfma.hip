// aih_qmatvec_mfma.hip -- small-batch decode matvec (3..8 activation columns)
// on the matrix cores, dequantization fused, fp32-equivalent arithmetic.
//
//   Y[b*ldy + n] = sum_k X[b*ldx + k] * W[n, k]        (b < batch, n < N)
//
// The single-column matvec (aih_qmatvec.hip) contracts each weight once per
// column, so its ALU work grows with the batch; above two columns it would
// re-read W once per pair of columns.  Here W is read from HBM exactly once
// and every product runs on v_mfma_f32_16x16x32_f16.
//
// Exact operands.  A code c masked out of its packed word into the top bits
// of an fp16 half (two per 32-bit register) is the fp16 subnormal
// f * c * 2^-24 (f = 64, 16 or 4): no conversion and no bias.  An
// activation is held as two fp16 numbers, hi = fp16(x') and lo =
// fp16(x' - hi), x' = x * S with S a power of two per (column, group of
// sub-blocks) that puts the group's largest |x'| in [2^13, 2^14).  Products
// of two fp16 numbers are exact in fp32, and the matrix core's fp32
// accumulation measured correctly rounded to within 1e-7 of the sum of
// |products|, so the two MFMAs (lo, then hi, into one accumulator) give
// sum(c * x') to about fp32 precision.  The reference's formulas are then
// applied per sub-block, in fp32, after the MFMA (ComputeOps.cs:1629-1678
// Q4_K, :1735-1774 Q6_K; GGUF Q8_0, Q4_0):
//   contribution = k_sb * sum(c * x) - o_sb * sum(x)
//   Q4_K: k = d*sc, o = dmin*mn      Q6_K: k = d*sc, o = 32*d*sc
//   Q8_0: k = d,    o = 128*d (codes biased by 128)      Q4_0: k = d, o = 8*d
//
// Sub-blocks as MFMA rows.  The MFMA's A operand is the activations and its
// B operand the codes: column j of the 16 x 16 tile is weight row j of the
// wave's tile, and row i is the pair (batch column b, sub-block t) with
// i = b*T + t, T = 16 / Bp (Bp = 8 for 5..8 columns, 4 for 3..4).  A group of
// T consecutive sub-blocks is contracted in 32-element windows; in window w a
// lane's 8 activations are those of its batch column where they belong to its
// sub-block t and zeros elsewhere (read from an all-zero LDS row).  So every
// output element belongs to exactly one (column, sub-block), and lane l holds
// rows 4(l/16)..+3 of weight row l%16: the very row whose header it decoded.
//
// Work split.  K is cut into 256-element units (one Q4_K/Q6_K super-block,
// eight Q8_0/Q4_0 blocks).  A workgroup of four waves owns 64 weight rows (a
// 16-row MFMA tile per wave) and a contiguous range of units (a split of K).
// In each round of up to UPW units the workgroup stages its slice of X
// (all columns) into LDS as hi/lo fp16 pieces, with the per-group scales and
// the per-sub-block sums of x, and each lane loads, for its weight row, the
// 8 codes of every 32-element window that its k-block covers.  Each workgroup
// writes its 64 x batch partial sums to the context workspace (or to the
// staging memory the allocation-free entry point supplies); a second
// kernel adds the splits in a fixed order (the result does not depend on
// timing).  With one split the first kernel stores Y itself.
//
// This replaces TempF32 + ComputeOps.MatMulWeights for M = batch in 3..8
// (AIHost/AIHost/Compute/TransformerBase.cs:254-271, ComputeOps.cs:275-309).
#include "aih_internal.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int TW = 4;            // waves per workgroup
constexpr int RWG = 16 * TW;     // weight rows per workgroup
constexpr int UNIT = 256;        // k per unit
constexpr int MAXB = 8;          // batch columns
constexpr int ZROW = MAXB;       // the all-zero activation row of the LDS image

typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u4 bld16(Rsrc r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
}
__device__ __forceinline__ uint64_t bld8(Rsrc r, uint32_t vo, uint32_t so)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
    return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
}
// The 8 bytes at vo + 2 for a 4-byte-aligned vo (Q8_0/Q4_0 code pieces that
// start at 2 mod 4): one aligned 12-byte load and two funnel shifts; an
// 8-byte load at 2 mod 4 takes the slow unaligned path.
__device__ __forceinline__ uint64_t bld8_at2(Rsrc r, uint32_t vo, uint32_t so)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, vo, so, 0);
    const uint32_t lo = __builtin_amdgcn_alignbit(v[1], v[0], 16), hi = __builtin_amdgcn_alignbit(v[2], v[1], 16);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}
__device__ __forceinline__ uint32_t bld2(Rsrc r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
}
__device__ __forceinline__ float f16_bits(uint32_t v)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
}
// (a & mask) | b, which the compiler emits as one v_and_or_b32 (mask in an
// SGPR).  It is written in C, not as inline asm: the compiler's hazard
// tracking does not see an inline-asm VGPR write, and gfx950 needs 2 wait
// states between a VALU write and an MFMA reading that VGPR.  The asm form
// left 1 in places (4 to 13 per Q6_K kernel instantiation), and a build whose
// schedule differed only elsewhere in the kernel produced wrong Q6_K partial
// sums at 5..8 columns.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t b)
{
    return (a & mask) | b;
}

// Fragment of 8 codes from two packed words (w0: elements j..j+3 in bytes
// 0..3, w1: j+4..j+7): the codes of bytes 0 and 2 shifted left by sl, those of
// bytes 1 and 3 right by sr, each masked by m to the top bits of its fp16
// mantissa: the fp16 subnormals f * c * 2^-24 (f = 64 for 4-bit codes, 16
// for 6-bit, 4 for 8-bit) of elements j, j+2, j+1, j+3, j+4, j+6, j+5, j+7
// (the order kPerm, which the activation pieces follow).  Codes are kept as
// high in the mantissa as they fit because the matrix core's products of
// small subnormals are less exact and slightly biased (on MI355X, codes 0..15
// at 2^-24 measured a normwise error of 2e-6, 16 times larger codes 1e-7;
// over K = 65536 a Q4_K product measured 7e-6 with 16c and 1.5e-6 with 64c).
__device__ __forceinline__ h8 frag(uint32_t w0, uint32_t w1, uint32_t sl, uint32_t sr, uint32_t m)
{
    const u4 r = {(w0 << sl) & m, (w0 >> sr) & m, (w1 << sl) & m, (w1 >> sr) & m};
    return __builtin_bit_cast(h8, r);
}
__device__ constexpr int kPerm[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// ---------------------------------------------------------------------------
// Per-format unit.  A lane (weight row n, k-block q < 4) holds, for each of
// the 8 windows w of a unit (elements 32w .. 32w+31), the codes of elements
// 32w + 8q .. +7.  load() reads them (raw, at the unit's byte offset `so`);
// coef() gives k (and, for Q4_K, o) of every sub-block of the unit; code()
// returns window w's fragment, which holds f * c (f = 64, 16 or 4): k
// carries the 1/f.  Where o is a fixed multiple of k (Q6_K, Q8_0, Q4_0) the
// staged sums of x carry the factor -o/k (kSumScale).

// Q4_K unit = one super-block (d, dmin, scales[12], qs[128]); sub-block j
// (32 elements) is nibble j%2 of qs[32(j/2) .. +31] (ComputeOps.cs:1642-1675),
// so window w = sub-block w, and lane q reads qs[32g + 8q .. +7] for g < 4.
struct UQ4K {
    static constexpr int kBytes = 144, kBlocks = 1, kBlockElems = 256, SB = 32;
    static constexpr bool kOwnMin = true;       // o independent of k
    static constexpr float kSumScale = 1.f;
    struct Raw { u4 hdr; uint64_t qs[4]; };
    __device__ static void load(Rsrc r, uint32_t rowoff, int q, uint32_t so, int, Raw &w)
    {
        w.hdr = bld16(r, rowoff, so);
#pragma unroll
        for (int g = 0; g < 4; ++g) w.qs[g] = bld8(r, rowoff + 16 + 32 * g + 8 * q, so);
    }
    __device__ static void coef(const Raw &r, float *k, float *o)
    {
        const float d64 = f16_bits(r.hdr.x) * 0.015625f, dmin = f16_bits(r.hdr.x >> 16);   // codes enter as 64c
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // get_scale_min_k4 (QuantizationFormats.cs:157-165) on scales =
            // header bytes 4..15 (hdr.y = scales[0..3], .z = [4..7], .w = [8..11])
            const int sh = 8 * (j & 3);
            const uint32_t a = r.hdr.y >> sh, b = r.hdr.z >> sh, c = r.hdr.w >> sh;
            const uint32_t sc = j < 4 ? (a & 63u) : ((c & 0xFu) | ((a >> 2) & 0x30u));
            const uint32_t mn = j < 4 ? (b & 63u) : (((c >> 4) & 0xFu) | ((b >> 2) & 0x30u));
            k[j] = d64 * (float)sc;
            o[j] = dmin * (float)mn;
        }
    }
    __device__ static h8 code(const Raw &r, int w, int)
    {
        // the low (even w) or high nibble of each byte, as 64c
        const uint64_t v = r.qs[w >> 1];
        return (w & 1) ? frag((uint32_t)v, (uint32_t)(v >> 32), 2, 6, 0x03C003C0u)
                       : frag((uint32_t)v, (uint32_t)(v >> 32), 6, 2, 0x03C003C0u);
    }
};

// Q6_K unit = one super-block (ql[128], qh[64], scales[16] int8, d); element
// 128h + 32Q + l (l < 32) is nibble Q/2 of ql[64h + 32(Q%2) + l] with bits 2Q,
// 2Q+1 of qh[32h + l] above it (ComputeOps.cs:1748-1771): window w = (h, Q) =
// (w/4, w%4), sub-block (16 elements) 2w + q/2 for lane q.  The lane reads
// ql[64h + 32(Q%2) + 8q .. +7] (4 pieces), qh[32h + 8q .. +7] (2), the 16
// scales and d.
struct UQ6K {
    static constexpr int kBytes = 210, kBlocks = 1, kBlockElems = 256, SB = 16;
    static constexpr bool kOwnMin = false;      // o = 32 d sc = 512 k
    static constexpr float kSumScale = -512.f;
    struct Raw { uint64_t ql[4], qh[2]; u4 sc; uint32_t d; };
    __device__ static void load(Rsrc r, uint32_t rowoff, int q, uint32_t so, int, Raw &w)
    {
        // Units are 210 bytes: an odd unit starts at 2 mod 4 (rows at
        // multiples of 4).  Its pieces come from aligned loads 2 bytes lower,
        // funnel-shifted by 16 bits (by 0 for an even unit).
        const uint32_t sa = so & ~3u, sh = (so & 3u) * 8;
        auto piece = [&](uint32_t vo) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, vo, sa, 0);
            return (uint64_t)__builtin_amdgcn_alignbit(v[1], v[0], sh) |
                   ((uint64_t)__builtin_amdgcn_alignbit(v[2], v[1], sh) << 32);
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) w.ql[i] = piece(rowoff + 64 * (i >> 1) + 32 * (i & 1) + 8 * q);
#pragma unroll
        for (int h = 0; h < 2; ++h) w.qh[h] = piece(rowoff + 128 + 32 * h + 8 * q);
        const u4 s4 = bld16(r, rowoff + 192, sa);
        const uint32_t s5 = __builtin_amdgcn_raw_buffer_load_b32(r, rowoff + 208, sa, 0);
        w.sc = u4{__builtin_amdgcn_alignbit(s4.y, s4.x, sh), __builtin_amdgcn_alignbit(s4.z, s4.y, sh),
                  __builtin_amdgcn_alignbit(s4.w, s4.z, sh), __builtin_amdgcn_alignbit(s5, s4.w, sh)};
        w.d = bld2(r, rowoff + 208, so);
    }
    __device__ static void coef(const Raw &r, float *k, float *)
    {
        const float d16 = f16_bits(r.d) * 0.0625f;   // codes enter as 16c
        const uint32_t s[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) k[j] = d16 * (float)(int)__builtin_amdgcn_sbfe((int)s[j >> 2], 8 * (j & 3), 8);
    }
    __device__ static h8 code(const Raw &r, int w, int)
    {
        const int h = w >> 2, Q = w & 3;
        const uint64_t l = r.ql[2 * h + (Q & 1)], hb = r.qh[h];
        const uint32_t l0 = (uint32_t)l, l1 = (uint32_t)(l >> 32), h0 = (uint32_t)hb, h1 = (uint32_t)(hb >> 32);
        // 6-bit code as 16c: the quarter's nibble at bits 4..7 of the fp16
        // half, bits 2Q, 2Q+1 of the qh byte at bits 8, 9
        const uint32_t nsl = Q < 2 ? 4 : 0, nsr = Q < 2 ? 4 : 8, hsl = 8 - 2 * Q, hsr = 2 * Q;
        const uint32_t nm = 0x00F000F0u, hm = 0x03000300u;
        const u4 f = {and_or(h0 << hsl, hm, (l0 << nsl) & nm), and_or(h0 >> hsr, hm, (l0 >> nsr) & nm),
                      and_or(h1 << hsl, hm, (l1 << nsl) & nm), and_or(h1 >> hsr, hm, (l1 >> nsr) & nm)};
        return __builtin_bit_cast(h8, f);
    }
};

// Q8_0 unit = 8 blocks (d, qs[32] int8): window w = block w; lane q reads
// qs[8q .. +7] of every block and the 8 scales.  Codes biased by 128 (xor
// 0x80) are unsigned.
struct UQ80 {
    static constexpr int kBytes = 272, kBlocks = 8, kBlockElems = 32, SB = 32;
    static constexpr bool kOwnMin = false;      // o = 128 d = 512 k
    static constexpr float kSumScale = -512.f;
    struct Raw { uint64_t qs[8]; uint32_t d[8]; };
    __device__ static void load(Rsrc r, uint32_t rowoff, int q, uint32_t so, int nb, Raw &w)
    {
        // a block past the row's end (only in a last, partial unit) re-reads
        // the start of the unit, so no read leaves the row, and gets scale 0.
        // Rows and units start at multiples of 4 bytes (K is a multiple of
        // 64): the pieces of even blocks lie at 2 mod 4, those of odd ones
        // are aligned.
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t o = b < nb ? rowoff + 34 * b : rowoff;
            if (b % 2 == 0) w.qs[b] = bld8_at2(r, o + 8 * q, so);
            else w.qs[b] = bld8(r, b < nb ? o + 2 + 8 * q : o + 8 * q, so);
            w.d[b] = b < nb ? bld2(r, o, so) : 0u;
        }
    }
    __device__ static void coef(const Raw &r, float *k, float *)
    {
#pragma unroll
        for (int j = 0; j < 8; ++j) k[j] = 0.25f * f16_bits(r.d[j]);   // codes enter as 4(c + 128)
    }
    __device__ static h8 code(const Raw &r, int w, int)
    {
        const uint64_t v = r.qs[w] ^ 0x8080808080808080ull;
        return frag((uint32_t)v, (uint32_t)(v >> 32), 2, 6, 0x03FC03FCu);
    }
};

// Q4_0 unit = 8 blocks (d, qs[16]): in block w, elements j < 16 are the low
// nibbles of qs[j], elements 16 + j the high nibbles; lane q reads
// qs[8(q%2) .. +7] and takes the low (q < 2) or high (q >= 2) nibbles.
struct UQ40 {
    static constexpr int kBytes = 144, kBlocks = 8, kBlockElems = 32, SB = 32;
    static constexpr bool kOwnMin = false;      // o = 8 d = 512 k
    static constexpr float kSumScale = -512.f;
    struct Raw { uint64_t qs[8]; uint32_t d[8]; };
    __device__ static void load(Rsrc r, uint32_t rowoff, int q, uint32_t so, int nb, Raw &w)
    {
        // as Q8_0: even blocks' pieces at 2 mod 4, odd ones aligned
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t o = b < nb ? rowoff + 18 * b : rowoff;
            if (b % 2 == 0) w.qs[b] = bld8_at2(r, o + 8 * (q & 1), so);
            else w.qs[b] = bld8(r, b < nb ? o + 2 + 8 * (q & 1) : o + 8 * (q & 1), so);
            w.d[b] = b < nb ? bld2(r, o, so) : 0u;
        }
    }
    __device__ static void coef(const Raw &r, float *k, float *)
    {
#pragma unroll
        for (int j = 0; j < 8; ++j) k[j] = 0.015625f * f16_bits(r.d[j]);   // codes enter as 64c
    }
    __device__ static h8 code(const Raw &r, int w, int q)
    {
        // low nibbles for lanes q < 2, high nibbles for q >= 2, both as 64c
        const uint64_t v = r.qs[w];
        return q >= 2 ? frag((uint32_t)v, (uint32_t)(v >> 32), 2, 6, 0x03C003C0u)
                      : frag((uint32_t)v, (uint32_t)(v >> 32), 6, 2, 0x03C003C0u);
    }
};

// Workgroup barrier for LDS traffic only (waits for this wave's LDS
// operations, then for every wave); __syncthreads() would also drain the
// weight loads in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Maximum / sum of v over aligned groups of G lanes (G = 2, 4, 8 or 16),
// returned to every lane of the group.
template <int G>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    if constexpr (G >= 4) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    if constexpr (G >= 8) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    if constexpr (G >= 16) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v)
{
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);
    if constexpr (G >= 4) v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);
    return v;
}

// LDS image of one round (R units) of X: for every activation row (batch
// column, and the zero row ZROW) the round's 32R 8-element pieces, hi then lo
// halves, each piece in the order kPerm (and a pad piece); then per (column, group) the factor
// 2^24 / S and per (column, sub-block) the fp32 sum of x.
template <int R, int G, int SB>
struct Img {
    static constexpr int P = 32 * R;              // pieces per row
    static constexpr int NG = UNIT * R / G;       // groups per row
    static constexpr int NS = UNIT * R / SB;      // sub-blocks per row
    // rows padded by one piece: the 16 lanes of a k-block read one piece of
    // 8 different rows, which then fall on different banks
    h8 hi[MAXB + 1][P + 1];
    h8 lo[MAXB + 1][P + 1];
    // per-column rows of factors and sums, padded to whole 16-byte vectors
    // plus one (the lanes of a wave read the rows of 2 or 4 columns)
    static constexpr int NGP = (NG + 3) / 4 * 4 + 4, NSP = (NS + 3) / 4 * 4 + 4;
    float f[MAXB][NGP];
    float sx[MAXB][NSP];
};

// One round: units ub .. ub+R-1 of the split.  WHOLE: every unit lies inside
// the row (always for Q4_K/Q6_K; for Q8_0/Q4_0 all but a last partial unit),
// and the code is straight-line, so that every load of the round is issued
// before the first wait.  Otherwise R = 1 and the unit may be partial (nb
// blocks of it inside the row; elements past K are zero).  X piece c =
// tid + 256 j of the round is column c / (32 R), elements 8 (c % (32 R)) ..
// +7, at byte offset xo[j] + 1024 ub in xr.  lead: a previous round of this
// workgroup may still be reading the image.
template <class U, int T, int R, bool WHOLE>
__device__ __forceinline__ void round_of(Rsrc wr, uint32_t rowoff, Rsrc xr, const uint32_t *xo, int ub, int nb,
                                         int64_t K, int batch, Img<R, T * U::SB, U::SB> &im, bool lead, int tid,
                                         int q, const int *xrow, float *out)
{
    constexpr int SB = U::SB, G = T * SB, WPG = G / 32, NGU = UNIT / G, CPC = 32 * R;
    const uint32_t xso = (uint32_t)ub * (UNIT * 4);
    f4 xv[R][2];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int c = tid + TW * 64 * j, col = c / CPC, kc = c % CPC;
        xv[j][0] = xv[j][1] = f4{0.f, 0.f, 0.f, 0.f};
        if (col < batch && (WHOLE || (int64_t)ub * UNIT + 8 * kc < K)) {
            xv[j][0] = __builtin_bit_cast(f4, bld16(xr, xo[j], xso));
            xv[j][1] = __builtin_bit_cast(f4, bld16(xr, xo[j] + 16, xso));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    typename U::Raw rw[R];
#pragma unroll
    for (int u = 0; u < R; ++u) U::load(wr, rowoff, q, (uint32_t)(ub + u) * U::kBytes, WHOLE ? U::kBlocks : nb, rw[u]);
    __builtin_amdgcn_sched_barrier(0);
    if (lead) lds_barrier();
    if constexpr (!WHOLE) {
        // single-unit rounds use a smaller layout of the same LDS: its zero
        // row lies in the rows of the larger one
        for (int p = tid; p < Img<R, G, SB>::P; p += TW * 64) {
            im.hi[ZROW][p] = h8{};
            im.lo[ZROW][p] = h8{};
        }
    }
    // Stage: per piece the group's max|x| (G/8 neighbouring lanes hold the
    // pieces of one group of one column), the power of two S, hi and lo, and
    // the sub-block sums (SB/8 lanes).  Every lane takes part in the lane
    // reductions; only pieces of real columns are stored.
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int c = tid + TW * 64 * j, col = c / CPC, kc = c % CPC;
        const float v[8] = {xv[j][0].x, xv[j][0].y, xv[j][0].z, xv[j][0].w,
                            xv[j][1].x, xv[j][1].y, xv[j][1].z, xv[j][1].w};
        uint32_t m = 0;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            m = max(m, __float_as_uint(v[i]) & 0x7FFFFFFFu);
            s += v[i];
        }
        m = group_max_u32<G / 8>(m);
        s = group_sum<SB / 8>(s);
        // S = 2^(140 - e) for the biased exponent e of the group max, clamped
        // to [13, 243] (S and 2^24 / S = 2^(e - 116) stay normal); inf or NaN
        // in the group makes 2^24 / S NaN.  A group max of 2^117 or more
        // overflows fp16.
        const int e0 = (int)(m >> 23), e = e0 < 13 ? 13 : e0 > 243 ? 243 : e0;
        const float S = __uint_as_float((uint32_t)(267 - e) << 23);
        const float fs = e0 == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float((uint32_t)(e + 11) << 23);
        h8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = v[kPerm[i]] * S;
            hi[i] = (_Float16)x;
            lo[i] = (_Float16)(x - (float)hi[i]);
        }
        if (col < batch) {
            im.hi[col][kc] = hi;
            im.lo[col][kc] = lo;
            if (kc % (G / 8) == 0) im.f[col][kc / (G / 8)] = fs;
            if (kc % (SB / 8) == 0) im.sx[col][kc / (SB / 8)] = U::kSumScale * s;
        }
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);   // keep the codes and MFMAs after the barrier
    // lane (n, q'): MFMA rows i = 4q' + r, i.e. column q' * NB + r / T and
    // sub-block r % T of each group
    constexpr int NB = 4 / T, NSB = UNIT / SB;
    const int q4 = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        float k[NSB], o[NSB];
        U::coef(rw[u], k, o);
        // the factors 2^24 / S of the unit's groups and the sums of its
        // sub-blocks, for the lane's columns
        float fv[NB][NGU], sv[NB][NSB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b = q4 * NB + j;
#pragma unroll
            for (int g = 0; g < NGU; ++g) fv[j][g] = im.f[b][u * NGU + g];
#pragma unroll
            for (int t = 0; t < NSB; ++t) sv[j][t] = im.sx[b][u * NSB + t];
        }
#pragma unroll
        for (int g = 0; g < NGU; ++g) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int wg = 0; wg < WPG; ++wg) {
                const int w = g * WPG + wg;
                const h8 c = U::code(rw[u], w, q);
                const int piece = u * 32 + w * 4 + q;
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(im.lo[xrow[wg]][piece], c, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(im.hi[xrow[wg]][piece], c, acc, 0, 0, 0);
            }
            // rows of columns past the batch hold zeros times stale factors:
            // computed, never stored
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = r / T, sb = g * T + r % T;
                if constexpr (U::kOwnMin)
                    out[r] = __builtin_fmaf(k[sb], acc[r] * fv[j][g], __builtin_fmaf(-o[sb], sv[j][sb], out[r]));
                else   // o = -kSumScale * k: the staged sums carry the factor
                    out[r] = __builtin_fmaf(k[sb], __builtin_fmaf(acc[r], fv[j][g], sv[j][sb]), out[r]);
            }
        }
    }
}

// Workgroup g: row tile g % ntiles, split g / ntiles, units [split * per,
// min(nunits, (split + 1) * per)) in rounds of UPW units (then single units).
// P != nullptr: partial sums of the split to P[(split * batch + b) * np + n];
// else Y directly.
template <class U, int T, int UPW>
__global__ void __launch_bounds__(TW * 64)
qmv_split_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes, const float *__restrict__ X,
                 int64_t ldx, int batch, int ntiles, int per, float *__restrict__ P, int64_t np,
                 float *__restrict__ Y, int64_t ldy)
{
    constexpr int SB = U::SB, G = T * SB, WPG = G / 32;
    __shared__ __align__(16) Img<UPW, G, SB> im;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n16 = lane & 15, q = lane >> 4;
    const int tile = (int)(blockIdx.x % (unsigned)ntiles), split = (int)(blockIdx.x / (unsigned)ntiles);
    const int64_t nblk = K / U::kBlockElems;                      // blocks per row
    const int nunits = (int)((nblk + U::kBlocks - 1) / U::kBlocks);
    const int ua = split * per, ue = min(nunits, ua + per);
    // a last unit only partly inside the row (Q8_0/Q4_0) goes to the single-unit path
    const int ue_whole = (ue == nunits && nblk % U::kBlocks) ? ue - 1 : ue;
    // weights: a resource over the tile's rows (rows past N read as the last)
    const int64_t row0 = (int64_t)tile * RWG;
    const int rows = (int)min<int64_t>(RWG, N - row0);
    const Rsrc wr = make_rsrc(W + row0 * row_bytes, (uint32_t)(rows * row_bytes));
    const int rr = min(16 * wave + n16, rows - 1);
    const uint32_t rowoff = (uint32_t)(rr * row_bytes);
    // activations: a resource over X, a lane's piece offsets for every round
    const Rsrc xr = make_rsrc(X, (uint32_t)(((int64_t)(batch - 1) * ldx + K) * 4));
    uint32_t xo[UPW];
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
        const int c = tid + TW * 64 * j, col = c / (32 * UPW), kc = c % (32 * UPW);
        xo[j] = (uint32_t)(((int64_t)min(col, batch - 1) * ldx + 8 * kc) * 4);
    }
    uint32_t xo1[1];
    {
        const int col = tid / 32, kc = tid % 32;
        xo1[0] = (uint32_t)(((int64_t)min(col, batch - 1) * ldx + 8 * kc) * 4);
    }
    // MFMA row i = n16 of this lane's A fragments: (column i / T, sub-block
    // i % T); in window wg of a group it reads its column's activations when
    // lane q's 8 elements lie in sub-block i % T, else the zero row
    int xrow[WPG];
#pragma unroll
    for (int wg = 0; wg < WPG; ++wg) {
        const int b = n16 / T, t = n16 % T, s = (32 * wg + 8 * q) / SB;
        xrow[wg] = (s == t && b < batch) ? b : ZROW;
    }
    // the zero row of the image (never written by the staging)
    for (int p = tid; p < Img<UPW, G, SB>::P; p += TW * 64) {
        im.hi[ZROW][p] = h8{};
        im.lo[ZROW][p] = h8{};
    }

    float out[4] = {0.f, 0.f, 0.f, 0.f};
    int ub = ua;
    for (; ub + UPW <= ue_whole; ub += UPW)
        round_of<U, T, UPW, true>(wr, rowoff, xr, xo, ub, U::kBlocks, K, batch, im, ub != ua, tid, q, xrow, out);
    for (; ub < ue; ++ub) {
        const int nb = (int)min<int64_t>(U::kBlocks, nblk - (int64_t)ub * U::kBlocks);
        round_of<U, T, 1, false>(wr, rowoff, xr, xo1, ub, nb, K, batch,
                                 *reinterpret_cast<Img<1, G, SB> *>(&im), ub != ua, tid, q, xrow, out);
    }

    // out[r] = row 4q + r = (column (4q + r) / T, sub-block (4q + r) % T) of
    // weight row n16: add the sub-blocks of each column
    const int64_t n = row0 + 16 * wave + n16;
    if (n < N) {
#pragma unroll
        for (int r = 0; r < 4; r += T < 4 ? T : 4) {
            float s = 0.f;
#pragma unroll
            for (int t = 0; t < (T < 4 ? T : 4); ++t) s += out[r + t];
            const int b = (4 * q + r) / T;
            if (b < batch) {
                if (P) P[((int64_t)split * batch + b) * np + n] = s;
                else Y[(int64_t)b * ldy + n] = s;
            }
        }
    }
}

// Y[b * ldy + n] = sum over s = 0 .. S-1, in order, of P[(s * batch + b) * np + n];
// one thread per output, the loads of up to 16 splits issued together.
__global__ void __launch_bounds__(256)
split_sum_kernel(const float *__restrict__ P, int64_t np, int S, int batch, int64_t N,
                 float *__restrict__ Y, int64_t ldy)
{
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int col = (int)(t / np);
    const int64_t n = t - (int64_t)col * np;
    if (col >= batch || n >= N) return;
    const float *p = P + (int64_t)col * np + n;
    const int64_t stride = (int64_t)batch * np;
    float s = 0.f;
    for (int j0 = 0; j0 < S; j0 += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = j0 + j < S ? p[(int64_t)(j0 + j) * stride] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (j0 + j < S) s = j0 + j == 0 ? v[j] : s + v[j];
    }
    Y[(int64_t)col * ldy + n] = s;
}

template <class U, int T>
int launch_t(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
             const float *X, int64_t ldx, float *Y, int64_t ldy, int batch, const aih_scratch *ext)
{
    const int64_t ntiles = (N + RWG - 1) / RWG;
    const int64_t nblk = K / U::kBlockElems;
    const int64_t nunits = (nblk + U::kBlocks - 1) / U::kBlocks;
    if (ntiles > 0x7FFFFFFF || nunits > 0x7FFFFFFF) return AIH_E_LIMIT;
    // buffer resources: a tile's rows and all of X within 31-bit offsets
    if (RWG * row_bytes > 0x7FFFFFFF || ((int64_t)(batch - 1) * ldx + K) * 4 > 0x7FFFFFFF) return AIH_E_LIMIT;
    // Splits of K: at least about two workgroups per CU (four waves each),
    // and at least min(8, units / 2) splits, since small per-workgroup K
    // ranges measured faster at every shape but the widest K (per call on
    // MI355X, 8 columns: Q4_0 14336 x 4096 41.2 -> 32.6 us, Q4_K 14336 x 4096
    // 22.2 -> 20.1 us, the Q6_K 32000 x 4096 head at 5 columns 42.2 -> 39.7
    // us; Q6_K 4096 x 14336 keeps its 8 splits of 7 units).  The partial sums stay
    // within the allocation-free entry point's buffer, so that both entry
    // points split a shape alike.
    const int64_t cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int64_t np = ntiles * RWG;
    int64_t S = std::max<int64_t>((2 * cu + ntiles - 1) / ntiles, std::min<int64_t>(8, (nunits + 1) / 2));
    S = std::min<int64_t>(S, nunits);
    S = std::max<int64_t>(1, std::min<int64_t>(S, (int64_t)(AIH_NOALLOC_SCRATCH_BYTES / ((size_t)batch * np * sizeof(float)))));
    int64_t per = (nunits + S - 1) / S;
    S = (nunits + per - 1) / per;
    float *P = nullptr;
    if (S > 1) {
        void *ws = nullptr;
        const int st = aih_stage(ctx, ext, (size_t)(S * batch * np) * sizeof(float), &ws);
        if (st == AIH_OK) {
            P = static_cast<float *>(ws);
        } else if (st == AIH_E_LIMIT && !ext) {
            // the workspace cannot grow during graph capture: one split per row tile
            S = 1;
            per = nunits;
        } else {
            return st;
        }
    }
    if (ntiles * S > 0x7FFFFFFF) return AIH_E_LIMIT;
    const dim3 grid((unsigned)(ntiles * S)), block(TW * 64);
    const int nt = (int)ntiles, pr = (int)per;
    if (per >= 4)
        hipLaunchKernelGGL((qmv_split_kernel<U, T, 4>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    else if (per >= 2)
        hipLaunchKernelGGL((qmv_split_kernel<U, T, 2>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    else
        hipLaunchKernelGGL((qmv_split_kernel<U, T, 1>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    int st = aih_launch_status();
    if (st != AIH_OK || !P) return st;
    const int64_t threads = (int64_t)batch * np;
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, ctx->stream,
                       P, np, (int)S, batch, N, Y, ldy);
    return aih_launch_status();
}

// 3..4 columns: four sub-blocks per column in the 16 MFMA rows; 5..8: two
template <class U>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
           const float *X, int64_t ldx, float *Y, int64_t ldy, int batch, const aih_scratch *ext)
{
    return batch <= 4 ? launch_t<U, 4>(ctx, W, N, K, row_bytes, X, ldx, Y, ldy, batch, ext)
                      : launch_t<U, 2>(ctx, W, N, K, row_bytes, X, ldx, Y, ldy, batch, ext);
}

}  // namespace

int aih_launch_qmatvec_mfma(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                            const float *X, int64_t ldx, float *Y, int64_t ldy, int batch, const aih_scratch *ext)
{
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch<UQ4K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, ext);
    case AIH_TYPE_Q6_K: return launch<UQ6K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, ext);
    case AIH_TYPE_Q8_0: return launch<UQ80>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, ext);
    case AIH_TYPE_Q4_0: return launch<UQ40>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, ext);
    default: return AIH_E_UNSUPPORTED;
    }
}
