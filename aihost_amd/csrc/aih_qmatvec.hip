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
// Work split.  K is cut into 64-element "units"; lane u of a row team owns
// unit u of every row it visits (a Q4_K (block, 64-group), a pair of Q8_0/Q4_0
// blocks, or a Q6_K (block, half, 16-column) slice).  A team is
// ceil(K/64 / 64) waves; a workgroup holds several teams that work on
// different rows, and the host launches one workgroup per CU.  The workgroup
// converts the activations once into an fp16 "image" in LDS (every thread
// converts a few 16-byte pieces); per row a lane reads the 32 image dwords of
// its unit with eight conflict-free 16-byte LDS reads.  Each wave walks its
// rows with a two-deep register pipeline (the next row's packed bytes are in
// flight while the current row is computed).  Partial sums are reduced with
// DPP inside a wave and through LDS across the waves of a team; row results
// stay in registers until the end of the launch.
//
// Arithmetic (fp32-equivalent).  Each workgroup turns x, per 64-element unit,
// into integers: X = round(x * S) with a power of two S = 2^(148 - e) chosen
// from the unit's max|x| (biased exponent e), so that |X| < 2^22, and writes X
// as three balanced signed-byte limbs (X = d0 + 2^8 d1 + 2^16 d2).  A weight
// code (4-bit, 6-bit, or the int8 of Q8_0) masked out of its packed word
// multiplies each limb exactly with v_dot4_i32_i8, four code/limb pairs per
// instruction, the products summed exactly in int32 per sub-block.  The limb
// sums are combined in fp32 (A0 + 2^8 A1 + 2^16 A2), the format's offset
// (-8 for Q4_0, -32 for Q6_K) enters as offset * sum(x) (sum of the scaled
// x, in fp32), the sub-block scales and mins are applied in fp32:
//   Q4_K: d*sc*S - dmin*mn*X      (S = sum q*x, X = sum x over the sub-block)
//   Q6_K: d*sc*sum((q-32)*x)      Q8_0: d*sum(q*x)      Q4_0: d*sum((q-8)*x)
// and each unit's contribution is multiplied by 1/S.  The fused
// multiply-adds are written out (the file is compiled with
// -ffp-contract=off), so every column is computed by the same instructions.
// The normwise error against an fp64 product is about 1e-6, against the
// reference's sequential fp32 product 1e-6 to 5e-6 (that product's own
// error).
#include "aih_internal.h"

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// (a & mask) | b as one v_and_or_b32.  Written out because VOP3 encodings on
// this architecture take no literal operand and read at most one scalar
// register, so with a literal mask the compiler emits a v_and_b32 + v_or_b32
// pair instead.  Here the mask travels in an SGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t b)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(b));
    return r;
}
__device__ __forceinline__ float f16lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu)); }
__device__ __forceinline__ float f16hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

template <class T>
__device__ __forceinline__ T ldg(const void *p)
{
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// Row addressing for the weight loads, in two forms with the same interface
// (16/8/4/2-byte loads at a 32-bit byte offset):
//   PtrRow - a per-lane 64-bit pointer to the row; offsets are added to it.
//   BufRow - a buffer resource over the launch's slice of W, with the row's
//            32-bit offset in a scalar register (soffset) and the lane offset
//            in a vector register (voffset): no 64-bit address arithmetic on
//            the vector ALUs.  Accesses past num_records read zeros.  Word 3
//            (0x00020000) is the raw-buffer configuration of the gfx9 family.
// Single-wave teams use PtrRow and multi-wave teams BufRow: on MI355X the
// buffer form ran 0.85 us faster on Q6_K 4096 x 14336 (four-wave teams) but
// 0.2 us slower on the single-wave-team kernel for matrices of 7-14k rows
// (any form with the row base in a scalar register did).
struct PtrRow {
    const uint8_t *p;
    __device__ __forceinline__ u4 ld16(uint32_t o) const { return ldg<u4>(p + o); }
    __device__ __forceinline__ uint64_t ld8(uint32_t o) const { return ldg<uint64_t>(p + o); }
    __device__ __forceinline__ uint32_t ld4(uint32_t o) const { return ldg<uint32_t>(p + o); }
    __device__ __forceinline__ uint32_t ld2(uint32_t o) const { return ldg<uint16_t>(p + o); }
};
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const uint8_t *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, (int)bytes, 0x00020000);
}
struct BufRow {
    Rsrc r;
    uint32_t soff;
    __device__ __forceinline__ u4 ld16(uint32_t o) const { return __builtin_amdgcn_raw_buffer_load_b128(r, o, soff, 0); }
    __device__ __forceinline__ uint64_t ld8(uint32_t o) const
    {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, o, soff, 0);
        return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
    }
    __device__ __forceinline__ uint32_t ld4(uint32_t o) const { return __builtin_amdgcn_raw_buffer_load_b32(r, o, soff, 0); }
    __device__ __forceinline__ uint32_t ld2(uint32_t o) const { return __builtin_amdgcn_raw_buffer_load_b16(r, o, soff, 0); }
};

// One prep step turns 4 consecutive activations x[src..src+3] (one 16-byte
// load) into their three limb words (word `step` of each limb image of the
// unit; see convert_step) and adds their fp32 sum to sum slot `slot`.  A unit
// needs 16 steps; the step's place in the unit and its slot depend only on
// the step.  A limb image
// is 16 words in 4 groups of 4 steps that a format's dot product reads one
// group (one 16-byte read) at a time: group(b, l, i) is group i of limb l of
// column b.
struct Step {
    int src;
    int slot;
};

// Signed 8-bit integer dot product of four byte pairs, accumulated in int32
// (v_dot4_i32_i8): exact.
__device__ __forceinline__ int sdot4(uint32_t codes, uint32_t limb, int acc)
{
    return __builtin_amdgcn_sdot4((int)codes, (int)limb, acc, false);
}

// sum over the three limbs of one code stream (limb l holds digit l, of
// weight 2^(8l)): A0 + 2^8 A1 + 2^16 A2 as fp32 (each term is exact in fp32;
// the sum is rounded once or twice)
__device__ __forceinline__ float limbs_f(const int *a)
{
    return __builtin_fmaf((float)a[2], 65536.f, __builtin_fmaf((float)a[1], 256.f, (float)a[0]));
}

// ---------------------------------------------------------------- Q4_K ----
// Unit u: block u/4, 64-group g = u%4 -> qs bytes 32g..32g+31 of the block,
// low nibbles are sub-block 2g (k0 + 0..31), high nibbles sub-block 2g+1
// (k0 + 32..63), k0 = 64u.  (Element order: ComputeOps.cs:1642-1675.)
// qs word k (k < 8) holds the low-nibble codes of elements 4k..4k+3 (step k)
// and the high-nibble codes of elements 32+4k.. (step 8+k).
// Sums: 0 low sub-block, 1 high sub-block.
struct Q4K {
    static constexpr int kRaw = 12;
    static constexpr int kSums = 2;
    __device__ static Step step(int u, int s) { return {64 * u + 4 * s, s >> 3}; }
    // unit and step of the 4 activations x[4e .. 4e+3] (step(u, s).src == 4e)
    __device__ static void inv(int e, int &u, int &s) { u = e >> 4; s = e & 15; }
    // The row starts at byte `off` of `w`; lane offsets are added to off.
    template <class A>
    __device__ static void load(const A &w, uint32_t off, int u, uint32_t *raw)
    {
        const uint32_t o = off + (uint32_t)(u >> 2) * 144u, oq = o + 16u + (uint32_t)(u & 3) * 32u;
        u4 h = w.ld16(o), qa = w.ld16(oq), qb = w.ld16(oq + 16u);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = qa.x; raw[5] = qa.y; raw[6] = qa.z; raw[7] = qa.w;
        raw[8] = qb.x; raw[9] = qb.y; raw[10] = qb.z; raw[11] = qb.w;
    }
    template <int B, class XA>
    __device__ static void dot(const uint32_t *raw, const XA &xa, int u, float *out)
    {
        // 6-bit (scale, min) of sub-blocks 2g and 2g+1 (get_scale_min_k4,
        // QuantizationFormats.cs:157-165), branch-free per lane.
        const int g = u & 3;
        const bool upper = g >= 2;
        const uint32_t s0 = (g & 1) * 16;
        const uint32_t wlo = upper ? 4u : 6u, whi = upper ? 2u : 0u, moff = upper ? 4u : 0u;
        const uint32_t a_sc = upper ? raw[3] : raw[1], a_mn = upper ? raw[3] : raw[2];
        const uint32_t sc0 = __builtin_amdgcn_ubfe(a_sc, s0, wlo) | (__builtin_amdgcn_ubfe(raw[1], s0 + 6, whi) << 4);
        const uint32_t sc1 = __builtin_amdgcn_ubfe(a_sc, s0 + 8, wlo) | (__builtin_amdgcn_ubfe(raw[1], s0 + 14, whi) << 4);
        const uint32_t mn0 = __builtin_amdgcn_ubfe(a_mn, s0 + moff, wlo) | (__builtin_amdgcn_ubfe(raw[2], s0 + 6, whi) << 4);
        const uint32_t mn1 = __builtin_amdgcn_ubfe(a_mn, s0 + 8 + moff, wlo) | (__builtin_amdgcn_ubfe(raw[2], s0 + 14, whi) << 4);
        const float d = f16lo(raw[0]), dmin = f16hi(raw[0]);
        const float fsc0 = (float)sc0, fsc1 = (float)sc1, fmn0 = (float)mn0, fmn1 = (float)mn1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            int lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const u4 gl[3] = {xa.group(b, 0, i), xa.group(b, 1, i), xa.group(b, 2, i)};
                const u4 gh[3] = {xa.group(b, 0, 2 + i), xa.group(b, 1, 2 + i), xa.group(b, 2, 2 + i)};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = raw[4 + 4 * i + j];
                    const uint32_t cl = w & 0x0F0F0F0Fu, ch = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int l = 0; l < 3; ++l) {
                        lo[l] = sdot4(cl, gl[l][j], lo[l]);
                        hi[l] = sdot4(ch, gh[l][j], hi[l]);
                    }
                }
            }
            const float s = __builtin_fmaf(fsc0, limbs_f(lo), fsc1 * limbs_f(hi));
            const float m = __builtin_fmaf(fmn0, xa.sum(b, 0), fmn1 * xa.sum(b, 1));
            out[b] = __builtin_fmaf(__builtin_fmaf(d, s, -dmin * m), xa.inv(b), out[b]);
        }
    }
};

// ---------------------------------------------------------------- Q8_0 ----
// Unit u: blocks 2u and 2u+1 (68 bytes, 4-byte aligned), k0 = 64u.
// Block A: d at byte 0, qs at 2..33 (realigned with alignbyte); block B: d at
// 34..35, qs at 36..67.  The int8 codes enter the dot products as they are.
// Code word m of block A (elements 4m..4m+3) is step m, of block B step 8+m.
struct Q80 {
    static constexpr int kRaw = 17;
    static constexpr int kSums = 1;
    __device__ static Step step(int u, int s) { return {64 * u + 4 * s, 0}; }
    __device__ static void inv(int e, int &u, int &s) { u = e >> 4; s = e & 15; }
    template <class A>
    __device__ static void load(const A &w, uint32_t off, int u, uint32_t *raw)
    {
        const uint32_t o = off + (uint32_t)u * 68u;
        u4 v0 = w.ld16(o), v1 = w.ld16(o + 16u), v2 = w.ld16(o + 32u), v3 = w.ld16(o + 48u);
        raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
        raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
        raw[8] = v2.x; raw[9] = v2.y; raw[10] = v2.z; raw[11] = v2.w;
        raw[12] = v3.x; raw[13] = v3.y; raw[14] = v3.z; raw[15] = v3.w;
        raw[16] = w.ld4(o + 64u);
    }
    template <int B, class XA>
    __device__ static void dot(const uint32_t *raw, const XA &xa, int, float *out)
    {
        const float dA = f16lo(raw[0]), dB = f16hi(raw[8]);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            int aA[3] = {0, 0, 0}, aB[3] = {0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u4 gr[3] = {xa.group(b, 0, i), xa.group(b, 1, i), xa.group(b, 2, i)};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int s = 4 * i + j;   // step: code word s % 8 of block s / 8
                    const uint32_t c = s < 8 ? __builtin_amdgcn_alignbyte(raw[s + 1], raw[s], 2) : raw[s + 1];
                    int *acc = s < 8 ? aA : aB;
#pragma unroll
                    for (int l = 0; l < 3; ++l) acc[l] = sdot4(c, gr[l][j], acc[l]);
                }
            }
            out[b] = __builtin_fmaf(__builtin_fmaf(dA, limbs_f(aA), dB * limbs_f(aB)), xa.inv(b), out[b]);
        }
    }
};

// ---------------------------------------------------------------- Q4_0 ----
// Unit u: blocks 2u and 2u+1 (36 bytes, 4-byte aligned), k0 = 64u.  In each
// block qs[j] holds element j (low nibble) and j+16 (high nibble): qs word i
// (i < 4) of block A holds the codes of steps i (low) and 4+i (high), of
// block B steps 8+i and 12+i.  Sums: block A, block B.
struct Q40 {
    static constexpr int kRaw = 9;
    static constexpr int kSums = 2;
    __device__ static Step step(int u, int s) { return {64 * u + 4 * s, s >> 3}; }
    __device__ static void inv(int e, int &u, int &s) { u = e >> 4; s = e & 15; }
    template <class A>
    __device__ static void load(const A &w, uint32_t off, int u, uint32_t *raw)
    {
        const uint32_t o = off + (uint32_t)u * 36u;
        u4 v0 = w.ld16(o), v1 = w.ld16(o + 16u);
        raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
        raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
        raw[8] = w.ld4(o + 32u);
    }
    template <int B, class XA>
    __device__ static void dot(const uint32_t *raw, const XA &xa, int, float *out)
    {
        const float d[2] = {f16lo(raw[0]), f16hi(raw[4])};
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float t = 0.f;
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
                // sum((q-8)*x) over the block: the offset enters as -8 * sum(x)
                int a[3] = {0, 0, 0};
                const u4 gl[3] = {xa.group(b, 0, 2 * blk), xa.group(b, 1, 2 * blk), xa.group(b, 2, 2 * blk)};
                const u4 gh[3] = {xa.group(b, 0, 2 * blk + 1), xa.group(b, 1, 2 * blk + 1),
                                  xa.group(b, 2, 2 * blk + 1)};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t w = blk == 0 ? __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2) : raw[5 + i];
                    const uint32_t cl = w & 0x0F0F0F0Fu, ch = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int l = 0; l < 3; ++l) {
                        a[l] = sdot4(cl, gl[l][i], a[l]);
                        a[l] = sdot4(ch, gh[l][i], a[l]);
                    }
                }
                t = __builtin_fmaf(d[blk], __builtin_fmaf(-8.f, xa.sum(b, blk), limbs_f(a)), t);
            }
            out[b] = __builtin_fmaf(t, xa.inv(b), out[b]);
        }
    }
};

// ---------------------------------------------------------------- Q6_K ----
// Unit u: block u/4, half h = (u/2)%2, column group t = u%2.  The lane reads
// ql[64h+16t .. +15] (quarters 0 and 2), ql[64h+32+16t .. +15] (quarters 1
// and 3) and qh[32h+16t .. +15] (high 2 bits of all four quarters), i.e.
// elements 128h + 32*quarter + 16t + i, i < 16 (ComputeOps.cs:1748-1771).
// Each quarter's 16 elements form one sub-block with an int8 scale; code
// word m (elements 4m..4m+3) of quarter Q is step 4Q + m.  Sums: one per
// quarter.
struct Q6K {
    static constexpr int kRaw = 15;
    static constexpr int kSums = 4;
    __device__ static Step step(int u, int s)
    {
        const int q = s >> 2, m = s & 3;
        const int base = (u >> 2) * 256 + 128 * ((u >> 1) & 1) + 16 * (u & 1);
        return {base + 32 * q + 4 * m, q};
    }
    // f4 index jb = 32h + 8q + 4t + m within the 256-element block
    __device__ static void inv(int e, int &u, int &s)
    {
        const int jb = e & 63;
        u = 4 * (e >> 6) + 2 * (jb >> 5) + ((jb >> 2) & 1);
        s = 4 * ((jb >> 3) & 3) + (jb & 3);
    }
    template <class A>
    __device__ static void load(const A &w, uint32_t off, int u, uint32_t *raw)
    {
        const uint32_t o = off + (uint32_t)(u >> 2) * 210u, h = (uint32_t)(u >> 1) & 1u, t = (uint32_t)u & 1u;
        const uint32_t oq = o + 64u * h + 16u * t;
        u4 qa = w.ld16(oq), qb = w.ld16(oq + 32u);
        u4 qh = w.ld16(o + 128u + 32u * h + 16u * t);
        const uint64_t sc = w.ld8(o + 192u + 8u * h);
        raw[0] = qa.x; raw[1] = qa.y; raw[2] = qa.z; raw[3] = qa.w;
        raw[4] = qb.x; raw[5] = qb.y; raw[6] = qb.z; raw[7] = qb.w;
        raw[8] = qh.x; raw[9] = qh.y; raw[10] = qh.z; raw[11] = qh.w;
        raw[12] = (uint32_t)sc; raw[13] = (uint32_t)(sc >> 32);
        raw[14] = w.ld2(o + 208u);
    }
    template <int B, class XA>
    __device__ static void dot(const uint32_t *raw, const XA &xa, int u, float *out)
    {
        const uint32_t t8 = (u & 1) * 8;
        // int8 sub-block scales (signed extract, then signed conversion)
        const float sc[4] = {(float)(int)__builtin_amdgcn_sbfe((int)raw[12], t8, 8),
                             (float)(int)__builtin_amdgcn_sbfe((int)raw[12], t8 + 16, 8),
                             (float)(int)__builtin_amdgcn_sbfe((int)raw[13], t8, 8),
                             (float)(int)__builtin_amdgcn_sbfe((int)raw[13], t8 + 16, 8)};
        const float d = f16lo(raw[14]);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float s = 0.f;
#pragma unroll
            for (int Q = 0; Q < 4; ++Q) {
                int a[3] = {0, 0, 0};
                const u4 gr[3] = {xa.group(b, 0, Q), xa.group(b, 1, Q), xa.group(b, 2, Q)};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    // 6-bit codes: nibble Q/2 of the quarter's ql word, bits
                    // 2Q, 2Q+1 of the qh word at bits 4, 5
                    const uint32_t l = (Q & 1) ? raw[4 + m] : raw[m], hb = raw[8 + m];
                    const uint32_t nib = (Q >> 1) ? (l >> 4) & 0x0F0F0F0Fu : l & 0x0F0F0F0Fu;
                    const uint32_t hsh = Q == 0 ? hb << 4 : Q == 1 ? hb << 2 : Q == 2 ? hb : hb >> 2;
                    const uint32_t c = and_or(hsh, 0x30303030u, nib);
#pragma unroll
                    for (int li = 0; li < 3; ++li) a[li] = sdot4(c, gr[li][m], a[li]);
                }
                s = __builtin_fmaf(sc[Q], __builtin_fmaf(-32.f, xa.sum(b, Q), limbs_f(a)), s);
            }
            out[b] = __builtin_fmaf(d * s, xa.inv(b), out[b]);
        }
    }
};

// Per-unit activation scale.  From the biased exponent e of max|x| over the
// unit's 64 activations (x after any fused prologue; e = 255 for inf or NaN),
// clamped to [22, 254]: every activation of the unit becomes the integer
// X = round(x * S), S = 2^(148 - e), so that |X| < 2^22 (the largest lands in
// [2^21, 2^22]).  Products of codes and X are summed exactly in int32; the
// unit's contribution to a row is multiplied by 1/S = 2^(e - 148).  S and 1/S
// are built from their exponent fields (exact, normal fp32 over the clamped
// range).  A non-finite activation makes every row NaN (1/S = NaN).
struct ColScale {
    float s, inv_s;
};
__device__ __forceinline__ ColScale col_scale(uint32_t maxabs_bits)
{
    const int e0 = (int)(maxabs_bits >> 23);
    const int e = e0 < 22 ? 22 : e0 > 254 ? 254 : e0;
    return {__uint_as_float((uint32_t)(275 - e) << 23),
            e0 == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float((uint32_t)(e - 21) << 23)};
}

// Limb words of one step's 4 activations.  Y = round(x * S) + 0x808080 lies
// in [0, 2^24); byte l of Y minus 128 (byte XOR 0x80) is the balanced signed
// digit d_l, with X = d_0 + 2^8 d_1 + 2^16 d_2 (|d_2| <= 64).  Limb word l
// packs d_l of x0..x3 as four int8 (x0 in the low byte), the operand layout
// of v_dot4_i32_i8.
__device__ __forceinline__ void convert_step(f4 v, float S, uint32_t &w0, uint32_t &w1, uint32_t &w2)
{
    const uint32_t ya = (uint32_t)__builtin_rintf(__builtin_fmaf(v.x, S, 8421504.f));
    const uint32_t yb = (uint32_t)__builtin_rintf(__builtin_fmaf(v.y, S, 8421504.f));
    const uint32_t yc = (uint32_t)__builtin_rintf(__builtin_fmaf(v.z, S, 8421504.f));
    const uint32_t yd = (uint32_t)__builtin_rintf(__builtin_fmaf(v.w, S, 8421504.f));
    const uint32_t ab = __builtin_amdgcn_perm(yb, ya, 0x05010400u);   // a0 b0 a1 b1
    const uint32_t cd = __builtin_amdgcn_perm(yd, yc, 0x05010400u);   // c0 d0 c1 d1
    const uint32_t ab2 = __builtin_amdgcn_perm(yb, ya, 0x0c0c0602u);  // a2 b2 0 0
    const uint32_t cd2 = __builtin_amdgcn_perm(yd, yc, 0x0c0c0602u);  // c2 d2 0 0
    w0 = __builtin_amdgcn_perm(cd, ab, 0x05040100u) ^ 0x80808080u;
    w1 = __builtin_amdgcn_perm(cd, ab, 0x07060302u) ^ 0x80808080u;
    w2 = __builtin_amdgcn_perm(cd2, ab2, 0x05040100u) ^ 0x80808080u;
}
__device__ __forceinline__ float sum4(f4 v) { return (v.x + v.y) + (v.z + v.w); }

// Limb images of one unit in registers (a single row team whose image does
// not fit in LDS converts its own; with one column, the LDS image is copied
// into them), with the unit's step sums (pre-scaled by S) and 1/S.
template <int B, int S>
struct XRegs {
    u4 g[B][3][4];
    float s[B][S];
    float iv[B];
    __device__ __forceinline__ u4 group(int b, int l, int i) const { return g[b][l][i]; }
    __device__ __forceinline__ float sum(int b, int k) const { return s[b][k]; }
    __device__ __forceinline__ float inv(int b) const { return iv[b]; }
};

// Limb images in LDS, shared by the teams of a workgroup (one entry per unit,
// i.e. per lane of a team).  Laid out unit-minor so that the lanes of a wave
// touch consecutive LDS words: group i (16 bytes) of limb l of unit u for
// column b is entry ((b*3 + l)*4 + i)*tt + u of the group array, step sum s
// (times S) is entry (b*16 + s)*tt + u of the sum array that follows, and 1/S
// entry b*tt + u of the scale array after it (tt = lanes per team).  A unit-major layout (each lane's image contiguous) would put the
// lanes of a read on a few banks and serialise every LDS access several-fold.
constexpr int kLdsBytesPerUnit = 3 * 4 * 16 + 16 * 4 + 4;   // limb groups, step sums, 1/S; per column
// Each row of the group and sum arrays holds kLdsPad entries past the team's
// units: the conversion writes a wave's 64 consecutive activation steps
// (4 units x 16 steps) to rows `step` and columns `unit`, and the pad spreads
// those writes over the banks.
constexpr int kLdsPad = 4;
constexpr size_t kLdsMax = 160 * 1024;   // LDS per workgroup on gfx950
template <int B, int S>
struct XLds {
    const u4 *grp;   // group 0 of limb 0 of column 0 of this lane's unit
    int tt;          // lanes per team
    float s[B][S];
    float iv[B];
    __device__ __forceinline__ u4 group(int b, int l, int i) const { return grp[((b * 3 + l) * 4 + i) * tt]; }
    __device__ __forceinline__ float sum(int b, int k) const { return s[b][k]; }
    __device__ __forceinline__ float inv(int b) const { return iv[b]; }
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

// Maximum of v over the 16 lanes of each DPP row (unsigned), in every lane
// of the row.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
    return v;
}

// Launch geometry shared by host and device.
struct Geom {
    int units;     // K / 64
    int wr;        // waves per row team = ceil(units / 64)
    int teams;     // row teams per workgroup (1, 2, 4 or 8)
};

// Work fused around the product (decode steps of a Llama layer):
//   pre = kPreNone:    x as given
//   pre = kPreRmsNorm: x <- (x / sqrt(mean(x^2) + eps)) * x2   (x2 = norm weights;
//                      every workgroup loads all of x anyway, so it reduces the
//                      sum of squares itself)
//   pre = kPreSiluMul: x <- SiLU(x) * x2   (x2 = the up projection, same layout as x)
//   post = kPostStore:      Y = W x
//   post = kPostAccumulate: Y += W x (the residual add)
//   post = kPostSiluPairs:  rows 2i and 2i+1 of W are a gate row and its up
//                      row (interleaved gate/up weights); Y[i] = SiLU(y[2i]) *
//                      y[2i+1], so Y holds N/2 values.  Teams 2j and 2j+1 of a
//                      workgroup compute such a pair for the same row groups
//                      and meet in LDS at the end.
// The formulas and their rounding are those of aih_rmsnorm, aih_silu_mul and
// aih_add; everything happens outside the row loop.
enum { kPreNone = 0, kPreRmsNorm = 1, kPreSiluMul = 2 };
enum { kPostStore = 0, kPostAccumulate = 1, kPostSiluPairs = 2 };
struct Fuse {
    const float *x2;
    float eps;
    int pre;
    int post;
};

__device__ __forceinline__ float silu_f(float g) { return g * (1.0f / (1.0f + expf(-g))); }

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// then for every wave.  __syncthreads() also waits for every global load in
// flight (s_waitcnt vmcnt(0)), which would drain the weight prefetch.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A workgroup is TEAMS row teams of geo.wr waves (ONEWAVE: geo.wr == 1).
// Team t of workgroup w visits the row groups c = w, w + gridDim.x, ... and
// computes row c*TEAMS + t of each.
//
// Software pipeline: the packed bytes of the team's first row are loaded
// before the activation conversion, or right after it where several teams of
// several waves share x through LDS, and its second row once x is in
// place; from then on each of the two register buffers is reloaded with the
// row two ahead as soon as its row is computed, so a wave always has one row
// of loads in flight while it computes.  The loop is unrolled twice so that
// each buffer keeps fixed registers.
//
// Several teams of several waves read a wide x (16-64 KB; 57 KB at K = 14336)
// that every workgroup fetches whole, which takes about two round trips of
// the CU's outstanding misses.  Issued behind the weight rows of all 256
// workgroups, those loads wait in a loaded memory system: on MI355X, loading
// the first row after the conversion instead ran the Q6_K 4096 x 14336
// product in 12.3-12.6 us instead of 13.0, and also loading the second row
// before the conversion's barrier measured 13.0 again.
//
// Loads complete in issue order, so waiting for the current row leaves the
// other buffer's loads in flight; the activation loads are issued first.
// The compiler can only rely on that where the order is the same on every
// path into a wait, hence:
//   - no load sits behind a data-dependent branch inside the loop, and the
//     loop runs only while both of its reloads are real rows; the last one
//     to three rows are computed after it in straight-line code;
//   - the loop has a single exit, at the bottom, on scalar row-group
//     indices: a loop with two exits is compiled with a flow block whose
//     (never taken) path back to the head skips half of the body, and the
//     compiler then waits at the head for loads meant to stay in flight.
// W is deliberately not __restrict__: that would let the compiler sink the
// first weight loads below the LDS barrier of the activation exchange.
template <class T, int B, int TEAMS, bool ONEWAVE, int MAXT, bool FUSED, bool REGS>
__global__ void __launch_bounds__(MAXT)
qmatvec_kernel(const uint8_t *W, int64_t N, int64_t row_bytes, Geom geo,
               const float *__restrict__ X, int64_t ldx, float *__restrict__ Y, int64_t ldy, Fuse fz)
{
    extern __shared__ __align__(16) uint32_t xs[];
    __shared__ float red[MAXT / 64][B];    // RMSNorm prologue: per-wave sums of squares
    // With one or two columns the limb image is copied from LDS into
    // registers once (48 VGPRs per column), so the row loop reads no LDS.
    // (Two columns read from LDS per row ran Q6_K 4096 x 14336 in 18.3 us
    // against 17.1 us hoisted, Q4_K 14336 x 4096 in 11.5 against 10.8.)
    constexpr bool HOIST = !REGS && B <= 2;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wr = ONEWAVE ? 1 : geo.wr;
    const int team_threads = wr * 64;
    // (The team index is wave-uniform, but making it a scalar with
    // readfirstlane measured 0.4 us slower per launch on MI355X.)
    const int team = TEAMS == 1 ? 0 : tid / team_threads;
    const int ut = tid - team * team_threads;   // unit index within the team
    const bool active = ut < geo.units;
    const int u = active ? ut : 0;
    // N is a multiple of TEAMS (the host computes a ragged remainder with
    // the single-team variant), so every team's row c*TEAMS + team exists.
    // The host keeps a launch's slice of W below 2^31 bytes.
    const int64_t ngroups = N / TEAMS;
    const uint32_t toff = (uint32_t)team * (uint32_t)row_bytes;
    const Rsrc wres = make_rsrc(W, (uint32_t)(N * row_bytes));
    const uint32_t gstride = (uint32_t)(TEAMS * row_bytes);   // bytes per row group
    // loads of the team's row in row group cc (see PtrRow / BufRow)
    auto load_group = [&](int cc, uint32_t *raw) {
        if constexpr (ONEWAVE)
            T::load(PtrRow{W + ((int64_t)cc * TEAMS + team) * row_bytes}, 0u, u, raw);
        else
            T::load(BufRow{wres, (uint32_t)cc * gstride}, toff, u, raw);
    };

    // Conversion mapping.  Several teams: piece p = k*blockDim.x + tid
    // (k < NST) is step p % 16 of unit p / 16, so the 16 lanes of a DPP row
    // hold the 16 steps of one unit and reduce its max|x| among themselves,
    // and a wave reads one contiguous KB of x (the order of the elements
    // inside a unit, T::step, only permutes lanes within it).  One team:
    // thread ut converts the 16 steps of its own unit.
    constexpr int NST = 16 / TEAMS;
    constexpr bool PIECES = TEAMS > 1;
    // Several teams of several waves share a wide x: their first weight row
    // is issued once x has landed (below); everyone else issues it now.
    constexpr bool SPREAD = TEAMS > 1 && !ONEWAVE;
    const int pieces = 16 * geo.units;
    auto piece = [&](int k) { return k * (int)blockDim.x + tid; };
    auto valid = [&](int k) { return PIECES ? piece(k) < pieces : active; };
    auto unit_of = [&](int k) { return PIECES ? (valid(k) ? piece(k) >> 4 : 0) : u; };
    auto step_of = [&](int k) { return PIECES ? piece(k) & 15 : k; };
    auto src_of = [&](int k) { return T::step(unit_of(k), step_of(k)).src; };
    f4 xv[B][NST];
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int k = 0; k < NST; ++k) xv[b][k] = ldg<f4>(X + b * ldx + src_of(k));
    // The second operand of a fused prologue: with several teams (a few
    // steps per thread) it is loaded with x, before the weights, so waiting
    // for it never waits for a weight row; a single team (16 steps per thread,
    // 128 registers) loads it where it is used.
    constexpr bool X2_EARLY = TEAMS > 1;
    f4 x2v[B][X2_EARLY ? NST : 1];
    auto x2_at = [&](int b, int k) {
        return ldg<f4>(fz.x2 + (fz.pre == kPreSiluMul ? b * ldx : 0) + src_of(k));
    };
    if (FUSED && X2_EARLY && fz.pre != kPreNone) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int k = 0; k < NST; ++k) x2v[b][X2_EARLY ? k : 0] = x2_at(b, k);
    }
    // The team visits row groups blockIdx.x + i*g while below ngroups (the
    // host launches at most ngroups workgroups and at most 64 row groups per
    // workgroup, so the indices fit in 32 bits and live in scalar registers).
    // A load past the end (only rb's first load, for a team of one row)
    // re-reads the team's first row instead.
    // Workgroups are dispatched round-robin over the 8 XCDs of MI355X, so
    // workgroup w runs on XCD w % 8.  The team's first row group is a
    // permutation of w that gives each XCD a contiguous piece of every band
    // of g row groups (XCD x: groups x*g/8 .. (x+1)*g/8 - 1 of the band); on
    // MI355X that ran the 14336 x 4096 Q4_0 and the 4096 x 14336 Q4_K / Q6_K
    // products about 3% faster than c0 = w.  The fused decode-step kernels
    // keep c0 = w: with the permutation the whole 8B-shaped decode step ran
    // 1.6% slower (1.476 -> 1.499 ms per token).
    const int ng = (int)ngroups, g = (int)gridDim.x;
    const int c0 = !FUSED && g % 8 == 0 ? (int)(blockIdx.x % 8) * (g / 8) + (int)(blockIdx.x / 8)
                                        : (int)blockIdx.x;
    // Lane i of the team's first wave stores row (c0 + i*g)*TEAMS + team.
    const int64_t n = (c0 + (int64_t)lane * g) * TEAMS + team;
    // The accumulate epilogue's old Y values are loaded here, before the
    // weights (lanes past the team's rows re-read row N - 1), so that the
    // kernel does not end on a round trip to Y.
    float yold[B];
    if (FUSED && fz.post == kPostAccumulate) {
#pragma unroll
        for (int b = 0; b < B; ++b) yold[b] = Y[b * ldy + (n < N ? n : N - 1)];
    }
    uint32_t ra[T::kRaw], rb[T::kRaw];
    // The fused decode-step kernels, whose x arrives late (written by the
    // previous kernel, behind a norm weight last read a token ago), also
    // load their second row here: the whole 8B-shaped decode step ran 0.5%
    // faster (1.450 -> 1.444 ms per token).  The plain kernel loads it after
    // the conversion (below).
    constexpr bool EARLY2 = FUSED && !SPREAD;
    if constexpr (!SPREAD) load_group(c0, ra);
    if constexpr (EARLY2) load_group(c0 + g < ng ? c0 + g : c0, rb);
    // keep the weight loads here, in flight during the conversion below
    __builtin_amdgcn_sched_barrier(0);

    auto x2_of = [&](int b, int k) { return X2_EARLY ? x2v[b][X2_EARLY ? k : 0] : x2_at(b, k); };
    if (FUSED && fz.pre == kPreSiluMul) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int k = 0; k < NST; ++k) {
                f4 &v = xv[b][k];
                const f4 up = x2_of(b, k);
                v.x = silu_f(v.x) * up.x;
                v.y = silu_f(v.y) * up.y;
                v.z = silu_f(v.z) * up.z;
                v.w = silu_f(v.w) * up.w;
            }
    }
    if (FUSED && fz.pre == kPreRmsNorm) {
        // the workgroup's threads hold every element of x once among their
        // valid steps
        float ss[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            ss[b] = 0.f;
#pragma unroll
            for (int k = 0; k < NST; ++k) {
                const f4 v = xv[b][k];
                const float q = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                ss[b] += valid(k) ? q : 0.f;
            }
            // DPP steps (a few cycles each; six LDS-permute shuffles cost
            // about a hundred cycles of latency apiece)
            const float t = wave_sum_to_lane63(ss[b]);
            if (lane == 63) red[wave][b] = t;
        }
        if constexpr (SPREAD) {
            __builtin_amdgcn_sched_barrier(0);
            load_group(c0, ra);
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_barrier();
        const int nw = (int)(blockDim.x >> 6);
        float rms[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float t = 0.f;
            for (int w = 0; w < nw; ++w) t += red[w][b];
            rms[b] = sqrtf(t / (float)(geo.units * 64) + fz.eps);
        }
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const f4 w = x2_of(0, k);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                f4 &v = xv[b][k];
                v.x = (v.x / rms[b]) * w.x;
                v.y = (v.y / rms[b]) * w.y;
                v.z = (v.z / rms[b]) * w.z;
                v.w = (v.w / rms[b]) * w.w;
            }
        }
    }

    // Per-unit scale from max|x| over the unit (bit patterns of |x|: unsigned
    // order is the float order, and a NaN is above every number).
    constexpr int NCS = PIECES ? NST : 1;   // one scale per held unit
    ColScale cs[B][NCS];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        uint32_t m = 0;
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const f4 v = xv[b][k];
            const uint32_t mk = max(max(__float_as_uint(v.x) & 0x7FFFFFFFu, __float_as_uint(v.y) & 0x7FFFFFFFu),
                                    max(__float_as_uint(v.z) & 0x7FFFFFFFu, __float_as_uint(v.w) & 0x7FFFFFFFu));
            if constexpr (PIECES) cs[b][PIECES ? k : 0] = col_scale(row16_max_u32(mk));
            else m = max(m, mk);
        }
        if constexpr (!PIECES) cs[b][0] = col_scale(m);
    }
    if (SPREAD && !(FUSED && fz.pre == kPreRmsNorm)) {
        // Wide x shared by several teams of several waves: its loads (16-64
        // KB per workgroup) have landed once the maxima above read them, so
        // the first weight row, issued here, does not queue them behind the
        // weight stream; it is in flight during the conversion.  (With the
        // RMSNorm prologue it was issued before that prologue's barrier.)
        __builtin_amdgcn_sched_barrier(0);
        load_group(c0, ra);
        __builtin_amdgcn_sched_barrier(0);
    }

    typedef typename std::conditional<REGS || HOIST, XRegs<B, T::kSums>, XLds<B, T::kSums>>::type XA;
    XA xa;
    if constexpr (REGS) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            uint32_t img[3][16];
#pragma unroll
            for (int k = 0; k < T::kSums; ++k) xa.s[b][k] = 0.f;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                convert_step(xv[b][s], cs[b][0].s, img[0][s], img[1][s], img[2][s]);
                xa.s[b][T::step(u, s).slot] += sum4(xv[b][s]);
            }
#pragma unroll
            for (int k = 0; k < T::kSums; ++k) xa.s[b][k] *= cs[b][0].s;
            xa.iv[b] = cs[b][0].inv_s;
#pragma unroll
            for (int l = 0; l < 3; ++l)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xa.g[b][l][i] = u4{img[l][4 * i], img[l][4 * i + 1], img[l][4 * i + 2], img[l][4 * i + 3]};
        }
    } else {
        // uint32 view of the limb groups, float views of the step sums and
        // of the per-unit inverse scales (rows of tp entries: the team's
        // units and the pad)
        const int tp = team_threads + kLdsPad;
        uint32_t *gw = xs;
        float *sums = reinterpret_cast<float *>(xs + (size_t)B * 3 * 4 * 4 * tp);
        float *uinv = sums + (size_t)B * 16 * tp;
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            if (!valid(k)) continue;
            const int pu = unit_of(k), ps = step_of(k);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                uint32_t w[3];
                const ColScale c = cs[b][PIECES ? k : 0];
                convert_step(xv[b][k], c.s, w[0], w[1], w[2]);
#pragma unroll
                for (int l = 0; l < 3; ++l) gw[((size_t)((b * 3 + l) * 4 + ps / 4) * tp + pu) * 4 + ps % 4] = w[l];
                sums[(b * 16 + ps) * tp + pu] = sum4(xv[b][k]) * c.s;
                if (ps == 0) uinv[b * tp + pu] = c.inv_s;
            }
        }
        lds_barrier();
        if constexpr (HOIST) {
            // the lane's 12 limb groups per column stay in registers for
            // the whole row loop
            const u4 *grp = reinterpret_cast<const u4 *>(xs) + ut;
#pragma unroll
            for (int b = 0; b < B; ++b)
#pragma unroll
                for (int l = 0; l < 3; ++l)
#pragma unroll
                    for (int i = 0; i < 4; ++i) xa.g[b][l][i] = grp[((b * 3 + l) * 4 + i) * tp];
        } else {
            xa.grp = reinterpret_cast<const u4 *>(xs) + ut;
            xa.tt = tp;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int k = 0; k < T::kSums; ++k) xa.s[b][k] = 0.f;
#pragma unroll
            for (int q = 0; q < 16; ++q) xa.s[b][T::step(u, q).slot] += sums[(b * 16 + q) * tp + ut];
            xa.iv[b] = uinv[b * tp + ut];
        }
    }

    // Row results are not stored inside the loop: lane i of the team's first
    // wave keeps the result of the team's i-th row in `yb` (the host limits a
    // launch to 64 rows per team), and the wave writes them out at the end.
    // With no stores between the loads, the compiler's count of outstanding
    // memory operations covers loads only, so waiting for the current row
    // never waits for the prefetch.
    const bool leader = ut < 64;   // the team's first wave
    float yb[B];
#pragma unroll
    for (int b = 0; b < B; ++b) yb[b] = 0.f;
    int kept = 0;

    // Dot product of one row, reduced over the wave into lane `kept` of yb.
    // A team of several waves adds its waves' yb once, after the last row:
    // no barrier inside the loop, so no wave waits for another's loads.
    auto row = [&](const uint32_t *raw) {
        float acc[B];
#pragma unroll
        for (int b = 0; b < B; ++b) acc[b] = 0.f;
        T::template dot<B>(raw, xa, u, acc);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v = wave_sum_to_lane63(active ? acc[b] : 0.f);
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
            yb[b] = lane == kept ? tot : yb[b];
        }
        ++kept;
    };

    // The loop runs while both reloads are real rows; the last one to three
    // rows are computed after it with exact loads, so no past-the-end load
    // is issued after the final row (its latency would then be exposed).
    // The second row is loaded only now: issued before the conversion as
    // well, it measured 0.35 us slower on MI355X for teams of 3-4 rows of
    // the plain kernel.
    if constexpr (!EARLY2) load_group(c0 + g < ng ? c0 + g : c0, rb);
    __builtin_amdgcn_sched_barrier(0);
    int c = c0;   // ra holds row group c, rb row group c + g
    while (c + 3 * g < ng) {
        row(ra);
        load_group(c + 2 * g, ra);
        __builtin_amdgcn_sched_barrier(0);   // reload issued before the other row is consumed
        row(rb);
        load_group(c + 3 * g, rb);
        __builtin_amdgcn_sched_barrier(0);
        c += 2 * g;
    }
    // here c < ng (c0 < ng, and every iteration leaves c + g < ng)
    if (c + 2 * g < ng) {
        row(ra);
        load_group(c + 2 * g, ra);
        __builtin_amdgcn_sched_barrier(0);
        row(rb);
        row(ra);
    } else if (c + g < ng) {
        row(ra);
        row(rb);
    } else {
        row(ra);
    }
    if constexpr (!ONEWAVE) {
        // the team's first wave adds the partial row sums of its waves, in
        // wave order
        __shared__ float part[MAXT / 64][B][64];
#pragma unroll
        for (int b = 0; b < B; ++b) part[wave][b][lane] = yb[b];
        __syncthreads();
        if (ut < 64) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float tot = 0.f;
                for (int w = 0; w < wr; ++w) tot += part[team * wr + w][b][lane];
                yb[b] = tot;
            }
        }
    }
    if constexpr (FUSED && TEAMS % 2 == 0) {
        if (fz.post == kPostSiluPairs) {
            __shared__ float pair_y[TEAMS][64];
            if (leader) pair_y[team][lane] = yb[0];
            __syncthreads();
            if (leader && team % 2 == 0 && lane < kept && n < N) {
                const float gt = pair_y[team][lane], up = pair_y[team + 1][lane];
                Y[n / 2] = silu_f(gt) * up;
            }
            return;
        }
    }
    if (leader && lane < kept && n < N) {
#pragma unroll
        for (int b = 0; b < B; ++b)
            Y[b * ldy + n] = FUSED && fz.post == kPostAccumulate ? yold[b] + yb[b] : yb[b];
    }
}

Geom make_geom(int64_t K)
{
    Geom g;
    g.units = (int)(K / 64);
    g.wr = (g.units + 63) / 64;
    g.teams = g.wr == 1 ? 8 : g.wr == 2 ? 4 : g.wr <= 4 ? 2 : 1;
    return g;
}

// One launch of one workgroup per CU: every workgroup pays the activation
// conversion once, so fewer, longer-lived workgroups win.  On MI355X
// (14336 x 4096 Q4_K, measured with an earlier form of the row loop) one
// workgroup of eight single-wave teams per CU ran 7.9 us, against 8.2 us
// with two per CU, 9.5 us with one 16-team workgroup per CU and 9.5-11.7 us
// with 4-7 workgroups per CU.
template <class T, int B, int TEAMS, bool ONEWAVE, int MAXT>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t row_bytes, Geom geo,
           const float *X, int64_t ldx, float *Y, int64_t ldy, Fuse fz)
{
    // fused prologue / epilogue kernels exist for one column only; gate/up
    // pairs need pairs of teams (an even team count and whole row groups)
    const bool fused = fz.pre != kPreNone || fz.post != kPostStore;
    if (fused && B != 1) return AIH_E_INVALID;
    if (fz.post == kPostSiluPairs && (TEAMS % 2 != 0 || N % TEAMS != 0)) return AIH_E_LIMIT;
    const int threads = TEAMS * geo.wr * 64;
    // The activation image goes to LDS whenever it fits (always for several
    // teams); a single team of a very wide row (K above about 32500) keeps
    // each unit's image in its own registers instead.
    size_t lds = (size_t)B * kLdsBytesPerUnit * (geo.wr * 64 + kLdsPad);
    const bool regs = TEAMS == 1 && lds > kLdsMax;
    if (regs) lds = 0;
    const int64_t cap = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // A workgroup computes at most 64 row groups per launch (its results are
    // held in one register per lane); taller matrices take several launches.
    // The kernel needs N to be a multiple of TEAMS; the last N % TEAMS rows
    // go to the single-team variant, one launch per column.
    const int64_t nmain = N - N % TEAMS;
    // at most 64 row groups per workgroup, and a slice of W below 2^31 bytes
    // (the kernel's buffer resource and offsets are 32-bit)
    int64_t rows_per_launch = cap * 64 * TEAMS;
    const int64_t by_bytes = (0x7FFFFFFFll / row_bytes) / TEAMS * TEAMS;
    if (by_bytes < rows_per_launch) rows_per_launch = by_bytes;
    if (rows_per_launch <= 0) return AIH_E_LIMIT;
    for (int64_t r0 = 0; r0 < nmain; r0 += rows_per_launch) {
        const int64_t nr = nmain - r0 < rows_per_launch ? nmain - r0 : rows_per_launch;
        const int64_t ng = nr / TEAMS;
        const int64_t grid = ng < cap ? ng : cap;
        // gate/up pairs write one value per two rows (r0 is a multiple of TEAMS)
        float *ys = Y + (fz.post == kPostSiluPairs ? r0 / 2 : r0);
        if (fused && regs)
            hipLaunchKernelGGL((qmatvec_kernel<T, B, TEAMS, ONEWAVE, MAXT, B == 1, TEAMS == 1>), dim3((unsigned)grid),
                               dim3(threads), lds, ctx->stream, W + r0 * row_bytes, nr, row_bytes, geo, X, ldx,
                               ys, ldy, fz);
        else if (fused)
            hipLaunchKernelGGL((qmatvec_kernel<T, B, TEAMS, ONEWAVE, MAXT, B == 1, false>), dim3((unsigned)grid),
                               dim3(threads), lds, ctx->stream, W + r0 * row_bytes, nr, row_bytes, geo, X, ldx,
                               ys, ldy, fz);
        else if (regs)
            hipLaunchKernelGGL((qmatvec_kernel<T, B, TEAMS, ONEWAVE, MAXT, false, TEAMS == 1>), dim3((unsigned)grid),
                               dim3(threads), lds, ctx->stream, W + r0 * row_bytes, nr, row_bytes, geo, X, ldx,
                               ys, ldy, fz);
        else
            hipLaunchKernelGGL((qmatvec_kernel<T, B, TEAMS, ONEWAVE, MAXT, false, false>), dim3((unsigned)grid),
                               dim3(threads), lds, ctx->stream, W + r0 * row_bytes, nr, row_bytes, geo, X, ldx,
                               ys, ldy, fz);
        const int rc = aih_launch_status();
        if (rc) return rc;
    }
    if constexpr (TEAMS > 1) {
        if (nmain < N) {
            Geom g1 = geo;
            g1.teams = 1;
            for (int b = 0; b < B; ++b) {
                Fuse f1 = fz;
                if (f1.pre == kPreSiluMul) f1.x2 += b * ldx;
                const int rc = launch<T, 1, 1, false, 1024>(ctx, W + nmain * row_bytes, N - nmain, row_bytes, g1,
                                                            X + b * ldx, ldx, Y + b * ldy + nmain, ldy, f1);
                if (rc) return rc;
            }
        }
    }
    return AIH_OK;
}

// One pass over W for `two` ? 2 : 1 activation columns.
template <class T>
int launch_pass(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t row_bytes, Geom geo,
                const float *X, int64_t ldx, float *Y, int64_t ldy, bool two, Fuse fz)
{
    switch (geo.teams) {
    case 8: return two ? launch<T, 2, 8, true, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz)
                       : launch<T, 1, 8, true, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz);
    case 4: return two ? launch<T, 2, 4, false, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz)
                       : launch<T, 1, 4, false, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz);
    case 2:
        // two columns of the widest two-team image (K up to 16384) exceed the
        // LDS of a workgroup: one column per pass there
        if (two && (size_t)2 * kLdsBytesPerUnit * (geo.wr * 64 + kLdsPad) > kLdsMax) {
            int rc = launch<T, 1, 2, false, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz);
            if (!rc) {
                Fuse f1 = fz;
                if (f1.pre == kPreSiluMul) f1.x2 += ldx;
                rc = launch<T, 1, 2, false, 512>(ctx, W, N, row_bytes, geo, X + ldx, ldx, Y + ldy, ldy, f1);
            }
            return rc;
        }
        return two ? launch<T, 2, 2, false, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz)
                   : launch<T, 1, 2, false, 512>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz);
    default: {  // one team of up to 16 waves: one column per pass within 128 VGPRs
        int rc = launch<T, 1, 1, false, 1024>(ctx, W, N, row_bytes, geo, X, ldx, Y, ldy, fz);
        if (!rc && two) {
            Fuse f1 = fz;
            if (f1.pre == kPreSiluMul) f1.x2 += ldx;
            rc = launch<T, 1, 1, false, 1024>(ctx, W, N, row_bytes, geo, X + ldx, ldx, Y + ldy, ldy, f1);
        }
        return rc;
    }
    }
}

template <class T>
int launch_type(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
                const float *X, int64_t ldx, float *Y, int64_t ldy, int batch, Fuse fz)
{
    const Geom geo = make_geom(K);
    // Columns are processed in passes of at most two; each pass re-reads W.
    for (int b0 = 0; b0 < batch; b0 += 2) {
        Fuse fb = fz;
        if (fb.pre == kPreSiluMul) fb.x2 += b0 * ldx;
        const int rc = launch_pass<T>(ctx, W, N, row_bytes, geo, X + b0 * ldx, ldx, Y + b0 * ldy, ldy,
                                      batch - b0 >= 2, fb);
        if (rc) return rc;
    }
    return AIH_OK;
}

// Batches from this size on go to the MFMA kernel (aih_qmatvec_mfma.hip).
constexpr int kMfmaMinBatch = 3;

}  // namespace

namespace {

int dispatch(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X, int64_t ldx, float *Y,
             int64_t ldy, int batch, Fuse fz)
{
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch_type<Q4K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, fz);
    case AIH_TYPE_Q6_K: return launch_type<Q6K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, fz);
    case AIH_TYPE_Q8_0: return launch_type<Q80>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, fz);
    case AIH_TYPE_Q4_0: return launch_type<Q40>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch, fz);
    default: return AIH_E_UNSUPPORTED;
    }
}

// Shape and pointer checks shared by both entry points.
int check_args(int64_t K, const void *W, const float *X, int64_t ldx)
{
    // Every kernel reads 64-element units: K must be a multiple of 64, and a
    // row team (one lane per unit) holds at most 1024 lanes.
    if (K % 64 != 0) return AIH_E_LIMIT;
    if (K / 64 > 1024) return AIH_E_LIMIT;
    if (reinterpret_cast<uintptr_t>(W) % 16 != 0) return AIH_E_INVALID;
    if (reinterpret_cast<uintptr_t>(X) % 16 != 0 || (ldx % 4) != 0) return AIH_E_INVALID;
    return AIH_OK;
}

}  // namespace

int aih_launch_qmatvec(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                       const float *X, int64_t ldx, float *Y, int64_t ldy, int batch, const aih_scratch *ext)
{
    const int rc = check_args(K, W, X, ldx);
    if (rc) return rc;
    // Three or more columns: the MFMA kernel reads W once for all of them.
    if (batch >= kMfmaMinBatch) return aih_launch_qmatvec_mfma(ctx, type, W, N, K, X, ldx, Y, ldy, batch, ext);
    return dispatch(ctx, type, W, N, K, X, ldx, Y, ldy, batch, Fuse{nullptr, 0.f, kPreNone, kPostStore});
}

int aih_launch_qmatvec_fused(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const float *X,
                             const float *X2, float eps, int pre, int post, float *Y)
{
    const int rc = check_args(K, W, X, K);
    if (rc) return rc;
    if (pre != kPreNone && reinterpret_cast<uintptr_t>(X2) % 16 != 0) return AIH_E_INVALID;
    return dispatch(ctx, type, W, N, K, X, K, Y, N, 1, Fuse{X2, eps, pre, post});
}
