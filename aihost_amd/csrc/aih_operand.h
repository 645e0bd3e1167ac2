// aih_operand.h -- the fp16 activation operand of the prefill GEMM: layout and
// range scaling, shared by every kernel that writes or reads it.
//
// The reference multiplies fp32 activations (ComputeShaders.cs:93-129); the
// GEMM rounds them to fp16 for the matrix cores.  fp16 holds 11 significant
// bits over 2^-14 .. 65504 (subnormals down to 2^-24), so an activation row
// is scaled by a power of two before the rounding and the product is scaled
// back in the GEMM's fp32 epilogue.  Powers of two change no significand:
// where a row's values are normal fp16 numbers with and without the scale,
// both give the same bits.
//
// Layout of the image of an M x K operand (K a multiple of 64, mpad = M
// rounded up to 32), in bytes from its start:
//   [0, 2 mpad K)        fp16 values in MFMA fragment order: the A operand of
//                        v_mfma_f32_32x32x16_f16 for rows 32 mb .. +31 and k
//                        16 kk .. +15 is the 1 KB block mb * K/16 + kk, lane
//                        l = row % 32 + 32 * (k / 8 % 2) at 16 bytes * l
//   [2 mpad K, + 4 mpad) int32 E[m]: row m holds x[m, k] 2^(E[m]) (rows past
//                        M: zero values, E = 0)
//   [.., + mpad K / 32)  int8 d[m][b], only in images that operators outside
//                        the GEMM write (aih_qgemm_fused's AIH_POST_SILU_PAIRS_F16
//                        output, aih_attention_operand): those writers see one
//                        32-column block of a row at a time, so block b of row
//                        m holds x 2^(E[m] + d[m][b]); a pass before the GEMM
//                        (operand_fixup_kernel) brings every row to one
//                        exponent.
#pragma once

#include <cstdint>

namespace aih_operand {

// A row (or block) whose largest magnitude lies in [2^-12, 2^15) is stored
// unscaled: every value then rounds to fp16 with an absolute error of at most
// 2^-13 of that maximum, the subnormals included, and nothing overflows.
// Outside that window the exponent puts the maximum in [2^14, 2^15).  Zero,
// infinite and NaN maxima keep exponent 0 (zeros stay zero; inf and NaN reach
// the output as the fp32 product would give them).
__device__ __forceinline__ int range_exp(float mx)
{
    if (!(mx < __builtin_inff()) || mx == 0.f) return 0;   // NaN, inf, zero
    if (mx >= 0x1p-12f && mx < 0x1p15f) return 0;          // the window
    // 14 - floor(log2 mx), from the frexp exponent (mx = f 2^e, f in
    // [0.5, 1)), subnormal maxima included
    return 15 - __builtin_amdgcn_frexp_expf(mx);
}

// Block exponents are stored as int8, in [-114, 127]: clamped to 127, a
// block of maxima below 2^-113 keeps a maximum below 2^14 (still no
// overflow).  An all-zero block stores kZeroBlock instead: it takes no part in
// choosing the row's common exponent and is never rescaled.
constexpr int kZeroBlock = -128;

__device__ __forceinline__ int block_exp(float mx)
{
    if (mx == 0.f) return kZeroBlock;
    const int e = range_exp(mx);
    return e > 127 ? 127 : e;
}

__host__ __device__ __forceinline__ int64_t mpad_of(int64_t m) { return (m + 31) / 32 * 32; }

// Byte offsets of the exponent arrays.
__host__ __device__ __forceinline__ int64_t row_exp_offset(int64_t mpad, int64_t k) { return 2 * mpad * k; }
__host__ __device__ __forceinline__ int64_t block_exp_offset(int64_t mpad, int64_t k) { return 2 * mpad * k + 4 * mpad; }

// Bytes of an image: values and row exponents (the GEMM's own staging), plus
// the block exponents for an image written outside the GEMM.
__host__ __device__ __forceinline__ int64_t image_bytes(int64_t mpad, int64_t k, bool blocks)
{
    return 2 * mpad * k + 4 * mpad + (blocks ? mpad * (k / 32) : 0);
}

// The 16-byte slot of row m holding k .. k + 7 (k % 8 == 0), in halves from
// the image start.
__host__ __device__ __forceinline__ int64_t slot_half(int64_t m, int64_t k, int64_t K)
{
    return (((m >> 5) * (K / 16) + (k >> 4)) * 64 + (m & 31) + 32 * ((k >> 3) & 1)) * 8;
}

}  // namespace aih_operand
