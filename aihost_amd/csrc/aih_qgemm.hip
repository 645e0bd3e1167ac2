// aih_qgemm.hip -- prefill GEMM with the GGUF block dequantization fused in.
//
//   Y[m*N + n] = sum_k X[m*K + k] * W[n, k]        (m < M, n < N)
//
// This replaces, for M > 8, the reference's TempF32 -> DequantizeInto ->
// MatMulWeights sequence (AIHost/AIHost/Compute/TransformerBase.cs:254-271,
// ComputeOps.cs:761-861, ComputeOps.cs:275-309, ComputeShaders.cs:93-129): the
// F32 SIMT matmul over a dequantized scratch copy becomes one kernel that
// dequantizes tiles of W into LDS as fp16 and contracts them on the matrix
// cores (v_mfma_f32_32x32x16_f16, fp32 accumulation).
//
// Tiling.  X is first converted to fp16 in the context's workspace, stored in
// MFMA fragment order.  A workgroup then owns a 128 (M) x 64 (N) tile of Y and
// walks K in steps of 64 elements (a Q4_K 64-group, a pair of Q8_0 or Q4_0
// blocks, two quarters of a Q6_K half-block).  Four producer waves dequantize
// W for the next step into LDS while four consumer waves multiply the current
// step (two 32x32x16 MFMAs per 16 k per wave), their A fragments loaded
// straight from the tiled X; one barrier per step.
//
// Precision.  Both operands are rounded to fp16 (11-bit significand) and the
// products accumulate in fp32: normwise error near 3e-4 against the fp32
// reference.  bf16 operands (8-bit significand) would give about 2.4e-3, more
// than the 1e-3 the path is held to.  Weights are dequantized in fp32 with the
// reference's formulas (ComputeOps.cs:1629-1678 for Q4_K, :1735-1774 for Q6_K,
// the GGUF definitions for Q8_0 and Q4_0) before the rounding to fp16.
#include "aih_pieces.h"

namespace {

using namespace aih_pieces;
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128;          // activation rows per workgroup
constexpr int BN = 64;           // weight rows per workgroup
constexpr int BK = 64;           // K per step
constexpr int LDK = BK + 8;      // LDS row stride in halves (16-byte pad against bank conflicts)

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, then for every wave.  __syncthreads() would also wait for the
// global loads in flight (its fences cover global memory), draining the
// prefetch at every step.  The "memory" clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// X (fp32, M x K) -> fp16, stored in the order the matrix cores read it.
// The A operand of v_mfma_f32_32x32x16_f16 for rows 32*mb .. +31 and k
// 16*kk .. +15 holds, in lane l, the 8 halves X[32*mb + l%32][16*kk +
// 8*(l/32) .. +7]; here that fragment is the 1 KB block (mb*KC + kk) of Xt
// (KC = K/16), lane l at 16 bytes * l.  A wave then loads a fragment with one
// fully coalesced 16-byte load per lane, straight into registers.  Rows past
// M (up to the next multiple of 32) are zero.  One thread per 8 halves.
__global__ void __launch_bounds__(256)
x_tile_kernel(const float *__restrict__ X, int64_t M, int64_t K, _Float16 *__restrict__ Xt, int64_t nslots)
{
    const int64_t kc = K / 16;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nslots; i += (int64_t)gridDim.x * 256) {
        const int l = (int)(i & 63);
        const int64_t frag = i >> 6;
        const int64_t mb = frag / kc, kk = frag - mb * kc;
        const int64_t row = 32 * mb + (l & 31);
        const int64_t k = 16 * kk + 8 * (l >> 5);
        h8 v = {};
        if (row < M) {
            const f4 a = ldg<f4>(X + row * K + k), b = ldg<f4>(X + row * K + k + 4);
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            v = pack8(f);
        }
        *reinterpret_cast<h8 *>(Xt + 8 * i) = v;
    }
}

// Eight waves per workgroup in two roles, one of each on every SIMD.
//   Consumers (waves 0..3) each own a 64 (M) x 32 (N) sub-tile of the
//   128 x 64 output tile (two 32x32 accumulators).  They load their A
//   fragments straight from the tiled fp16 copy of X into registers, one
//   step ahead in a ring of two register sets, and read the dequantized
//   weights (B) from LDS.  The short ring keeps the kernel within 128
//   registers, so two workgroups share a CU where the grid has enough of
//   them (on MI355X, the 4096 x 4096 x 512 product ran 39.8 us against 43.2
//   with four sets, three steps ahead).
//   Producers (waves 4..7) load the packed weights four steps ahead, dequantize
//   the next step into the other LDS buffer while the consumers multiply the
//   current one.
// One LDS barrier per step joins the roles.  Keeping X out of LDS leaves LDS
// with the weight tile only (8 KB per step written, 16 KB read).
template <class T>
__global__ void __launch_bounds__(512, 2)
qgemm_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
             const _Float16 *__restrict__ Xt, int64_t M, float *__restrict__ Y)
{
    __shared__ __align__(16) _Float16 wsh[2][BN][LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool producer = wave >= 4;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int ns = (int)(K / BK);

    if (producer) {
        // The four lanes of a quad share weight row t/4 and take its pieces
        // 0..3, so they read the same header and the same 32 bytes of codes.
        const int ptid = tid - 256;
        const int wr = ptid >> 2, wp = ptid & 3;
        const int64_t wn = n0 + wr < N ? n0 + wr : N - 1;
        const uint8_t *wrow = W + wn * row_bytes;
        // loads for step kb, clamped so that no load sits behind a branch
        auto gload = [&](int kb, typename T::Raw &r) {
            kb = kb < ns ? kb : ns - 1;
            T::load(wrow, kb, wp, r);
        };
        auto stage = [&](int buf, int kb, const typename T::Raw &r) {
            // The step index is hidden from the optimiser: in the unrolled
            // loop it would otherwise know kb % 4, find some loaded dwords
            // unused (e.g. the scale bytes of the other sub-blocks), reuse
            // their registers while the load is in flight and so wait for it.
            asm volatile("" : "+s"(kb));
            h8 lo, hi;
            piece16h<T>(r, kb, wp, lo, hi);
            *reinterpret_cast<h8 *>(&wsh[buf][wr][16 * wp]) = lo;
            *reinterpret_cast<h8 *>(&wsh[buf][wr][16 * wp + 8]) = hi;
        };
        // Four register sets in a ring: the loads for step kb+4 are issued
        // while step kb+1 is staged.  The loop has a single exit at the bottom
        // (an exit between a load and the loop head would make the compiler
        // wait for every load there); the last one to three steps follow it.
        typename T::Raw s0, s1, s2, s3;
        gload(0, s0);
        gload(1, s1);
        gload(2, s2);
        gload(3, s3);
        stage(0, 0, s0);
        lds_barrier();
        int kb = 0;
        for (; kb + 4 < ns; kb += 4) {
            gload(kb + 4, s0);
            __builtin_amdgcn_sched_barrier(0);
            stage(1, kb + 1, s1);
            lds_barrier();
            gload(kb + 5, s1);
            __builtin_amdgcn_sched_barrier(0);
            stage(0, kb + 2, s2);
            lds_barrier();
            gload(kb + 6, s2);
            __builtin_amdgcn_sched_barrier(0);
            stage(1, kb + 3, s3);
            lds_barrier();
            gload(kb + 7, s3);
            __builtin_amdgcn_sched_barrier(0);
            stage(0, kb + 4, s0);
            lds_barrier();
        }
        if (kb + 1 < ns) {
            stage(1, kb + 1, s1);
            lds_barrier();
        }
        if (kb + 2 < ns) {
            stage(0, kb + 2, s2);
            lds_barrier();
        }
        if (kb + 3 < ns) {
            stage(1, kb + 3, s3);
            lds_barrier();
        }
        return;
    }

    // consumer: rows wm .. wm+63 of the M tile (M blocks mb0, mb0+1), columns
    // wc .. wc+31 of the N tile
    const int wm = (wave >> 1) * 64, wc = (wave & 1) * 32;
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const int64_t kc = K / 16, mblocks = (M + 31) / 32;
    int64_t mb0 = (m0 + wm) / 32, mb1 = mb0 + 1;
    mb0 = mb0 < mblocks ? mb0 : mblocks - 1;
    mb1 = mb1 < mblocks ? mb1 : mblocks - 1;
    const _Float16 *xa0 = Xt + (mb0 * kc * 64 + lane) * 8;
    const _Float16 *xa1 = Xt + (mb1 * kc * 64 + lane) * 8;
    struct AF { h8 a0[4], a1[4]; };
    auto aload = [&](int kb, AF &f) {
        kb = kb < ns ? kb : ns - 1;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            f.a0[kk] = ldg<h8>(xa0 + ((int64_t)kb * 4 + kk) * 512);
            f.a1[kk] = ldg<h8>(xa1 + ((int64_t)kb * 4 + kk) * 512);
        }
    };
    f16v acc0 = {}, acc1 = {};
    auto mfma = [&](int buf, const AF &f) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const h8 b = *reinterpret_cast<const h8 *>(&wsh[buf][wc + fr][16 * kk + fk]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a0[kk], b, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a1[kk], b, acc1, 0, 0, 0);
        }
    };
    // the same barrier sequence as the producers; A loads one step ahead
    AF f0, f1;
    aload(0, f0);
    aload(1, f1);
    lds_barrier();
    int kb = 0;
    for (; kb + 2 < ns; kb += 2) {
        mfma(kb & 1, f0);
        aload(kb + 2, f0);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
        mfma((kb + 1) & 1, f1);
        aload(kb + 3, f1);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
    }
    mfma(kb & 1, f0);
    if (kb + 1 < ns) {
        lds_barrier();
        mfma((kb + 1) & 1, f1);
    }

    // acc element r of lane l is C[8*(r/4) + 4*(l/32) + r%4][l%32] of its 32x32 block
    const int64_t n = n0 + wc + fr;
    if (n < N) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int64_t ma = m0 + wm + i, mb = m0 + wm + 32 + i;
            if (ma < M) Y[ma * N + n] = acc0[r];
            if (mb < M) Y[mb * N + n] = acc1[r];
        }
    }
}

template <class T>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
           const _Float16 *Xh, int64_t M, float *Y)
{
    const int64_t gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM;
    if (gy > 65535 || gx > 0x7FFFFFFF) return AIH_E_LIMIT;
    hipLaunchKernelGGL((qgemm_kernel<T>), dim3((unsigned)gx, (unsigned)gy), dim3(512), 0, ctx->stream,
                       W, N, K, row_bytes, Xh, M, Y);
    return aih_launch_status();
}

}  // namespace

int aih_launch_qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                     const float *X, int64_t M, float *Y)
{
    // K advances in 64-element steps.
    if (K % BK != 0) return AIH_E_LIMIT;
    if ((reinterpret_cast<uintptr_t>(X) & 15) != 0) return AIH_E_INVALID;
    const int64_t mpad = (M + 31) / 32 * 32;
    void *work = nullptr;
    int rc = aih_workspace(ctx, (size_t)mpad * (size_t)K * sizeof(_Float16), &work);
    if (rc) return rc;
    _Float16 *xh = static_cast<_Float16 *>(work);
    const int64_t nslots = mpad * K / 8;
    const int64_t blocks = (nslots + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);
    hipLaunchKernelGGL(x_tile_kernel, dim3(grid), dim3(256), 0, ctx->stream, X, M, K, xh, nslots);
    rc = aih_launch_status();
    if (rc) return rc;
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch<G4K>(ctx, w, N, K, rb, xh, M, Y);
    case AIH_TYPE_Q6_K: return launch<G6K>(ctx, w, N, K, rb, xh, M, Y);
    case AIH_TYPE_Q8_0: return launch<G80>(ctx, w, N, K, rb, xh, M, Y);
    case AIH_TYPE_Q4_0: return launch<G40>(ctx, w, N, K, rb, xh, M, Y);
    default: return AIH_E_UNSUPPORTED;
    }
}
