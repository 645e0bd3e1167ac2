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
// Tiling.  X is first converted to an fp16 copy in the context's workspace.
// A workgroup of four waves then owns a 128 (M) x 64 (N) tile of Y and walks
// K in steps of 64 elements (a Q4_K 64-group, a pair of Q8_0 or Q4_0 blocks,
// two quarters of a Q6_K half-block).  Per step every thread copies 32 fp16
// activations and dequantizes 16 weights into LDS; each wave then multiplies
// its 64 x 32 sub-tile with two MFMAs per 16 k.  LDS is double buffered and
// the global loads run two steps ahead in registers, one barrier per step.
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

// X (fp32, M x K) -> fp16 copy, 8 elements per thread.  Every workgroup of
// the GEMM re-reads its X rows once per N tile, so converting once here
// halves that traffic and takes the conversion out of the GEMM's loop.
__global__ void __launch_bounds__(256)
x_to_f16_kernel(const float *__restrict__ X, _Float16 *__restrict__ Xh, int64_t n8)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
        const f4 a = ldg<f4>(X + 8 * i), b = ldg<f4>(X + 8 * i + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        *reinterpret_cast<h8 *>(Xh + 8 * i) = pack8(v);
    }
}

// Registers of one K step's staging loads: 64 bytes of X (32 halves of one
// row) and the packed bytes of one weight piece.
template <class T>
struct Stage {
    u4 x[4];
    typename T::Raw w;
};

template <class T>
__global__ void __launch_bounds__(256)
qgemm_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
             const _Float16 *__restrict__ Xh, int64_t M, float *__restrict__ Y)
{
    __shared__ __align__(16) _Float16 xs[2][BM][LDK];
    __shared__ __align__(16) _Float16 wsh[2][BN][LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

    // staging roles: X row xr, halves 32*xh .. +31 of the step; W row wr, piece wp
    const int xr = tid >> 1, xh = tid & 1;
    const int64_t xm = m0 + xr < M ? m0 + xr : M - 1;
    const _Float16 *xrow = Xh + xm * K + 32 * xh;
    const int wr = tid >> 2, wp = tid & 3;
    const int64_t wn = n0 + wr < N ? n0 + wr : N - 1;
    const uint8_t *wrow = W + wn * row_bytes;

    // wave sub-tile: rows wm .. wm+63 of the M tile, columns wc .. wc+31 of the N tile
    const int wm = (wave >> 1) * 64, wc = (wave & 1) * 32;
    const int fr = lane & 31, fk = 8 * (lane >> 5);

    f16v acc0 = {}, acc1 = {};
    const int ns = (int)(K / BK);

    // Loads for step kb (clamped to the last step, so that no load sits behind
    // a branch and the compiler can wait for exactly the set it consumes).
    auto gload = [&](int kb, Stage<T> &st) {
        kb = kb < ns ? kb : ns - 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) st.x[i] = ldg<u4>(xrow + (int64_t)kb * BK + 8 * i);
        T::load(wrow, kb, wp, st.w);
    };
    auto stage = [&](int buf, int kb, const Stage<T> &st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u4 *>(&xs[buf][xr][32 * xh + 8 * i]) = st.x[i];
        float y[16];
        T::piece(st.w, kb, wp, y);
        *reinterpret_cast<h8 *>(&wsh[buf][wr][16 * wp]) = pack8(y);
        *reinterpret_cast<h8 *>(&wsh[buf][wr][16 * wp + 8]) = pack8(y + 8);
    };
    auto mfma = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            const h8 a0 = *reinterpret_cast<const h8 *>(&xs[buf][wm + fr][kk + fk]);
            const h8 a1 = *reinterpret_cast<const h8 *>(&xs[buf][wm + 32 + fr][kk + fk]);
            const h8 b = *reinterpret_cast<const h8 *>(&wsh[buf][wc + fr][kk + fk]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc1, 0, 0, 0);
        }
    };

    // Two register sets: the loads for step kb+2 are issued while step kb is
    // multiplied and step kb+1 is staged, so every load has about one and a
    // half steps to arrive.  The loop has a single exit at the bottom (the
    // last one or two steps follow it): an exit between a load and the loop
    // head would make the compiler wait for every load at the head.
    Stage<T> sa, sb;
    gload(0, sa);
    gload(1, sb);
    stage(0, 0, sa);
    lds_barrier();
    int kb = 0;
    for (; kb + 2 < ns; kb += 2) {
        gload(kb + 2, sa);
        __builtin_amdgcn_sched_barrier(0);
        mfma(0);
        stage(1, kb + 1, sb);
        lds_barrier();
        gload(kb + 3, sb);
        __builtin_amdgcn_sched_barrier(0);
        mfma(1);
        stage(0, kb + 2, sa);
        lds_barrier();
    }
    mfma(0);
    if (kb + 1 < ns) {
        stage(1, kb + 1, sb);
        lds_barrier();
        mfma(1);
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
    hipLaunchKernelGGL((qgemm_kernel<T>), dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, ctx->stream,
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
    void *work = nullptr;
    int rc = aih_workspace(ctx, (size_t)M * (size_t)K * sizeof(_Float16), &work);
    if (rc) return rc;
    _Float16 *xh = static_cast<_Float16 *>(work);
    const int64_t n8 = M * K / 8;
    const int64_t blocks = (n8 + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 4096 ? blocks : 4096);
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(grid), dim3(256), 0, ctx->stream, X, xh, n8);
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
