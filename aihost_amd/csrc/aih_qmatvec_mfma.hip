// aih_qmatvec_mfma.hip -- small-batch decode matvec (3..8 activation columns)
// on the matrix cores, dequantization fused.
//
//   Y[b*ldy + n] = sum_k X[b*ldx + k] * W[n, k]        (b < batch, n < N)
//
// The single-column matvec (aih_qmatvec.hip) contracts each weight once per
// column with v_dot2_f32_f16, so its ALU work grows with the batch; above two
// columns it would re-read W once per pair of columns.  Here every weight is
// dequantized once (to fp16, with the reference's formulas) and multiplied
// against all columns at once by v_mfma_f32_16x16x32_f16: the 16 rows of the
// MFMA's A operand are 16 weight rows, the 16 columns of its B operand are
// the batch columns (columns past the batch duplicate the last one and are
// not stored).  W is read from HBM exactly once whatever the batch.
//
// Work split.  A workgroup of eight waves owns a tile of 16 weight rows and
// walks K in steps of 512 (eight 64-element chunks).  In each step:
//   - thread t dequantizes piece t % 32 of the step of row t / 32 (16
//     weights) into an fp16 LDS tile of 16 rows x 512 k.  The 32 lanes of a
//     row read its step's bytes (2 super-blocks of Q4_K/Q6_K, 16 blocks of
//     Q8_0/Q4_0) as one contiguous span.  Giving each lane the piece its
//     MFMA operand needs instead put 16 rows and 1-64 bytes per row under
//     every load (W streamed at about 1.3 TB/s);
//   - wave w multiplies the k-slices 2w and 2w+1 (32 k each) of the tile:
//     A fragments from LDS, B fragments (the batch columns) straight from X
//     in fp32, 32 bytes per lane over whole cache lines; columns past the
//     batch are zero.
// The weight and activation loads of a step are issued D steps ahead into a
// ring of register sets; one LDS barrier per step (two tile buffers).  The
// eight partial 16x16 accumulators are summed through LDS at the end.
//
// This replaces TempF32 + ComputeOps.MatMulWeights for M = batch in 3..8
// (AIHost/AIHost/Compute/TransformerBase.cs:254-271, ComputeOps.cs:275-309).
// Precision: weights and activations rounded to fp16, fp32 accumulation.
#include "aih_pieces.h"

namespace {

using namespace aih_pieces;

constexpr int RT = 16;   // weight rows per workgroup (MFMA rows)
constexpr int KW = 8;    // waves per workgroup, each on its own K range

constexpr int CPS = 8;          // 64-element chunks per step
constexpr int KS = 64 * CPS;    // k per step
constexpr int LDA = KS + 8;     // LDS row stride of the tile, in halves (16-byte pad)
constexpr int D = 2;            // steps in flight

// Workgroup barrier for LDS traffic only (waits for this wave's LDS
// operations, then for every wave); __syncthreads() would also drain the
// global loads in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <class T>
__global__ void __launch_bounds__(KW * 64)
qmv_mfma_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
                const float *__restrict__ X, int64_t ldx, float *__restrict__ Y, int64_t ldy, int batch)
{
    __shared__ __align__(16) _Float16 at[2][RT][LDA];
    __shared__ float part[KW][RT * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * RT;
    const int nch = (int)(K / 64);
    const int nsteps = (nch + CPS - 1) / CPS;
    // dequantization role: row pr of the tile, chunk pc of the step, piece ps
    const int pr = tid >> 5, pc = (tid >> 2) & (CPS - 1), ps = tid & 3;
    const uint8_t *prow = W + (n0 + pr < N ? n0 + pr : N - 1) * row_bytes;
    // multiplication role: lane (i, q) -> MFMA row / column i, k group q
    const int i = lane & 15, q = lane >> 4;
    const float *xbase = X + (int64_t)(i < batch ? i : batch - 1) * ldx;
    const float *xcol = xbase + 8 * q + 64 * wave;

    // loads of step st (chunks past the end re-read the last one; they are
    // zeroed when staged)
    auto wload = [&](int st, typename T::Raw &r) {
        const int c = st * CPS + pc;
        T::load(prow, c < nch ? c : nch - 1, ps, r);
    };
    // activations of k-slices 2*wave and 2*wave+1 of step st: 8 floats each
    // (slices past K, only in a last partial step, re-read the column's
    // first 8 floats)
    auto xload = [&](int st, f4 *xv) {
        const float *p = xcol + (int64_t)st * KS;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float *ph = (int64_t)st * KS + 64 * wave + 32 * h + 8 * q + 8 <= K ? p + 32 * h : xbase;
            xv[2 * h] = ldg<f4>(ph);
            xv[2 * h + 1] = ldg<f4>(ph + 4);
        }
    };
    // chunks past the end (only in a last, partial step) are staged as zeros
    const bool partial = nch % CPS != 0;
    auto stage = [&](int st, int buf, const typename T::Raw &r) {
        const int c = st * CPS + pc;
        h8 lo, hi;
        piece16h<T>(r, c, ps, lo, hi);
        if (partial && st == nsteps - 1 && c >= nch) lo = hi = h8{};
        *reinterpret_cast<h8 *>(&at[buf][pr][64 * pc + 16 * ps]) = lo;
        *reinterpret_cast<h8 *>(&at[buf][pr][64 * pc + 16 * ps + 8]) = hi;
    };
    // Columns past the batch hold copies of the last column: column i of the
    // product depends on column i of B only, and those are not stored.  In a
    // last, partial step the activations past K are zeroed (the weight tile
    // is zero there, but an infinite activation would still give NaN).
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    auto mma = [&](int st, int buf, const f4 *xv) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float xf[8] = {xv[2 * h].x, xv[2 * h].y, xv[2 * h].z, xv[2 * h].w,
                           xv[2 * h + 1].x, xv[2 * h + 1].y, xv[2 * h + 1].z, xv[2 * h + 1].w};
            if (partial && st == nsteps - 1) {
                const bool in = (int64_t)st * KS + 32 * (2 * wave + h) + 8 * q < K;
#pragma unroll
                for (int e = 0; e < 8; ++e) xf[e] = in ? xf[e] : 0.f;
            }
            const h8 a = *reinterpret_cast<const h8 *>(&at[buf][i][32 * (2 * wave + h) + 8 * q]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pack8(xf), acc, 0, 0, 0);
        }
    };

    typename T::Raw rw[D];
    f4 xx[D][4];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        wload(j, rw[j]);
        xload(j, xx[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // slot j holds step st + j (D is even, so its tile buffer is j % 2); the
    // loop runs while every reload is a real step and has its one exit at the
    // bottom; the last D .. 2D-1 steps follow it.
    int st = 0;
    for (; st + 2 * D <= nsteps; st += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            stage(st + j, j & 1, rw[j]);
            wload(st + j + D, rw[j]);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            mma(st + j, j & 1, xx[j]);
            xload(st + j + D, xx[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
        if (st + j < nsteps) {
            stage(st + j, j & 1, rw[j]);
            if (st + j + D < nsteps) wload(st + j + D, rw[j]);
            lds_barrier();
            mma(st + j, j & 1, xx[j]);
            if (st + j + D < nsteps) xload(st + j + D, xx[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
        if (st + D + j < nsteps) {
            stage(st + D + j, j & 1, rw[j]);
            lds_barrier();
            mma(st + D + j, j & 1, xx[j]);
        }
    }

    // acc element r of lane l is C[4*(l/16) + r][l%16]: weight row 4q + r, column i
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][(4 * q + r) * 16 + i] = acc[r];
    __syncthreads();
    if (tid < RT * 16) {
        const int row = tid >> 4, col = tid & 15;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < KW; ++w) s += part[w][tid];
        if (col < batch && n0 + row < N) Y[(int64_t)col * ldy + n0 + row] = s;
    }
}

template <class T>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
           const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    const int64_t grid = (N + RT - 1) / RT;
    if (grid > 0x7FFFFFFF) return AIH_E_LIMIT;
    hipLaunchKernelGGL((qmv_mfma_kernel<T>), dim3((unsigned)grid), dim3(KW * 64), 0, ctx->stream,
                       W, N, K, row_bytes, X, ldx, Y, ldy, batch);
    return aih_launch_status();
}

}  // namespace

int aih_launch_qmatvec_mfma(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                            const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch<G4K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q6_K: return launch<G6K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q8_0: return launch<G80>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q4_0: return launch<G40>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    default: return AIH_E_UNSUPPORTED;
    }
}
