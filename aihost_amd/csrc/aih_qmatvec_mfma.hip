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
// Work split.  A workgroup of eight waves owns a tile of 16 weight rows; wave
// w walks its own eighth of K in 64-element chunks (lane (i, q) dequantizes
// piece q of chunk c of row i: 16 weights, two MFMA k-slices), with the next
// chunk's loads in flight while the current one is computed.  The eight
// partial 16x16 accumulators are summed through LDS.
//
// This replaces TempF32 + ComputeOps.MatMulWeights for M = batch in 3..8
// (AIHost/AIHost/Compute/TransformerBase.cs:254-271, ComputeOps.cs:275-309).
// Precision: weights and activations rounded to fp16, fp32 accumulation.
#include "aih_pieces.h"

namespace {

using namespace aih_pieces;

constexpr int RT = 16;   // weight rows per workgroup (MFMA rows)
constexpr int KW = 8;    // waves per workgroup, each on its own K range

template <class T>
__global__ void __launch_bounds__(KW * 64)
qmv_mfma_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
                const float *__restrict__ X, int64_t ldx, float *__restrict__ Y, int64_t ldy, int batch)
{
    __shared__ float part[KW][RT * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, q = lane >> 4;   // weight row of the tile (A) / column (B); piece
    const int64_t n0 = (int64_t)blockIdx.x * RT;
    const uint8_t *wrow = W + (n0 + i < N ? n0 + i : N - 1) * row_bytes;
    const float *xcol = X + (int64_t)(i < batch ? i : batch - 1) * ldx;
    const int nch = (int)(K / 64);
    const int per = (nch + KW - 1) / KW;
    const int c_begin = wave * per;
    const int c_end = c_begin + per < nch ? c_begin + per : nch;

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if (c_begin < c_end) {   // uniform per wave
        // loads of chunk c (clamped into the wave's range so that no load sits
        // behind a branch)
        auto gl = [&](int c, typename T::Raw &r, f4 *xv) {
            c = c < c_end ? c : c_end - 1;
            T::load(wrow, c, q, r);
            const float *xp = xcol + (int64_t)c * 64 + 16 * q;
#pragma unroll
            for (int t = 0; t < 4; ++t) xv[t] = ldg<f4>(xp + 4 * t);
        };
        // A: weights 16q .. 16q+15 of chunk c of row i; B: the same elements of column i
        auto mm = [&](int c, const typename T::Raw &r, const f4 *xv) {
            float y[16];
            T::piece(r, c, q, y);
            const float xf[16] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w,
                                  xv[2].x, xv[2].y, xv[2].z, xv[2].w, xv[3].x, xv[3].y, xv[3].z, xv[3].w};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pack8(y), pack8(xf), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pack8(y + 8), pack8(xf + 8), acc, 0, 0, 0);
        };
        typename T::Raw ra, rb;
        f4 xa[4], xb[4];
        gl(c_begin, ra, xa);
        int c = c_begin;
        for (; c + 1 < c_end; c += 2) {
            gl(c + 1, rb, xb);
            __builtin_amdgcn_sched_barrier(0);   // next chunk's loads before this chunk's math
            mm(c, ra, xa);
            gl(c + 2, ra, xa);
            __builtin_amdgcn_sched_barrier(0);
            mm(c + 1, rb, xb);
        }
        if (c < c_end) mm(c, ra, xa);
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
