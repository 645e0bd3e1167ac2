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
// MFMA's A operand are 16 weight rows, the 16 columns of its B operand the
// batch columns (columns past the batch repeat the last one and are not
// stored).  W is read from HBM exactly once whatever the batch.
//
// Work split.  K is cut into 256-element units (one Q4_K/Q6_K super-block,
// eight Q8_0/Q4_0 blocks).  A workgroup of four waves owns 64 weight rows (a
// 16-row MFMA tile per wave) and a contiguous range of units (a split of K);
// a square-ish 4096 x 14336 matrix has only 16 rows per CU, so without the
// split every CU would stream all of X for its 16 rows.  In each round of up
// to UPW units:
//   - the workgroup stages its slice of X (batch columns x 256*UPW k) into
//     LDS as fp16, once for its 64 rows;
//   - lane (i, q) of a wave loads, for weight row i of its tile, the quarter
//     q of every unit (16-byte pieces, the four lanes of a row cover the
//     unit's bytes) and dequantizes it straight into the eight A fragments
//     it feeds, 8 weights each; the element order inside a unit is chosen
//     per format so that every fragment is 8 consecutive elements, and the B
//     fragment is one 16-byte LDS read of X at the same elements;
//   - all loads of a round are issued before the first fragment is built, X
//     first (its staging waits only for X).
// Each workgroup writes its 64 x batch partial sums to a workspace; a second
// kernel adds the splits in a fixed order (the result does not depend on
// timing).  With one split the first kernel stores Y itself.
//
// Dequantization (aih_pieces.h weights8).  A code byte c placed under the
// exponent byte 0x64 is the fp16 value 1024 + c (v_perm_b32 builds two such
// halves from two bytes); one fp32 multiply-add each (v_fma_mix_f32) gives
// (1024 + c) * s - (1024 * s + m) = c * s - m with the reference's scale s and
// offset m (ComputeOps.cs:1629-1678 Q4_K, :1735-1774 Q6_K; GGUF Q8_0/Q4_0),
// rounded to fp16 in pairs (v_cvt_pk_f16_f32).
//
// This replaces TempF32 + ComputeOps.MatMulWeights for M = batch in 3..8
// (AIHost/AIHost/Compute/TransformerBase.cs:254-271, ComputeOps.cs:275-309).
// Precision: weights and activations rounded to fp16, fp32 accumulation.
#include "aih_pieces.h"

namespace {

using namespace aih_pieces;

constexpr int TW = 4;            // waves per workgroup
constexpr int RWG = 16 * TW;     // weight rows per workgroup
constexpr int UNIT = 256;        // k per unit
constexpr int MAXB = 8;          // batch columns

// Weights are read with buffer loads from a resource over the workgroup's 64
// rows: a lane's byte offsets are set up once (Lane), a unit's offset is the
// scalar `so`.  Every weight read stays inside its row, and activation chunks
// outside the batch or K are not loaded.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u4 bld16(Rsrc r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
}
__device__ __forceinline__ uint32_t bld4(Rsrc r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
}
__device__ __forceinline__ uint32_t bld2(Rsrc r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
}

// Per-format unit: lane(rowoff, q) = the lane's offsets for lane group q of a
// row starting at rowoff; load(r, L, so, nb, raw) reads the lane group's bytes
// of the unit at offset so (nb = whole blocks of the unit inside the row);
// frags(raw, q, a) builds the eight A fragments; xoff(q, m) is the unit
// element where fragment m of lane group q starts (8 consecutive elements).

// Q4_K unit = one super-block (d, dmin, scales[12], qs[128]).  Lane group q
// takes 64-group q: the low nibbles of qs[32q .. 32q+31] are elements
// 64q .. 64q+31 (sub-block 2q), the high nibbles 64q+32 .. 64q+63 (sub-block
// 2q+1) (ComputeOps.cs:1642-1675).
struct UQ4K {
    static constexpr int kBytes = 144, kBlocks = 1, kBlockElems = 256;
    struct Lane { uint32_t h, v; };
    struct Raw { u4 hdr, qa, qb; };
    __device__ static Lane lane(uint32_t rowoff, int q) { return {rowoff, rowoff + 16 + 32 * (uint32_t)q}; }
    __device__ static void load(Rsrc r, const Lane &L, uint32_t so, int, int, Raw &w)
    {
        w.hdr = bld16(r, L.h, so);
        w.qa = bld16(r, L.v, so);
        w.qb = bld16(r, L.v + 16, so);
    }
    __device__ static int xoff(int q, int m) { return 64 * q + 8 * m; }
    __device__ static void frags(const Raw &r, int q, h8 *a)
    {
        // get_scale_min_k4 (QuantizationFormats.cs:157-165) for j = 2q, 2q+1:
        // byte t of sc/mn is the 6-bit value of sub-block 2q + t.  scales[]
        // are header bytes 4..15 (hdr.y = scales[0..3], hdr.z = [4..7],
        // hdr.w = [8..11]).
        const int sh = 16 * (q & 1);
        const uint32_t s03 = r.hdr.y >> sh, s47 = r.hdr.z >> sh, s8b = r.hdr.w >> sh;
        const uint32_t sc = q < 2 ? (s03 & 0x3F3Fu) : ((s8b & 0x0F0Fu) | ((s03 >> 2) & 0x3030u));
        const uint32_t mn = q < 2 ? (s47 & 0x3F3Fu) : (((s8b >> 4) & 0x0F0Fu) | ((s47 >> 2) & 0x3030u));
        const float d = f16_bits(r.hdr.x), dmin = f16_bits(r.hdr.x >> 16);
        const float D0 = d * (float)(sc & 0xFFu), M0 = dmin * (float)(mn & 0xFFu);
        const float D1 = d * (float)((sc >> 8) & 0xFFu), M1 = dmin * (float)((mn >> 8) & 0xFFu);
        // a high nibble left in place is 16 * code: scale D1 / 16
        const float s0 = D0, c0 = 1024.f * D0 + M0;
        const float s1 = D1 * 0.0625f, c1 = 1024.f * s1 + M1;
        const uint32_t w[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            a[m] = weights8(w[2 * m] & 0x0F0F0F0Fu, w[2 * m + 1] & 0x0F0F0F0Fu, s0, c0);
            a[m + 4] = weights8(w[2 * m] & 0xF0F0F0F0u, w[2 * m + 1] & 0xF0F0F0F0u, s1, c1);
        }
    }
};

// Q6_K unit = one super-block (ql[128], qh[64], scales[16] int8, d).  Element
// e = 128h + 32Q + l (half h, quarter Q, l < 32) is the nibble Q/2 of
// ql[64h + 32(Q%2) + l] with bits 2Q, 2Q+1 of qh[32h + l] above it, minus 32,
// times d * scales[e/16] (ComputeOps.cs:1748-1771).  Lane group q takes half
// h = q/2, l in [16t, 16t+16) (t = q%2), all four quarters: three 16-byte
// pieces (ql for Q = 0/2, ql for Q = 1/3, qh) and the half's 8 scales.
// Fragment m is quarter m/2, l = 16t + 8(m%2) .. +7.
struct UQ6K {
    static constexpr int kBytes = 210, kBlocks = 1, kBlockElems = 256;
    struct Lane { uint32_t l, h, s, d; };
    struct Raw { u4 la, lb, qh; uint32_t s0, s1, d; };
    __device__ static Lane lane(uint32_t rowoff, int q)
    {
        const uint32_t h = (uint32_t)q >> 1, t = (uint32_t)q & 1;
        return {rowoff + 64 * h + 16 * t, rowoff + 128 + 32 * h + 16 * t, rowoff + 192 + 8 * h, rowoff + 208};
    }
    __device__ static void load(Rsrc r, const Lane &L, uint32_t so, int, int, Raw &w)
    {
        w.la = bld16(r, L.l, so);
        w.lb = bld16(r, L.l + 32, so);
        w.qh = bld16(r, L.h, so);
        w.s0 = bld4(r, L.s, so);
        w.s1 = bld4(r, L.s + 4, so);
        w.d = bld2(r, L.d, so);
    }
    __device__ static int xoff(int q, int m)
    {
        return 128 * (q >> 1) + 32 * (m >> 1) + 16 * (q & 1) + 8 * (m & 1);
    }
    // 6-bit codes of quarter Q for four consecutive l: ql nibble Q/2 of the
    // quarter's ql dword with bits 2Q, 2Q+1 of the qh dword at bits 4, 5
    template <int Q>
    __device__ static uint32_t codes(uint32_t l, uint32_t h)
    {
        if constexpr (Q == 0) return (l & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
        if constexpr (Q == 1) return (l & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
        if constexpr (Q == 2) return ((l >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
        return ((l >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
    template <int Q>
    __device__ static void quarter(const Raw &r, float d, int t, h8 *a)
    {
        // scales[8h + 2Q + t] is byte 2Q + t of the half's eight
        const uint32_t sw = Q < 2 ? r.s0 : r.s1;
        const int sb = (int)(int8_t)(uint8_t)(sw >> (8 * (2 * (Q & 1) + t)));
        const float ds = d * (float)sb, cst = 1056.f * ds;
        const u4 &l = (Q & 1) ? r.lb : r.la;
        a[2 * Q] = weights8(codes<Q>(l.x, r.qh.x), codes<Q>(l.y, r.qh.y), ds, cst);
        a[2 * Q + 1] = weights8(codes<Q>(l.z, r.qh.z), codes<Q>(l.w, r.qh.w), ds, cst);
    }
    __device__ static void frags(const Raw &r, int q, h8 *a)
    {
        const float d = f16_bits(r.d);
        const int t = q & 1;
        quarter<0>(r, d, t, a);
        quarter<1>(r, d, t, a);
        quarter<2>(r, d, t, a);
        quarter<3>(r, d, t, a);
    }
};

// Q8_0 unit = 8 blocks (d, qs[32] int8).  Lane group q takes blocks 2q, 2q+1
// (elements 64q .. 64q+63 in order); y = d * q.  A code biased by 128
// (xor 0x80) gives (1024 + 128 + q) * d - 1152 * d.
struct UQ80 {
    static constexpr int kBytes = 272, kBlocks = 8, kBlockElems = 32;
    struct Lane { uint32_t row, b; };
    struct Raw { u4 q0a, q0b, q1a, q1b; uint32_t d0, d1; };
    __device__ static Lane lane(uint32_t rowoff, int q) { return {rowoff, rowoff + 68 * (uint32_t)q}; }
    __device__ static void load(Rsrc r, const Lane &L, uint32_t so, int q, int nb, Raw &w)
    {
        // a block past the row's end (only in a last, partial unit) re-reads
        // block 0 of the unit, so no read leaves the row, and gets scale 0
        const uint32_t o0 = 2 * q < nb ? L.b : L.row, o1 = 2 * q + 1 < nb ? L.b + 34 : L.row;
        w.q0a = bld16(r, o0 + 2, so);
        w.q0b = bld16(r, o0 + 18, so);
        w.q1a = bld16(r, o1 + 2, so);
        w.q1b = bld16(r, o1 + 18, so);
        w.d0 = 2 * q < nb ? bld2(r, o0, so) : 0u;
        w.d1 = 2 * q + 1 < nb ? bld2(r, o1, so) : 0u;
    }
    __device__ static int xoff(int q, int m) { return 64 * q + 8 * m; }
    __device__ static void frags(const Raw &r, int, h8 *a)
    {
        const float d0 = f16_bits(r.d0), d1 = f16_bits(r.d1);
        const uint32_t w[8] = {r.q0a.x, r.q0a.y, r.q0a.z, r.q0a.w, r.q0b.x, r.q0b.y, r.q0b.z, r.q0b.w};
        const uint32_t v[8] = {r.q1a.x, r.q1a.y, r.q1a.z, r.q1a.w, r.q1b.x, r.q1b.y, r.q1b.z, r.q1b.w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            a[m] = weights8(w[2 * m] ^ 0x80808080u, w[2 * m + 1] ^ 0x80808080u, d0, 1152.f * d0);
            a[m + 4] = weights8(v[2 * m] ^ 0x80808080u, v[2 * m + 1] ^ 0x80808080u, d1, 1152.f * d1);
        }
    }
};

// Q4_0 unit = 8 blocks (d, qs[16]).  Lane group q takes blocks 2q, 2q+1;
// elements 0..15 of a block are the low nibbles of qs[0..15], 16..31 the high
// nibbles; y = d * (q - 8).
struct UQ40 {
    static constexpr int kBytes = 144, kBlocks = 8, kBlockElems = 32;
    struct Lane { uint32_t row, b; };
    struct Raw { u4 q0, q1; uint32_t d0, d1; };
    __device__ static Lane lane(uint32_t rowoff, int q) { return {rowoff, rowoff + 36 * (uint32_t)q}; }
    __device__ static void load(Rsrc r, const Lane &L, uint32_t so, int q, int nb, Raw &w)
    {
        const uint32_t o0 = 2 * q < nb ? L.b : L.row, o1 = 2 * q + 1 < nb ? L.b + 18 : L.row;
        w.q0 = bld16(r, o0 + 2, so);
        w.q1 = bld16(r, o1 + 2, so);
        w.d0 = 2 * q < nb ? bld2(r, o0, so) : 0u;
        w.d1 = 2 * q + 1 < nb ? bld2(r, o1, so) : 0u;
    }
    __device__ static int xoff(int q, int m) { return 64 * q + 8 * m; }
    __device__ static void frags(const Raw &r, int, h8 *a)
    {
        const float dd[2] = {f16_bits(r.d0), f16_bits(r.d1)};
        const u4 qq[2] = {r.q0, r.q1};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float d = dd[b], dh = d * 0.0625f;
            const uint32_t w[4] = {qq[b].x, qq[b].y, qq[b].z, qq[b].w};
            a[4 * b + 0] = weights8(w[0] & 0x0F0F0F0Fu, w[1] & 0x0F0F0F0Fu, d, 1024.f * d + 8.f * d);
            a[4 * b + 1] = weights8(w[2] & 0x0F0F0F0Fu, w[3] & 0x0F0F0F0Fu, d, 1024.f * d + 8.f * d);
            a[4 * b + 2] = weights8(w[0] & 0xF0F0F0F0u, w[1] & 0xF0F0F0F0u, dh, 1024.f * dh + 8.f * d);
            a[4 * b + 3] = weights8(w[2] & 0xF0F0F0F0u, w[3] & 0xF0F0F0F0u, dh, 1024.f * dh + 8.f * d);
        }
    }
};

// Workgroup barrier for LDS traffic only (waits for this wave's LDS
// operations, then for every wave); __syncthreads() would also drain the
// weight loads in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One round: units ub .. ub+R-1 of the split.  WHOLE: every unit lies inside
// the row (always for Q4_K/Q6_K; for Q8_0/Q4_0 all but a last partial unit),
// and the code is straight-line, so that every load of the round is issued
// before the first wait.  Otherwise R = 1 and the unit may be partial (nb
// blocks of it inside the row; elements past K are zero).  The X slice of the
// round is staged in xs (column stride ldx_s halves); X chunk c = tid + 256 j
// of the round is column c / (32 R), elements 8 (c % (32 R)) .. +7, at byte
// offset xo[j] + 1024 ub in xr.  lead: a previous round of this workgroup may
// still be reading xs.
template <class U, int R, bool WHOLE>
__device__ __forceinline__ void round_of(Rsrc wr, const typename U::Lane &L, Rsrc xr, const uint32_t *xo, int ub,
                                         int nb, int64_t K, int batch, _Float16 *xs, int ldx_s, bool lead,
                                         int tid, int q, int bc, f4 &acc)
{
    constexpr int CPC = 32 * R;         // 8-element chunks per column
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
    for (int u = 0; u < R; ++u)
        U::load(wr, L, (uint32_t)(ub + u) * U::kBytes, q, WHOLE ? U::kBlocks : nb, rw[u]);
    __builtin_amdgcn_sched_barrier(0);
    if (lead) lds_barrier();
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int c = tid + TW * 64 * j, col = c / CPC, kc = c % CPC;
        if (col < batch) {
            const float v[8] = {xv[j][0].x, xv[j][0].y, xv[j][0].z, xv[j][0].w,
                                xv[j][1].x, xv[j][1].y, xv[j][1].z, xv[j][1].w};
            *reinterpret_cast<h8 *>(xs + col * ldx_s + 8 * kc) = pack8(v);
        }
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);   // keep the dequantization after the barrier
#pragma unroll
    for (int u = 0; u < R; ++u) {
        h8 a[8];
        U::frags(rw[u], q, a);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const h8 b = *reinterpret_cast<const h8 *>(xs + bc * ldx_s + UNIT * u + U::xoff(q, m));
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b, acc, 0, 0, 0);
        }
    }
}

// Workgroup g: row tile g % ntiles, split g / ntiles, units [split * per,
// min(nunits, (split + 1) * per)) in rounds of UPW units (then single units).
// P != nullptr: partial sums of the split to P[(split * batch + b) * np + n];
// else Y directly.
template <class U, int UPW>
__global__ void __launch_bounds__(TW * 64)
qmv_split_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes, const float *__restrict__ X,
                 int64_t ldx, int batch, int ntiles, int per, float *__restrict__ P, int64_t np,
                 float *__restrict__ Y, int64_t ldy)
{
    constexpr int LDX = UNIT * UPW + 8;   // LDS column stride in halves (16-byte pad)
    __shared__ __align__(16) _Float16 xs[MAXB * LDX];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, q = lane >> 4;
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
    const int rr = min(16 * wave + i, rows - 1);
    const typename U::Lane L = U::lane((uint32_t)(rr * row_bytes), q);
    // activations: a resource over X, a lane's chunk offsets for every round
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
    const int bc = i < batch ? i : batch - 1;   // B column of this lane

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    int ub = ua;
    for (; ub + UPW <= ue_whole; ub += UPW)
        round_of<U, UPW, true>(wr, L, xr, xo, ub, U::kBlocks, K, batch, xs, LDX, ub != ua, tid, q, bc, acc);
    for (; ub < ue; ++ub) {
        const int nb = (int)min<int64_t>(U::kBlocks, nblk - (int64_t)ub * U::kBlocks);
        round_of<U, 1, false>(wr, L, xr, xo1, ub, nb, K, batch, xs, LDX, ub != ua, tid, q, bc, acc);
    }

    // acc[r] = C[4q + r][i]: weight row tile * 64 + 16 * wave + 4q + r, column i
    if (i < batch) {
        const int64_t r0 = row0 + 16 * wave + 4 * q;
        if (P) {
            *reinterpret_cast<f4 *>(P + ((int64_t)split * batch + i) * np + r0) = acc;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r0 + r < N) Y[(int64_t)i * ldy + r0 + r] = acc[r];
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

template <class U>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
           const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    const int64_t ntiles = (N + RWG - 1) / RWG;
    const int64_t nblk = K / U::kBlockElems;
    const int64_t nunits = (nblk + U::kBlocks - 1) / U::kBlocks;
    if (ntiles > 0x7FFFFFFF || nunits > 0x7FFFFFFF) return AIH_E_LIMIT;
    // buffer resources: a tile's rows and all of X within 31-bit offsets
    if (RWG * row_bytes > 0x7FFFFFFF || ((int64_t)(batch - 1) * ldx + K) * 4 > 0x7FFFFFFF) return AIH_E_LIMIT;
    // Splits: about two workgroups per CU (four waves each); measured within a
    // few per cent of one, four and eight per CU at the benchmark shapes.
    const int64_t cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    int64_t S = std::min<int64_t>(nunits, std::max<int64_t>(1, (2 * cu + ntiles - 1) / ntiles));
    int64_t per = (nunits + S - 1) / S;
    S = (nunits + per - 1) / per;
    const int64_t np = ntiles * RWG;
    float *P = nullptr;
    if (S > 1) {
        void *ws = nullptr;
        const int st = aih_workspace(ctx, (size_t)(S * batch * np) * sizeof(float), &ws);
        if (st == AIH_OK) {
            P = static_cast<float *>(ws);
        } else if (st == AIH_E_LIMIT) {
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
        hipLaunchKernelGGL((qmv_split_kernel<U, 4>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    else if (per >= 2)
        hipLaunchKernelGGL((qmv_split_kernel<U, 2>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    else
        hipLaunchKernelGGL((qmv_split_kernel<U, 1>), grid, block, 0, ctx->stream,
                           W, N, K, row_bytes, X, ldx, batch, nt, pr, P, np, Y, ldy);
    int st = aih_launch_status();
    if (st != AIH_OK || !P) return st;
    const int64_t threads = (int64_t)batch * np;
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, ctx->stream,
                       P, np, (int)S, batch, N, Y, ldy);
    return aih_launch_status();
}

}  // namespace

int aih_launch_qmatvec_mfma(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                            const float *X, int64_t ldx, float *Y, int64_t ldy, int batch)
{
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch<UQ4K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q6_K: return launch<UQ6K>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q8_0: return launch<UQ80>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    case AIH_TYPE_Q4_0: return launch<UQ40>(ctx, w, N, K, rb, X, ldx, Y, ldy, batch);
    default: return AIH_E_UNSUPPORTED;
    }
}
