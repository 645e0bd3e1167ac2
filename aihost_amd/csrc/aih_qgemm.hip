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
// MFMA fragment order with a power of two per row (aih_operand.h; the
// conversion is aih_decoder.hip's x_tile_pre_kernel, which also computes the
// element-wise step before the GEMM when there is one).  A
// workgroup then owns a 128 (M) x 64 (N) tile of Y and walks K in super-steps
// of 256 elements: four producer waves dequantize W for the next super-step
// into LDS while four consumer waves multiply the current one, their A
// fragments loaded straight from the tiled X (see qgemm_kernel).  Large grids
// use 256 x 64 or 512 x 64 tiles with every wave in both roles
// (qgemm256_kernel); tall products whose 512-row grid leaves CUs idle split
// K over workgroups and sum the partials in a second pass
// (split_k_sum_kernel).  The epilogue stores Y or adds into it (the residual
// add of a layer).
//
// Precision.  Both operands are rounded to fp16 (11-bit significand) and the
// products accumulate in fp32: normwise error near 3e-4 against the fp32
// reference.  Each activation row carries a power of two that keeps its
// largest value inside fp16's range (aih_operand.h), undone exactly in the
// fp32 epilogue, so that rows above 65504 or far below 1 keep their 11 bits.
// bf16 operands (8-bit significand) would give about 2.4e-3, more than the
// 1e-3 the path is held to.  Weights are dequantized in fp32 with the
// reference's formulas (ComputeOps.cs:1629-1678 for Q4_K, :1735-1774 for Q6_K,
// the GGUF definitions for Q8_0 and Q4_0), computed as one fused fp32
// multiply-add per weight with fp16 output (aih_pieces.h).
#include "aih_pieces.h"
#include "aih_operand.h"

#include <type_traits>

namespace {

using namespace aih_pieces;
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128;          // activation rows per workgroup
constexpr int BN = 64;           // weight rows per workgroup
constexpr int BK = 64;           // K granularity (one 64-element chunk)

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, then for every wave.  __syncthreads() would also wait for the
// global loads in flight (its fences cover global memory), draining the
// prefetch at every step.  The "memory" clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogues: 0 store Y, 1 add into Y, 2 the SiLU-pairs operand (below).
constexpr int kEpiStore = 0, kEpiAccumulate = 1, kEpiSiluOperand = 2, kEpiRopeQKV = 3;

// SiLU(gate) * up of a wave's 32 x 64 output block whose column pairs
// (2j, 2j+1) are gate and up rows (W interleaved), written as the fp16
// operand image of a following GEMM with K = N / 2 (aih_operand.h).  The
// wave's block is one 32-column block of that operand, so each of its rows
// gets its own block exponent; the row exponents are 0, and the image's
// fixup pass (operand_fixup_kernel) brings every row to one exponent before
// that GEMM.  The 32 x 32 fp32 results pass through `lds` (32 rows x 36
// floats, private to the wave) so that every lane writes whole 16-byte
// fragment slots.  Rows at or past M are zero; m0w is the wave's first row,
// n0 the block's first column.  The arithmetic is silu_mul_pairs_kernel's,
// (g * (1 / (1 + e^-g))) * u in fp32, so a row within the unscaled window
// holds the bits the GEMM's own conversion of that kernel's output gives.
__device__ __forceinline__ void silu_pairs_operand(const f16v &acc0, const f16v &acc1, int lane, int64_t m0w,
                                                   int64_t n0, int64_t M, int64_t N, float *lds,
                                                   _Float16 *__restrict__ out)
{
    const int fr = lane & 31, hf = lane >> 5;
    constexpr int LS = 36;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        // the up value of this lane's column pair, from the odd neighbour
        const float u0 = __builtin_amdgcn_update_dpp(0.0f, acc0[r], 0xB1, 0xF, 0xF, false);
        const float u1 = __builtin_amdgcn_update_dpp(0.0f, acc1[r], 0xB1, 0xF, 0xF, false);
        if ((fr & 1) == 0) {
            const int i = 8 * (r >> 2) + 4 * hf + (r & 3);
            const float g0 = acc0[r], g1 = acc1[r];
            lds[i * LS + (fr >> 1)] = (g0 * (1.0f / (1.0f + expf(-g0)))) * u0;
            lds[i * LS + 16 + (fr >> 1)] = (g1 * (1.0f / (1.0f + expf(-g1)))) * u1;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane: row fr of the block, outputs 16 hf .. 16 hf + 15 (two slots)
    const int64_t m = m0w + fr;
    const int64_t mpad = aih_operand::mpad_of(M);
    if (m >= mpad) return;   // both lanes of a row (fr, fr + 32) alike
    f4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        v[q] = m < M ? *reinterpret_cast<const f4 *>(&lds[fr * LS + 16 * hf + 4 * q]) : f4{0.f, 0.f, 0.f, 0.f};
    float mx = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[q].x), fabsf(v[q].y)), fmaxf(fabsf(v[q].z), fabsf(v[q].w))));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int eb = aih_operand::block_exp(mx), e = eb == aih_operand::kZeroBlock ? 0 : eb;
    const int64_t kd = N / 2;
    const int64_t k0 = n0 / 2 + 16 * hf;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        h8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (_Float16)ldexpf(v[2 * q + j / 4][j % 4], e);
        *reinterpret_cast<h8 *>(out + aih_operand::slot_half(m, k0 + 8 * q, kd)) = h;
    }
    char *const img = reinterpret_cast<char *>(out);
    if (hf == 0) {
        reinterpret_cast<int8_t *>(img + aih_operand::block_exp_offset(mpad, kd))[m * (kd / 32) + n0 / 64] = (int8_t)eb;
        if (n0 == 0) reinterpret_cast<int32_t *>(img + aih_operand::row_exp_offset(mpad, kd))[m] = 0;
    }
}

// The row exponents of the operand (aih_operand.h) undone in a wave's 32 x 32
// accumulator: lane l holds rows 8 (r / 4) + 4 (l / 32) + r % 4 of the
// wave's 32 rows from row mrow0, whose exponents start at E + mrow0.  `ev`,
// loaded when the kernel started, is lane l's row l % 32 exponent: when all
// are zero (rows within the unscaled window) nothing is done.
typedef int32_t i4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void undo_row_exp(f16v &acc0, f16v &acc1, int32_t ev, const int32_t *E, int64_t mrow0,
                                             int lane)
{
    if (__builtin_amdgcn_ballot_w64(ev != 0) == 0) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const i4 e = *reinterpret_cast<const i4 *>(E + mrow0 + 8 * q + 4 * (lane >> 5));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc0[4 * q + j] = ldexpf(acc0[4 * q + j], -e[j]);
            acc1[4 * q + j] = ldexpf(acc1[4 * q + j], -e[j]);
        }
    }
}

// A wave's two 32 x 32 accumulators stored into Y (rows mrow0 .., columns
// n0 + lane % 32 and n0 + 32 + lane % 32), or added into it (Y + acc, the
// operand order of aih_add).  A block wholly inside Y is written without
// per-value guards, and for the add all 32 of its lane's Y values are loaded
// before the first add, so that they are in flight together rather than one
// round trip per register.  On MI355X, 4096 x 4096 x 512 per call: the
// accumulate epilogue 42.5 -> 33.5-34.4 us (the guarded form cost 3-5 us
// over a plain store).
__device__ __forceinline__ void store_tile(const f16v &acc0, const f16v &acc1, int lane, int64_t mrow0, int64_t n0,
                                           int64_t M, int64_t N, float *__restrict__ Y, bool accumulate)
{
    const int64_t na = n0 + (lane & 31), nb = na + 32;
    auto row = [&](int r) { return mrow0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); };
    if (mrow0 + 32 <= M && n0 + 64 <= N) {
        if (accumulate) {
            float ya[16], yb[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                ya[r] = Y[row(r) * N + na];
                yb[r] = Y[row(r) * N + nb];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                Y[row(r) * N + na] = ya[r] + acc0[r];
                Y[row(r) * N + nb] = yb[r] + acc1[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                Y[row(r) * N + na] = acc0[r];
                Y[row(r) * N + nb] = acc1[r];
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t m = row(r);
        if (m < M) {
            if (na < N) Y[m * N + na] = accumulate ? Y[m * N + na] + acc0[r] : acc0[r];
            if (nb < N) Y[m * N + nb] = accumulate ? Y[m * N + nb] + acc1[r] : acc1[r];
        }
    }
}

// The Q|K|V epilogue (aih_rope_qkv_args): a wave's two 32 x 32 blocks
// (rows mrow0 .., columns n0 + lane % 32 and + 32) rotated and stored as
// aih_rope_qkv would rotate and store the stored product: for query and key
// columns the pair (2i, 2i + 1) of a head (adjacent lanes) becomes
// (x0 c - x1 s, x0 s + x1 c) with (c, s) the table's row p, pair i; queries
// go to Y (unrotated when p is outside the table), keys and values to the
// caches' row p (nothing outside the table or past the cache).  The head
// boundaries fall on multiples of 32 columns, so a block is one kind.
__device__ __forceinline__ void rope_qkv_block(const f16v acc, int lane, int64_t mrow0, int64_t nb0, int64_t M,
                                               int64_t N, float *__restrict__ Y, const aih_rope_qkv_args ra)
{
#pragma clang fp contract(off)
    if (nb0 >= N) return;
    const int32_t p0 = ra.start + (ra.pos ? *ra.pos : 0);
    const int64_t n = nb0 + (lane & 31);
    // query, key or value: the same for the whole block (wave-uniform)
    const int kind = nb0 < ra.qd ? 0 : nb0 < (int64_t)ra.qd + ra.kvd ? 1 : 2;
    const int64_t cn = kind == 0 ? n : kind == 1 ? n - ra.qd : n - ra.qd - ra.kvd;
    auto row = [&](int r) { return mrow0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); };
    if (kind == 2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t m = row(r), p = (int64_t)p0 + m;
            if (m < M && p >= 0 && p < ra.table_rows && p < ra.cache_rows) ra.Vc[p * ra.kvd + cn] = acc[r];
        }
        return;
    }
    // the rows' cos/sin, all loads issued before the first use (rows outside
    // the table read row 0 and are not rotated)
    const int half = ra.head_dim / 2;
    const int i = (int)(cn % ra.head_dim) / 2;
    float cv[16], sv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t p = (int64_t)p0 + row(r);
        const int64_t pt = p >= 0 && p < ra.table_rows ? p : 0;
        const float2 t = *reinterpret_cast<const float2 *>(ra.table + 2 * (pt * half + i));
        cv[r] = t.x;
        sv[r] = t.y;
    }
    const bool odd = lane & 1;
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        // the pair's other element, from the neighbouring lane
        const float other = __builtin_amdgcn_update_dpp(0.0f, acc[r], 0xB1, 0xF, 0xF, false);
        const float x0 = odd ? other : acc[r], x1 = odd ? acc[r] : other;
        v[r] = odd ? x0 * sv[r] + x1 * cv[r] : x0 * cv[r] - x1 * sv[r];
    }
    if (kind == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t m = row(r), p = (int64_t)p0 + m;
            if (m < M) Y[m * N + n] = p >= 0 && p < ra.table_rows ? v[r] : acc[r];
        }
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t m = row(r), p = (int64_t)p0 + m;
            if (m < M && p >= 0 && p < ra.table_rows && p < ra.cache_rows) ra.Kc[p * ra.kvd + cn] = v[r];
        }
    }
}

__device__ __forceinline__ void rope_qkv_tile(const f16v &acc0, const f16v &acc1, int lane, int64_t mrow0, int64_t n0,
                                              int64_t M, int64_t N, float *__restrict__ Y,
                                              const aih_rope_qkv_args ra)
{
    rope_qkv_block(acc0, lane, mrow0, n0, M, N, Y, ra);
    rope_qkv_block(acc1, lane, mrow0, n0 + 32, M, N, Y, ra);
}

// Eight waves per workgroup in two roles, one of each on every SIMD; the
// workgroup owns a 128 (M) x 64 (N) tile of Y and walks K in super-steps of
// 256 (a Q4_K/Q6_K super-block, 8 blocks of Q8_0/Q4_0), with one LDS barrier
// per super-step and two tile buffers.
//   Producers (waves 4..7) dequantize the next super-step of the 64 weight
//   rows into LDS: wave p owns rows 16p .. 16p+15.  For Q4_K, Q4_0 and Q8_0
//   eight lanes per row take 32 weights each (the wide-tile kernel's pieces
//   and LDS positions: two row groups of 8 per wave); for Q6_K sixteen lanes
//   per row take pieces 0..15 of the row's 256-k span (four row groups of 4,
//   each row read as one contiguous span), which measured faster there
//   (4096 x 4096 x 512: 39.9 against 40.5 us per call; the 32-weight form
//   gave Q4_0 36.2 -> 34.6 and Q8_0 36.5 -> 35.9).  Their packed loads run
//   PR super-steps ahead in a ring of register sets.
//   Consumers (waves 0..3): wave w owns rows 32w .. 32w+31 of the M tile and
//   all 64 columns (two 32x32 accumulators sharing each A fragment).  A
//   fragments come straight from the tiled fp16 copy of X, one super-step
//   ahead; B fragments from LDS.
// On MI355X the 4096 x 4096 x 512 Q4_K product takes 35-37 us per call (the
// kernel 27-28 us, the X conversion 7.5 us), against 42 us for an earlier
// form with one barrier per 64 k.
constexpr int SK = 256;            // k per super-step (one barrier)
constexpr int SC = SK / 64;        // 64-k steps per super-step
constexpr int LD2 = SK + 8;        // LDS row stride in halves (16-byte pad against bank conflicts)
// producer ring depth in super-steps (Q6_K's larger raw sets: 2, within 256
// registers) and piece layout (P32: 32-weight pieces, else 16-weight)
template <class T> struct GRing { static constexpr int PR = 3; static constexpr bool P32 = true; };
template <> struct GRing<G6K> { static constexpr int PR = 2; static constexpr bool P32 = false; };

// LDS position (in 16-byte granules) of chunk granule g of a super-step (the
// k values 8g .. 8g+7): the 32-weight pieces' swizzle, or for 16-weight
// pieces s of chunk c (granules 8c + 2s, + 1) 4c + s and 16 + 4c + s, so that
// the 16 lanes of a row store 256 contiguous bytes
template <class T, bool P32 = GRing<T>::P32> struct BPos {
    __device__ static constexpr int pos(int g) { return Piece32<T>::type::swz(g); }
};
template <class T> struct BPos<T, false> {
    __device__ static constexpr int pos(int g) { return 16 * (g & 1) + 4 * (g >> 3) + ((g >> 1) & 3); }
};

template <class T>
__global__ void __launch_bounds__(512)
qgemm_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
             const _Float16 *__restrict__ Xt, int64_t M, float *__restrict__ Y, int epi, aih_rope_qkv_args ra)
{
    constexpr int PR = GRing<T>::PR;
    constexpr bool P32 = GRing<T>::P32;
    typedef typename Piece32<T>::type Pc;
    typedef std::conditional_t<P32, typename Pc::Raw, typename T::Raw> Raw;
    constexpr int NR = P32 ? 2 : 4;   // row groups per producer wave
    __shared__ __align__(16) _Float16 wsh[2][BN][LD2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int nch = (int)(K / 64);
    const int nss = (nch + SC - 1) / SC;

    if (wave >= 4) {
        // rows 16 pw + (16 / NR) i + rl; P32: chunk pc, half ps of it (32
        // weights); else chunk pc, piece ps (16 weights)
        const int pw = wave - 4;
        constexpr int LPR = 64 * NR / 16;   // lanes per row
        const int rl = lane / LPR, p = lane % LPR, pc = p / (LPR / 4), ps = p % (LPR / 4);
        const uint8_t *wrow[NR];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int64_t wn = n0 + 16 * pw + (16 / NR) * i + rl;
            wrow[i] = W + (wn < N ? wn : N - 1) * row_bytes;
        }
        auto gload = [&](int ss, Raw *r) {
            int c = ss * SC + pc;
            c = c < nch ? c : nch - 1;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                if constexpr (P32) Pc::load(wrow[i], c, ps, r[i]);
                else T::load(wrow[i], c, ps, r[i]);
            }
        };
        // chunks past K exist only in a last, partial super-step, staged as
        // zeros: only the stages after the main loop test for them
        auto stage = [&](auto tail, int ss, int buf, const Raw *r) {
            asm volatile("" : "+s"(ss));
            const int c = ss * SC + pc;
            const bool zero = decltype(tail)::value && c >= nch;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                _Float16 *d = &wsh[buf][16 * pw + (16 / NR) * i + rl][0];
                if constexpr (P32) {
                    h8 o[4];
                    Pc::piece(r[i], c, ps, o);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<h8 *>(d + 8 * Pc::swz(8 * pc + Pc::col(ps, q) / 8)) = zero ? h8{} : o[q];
                } else {
                    h8 lo, hi;
                    piece16h<T>(r[i], c, ps, lo, hi);
                    *reinterpret_cast<h8 *>(d + 8 * BPos<T>::pos(8 * pc + 2 * ps)) = zero ? h8{} : lo;
                    *reinterpret_cast<h8 *>(d + 8 * BPos<T>::pos(8 * pc + 2 * ps + 1)) = zero ? h8{} : hi;
                }
            }
        };
        Raw ring[PR][NR];
#pragma unroll
        for (int j = 0; j < PR; ++j) gload(j, ring[j]);
        __builtin_amdgcn_sched_barrier(0);
        int ss = 0;
        for (; ss + 2 * PR <= nss; ss += PR) {
#pragma unroll
            for (int j = 0; j < PR; ++j) {
                stage(std::false_type{}, ss + j, (ss + j) & 1, ring[j]);
                gload(ss + j + PR, ring[j]);
                __builtin_amdgcn_sched_barrier(0);
                lds_barrier();
            }
        }
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            if (ss + j < nss) {
                stage(std::true_type{}, ss + j, (ss + j) & 1, ring[j]);
                if (ss + j + PR < nss) gload(ss + j + PR, ring[j]);
                lds_barrier();
            }
        }
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            if (ss + PR + j < nss) {
                stage(std::true_type{}, ss + PR + j, (ss + PR + j) & 1, ring[j]);
                lds_barrier();
            }
        }
        return;
    }

    // consumer wave w: rows 32w .. 32w+31 of the M tile, all 64 columns
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const int64_t kc = K / 16, mblocks = (M + 31) / 32;
    int64_t mb = (m0 + 32 * wave) / 32;
    mb = mb < mblocks ? mb : mblocks - 1;
    const _Float16 *xa = Xt + (mb * kc * 64 + lane) * 8;
    // the row exponents of the operand, after its mblocks * 32 rows of values
    const int32_t *const E = reinterpret_cast<const int32_t *>(Xt + mblocks * 32 * K);
    const int32_t ev = E[mb * 32 + (lane & 31)];
    struct AF { h8 a[4]; };
    auto aload = [&](int kb, AF &f) {
        kb = kb < nch ? kb : nch - 1;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) f.a[kk] = ldg<h8>(xa + ((int64_t)kb * 4 + kk) * 512);
    };
    f16v acc0 = {}, acc1 = {};
    // B fragments of one 64-k step (both 32-column halves, four k16 slices),
    // read from LDS one step ahead of their MFMAs so that the reads' latency
    // is covered by the previous step's matrix work
    struct BF { h8 b0[4], b1[4]; };
    auto bload = [&](int buf, int t, BF &b) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            b.b0[kk] = *reinterpret_cast<const h8 *>(&wsh[buf][fr][8 * BPos<T>::pos(8 * t + 2 * kk + fk / 8)]);
            b.b1[kk] = *reinterpret_cast<const h8 *>(&wsh[buf][32 + fr][8 * BPos<T>::pos(8 * t + 2 * kk + fk / 8)]);
        }
    };
    auto mm = [&](const AF &f, const BF &b) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[kk], b.b0[kk], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[kk], b.b1[kk], acc1, 0, 0, 0);
        }
    };
    // A ring of one super-step: slot t holds 64-k step SC*ss + t
    AF f[SC];
#pragma unroll
    for (int t = 0; t < SC; ++t) aload(t, f[t]);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    BF bb[2];
    int ss = 0;
    for (; ss + 2 <= nss; ++ss) {
        const int buf = ss & 1;
        bload(buf, 0, bb[0]);
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t + 1 < SC) bload(buf, t + 1, bb[(t + 1) & 1]);
            mm(f[t], bb[t & 1]);
            aload(SC * (ss + 1) + t, f[t]);
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_barrier();
    }
    {
        const int buf = ss & 1;
        bload(buf, 0, bb[0]);
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t + 1 < SC && SC * ss + t + 1 < nch) bload(buf, t + 1, bb[(t + 1) & 1]);
            if (SC * ss + t < nch) mm(f[t], bb[t & 1]);
        }
    }

    undo_row_exp(acc0, acc1, ev, E, mb * 32, lane);
    if (epi == kEpiSiluOperand) {
        // the tile buffer of super-step nss: nothing reads or writes it any more
        silu_pairs_operand(acc0, acc1, lane, m0 + 32 * wave, n0, M, N,
                           reinterpret_cast<float *>(&wsh[nss & 1][0][0]) + wave * 32 * 36,
                           reinterpret_cast<_Float16 *>(Y));
        return;
    }
    if (epi == kEpiRopeQKV) {
        rope_qkv_tile(acc0, acc1, lane, m0 + 32 * wave, n0, M, N, Y, ra);
        return;
    }
    store_tile(acc0, acc1, lane, m0 + 32 * wave, n0, M, N, Y, epi == kEpiAccumulate);
}

// Wide tiles for large products: a workgroup of eight waves owns a 256 MB (M)
// x 64 (N) tile (MB = 1 or 2), so each dequantized weight feeds 2 MB times as
// many outputs as in qgemm_kernel.  Every wave takes both roles in each
// super-step s:
//   - it dequantizes its 8 of the 64 weight rows (row 8w + lane / 8) for
//     super-step s+1 into the other LDS buffer, 32 weights per lane
//     (Piece32), from packed loads PR256 super-steps ahead;
//   - it multiplies super-step s: wave w owns rows 32 MB w .. +32 MB - 1 of
//     the M tile and all 64 columns (2 MB 32x32 accumulators: each A fragment
//     feeds two, each B fragment MB), A fragments from the tiled X AD 64-k
//     chunks ahead, B fragments from LDS.
// The two waves of a SIMD (w and w + 4) run the two halves in opposite
// orders, so that one dequantizes while the other multiplies.  On MI355X a
// 256-row workgroup takes about 1.25 times as long as a 128-row one, for
// twice the outputs.
constexpr int BM2 = 256;
constexpr int PR256 = 2;

template <class T, int MB, int AD>
__global__ void __launch_bounds__(512)
qgemm256_kernel(const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
                const _Float16 *__restrict__ Xt, int64_t M, float *__restrict__ Y, int epi,
                float *__restrict__ P, int ssper, aih_rope_qkv_args ra)
{
    static_assert(SC % AD == 0, "A ring depth divides a super-step");
    constexpr int PR = PR256;
    typedef typename Piece32<T>::type Pc;
    typedef typename Pc::Raw Raw;
    __shared__ __align__(16) _Float16 wsh[2][BN][LD2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM2 * MB, n0 = (int64_t)blockIdx.x * BN;
    const int nch = (int)(K / 64);
    // split z of K (gridDim.z > 1: partial sums into P): super-steps
    // ss0 .. ss0 + nss - 1; chunk indices below stay absolute
    const int ss0 = (int)blockIdx.z * ssper;
    const int nss = min(ssper, (nch + SC - 1) / SC - ss0);

    // dequantization share: row 8 wave + rl, 32 weights per lane (chunk pc, half ph)
    const int rl = lane >> 3, p = lane & 7, pc = p >> 1, ph = p & 1;
    const int64_t wn = n0 + 8 * wave + rl;
    const uint8_t *wrow = W + (wn < N ? wn : N - 1) * row_bytes;
    auto gload = [&](int ss, Raw *r) {
        int c = (ss0 + ss) * SC + pc;
        c = c < nch ? c : nch - 1;
        Pc::load(wrow, c, ph, r[0]);
    };
    // chunks past K exist only in a last, partial super-step, staged as zeros
    auto stage = [&](auto tail, int ss, int buf, const Raw *r) {
        const int c = (ss0 + ss) * SC + pc;
        h8 o[4];
        Pc::piece(r[0], c, ph, o);
        _Float16 *d = &wsh[buf][8 * wave + rl][0];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<h8 *>(d + 8 * Pc::swz(8 * pc + Pc::col(ph, q) / 8)) =
                decltype(tail)::value && c >= nch ? h8{} : o[q];
    };

    // multiplication share: rows 32 MB wave .. +32 MB - 1 of the M tile
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const int64_t kc = K / 16, mblocks = (M + 31) / 32;
    const _Float16 *xa[MB];
    const int32_t *const E = reinterpret_cast<const int32_t *>(Xt + mblocks * 32 * K);
    int32_t ev[MB];   // the row exponents of the operand (lane: row lane % 32 of fragment j)
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        int64_t mb = (m0 + 32 * (MB * wave + j)) / 32;
        mb = mb < mblocks ? mb : mblocks - 1;
        xa[j] = Xt + (mb * kc * 64 + lane) * 8;
        ev[j] = E[mb * 32 + (lane & 31)];
    }
    struct AF { h8 a[MB][4]; };
    auto aload = [&](int kb, AF &f) {
        kb += SC * ss0;
        kb = kb < nch ? kb : nch - 1;
#pragma unroll
        for (int j = 0; j < MB; ++j)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) f.a[j][kk] = ldg<h8>(xa[j] + ((int64_t)kb * 4 + kk) * 512);
    };
    f16v acc[MB][2] = {};
    struct BF { h8 b0[4], b1[4]; };
    auto bload = [&](int buf, int t, BF &b) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            b.b0[kk] = *reinterpret_cast<const h8 *>(&wsh[buf][fr][8 * Pc::swz(8 * t + 2 * kk + fk / 8)]);
            b.b1[kk] = *reinterpret_cast<const h8 *>(&wsh[buf][32 + fr][8 * Pc::swz(8 * t + 2 * kk + fk / 8)]);
        }
    };
    auto mm = [&](const AF &f, const BF &b) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int j = 0; j < MB; ++j) {
                acc[j][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[j][kk], b.b0[kk], acc[j][0], 0, 0, 0);
                acc[j][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[j][kk], b.b1[kk], acc[j][1], 0, 0, 0);
            }
    };

    // Iteration it: products of super-step it from buffer it & 1, and, if
    // `more`, the dequantization of super-step it + 1 into the other buffer
    // from ring slot r, whose loads are then reissued for super-step
    // it + 1 + PR when `reload`.
    Raw ring[PR][1];
    AF f[AD];   // chunk g of the A operand in f[g % AD]
    constexpr int BD = MB == 1 ? 2 : 1;   // B chunks in registers (the next one loaded early when 2)
    BF bb[BD];
    // The two waves of a SIMD (w and w + 4) take the two halves in opposite
    // orders, so that one dequantizes while the other multiplies.
    const bool valu_first = wave < 4;
    auto body = [&](auto tail, int it, Raw *r, bool more, bool reload) {
        const int buf = it & 1;
        auto deq = [&] {
            if (more) {
                stage(tail, it + 1, buf ^ 1, r);
                if (reload) gload(it + 1 + PR, r);
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        if (BD == 2) bload(buf, 0, bb[0]);
        if (valu_first) deq();
        // the multiplying half at raised wave priority, so that the SIMD
        // issues its MFMAs ahead of the other wave's dequantization when both
        // are ready (6144 x 4096 and 28672 x 4096 at M = 512: 2% faster)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (BD == 1)
                bload(buf, t, bb[0]);
            else if (t + 1 < SC)
                bload(buf, t + 1, bb[(t + 1) % BD]);
            __builtin_amdgcn_sched_barrier(0);
            mm(f[t % AD], bb[t % BD]);
            aload(SC * it + t + AD, f[t % AD]);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (!valu_first) deq();
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
    };

#pragma unroll
    for (int j = 0; j < PR; ++j) gload(j, ring[j]);
#pragma unroll
    for (int t = 0; t < AD; ++t) aload(t, f[t]);
    stage(std::true_type{}, 0, 0, ring[0]);
    gload(PR, ring[0]);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    // iteration it stages super-step it + 1 from ring slot (it + 1) % PR; the
    // main loop's stages are all full super-steps before the last
    int ss = 0;
    for (; ss + PR + 1 < nss; ss += PR) {
#pragma unroll
        for (int j = 0; j < PR; ++j) body(std::false_type{}, ss + j, ring[(j + 1) % PR], true, true);
    }
#pragma unroll
    for (int j = 0; j <= PR; ++j) {
        const int it = ss + j;
        if (it < nss) body(std::true_type{}, it, ring[(j + 1) % PR], it + 1 < nss, it + 1 + PR < nss);
    }

#pragma unroll
    for (int j = 0; j < MB; ++j) {
        int64_t mb = (m0 + 32 * (MB * wave + j)) / 32;
        mb = mb < mblocks ? mb : mblocks - 1;
        undo_row_exp(acc[j][0], acc[j][1], ev[j], E, mb * 32, lane);
    }
    if (epi == kEpiSiluOperand) {
        // after the last barrier the tile buffers are free
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            silu_pairs_operand(acc[j][0], acc[j][1], lane, m0 + 32 * (MB * wave + j), n0, M, N,
                               reinterpret_cast<float *>(&wsh[0][0][0]) + wave * 32 * 36,
                               reinterpret_cast<_Float16 *>(Y));
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the block is read before it is rewritten
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        return;
    }
    if (epi == kEpiRopeQKV) {   // never split (the plan does not split this epilogue)
#pragma unroll
        for (int j = 0; j < MB; ++j) rope_qkv_tile(acc[j][0], acc[j][1], lane, m0 + 32 * (MB * wave + j), n0, M, N, Y, ra);
        return;
    }
    // a split's partial sums are stored (the summing pass adds them into Y)
    float *const Pz = P ? P + (int64_t)blockIdx.z * M * N : nullptr;
#pragma unroll
    for (int j = 0; j < MB; ++j)
        store_tile(acc[j][0], acc[j][1], lane, m0 + 32 * (MB * wave + j), n0, M, N, Pz ? Pz : Y,
                   !Pz && epi == kEpiAccumulate);
}

// The splits of a GEMM split over K: Y = P_0 + P_1 + ... (in that order),
// added into Y (Y + sum, the order of the accumulate epilogue) when
// `accumulate`.  Four elements per thread (16-byte accesses of Y when it is
// 16-byte aligned).
template <bool VEC>
__global__ void __launch_bounds__(256)
split_k_sum_kernel(const float *__restrict__ P, int S, int64_t MN, float *__restrict__ Y, int accumulate)
{
    for (int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x); i < MN; i += 4 * (int64_t)gridDim.x * 256) {
        f4 s = *reinterpret_cast<const f4 *>(P + i);
        for (int z = 1; z < S; ++z) s += *reinterpret_cast<const f4 *>(P + (int64_t)z * MN + i);
        if (VEC) {
            f4 *y = reinterpret_cast<f4 *>(Y + i);
            *y = accumulate ? *y + s : s;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) Y[i + j] = accumulate ? Y[i + j] + s[j] : s[j];
        }
    }
}

// Before a GEMM reads an image written one 32-column block at a time
// (aih_operand.h), every row is brought to one exponent: one wave per row.
// A row whose block exponents are all 0 (or mark all-zero blocks) -- its
// values within the unscaled window -- is left as it is.  Otherwise each
// block of exponent d is scaled to the row's smallest exponent D (the block
// of its largest values): every half multiplied by 2^(D - d) <= 1 in fp32
// (exact) and rounded to fp16 once; then E[m] += D and the block exponents
// become 0, so a second pass changes nothing.
__global__ void __launch_bounds__(256)
operand_fixup_kernel(_Float16 *__restrict__ Xt, int64_t mpad, int64_t K)
{
    const int lane = threadIdx.x & 63;
    const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= mpad) return;
    const int64_t nb = K / 32;   // a multiple of 2 (K % 64 == 0)
    char *const img = reinterpret_cast<char *>(Xt);
    int8_t *const d = reinterpret_cast<int8_t *>(img + aih_operand::block_exp_offset(mpad, K)) + m * nb;
    int mn = 127;
    bool odd = false;
    // the row's exponents two at a time (rows start 2-byte aligned), the loads
    // of four passes issued together (K up to 16384 in one round trip)
#pragma unroll 4
    for (int64_t b = 2 * lane; b < nb; b += 128) {
        const uint16_t w2 = *reinterpret_cast<const uint16_t *>(d + b);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int v = (int8_t)(w2 >> (8 * j));
            if (v != aih_operand::kZeroBlock) {
                mn = min(mn, v);
                odd = odd || v != 0;
            }
        }
    }
    if (__builtin_amdgcn_ballot_w64(odd) == 0) return;
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mn = min(mn, __shfl_xor(mn, s));
    for (int64_t b = lane; b < nb; b += 64) {
        const int v = d[b];
        if (v != aih_operand::kZeroBlock && v != mn) {
            const float f = ldexpf(1.f, mn - v);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                h8 *const p = reinterpret_cast<h8 *>(Xt + aih_operand::slot_half(m, 32 * b + 8 * q, K));
                h8 h = *p;
#pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = (_Float16)((float)h[j] * f);
                *p = h;
            }
        }
        d[b] = 0;
    }
    if (lane == 0) reinterpret_cast<int32_t *>(img + aih_operand::row_exp_offset(mpad, K))[m] += mn;
}

// The tiling of a GEMM: rows per workgroup tile (128, 256 or 512) and, for
// 512-row tiles, the number of K splits (splits > 1: partial sums in the
// second workspace, then split_k_sum_kernel) of ssper super-steps each.
struct GemmPlan {
    int tile = 128;
    int splits = 1;
    int ssper = 0;
};

// 256-row tiles halve the dequantization per output and 512-row tiles halve
// it again; a workgroup of them takes about 1.25 and 2.35 times as long as
// one of 128 rows (measured on MI355X).  The shape with the fewest such
// rounds of workgroups over the device's CUs wins (ties to the smaller tile).
// Costs in units of 1/20 of a 128-row workgroup.  Products of more than 256
// rows whose 512-row tiles leave CUs idle split K over workgroups: S splits
// of at least two whole super-steps, partial sums in the second workspace,
// then a summing pass (estimated at 5 TB/s over the partials, Y and the
// output, plus 2 us of launch; a 128-row workgroup takes about 29 us per
// 4096 of K).  The plan depends only on the shape, the epilogue, the CU count
// and whether the call may split, never on what the context has allocated.
GemmPlan plan_gemm(int64_t cu_count, int64_t N, int64_t K, int64_t M, int epi, bool may_split)
{
    const int64_t gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM, gy2 = (M + BM2 - 1) / BM2;
    const int64_t gy4 = (M + 2 * BM2 - 1) / (2 * BM2);
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    auto rounds = [&](int64_t wgs) { return (double)((wgs + cus - 1) / cus); };
    const double c1 = 20 * rounds(gx * gy), c2 = 25 * rounds(gx * gy2), c4 = 47 * rounds(gx * gy4);
    const int nss = (int)((K / 64 + SC - 1) / SC);
    GemmPlan p;
    p.ssper = nss;
    if (may_split && epi != kEpiSiluOperand && epi != kEpiRopeQKV && M > BM2 && gx * gy4 < cus && M * N % 4 == 0) {
        const int want = (int)std::min<int64_t>(std::min<int64_t>(cus / (gx * gy4), nss / 2), 8);
        if (want >= 2) {
            const int ssper = (nss + want - 1) / want;
            const int S = (nss + ssper - 1) / ssper;
            const double unit_us = 29.0 * (double)K / 4096.0 / 20.0;
            const double sum_us = (double)(S + 2) * (double)(M * N) * 4.0 / 5e12 * 1e6 + 2.0;
            const double cs = 47 * rounds(gx * gy4 * S) * (double)ssper / (double)nss + sum_us / unit_us;
            if (S > 1 && cs < c1 && cs < c2 && cs < c4) {
                p.tile = 512;
                p.splits = S;
                p.ssper = ssper;
                return p;
            }
        }
    }
    p.tile = c4 < c2 && c4 < c1 ? 512 : c2 < c1 ? 256 : 128;
    return p;
}

template <class T>
int launch(aih_ctx *ctx, const uint8_t *W, int64_t N, int64_t K, int64_t row_bytes,
           const _Float16 *Xh, int64_t M, float *Y, int epi, bool may_split, const aih_rope_qkv_args &ra)
{
    const int64_t gx = (N + BN - 1) / BN, gy = (M + BM - 1) / BM, gy2 = (M + BM2 - 1) / BM2;
    const int64_t gy4 = (M + 2 * BM2 - 1) / (2 * BM2);
    if (gy > 65535 || gx > 0x7FFFFFFF) return AIH_E_LIMIT;
    const GemmPlan p = plan_gemm(ctx->cu_count, N, K, M, epi, may_split);
    if (p.splits > 1) {
        // the split's partial sums: a shape that splits always splits (a
        // workspace that cannot grow here, as during a graph capture, is an
        // error, not a silent change of summation order)
        void *ws = nullptr;
        int rc = aih_workspace2(ctx, (size_t)p.splits * (size_t)(M * N) * sizeof(float), &ws);
        if (rc) return rc;
        hipLaunchKernelGGL((qgemm256_kernel<T, 2, 2>), dim3((unsigned)gx, (unsigned)gy4, (unsigned)p.splits),
                           dim3(512), 0, ctx->stream, W, N, K, row_bytes, Xh, M, Y, epi, static_cast<float *>(ws),
                           p.ssper, ra);
        rc = aih_launch_status();
        if (rc) return rc;
        const int64_t cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
        const int64_t groups = (M * N / 4 + 255) / 256;
        const dim3 grid((unsigned)std::min<int64_t>(groups, 8 * cus));
        if (reinterpret_cast<uintptr_t>(Y) % 16 == 0)
            hipLaunchKernelGGL(split_k_sum_kernel<true>, grid, dim3(256), 0, ctx->stream,
                               static_cast<const float *>(ws), p.splits, M * N, Y, epi == kEpiAccumulate ? 1 : 0);
        else
            hipLaunchKernelGGL(split_k_sum_kernel<false>, grid, dim3(256), 0, ctx->stream,
                               static_cast<const float *>(ws), p.splits, M * N, Y, epi == kEpiAccumulate ? 1 : 0);
        return aih_launch_status();
    }
    if (p.tile == 512)
        hipLaunchKernelGGL((qgemm256_kernel<T, 2, 2>), dim3((unsigned)gx, (unsigned)gy4), dim3(512), 0, ctx->stream,
                           W, N, K, row_bytes, Xh, M, Y, epi, nullptr, p.ssper, ra);
    else if (p.tile == 256)
        hipLaunchKernelGGL((qgemm256_kernel<T, 1, SC>), dim3((unsigned)gx, (unsigned)gy2), dim3(512), 0, ctx->stream,
                           W, N, K, row_bytes, Xh, M, Y, epi, nullptr, p.ssper, ra);
    else
        hipLaunchKernelGGL((qgemm_kernel<T>), dim3((unsigned)gx, (unsigned)gy), dim3(512), 0, ctx->stream,
                           W, N, K, row_bytes, Xh, M, Y, epi, ra);
    return aih_launch_status();
}

}  // namespace

int aih_launch_qgemm_tiled(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K, const void *Xtv,
                           int64_t M, float *Y, int epi, bool may_split, const aih_rope_qkv_args *rope)
{
    const aih_rope_qkv_args ra = rope ? *rope : aih_rope_qkv_args{};
    if (K % BK != 0) return AIH_E_LIMIT;
    const int64_t rb = aih_row_bytes(type, K);
    const uint8_t *w = static_cast<const uint8_t *>(W);
    const _Float16 *Xt = static_cast<const _Float16 *>(Xtv);
    switch (type) {
    case AIH_TYPE_Q4_K: return launch<G4K>(ctx, w, N, K, rb, Xt, M, Y, epi, may_split, ra);
    case AIH_TYPE_Q6_K: return launch<G6K>(ctx, w, N, K, rb, Xt, M, Y, epi, may_split, ra);
    case AIH_TYPE_Q8_0: return launch<G80>(ctx, w, N, K, rb, Xt, M, Y, epi, may_split, ra);
    case AIH_TYPE_Q4_0: return launch<G40>(ctx, w, N, K, rb, Xt, M, Y, epi, may_split, ra);
    default: return AIH_E_UNSUPPORTED;
    }
}

int aih_launch_x_tile(aih_ctx *ctx, const float *X, int64_t M, int64_t K, void *Xt)
{
    return aih_launch_x_tile_pre(ctx, AIH_PRE_NONE, X, nullptr, 0.f, M, K, Xt);
}

int aih_launch_operand_fixup(aih_ctx *ctx, void *Xt, int64_t M, int64_t K)
{
    const int64_t mpad = aih_operand::mpad_of(M);
    hipLaunchKernelGGL(operand_fixup_kernel, dim3((unsigned)((mpad + 3) / 4)), dim3(256), 0, ctx->stream,
                       static_cast<_Float16 *>(Xt), mpad, K);
    return aih_launch_status();
}

int aih_launch_qgemm(aih_ctx *ctx, int type, const void *W, int64_t N, int64_t K,
                     const float *X, int64_t M, float *Y, const aih_scratch *ext, bool may_split)
{
    // K advances in 64-element steps.
    if (K % BK != 0) return AIH_E_LIMIT;
    if ((reinterpret_cast<uintptr_t>(X) & 15) != 0) return AIH_E_INVALID;
    void *work = nullptr;
    int rc = aih_stage(ctx, ext, (size_t)aih_operand::image_bytes(aih_operand::mpad_of(M), K, false), &work);
    if (rc) return rc;
    rc = aih_launch_x_tile(ctx, X, M, K, work);
    if (rc) return rc;
    return aih_launch_qgemm_tiled(ctx, type, W, N, K, work, M, Y, 0, may_split && ext == nullptr);
}

extern "C" int aih_qgemm_plan(aih_ctx *ctx, int64_t N, int64_t K, int64_t M, int may_split, int32_t *tile_rows,
                              int32_t *splits)
{
    if (!ctx || !tile_rows || !splits || N <= 0 || M <= 0 || K <= 0 || K % BK) return AIH_E_INVALID;
    const GemmPlan p = plan_gemm(ctx->cu_count, N, K, M, kEpiStore, may_split != 0);
    *tile_rows = p.tile;
    *splits = p.splits;
    return AIH_OK;
}
