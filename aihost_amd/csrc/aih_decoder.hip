// aih_decoder.hip -- the non-matmul operators of a Llama decoder layer, so
// that a whole decode step (and prefill) runs on the device around the fused
// quantized matmuls:
//
//   RMSNorm            ComputeOps.LayerNorm (ComputeOps.cs:517-542),
//                      shader ComputeShaders.cs:247-278
//   RoPE (interleaved) ComputeOps.ApplyRoPEFull (ComputeOps.cs:959-979),
//                      shader ComputeShaders.cs:517-543
//   causal GQA attention   ComputeOps.MultiHeadAttention (ComputeOps.cs:1055-1102)
//                      and FusedMHAGenerate (ComputeOps.cs:1015-1043, shader
//                      ComputeShaders.cs:656-733)
//   SiLU(gate) * up, residual add   ComputeOps.FeedForward / Add
//                      (ComputeOps.cs:1218-1241, 389-...), shaders
//                      ComputeShaders.cs:280-320
//   KV cache append    KVCache.Add (InferenceEngine.cs:598-622), here an
//                      in-place row store instead of an O(L^2) concat
//   greedy argmax      the sampling step of InferenceEngine for a greedy
//                      configuration
//
// Positions.  Every position-dependent operator takes `start` and an
// optional device pointer `pos`: the position of row r is start + r, plus
// *pos when pos is not null.  A decode step captured into a HIP graph reads
// its position from device memory, and the argmax operator advances it, so
// the graph can be replayed token after token without the host.
//
// This file is compiled without FMA contraction, so that the element-wise
// formulas round like the reference's (x / rms * w, x1*c - x2*s, ...);
// attention contracts its dot products with explicit fmaf.
#include "aih_internal.h"
#include "aih_operand.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// Read by dev_pos when the caller passes no position; never written.
__device__ int32_t no_pos = 0;

// start + *pos, or start when pos is null.  The load goes through a pointer
// that is never null, so it is not behind a branch: a scalar load inside a
// branch is waited for before the branch closes, which would put the round
// trip ahead of every vector load issued after it.
__device__ __forceinline__ int32_t dev_pos(int32_t start, const int32_t *pos)
{
    return start + *(pos ? pos : &no_pos);
}

// Cross-lane steps on the DPP path: a few cycles each, where __shfl_xor goes
// through an LDS permute of about a hundred cycles of latency.
__device__ __forceinline__ float xor1(float v)   // lane ^ 1 (quad_perm [1,0,3,2])
{
    return __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ float xor2(float v)   // lane ^ 2 (quad_perm [2,3,0,1])
{
    return __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);
}

// Maximum / sum over the aligned 16 lanes of a row, returned to every lane
// of the row: pairs, quads, half rows (row_half_mirror), rows (row_mirror).
__device__ __forceinline__ float row16_max(float v)
{
    v = fmaxf(v, xor1(v));
    v = fmaxf(v, xor2(v));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false));
    return fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += xor1(v);
    v += xor2(v);
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);
    return v + __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);
}

// Sum over the 64 lanes of a wave, returned to every lane: pairs, quads,
// half rows and rows of 16 by DPP, then rows 0+1, 2+3 and 0..3 into lane 63
// (row_bcast), read back with readlane.
__device__ __forceinline__ float wave_sum(float v)
{
    v += xor1(v);
    v += xor2(v);
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);   // row_half_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);   // row_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x142, 0xA, 0xF, false);   // row_bcast:15 -> rows 1, 3
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x143, 0xC, 0xF, false);   // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over the 64 lanes of a wave (same steps), returned to every lane.
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0xB1, 0xF, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x4E, 0xF, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x141, 0xF, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x140, 0xF, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x142, 0xA, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(-INFINITY, v, 0x143, 0xC, 0xF, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over a workgroup of `NT` threads (multiple of 64); every thread gets it.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += red[i];
    return t;
}

// ---------------------------------------------------------------- RMSNorm
// One workgroup per row: rms = sqrt(sum(x^2)/cols + eps); y = (x / rms) * w.
// Y may alias X.
template <bool VEC>
__global__ void __launch_bounds__(256)
rmsnorm_kernel(const float *X, const float *__restrict__ Wt, float *Y, int64_t cols, float eps)
{
    __shared__ float red[4];
    const float *x = X + (int64_t)blockIdx.x * cols;
    float *y = Y + (int64_t)blockIdx.x * cols;
    float ss = 0.f;
    if (VEC) {
        const f4 *x4 = reinterpret_cast<const f4 *>(x);
        for (int64_t i = threadIdx.x; i < cols / 4; i += 256) {
            const f4 v = x4[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (int64_t i = threadIdx.x; i < cols; i += 256) ss += x[i] * x[i];
    }
    ss = block_sum<256>(ss, red);
    const float rms = sqrtf(ss / (float)cols + eps);
    if (VEC) {
        const f4 *x4 = reinterpret_cast<const f4 *>(x);
        const f4 *w4 = reinterpret_cast<const f4 *>(Wt);
        f4 *y4 = reinterpret_cast<f4 *>(y);
        for (int64_t i = threadIdx.x; i < cols / 4; i += 256) {
            const f4 v = x4[i], w = w4[i];
            f4 o;
            o.x = (v.x / rms) * w.x;
            o.y = (v.y / rms) * w.y;
            o.z = (v.z / rms) * w.z;
            o.w = (v.w / rms) * w.w;
            y4[i] = o;
        }
    } else {
        for (int64_t i = threadIdx.x; i < cols; i += 256) y[i] = (x[i] / rms) * Wt[i];
    }
}

// ---------------------------------------------------------------- RoPE
// Table of (cos, sin) per (position, pair): angle = (float)pos * freq with
// freq = 1 / theta^((2i)/d) -- the reference's fp32 formula -- where the
// power, cosine and sine are evaluated in double and rounded to float.
__global__ void __launch_bounds__(256)
rope_table_kernel(float *table, int32_t max_pos, int32_t head_dim, float theta)
{
    const int half = head_dim / 2;
    const int64_t total = (int64_t)max_pos * half;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int32_t pos = (int32_t)(t / half), i = (int32_t)(t % half);
        const float e = (float)(2 * i) / (float)head_dim;
        const float pw = (float)pow((double)theta, (double)e);
        const float freq = 1.0f / pw;
        const float ang = (float)pos * freq;
        table[2 * t] = (float)cos((double)ang);
        table[2 * t + 1] = (float)sin((double)ang);
    }
}

// Pair (2i, 2i+1) of head h of row r at position p:
//   y0 = x0*c - x1*s,  y1 = x0*s + x1*c.
// The output row is r, or the position p itself when y_at_pos (the row of a
// KV cache); rows at or past y_rows are not written.
__global__ void __launch_bounds__(256)
rope_kernel(const float *X, int64_t ldx, float *Y, int64_t ldy, int64_t rows, int32_t n_heads, int32_t head_dim,
            int32_t start, const int32_t *pos, const float *__restrict__ table, int32_t table_rows, int y_at_pos,
            int64_t y_rows)
{
    const int half = head_dim / 2;
    const int64_t per_row = (int64_t)n_heads * half;
    const int64_t total = rows * per_row;
    const int32_t p0 = dev_pos(start, pos);
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / per_row, rem = t % per_row;
        const int h = (int)(rem / half), i = (int)(rem % half);
        const int64_t p = p0 + r;
        if (p < 0 || p >= table_rows) continue;
        const int64_t yr = y_at_pos ? p : r;
        if (yr >= y_rows) continue;
        const float c = table[2 * (p * half + i)], s = table[2 * (p * half + i) + 1];
        const float *x = X + r * ldx + (int64_t)h * head_dim + 2 * i;
        float *y = Y + yr * ldy + (int64_t)h * head_dim + 2 * i;
        const float x0 = x[0], x1 = x[1];
        y[0] = x0 * c - x1 * s;
        y[1] = x0 * s + x1 * c;
    }
}

// Q/K/V of one layer after the projections, in one launch: RoPE of the
// query heads in place, RoPE of the key heads into the K cache at their
// positions, the value rows into the V cache.  Q, K and V rows have strides
// ldq / ldk / ldv (the three may be parts of one fused projection output).
__global__ void __launch_bounds__(256)
rope_qkv_kernel(float *Q, int64_t ldq, const float *K, int64_t ldk, const float *V, int64_t ldv, float *Kc,
                float *Vc, int64_t rows, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start,
                const int32_t *pos, const float *__restrict__ table, int32_t table_rows, int64_t cache_rows)
{
    const int half = head_dim / 2;
    const int64_t nq = (int64_t)n_heads * half, nk = (int64_t)n_kv_heads * half, nv = (int64_t)n_kv_heads * half;
    const int64_t per_row = nq + nk + nv;           // pairs per row: q, k, v (v "pairs" are plain copies)
    const int64_t kv_dim = (int64_t)n_kv_heads * head_dim;
    const int32_t p0 = dev_pos(start, pos);
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < rows * per_row;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / per_row, e = t % per_row;
        const int64_t p = p0 + r;
        if (p < 0 || p >= table_rows) continue;
        if (e < nq + nk) {
            const bool is_q = e < nq;
            const int64_t pe = is_q ? e : e - nq;
            const int hh = (int)(pe / half), i = (int)(pe % half);
            const float c = table[2 * (p * half + i)], sn = table[2 * (p * half + i) + 1];
            const float *x = (is_q ? Q + r * ldq : K + r * ldk) + (int64_t)hh * head_dim + 2 * i;
            const float x0 = x[0], x1 = x[1];
            float *y;
            if (is_q) {
                y = Q + r * ldq + (int64_t)hh * head_dim + 2 * i;
            } else {
                if (p >= cache_rows) continue;
                y = Kc + p * kv_dim + (int64_t)hh * head_dim + 2 * i;
            }
            y[0] = x0 * c - x1 * sn;
            y[1] = x0 * sn + x1 * c;
        } else {
            if (p >= cache_rows) continue;
            const int64_t c2 = 2 * (e - nq - nk);
            Vc[p * kv_dim + c2] = V[r * ldv + c2];
            Vc[p * kv_dim + c2 + 1] = V[r * ldv + c2 + 1];
        }
    }
}

// rope_qkv_kernel four floats at a time (two rotation pairs), with 32-bit
// column arithmetic: workgroup (x, y) takes columns 1024 x .. + 1023 of the
// q|k|v row y (and y + gridDim.y, ...).  Needs head_dim, the row strides and
// the cache and Q/K/V bases in units of 4 floats and 16-byte aligned, and
// the table 16-byte aligned; the same products and roundings per element.
__global__ void __launch_bounds__(256)
rope_qkv_vec_kernel(float *Q, int64_t ldq, const float *K, int64_t ldk, const float *V, int64_t ldv,
                    float *__restrict__ Kc, float *__restrict__ Vc, int64_t rows, int32_t q_dim, int32_t kv_dim,
                    int32_t head_dim, int32_t start, const int32_t *pos, const float *__restrict__ table,
                    int32_t table_rows, int64_t cache_rows)
{
    const int half = head_dim / 2;
    const int c = 4 * ((int)blockIdx.x * 256 + (int)threadIdx.x);
    if (c >= q_dim + 2 * kv_dim) return;
    const int32_t p0 = dev_pos(start, pos);
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t p = p0 + r;
        if (p < 0 || p >= table_rows) continue;
        if (c >= q_dim && p >= cache_rows) continue;
        if (c < q_dim + kv_dim) {
            const bool is_q = c < q_dim;
            const int cc = is_q ? c : c - q_dim;
            const int i = (cc % head_dim) / 2;   // first of the two pairs
            const f4 t = *reinterpret_cast<const f4 *>(table + 2 * (p * half + i));   // c0, s0, c1, s1
            const f4 x = *reinterpret_cast<const f4 *>(is_q ? Q + r * ldq + cc : K + r * ldk + cc);
            f4 y;
            y.x = x.x * t.x - x.y * t.y;
            y.y = x.x * t.y + x.y * t.x;
            y.z = x.z * t.z - x.w * t.w;
            y.w = x.z * t.w + x.w * t.z;
            *reinterpret_cast<f4 *>(is_q ? Q + r * ldq + cc : Kc + p * kv_dim + cc) = y;
        } else {
            const int cv = c - q_dim - kv_dim;
            *reinterpret_cast<f4 *>(Vc + p * kv_dim + cv) = *reinterpret_cast<const f4 *>(V + r * ldv + cv);
        }
    }
}

// ---------------------------------------------------------------- row store
// Y[(p + r) * cols + c] = X[r * cols + c] for rows whose position p + r is
// below y_rows (a KV cache append).
__global__ void __launch_bounds__(256)
store_rows_kernel(const float *__restrict__ X, int64_t rows, int64_t cols, float *__restrict__ Y, int64_t y_rows,
                  int32_t start, const int32_t *pos)
{
    const int64_t p0 = dev_pos(start, pos);
    const int64_t total = rows * cols;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / cols;
        if (p0 + r >= 0 && p0 + r < y_rows) Y[(p0 + r) * cols + t % cols] = X[t];
    }
}

// ---------------------------------------------------------------- SiLU * up, add
__global__ void __launch_bounds__(256)
silu_mul_kernel(const float *G, const float *U, float *Y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float g = G[i];
        const float sig = 1.0f / (1.0f + expf(-g));
        Y[i] = (g * sig) * U[i];
    }
}

__global__ void __launch_bounds__(256)
silu_mul_pairs_kernel(const float *__restrict__ X, float *__restrict__ Y, int64_t rows, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows * n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / n, c = i % n;
        const float g = X[r * 2 * n + 2 * c];
        const float sig = 1.0f / (1.0f + expf(-g));
        Y[i] = (g * sig) * X[r * 2 * n + 2 * c + 1];
    }
}

__global__ void __launch_bounds__(256)
add_kernel(const float *A, const float *B, float *Y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        Y[i] = A[i] + B[i];
}

// The two halves of silu_mul_kernel as the reference's separate operators:
// SiLU in place (Y may alias X) and the element-wise product.
__global__ void __launch_bounds__(256)
silu_kernel(const float *X, float *Y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float x = X[i];
        Y[i] = x * (1.0f / (1.0f + expf(-x)));
    }
}

__global__ void __launch_bounds__(256)
mul_kernel(const float *A, const float *B, float *Y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        Y[i] = A[i] * B[i];
}

// Rows of an fp32 embedding table by device token ids (zeros for an id
// outside [0, vocab)).
__global__ void __launch_bounds__(256)
embed_f32_kernel(const float *__restrict__ T, int64_t vocab, int64_t dim, const int32_t *__restrict__ ids, int64_t n,
                 float *__restrict__ Y)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n * dim; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / dim, c = i - r * dim;
        const int32_t id = ids[r];
        Y[i] = id >= 0 && id < vocab ? T[(int64_t)id * dim + c] : 0.f;
    }
}

// ---------------------------------------------------------------- attention
// Query row i (position p_i = p0 + i) of head h attends to cache rows
// 0..p_i of KV head h / (n_heads / n_kv_heads):
//   o = sum_j softmax_j(scale * q.k_j) v_j.
// Q/O rows hold n_heads*head_dim floats, K/V cache rows n_kv_heads*head_dim.

constexpr int kHD = 128;      // head_dim supported by the attention kernels
constexpr int kSub = 64;      // keys per decode sub-chunk (one pass of the score step)
constexpr int kMaxSplit = 64; // decode splits per head (upper bound)
constexpr int kQTile = 64;    // queries per prefill workgroup
constexpr int kSplitKeys = 64;  // keys per decode split of attn_decode_gqa
constexpr int kShortKeys = 32;  // keys per decode split of attn_decode_short
constexpr int kShortWaves = 8;  // waves per workgroup of attn_decode_short (at most)

// Decode splits of a cache of max_len rows: ranges of kShortKeys keys
// (attn_decode_short) while there are at most kMaxSplit of them, else
// ranges of 64 keys (attn_decode_gqa) until there are kMaxSplit of those,
// then longer ranges.
int32_t decode_splits(int32_t max_len)
{
    const int32_t ns = (max_len + kShortKeys - 1) / kShortKeys;
    if (ns <= kMaxSplit) return ns;
    const int32_t n = (max_len + kSplitKeys - 1) / kSplitKeys;
    return n < kMaxSplit ? n : kMaxSplit;
}

// Waves per workgroup of the grouped decode kernel: a split's keys in
// sub-chunks of 16 per wave, at most four waves.
int decode_waves(int32_t max_len, int32_t n_split)
{
    const int32_t chunk = (max_len + n_split - 1) / n_split;
    return chunk <= 16 ? 1 : chunk <= 32 ? 2 : 4;
}

// Decode (one query row), split over keys.  Workgroup (h, s) of 256 threads
// walks the keys of split s in sub-chunks of kSub with an online softmax and
// writes its partial (max, sum, unnormalised output) to `part`;
// attn_decode_combine then merges the splits of each head.  (A single kernel
// whose last workgroup per head combines, found through a device counter,
// measured slower on MI355X: the agent-scope fences it needs write back the
// XCD's L2.)
//   scores: thread t -> key t/4 of the sub-chunk, dims 32*(t%4) .. +31
//   values: thread t -> dims 4*(t%32) .. +3 of keys t/32, t/32 + 8, ...
__global__ void __launch_bounds__(256)
attn_decode_partial(const float *__restrict__ Q, const float *__restrict__ Kc, const float *__restrict__ Vc,
                    float *__restrict__ part, int32_t n_heads, int32_t n_kv_heads, int32_t start,
                    const int32_t *pos, int32_t max_len, float scale, int32_t n_split)
{
    __shared__ float qs[kHD];
    __shared__ float ps[kSub];
    __shared__ float red[4];
    __shared__ f4 accs[8][kHD / 4];
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t kv_stride = (int64_t)n_kv_heads * kHD;
    const int32_t L = max(0, min(dev_pos(start, pos) + 1, max_len));   // keys 0..p, within the cache
    const int32_t chunk = (L + n_split - 1) / n_split;
    const int32_t j0 = min(s * chunk, L), j1 = min(L, j0 + chunk);
    if (t < kHD) qs[t] = Q[(int64_t)h * kHD + t];
    __syncthreads();
    const int kk = t >> 2, part4 = t & 3;
    const int vc = t & 31, vr = t >> 5;
    float m = -INFINITY, l = 0.f;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int32_t c0 = j0; c0 < j1; c0 += kSub) {
        const int n = min(kSub, j1 - c0);
        // V rows of this sub-chunk are loaded together with the K rows (their
        // addresses do not depend on the scores): one memory round trip
        f4 vv[kSub / 8];
#pragma unroll
        for (int u = 0; u < kSub / 8; ++u) {
            const int j = vr + 8 * u;
            vv[u] = j < n ? reinterpret_cast<const f4 *>(Vc + (int64_t)(c0 + j) * kv_stride + kvh * kHD)[vc]
                          : f4{0.f, 0.f, 0.f, 0.f};
        }
        float sc = -INFINITY;
        if (kk < n) {
            const f4 *k4 = reinterpret_cast<const f4 *>(Kc + (int64_t)(c0 + kk) * kv_stride + kvh * kHD + part4 * 32);
            float a = 0.f;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const f4 k = k4[d];
                a = fmaf(qs[part4 * 32 + 4 * d], k.x, a);
                a = fmaf(qs[part4 * 32 + 4 * d + 1], k.y, a);
                a = fmaf(qs[part4 * 32 + 4 * d + 2], k.z, a);
                a = fmaf(qs[part4 * 32 + 4 * d + 3], k.w, a);
            }
            a += xor1(a);
            a += xor2(a);
            sc = a * scale;
        }
        const float mc = wave_max(sc);
        if ((t & 63) == 0) red[t >> 6] = mc;
        __syncthreads();
        const float mn = fmaxf(m, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
        __syncthreads();
        const float e = kk < n ? expf(sc - mn) : 0.f;
        if (part4 == 0) ps[kk] = e;
        const float lc = block_sum<256>(part4 == 0 ? e : 0.f, red);   // its barrier publishes ps
        const float corr = expf(m - mn);                              // 0 on the first sub-chunk
        l = l * corr + lc;
        f4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kSub / 8; ++u) {
            const int j = vr + 8 * u;
            const float pj = j < n ? ps[j] : 0.f;
            a.x = fmaf(pj, vv[u].x, a.x);
            a.y = fmaf(pj, vv[u].y, a.y);
            a.z = fmaf(pj, vv[u].z, a.z);
            a.w = fmaf(pj, vv[u].w, a.w);
        }
        acc = acc * corr + a;
        m = mn;
        __syncthreads();   // ps and red reused by the next sub-chunk
    }
    // partial of this split: sum the eight key groups
    accs[vr][vc] = acc;
    __syncthreads();
    float *mine = part + ((int64_t)h * n_split + s) * (kHD + 2);
    if (t < kHD) {
        const float *af = reinterpret_cast<const float *>(&accs[0][0]);
        float v = 0.f;
#pragma unroll
        for (int r = 0; r < 8; ++r) v += af[r * kHD + t];
        mine[2 + t] = v;
    }
    if (t == 0) {
        mine[0] = j1 > j0 ? m : -INFINITY;
        mine[1] = j1 > j0 ? l : 0.f;
    }
}

// Decode attention of one query row for the G = n_heads / n_kv_heads query
// heads of one KV head: workgroup (kvh, s) serves those heads over split s of
// the cache, so each cached K/V row is read once for the G heads.
//
// Splits cover fixed key ranges of the cache (chunk = ceil(cache_rows /
// n_split) keys each), not ranges of the keys 0..p: the first K/V rows are
// loaded before the position p = start + *pos arrives, and keys past p are
// masked (a split past p writes an empty partial).
//
// Each wave keeps its own online softmax (running max, sum and V
// accumulator) over its 16 keys of every 64-key sub-chunk, with no barrier
// inside the key loop; the four waves are merged through LDS at the end.
// Thread (key lane / 4, dims 32 * (lane % 4) ..) scores, thread lane
// accumulates V dims 2 * lane, 2 * lane + 1.
//
// FUSE: the query comes from the projection output QKV (q | k | v of one
// row); the kernel applies RoPE to q and to the new key itself, the split
// holding key p stores the key and value rows into the caches at row p and
// uses them from LDS (no other workgroup reads row p).  The arithmetic is
// that of rope_qkv_kernel, so the FUSE and plain forms give the same bits.
// Plain: the query rows are Q (already rotated) and every key comes from the
// cache.
template <int G, bool FUSE, int NW>
__global__ void __launch_bounds__(64 * NW)
attn_decode_gqa(const float *__restrict__ Qsrc, float *Kc, float *Vc, float *__restrict__ part, int32_t n_heads,
                int32_t n_kv_heads, int32_t start, const int32_t *pos, const float *__restrict__ table,
                int32_t table_rows, int32_t cache_rows, float scale, int32_t n_split)
{
    constexpr int half = kHD / 2;
    constexpr int NT = 64 * NW;                 // threads
    constexpr int QP = (G * half + NT - 1) / NT;   // query pairs per thread
    __shared__ f4 qs[G][kHD / 4];
    __shared__ f4 kn[kHD / 4], vn[kHD / 4];
    __shared__ float ps[NW][G][16];
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float wacc[NW][G][kHD];
    const int kvh = blockIdx.x, s = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kk = lane >> 2, part4 = lane & 3;
    const int64_t kv_stride = (int64_t)n_kv_heads * kHD;
    const int32_t chunk = (cache_rows + n_split - 1) / n_split;
    const int32_t j0 = s * chunk, jc = min(j0 + chunk, cache_rows);   // the split, whatever p
    const float *kbase = Kc + (int64_t)kvh * kHD + part4 * 32;
    const float *vbase = Vc + (int64_t)kvh * kHD + 2 * lane;

    // Loads are issued in the order their data is needed and none waits for
    // the position: the position itself (a scalar load, counted apart from
    // the vector loads), the query pairs and the new key and value rows, the
    // first sub-chunk's K and V rows, and last the rotation table's row p.
    // Vector loads complete in issue order, so the wait for the table also
    // waits for the K and V rows, which the scores need next anyway.
    // (Loading the query and the new rows after the position, as the plain
    // program order would, put up to three more round trips in a row.)
    const int32_t p = dev_pos(start, pos);
    float qx[QP][2];
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        if (e < G * half) {
            const float *x = Qsrc + (int64_t)(kvh * G + e / half) * kHD + 2 * (e % half);
            qx[i][0] = x[0];
            qx[i][1] = x[1];
        }
    }
    // FUSE: key pair t of the new row by threads t < half, value quad t - v0
    // by threads v0 .. v0 + kHD / 4 - 1 (v0 = half, or 0 when the workgroup
    // has fewer than half + kHD / 4 threads)
    constexpr int v0 = NT >= half + kHD / 4 ? half : 0;
    const bool kt = FUSE && t < half, vt = FUSE && t >= v0 && t - v0 < kHD / 4;
    const float *kx = Qsrc + (int64_t)n_heads * kHD + (int64_t)kvh * kHD;
    const float *vx = kx + kv_stride;
    float knew[2] = {0.f, 0.f};
    f4 vnew = {0.f, 0.f, 0.f, 0.f};
    if (kt) {
        knew[0] = kx[2 * t];
        knew[1] = kx[2 * t + 1];
    }
    if (vt) vnew = reinterpret_cast<const f4 *>(vx)[t - v0];

    f4 k[8];
    float2 v[16];
    auto load_k = [&](int32_t c0) {
        const int32_t j = c0 + 16 * w + kk;
        if (j < jc) {
            const f4 *k4 = reinterpret_cast<const f4 *>(kbase + (int64_t)j * kv_stride);
#pragma unroll
            for (int d = 0; d < 8; ++d) k[d] = k4[d];
        }
    };
    auto load_v = [&](int32_t c0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int32_t j = c0 + 16 * w + i;
            v[i] = j < jc ? *reinterpret_cast<const float2 *>(vbase + (int64_t)j * kv_stride) : float2{0.f, 0.f};
        }
    };
    load_k(j0);
    load_v(j0);

    const int32_t L = max(0, min(p + 1, cache_rows));
    const int32_t j1 = min(jc, L);                      // active keys: j0 .. j1-1
    const bool own = FUSE && j0 <= p && p < j1;        // this split holds the new key
    const bool rot = p >= 0 && p < table_rows;
    const float *tp = table + 2 * (int64_t)(rot ? p : 0) * half;
    float cq[QP][2], ck[2] = {1.f, 0.f};
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        cq[i][0] = 1.f;
        cq[i][1] = 0.f;
        if (FUSE && rot && e < G * half) {
            cq[i][0] = tp[2 * (e % half)];
            cq[i][1] = tp[2 * (e % half) + 1];
        }
    }
    if (kt) {
        ck[0] = tp[2 * t];
        ck[1] = tp[2 * t + 1];
    }

    // query heads into LDS (rotated here when FUSE), the new key row when owned
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        if (e < G * half) {
            const float x0 = qx[i][0], x1 = qx[i][1];
            float *y = reinterpret_cast<float *>(&qs[e / half][0]) + 2 * (e % half);
            if (FUSE && rot) {
                const float c = cq[i][0], sn = cq[i][1];
                y[0] = x0 * c - x1 * sn;
                y[1] = x0 * sn + x1 * c;
            } else {
                y[0] = x0;
                y[1] = x1;
            }
        }
    }
    // the new key, rotated (stored into the cache at the end: a barrier waits
    // for every store issued before it)
    if (kt) {
        const float c = ck[0], sn = ck[1];
        const float x0 = knew[0], x1 = knew[1];
        knew[0] = x0 * c - x1 * sn;
        knew[1] = x0 * sn + x1 * c;
    }
    if (own) {
        if (kt) {
            float *kq = reinterpret_cast<float *>(kn) + 2 * t;
            kq[0] = knew[0];
            kq[1] = knew[1];
        }
        if (vt) vn[t - v0] = vnew;
    }
    __syncthreads();

    float m[G], l[G];
    float2 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
        acc[g] = float2{0.f, 0.f};
    }
    for (int32_t c0 = j0; c0 < j1; c0 += 16 * NW) {
        const int32_t jk = c0 + 16 * w + kk;              // this thread's key
        if (own && jk == p) {
#pragma unroll
            for (int d = 0; d < 8; ++d) k[d] = kn[part4 * 8 + d];
        }
        if (own) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (c0 + 16 * w + i == p) v[i] = reinterpret_cast<const float2 *>(vn)[lane];
        }
        // rows past p were loaded before p was known: their weights are 0,
        // and their values are zeroed too (a stale row may hold NaN)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (c0 + 16 * w + i >= j1) v[i] = float2{0.f, 0.f};
        // query heads in blocks of at most four (the block's scores, weights
        // and corrections in registers; K and V rows shared by all blocks)
        constexpr int GB = G < 4 ? G : 4;
#pragma unroll
        for (int g0 = 0; g0 < G; g0 += GB) {
            float sc[GB];
#pragma unroll
            for (int gb = 0; gb < GB; ++gb) {
                const int g = g0 + gb;
                float a = 0.f;
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    const f4 q = qs[g][part4 * 8 + d];
                    a = fmaf(q.x, k[d].x, a);
                    a = fmaf(q.y, k[d].y, a);
                    a = fmaf(q.z, k[d].z, a);
                    a = fmaf(q.w, k[d].w, a);
                }
                a += xor1(a);
                a += xor2(a);
                sc[gb] = jk < j1 ? a * scale : -INFINITY;
            }
            float corr[GB];
#pragma unroll
            for (int gb = 0; gb < GB; ++gb) {
                const int g = g0 + gb;
                const float mn = fmaxf(m[g], wave_max(sc[gb]));
                const float e = jk < j1 ? expf(sc[gb] - mn) : 0.f;
                if (part4 == 0) ps[w][g][kk] = e;
                const float lw = wave_sum(part4 == 0 ? e : 0.f);
                corr[gb] = mn == -INFINITY ? 1.f : expf(m[g] - mn);
                l[g] = l[g] * corr[gb] + lw;
                m[g] = mn;
            }
            // ps[w] is written and read by this wave only (LDS order within a wave)
#pragma unroll
            for (int gb = 0; gb < GB; ++gb) {
                const int g = g0 + gb;
                float2 a = {0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float pi = ps[w][g][i];
                    a.x = fmaf(pi, v[i].x, a.x);
                    a.y = fmaf(pi, v[i].y, a.y);
                }
                acc[g].x = acc[g].x * corr[gb] + a.x;
                acc[g].y = acc[g].y * corr[gb] + a.y;
            }
        }
        if (c0 + 16 * NW < j1) load_k(c0 + 16 * NW);   // the next sub-chunk's keys
        if (c0 + 16 * NW < j1) load_v(c0 + 16 * NW);
    }

    // merge the NW waves: M = max of the wave maxima; weights e^(m_w - M)
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (lane == 0) {
            wm[w][g] = m[g];
            wl[w][g] = l[g];
        }
        wacc[w][g][2 * lane] = acc[g].x;
        wacc[w][g][2 * lane + 1] = acc[g].y;
    }
    __syncthreads();
    for (int e = t; e < G * kHD; e += NT) {
        const int g = e / kHD, d = e % kHD;
        float M = wm[0][g];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) M = fmaxf(M, wm[ww][g]);
        float o = 0.f, lt = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
            const float f = wm[ww][g] == -INFINITY ? 0.f : expf(wm[ww][g] - M);
            o = fmaf(wacc[ww][g][d], f, o);
            lt = fmaf(wl[ww][g], f, lt);
        }
        float *mine = part + ((int64_t)(kvh * G + g) * n_split + s) * (kHD + 2);
        mine[2 + d] = o;
        if (d == 0) {
            mine[0] = M;          // -inf for a split with no key at or before p
            mine[1] = lt;
        }
    }
    // the split holding key p stores the new key and value rows into the
    // caches (no other workgroup of this launch reads row p)
    if (own) {
        if (kt) {
            float *kc = Kc + (int64_t)p * kv_stride + (int64_t)kvh * kHD + 2 * t;
            kc[0] = knew[0];
            kc[1] = knew[1];
        }
        if (vt) reinterpret_cast<f4 *>(Vc + (int64_t)p * kv_stride + (int64_t)kvh * kHD)[t - v0] = vnew;
    }
}

// Maximum / sum over aligned groups of N lanes (N = 8, 16, 32 or 64),
// returned to every lane of the group: DPP within rows of 16, then lane
// permutes across rows.
template <int N>
__device__ __forceinline__ float group_max(float v)
{
    v = fmaxf(v, xor1(v));
    v = fmaxf(v, xor2(v));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false));   // row_half_mirror
    if (N >= 16) v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false));   // row_mirror
    if (N >= 32) v = fmaxf(v, __shfl_xor(v, 16));
    if (N >= 64) v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
template <int N>
__device__ __forceinline__ float group_sum(float v)
{
    v += xor1(v);
    v += xor2(v);
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);
    if (N >= 16) v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);
    if (N >= 32) v += __shfl_xor(v, 16);
    if (N >= 64) v += __shfl_xor(v, 32);
    return v;
}

// Decode attention over short splits (at most kShortKeys keys each): the
// G = n_heads / n_kv_heads query heads of KV head kvh over the keys of split
// s, in one memory round trip and short dependency chains, so that many
// small workgroups spread the work over the CUs (attn_decode_gqa's 64-key
// splits leave one wave per SIMD on a few CUs, with a serial chain of
// reductions per query head).
//
// Lane layout: dq = lane % 4 (a quarter of the head dims), kk = (lane / 4)
// % KW (a key), g = lane / (4 KW) (a query head), KW = 16 / G keys per wave
// and sub-step.  Each lane forms the 32-dim partial dot of its quarter, the
// four quarters are summed by DPP (the same products and order as
// attn_decode_gqa, so the scores have the same bits), the online softmax of
// head g is reduced over its 4 KW lanes, and for P.V lane l holds dims
// 2l, 2l + 1 of every head.  A workgroup of NW waves covers NW KW SUB keys;
// its K and V rows are all loaded before anything waits.  The new row's
// RoPE, its cache store and the rotation of the queries are those of
// attn_decode_gqa (FUSE); the waves are merged through LDS at the end.
template <int G, bool FUSE, int NW, int SUB>
__global__ void __launch_bounds__(64 * NW)
attn_decode_short(const float *__restrict__ Qsrc, float *Kc, float *Vc, float *__restrict__ part, int32_t n_heads,
                  int32_t n_kv_heads, int32_t start, const int32_t *pos, const float *__restrict__ table,
                  int32_t table_rows, int32_t cache_rows, float scale, int32_t n_split)
{
    constexpr int half = kHD / 2;
    constexpr int NT = 64 * NW;
    constexpr int KW = 16 / G;                      // keys per wave and sub-step
    constexpr int QP = (G * half + NT - 1) / NT;    // query pairs per thread
    constexpr int QR = kHD + 4;                     // LDS row of a query head (padded)
    __shared__ __align__(16) float qs[G][QR];
    __shared__ f4 kn[kHD / 4], vn[kHD / 4];
    __shared__ __align__(16) float ps[NW][KW][G];
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float wacc[NW][G][kHD];
    const int kvh = blockIdx.x, s = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int dq = lane & 3, kk = (lane >> 2) % KW, g = (lane >> 2) / KW;
    const int64_t kv_stride = (int64_t)n_kv_heads * kHD;
    const int32_t chunk = (cache_rows + n_split - 1) / n_split;      // <= NW * KW * SUB (host)
    const int32_t j0 = s * chunk, jc = min(j0 + chunk, cache_rows);   // the split, whatever p

    // loads in the order of attn_decode_gqa: position, query pairs, the new
    // row, K and V, and the rotation table's row p last
    const int32_t p = dev_pos(start, pos);
    float qx[QP][2];
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        if (e < G * half) {
            const float *x = Qsrc + (int64_t)(kvh * G + e / half) * kHD + 2 * (e % half);
            qx[i][0] = x[0];
            qx[i][1] = x[1];
        }
    }
    constexpr int v0 = NT >= half + kHD / 4 ? half : 0;
    const bool kt = FUSE && t < half, vt = FUSE && t >= v0 && t - v0 < kHD / 4;
    const float *kx = Qsrc + (int64_t)n_heads * kHD + (int64_t)kvh * kHD;
    const float *vx = kx + kv_stride;
    float knew[2] = {0.f, 0.f};
    f4 vnew = {0.f, 0.f, 0.f, 0.f};
    if (kt) {
        knew[0] = kx[2 * t];
        knew[1] = kx[2 * t + 1];
    }
    if (vt) vnew = reinterpret_cast<const f4 *>(vx)[t - v0];

    // key of this lane in sub-step sb; the wave's KW keys of sub-step sb
    auto key_of = [&](int sb) { return j0 + (sb * NW + w) * KW + kk; };
    auto vkey_of = [&](int sb, int i) { return j0 + (sb * NW + w) * KW + i; };
    f4 k[SUB][8];
    float2 v[SUB][KW];
#pragma unroll
    for (int sb = 0; sb < SUB; ++sb) {
        const int32_t j = key_of(sb);
        if (j < jc) {
            const f4 *k4 = reinterpret_cast<const f4 *>(Kc + (int64_t)j * kv_stride + (int64_t)kvh * kHD + dq * 32);
#pragma unroll
            for (int d = 0; d < 8; ++d) k[sb][d] = k4[d];
        }
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const int32_t jv = vkey_of(sb, i);
            v[sb][i] = jv < jc ? *reinterpret_cast<const float2 *>(Vc + (int64_t)jv * kv_stride + (int64_t)kvh * kHD +
                                                                   2 * lane)
                               : float2{0.f, 0.f};
        }
    }

    const int32_t L = max(0, min(p + 1, cache_rows));
    const int32_t j1 = min(jc, L);                      // active keys: j0 .. j1-1
    const bool own = FUSE && j0 <= p && p < j1;
    const bool rot = p >= 0 && p < table_rows;
    const float *tp = table + 2 * (int64_t)(rot ? p : 0) * half;
    float cq[QP][2], ck[2] = {1.f, 0.f};
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        cq[i][0] = 1.f;
        cq[i][1] = 0.f;
        if (FUSE && rot && e < G * half) {
            cq[i][0] = tp[2 * (e % half)];
            cq[i][1] = tp[2 * (e % half) + 1];
        }
    }
    if (kt) {
        ck[0] = tp[2 * t];
        ck[1] = tp[2 * t + 1];
    }
#pragma unroll
    for (int i = 0; i < QP; ++i) {
        const int e = t + NT * i;
        if (e < G * half) {
            const float x0 = qx[i][0], x1 = qx[i][1];
            float *y = &qs[e / half][2 * (e % half)];
            if (FUSE && rot) {
                const float c = cq[i][0], sn = cq[i][1];
                y[0] = x0 * c - x1 * sn;
                y[1] = x0 * sn + x1 * c;
            } else {
                y[0] = x0;
                y[1] = x1;
            }
        }
    }
    if (kt) {
        const float c = ck[0], sn = ck[1];
        const float x0 = knew[0], x1 = knew[1];
        knew[0] = x0 * c - x1 * sn;
        knew[1] = x0 * sn + x1 * c;
    }
    if (own) {
        if (kt) {
            float *kq = reinterpret_cast<float *>(kn) + 2 * t;
            kq[0] = knew[0];
            kq[1] = knew[1];
        }
        if (vt) vn[t - v0] = vnew;
    }
    __syncthreads();

    float m_l = -INFINITY, l_l = 0.f;   // running max and sum of head g (same in all its lanes)
    float2 acc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) acc[gg] = float2{0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < SUB; ++sb) {
        const int32_t jk = key_of(sb);
        if (own && jk == p) {
#pragma unroll
            for (int d = 0; d < 8; ++d) k[sb][d] = kn[dq * 8 + d];
        }
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const int32_t jv = vkey_of(sb, i);
            if (own && jv == p) v[sb][i] = reinterpret_cast<const float2 *>(vn)[lane];
            // rows past p were loaded before p was known: weight 0 and value 0
            // (a stale row may hold NaN)
            if (jv >= j1) v[sb][i] = float2{0.f, 0.f};
        }
        float a = 0.f;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const f4 q = *reinterpret_cast<const f4 *>(&qs[g][dq * 32 + 4 * d]);
            a = fmaf(q.x, k[sb][d].x, a);
            a = fmaf(q.y, k[sb][d].y, a);
            a = fmaf(q.z, k[sb][d].z, a);
            a = fmaf(q.w, k[sb][d].w, a);
        }
        a += xor1(a);
        a += xor2(a);
        const float sc = jk < j1 ? a * scale : -INFINITY;
        const float mn = fmaxf(m_l, group_max<4 * KW>(sc));
        const float e = jk < j1 ? expf(sc - mn) : 0.f;
        const float corr = mn == -INFINITY ? 1.f : expf(m_l - mn);
        l_l = l_l * corr + group_sum<4 * KW>(dq == 0 ? e : 0.f);
        m_l = mn;
        if (dq == 0) ps[w][kk][g] = e;
        // ps[w] is written and read by this wave only (LDS order within a wave)
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float cg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr), 4 * KW * gg));
            float2 pv = {0.f, 0.f};
#pragma unroll
            for (int i = 0; i < KW; ++i) {
                const float pi = ps[w][i][gg];
                pv.x = fmaf(pi, v[sb][i].x, pv.x);
                pv.y = fmaf(pi, v[sb][i].y, pv.y);
            }
            acc[gg].x = acc[gg].x * cg + pv.x;
            acc[gg].y = acc[gg].y * cg + pv.y;
        }
    }

    if constexpr (NW == 1) {
        // one wave: its partial is the split's (the merge below would
        // multiply by e^0 = 1)
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float mg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_l), 4 * KW * gg));
            const float lg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l_l), 4 * KW * gg));
            float *mine = part + ((int64_t)(kvh * G + gg) * n_split + s) * (kHD + 2);
            *reinterpret_cast<float2 *>(mine + 2 + 2 * lane) = acc[gg];
            if (lane == 0) {
                mine[0] = mg;     // -inf for a split with no key at or before p
                mine[1] = lg;
            }
        }
    } else {
        // merge the NW waves: M = max of the wave maxima; weights e^(m_w - M)
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float mg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_l), 4 * KW * gg));
            const float lg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l_l), 4 * KW * gg));
            if (lane == 0) {
                wm[w][gg] = mg;
                wl[w][gg] = lg;
            }
            wacc[w][gg][2 * lane] = acc[gg].x;
            wacc[w][gg][2 * lane + 1] = acc[gg].y;
        }
        __syncthreads();
        for (int e = t; e < G * kHD; e += NT) {
            const int gg = e / kHD, d = e % kHD;
            float M = wm[0][gg];
#pragma unroll
            for (int ww = 1; ww < NW; ++ww) M = fmaxf(M, wm[ww][gg]);
            float o = 0.f, lt = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                const float f = wm[ww][gg] == -INFINITY ? 0.f : expf(wm[ww][gg] - M);
                o = fmaf(wacc[ww][gg][d], f, o);
                lt = fmaf(wl[ww][gg], f, lt);
            }
            float *mine = part + ((int64_t)(kvh * G + gg) * n_split + s) * (kHD + 2);
            mine[2 + d] = o;
            if (d == 0) {
                mine[0] = M;          // -inf for a split with no key at or before p
                mine[1] = lt;
            }
        }
    }
    if (own) {
        if (kt) {
            float *kc = Kc + (int64_t)p * kv_stride + (int64_t)kvh * kHD + 2 * t;
            kc[0] = knew[0];
            kc[1] = knew[1];
        }
        if (vt) reinterpret_cast<f4 *>(Vc + (int64_t)p * kv_stride + (int64_t)kvh * kHD)[t - v0] = vnew;
    }
}

// Combine the splits of head h: o = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// NS >= n_split: every split's accumulator element and (m, l) is loaded at
// once, with no branch (indices past n_split re-read the last split, whose
// weight is then 0), so the loads take one memory round trip; the weights go
// through LDS.  The products are summed in split order (the terms past
// n_split are +0 and change nothing).
template <int NS>
__global__ void __launch_bounds__(kHD)
attn_decode_combine(const float *__restrict__ part, float *__restrict__ O, int32_t n_split)
{
    __shared__ float ws[NS];
    __shared__ float red[2];
    const int h = blockIdx.x, t = threadIdx.x;
    const float *ph = part + (int64_t)h * n_split * (kHD + 2);
    float vp[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) vp[u] = ph[(u < n_split ? u : n_split - 1) * (kHD + 2) + 2 + t];
    const int tu = t < n_split ? t : n_split - 1;
    const float mt = t < n_split ? ph[tu * (kHD + 2)] : -INFINITY;
    const float lt = t < n_split ? ph[tu * (kHD + 2) + 1] : 0.f;
    float M = wave_max(mt);
    if ((t & 63) == 0) red[t >> 6] = M;
    __syncthreads();
    M = fmaxf(red[0], red[1]);
    const float w = mt == -INFINITY ? 0.f : expf(mt - M);
    if (t < NS) ws[t] = w;
    float lw = wave_sum(lt * w);
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = lw;
    __syncthreads();
    const float lsum = red[0] + red[1];
    float a = 0.f;
#pragma unroll
    for (int u = 0; u < NS; ++u) a = fmaf(u < n_split ? vp[u] : 0.f, ws[u], a);
    O[(int64_t)h * kHD + t] = lsum > 0.f ? a / lsum : 0.f;
}

// The combine for n_split <= kMaxSplit splits of n_heads heads.
void launch_combine(aih_ctx *ctx, const float *part, float *O, int32_t n_heads, int32_t n_split)
{
    const dim3 grid(n_heads), block(kHD);
    if (n_split <= 16) hipLaunchKernelGGL(attn_decode_combine<16>, grid, block, 0, ctx->stream, part, O, n_split);
    else if (n_split <= 32) hipLaunchKernelGGL(attn_decode_combine<32>, grid, block, 0, ctx->stream, part, O, n_split);
    else hipLaunchKernelGGL(attn_decode_combine<kMaxSplit>, grid, block, 0, ctx->stream, part, O, n_split);
}

// Prefill on the fp16 matrix cores with split operands.  Every fp32
// operand x becomes x 2^e = hi + lo, two fp16 values, with a power of two
// 2^e that puts the largest |x| of its group in [2^14, 2^15): hi = fp16(x 2^e)
// and lo = fp16(x 2^e - hi), 22 significant bits, and an absolute error of at
// most 2^-25 in the scaled units, so small members of a group lose nothing
// that matters beside its largest.  v_mfma_f32_16x16x32_f16 forms
// hi.hi + hi.lo + lo.hi (each product exact in fp32, sums in fp32); the
// dropped lo.lo term is below 2^-22 of a product.  Three fp16 MFMAs cost a
// sixth of the cycles of the fp32 MFMAs for the same products.
//
// Groups: a query row (Q), and per KV head the K and the V rows of a 64-key
// tile (one power of two each).  Scores are unscaled exactly (the power of
// two joins the reference's scale), and the softmax runs in base 2:
// t = score log2(e), p = 2^(t - max).  The V tile's factor goes into P:
// P'' = P 2^(A - ev) with A = 15 + the smallest ev seen so far, so
// P'' <= 2^15 and the O accumulators hold 2^A O; when A drops, they are
// rescaled by the exact power of two with the softmax correction.
//
// Workgroup (h, tile) owns kQTile = 64 queries; wave w of each half (below)
// the 16 queries 16w .. 16w+15.  The products are transposed, S^T = K Q^T and
// O^T = V^T P^T, so that the softmax output is already the B operand of the
// second product and never leaves the registers.  16x16x32 layouts (lane l,
// g = l/16, c = l%16): A[i][k] lane i + 16(k/8) element k%8, B[k][j] lane
// j + 16(k/8) element k%8, D[i][j] lane j + 16(i/4) register i%4.
//   S^T block kb (keys 16kb .. +15): A = K (key c, dims 32s + 8g .. +7),
//      B = Q^T (query c, the same dims): lane (c, g) gets query c's scores
//      for keys 16kb + 4g + r, r = 0..3.
//   O^T block db (dims 16db .. +15), key step t (keys 32t .. +31): the 32
//      k-slots are ordered so that slot 8g + e holds key
//      32t + 16(e/4) + 4g + e%4, i.e. P of block kb = 2t + e/4, register
//      e%4 of the lane itself.  A = V^T in the same slot order.
// Every lane keeps the running max of its query (reduced over the four
// lanes that hold it), a partial sum over its own keys and the rows
// 16db + 4g + r of O^T.
//
// LDS holds the split tile as four images: K hi, K lo (row = key, 128 dims)
// and V^T hi, V^T lo (row = dim, 64 slots).  Rows are padded by 16 bytes,
// so that the 16 lanes of a quarter wave read 16 different rows on disjoint
// banks.
constexpr int kKT = 64;       // keys per tile
constexpr int kRKH = 136;     // K image row (key) stride in LDS, halves: 128 dims + 16 bytes
constexpr int kRVH = 72;      // V^T image row (dim) stride in LDS, halves: 64 slots + 16 bytes

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 hl2 __attribute__((ext_vector_type(2)));   // {hi, lo}

// Causal balance: a workgroup of 512 threads owns a query tile, dispatched
// longest first, as two halves of four waves with an LDS image each.  A tile
// whose keys span at least kSplitKT key tiles gives half 0 its first n_kt / 2
// key tiles and half 1 the last n_kt - n_kt / 2; a shorter one gives half 1
// all of them.  Every row of a split tile attends to the first key of half
// 1's range (its positions are at least p_last - 63 >= 64 (n_kt / 2) when
// n_kt >= 3, since p_last >= 64 (n_kt - 1)), so both halves' softmax states
// start finite.  The halves merge through LDS at the end.
constexpr int kSplitKT = 3;

__device__ __forceinline__ int64_t prefill_key_tiles(int64_t i0, int64_t n_q, int32_t p0, int32_t max_len)
{
    const int64_t p_last = min<int64_t>(p0 + min<int64_t>(i0 + kQTile, n_q) - 1, (int64_t)max_len - 1);
    return p_last < 0 ? 0 : p_last / kKT + 1;
}

// The power of two 2^e that puts amax in [2^14, 2^15) (e = 15 for zero).
__device__ __forceinline__ int split_exp(float amax)
{
    return 15 - __builtin_amdgcn_frexp_expf(amax);
}

__device__ __forceinline__ hl2 split_f16(float x, int e)
{
    const float xs = ldexpf(x, e);
    const _Float16 hi = (_Float16)xs;
    return hl2{hi, (_Float16)(xs - (float)hi)};
}

typedef float fl2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4x __attribute__((ext_vector_type(4)));

// split_f16 of two values at once (the conversions as packed pairs):
// {hi, lo} as two words of two halves
__device__ __forceinline__ void split_pair(float x0, float x1, int e, uint32_t &hi, uint32_t &lo)
{
    const fl2 xs = {ldexpf(x0, e), ldexpf(x1, e)};
    const hl2 h = __builtin_convertvector(xs, hl2);
    const hl2 l = __builtin_convertvector(xs - __builtin_convertvector(h, fl2), hl2);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, l);
}

// 8 values (a: elements 0..3, b: 4..7) split into an h8 of hi and one of lo
__device__ __forceinline__ void split8(const f4 &a, const f4 &b, int e, h8 &hi, h8 &lo)
{
    uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
    split_pair(a[0], a[1], e, h0, l0);
    split_pair(a[2], a[3], e, h1, l1);
    split_pair(b[0], b[1], e, h2, l2);
    split_pair(b[2], b[3], e, h3, l3);
    hi = __builtin_bit_cast(h8, u4x{h0, h1, h2, h3});
    lo = __builtin_bit_cast(h8, u4x{l0, l1, l2, l3});
}

typedef __amdgpu_buffer_rsrc_t Rsrc;

// a raw buffer over `bytes` bytes from base: 16-byte loads at or past the
// end return zeros
__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// a pointer the compiler cannot prove uniform, read from the first lane
__device__ __forceinline__ const float *uniform_ptr(const float *p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const float *>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ f4 bld16(Rsrc r, uint32_t vo)
{
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, 0, 0));
}

__device__ __forceinline__ float xor_lanes_max(float v)   // over lanes l, l^16, l^32, l^48
{
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

// One tile of one KV head in registers, as the 256 threads of a workgroup
// load it: K thread (keys kt_key + 16i, dims 8 kt_ch .. +7), V thread (dims
// 4 vt_dq .. +3 of the 8 keys of slots 32 vt_t + 8 vt_g .. +7); rows past
// p_last are zeros.
struct KVTile {
    f4 kr[8], vr[8];

    __device__ __forceinline__ void load(const float *__restrict__ Kc, const float *__restrict__ Vc,
                                         int64_t kv_stride, int kvh, int64_t j0, int64_t p_last, int tid)
    {
        // one buffer per tile over its rows up to p_last: the rows past it
        // (all of them when p_last < j0, as for a position before the
        // cache) load as zeros
        const uint32_t row = (uint32_t)kv_stride * 4;
        const int64_t valid = max<int64_t>(0, min<int64_t>(p_last + 1 - j0, kKT));
        const uint32_t bytes = __builtin_amdgcn_readfirstlane((uint32_t)valid * row);
        const int64_t base = j0 * kv_stride + kvh * kHD;
        const Rsrc rk = make_rsrc(uniform_ptr(Kc + base), bytes), rv = make_rsrc(uniform_ptr(Vc + base), bytes);
        const int kt_key = tid >> 4, kt_ch = tid & 15;
        const int vt_t = tid >> 7, vt_g = (tid >> 5) & 3, vt_dq = tid & 31;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t at = (uint32_t)(kt_key + 16 * i) * row + 32 * kt_ch;
            kr[2 * i] = bld16(rk, at);
            kr[2 * i + 1] = bld16(rk, at + 16);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            vr[e] = bld16(rv, (uint32_t)(32 * vt_t + 16 * (e / 4) + 4 * vt_g + e % 4) * row + 16 * vt_dq);
    }

    // this wave's max |K| and |V|, into tmax[0][w] and tmax[1][w]
    __device__ __forceinline__ void wave_max(float (*tmax)[4], int lane, int w) const
    {
        float mk = 0.f, mv = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                mk = fmaxf(mk, fabsf(kr[i][u]));
                mv = fmaxf(mv, fabsf(vr[i][u]));
            }
        mk = xor_lanes_max(row16_max(mk));
        mv = xor_lanes_max(row16_max(mv));
        if (lane == 0) {
            tmax[0][w] = mk;
            tmax[1][w] = mv;
        }
    }

    // this thread's 16 split chunks into the padded LDS images (K hi, K lo,
    // V^T hi, V^T lo from lds)
    __device__ __forceinline__ void split_to_lds(int ek, int ev, int tid, _Float16 *lds) const
    {
        const int kt_key = tid >> 4, kt_ch = tid & 15;
        const int vt_t = tid >> 7, vt_g = (tid >> 5) & 3, vt_dq = tid & 31;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h8 hi, lo;
            split8(kr[2 * i], kr[2 * i + 1], ek, hi, lo);
            _Float16 *at = lds + (kt_key + 16 * i) * kRKH + 8 * kt_ch;
            *reinterpret_cast<h8 *>(at) = hi;
            *reinterpret_cast<h8 *>(at + kKT * kRKH) = lo;
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            h8 hi, lo;
            split8(f4{vr[0][d], vr[1][d], vr[2][d], vr[3][d]}, f4{vr[4][d], vr[5][d], vr[6][d], vr[7][d]}, ev, hi,
                   lo);
            _Float16 *at = lds + 2 * kKT * kRKH + (4 * vt_dq + d) * kRVH + 32 * vt_t + 8 * vt_g;
            *reinterpret_cast<h8 *>(at) = hi;
            *reinterpret_cast<h8 *>(at + kHD * kRVH) = lo;
        }
    }
};

__device__ __forceinline__ int split_exp_of(const float (*tmax)[4], int which)
{
    return split_exp(fmaxf(fmaxf(tmax[which][0], tmax[which][1]), fmaxf(tmax[which][2], tmax[which][3])));
}


// Four consecutive values k0 .. k0 + 3 (k0 % 4 == 0) of row m of a GEMM
// operand with K columns, rounded to fp16 into its MFMA fragment-order image
// (the layout x_tile_kernel writes: 32-row blocks, 16-column k steps, 8
// halves per lane slot).
__device__ __forceinline__ void store_operand4(_Float16 *Xt, int64_t K, int64_t m, int64_t k0, f4 v)
{
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const int64_t slot = ((m >> 5) * (K / 16) + (k0 >> 4)) * 64 + (m & 31) + 32 * ((k0 >> 3) & 1);
    *reinterpret_cast<h4 *>(Xt + slot * 8 + (k0 & 7)) = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
}

__global__ void __launch_bounds__(512, 1)
attn_prefill_kernel(const float *__restrict__ Q, int64_t ldq, const float *__restrict__ Kc,
                    const float *__restrict__ Vc, float *__restrict__ O, int64_t n_q, int32_t n_heads,
                    int32_t n_kv_heads, int32_t start, const int32_t *pos, int32_t max_len, float scale,
                    _Float16 *__restrict__ Xt)
{
    // per half: K hi, K lo, V^T hi, V^T lo
    __shared__ __align__(16) _Float16 lds2[2][2 * kKT * kRKH + 2 * kHD * kRVH];
    __shared__ float tmax2[2][2][4];   // [half][K, V][wave]: the half's next tile
    const int tid = threadIdx.x, half = tid >> 8, ht = tid & 255, lane = tid & 63, w = (tid >> 6) & 3;
    _Float16 *const lds = lds2[half], *const ksh = lds, *const vsh = lds + 2 * kKT * kRKH;
    float(*const tmax)[4] = tmax2[half];
    const int h = blockIdx.x;
    const int g = lane >> 4, c = lane & 15;
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t kv_stride = (int64_t)n_kv_heads * kHD, q_stride = (int64_t)n_heads * kHD;
    const int32_t p0 = dev_pos(start, pos);
    // query tiles longest first
    const int64_t i0 = (int64_t)(gridDim.y - 1 - blockIdx.y) * kQTile;
    // keys beyond the cache (a position past max_len) are never read
    const int64_t p_last = min<int64_t>(p0 + min<int64_t>(i0 + kQTile, n_q) - 1, (int64_t)max_len - 1);
    const int64_t n_kt = prefill_key_tiles(i0, n_q, p0, max_len);
    // key ranges: half 0 the first n_kt / 2 tiles and half 1 the rest when
    // the tile spans kSplitKT or more, else half 1 all of them
    const int64_t mid = n_kt >= kSplitKT ? kKT * (n_kt / 2) : 0;
    const int64_t j_begin = half ? mid : 0, j_end = half ? p_last + 1 : mid;
    const int64_t n_iter = (p_last + 1 - mid + kKT - 1) / kKT;   // the longer (second) half's tiles

    // Q^T operand: query 16w + c, dims 32s + 8g .. +7, split with the row's
    // power of two (rows past n_q read the last row, never stored)
    h8 qh[4], ql[4];
    int eq;
    {
        const float *qrow = Q + min<int64_t>(i0 + 16 * w + c, n_q - 1) * ldq + (int64_t)h * kHD + 8 * g;
        f4 qv[8];
        float mx = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            qv[2 * s] = *reinterpret_cast<const f4 *>(qrow + 32 * s);
            qv[2 * s + 1] = *reinterpret_cast<const f4 *>(qrow + 32 * s + 4);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fabsf(qv[i][u]));
        eq = split_exp(xor_lanes_max(mx));
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const hl2 v = split_f16(qv[2 * s + e / 4][e % 4], eq);
                qh[s][e] = v.x;
                ql[s][e] = v.y;
            }
    }
    const int64_t qpos = p0 + min<int64_t>(i0 + 16 * w + c, n_q - 1);   // last key the query attends to
    const float sl = scale * 1.44269504088896341f;                       // scale log2(e)
    float m = -INFINITY, l = 0.f;
    int A = 1 << 20;   // O accumulators hold 2^A O (lowered by the first tile)
    f4 o[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] = f4{0.f, 0.f, 0.f, 0.f};

    // the next tile's rows in registers; both halves take n_iter steps (a
    // half whose range has ended idles through its last ones), so that the
    // workgroup barriers line up
    KVTile kv;
    if (j_begin < j_end) {
        kv.load(Kc, Vc, kv_stride, kvh, j_begin, p_last, ht);
        kv.wave_max(tmax, lane, w);
    }
    for (int64_t it = 0; it < n_iter; ++it) {
        const int64_t j0 = j_begin + kKT * it;
        const bool act = j0 < j_end;
        __syncthreads();   // the previous tile is consumed; tmax holds this one's maxima
        const int ek = split_exp_of(tmax, 0), ev = split_exp_of(tmax, 1);
        if (act) kv.split_to_lds(ek, ev, ht, lds);
        __syncthreads();
        if (!act) continue;
        if (j0 + kKT < j_end) kv.load(Kc, Vc, kv_stride, kvh, j0 + kKT, p_last, ht);   // the next tile in flight

        // S^T = K Q^T, four blocks of 16 keys
        f4 sc[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            const int at = (16 * kb + c) * kRKH + 8 * g;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const h8 kh = *reinterpret_cast<const h8 *>(&ksh[at + 32 * s]);
                const h8 kl = *reinterpret_cast<const h8 *>(&ksh[kKT * kRKH + at + 32 * s]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[s], acc, 0, 0, 0);
            }
            sc[kb] = acc;
        }
        // t = score log2(e) (the powers of two undone exactly in the
        // multiplier), causal mask, online softmax of query c in base 2
        const float cs = ldexpf(sl, -(eq + ek));
        float mx = -INFINITY;
        const int lim = (int)min<int64_t>(qpos - j0, kKT);   // keys past j0 + lim are masked
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = 16 * kb + 4 * g + r > lim ? -INFINITY : sc[kb][r] * cs;
                sc[kb][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = xor_lanes_max(mx);
        // part 0 starts at key 0 and part 1 at a key every row attends to: mn is finite
        const float mn = fmaxf(m, mx), corr = __builtin_amdgcn_exp2f(m - mn);
        const int An = min(A, ev + 15);
        const float f = corr * ldexpf(1.f, max(An - A, -160));
        m = mn;
        A = An;
        const int ep = An - ev;   // P'' = P 2^(A - ev) <= 2^15
        h8 ph[2], pl[2];
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sc[kb][r] = __builtin_amdgcn_exp2f(sc[kb][r] - mn);
                sum += sc[kb][r];
            }
#pragma unroll
        for (int t = 0; t < 2; ++t) split8(sc[2 * t], sc[2 * t + 1], ep, ph[t], pl[t]);
        l = l * corr + sum;
#pragma unroll
        for (int db = 0; db < 8; ++db) o[db] *= f;
        // O^T += V^T P^T, eight blocks of 16 dims, two steps of 32 keys
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const int at = (16 * db + c) * kRVH + 8 * g;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const h8 vh = *reinterpret_cast<const h8 *>(&vsh[at + 32 * t]);
                const h8 vl = *reinterpret_cast<const h8 *>(&vsh[kHD * kRVH + at + 32 * t]);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph[t], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl[t], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph[t], o[db], 0, 0, 0);
            }
        }
        if (j0 + kKT < j_end) kv.wave_max(tmax, lane, w);   // the next tile's maxima (its loads have landed)
    }
    // the four lanes of a query hold sums over disjoint keys, all scaled by the same corrections
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    // half 1 leaves its unnormalised output and (max, sum) per query in its
    // LDS (64 rows of 132 floats); half 0 merges:
    //   O = (2^(m0 - M) o0 + 2^(m1 - M) o1) / (2^(m0 - M) l0 + 2^(m1 - M) l1),  M = max(m0, m1)
    // (a half with no keys has m = -inf, l = 0, o = 0 and weight 0; half 1
    // always has keys)
    const float u = ldexpf(1.f, -A);
    float *const pub = reinterpret_cast<float *>(lds2[1]) + (16 * w + c) * 132;
    __syncthreads();
    if (half == 1) {
#pragma unroll
        for (int db = 0; db < 8; ++db) *reinterpret_cast<f4 *>(pub + 16 * db + 4 * g) = o[db] * u;
        if (g == 0) {
            pub[128] = m;
            pub[129] = l;
        }
    }
    __syncthreads();
    if (half == 1) return;
    const int64_t i = i0 + 16 * w + c;
    f4 r[8];
    {
        const float m1 = pub[128], l1 = pub[129];
        const float mm = fmaxf(m, m1), a0 = exp2f(m - mm), a1 = exp2f(m1 - mm);
        const float den = a0 * l + a1 * l1;
#pragma unroll
        for (int db = 0; db < 8; ++db)
            r[db] = (a0 * (o[db] * u) + a1 * *reinterpret_cast<const f4 *>(pub + 16 * db + 4 * g)) / den;
    }
    if (!Xt) {
        if (i < n_q)
#pragma unroll
            for (int db = 0; db < 8; ++db)
                *reinterpret_cast<f4 *>(O + i * q_stride + (int64_t)h * kHD + 16 * db + 4 * g) = r[db];
        return;
    }
    // The operand image: block b of this head (columns 32 b .. +31 of the
    // head, dims 16 db + 4 g with db = 2b, 2b + 1) of row i is held by the
    // four lanes g of the row; its exponent comes from their maximum
    // (aih_operand.h).  Rows past n_q, up to the next multiple of 32, are zero.
    if (i >= n_q)
#pragma unroll
        for (int db = 0; db < 8; ++db) r[db] = f4{0.f, 0.f, 0.f, 0.f};
    int eb[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        float mx = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) mx = fmaxf(mx, fmaxf(fabsf(r[2 * b][q]), fabsf(r[2 * b + 1][q])));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        eb[b] = aih_operand::block_exp(mx);
    }
    const int64_t mpad = aih_operand::mpad_of(n_q);
    if (i < mpad) {
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const int e = eb[db >> 1] == aih_operand::kZeroBlock ? 0 : eb[db >> 1];
            store_operand4(Xt, q_stride, i, (int64_t)h * kHD + 16 * db + 4 * g,
                           f4{ldexpf(r[db].x, e), ldexpf(r[db].y, e), ldexpf(r[db].z, e), ldexpf(r[db].w, e)});
        }
        char *const img = reinterpret_cast<char *>(Xt);
        const int eg = g == 0 ? eb[0] : g == 1 ? eb[1] : g == 2 ? eb[2] : eb[3];
        reinterpret_cast<int8_t *>(img + aih_operand::block_exp_offset(mpad, q_stride))[i * (q_stride / 32) + 4 * h + g] =
            (int8_t)eg;
        if (h == 0 && g == 0) reinterpret_cast<int32_t *>(img + aih_operand::row_exp_offset(mpad, q_stride))[i] = 0;
    }
}

// ---------------------------------------------------------------- argmax
// First index of the maximum of X[0..n) (NaN never wins).  Writes it to
// *token; when pos is given, also stores it in history[*pos - hist_offset]
// (when inside [0, hist_len)) and advances *pos by one.
__global__ void __launch_bounds__(1024)
argmax_kernel(const float *__restrict__ X, int64_t n, int32_t *token, int32_t *pos, int32_t *history,
              int64_t hist_len, int32_t hist_offset)
{
    __shared__ float bv[16];
    __shared__ int32_t bi[16];
    // the position is read now, while the scan runs (n < 2^31: 32-bit indices)
    const int32_t p0 = pos && threadIdx.x == 0 ? *pos : 0;
    const int32_t nn = (int32_t)n;
    float v = -INFINITY;
    int32_t idx = INT32_MAX;
    // 32 elements per thread per round, all loads issued before the
    // comparisons (one memory round trip for a vocabulary up to 32768), which
    // then run in index order; positions past n read as NaN, which never wins.
    // A 16-byte aligned X is read as 8 vectors per thread (plus a tail of at
    // most 3 elements), otherwise element by element.
    auto take = [&](float x, int32_t i) {
        if (x > v || (idx == INT32_MAX && x == v)) { v = x; idx = i; }
    };
    if ((reinterpret_cast<uintptr_t>(X) & 15) == 0) {
        const f4 *X4 = reinterpret_cast<const f4 *>(X);
        const int32_t n4 = nn >> 2;
        const f4 nan4 = {__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
        for (int32_t b0 = 0; b0 < n4; b0 += 1024 * 8) {
            f4 xs[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t i4 = (int64_t)b0 + j * 1024 + threadIdx.x;
                xs[j] = i4 < n4 ? X4[i4] : nan4;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int32_t i = 4 * (b0 + j * 1024 + (int32_t)threadIdx.x);
                take(xs[j].x, i);
                take(xs[j].y, i + 1);
                take(xs[j].z, i + 2);
                take(xs[j].w, i + 3);
            }
            if (n4 - b0 <= 1024 * 8) break;
        }
        if ((int32_t)threadIdx.x < nn - 4 * n4) take(X[4 * n4 + threadIdx.x], 4 * n4 + (int32_t)threadIdx.x);
    } else {
        constexpr int U = 32;
        for (int32_t b0 = 0; b0 < nn; b0 += 1024 * U) {
            float xs[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = (int64_t)b0 + u * 1024 + threadIdx.x;
                xs[u] = i < nn ? X[i] : __builtin_nanf("");
            }
#pragma unroll
            for (int u = 0; u < U; ++u) take(xs[u], b0 + u * 1024 + (int32_t)threadIdx.x);
            if (nn - b0 <= 1024 * U) break;
        }
    }
    // (value desc, index asc) reduction
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int32_t oi = __shfl_xor(idx, o);
        if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = v; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > v || (bv[w] == v && bi[w] < idx)) { v = bv[w]; idx = bi[w]; }
        const int32_t tok = idx == INT32_MAX ? 0 : idx;
        *token = tok;
        if (pos) {
            const int64_t k = (int64_t)p0 - hist_offset;
            if (history && k >= 0 && k < hist_len) history[k] = tok;
            *pos = p0 + 1;
        }
    }
}

// ---------------------------------------------------------------- GEMM operand
// The activation operand of the prefill GEMM computed by the element-wise step
// before it and written straight in the GEMM's fp16 fragment-order image
// (aih_operand.h), with the row's power of two (the row exponent) chosen from
// the largest magnitude of its values.  One workgroup per row; rows M ..
// mpad-1 (mpad = M rounded up to 32) are zero.  The arithmetic is that of
// rmsnorm_kernel, silu_mul_kernel and silu_mul_pairs_kernel, so the operand
// is the one the separate operator and the GEMM's own conversion
// (PRE = AIH_PRE_NONE) would have built:
//   PRE = AIH_PRE_NONE        x = X
//   PRE = AIH_PRE_RMSNORM     x = (X / sqrt(mean(X^2) + eps)) * X2   (X2: K weights)
//   PRE = AIH_PRE_SILU_MUL    x = SiLU(X) * X2                        (X2: M x K)
//   PRE = AIH_PRE_SILU_PAIRS  x[k] = SiLU(X[2k]) * X[2k+1]            (X: M x 2K)
// Rows of up to 8 * 256 * kRowIt values stay in registers between the maximum
// and the rounding; longer rows are computed twice.  (For AIH_PRE_NONE, at
// 512 x 4096 on MI355X: 7.3 us, against 6.2 us for a conversion without the
// row maximum, one 8-value slot per thread, and 8.7 us with one wave per row.)
constexpr int kRowIt = 8;

template <int NT>
__device__ __forceinline__ float block_max(float v, float *red)
{
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) t = fmaxf(t, red[i]);
    return t;
}

template <int PRE>
__global__ void __launch_bounds__(256)
x_tile_pre_kernel(const float *__restrict__ X, const float *__restrict__ X2, float eps, int64_t M, int64_t K,
                  _Float16 *__restrict__ Xt)
{
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    __shared__ float red[4], redm[4];
    // Workgroup w runs on XCD w % 8.  The 8 rows of an aligned octet share
    // every 128-byte line of the operand (16 bytes each), so they are given
    // workgroups of one XCD: a line is then completed in one L2 instead of
    // being merged from partial lines of eight.  On MI355X, per aih_qgemm
    // call at M = 512: K = 4096 37.4 -> 37.0 us, K = 14336 93.4 -> 88.4 us.
    int64_t m = blockIdx.x;
    if (m < (int64_t)(gridDim.x & ~63u)) m = 8 * ((m >> 6) * 8 + (m & 7)) + ((m >> 3) & 7);
    const int64_t mpad = aih_operand::mpad_of(M);
    int32_t *const E = reinterpret_cast<int32_t *>(reinterpret_cast<char *>(Xt) + aih_operand::row_exp_offset(mpad, K));
    _Float16 *base = Xt + (((m >> 5) * (K / 16)) * 64 + (m & 31)) * 8;
    auto slot = [&](int64_t k) { return reinterpret_cast<h8 *>(base + ((k >> 4) * 64 + ((k >> 3) & 1) * 32) * 8); };
    if (m >= M) {
        for (int64_t k = 8 * (int64_t)threadIdx.x; k < K; k += 8 * 256) *slot(k) = h8{};
        if (threadIdx.x == 0) E[m] = 0;
        return;
    }
    const f4 *x4 = reinterpret_cast<const f4 *>(X + m * (PRE == AIH_PRE_SILU_PAIRS ? 2 * K : K));
    float rms = 1.f;
    if (PRE == AIH_PRE_RMSNORM) {
        float ss = 0.f;
        for (int64_t i = threadIdx.x; i < K / 4; i += 256) {
            const f4 v = x4[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = block_sum<256>(ss, red);
        rms = sqrtf(ss / (float)K + eps);
    }
    // the 8 values x[k .. k+7]
    auto values = [&](int64_t k, float *o) {
        if (PRE == AIH_PRE_NONE) {
            const f4 a = x4[k / 4], b = x4[k / 4 + 1];
            o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
        } else if (PRE == AIH_PRE_RMSNORM) {
            const f4 *w4 = reinterpret_cast<const f4 *>(X2);
            const f4 v[2] = {x4[k / 4], x4[k / 4 + 1]}, w[2] = {w4[k / 4], w4[k / 4 + 1]};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                o[4 * j] = (v[j].x / rms) * w[j].x;
                o[4 * j + 1] = (v[j].y / rms) * w[j].y;
                o[4 * j + 2] = (v[j].z / rms) * w[j].z;
                o[4 * j + 3] = (v[j].w / rms) * w[j].w;
            }
        } else {
            float g[8], u[8];
            if (PRE == AIH_PRE_SILU_MUL) {
                const f4 *u4 = reinterpret_cast<const f4 *>(X2 + m * K);
                const f4 a = x4[k / 4], b = x4[k / 4 + 1], c = u4[k / 4], d = u4[k / 4 + 1];
                const float gg[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                const float uu[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) { g[j] = gg[j]; u[j] = uu[j]; }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4 p = x4[k / 2 + j];
                    g[2 * j] = p.x;
                    u[2 * j] = p.y;
                    g[2 * j + 1] = p.z;
                    u[2 * j + 1] = p.w;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float sig = 1.0f / (1.0f + expf(-g[j]));
                o[j] = (g[j] * sig) * u[j];
            }
        }
    };
    auto store = [&](int64_t k, const float *o, int e) {
        h8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (_Float16)ldexpf(o[j], e);
        *slot(k) = r;
    };
    if (K <= 8 * 256 * kRowIt) {
        float o[kRowIt][8];
        float mx = 0.f;
#pragma unroll
        for (int it = 0; it < kRowIt; ++it) {
            const int64_t k = 8 * (int64_t)threadIdx.x + 2048 * it;
            if (k < K) {
                values(k, o[it]);
#pragma unroll
                for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(o[it][j]));
            }
        }
        const int e = aih_operand::range_exp(block_max<256>(mx, redm));
#pragma unroll
        for (int it = 0; it < kRowIt; ++it) {
            const int64_t k = 8 * (int64_t)threadIdx.x + 2048 * it;
            if (k < K) store(k, o[it], e);
        }
        if (threadIdx.x == 0) E[m] = e;
    } else {
        float o[8], mx = 0.f;
        for (int64_t k = 8 * (int64_t)threadIdx.x; k < K; k += 8 * 256) {
            values(k, o);
#pragma unroll
            for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(o[j]));
        }
        const int e = aih_operand::range_exp(block_max<256>(mx, redm));
        for (int64_t k = 8 * (int64_t)threadIdx.x; k < K; k += 8 * 256) {
            values(k, o);
            store(k, o, e);
        }
        if (threadIdx.x == 0) E[m] = e;
    }
}

unsigned grid_for(aih_ctx *ctx, int64_t work, int per_block = 256)
{
    const int64_t want = (work + per_block - 1) / per_block;
    const int64_t cap = (int64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256) * 8;
    return (unsigned)(want < 1 ? 1 : want < cap ? want : cap);
}

bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

namespace {

// Grouped decode attention for query groups of 1, 2, 4 or 8 heads
// (AIH_E_UNSUPPORTED otherwise); FUSE selects aih_attention_decode_qkv's form.
template <bool FUSE, int NW>
int launch_gqa_nw(aih_ctx *ctx, int group, dim3 grid, const float *Qsrc, float *Kc, float *Vc, float *part,
                  int32_t n_heads, int32_t n_kv_heads, int32_t start, const int32_t *pos, const float *table,
                  int32_t table_rows, int32_t cache_rows, float scale, int32_t n_split)
{
    const dim3 block(64 * NW);
    switch (group) {
    case 1: hipLaunchKernelGGL((attn_decode_gqa<1, FUSE, NW>), grid, block, 0, ctx->stream, Qsrc, Kc, Vc, part,
                               n_heads, n_kv_heads, start, pos, table, table_rows, cache_rows, scale, n_split); break;
    case 2: hipLaunchKernelGGL((attn_decode_gqa<2, FUSE, NW>), grid, block, 0, ctx->stream, Qsrc, Kc, Vc, part,
                               n_heads, n_kv_heads, start, pos, table, table_rows, cache_rows, scale, n_split); break;
    case 4: hipLaunchKernelGGL((attn_decode_gqa<4, FUSE, NW>), grid, block, 0, ctx->stream, Qsrc, Kc, Vc, part,
                               n_heads, n_kv_heads, start, pos, table, table_rows, cache_rows, scale, n_split); break;
    case 8: hipLaunchKernelGGL((attn_decode_gqa<8, FUSE, NW>), grid, block, 0, ctx->stream, Qsrc, Kc, Vc, part,
                               n_heads, n_kv_heads, start, pos, table, table_rows, cache_rows, scale, n_split); break;
    default: return AIH_E_UNSUPPORTED;
    }
    return aih_launch_status();
}

// The short-split kernel: kShortKeys keys per workgroup = NW waves x 16 / G
// keys x SUB sub-steps, NW = min(2 G, 8).  (Groups of 4 heads at 640 cache
// rows, decode step of the 8B-shaped decoder: 8 waves x 4 keys ran 1.431
// ms per token, 4 waves x 4 keys 1.449, 8 waves x 8 keys 1.486 and 16
// waves x 4 keys 1.515.)
template <bool FUSE, int G>
void launch_short(aih_ctx *ctx, dim3 grid, const float *Qsrc, float *Kc, float *Vc, float *part, int32_t n_heads,
                  int32_t n_kv_heads, int32_t start, const int32_t *pos, const float *table, int32_t table_rows,
                  int32_t cache_rows, float scale, int32_t n_split)
{
    constexpr int NW = kShortKeys * G / 16 < kShortWaves ? kShortKeys * G / 16 : kShortWaves;
    constexpr int SUB = kShortKeys * G / (16 * NW);
    static_assert(NW * (16 / G) * SUB == kShortKeys, "short split geometry");
    hipLaunchKernelGGL((attn_decode_short<G, FUSE, NW, SUB>), grid, dim3(64 * NW), 0, ctx->stream, Qsrc, Kc, Vc, part,
                       n_heads, n_kv_heads, start, pos, table, table_rows, cache_rows, scale, n_split);
}

template <bool FUSE>
int launch_gqa(aih_ctx *ctx, int group, dim3 grid, const float *Qsrc, float *Kc, float *Vc, float *part,
               int32_t n_heads, int32_t n_kv_heads, int32_t start, const int32_t *pos, const float *table,
               int32_t table_rows, int32_t cache_rows, float scale, int32_t n_split)
{
    if ((cache_rows + n_split - 1) / n_split <= kShortKeys) {
        switch (group) {
        case 1: launch_short<FUSE, 1>(ctx, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                      table_rows, cache_rows, scale, n_split); break;
        case 2: launch_short<FUSE, 2>(ctx, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                      table_rows, cache_rows, scale, n_split); break;
        case 4: launch_short<FUSE, 4>(ctx, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                      table_rows, cache_rows, scale, n_split); break;
        case 8: launch_short<FUSE, 8>(ctx, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                      table_rows, cache_rows, scale, n_split); break;
        default: return AIH_E_UNSUPPORTED;
        }
        return aih_launch_status();
    }
    switch (decode_waves(cache_rows, n_split)) {
    case 1: return launch_gqa_nw<FUSE, 1>(ctx, group, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                          table_rows, cache_rows, scale, n_split);
    case 2: return launch_gqa_nw<FUSE, 2>(ctx, group, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos, table,
                                          table_rows, cache_rows, scale, n_split);
    default: return launch_gqa_nw<FUSE, 4>(ctx, group, grid, Qsrc, Kc, Vc, part, n_heads, n_kv_heads, start, pos,
                                           table, table_rows, cache_rows, scale, n_split);
    }
}

}  // namespace

int aih_launch_x_tile_pre(aih_ctx *ctx, int pre, const float *X, const float *X2, float eps, int64_t M, int64_t K,
                          void *Xt)
{
    const int64_t mpad = (M + 31) / 32 * 32;
    if (mpad > 0x7FFFFFFF) return AIH_E_LIMIT;
    _Float16 *xt = static_cast<_Float16 *>(Xt);
    switch (pre) {
    case AIH_PRE_NONE:
        hipLaunchKernelGGL(x_tile_pre_kernel<AIH_PRE_NONE>, dim3((unsigned)mpad), dim3(256), 0, ctx->stream, X, X2,
                           eps, M, K, xt);
        break;
    case AIH_PRE_RMSNORM:
        hipLaunchKernelGGL(x_tile_pre_kernel<AIH_PRE_RMSNORM>, dim3((unsigned)mpad), dim3(256), 0, ctx->stream, X, X2,
                           eps, M, K, xt);
        break;
    case AIH_PRE_SILU_MUL:
        hipLaunchKernelGGL(x_tile_pre_kernel<AIH_PRE_SILU_MUL>, dim3((unsigned)mpad), dim3(256), 0, ctx->stream, X, X2,
                           eps, M, K, xt);
        break;
    case AIH_PRE_SILU_PAIRS:
        hipLaunchKernelGGL(x_tile_pre_kernel<AIH_PRE_SILU_PAIRS>, dim3((unsigned)mpad), dim3(256), 0, ctx->stream, X,
                           X2, eps, M, K, xt);
        break;
    default: return AIH_E_INVALID;
    }
    return aih_launch_status();
}

extern "C" {

int aih_rmsnorm(aih_ctx *ctx, const float *X, const float *W, float *Y, int64_t rows, int64_t cols, float eps)
{
    if (!ctx || !X || !W || !Y || rows < 0 || cols <= 0) return AIH_E_INVALID;
    if (rows == 0) return AIH_OK;
    if (rows > 0x7FFFFFFF) return AIH_E_LIMIT;
    const bool vec = cols % 4 == 0 && aligned16(X) && aligned16(W) && aligned16(Y);
    if (vec)
        hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3((unsigned)rows), dim3(256), 0, ctx->stream, X, W, Y, cols, eps);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3((unsigned)rows), dim3(256), 0, ctx->stream, X, W, Y, cols, eps);
    return aih_launch_status();
}

int aih_rope_table(aih_ctx *ctx, float *table, int32_t max_pos, int32_t head_dim, float theta)
{
    if (!ctx || !table || max_pos <= 0 || head_dim <= 0 || head_dim % 2) return AIH_E_INVALID;
    hipLaunchKernelGGL(rope_table_kernel, dim3(grid_for(ctx, (int64_t)max_pos * head_dim / 2)), dim3(256), 0,
                       ctx->stream, table, max_pos, head_dim, theta);
    return aih_launch_status();
}

int aih_rope(aih_ctx *ctx, const float *X, int64_t ldx, float *Y, int64_t ldy, int64_t rows, int32_t n_heads,
             int32_t head_dim, int32_t start, const int32_t *pos, const float *table, int32_t table_rows,
             int y_at_pos, int64_t y_rows)
{
    if (!ctx || !X || !Y || !table || rows < 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 2) return AIH_E_INVALID;
    if (ldx < (int64_t)n_heads * head_dim || ldy < (int64_t)n_heads * head_dim) return AIH_E_INVALID;
    if (rows == 0) return AIH_OK;
    if (!pos && (start < 0 || start + rows > table_rows || (y_at_pos && start + rows > y_rows))) return AIH_E_LIMIT;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(ctx, rows * n_heads * (head_dim / 2))), dim3(256), 0, ctx->stream,
                       X, ldx, Y, ldy, rows, n_heads, head_dim, start, pos, table, table_rows, y_at_pos, y_rows);
    return aih_launch_status();
}

int aih_rope_qkv(aih_ctx *ctx, float *Q, int64_t ldq, const float *K, int64_t ldk, const float *V, int64_t ldv,
                 float *Kc, float *Vc, int64_t rows, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                 int32_t start, const int32_t *pos, const float *table, int32_t table_rows, int64_t cache_rows)
{
    if (!ctx || !Q || !K || !V || !Kc || !Vc || !table || rows < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
        head_dim <= 0 || head_dim % 2)
        return AIH_E_INVALID;
    if (ldq < (int64_t)n_heads * head_dim || ldk < (int64_t)n_kv_heads * head_dim ||
        ldv < (int64_t)n_kv_heads * head_dim)
        return AIH_E_INVALID;
    if (rows == 0) return AIH_OK;
    if (!pos && (start < 0 || start + rows > table_rows || start + rows > cache_rows)) return AIH_E_LIMIT;
    const int64_t q_dim = (int64_t)n_heads * head_dim, kv_dim = (int64_t)n_kv_heads * head_dim;
    if (head_dim % 4 == 0 && ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && q_dim + 2 * kv_dim < (1 << 30) &&
        aligned16(Q) && aligned16(K) && aligned16(V) && aligned16(Kc) && aligned16(Vc) && aligned16(table)) {
        const int64_t gx = (q_dim + 2 * kv_dim + 1023) / 1024;
        hipLaunchKernelGGL(rope_qkv_vec_kernel, dim3((unsigned)gx, (unsigned)std::min<int64_t>(rows, 65535)),
                           dim3(256), 0, ctx->stream, Q, ldq, K, ldk, V, ldv, Kc, Vc, rows, (int32_t)q_dim,
                           (int32_t)kv_dim, head_dim, start, pos, table, table_rows, cache_rows);
        return aih_launch_status();
    }
    const int64_t work = rows * (int64_t)(n_heads + 2 * n_kv_heads) * (head_dim / 2);
    hipLaunchKernelGGL(rope_qkv_kernel, dim3(grid_for(ctx, work)), dim3(256), 0, ctx->stream, Q, ldq, K, ldk, V, ldv,
                       Kc, Vc, rows, n_heads, n_kv_heads, head_dim, start, pos, table, table_rows, cache_rows);
    return aih_launch_status();
}

int aih_store_rows(aih_ctx *ctx, const float *X, int64_t rows, int64_t cols, float *Y, int64_t y_rows, int32_t start,
                   const int32_t *pos)
{
    if (!ctx || !X || !Y || rows < 0 || cols <= 0) return AIH_E_INVALID;
    if (rows == 0) return AIH_OK;
    if (!pos && (start < 0 || start + rows > y_rows)) return AIH_E_LIMIT;
    hipLaunchKernelGGL(store_rows_kernel, dim3(grid_for(ctx, rows * cols)), dim3(256), 0, ctx->stream, X, rows, cols,
                       Y, y_rows, start, pos);
    return aih_launch_status();
}

int aih_silu_mul(aih_ctx *ctx, const float *G, const float *U, float *Y, int64_t n)
{
    if (!ctx || !G || !U || !Y || n < 0) return AIH_E_INVALID;
    if (n == 0) return AIH_OK;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(ctx, n)), dim3(256), 0, ctx->stream, G, U, Y, n);
    return aih_launch_status();
}

int aih_silu_mul_pairs(aih_ctx *ctx, const float *X, float *Y, int64_t rows, int64_t n)
{
    if (!ctx || !X || !Y || rows < 0 || n < 0) return AIH_E_INVALID;
    if (rows == 0 || n == 0) return AIH_OK;
    hipLaunchKernelGGL(silu_mul_pairs_kernel, dim3(grid_for(ctx, rows * n)), dim3(256), 0, ctx->stream, X, Y, rows, n);
    return aih_launch_status();
}

int aih_silu(aih_ctx *ctx, const float *X, float *Y, int64_t n)
{
    if (!ctx || !X || !Y || n < 0) return AIH_E_INVALID;
    if (n == 0) return AIH_OK;
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(ctx, n)), dim3(256), 0, ctx->stream, X, Y, n);
    return aih_launch_status();
}

int aih_mul(aih_ctx *ctx, const float *A, const float *B, float *Y, int64_t n)
{
    if (!ctx || !A || !B || !Y || n < 0) return AIH_E_INVALID;
    if (n == 0) return AIH_OK;
    hipLaunchKernelGGL(mul_kernel, dim3(grid_for(ctx, n)), dim3(256), 0, ctx->stream, A, B, Y, n);
    return aih_launch_status();
}

int aih_add(aih_ctx *ctx, const float *A, const float *B, float *Y, int64_t n)
{
    if (!ctx || !A || !B || !Y || n < 0) return AIH_E_INVALID;
    if (n == 0) return AIH_OK;
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(ctx, n)), dim3(256), 0, ctx->stream, A, B, Y, n);
    return aih_launch_status();
}

// The tiled (prefill) attention: the output as fp32 rows in O, or, with Xt,
// as the fp16 operand image of a GEMM over its n_heads * kHD columns.
static int prefill_attention(aih_ctx *ctx, const float *Q, int64_t ldq, const float *Kc, const float *Vc, float *O,
                             _Float16 *Xt, int64_t n_q, int32_t n_heads, int32_t n_kv_heads, int32_t start,
                             const int32_t *pos, int32_t max_len, float scale)
{
    const int64_t tiles = (n_q + kQTile - 1) / kQTile;
    if (tiles > 65535) return AIH_E_LIMIT;
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_heads, (unsigned)tiles), dim3(512), 0, ctx->stream, Q, ldq, Kc,
                       Vc, O, n_q, n_heads, n_kv_heads, start, pos, max_len, scale, Xt);
    return aih_launch_status();
}

int64_t aih_attention_scratch_floats(int32_t n_heads, int32_t max_len)
{
    if (n_heads <= 0 || max_len <= 0) return AIH_E_INVALID;
    // partials of every (head, split)
    return (int64_t)n_heads * decode_splits(max_len) * (kHD + 2);
}

int aih_attention(aih_ctx *ctx, const float *Q, const float *Kc, const float *Vc, float *O, int64_t n_q,
                  int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start, const int32_t *pos,
                  int32_t max_len, float scale, float *scratch, int64_t scratch_floats)
{
    return aih_attention_strided(ctx, Q, (int64_t)n_heads * head_dim, Kc, Vc, O, n_q, n_heads, n_kv_heads, head_dim,
                                 start, pos, max_len, scale, scratch, scratch_floats);
}

int aih_attention_strided(aih_ctx *ctx, const float *Q, int64_t ldq, const float *Kc, const float *Vc, float *O,
                          int64_t n_q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start,
                          const int32_t *pos, int32_t max_len, float scale, float *scratch,
                          int64_t scratch_floats)
{
    if (!ctx || !Q || !Kc || !Vc || !O || n_q < 0 || n_heads <= 0 || n_kv_heads <= 0 || max_len <= 0)
        return AIH_E_INVALID;
    if (ldq < (int64_t)n_heads * head_dim || ldq % 4) return AIH_E_INVALID;
    if (n_heads % n_kv_heads) return AIH_E_INVALID;
    if (head_dim != kHD) return AIH_E_UNSUPPORTED;
    if (!aligned16(Q) || !aligned16(Kc) || !aligned16(Vc) || !aligned16(O)) return AIH_E_INVALID;
    if (n_q == 0) return AIH_OK;
    if (!pos && (start < 0 || start + n_q > max_len)) return AIH_E_LIMIT;
    if (n_q == 1) {
        const int32_t n_split = decode_splits(max_len);
        const int64_t n_part = (int64_t)n_heads * n_split * (kHD + 2);
        if (!scratch || scratch_floats < n_part) return AIH_E_INVALID;
        // query groups of 1, 2, 4 or 8 heads: the grouped kernel (the plain
        // form of aih_attention_decode_qkv's); others: one workgroup per head
        int rc = launch_gqa<false>(ctx, n_heads / n_kv_heads, dim3(n_kv_heads, n_split), Q,
                                   const_cast<float *>(Kc), const_cast<float *>(Vc), scratch, n_heads, n_kv_heads,
                                   start, pos, nullptr, 0, max_len, scale, n_split);
        if (rc == AIH_E_UNSUPPORTED) {
            hipLaunchKernelGGL(attn_decode_partial, dim3(n_heads, n_split), dim3(256), 0, ctx->stream, Q, Kc, Vc,
                               scratch, n_heads, n_kv_heads, start, pos, max_len, scale, n_split);
            rc = aih_launch_status();
        }
        if (rc) return rc;
        launch_combine(ctx, scratch, O, n_heads, n_split);
        return aih_launch_status();
    }
    return prefill_attention(ctx, Q, ldq, Kc, Vc, O, nullptr, n_q, n_heads, n_kv_heads, start, pos, max_len, scale);
}

int aih_attention_operand(aih_ctx *ctx, const float *Q, int64_t ldq, const float *Kc, const float *Vc, void *Xt,
                          int64_t n_q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t start,
                          const int32_t *pos, int32_t max_len, float scale)
{
    if (!ctx || !Q || !Kc || !Vc || !Xt || n_q < 0 || n_heads <= 0 || n_kv_heads <= 0 || max_len <= 0)
        return AIH_E_INVALID;
    if (ldq < (int64_t)n_heads * head_dim || ldq % 4) return AIH_E_INVALID;
    if (n_heads % n_kv_heads) return AIH_E_INVALID;
    if (head_dim != kHD) return AIH_E_UNSUPPORTED;
    if (!aligned16(Q) || !aligned16(Kc) || !aligned16(Vc) || !aligned16(Xt)) return AIH_E_INVALID;
    if (n_q == 0) return AIH_OK;
    if (!pos && (start < 0 || start + n_q > max_len)) return AIH_E_LIMIT;
    return prefill_attention(ctx, Q, ldq, Kc, Vc, nullptr, static_cast<_Float16 *>(Xt), n_q, n_heads, n_kv_heads,
                             start, pos, max_len, scale);
}

int aih_attention_decode_qkv(aih_ctx *ctx, const float *QKV, float *Kc, float *Vc, float *O, int32_t n_heads,
                             int32_t n_kv_heads, int32_t head_dim, int32_t start, const int32_t *pos,
                             const float *table, int32_t table_rows, int32_t max_len, float scale, float *scratch,
                             int64_t scratch_floats)
{
    if (!ctx || !QKV || !Kc || !Vc || !O || !table || n_heads <= 0 || n_kv_heads <= 0 || max_len <= 0)
        return AIH_E_INVALID;
    if (n_heads % n_kv_heads) return AIH_E_INVALID;
    if (head_dim != kHD) return AIH_E_UNSUPPORTED;
    if (!aligned16(QKV) || !aligned16(Kc) || !aligned16(Vc) || !aligned16(O)) return AIH_E_INVALID;
    if (table_rows < max_len) return AIH_E_LIMIT;
    if (!pos && (start < 0 || start >= max_len)) return AIH_E_LIMIT;
    const int32_t n_split = decode_splits(max_len);
    const int64_t n_part = (int64_t)n_heads * n_split * (kHD + 2);
    if (!scratch || scratch_floats < n_part) return AIH_E_INVALID;
    const int rc = launch_gqa<true>(ctx, n_heads / n_kv_heads, dim3(n_kv_heads, n_split), QKV, Kc, Vc, scratch,
                                    n_heads, n_kv_heads, start, pos, table, table_rows, max_len, scale, n_split);
    if (rc) return rc;
    launch_combine(ctx, scratch, O, n_heads, n_split);
    return aih_launch_status();
}

int aih_embed_q(aih_ctx *ctx, int type, const void *table, int64_t vocab, int64_t dim, const int32_t *ids, int64_t n,
                float *Y)
{
    if (!ctx || !table || !ids || !Y || vocab <= 0 || dim <= 0 || n < 0) return AIH_E_INVALID;
    if (type == AIH_TYPE_F32) {
        if (n == 0) return AIH_OK;
        hipLaunchKernelGGL(embed_f32_kernel, dim3(grid_for(ctx, n * dim)), dim3(256), 0, ctx->stream,
                           static_cast<const float *>(table), vocab, dim, ids, n, Y);
        return aih_launch_status();
    }
    const aih_block_geom g = aih_geom(type);
    if (!aih_is_quant(type)) return AIH_E_UNSUPPORTED;
    if (dim % g.elems) return AIH_E_INVALID;
    return aih_launch_embed(ctx, type, table, vocab, dim, ids, n, Y);
}

int aih_argmax(aih_ctx *ctx, const float *X, int64_t n, int32_t *token, int32_t *pos, int32_t *history,
               int64_t hist_len, int32_t hist_offset)
{
    if (!ctx || !X || !token || n <= 0) return AIH_E_INVALID;
    if (n > 0x7FFFFFFF) return AIH_E_LIMIT;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, ctx->stream, X, n, token, pos, history, hist_len,
                       hist_offset);
    return aih_launch_status();
}

}  // extern "C"
