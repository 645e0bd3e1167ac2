// aih_probe.hip -- the memory-system ceilings the matvec is measured against.
//
// aih_probe_stream_read streams a buffer through the compute units with
// 16-byte loads and nothing else: one workgroup of 512 threads per CU (the
// matvec's launch shape), each thread reading consecutive 16-byte pieces
// strided by the whole grid, XOR-folding them so that the loads stay live.
// Its time per launch, replayed from a graph over rotating copies larger than
// the Infinity Cache, is the ceiling for one kernel that reads that many
// bytes once: the matvec reads the same bytes and also computes.  With
// nontemporal != 0 the loads carry the non-temporal hint (the lines are not
// kept in the caches).  bytes == 0 launches the same grid with nothing to
// read: the fixed cost of one launch.  `out` receives one word per wave: it
// must hold 8192 words.
#include "aih_internal.h"

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <bool NT>
__global__ void __launch_bounds__(512) stream_read_kernel(const u4 *__restrict__ src, uint64_t n16,
                                                          uint32_t *__restrict__ out)
{
    const uint64_t stride = (uint64_t)gridDim.x * 512;
    u4 acc = {0u, 0u, 0u, 0u};
    uint64_t i = (uint64_t)blockIdx.x * 512 + threadIdx.x;
    // four loads in flight per thread per step
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = NT ? __builtin_nontemporal_load(src + i + j * stride) : src[i + j * stride];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    for (; i < n16; i += stride) acc ^= NT ? __builtin_nontemporal_load(src + i) : src[i];
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    // one word per wave (one per thread would be traffic of its own)
    uint32_t w = x;
    for (int o = 32; o > 0; o >>= 1) w ^= (uint32_t)__shfl_xor((int)w, o);
    if ((threadIdx.x & 63) == 0) out[(uint64_t)blockIdx.x * 8 + (threadIdx.x >> 6)] = w;
}

// bytes == 0: the same grid, nothing to read (its own name in a kernel trace)
__global__ void __launch_bounds__(512) launch_floor_kernel(uint32_t *__restrict__ out)
{
    if ((threadIdx.x & 63) == 0) out[(uint64_t)blockIdx.x * 8 + (threadIdx.x >> 6)] = 0u;
}

}  // namespace

extern "C" int aih_probe_stream_read(aih_ctx *ctx, const void *src, uint64_t bytes, int nontemporal, uint32_t *out)
{
    if (!ctx || !out || (bytes && !src) || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15)) return AIH_E_INVALID;
    int cur = -1;
    AIH_TRY(hipGetDevice(&cur));
    if (cur != ctx->device) AIH_TRY(hipSetDevice(ctx->device));
    // one workgroup per CU, at most 1024 (out holds 8 words per workgroup)
    const unsigned grid = ctx->cu_count > 0 && ctx->cu_count <= 1024 ? (unsigned)ctx->cu_count : 256u;
    const u4 *s = static_cast<const u4 *>(src);
    if (!bytes)
        hipLaunchKernelGGL(launch_floor_kernel, dim3(grid), dim3(512), 0, ctx->stream, out);
    else if (nontemporal)
        hipLaunchKernelGGL(stream_read_kernel<true>, dim3(grid), dim3(512), 0, ctx->stream, s, bytes / 16, out);
    else
        hipLaunchKernelGGL(stream_read_kernel<false>, dim3(grid), dim3(512), 0, ctx->stream, s, bytes / 16, out);
    return aih_launch_status();
}
