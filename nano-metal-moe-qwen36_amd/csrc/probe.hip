/*
 * probe.hip -- the streaming ceiling of the batch-1 decode step.
 *
 * nmoe_hip_read_probe reads `bytes` of device memory once with the access
 * pattern of the fused decode step's expert loads -- 256 blocks, every
 * 16-byte load of a block issued before any is used, non-temporal -- and
 * does nothing else but fold the words into one value per wavefront.  Its
 * launch time is the floor the fused step's expert phase cannot go below:
 * the time to stream the step's 14.2 MB of expert bytes from a cold start
 * (latency of the first bytes plus the transfer), with no routing before it
 * and no exchange after it.  nmoe_hip_read_probe_grid is the same kernel at
 * any launch shape (blocks, threads a block, loads a thread a round) and
 * size, so that the part's sustained read rate, and whether another shape
 * streams the step's bytes sooner, can be measured; a 16-byte read is the
 * period of a near-empty launch of that grid.  No reference counterpart (a
 * measurement entry point, like the reference's matvec micro-benchmark
 * scripts/matvec_bench.m, which sweeps its launch shape over a rotating
 * 512 MB pool).
 *
 * Block b reads the 16-byte items [b * per, min((b + 1) * per, n)),
 * per = ceil(n / blocks), in rounds of threads * loads items: in a round,
 * lane t loads items base + t + threads * j (j < loads), all in flight
 * before any is folded.  sink[b * (threads / 64) + w] is the XOR of every
 * 32-bit word wavefront w of block b loaded.
 */
#include "nmoe_device.h"

#define NMOE_PROBE_BLOCKS 256
#define NMOE_PROBE_THREADS 512
#define NMOE_PROBE_LOADS 8 /* 16-byte loads per thread and round, all in flight together */
#define NMOE_PROBE_MAX_BLOCKS 8192
#define NMOE_PROBE_MAX_THREADS 1024

typedef unsigned int nmoe_probe_u32x4 __attribute__((ext_vector_type(4)));

template <int LOADS>
__global__ void __launch_bounds__(NMOE_PROBE_MAX_THREADS) nmoe_read_probe_kernel(const uint4 *src, uint64_t n16,
                                                                                uint32_t *sink) {
    const uint32_t nt = blockDim.x;
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t b0 = (uint64_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    uint32_t x = 0;
    for (uint64_t base = b0; base < b1; base += (uint64_t)nt * LOADS) {
        nmoe_probe_u32x4 v[LOADS];
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const uint64_t i = base + threadIdx.x + (uint64_t)nt * j;
            v[j] = i < b1 ? __builtin_nontemporal_load((const nmoe_probe_u32x4 *)(src + i)) : nmoe_probe_u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < LOADS; j++) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    /* the wavefront's fold, one word per wavefront */
    for (int d = 32; d >= 1; d >>= 1) x ^= (uint32_t)__shfl_xor((int)x, d, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (nt / 64) + (threadIdx.x >> 6)] = x;
}

extern "C" int nmoe_hip_read_probe_grid(nmoe_hip_ctx *ctx, const void *src, size_t bytes, int blocks, int threads,
                                        int loads, uint32_t *sink, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (src == NULL || sink == NULL || !nmoe_aligned(src, 16) || !nmoe_aligned(sink, 4) || bytes == 0 ||
        bytes % 16 != 0)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "probe: src (16-byte aligned), sink and 0 < bytes, a multiple of 16, "
                                               "are required");
    if (blocks < 1 || blocks > NMOE_PROBE_MAX_BLOCKS || threads < 64 || threads > NMOE_PROBE_MAX_THREADS ||
        threads % 64 != 0 || (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16))
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "probe: 1..%d blocks of 64..%d threads (a multiple of 64), loads 1, 2, "
                                               "4, 8 or 16", NMOE_PROBE_MAX_BLOCKS, NMOE_PROBE_MAX_THREADS);
    hipStream_t s = nmoe_stream_of(ctx, stream);
    const uint64_t n16 = (uint64_t)(bytes / 16);
    const dim3 g(blocks), b(threads);
    switch (loads) {
    case 1: hipLaunchKernelGGL(nmoe_read_probe_kernel<1>, g, b, 0, s, (const uint4 *)src, n16, sink); break;
    case 2: hipLaunchKernelGGL(nmoe_read_probe_kernel<2>, g, b, 0, s, (const uint4 *)src, n16, sink); break;
    case 4: hipLaunchKernelGGL(nmoe_read_probe_kernel<4>, g, b, 0, s, (const uint4 *)src, n16, sink); break;
    case 8: hipLaunchKernelGGL(nmoe_read_probe_kernel<8>, g, b, 0, s, (const uint4 *)src, n16, sink); break;
    default: hipLaunchKernelGGL(nmoe_read_probe_kernel<16>, g, b, 0, s, (const uint4 *)src, n16, sink); break;
    }
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}

extern "C" int nmoe_hip_read_probe(nmoe_hip_ctx *ctx, const void *src, size_t bytes, uint32_t *sink, void *stream) {
    return nmoe_hip_read_probe_grid(ctx, src, bytes, NMOE_PROBE_BLOCKS, NMOE_PROBE_THREADS, NMOE_PROBE_LOADS, sink,
                                    stream);
}
