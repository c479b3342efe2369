/*
 * probe.hip -- the streaming ceiling of the batch-1 decode step.
 *
 * nmoe_hip_read_probe reads `bytes` of device memory once with the access
 * pattern of the fused decode step's expert loads -- 256 blocks, every
 * 16-byte load of a block issued before any is used, non-temporal -- and
 * does nothing else but fold the words into one value per block.  Its
 * launch time is the floor the fused step's expert phase cannot go below:
 * the time to stream the step's 14.2 MB of expert bytes from a cold start
 * (latency of the first bytes plus the transfer), with no routing before it
 * and no exchange after it.  No reference counterpart (a measurement entry
 * point, like the reference's matvec micro-benchmark scripts/matvec_bench.m).
 */
#include "nmoe_device.h"

#define NMOE_PROBE_BLOCKS 256
#define NMOE_PROBE_THREADS 512
#define NMOE_PROBE_LOADS 8 /* 16-byte loads per thread, all in flight together */

typedef unsigned int nmoe_probe_u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(NMOE_PROBE_THREADS) nmoe_read_probe_kernel(const uint4 *src, uint64_t n16,
                                                                            uint32_t *sink) {
    const uint64_t per = (n16 + NMOE_PROBE_BLOCKS - 1) / NMOE_PROBE_BLOCKS;
    const uint64_t b0 = (uint64_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    nmoe_probe_u32x4 v[NMOE_PROBE_LOADS];
#pragma unroll
    for (int j = 0; j < NMOE_PROBE_LOADS; j++) {
        const uint64_t i = b0 + threadIdx.x + (uint64_t)NMOE_PROBE_THREADS * j;
        v[j] = i < b1 ? __builtin_nontemporal_load((const nmoe_probe_u32x4 *)(src + i)) : nmoe_probe_u32x4{0, 0, 0, 0};
    }
    uint32_t x = 0;
#pragma unroll
    for (int j = 0; j < NMOE_PROBE_LOADS; j++) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    /* the block's fold: a wave sum, then one word per wavefront */
    for (int d = 32; d >= 1; d >>= 1) x ^= (uint32_t)__shfl_xor((int)x, d, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (NMOE_PROBE_THREADS / 64) + (threadIdx.x >> 6)] = x;
}

extern "C" int nmoe_hip_read_probe(nmoe_hip_ctx *ctx, const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    const uint64_t cap = (uint64_t)NMOE_PROBE_BLOCKS * NMOE_PROBE_THREADS * NMOE_PROBE_LOADS * 16u;
    if (src == NULL || sink == NULL || !nmoe_aligned(src, 16) || bytes == 0 || bytes % 16 != 0 || bytes > cap)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "probe: src (16-byte aligned), sink and 0 < bytes <= %llu, a multiple "
                                               "of 16, are required", (unsigned long long)cap);
    hipLaunchKernelGGL(nmoe_read_probe_kernel, dim3(NMOE_PROBE_BLOCKS), dim3(NMOE_PROBE_THREADS), 0,
                       nmoe_stream_of(ctx, stream), (const uint4 *)src, (uint64_t)(bytes / 16), sink);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}
