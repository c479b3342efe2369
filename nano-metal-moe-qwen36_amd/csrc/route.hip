/*
 * route.hip -- router logits and bit-exact softmax / top-k / renormalise.
 *
 * Reference behaviour (file:line relative to the reference root):
 *   logits : metal/kernels.metal:472-513 (q4 router rows of
 *            nmoe_route_shared_q4); the benchmark configs use a dense bf16
 *            router [256][2048] instead.
 *   routing: src/runtime.m:1498-1511 runs, on the host,
 *            math.m:67-93  softmax  (max; expf(v-max); long double sum;
 *                                    multiply by 1/(float)sum)
 *            math.m:95-132 top-k    (k arg-max passes; a tie goes to the
 *                                    lower index)
 *            math.m:134-153 renormalise (fp32 sum; multiply by 1/sum).
 *
 * Here the whole routing runs in one wavefront per token.  The selected
 * indices depend on exact probability ties, so every step reproduces the
 * host arithmetic bit for bit: expf is glibc's algorithm restated in double
 * (nmoe_exact.h), and the long double running sum is either proven exact
 * (every term >= 2^-32, summed as integers in units of 2^-55) or replayed
 * sequentially with an emulated 64-bit-significand adder in lane 0.
 *
 * Logits use a fixed reduction order (lane L accumulates its 16-byte chunks
 * L, L+64, ... with fma, then an xor butterfly), so identical inputs give
 * identical logits on every run.
 */
#include "nmoe_hip_internal.h"

#pragma clang fp contract(off)

__constant__ uint64_t nmoe_exp2_tab[32] = NMOE_EXP2_TAB32;

/* ------------------------------------------------------------- logits */

template <typename XT>
__device__ __forceinline__ void nmoe_load_x8(const XT *x, int chunk, float out[8]);

template <>
__device__ __forceinline__ void nmoe_load_x8<uint16_t>(const uint16_t *x, int chunk, float out[8]) {
    uint4 v = ((const uint4 *)x)[chunk];
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

template <>
__device__ __forceinline__ void nmoe_load_x8<float>(const float *x, int chunk, float out[8]) {
    float4 a = ((const float4 *)x)[2 * chunk];
    float4 b = ((const float4 *)x)[2 * chunk + 1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

/* One wavefront computes logit e for tokens [t0, t1). */
template <typename XT>
__global__ void __launch_bounds__(64) nmoe_router_bf16_kernel(const uint16_t *__restrict__ w, const XT *__restrict__ x,
                                                              int ntok, int num_experts, int tok_per_block,
                                                              float *__restrict__ logits) {
    const int e = blockIdx.x;
    const int lane = threadIdx.x;
    const uint4 *row = (const uint4 *)(w + (size_t)e * NMOE_HIDDEN);
    uint4 wv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) wv[j] = row[lane + 64 * j];
    int t0 = blockIdx.y * tok_per_block;
    int t1 = min(ntok, t0 + tok_per_block);
    for (int t = t0; t < t1; t++) {
        const XT *xt = x + (size_t)t * NMOE_HIDDEN;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float xv[8];
            nmoe_load_x8<XT>(xt, lane + 64 * j, xv);
            uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc = __builtin_fmaf(__uint_as_float(ww[i] << 16), xv[2 * i], acc);
                acc = __builtin_fmaf(__uint_as_float(ww[i] & 0xffff0000u), xv[2 * i + 1], acc);
            }
        }
        acc = nmoe_wave_sum_butterfly(acc);
        if (lane == 0) logits[(size_t)t * num_experts + e] = acc;
    }
}

/* q4 router row: 256 words; lane L owns words L, L+64, L+128, L+192. */
template <typename XT>
__global__ void __launch_bounds__(64) nmoe_router_q4_kernel(const uint32_t *__restrict__ w,
                                                            const uint16_t *__restrict__ sc,
                                                            const uint16_t *__restrict__ bi, const XT *__restrict__ x,
                                                            int ntok, int num_experts, int tok_per_block,
                                                            float *__restrict__ logits) {
    const int e = blockIdx.x;
    const int lane = threadIdx.x;
    uint32_t wv[4];
    float s[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int c = lane + 64 * j;
        wv[j] = w[(size_t)e * (NMOE_HIDDEN / 8) + c];
        s[j] = nmoe_bf16f(sc[(size_t)e * (NMOE_HIDDEN / NMOE_GROUP) + c / 8]);
        b[j] = nmoe_bf16f(bi[(size_t)e * (NMOE_HIDDEN / NMOE_GROUP) + c / 8]);
    }
    int t0 = blockIdx.y * tok_per_block;
    int t1 = min(ntok, t0 + tok_per_block);
    for (int t = t0; t < t1; t++) {
        const XT *xt = x + (size_t)t * NMOE_HIDDEN;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float xv[8];
            nmoe_load_x8<XT>(xt, lane + 64 * j, xv);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float q = (float)((wv[j] >> (4 * i)) & 0xFu);
                acc = __builtin_fmaf(__builtin_fmaf(q, s[j], b[j]), xv[i], acc);
            }
        }
        acc = nmoe_wave_sum_butterfly(acc);
        if (lane == 0) logits[(size_t)t * num_experts + e] = acc;
    }
}

/* ------------------------------------------------------------ routing */

__device__ __forceinline__ uint64_t nmoe_wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
        uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
        v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}

__device__ __forceinline__ bool nmoe_better(float va, uint32_t ia, float vb, uint32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

/* Routes one token with a full wavefront.  On return every lane holds the
 * same sel_i / sel_w (slots >= n are 0).  `scratch` is 256 floats of LDS
 * (used only by the exact sequential-sum path).  Returns n = min(k, E). */
__device__ int nmoe_wave_route(const float *__restrict__ lg, int num_experts, int k, float *scratch,
                               uint32_t sel_i[NMOE_MAX_K], float sel_w[NMOE_MAX_K], float *__restrict__ probs) {
    const int lane = threadIdx.x & 63;
    float l[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int i = lane + 64 * j;
        l[j] = i < num_experts ? lg[i] : -__builtin_inff();
    }
    /* max: order-independent for finite inputs (equal zeros of either sign
     * give identical exp arguments' results) */
    float m = fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));

    float e[4];
    uint64_t fx = 0;
    int ok = 1;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int i = lane + 64 * j;
        e[j] = i < num_experts ? nmoe_expf_glibc(l[j] - m, nmoe_exp2_tab) : 0.0f;
        uint64_t f = 0;
        ok &= nmoe_softmax_term_fixed(e[j], &f);
        fx += f;
    }
    float total;
    if (__ballot(!ok) == 0) {
        /* every term is a multiple of 2^-55 and the sum < 2^63: the x87
         * running sum was exact, so it equals this integer sum */
        total = nmoe_u64_scaled_to_f32_rne(nmoe_wave_sum_u64(fx));
    } else {
        /* replay math.m's long double running sum in index order */
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int i = lane + 64 * j;
            if (i < num_experts) scratch[i] = e[j];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        float t = 0.0f;
        if (lane == 0) {
            nmoe_x87 acc = nmoe_x87_zero();
            for (int i = 0; i < num_experts; i++) acc = nmoe_x87_add(acc, nmoe_x87_from_float(scratch[i]));
            t = nmoe_x87_to_float(acc);
        }
        total = __shfl(t, 0, 64);
        __builtin_amdgcn_wave_barrier();
    }
    float p[4];
    if (total == 0.0f) {
        float u = 1.0f / (float)num_experts;
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = u;
    } else {
        float inv = 1.0f / total;
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = e[j] * inv;
    }
    if (probs != NULL) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int i = lane + 64 * j;
            if (i < num_experts) probs[i] = p[j];
        }
    }

    int n = min(k, num_experts);
    uint32_t taken = 0;
    float sel_v[NMOE_MAX_K];
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        sel_i[s] = 0;
        sel_v[s] = 0.0f;
    }
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) {
        if (s >= n) break;
        float bv = -__builtin_inff();
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t i = (uint32_t)(lane + 64 * j);
            if (i < (uint32_t)num_experts && !((taken >> j) & 1u) && nmoe_better(p[j], i, bv, bi)) {
                bv = p[j];
                bi = i;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            float ov = __shfl_xor(bv, off, 64);
            uint32_t oi = __shfl_xor(bi, off, 64);
            if (nmoe_better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi & 63u) == (uint32_t)lane) taken |= 1u << (bi >> 6);
        sel_i[s] = bi;
        sel_v[s] = bv;
    }
    /* math.m:134-153 */
    float sum = 0.0f;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++)
        if (s < n) sum += sel_v[s];
    float inv = sum == 0.0f ? 1.0f / (float)n : 1.0f / sum;
#pragma unroll
    for (int s = 0; s < NMOE_MAX_K; s++) sel_w[s] = s < n ? (sum == 0.0f ? inv : sel_v[s] * inv) : 0.0f;
    return n;
}

__global__ void __launch_bounds__(64) nmoe_topk_kernel(const float *__restrict__ logits, int ntok, int num_experts,
                                                       int k, uint32_t *__restrict__ idx, float *__restrict__ w,
                                                       float *__restrict__ probs) {
    __shared__ float scratch[NMOE_EXPERTS];
    int t = blockIdx.x;
    if (t >= ntok) return;
    uint32_t si[NMOE_MAX_K];
    float sw[NMOE_MAX_K];
    nmoe_wave_route(logits + (size_t)t * num_experts, num_experts, k, scratch, si, sw,
                    probs != NULL ? probs + (size_t)t * num_experts : NULL);
    int lane = threadIdx.x;
    if (lane < NMOE_MAX_K) {
        uint32_t vi = 0;
        float vw = 0.0f;
#pragma unroll
        for (int s = 0; s < NMOE_MAX_K; s++)
            if (s == lane) {
                vi = si[s];
                vw = sw[s];
            }
        idx[(size_t)t * NMOE_MAX_K + lane] = vi;
        w[(size_t)t * NMOE_MAX_K + lane] = vw;
    }
}

/* ------------------------------------------------------- entry points */

int nmoe_check_router(nmoe_hip_ctx *ctx, const nmoe_hip_router *r) {
    if (r == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL router");
    if (r->num_experts < 1 || r->num_experts > NMOE_EXPERTS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "num_experts %d outside 1..256", r->num_experts);
    if (r->kind == NMOE_HIP_ROUTER_BF16) {
        if (r->w_bf16 == NULL || !nmoe_aligned(r->w_bf16, 16))
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "bf16 router weights NULL or not 16-byte aligned");
    } else if (r->kind == NMOE_HIP_ROUTER_Q4) {
        if (r->w_q4 == NULL || r->scales == NULL || r->biases == NULL || !nmoe_aligned(r->w_q4, 4))
            return nmoe_fail(ctx, NMOE_HIP_EINVAL, "q4 router tensors NULL or misaligned");
    } else {
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "unknown router kind %d", r->kind);
    }
    return NMOE_HIP_OK;
}

int nmoe_check_x(nmoe_hip_ctx *ctx, const void *x, int x_dtype, int ntok) {
    if (x == NULL || !nmoe_aligned(x, 16)) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "x NULL or not 16-byte aligned");
    if (x_dtype != NMOE_HIP_F32 && x_dtype != NMOE_HIP_BF16)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "x_dtype must be NMOE_HIP_F32 or NMOE_HIP_BF16");
    if (ntok < 1 || ntok > ctx->max_tokens)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "ntok %d outside 1..%d (max_tokens at create)", ntok, ctx->max_tokens);
    return NMOE_HIP_OK;
}

extern "C" int nmoe_moe_router_logits(nmoe_hip_ctx *ctx, const nmoe_hip_router *router, const void *x, int x_dtype,
                                      int ntok, float *logits, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    int rc = nmoe_check_router(ctx, router);
    if (rc == NMOE_HIP_OK) rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    if (logits == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL logits");
    int tpb = ntok <= 4 ? ntok : 4;
    dim3 grid(router->num_experts, (ntok + tpb - 1) / tpb);
    hipStream_t s = nmoe_stream_of(ctx, stream);
    if (router->kind == NMOE_HIP_ROUTER_BF16) {
        if (x_dtype == NMOE_HIP_BF16)
            hipLaunchKernelGGL(nmoe_router_bf16_kernel<uint16_t>, grid, dim3(64), 0, s, router->w_bf16,
                               (const uint16_t *)x, ntok, router->num_experts, tpb, logits);
        else
            hipLaunchKernelGGL(nmoe_router_bf16_kernel<float>, grid, dim3(64), 0, s, router->w_bf16,
                               (const float *)x, ntok, router->num_experts, tpb, logits);
    } else {
        if (x_dtype == NMOE_HIP_BF16)
            hipLaunchKernelGGL(nmoe_router_q4_kernel<uint16_t>, grid, dim3(64), 0, s, router->w_q4, router->scales,
                               router->biases, (const uint16_t *)x, ntok, router->num_experts, tpb, logits);
        else
            hipLaunchKernelGGL(nmoe_router_q4_kernel<float>, grid, dim3(64), 0, s, router->w_q4, router->scales,
                               router->biases, (const float *)x, ntok, router->num_experts, tpb, logits);
    }
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}

extern "C" int nmoe_moe_topk(nmoe_hip_ctx *ctx, const float *logits, int ntok, int num_experts, int k, uint32_t *idx,
                             float *w, float *probs, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (logits == NULL || idx == NULL || w == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL argument");
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    if (num_experts < 1 || num_experts > NMOE_EXPERTS)
        return nmoe_fail(ctx, NMOE_HIP_EINVAL, "num_experts %d outside 1..256", num_experts);
    if (ntok < 1) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "ntok must be >= 1");
    hipLaunchKernelGGL(nmoe_topk_kernel, dim3(ntok), dim3(64), 0, nmoe_stream_of(ctx, stream), logits, ntok,
                       num_experts, k, idx, w, probs);
    NMOE_HIP_TRY(ctx, hipGetLastError());
    return NMOE_HIP_OK;
}

extern "C" int nmoe_moe_route(nmoe_hip_ctx *ctx, const nmoe_hip_router *router, const void *x, int x_dtype, int ntok,
                              int k, uint32_t *idx, float *w, float *logits, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    if (k < 1 || k > NMOE_MAX_K) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "k=%d outside 1..8", k);
    int rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    float *lg = logits != NULL ? logits : ctx->logits;
    rc = nmoe_moe_router_logits(ctx, router, x, x_dtype, ntok, lg, stream);
    if (rc != NMOE_HIP_OK) return rc;
    return nmoe_moe_topk(ctx, lg, ntok, router->num_experts, k, idx, w, NULL, stream);
}
