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
 * L, L+64, ... with fma; the 64 lane partials are combined by the balanced
 * pairwise tree over lanes in order), so identical inputs give identical
 * logits on every run, in both the standalone and the fused kernels.
 */
#include "nmoe_device.h"

#pragma clang fp contract(off)

static __constant__ uint64_t nmoe_exp2_tab[32] = NMOE_EXP2_TAB32;

/* ------------------------------------------------------------- logits */

/* One wavefront per (row, token block): logits[t][e] for t in [t0, t1). */
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
        float xs[32];
#pragma unroll
        for (int j = 0; j < 4; j++) nmoe_load_cols<XT>(xt, (lane + 64 * j) * 8, 8, xs + 8 * j);
        float logit = nmoe_router_row_bf16(wv, xs);
        if (lane == 0) logits[(size_t)t * num_experts + e] = logit;
    }
}

/* q4 router row (the reference model's router, kernels.metal:472-513):
 * 256 words; lane L owns words L, L+64, L+128, L+192 and accumulates
 * acc + fma(q, s*x, b*x) per column (kernels.metal:500-508); lane partials
 * combined by the pairwise tree. */
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
            nmoe_load_cols<XT>(xt, (lane + 64 * j) * 8, 8, xv);
#pragma unroll
            for (int i = 0; i < 8; i++) acc = nmoe_router_q4_term(acc, (wv[j] >> (4 * i)) & 0xFu, s[j], b[j], xv[i]);
        }
        acc = nmoe_wave_sum_tree(acc);
        if (lane == 0) logits[(size_t)t * num_experts + e] = acc;
    }
}

/* ------------------------------------------------------------ routing */

__global__ void __launch_bounds__(64) nmoe_topk_kernel(const float *__restrict__ logits, int ntok, int num_experts,
                                                       int k, uint32_t *__restrict__ idx, float *__restrict__ w,
                                                       float *__restrict__ probs) {
    __shared__ float scratch[NMOE_EXPERTS];
    int t = blockIdx.x;
    if (t >= ntok) return;
    uint32_t si[NMOE_MAX_K];
    float sw[NMOE_MAX_K];
    nmoe_wave_route(logits + (size_t)t * num_experts, num_experts, k, scratch, nmoe_exp2_tab, si, sw,
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

/* The router launch with its arguments already checked. */
extern "C" hipError_t nmoe_router_logits_launch(const nmoe_hip_router *router, const void *x, int x_dtype, int ntok,
                                               float *logits, hipStream_t s) {
    int tpb = ntok <= 4 ? ntok : 4;
    dim3 grid(router->num_experts, (ntok + tpb - 1) / tpb);
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
    return hipGetLastError();
}

extern "C" hipError_t nmoe_topk_launch(const float *logits, int ntok, int num_experts, int k, uint32_t *idx, float *w,
                                      float *probs, hipStream_t s) {
    hipLaunchKernelGGL(nmoe_topk_kernel, dim3(ntok), dim3(64), 0, s, logits, ntok, num_experts, k, idx, w, probs);
    return hipGetLastError();
}

extern "C" int nmoe_moe_router_logits(nmoe_hip_ctx *ctx, const nmoe_hip_router *router, const void *x, int x_dtype,
                                      int ntok, float *logits, void *stream) {
    if (ctx == NULL) return NMOE_HIP_EINVAL;
    int rc = nmoe_check_router(ctx, router);
    if (rc == NMOE_HIP_OK) rc = nmoe_check_x(ctx, x, x_dtype, ntok);
    if (rc != NMOE_HIP_OK) return rc;
    if (logits == NULL) return nmoe_fail(ctx, NMOE_HIP_EINVAL, "NULL logits");
    NMOE_HIP_TRY(ctx, nmoe_router_logits_launch(router, x, x_dtype, ntok, logits, nmoe_stream_of(ctx, stream)));
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
    NMOE_HIP_TRY(ctx, nmoe_topk_launch(logits, ntok, num_experts, k, idx, w, probs, nmoe_stream_of(ctx, stream)));
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
